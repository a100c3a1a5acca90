"""Row-pair operands (``data_layout="pairs"`` / ``MXGG_DATA_PAIRS``,
``MXGG_A_PAIRS`` / ``MXGG_B_PAIRS``): rows 2i and 2i+1 interleaved in 64-byte
pieces, so the GEMMs copy whole 128-byte lines; and row quads of packed e2m1
weights (``data_layout="quads"``, ``MXGG_B_QUADS``: 4 rows in 32-byte
pieces).  A layout of this build with no counterpart in the reference, held
to the row-major path bit for bit:

* the quantizers' row-pair output holds the bytes of their row-major output
  (read back through the returned view, and at the byte offsets the C header
  documents, on the raw storage), the pad past an odd multiple of 32 is
  zero, and the scales are unchanged;
* ``to_row_pairs`` / ``to_row_quads`` of row-major data equal the quantizers'
  row-group output;
* the forward / dgrad and wgrad GEMMs return the same bits with either
  operand, or both, in row pairs as with both row-major: group starts at odd
  rows (a tile whose first row is the second of a pair), partial tiles,
  128 x 128 tiles, split launches and (among the benchmark shapes)
  quarter-tile ones, f32 / f16 outputs, an e2m1 weight row-major or in row
  quads beside a row-major or row-pair A (BASELINE config 5 at full size),
  token ranges off the 16 grid (the wgrad's edge chunks), 2080 tokens (rows
  padded to 2112), and every benchmark shape.
"""

import numpy as np
import pytest
import torch

from oracle import mx_oracle as O

pytestmark = pytest.mark.gpu

M_TOKENS = 16640
SHAPES = [(e, n, k) for e in (1, 2, 4, 8) for n in (2048, 5120, 8192) for k in (2048, 5120, 8192)]


def _x(shape, seed, dev, std=1.0, dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * std).to(dtype)


def _u8(t):
    return t.view(torch.uint8)


def _rows_of(pairs, L):
    """Row-major bytes (.., R, L) and the pad (.., R, Lp - L) of a row-pair view."""
    *b, P, two, S, w = pairs.shape
    r = _u8(pairs).reshape(tuple(b) + (2 * P, 64 * S))
    return r[..., :L], r[..., L:]


def _odd_offs(E, M, seed):
    """Cumulative group ends with odd starts and bounds off the 16 grid."""
    rng = np.random.default_rng(seed)
    cuts = np.sort(rng.choice(np.arange(1, M), size=E - 1, replace=False)) if E > 1 else np.array([], dtype=np.int64)
    cuts = [c | 1 for c in cuts]                     # odd: the next group starts on the second row of a pair
    return np.array(sorted(cuts) + [M], dtype=np.int32)


# ---------------------------------------------------------------------------
# quantizers
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(96, 544), (3, 40, 96), (8, 128), (2080, 96)])
def test_to_mx_pairs_holds_the_rows(gpu, dtype, shape):
    import kernels
    from kernels._common import to_row_pairs
    x = _x(shape, sum(shape), gpu, 3.0, dtype)
    s_r, q_r = kernels.to_mx(x, scale_layout="steps")
    s_p, q_p = kernels.to_mx(x, scale_layout="steps", data_layout="pairs")
    L = shape[-1]
    assert q_p.dtype == torch.float8_e4m3fn
    assert tuple(q_p.shape) == shape[:-2] + (shape[-2] // 2, 2, -(-L // 64), 64)
    assert torch.equal(s_p, s_r)
    rows, pad = _rows_of(q_p, L)
    assert torch.equal(rows, _u8(q_r))
    assert not pad.any()
    assert torch.equal(_u8(to_row_pairs(q_r)).reshape(rows.shape[:-1] + (-1,)),
                       _u8(q_p).reshape(rows.shape[:-1] + (-1,)))


@pytest.mark.parametrize("shape", [(96, 544), (3, 40, 96), (8, 128), (2080, 96)])
def test_to_mx_e2m1_quads_hold_the_rows(gpu, shape):
    import kernels
    from kernels._common import to_row_quads
    fp4 = torch.float4_e2m1fn_x2
    x = _x(shape, sum(shape) + 3, gpu, 3.0)
    s_r, q_r = kernels.to_mx(x, elem_dtype=fp4, scale_layout="steps")
    s_q, q_q = kernels.to_mx(x, elem_dtype=fp4, scale_layout="steps", data_layout="quads")
    Lb = shape[-1] // 2
    assert q_q.dtype == fp4
    assert tuple(q_q.shape) == shape[:-2] + (shape[-2] // 4, 4, -(-Lb // 32), 32)
    assert torch.equal(s_q, s_r)
    *b, G, four, S, P = q_q.shape
    r = _u8(q_q).reshape(tuple(b) + (4 * G, 32 * S))
    assert torch.equal(r[..., :Lb], _u8(q_r))
    assert not r[..., Lb:].any()
    assert torch.equal(_u8(to_row_quads(q_r)).reshape(r.shape), r)
    # byte k of row r at (r/4) 4 ld + (k/32) 128 + (r%4) 32 + k%32 of the storage
    if len(shape) == 2:
        R, ld = shape[0], 32 * S
        flat = torch.as_strided(_u8(q_q), (R * ld,), (1,)).cpu().numpy()
        rr, kk = np.meshgrid(np.arange(R), np.arange(Lb), indexing="ij")
        np.testing.assert_array_equal(flat[(rr // 4) * 4 * ld + (kk // 32) * 128 + (rr % 4) * 32 + kk % 32],
                                      _u8(q_r).cpu().numpy())


def test_pair_storage_matches_documented_offsets(gpu):
    """Byte k of row r at (r/2) 2 ld + (k/64) 128 + (r%2) 64 + k%64 of the
    storage (the formula of include/mxgg.h), pad bytes zero."""
    import kernels
    R, L = 6, 96
    x = _x((R, L), 5, gpu, 2.0)
    _, q_r = kernels.to_mx(x)
    _, q_p = kernels.to_mx(x, data_layout="pairs")
    ld = 128
    flat = torch.as_strided(_u8(q_p), (R // 2 * 2 * ld,), (1,)).cpu().numpy()
    rows = _u8(q_r).cpu().numpy()
    r, k = np.meshgrid(np.arange(R), np.arange(ld), indexing="ij")
    at = (r // 2) * 2 * ld + (k // 64) * 128 + (r % 2) * 64 + k % 64
    np.testing.assert_array_equal(flat[at[:, :L]], rows)
    assert not flat[at[:, L:]].any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2080, 256), (96, 544), (2, 160, 96), (64, 32)])
def test_to_mx_both_and_dim0_pairs_hold_the_rows(gpu, dtype, shape):
    import kernels
    x = _x(shape, sum(shape) + 7, gpu, 3.0, dtype)
    (s_r, q_r), (s_c, q_c) = kernels.to_mx_both(x, scale_layout="steps")
    (t_r, p_r), (t_c, p_c) = kernels.to_mx_both(x, scale_layout="steps", data_layout="pairs")
    R, C = shape[-2:]
    assert torch.equal(t_r, s_r) and torch.equal(t_c, s_c)
    for q, p, L in ((q_r, p_r, C), (q_c, p_c, R)):
        rows, pad = _rows_of(p, L)
        assert torch.equal(rows, _u8(q))
        assert not pad.any()
    if x.dim() == 2:
        s_d, q_d = kernels.to_mx_dim0(x, scale_layout="steps", data_layout="pairs")
        assert torch.equal(s_d, s_c)
        rows, pad = _rows_of(q_d, R)
        assert torch.equal(rows, _u8(q_c)) and not pad.any()


def test_pairs_need_e4m3_and_even_rows(gpu):
    import kernels
    with pytest.raises(ValueError):
        kernels.to_mx(_x((3, 64), 1, gpu), data_layout="pairs")
    with pytest.raises(ValueError):
        kernels.to_mx(_x((4, 64), 1, gpu), elem_dtype=torch.float4_e2m1fn_x2, data_layout="pairs")
    with pytest.raises(ValueError):
        kernels.to_mx(_x((4, 64), 1, gpu), data_layout="quads")
    with pytest.raises(ValueError):
        kernels.to_mx(_x((6, 64), 1, gpu), elem_dtype=torch.float4_e2m1fn_x2, data_layout="quads")
    with pytest.raises(ValueError):
        kernels.to_mx(_x((4, 64), 1, gpu), data_layout="cols")


# ---------------------------------------------------------------------------
# forward / dgrad
# ---------------------------------------------------------------------------

def _fwd_all_layouts(gpu, E, M, N, K, offs, seed, out_dtype=torch.bfloat16, fp4=False):
    """Forward with A / B row-major and in row pairs: every layout's valid
    rows equal the row-major call's bit for bit."""
    import kernels
    from kernels._common import to_row_pairs
    a = _x((M, K), seed, gpu)
    w = _x((E, N, K), seed + 1, gpu, 0.05)
    sa, qa = kernels.to_mx(a, scale_layout="steps")
    fp = torch.float4_e2m1fn_x2 if fp4 else torch.float8_e4m3fn
    sw, qw = kernels.to_mx(w, elem_dtype=fp, scale_layout="steps")
    o = torch.tensor(offs, dtype=torch.int32, device=gpu)
    rows = int(offs[-1])
    ref = kernels.triton_mxfp8_grouped_mm(qa, qw, sa, sw, o, out_dtype=out_dtype)[:rows]
    pa = to_row_pairs(qa)
    cases = {"A pairs": (pa, qw)}
    if fp4:
        from kernels._common import to_row_quads
        _, qq = kernels.to_mx(w, elem_dtype=fp, scale_layout="steps", data_layout="quads")
        assert torch.equal(_u8(to_row_quads(qw)).reshape(-1), _u8(qq).reshape(-1))
        cases.update({"B quads": (qa, qq), "both": (pa, qq)})
    else:
        pw = to_row_pairs(qw)
        cases.update({"B pairs": (qa, pw), "both": (pa, pw)})
    for what, (x_, w_) in cases.items():
        got = kernels.triton_mxfp8_grouped_mm(x_, w_, sa, sw, o, out_dtype=out_dtype)[:rows]
        assert torch.equal(got.view(torch.uint8), ref.view(torch.uint8)), f"{what}: E={E} M={M} N={N} K={K}"
    return ref


@pytest.mark.parametrize("case", [
    (4, 4096, 512, 1024, "odd"),          # odd group starts: shifted pairs
    (2, 512, 256, 512, "odd"),            # small problem: 128 x 128 tiles
    (1, 512, 512, 8192, "even"),          # a lone round split along K
    (3, 1000, 320, 1056, "odd"),          # K % 64 == 32, partial row and column tiles
    (1, 2080, 2048, 2048, "even"),        # one GPU's share under 8-way expert parallelism
    (16, 16640, 256, 2048, "odd"),        # many groups, 256-wide N
], ids=lambda c: "E{}_M{}_N{}_K{}_{}".format(*c))
def test_fwd_pairs_bitwise(gpu, case):
    import random
    E, M, N, K, kind = case
    offs = _odd_offs(E, M, E + M) if kind == "odd" else O.generate_jagged_offs(E, M, 32, rng=random.Random(E * 7 + N))
    _fwd_all_layouts(gpu, E, M, N, K, offs, seed=M + K)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_fwd_pairs_other_outputs(gpu, out_dtype):
    _fwd_all_layouts(gpu, 3, 1536, 384, 768, _odd_offs(3, 1536, 9), seed=4, out_dtype=out_dtype)


def test_fwd_pairs_beside_e2m1_weight(gpu):
    _fwd_all_layouts(gpu, 4, 2048, 512, 1024, _odd_offs(4, 2048, 3), seed=11, fp4=True)
    _fwd_all_layouts(gpu, 3, 1000, 324, 1056, _odd_offs(3, 1000, 5), seed=12, fp4=True)   # K/2 % 32 == 16, N % 256


def test_fwd_e2m1_quads_config5(gpu):
    """BASELINE config 5 (e4m3 x e2m1, E=8, M=16640, N=8192, K=5120) at full size."""
    import random
    offs = O.generate_jagged_offs(8, M_TOKENS, 32, rng=random.Random(4))
    _fwd_all_layouts(gpu, 8, M_TOKENS, 8192, 5120, offs, seed=5, fp4=True)


def test_fwd_pairs_need_step_scales(gpu):
    import kernels
    from kernels._common import to_row_pairs
    a = _x((64, 128), 1, gpu)
    w = _x((2, 64, 128), 2, gpu)
    sa, qa = kernels.to_mx(a)
    sw, qw = kernels.to_mx(w)
    o = torch.tensor([32, 64], dtype=torch.int32, device=gpu)
    with pytest.raises(TypeError):
        kernels.triton_mxfp8_grouped_mm(to_row_pairs(qa), qw, sa, sw, o)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "E{}_N{}_K{}".format(*s))
def test_sweep_fwd_pairs(gpu, shape):
    """Every benchmark forward shape at 16640 tokens: both operands in row
    pairs give the row-major bits."""
    import random
    E, N, K = shape
    offs = O.generate_jagged_offs(E, M_TOKENS, 32, rng=random.Random(E * 131 + N + K))
    _fwd_all_layouts(gpu, E, M_TOKENS, N, K, offs, seed=E + N + K)


# ---------------------------------------------------------------------------
# forward on plain scales: the e4m3 weight staged in row pairs by the call
# ---------------------------------------------------------------------------

def _staged_call(qa, sa, qw, sw, offs_t, out_dtype, ws_bytes):
    from kernels import _lib
    lib = _lib.load()
    M, K = qa.shape
    E, N = qw.shape[0], qw.shape[1]
    a, a_s, b, b_s = _u8(qa), _u8(sa), _u8(qw), _u8(sw)
    code = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}[out_dtype]
    out = torch.full((M, N), float("nan"), dtype=out_dtype, device=qa.device)
    ws = torch.full((ws_bytes,), 0xA5, dtype=torch.uint8, device=qa.device)
    print(f"fwd staged E={E} M={M} N={N} K={K} out={out_dtype} ws={ws_bytes}", flush=True)
    _lib.check(lib.mxgg_grouped_mm(a.data_ptr(), a.stride(0), a_s.data_ptr(), a_s.stride(0),
                                   b.data_ptr(), 0, b.stride(1), b.stride(0),
                                   b_s.data_ptr(), b_s.stride(1), b_s.stride(0),
                                   offs_t.data_ptr(), E, M, N, K, out.data_ptr(), code, out.stride(0),
                                   0, 0, 0, 0, ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return out, ws


@pytest.mark.parametrize("case", [
    (1, 8192, 512, 4096, "even", torch.bfloat16),     # smallest staged shape: 32 steps, a lone round split
    (1, 8192, 384, 4128, "odd", torch.bfloat16),      # K % 64 == 32: the staged rows' zero pad
    (2, 16384, 640, 8192, "odd", torch.float32),      # two experts, partial column tile, f32 out
    (1, 12000, 256, 5120, "odd", torch.float16),      # tail rows unrouted, f16 out
    (1, 8192, 8192, 2048, "odd", torch.bfloat16),     # N = 8192: A staged as well
    (4, 8192, 8192, 2080, "odd", torch.bfloat16),     # A staged alone (E > M / 8192), K % 64 == 32
], ids=lambda c: "E{}_M{}_N{}_K{}_{}".format(*c[:5]))
def test_fwd_staged_weight_bitwise(gpu, case):
    """mxgg_grouped_mm given mxgg_grouped_mm_staging_size more workspace
    copies an e4m3 weight (and, at N >= 8192, A) into row pairs at the end of
    the workspace (the documented row-pair byte order, zero pad) and returns
    the bits of the call without staging and of the step-scale call on
    row-major data."""
    import random
    import kernels
    from kernels import _lib
    E, M, N, K, kind, out_dtype = case
    lib = _lib.load()
    stage = lib.mxgg_grouped_mm_staging_size(E, M, N, K, _lib.FMT_E4M3)
    ldp = (K + 63) // 64 * 64
    stage_b = E * N * ldp + 256 if E * 8192 <= M and (K >= 4096 or (K >= 2048 and N >= 4096)) else 0
    stage_a = M * ldp + 256 if N >= 8192 and K >= 2048 and M % 2 == 0 and M * N * K > 6e10 else 0
    assert stage == stage_b + stage_a > 0
    offs = _odd_offs(E, M - 100, E + K) if kind == "odd" else \
        O.generate_jagged_offs(E, M, 32, rng=random.Random(E * 7 + N))
    o = torch.tensor(offs, dtype=torch.int32, device=gpu)
    a = _x((M, K), M + K, gpu)
    w = _x((E, N, K), M + K + 1, gpu, 0.05)
    sa, qa = kernels.to_mx(a)
    sw, qw = kernels.to_mx(w)
    full = lib.mxgg_grouped_mm_workspace_size(E, M, N, K)
    plain, ws0 = _staged_call(qa, sa, qw, sw, o, out_dtype, full)
    staged, ws = _staged_call(qa, sa, qw, sw, o, out_dtype, full + stage)
    rows = int(offs[-1])
    assert torch.equal(staged[:rows].view(torch.uint8), plain[:rows].view(torch.uint8))
    ssa, _ = kernels.to_mx(a, scale_layout="steps")
    ssw, _ = kernels.to_mx(w, scale_layout="steps")
    steps = kernels.triton_mxfp8_grouped_mm(qa, qw, ssa, ssw, o, out_dtype=out_dtype)
    assert torch.equal(staged[:rows].view(torch.uint8), steps[:rows].view(torch.uint8))
    # the staged copies after the partial-tile room the plain call had, each
    # 256-byte aligned: the weight at the end, A before it
    end = ws.data_ptr() + full + stage
    if stage_b:
        dst = (end - stage_b + 255) // 256 * 256 - ws.data_ptr()
        want = torch.zeros((E, N, ldp), dtype=torch.uint8, device=gpu)
        want[..., :K] = _u8(qw)
        want = want.view(E, N // 2, 2, ldp // 64, 64).permute(0, 1, 3, 2, 4).reshape(-1)
        assert torch.equal(ws[dst:dst + want.numel()], want)
        # the recommended size alone stages nothing: no copy of the weight where
        # staging out of the partial room would have put it
        d0 = (ws0.data_ptr() + full - stage_b + 255) // 256 * 256 - ws0.data_ptr()
        if d0 >= 0:
            assert not torch.equal(ws0[d0:d0 + want.numel()], want)
    if stage_a:
        dst = (end - stage_b - stage_a + 255) // 256 * 256 - ws.data_ptr()
        want = torch.zeros((M, ldp), dtype=torch.uint8, device=gpu)
        want[:, :K] = _u8(qa)
        want = want.view(M // 2, 2, ldp // 64, 64).permute(0, 2, 1, 3).reshape(-1)
        assert torch.equal(ws[dst:dst + want.numel()], want)


def test_fwd_staged_activations_beside_e2m1_weight(gpu):
    """With an e2m1 weight (not staged) and N >= 8192, A alone is staged in
    row pairs: same bits as the unstaged call, staged bytes as documented."""
    import kernels
    from kernels import _lib
    lib = _lib.load()
    E, M, N, K = 2, 4096, 8192, 2080
    stage = lib.mxgg_grouped_mm_staging_size(E, M, N, K, _lib.FMT_E2M1)
    ldp = (K + 63) // 64 * 64
    assert stage == M * ldp + 256
    offs = _odd_offs(E, M - 40, 17)
    o = torch.tensor(offs, dtype=torch.int32, device=gpu)
    a = _x((M, K), 31, gpu)
    w = _x((E, N, K), 32, gpu, 0.05)
    sa, qa = kernels.to_mx(a)
    sw, qw = kernels.to_mx(w, elem_dtype=torch.float4_e2m1fn_x2)
    full = lib.mxgg_grouped_mm_workspace_size(E, M, N, K)
    outs, wss = [], []
    for ws_bytes in (full, full + stage):
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
        print(f"fwd e2m1 staged E={E} M={M} N={N} K={K} ws={ws_bytes}", flush=True)
        _lib.check(lib.mxgg_grouped_mm(_u8(qa).data_ptr(), qa.stride(0), _u8(sa).data_ptr(), sa.stride(0),
                                       _u8(qw).data_ptr(), _lib.FMT_E2M1, qw.stride(1), qw.stride(0),
                                       _u8(sw).data_ptr(), sw.stride(1), sw.stride(0), o.data_ptr(), E, M, N, K,
                                       out.data_ptr(), 0, out.stride(0), 0, 0, 0, 0, ws.data_ptr(), ws_bytes,
                                       torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        outs.append(out)
        wss.append(ws)
    rows = int(offs[-1])
    assert torch.equal(outs[1][:rows].view(torch.uint8), outs[0][:rows].view(torch.uint8))
    ws = wss[1]
    dst = (ws.data_ptr() + full + 255) // 256 * 256 - ws.data_ptr()
    want = torch.zeros((M, ldp), dtype=torch.uint8, device=gpu)
    want[:, :K] = _u8(qa)
    want = want.view(M // 2, 2, ldp // 64, 64).permute(0, 2, 1, 3).reshape(-1)
    assert torch.equal(ws[dst:dst + want.numel()], want)


@pytest.mark.parametrize("L,ld", [(5120, 5120 + 192), (3072, 3072 + 192), (6144, 6144 + 192), (4096, 4096),
                                  (8192, 8192), (2080, 2112)])
def test_pair_stride_padded_at_bad_line_counts(gpu, L, ld):
    """Row pairs of rows spanning a multiple of 8 cache lines that is not a
    power of two get 192 unread bytes more per row in their stride
    (_common._row_group_ld); the bytes sit at the documented offsets with
    that ld, and the view still spans the row rounded up to 64."""
    import kernels
    from kernels._common import _pair_geometry
    R = 4
    x = _x((R, L), 7, gpu, 2.0)
    _, q_r = kernels.to_mx(x)
    _, q_p = kernels.to_mx(x, data_layout="pairs")
    rows_, padded, got_ld = _pair_geometry(q_p, 0)
    assert (rows_, padded, got_ld) == (R, (L + 63) // 64 * 64, ld)
    flat = torch.as_strided(_u8(q_p), (R // 2 * 2 * ld,), (1,)).cpu().numpy()
    r, k = np.meshgrid(np.arange(R), np.arange(L), indexing="ij")
    at = (r // 2) * 2 * ld + (k // 64) * 128 + (r % 2) * 64 + k % 64
    np.testing.assert_array_equal(flat[at], _u8(q_r).cpu().numpy())


def test_drop_in_staging_opt_out(gpu, monkeypatch):
    """MXGG_STAGING=0 drops the staging room from the drop-in calls' workspace
    (forward and wgrad at staged benchmark shapes): the same bits."""
    import random
    import kernels
    E, N, K = 1, 2048, 8192
    offs = O.generate_jagged_offs(E, M_TOKENS, 32, rng=random.Random(4))
    o = torch.tensor(offs, dtype=torch.int32, device=gpu)
    a = _x((M_TOKENS, K), 31, gpu)
    w = _x((E, N, K), 32, gpu, 0.05)
    sa, qa = kernels.to_mx(a)
    sw, qw = kernels.to_mx(w)
    sg, qg = kernels.to_mx_dim0(_x((M_TOKENS, N), 33, gpu))
    si, qi = kernels.to_mx_dim0(a)
    staged = kernels.triton_mxfp8_grouped_mm(qa, qw, sa, sw, o)
    staged_w = kernels.triton_mxfp8_wgrad(qg, sg, qi, si, o)
    monkeypatch.setenv("MXGG_STAGING", "0")
    plain = kernels.triton_mxfp8_grouped_mm(qa, qw, sa, sw, o)
    plain_w = kernels.triton_mxfp8_wgrad(qg, sg, qi, si, o)
    assert torch.equal(staged.view(torch.uint8), plain.view(torch.uint8))
    assert torch.equal(staged_w.view(torch.uint8), plain_w.view(torch.uint8))


def test_fwd_drop_in_stages_the_weight(gpu):
    """The Python drop-in call on plain scales asks for the staging room
    (benchmark shape E=1, N=2048, K=8192): same bits as the step-scale call."""
    import random
    import kernels
    E, N, K = 1, 2048, 8192
    offs = O.generate_jagged_offs(E, M_TOKENS, 32, rng=random.Random(3))
    o = torch.tensor(offs, dtype=torch.int32, device=gpu)
    a = _x((M_TOKENS, K), 21, gpu)
    w = _x((E, N, K), 22, gpu, 0.05)
    sa, qa = kernels.to_mx(a)
    sw, qw = kernels.to_mx(w)
    ssa, _ = kernels.to_mx(a, scale_layout="steps")
    ssw, _ = kernels.to_mx(w, scale_layout="steps")
    got = kernels.triton_mxfp8_grouped_mm(qa, qw, sa, sw, o)
    ref = kernels.triton_mxfp8_grouped_mm(qa, qw, ssa, ssw, o)
    assert torch.equal(got.view(torch.uint8), ref.view(torch.uint8))


# ---------------------------------------------------------------------------
# wgrad
# ---------------------------------------------------------------------------

def _wgrad_all_layouts(gpu, E, M, N, K, offs, seed, out_dtype=torch.bfloat16, quantizer_pairs=False):
    import kernels
    from kernels._common import to_row_pairs
    go = _x((M, N), seed, gpu, 0.5)
    ia = _x((M, K), seed + 1, gpu)
    sg, qg = kernels.to_mx_dim0(go, scale_layout="steps")      # (N, M) along M
    si, qi = kernels.to_mx_dim0(ia, scale_layout="steps")      # (K, M) along M
    o = torch.tensor(offs, dtype=torch.int32, device=gpu)
    ref = kernels.triton_mxfp8_wgrad(qg, sg, qi, si, o, out_dtype=out_dtype)
    if quantizer_pairs:
        _, pg = kernels.to_mx_dim0(go, scale_layout="steps", data_layout="pairs")
        _, pi = kernels.to_mx_dim0(ia, scale_layout="steps", data_layout="pairs")
    else:
        pg, pi = to_row_pairs(qg), to_row_pairs(qi)
    for what, (g_, i_) in {"go pairs": (pg, qi), "ia pairs": (qg, pi), "both": (pg, pi)}.items():
        got = kernels.triton_mxfp8_wgrad(g_, sg, i_, si, o, out_dtype=out_dtype)
        assert torch.equal(got.view(torch.uint8), ref.view(torch.uint8)), f"{what}: E={E} M={M} N={N} K={K}"
    return ref


@pytest.mark.parametrize("case", [
    (4, 2080, 512, 768, "odd"),           # 2080 tokens (rows padded to 2112), bounds off the 16 grid
    (1, 16384, 256, 256, "even"),         # E = 1, few tiles: cut along the tokens
    (3, 1056, 320, 192, "odd"),           # partial tiles in N and K
    (80, 38048, 256, 256, "even"),        # more groups than the wave holds: device-planned split
    (1, 2080, 2048, 2048, "even"),        # one GPU's share under 8-way expert parallelism
], ids=lambda c: "E{}_M{}_N{}_K{}_{}".format(*c))
def test_wgrad_pairs_bitwise(gpu, case):
    import random
    E, M, N, K, kind = case
    offs = _odd_offs(E, M, E + N) if kind == "odd" else O.generate_jagged_offs(E, M, 32, rng=random.Random(E + M))
    _wgrad_all_layouts(gpu, E, M, N, K, offs, seed=N + K)


def _wgrad_plain_call(qg, sg, qi, si, offs_t, out_dtype, ws_bytes):
    from kernels import _lib
    lib = _lib.load()
    N, M = qg.shape
    K = qi.shape[0]
    E = offs_t.numel()
    g, gs, i, is_ = _u8(qg), _u8(sg), _u8(qi), _u8(si)
    code = {torch.bfloat16: 0, torch.float32: 2}[out_dtype]
    out = torch.full((E, N, K), float("nan"), dtype=out_dtype, device=qg.device)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=qg.device)
    print(f"wgrad staged E={E} M={M} N={N} K={K} out={out_dtype} ws={ws_bytes}", flush=True)
    _lib.check(lib.mxgg_wgrad(g.data_ptr(), g.stride(0), gs.data_ptr(), gs.stride(0), i.data_ptr(), i.stride(0),
                              is_.data_ptr(), is_.stride(0), offs_t.data_ptr(), E, M, N, K, out.data_ptr(), code,
                              ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return out, ws


def _pairs_bytes(q, rows, L, dev):
    """Row-pair bytes of a row-major (rows, L) e4m3 operand, per the header's formula."""
    ldp = (L + 63) // 64 * 64
    want = torch.zeros((rows, ldp), dtype=torch.uint8, device=dev)
    want[:, :L] = _u8(q)
    return want.view(rows // 2, 2, ldp // 64, 64).permute(0, 2, 1, 3).reshape(-1)


@pytest.mark.parametrize("case", [
    (8, 4096, 2048, 8192, "odd", torch.bfloat16),      # many small groups, bounds off the 16 grid
    (8, 2080, 5120, 5120, "even", torch.bfloat16),     # 2080 tokens: rows padded to 2112 when staged
    (1, 8192, 8192, 8192, "even", torch.float32),      # E = 1, tiles cut along the tokens, f32 out
], ids=lambda c: "E{}_M{}_N{}_K{}_{}".format(*c[:5]))
def test_wgrad_staged_operands_bitwise(gpu, case):
    """mxgg_wgrad given mxgg_wgrad_staging_size more workspace copies go_t
    and ia_t into row pairs at the end of the workspace (the documented byte
    order, zero pad) and returns the bits of the call without staging and of
    the step-scale call on row-major data."""
    import random
    import kernels
    from kernels import _lib
    E, M, N, K, kind, out_dtype = case
    lib = _lib.load()
    ldp = (M + 63) // 64 * 64
    stage = lib.mxgg_wgrad_staging_size(E, M, N, K)
    assert stage == (N + K) * ldp + 512
    offs = _odd_offs(E, M, E + N) if kind == "odd" else O.generate_jagged_offs(E, M, 32, rng=random.Random(E + M))
    o = torch.tensor(offs, dtype=torch.int32, device=gpu)
    go = _x((M, N), N + K, gpu, 0.5)
    ia = _x((M, K), N + K + 1, gpu)
    sg, qg = kernels.to_mx_dim0(go)
    si, qi = kernels.to_mx_dim0(ia)
    full = lib.mxgg_wgrad_workspace_size(E, M, N, K)
    plain, _ = _wgrad_plain_call(qg, sg, qi, si, o, out_dtype, full)
    staged, ws = _wgrad_plain_call(qg, sg, qi, si, o, out_dtype, full + stage)
    assert torch.equal(staged.view(torch.uint8), plain.view(torch.uint8))
    ssg, _ = kernels.to_mx_dim0(go, scale_layout="steps")
    ssi, _ = kernels.to_mx_dim0(ia, scale_layout="steps")
    steps = kernels.triton_mxfp8_wgrad(qg, ssg, qi, ssi, o, out_dtype=out_dtype)
    assert torch.equal(staged.view(torch.uint8), steps.view(torch.uint8))
    base = ws.data_ptr() + full          # where the partial-tile room of the unstaged call ends
    dg = (base + 255) // 256 * 256 - ws.data_ptr()
    di = (ws.data_ptr() + dg + N * ldp + 255) // 256 * 256 - ws.data_ptr()
    assert torch.equal(ws[dg:dg + N * ldp], _pairs_bytes(qg, N, M, gpu))
    assert torch.equal(ws[di:di + K * ldp], _pairs_bytes(qi, K, M, gpu))


def test_wgrad_pairs_from_the_quantizer_f32(gpu):
    _wgrad_all_layouts(gpu, 5, 2080, 384, 256, _odd_offs(5, 2080, 1), seed=3, out_dtype=torch.float32,
                       quantizer_pairs=True)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "E{}_N{}_K{}".format(*s))
def test_sweep_wgrad_pairs(gpu, shape):
    """Every benchmark wgrad shape at 16640 tokens, row pairs against row-major."""
    import random
    E, N, K = shape
    offs = O.generate_jagged_offs(E, M_TOKENS, 32, rng=random.Random(E * 137 + N + K))
    _wgrad_all_layouts(gpu, E, M_TOKENS, N, K, offs, seed=E * N + K)
