"""GPU parity for the grouped GEMMs against the oracle's dequantize -> fp64
per-group matmul (kernels/forward.py:81-294, kernels/backward.py:31-215).

Tolerances: relative Frobenius error <= 1e-2 vs the
dequantize-then-matmul reference, and SQNR >= 27 dB vs the unquantized bf16
product.  The kernel's only rounding is fp32 accumulation plus one bf16
store, so the observed error is ~1e-3; the tests also check that bound at
3e-3 so a real regression (a dropped block, a wrong scale) cannot hide
under the loose gate.
"""

import numpy as np
import pytest
import torch

from helpers import bits_u8, bits_u16, f32, randn_bf16, seeded_offs
from oracle import mx_oracle as O

pytestmark = pytest.mark.gpu

REL_FRO_GATE = 1e-2
REL_FRO_TIGHT = 3e-3
SQNR_GATE = 27.0


def _quant(x_bf16_cpu, gpu):
    import kernels
    s, q = kernels.to_mx(x_bf16_cpu.to(gpu))
    return s, q


def _fwd_case(E, M, N, K, offs, gpu, seed=0, std_b=0.02, out_dtype=torch.bfloat16, **kw):
    import kernels
    a = randn_bf16((M, K), 1.0, seed)
    b = randn_bf16((E, N, K), std_b, seed + 1)
    sa, qa = _quant(a, gpu)
    sb, qb = _quant(b, gpu)
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    out = kernels.triton_mxfp8_grouped_mm(qa, qb, sa, sb, offs_t, out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    ref = O.grouped_mm(bits_u8(qa), bits_u8(sa), bits_u8(qb), bits_u8(sb), offs)
    hp = O.grouped_mm_hp(O.bf16_bits_to_f32(bits_u16(a)), O.bf16_bits_to_f32(bits_u16(b)), offs)
    return f32(out), ref, hp


def _assert_close(out, ref, hp=None, rows=None, tight=True):
    if rows is not None:
        out, ref = out[:rows], ref[:rows]
        hp = hp[:rows] if hp is not None else None
    assert np.isfinite(out).all()
    err = O.rel_fro(ref, out)
    assert err <= REL_FRO_GATE, err
    if tight:
        assert err <= REL_FRO_TIGHT, err
    if hp is not None:
        assert O.sqnr_db(hp, out) >= SQNR_GATE


@pytest.mark.parametrize("E,M,N,K,std_b", [(4, 1024, 512, 512, 0.02),      # BASELINE cfg1
                                           (1, 1024, 1024, 1024, 1.0),    # test_correctness.py:70-73
                                           (8, 1024, 4096, 2048, 1.0),
                                           (4, 1024, 2048, 2048, 1.0),
                                           (8, 2048, 5120, 2048, 1.0)])
def test_fwd_reference_shapes(gpu, E, M, N, K, std_b):
    """cfg1 plus the four shapes of the reference's correctness script."""
    offs = seeded_offs(E, M, seed=E * 1000 + N)
    out, ref, hp = _fwd_case(E, M, N, K, offs, gpu, seed=E + K, std_b=std_b)
    _assert_close(out, ref, hp)


def test_fwd_golden_cfg1(gpu):
    """Committed cfg1 fixture: GPU output vs the frozen oracle output."""
    import os
    import kernels
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1.npz"))
    dev = gpu
    qa = torch.from_numpy(z["a_q"]).to(dev).view(torch.float8_e4m3fn)
    qb = torch.from_numpy(z["b_q"]).to(dev).view(torch.float8_e4m3fn)
    sa = torch.from_numpy(z["a_scales"]).to(dev)
    sb = torch.from_numpy(z["b_scales"]).to(dev)
    offs = torch.from_numpy(z["offs"]).to(dev)
    out = kernels.triton_mxfp8_grouped_mm(qa, qb, sa, sb, offs)
    torch.cuda.synchronize()
    ref = O.bf16_bits_to_f32(z["out_bf16"])
    got = f32(out)
    assert O.rel_fro(ref, got) <= REL_FRO_TIGHT
    # bf16 outputs: at most a 1-ulp difference from the frozen bf16 result
    d = np.abs(bits_u16(out).astype(np.int32) - z["out_bf16"].astype(np.int32))
    assert (d <= 1).mean() > 0.99


@pytest.mark.parametrize("tile", [(128, 128), (256, 256)])
@pytest.mark.parametrize("offs", [[0, 32, 32, 300 - 300 % 32, 640],   # empty groups, ragged
                                  [640, 640, 640],                      # all rows in group 0
                                  [7, 100, 333, 640]])                  # not multiples of 32
def test_fwd_ragged_and_empty_groups(gpu, tile, offs):
    E, M, N, K = len(offs), 640, 384, 256
    out, ref, hp = _fwd_case(E, M, N, K, offs, gpu, seed=3, std_b=1.0,
                             BLOCK_M=tile[0], BLOCK_N=tile[1])
    _assert_close(out, ref, hp, rows=offs[-1])


def test_fwd_rows_past_last_offset_untouched(gpu):
    import kernels
    E, M, N, K = 2, 512, 256, 128
    offs = [96, 320]
    a = randn_bf16((M, K), 1.0, 1)
    b = randn_bf16((E, N, K), 1.0, 2)
    sa, qa = _quant(a, gpu)
    sb, qb = _quant(b, gpu)
    out = kernels.triton_mxfp8_grouped_mm(qa, qb, sa, sb, torch.tensor(offs, dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    ref = O.grouped_mm(bits_u8(qa), bits_u8(sa), bits_u8(qb), bits_u8(sb), offs)
    _assert_close(f32(out), ref, rows=320)


def test_fwd_empty_reduction_gives_zeros(gpu):
    """K = 0 through the C ABI, on an output pre-filled with NaN: every routed
    row becomes zero (the ring runs one stage wholly outside the reduction,
    whose MFMAs start the accumulators from zero), rows past offs[-1] stay."""
    from kernels import _lib
    lib = _lib.load()
    M, N, E = 96, 64, 2
    dummy = torch.zeros(4096, dtype=torch.uint8, device=gpu)   # holds every row range the calls name
    offs = torch.tensor([40, 80], dtype=torch.int32, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    # step-major scales; plain scales with 1-byte rows (re-layout path); plain scales with 16-byte rows (read by the
    # GEMM itself: 96 * 16 and 2 * 64 * 16 bytes, inside the dummy buffer)
    for mode in ("steps", "plain", "plain16"):
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        p = dummy.data_ptr()
        if mode == "steps":
            rc = lib.mxgg_grouped_mm_steps(p, 16, p, p, 0, 16, 16 * N, p, offs.data_ptr(), E, M, N, 0,
                                           out.data_ptr(), 0, N, 0, 0, 0, 0, 0, None, 0, stream)
        else:
            ls = 1 if mode == "plain" else 16
            rc = lib.mxgg_grouped_mm(p, 16, p, ls, p, 0, 16, 16 * N, p, ls, ls * N, offs.data_ptr(), E, M, N, 0,
                                     out.data_ptr(), 0, N, 0, 0, 0, 0, None, 0, stream)
        _lib.check(rc)
        torch.cuda.synchronize()
        assert not out[:80].float().abs().sum().item(), mode
        assert out[80:].float().isnan().all(), mode


@pytest.mark.parametrize("N,K", [(200, 96), (33, 160), (4096, 32)])
def test_fwd_odd_shapes(gpu, N, K):
    """N not a multiple of the tile / of 4, K not a multiple of 128 (masked tail)."""
    E, M = 3, 448
    offs = [64, 256, 448]
    out, ref, hp = _fwd_case(E, M, N, K, offs, gpu, seed=N + K, std_b=1.0)
    _assert_close(out, ref, hp)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_fwd_out_dtypes(gpu, out_dtype):
    E, M, N, K = 2, 512, 256, 512
    offs = [192, 512]
    out, ref, hp = _fwd_case(E, M, N, K, offs, gpu, seed=9, std_b=0.1, out_dtype=out_dtype)
    err = O.rel_fro(ref, out)
    # fp32 output: only the MFMA's internal fp32 accumulation differs from fp64
    assert err <= (1e-4 if out_dtype == torch.float32 else 1e-3), err


@pytest.mark.parametrize("gm", [3, 12])
def test_fwd_many_groups(gpu, gm):
    """80 groups, a fifth of them empty, sizes 0..96 rows: the in-kernel tile
    order (groups contiguous, bands of at most GROUP_M m-blocks inside a
    group) scans the groups in two 64-lane passes; every tile must be
    computed exactly once."""
    E, M, N, K = 80, 8192, 384, 256
    rng = np.random.default_rng(80 + gm)
    sizes = rng.integers(1, 4, size=E) * 32
    sizes[rng.choice(E, 16, replace=False)] = 0
    offs = [int(v) for v in np.cumsum(sizes)]
    out, ref, hp = _fwd_case(E, M, N, K, offs, gpu, seed=gm, std_b=1.0, GROUP_M=gm)
    _assert_close(out, ref, hp, rows=offs[-1])


def test_fwd_group_m_xcd_options(gpu):
    E, M, N, K = 3, 1536, 1024, 256
    offs = [512, 1024, 1536]
    outs = []
    for gm, x in ((1, 1), (4, 8), (8, 4), (16, 8)):
        out, ref, _ = _fwd_case(E, M, N, K, offs, gpu, seed=4, GROUP_M=gm, XCD_SWIZZLE=x)
        _assert_close(out, ref)
        outs.append(out)
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])     # schedule never changes the numbers


def test_dgrad_shape(gpu):
    """dgrad = same op with grad_out (M, N) against W^T (E, K, N) quantized along N."""
    import kernels
    E, M, N, K = 4, 1024, 512, 768
    offs = seeded_offs(E, M, seed=21)
    go = randn_bf16((M, N), 1.0, 30)
    w = randn_bf16((E, N, K), 0.02, 31)
    wt = w.transpose(-2, -1).contiguous()            # (E, K, N)
    sg, qg = _quant(go, gpu)
    sw, qw = _quant(wt, gpu)
    out = kernels.triton_mxfp8_grouped_mm(qg, qw, sg, sw, torch.tensor(offs, device=gpu))
    torch.cuda.synchronize()
    ref = O.grouped_mm(bits_u8(qg), bits_u8(sg), bits_u8(qw), bits_u8(sw), offs)
    hp = O.grouped_mm_hp(f32(go), f32(wt), offs)
    _assert_close(f32(out), ref, hp)


def test_fwd_mxfp4_weights(gpu):
    """Mixed e4m3 activations x e2m1 weights (f8f6f4 MFMA with the fp4 B format)."""
    import kernels
    fp4 = torch.float4_e2m1fn_x2
    E, M, N, K = 4, 1024, 512, 512
    offs = seeded_offs(E, M, seed=44)
    a = randn_bf16((M, K), 1.0, 40)
    b = randn_bf16((E, N, K), 0.02, 41)
    sa, qa = _quant(a, gpu)
    sb, qb = kernels.to_mx(b.to(gpu), elem_dtype=fp4)
    out = kernels.triton_mxfp8_grouped_mm(qa, qb, sa, sb, torch.tensor(offs, device=gpu))
    torch.cuda.synchronize()
    ref = O.grouped_mm(bits_u8(qa), bits_u8(sa), bits_u8(qb), bits_u8(sb), offs, b_elem="e2m1")
    _assert_close(f32(out), ref)
    # fp4 weights lose more than fp8 vs bf16; only check it is sane
    hp = O.grouped_mm_hp(f32(a), f32(b), offs)
    assert O.sqnr_db(hp, f32(out)) > 12.0


def test_fwd_full_size_cfg2(gpu):
    """BASELINE config 2 at full size (E=1, M=16640, N=K=2048) against a GPU
    fp32 dequantize -> matmul of the same quantized operands."""
    import kernels
    M, N, K = 16640, 2048, 2048
    g = torch.Generator(device=gpu).manual_seed(1)
    a = torch.randn((M, K), device=gpu, generator=g).to(torch.bfloat16)
    b = (torch.randn((1, N, K), device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    sa, qa = kernels.to_mx(a)
    sb, qb = kernels.to_mx(b)
    out = kernels.triton_mxfp8_grouped_mm(qa, qb, sa, sb, torch.tensor([M], dtype=torch.int32, device=gpu))

    def deq(q, s):
        v = q.float().reshape(*q.shape[:-1], -1, 32)
        return (v * torch.exp2(s.float() - 127).unsqueeze(-1)).reshape(q.shape)

    ref = deq(qa, sa) @ deq(qb, sb)[0].t()
    err = (out.float() - ref).norm() / ref.norm()
    assert err.item() <= REL_FRO_TIGHT
    hp = a.float() @ b[0].float().t()
    sq = 20 * torch.log10(hp.norm() / (hp - out.float()).norm())
    assert sq.item() >= SQNR_GATE


def test_fwd_full_size_cfg5_mxfp4(gpu):
    """BASELINE config 5 at full size: E=8, M=16640, N=8192, K=5120, e4m3
    activations x packed e2m1 weights (jagged groups), against a GPU fp32
    dequantize -> per-group matmul of the same quantized operands.  The e2m1
    codes decode by the OCP MX table (sign bit 3, magnitudes 0 .. 6), element
    2i in the low nibble; that GPU reference is itself pinned to the oracle
    (``grouped_mm(..., b_elem="e2m1")``, fp64) on 256 rows across a group
    boundary x 128 columns, and so is the kernel's output there."""
    import random

    import kernels
    E, M, N, K = 8, 16640, 8192, 5120
    offs = O.generate_jagged_offs(E, M, 32, rng=random.Random(4))
    print(f"cfg5 E={E} M={M} N={N} K={K} offs={offs}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(4)
    a = torch.randn((M, K), device=gpu, generator=g).to(torch.bfloat16)
    b = (torch.randn((E, N, K), device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    sa, qa = kernels.to_mx(a)
    sb, qb = kernels.to_mx(b, elem_dtype=torch.float4_e2m1fn_x2)
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    out = kernels.triton_mxfp8_grouped_mm(qa, qb, sa, sb, offs_t)
    torch.cuda.synchronize()

    lut = torch.tensor([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], device=gpu)
    pb = qb.view(torch.uint8).long()
    wv = torch.stack([lut[pb & 15], lut[pb >> 4]], dim=-1).reshape(E, N, K)
    wd = (wv.reshape(E, N, K // 32, 32) * torch.exp2(sb.view(torch.uint8).float() - 127).unsqueeze(-1)).reshape(E, N, K)
    ad = (qa.float().reshape(M, K // 32, 32) * torch.exp2(sa.view(torch.uint8).float() - 127).unsqueeze(-1)).reshape(M, K)
    del wv
    r0 = max(0, min(int(offs[0]) - 128, M - 256))   # rows r0 .. r0+255 straddle the first group end
    ref_slice = torch.empty((256, 128), device=gpu)
    lo = 0
    err2 = ref2 = 0.0
    hp_err2 = hp2 = 0.0
    for e in range(E):
        hi = offs[e]
        if hi > lo:
            ref = ad[lo:hi] @ wd[e].t()
            o = out[lo:hi].float()
            err2 += (o - ref).square().sum().item()
            ref2 += ref.square().sum().item()
            hp = a[lo:hi].float() @ b[e].float().t()
            hp_err2 += (o - hp).square().sum().item()
            hp2 += hp.square().sum().item()
            s0, s1 = max(lo, r0), min(hi, r0 + 256)
            if s0 < s1:
                ref_slice[s0 - r0:s1 - r0] = ref[s0 - lo:s1 - lo, :128]
        lo = hi
    assert (err2 / ref2) ** 0.5 <= REL_FRO_TIGHT
    so = np.clip(np.asarray(offs, np.int64) - r0, 0, 256)
    ora = O.grouped_mm(bits_u8(qa[r0:r0 + 256]), bits_u8(sa[r0:r0 + 256]), bits_u8(qb[:, :128]),
                       bits_u8(sb[:, :128]), so, b_elem="e2m1")
    assert O.rel_fro(ora, ref_slice.double().cpu().numpy()) <= 1e-4
    assert O.rel_fro(ora, out[r0:r0 + 256, :128].float().cpu().numpy()) <= REL_FRO_TIGHT
    # fp4 weights lose more than fp8 against bf16: a sanity floor only
    assert 10 * torch.log10(torch.tensor(hp2 / hp_err2)).item() > 12.0


# ---------------------------------------------------------------- wgrad

def _wgrad_case(E, M, N, K, offs, gpu, seed=0, out_dtype=torch.bfloat16):
    import kernels
    go = randn_bf16((M, N), 1.0, seed)
    ia = randn_bf16((M, K), 1.0, seed + 1)
    sg, qg = kernels.to_mx_dim0(go.to(gpu))        # (N, M), (N, M/32)
    si, qi = kernels.to_mx_dim0(ia.to(gpu))        # (K, M), (K, M/32)
    out = kernels.triton_mxfp8_wgrad(qg, sg, qi, si, torch.tensor(offs, dtype=torch.int32, device=gpu),
                                     out_dtype=out_dtype)
    torch.cuda.synchronize()
    ref = O.wgrad(bits_u8(qg), bits_u8(sg), bits_u8(qi), bits_u8(si), offs)
    return out, ref, go, ia


@pytest.mark.parametrize("E,M,N,K,block", [
    (2, 16640, 2048, 2048, 128),    # 128 tiles of 256 (half a round, split) -> 512 of 128 fill a round
    (1, 16640, 2048, 2048, 256),    # 64 tiles, split along 130 steps; 256 tiles of 128 would not fill a round
    (1, 2080, 2048, 2048, 128),     # 17 steps: too short to split, 64 tiles of 256
    (4, 16640, 2048, 2048, 256),    # 256 tiles: a full round
    (8, 16640, 8192, 8192, 256),
])
def test_wgrad_config_tiles(gpu, E, M, N, K, block):
    """mxgg_wgrad_config on MI355X (256 CUs, one 256 x 256 workgroup each)."""
    import ctypes
    from kernels import _lib
    if torch.cuda.get_device_properties(gpu).multi_processor_count != 256:
        pytest.skip("expected tile choices are for 256 CUs")
    b = ctypes.c_int32(0)
    _lib.check(_lib.load().mxgg_wgrad_config(E, M, N, K, ctypes.byref(b)))
    assert b.value == block


@pytest.mark.parametrize("E,M,N,K", [(4, 1024, 512, 512), (1, 1024, 256, 384), (8, 2048, 512, 256)])
def test_wgrad_random(gpu, E, M, N, K):
    offs = seeded_offs(E, M, seed=M + E)
    out, ref, go, ia = _wgrad_case(E, M, N, K, offs, gpu, seed=E)
    _assert_close(f32(out), ref)
    # vs unquantized bf16 product per group
    g32, i32 = f32(go), f32(ia)
    prev = 0
    hp = np.zeros_like(ref)
    for e, end in enumerate(offs):
        hp[e] = g32[prev:end].T.astype(np.float64) @ i32[prev:end].astype(np.float64)
        prev = end
    assert O.sqnr_db(hp, f32(out)) >= SQNR_GATE


def test_wgrad_empty_and_unaligned_groups(gpu):
    """Empty groups give zeros; group bounds at 32 but not 128 multiples."""
    E, M, N, K = 5, 1024, 320, 288
    offs = [0, 160, 160, 544, 1024]
    out, ref, _, _ = _wgrad_case(E, M, N, K, offs, gpu, seed=12)
    o = f32(out)
    assert (o[0] == 0).all() and (o[2] == 0).all()
    _assert_close(o, ref)


def test_wgrad_fp32_out_is_bf16_rounded(gpu):
    """The reference stores acc.to(bf16) even for out_dtype=float32 (backward.py:103)."""
    E, M, N, K = 2, 512, 256, 256
    offs = [256, 512]
    out, ref, _, _ = _wgrad_case(E, M, N, K, offs, gpu, seed=13, out_dtype=torch.float32)
    assert out.dtype == torch.float32
    o = out.cpu()
    assert torch.equal(o, o.to(torch.bfloat16).float())
    _assert_close(f32(out), ref)


@pytest.mark.parametrize("E,M,N,K,offs", [
    (2, 512, 256, 256, [256, 512]),              # whole tiles, 16-byte rows: the LDS-staged f16 epilogue
    (3, 1024, 320, 200, [100, 600, 1024]),       # K % 8 != 0: the per-element epilogue; bounds off the 32 grid
    (1, 8192, 256, 512, [8192]),                 # E = 1, few tiles: pieces along the tokens and the reduce
])
def test_wgrad_fp16_out_is_bf16_converted(gpu, E, M, N, K, offs):
    """out_dtype=float16: the reference allocates an fp16 output and its store
    converts the bf16-rounded accumulator to it (kernels/backward.py:101-104,
    251).  Bit for bit the same call's bf16 output converted to fp16 (torch's
    RNE cast), on every epilogue path, and within tolerance of the oracle's
    wgrad rounded to bf16 then fp16."""
    out16, ref, _, _ = _wgrad_case(E, M, N, K, offs, gpu, seed=21, out_dtype=torch.float16)
    outb, _, _, _ = _wgrad_case(E, M, N, K, offs, gpu, seed=21, out_dtype=torch.bfloat16)
    assert out16.dtype == torch.float16
    assert torch.equal(out16.view(torch.int16), outb.to(torch.float16).view(torch.int16))
    want = torch.from_numpy(O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32)))).to(torch.float16)
    _assert_close(f32(out16), want.double().numpy())


@pytest.mark.parametrize("M,offs", [(1024, [16, 48, 1000, 1024]),          # 16- but not 32-aligned bounds
                                    (1024, [7, 100, 333, 1024]),           # bounds off the 16 grid
                                    (1024, [3, 10, 10, 517, 1024]),        # two bounds in one 16-chunk, empty group
                                    (1024, [0, 1, 1023, 1024]),            # one-token groups at both ends
                                    (8192, [4100, 8190])])                 # long groups (split plan), tail unrouted
def test_wgrad_any_offsets(gpu, M, offs):
    """Group bounds need not be multiples of 32 (the reference masks tokens by
    group and indexes scales by token // 32, kernels/backward.py:67-98): a
    32-token scale block shared by two groups scales both groups' tokens."""
    E, N, K = len(offs), 320, 288
    out, ref, _, _ = _wgrad_case(E, M, N, K, offs, gpu, seed=len(offs) + M)
    o = f32(out)
    prev = 0
    for e, end in enumerate(offs):
        if end == prev:
            assert (o[e] == 0).all()
        prev = end
    _assert_close(o, ref)


# ---------------------------------------------------------------- routing / schedule

def test_routing_table_kat(gpu):
    from kernels import _lib
    lib = _lib.load()
    offs = torch.tensor([96, 352, 640, 1024], dtype=torch.int32, device=gpu)
    n = lib.mxgg_routing_words(4, 1024, 128)
    out = torch.full((n,), -7, dtype=torch.int32, device=gpu)
    _lib.check(lib.mxgg_build_routing(offs.data_ptr(), 4, 1024, 128, out.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    want = [96, 256, 288, 384, 0, 96, 352, 640, 9,
            0x0, 0x1, 0x10001, 0x2, 0x10002, 0x20002, 0x3, 0x10003, 0x20003, -1, -1]
    assert out.cpu().tolist() == want


@pytest.mark.parametrize("E,M,BM", [(1, 16640, 256), (8, 16640, 256), (8, 16640, 128), (70, 4096, 128),
                                    (200, 8192, 64)])
def test_routing_matches_oracle(gpu, E, M, BM):
    from kernels import _lib
    lib = _lib.load()
    offs = seeded_offs(E, M, seed=E * 7 + BM)
    n = lib.mxgg_routing_words(E, M, BM)
    out = torch.empty((n,), dtype=torch.int32, device=gpu)
    _lib.check(lib.mxgg_build_routing(torch.tensor(offs, device=gpu).data_ptr(), E, M, BM, out.data_ptr(),
                                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ref, _ = O.routing_table(offs, M, BM)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)


def _order_offs(case):
    """Offsets for the tile-order test: seeded jagged groups, or (for
    'many') 80 groups with a fifth of them empty and sizes off the 32 grid."""
    kind, E, M = case
    if kind == "jagged":
        return seeded_offs(E, M, seed=E * 31 + M)
    rng = np.random.default_rng(E)
    sizes = rng.integers(1, 6, size=E) * 37
    sizes[rng.choice(E, E // 5, replace=False)] = 0
    return np.cumsum(sizes).astype(np.int32)


@pytest.mark.parametrize("case", [("jagged", 8, 16640), ("jagged", 1, 16640), ("jagged", 3, 1024), ("many", 80, 9000)])
@pytest.mark.parametrize("BM", [256, 128])
@pytest.mark.parametrize("GM,X", [(1, 1), (3, 8), (12, 8), (12, 1)])
def test_tile_schedule_matches_oracle(gpu, case, BM, GM, X):
    """The forward kernel's own tile lookup (fwd_tile: XCD swizzle, then
    expert-aligned bands), run for every program of the launch grid, equals
    the oracle's restatement, which the CPU tests pin to cover every output
    element exactly once."""
    from kernels import _lib
    lib = _lib.load()
    offs = _order_offs(case)
    E, M = len(offs), case[2]
    for N in (2048, 700):
        progs = lib.mxgg_schedule_programs(E, M, N, BM, BM)
        out = torch.full((5 * progs,), -7, dtype=torch.int32, device=gpu)
        _lib.check(lib.mxgg_tile_schedule(torch.tensor(offs, device=gpu).data_ptr(), E, M, N, BM, BM, GM, X,
                                          out.data_ptr(), torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        ref = O.fwd_tile_order(offs, M, N, BM, BM, GM, X)
        np.testing.assert_array_equal(out.cpu().numpy().reshape(-1, 5), ref)
