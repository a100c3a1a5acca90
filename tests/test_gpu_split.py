"""GPU parity of the split last round (fp32 partial tiles summed by a second
kernel), called through the C ABI.

A workspace of mxgg_*_workspace_size bytes lets the library cut the tiles of
a partial last round (or of a lone under-filled round) along the reduction;
a workspace holding only the re-laid scales (4 * ceil(red/128) bytes per
operand row) runs every tile whole.  Each case below is sized so that the
split is certain on any device with at least 16 resident workgroups: few
tiles, a reduction of 64 steps of 128 (the split's cost model accepts every
case below with a wide margin; reductions under 32 steps are never split),
and a full workspace.  Both runs are
checked against the oracle (same gates as test_gpu_gemm.py), and repeated
split runs must agree bit for bit (pieces are added in a fixed order).
"""

import numpy as np
import pytest
import torch

from helpers import bits_u8, f32, randn_bf16, seeded_offs
from oracle import mx_oracle as O

pytestmark = pytest.mark.gpu

REL_FRO_TIGHT = 3e-3
CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _u8(t):
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def _fwd_abi(qa, sa, qb, sb, offs_t, b_fmt, out_dtype, ws_bytes, tile=0):
    from kernels import _lib
    lib = _lib.load()
    M, K = qa.shape
    E, N = qb.shape[0], qb.shape[1]
    a, a_s, b, b_s = _u8(qa), _u8(sa), _u8(qb), _u8(sb)
    out = torch.full((M, N), float("nan"), dtype=out_dtype, device=qa.device)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=qa.device)
    print(f"fwd E={E} M={M} N={N} K={K} fmt={b_fmt} out={out_dtype} tile={tile} ws={ws_bytes}", flush=True)
    _lib.check(lib.mxgg_grouped_mm(a.data_ptr(), a.stride(0), a_s.data_ptr(), a_s.stride(0),
                                   b.data_ptr(), b_fmt, b.stride(1), b.stride(0),
                                   b_s.data_ptr(), b_s.stride(1), b_s.stride(0),
                                   offs_t.data_ptr(), E, M, N, K, out.data_ptr(), CODES[out_dtype],
                                   out.stride(0), tile, tile, 0, 0, ws.data_ptr(), ws_bytes,
                                   torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return out


def _fwd_sizes(E, M, N, K):
    from kernels import _lib
    full = _lib.load().mxgg_grouped_mm_workspace_size(E, M, N, K)
    scales = 4 * ((K + 127) // 128) * (M + E * N)
    assert full > scales + 2 * 128 * 128 * 4, "case too small to split"
    return full, scales


@pytest.mark.parametrize("E,M,N,K,fmt,out_dtype,tile", [
    (1, 1024, 512, 8192, "e4m3", torch.bfloat16, 0),     # 8 tiles of 256, 64 steps: one lone round
    (4, 1024, 512, 8224, "e4m3", torch.bfloat16, 128),   # 128x128 tiles, K % 128 = 32, jagged groups
    (3, 768, 640, 8256, "e4m3", torch.float32, 0),       # 256x256, K % 128 = 64, ragged N, f32 out
    (2, 512, 384, 8192, "e4m3", torch.float16, 128),     # f16 out
    (4, 1024, 512, 8192, "e2m1", torch.bfloat16, 0),     # fp4 weights
])
def test_fwd_split_matches_whole_tiles(gpu, E, M, N, K, fmt, out_dtype, tile):
    import kernels
    from kernels import _lib
    offs = seeded_offs(E, M, seed=E * 31 + K)
    if E >= 3:
        offs[1] = offs[0]                               # an empty group
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    a = randn_bf16((M, K), 1.0, 7 + K)
    b = randn_bf16((E, N, K), 0.05, 8 + K)
    sa, qa = kernels.to_mx(a.to(gpu))
    if fmt == "e2m1":
        sb, qb = kernels.to_mx(b.to(gpu), elem_dtype=torch.float4_e2m1fn_x2)
        b_fmt = _lib.FMT_E2M1
    else:
        sb, qb = kernels.to_mx(b.to(gpu))
        b_fmt = _lib.FMT_E4M3
    full, scales = _fwd_sizes(E, M, N, K)
    split1 = _fwd_abi(qa, sa, qb, sb, offs_t, b_fmt, out_dtype, full, tile)
    split2 = _fwd_abi(qa, sa, qb, sb, offs_t, b_fmt, out_dtype, full, tile)
    whole = _fwd_abi(qa, sa, qb, sb, offs_t, b_fmt, out_dtype, scales, tile)
    ref = O.grouped_mm(bits_u8(qa), bits_u8(sa), bits_u8(qb), bits_u8(sb), offs,
                       b_elem="e2m1" if fmt == "e2m1" else "e4m3")
    rows = offs[-1]
    assert torch.equal(split1[:rows], split2[:rows])
    for out in (split1, whole):
        o = f32(out)[:rows]
        assert np.isfinite(o).all()
        assert O.rel_fro(ref[:rows], o) <= REL_FRO_TIGHT
    # the two paths differ only in fp32 summation order
    tol = 4e-3 if out_dtype != torch.float32 else 1e-5
    assert O.rel_fro(f32(whole)[:rows], f32(split1)[:rows]) <= tol


def test_fwd_split_tail_full_size(gpu):
    """E=1, M=16640, N=2048, K=8192: 65 x 8 = 520 tiles of 256x256 -- two full
    rounds on 256 CUs and an 8-tile last round cut into pieces.  Against a GPU
    fp32 dequantize -> matmul and against the whole-tile path."""
    import kernels
    from kernels import _lib
    M, N, K = 16640, 2048, 8192
    g = torch.Generator(device=gpu).manual_seed(5)
    a = torch.randn((M, K), device=gpu, generator=g).to(torch.bfloat16)
    b = (torch.randn((1, N, K), device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    sa, qa = kernels.to_mx(a)
    sb, qb = kernels.to_mx(b)
    offs_t = torch.tensor([M], dtype=torch.int32, device=gpu)
    full, scales = _fwd_sizes(1, M, N, K)
    split = _fwd_abi(qa, sa, qb, sb, offs_t, _lib.FMT_E4M3, torch.bfloat16, full)
    whole = _fwd_abi(qa, sa, qb, sb, offs_t, _lib.FMT_E4M3, torch.bfloat16, scales)

    def deq(q, s):
        v = q.float().reshape(*q.shape[:-1], -1, 32)
        return (v * torch.exp2(s.float() - 127).unsqueeze(-1)).reshape(q.shape)

    ref = deq(qa, sa) @ deq(qb, sb)[0].t()
    for out in (split, whole):
        err = (out.float() - ref).norm() / ref.norm()
        assert err.item() <= REL_FRO_TIGHT
    # every tile, split or not, agrees with the whole-tile result to bf16 rounding
    d = (split.float() - whole.float()).abs().amax(dim=1)
    assert (d <= 2.0 ** -6 * whole.float().abs().amax(dim=1).clamp_min(1.0)).all()


# ------------------------------------------------- quarter-tile last round
#
# A reduction under 32 steps is never split; instead, a last round of at most
# P / 4 tiles of 256 x 256 after at most two full rounds runs as 128 x 128
# quarter tiles (quad_dp).  The small cases below have far fewer than P / 4
# tiles (P = resident workgroups, 256 on MI355X), so every tile is quartered;
# quarters compute each output element with the same MFMA sequence as a
# 128 x 128 launch, so the two agree bit for bit.

@pytest.mark.parametrize("E,M,N,K,out_dtype", [
    (3, 992, 300, 1024, torch.bfloat16),      # empty group, partial quarters in rows and columns
    (4, 2048, 512, 2048, torch.float32),      # f32 out
    (2, 608, 256, 128, torch.float16),        # one step, f16 out
])
def test_fwd_quarter_tiles(gpu, E, M, N, K, out_dtype):
    import kernels
    from kernels import _lib
    offs = seeded_offs(E, M, seed=E * 17 + K)
    if E >= 3:
        offs[1] = offs[0]
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    sa, qa = kernels.to_mx(randn_bf16((M, K), 1.0, 3 + K).to(gpu))
    sb, qb = kernels.to_mx(randn_bf16((E, N, K), 0.05, 4 + K).to(gpu))
    full = _lib.load().mxgg_grouped_mm_workspace_size(E, M, N, K)
    quarters = _fwd_abi(qa, sa, qb, sb, offs_t, _lib.FMT_E4M3, out_dtype, full, 256)
    small = _fwd_abi(qa, sa, qb, sb, offs_t, _lib.FMT_E4M3, out_dtype, full, 128)
    rows = offs[-1]
    assert torch.equal(quarters[:rows], small[:rows])
    ref = O.grouped_mm(bits_u8(qa), bits_u8(sa), bits_u8(qb), bits_u8(sb), offs)
    o = f32(quarters)[:rows]
    assert np.isfinite(o).all()
    assert O.rel_fro(ref[:rows], o) <= REL_FRO_TIGHT


@pytest.mark.parametrize("E", [1, 8])
def test_fwd_quarter_tail_full_size(gpu, E):
    """M=16640, N=K=2048 with 256 x 256 tiles: 520 (E=1) or about 550 (E=8,
    jagged) tiles -- two full rounds on 256 CUs and a last round of quarter
    tiles.  Against a GPU fp32 dequantize -> matmul per group."""
    import kernels
    from kernels import _lib
    M, N, K = 16640, 2048, 2048
    g = torch.Generator(device=gpu).manual_seed(11 + E)
    a = torch.randn((M, K), device=gpu, generator=g).to(torch.bfloat16)
    b = (torch.randn((E, N, K), device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    sa, qa = kernels.to_mx(a)
    sb, qb = kernels.to_mx(b)
    offs = seeded_offs(E, M, seed=E) if E > 1 else [M]
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    full = _lib.load().mxgg_grouped_mm_workspace_size(E, M, N, K)
    out = _fwd_abi(qa, sa, qb, sb, offs_t, _lib.FMT_E4M3, torch.bfloat16, full, 256)

    def deq(q, s):
        v = q.float().reshape(*q.shape[:-1], -1, 32)
        return (v * torch.exp2(s.float() - 127).unsqueeze(-1)).reshape(q.shape)

    da, db = deq(qa, sa), deq(qb, sb)
    lo = 0
    for e, hi in enumerate(offs):
        if hi > lo:
            ref = da[lo:hi] @ db[e].t()
            err = (out[lo:hi].float() - ref).norm() / ref.norm()
            assert err.item() <= REL_FRO_TIGHT, (e, lo, hi, err.item())
        lo = hi


# ---------------------------------------------------------------- wgrad

def _wgrad_abi(qg, sg, qi, si, offs_t, out_dtype, ws_bytes):
    from kernels import _lib
    lib = _lib.load()
    N, M = qg.shape
    K = qi.shape[0]
    E = offs_t.numel()
    go, go_s, ia, ia_s = _u8(qg), _u8(sg), _u8(qi), _u8(si)
    out = torch.full((E, N, K), float("nan"), dtype=out_dtype, device=qg.device)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=qg.device)
    print(f"wgrad E={E} M={M} N={N} K={K} out={out_dtype} ws={ws_bytes}", flush=True)
    _lib.check(lib.mxgg_wgrad(go.data_ptr(), go.stride(0), go_s.data_ptr(), go_s.stride(0),
                              ia.data_ptr(), ia.stride(0), ia_s.data_ptr(), ia_s.stride(0),
                              offs_t.data_ptr(), E, M, N, K, out.data_ptr(), CODES[out_dtype],
                              ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return out


def _many_groups():
    """80 groups (a fifth empty, sizes off the 32 grid) with one long group:
    E > 64 takes the device plan's single piece count, set by the longest
    group, for a lone under-filled round of 80 tiles."""
    rng = np.random.default_rng(2080)
    sizes = rng.integers(0, 600, 80)
    sizes[rng.choice(80, 16, replace=False)] = 0
    sizes[37] = 20000
    offs = np.cumsum(sizes)
    return [int(v) for v in offs], int(offs[-1] + 31) // 32 * 32 + 64


@pytest.mark.parametrize("E,M,N,K,offs,out_dtype", [
    (1, 8192, 512, 512, [8192], torch.bfloat16),               # 4 tiles, 64 steps -> 8 pieces
    (3, 24576, 320, 288, [0, 8000, 24576], torch.bfloat16),    # empty group, bounds not at 128
    (2, 16384, 256, 512, [8160, 16384], torch.float32),        # f32 out (bf16-rounded values)
    (2, 16384, 512, 512, [1024, 16384], torch.bfloat16),       # 8 vs 120 steps: per-group piece counts
    (1, 16640, 2560, 3584, [16640], torch.bfloat16),           # 140 tiles > P / 2: pieces in two rounds
    (80, _many_groups()[1], 256, 256, _many_groups()[0], torch.bfloat16),   # E > 64: one piece count
])
def test_wgrad_split_matches_whole_tiles(gpu, E, M, N, K, offs, out_dtype):
    import kernels
    from kernels import _lib
    lib = _lib.load()
    go = randn_bf16((M, N), 1.0, 60 + E)
    ia = randn_bf16((M, K), 1.0, 61 + E)
    sg, qg = kernels.to_mx_dim0(go.to(gpu))
    si, qi = kernels.to_mx_dim0(ia.to(gpu))
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    full = lib.mxgg_wgrad_workspace_size(E, M, N, K)
    scales = 4 * ((M + 127) // 128) * (N + K)
    assert full > scales + 2 * 256 * 256 * 4, "case too small to split"
    split1 = _wgrad_abi(qg, sg, qi, si, offs_t, out_dtype, full)
    split2 = _wgrad_abi(qg, sg, qi, si, offs_t, out_dtype, full)
    whole = _wgrad_abi(qg, sg, qi, si, offs_t, out_dtype, scales)
    assert torch.equal(split1, split2)
    ref = O.wgrad(bits_u8(qg), bits_u8(sg), bits_u8(qi), bits_u8(si), offs)
    for out in (split1, whole):
        o = f32(out)
        assert np.isfinite(o).all()
        assert O.rel_fro(ref, o) <= REL_FRO_TIGHT
        if out_dtype == torch.float32:
            c = out.cpu()
            assert torch.equal(c, c.to(torch.bfloat16).float())
    for e in range(E):
        if offs[e] == (offs[e - 1] if e else 0):
            assert (f32(split1)[e] == 0).all()
    assert O.rel_fro(f32(whole), f32(split1)) <= (4e-3 if out_dtype != torch.float32 else 1e-5)
