"""Seeded randomized GPU parity for the grouped GEMMs, through the drop-in
operators, against the oracle (same gates as test_gpu_gemm.py).

Each case draws its shape, group offsets, launch tile, output dtype and
operand layout from its own seed, so a failure names a reproducible case
(the parameters are printed before the GPU runs it).  Forward: any E up to
13 with empty groups, rows past the last offset, group bounds anywhere, N
not a multiple of anything, K any multiple of 32; the operands row-major on
plain scales (the drop-in path, which may stage them in row pairs) or
quantized straight into the native layout (step-major scales, row pairs).
Forward K is a multiple of 512 in about 2 of 5 cases (plain scales read by the
GEMM itself), any multiple of 32 otherwise (re-laid scales).  wgrad: group
bounds off the 32-token grid, empty groups, ragged N and K
(operands from the fused transposing quantizer where their rows allow it,
else from to_mx of the transposed copy, as the reference quantizes them).
Sizes keep the fp64 oracle near a second per case.  Row-major against row
pairs: the XLine main loop and the one-stage one give the same bits on random
256 x 256 launches (no oracle needed: the two layouts are the same numbers).
"""

import random

import numpy as np
import pytest
import torch

from helpers import bits_u8, f32, randn_bf16
from oracle import mx_oracle as O

pytestmark = pytest.mark.gpu

REL_FRO_TIGHT = 3e-3


def _ends(rng: random.Random, E: int, M: int, mult: int, cover: bool) -> list:
    """E non-decreasing group end offsets in [0, M], multiples of `mult`; the
    last is M when `cover`, else possibly short of it (unrouted rows)."""
    top = M // mult
    last = top if cover else rng.randrange(0, top + 1)
    cuts = sorted(rng.randrange(0, last + 1) for _ in range(E - 1))
    return [c * mult for c in cuts] + [last * mult]


@pytest.mark.parametrize("case", range(24))
def test_fwd_fuzz(gpu, case):
    import kernels
    rng = random.Random(7001 + case)
    E = rng.choice([1, 1, 2, 3, 4, 5, 8, 13])
    M = 2 * rng.randrange(1, 640)                 # even: the native layout keeps rows in pairs
    N = rng.randrange(1, 720)
    # K a multiple of 512 in 2 of 5 cases: scale rows of 16-byte multiples, which these small calls read
    # directly (plain-scale kernels, no re-layout launch); other K go through the re-layout
    K = 512 * rng.randrange(1, 5) if rng.random() < 0.4 else 32 * rng.randrange(1, 48)
    offs = _ends(rng, E, M, rng.choice([1, 16, 32]), cover=rng.random() < 0.75)
    tile = rng.choice([None, (128, 128), (256, 256)])
    out_dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    native = rng.random() < 0.3 and N % 2 == 0   # row pairs of the weight need an even N
    print(f"fwd fuzz case {case}: E={E} M={M} N={N} K={K} offs={offs} tile={tile} out={out_dtype} "
          f"native={native}", flush=True)
    a = randn_bf16((M, K), 1.0, 100 + case)
    b = randn_bf16((E, N, K), 0.05, 200 + case)
    sa, qa = kernels.to_mx(a.to(gpu))
    sb, qb = kernels.to_mx(b.to(gpu))
    if native:
        lay = {"scale_layout": "steps", "data_layout": "pairs"}
        xa, pa = kernels.to_mx(a.to(gpu), **lay)
        xb, pb = kernels.to_mx(b.to(gpu), **lay)
        args = (pa, pb, xa, xb)
    else:
        args = (qa, qb, sa, sb)
    kw = {} if tile is None else {"BLOCK_M": tile[0], "BLOCK_N": tile[1]}
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    out = kernels.triton_mxfp8_grouped_mm(*args, offs_t, out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    assert out.shape == (M, N) and out.dtype == out_dtype
    rows = offs[-1]
    ref = O.grouped_mm(bits_u8(qa), bits_u8(sa), bits_u8(qb), bits_u8(sb), offs)[:rows]
    o = f32(out)[:rows]
    assert np.isfinite(o).all()
    if rows:
        tol = 1e-4 if out_dtype == torch.float32 else REL_FRO_TIGHT
        assert O.rel_fro(ref, o) <= tol


@pytest.mark.parametrize("case", range(16))
def test_wgrad_fuzz(gpu, case):
    import kernels
    rng = random.Random(9001 + case)
    E = rng.choice([1, 1, 2, 3, 4, 6, 8])
    M = 32 * rng.randrange(1, 96)
    N = rng.randrange(1, 640)
    K = rng.randrange(1, 640)
    offs = _ends(rng, E, M, rng.choice([1, 16, 32]), cover=rng.random() < 0.8)
    out_dtype = rng.choice([torch.bfloat16, torch.bfloat16, torch.float16, torch.float32])
    print(f"wgrad fuzz case {case}: E={E} M={M} N={N} K={K} offs={offs} out={out_dtype}", flush=True)
    go = randn_bf16((M, N), 1.0, 300 + case)
    ia = randn_bf16((M, K), 1.0, 400 + case)

    def dim0(x):
        # the fused transposing quantizer needs 16-byte rows of x; the
        # reference's own path (kernels/backward.py:232-243) takes any width
        if x.shape[1] % 8 == 0:
            return kernels.to_mx_dim0(x.to(gpu))
        return kernels.to_mx(x.to(gpu).t().contiguous())

    sg, qg = dim0(go)
    si, qi = dim0(ia)
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    out = kernels.triton_mxfp8_wgrad(qg, sg, qi, si, offs_t, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert out.shape == (E, N, K) and out.dtype == out_dtype
    ref = O.wgrad(bits_u8(qg), bits_u8(sg), bits_u8(qi), bits_u8(si), offs)
    o = f32(out)
    assert np.isfinite(o).all()
    prev = 0
    for e, end in enumerate(offs):
        if end == prev:
            assert (o[e] == 0).all(), f"group {e} is empty"
        prev = end
    # every output holds the bf16-rounded product (kernels/backward.py:101-104)
    want = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.astype(np.float32)))
    if np.abs(want).sum():
        assert O.rel_fro(want.astype(np.float64), o) <= REL_FRO_TIGHT


@pytest.mark.parametrize("case", range(24))
def test_row_major_matches_row_pairs_fuzz(gpu, case):
    """256 x 256 tiles on random shapes: row-major operands (the XLine main
    loop, the X operand in two-stage LDS slots) give, bit for bit, the
    one-stage kernel's result on the same operands in row pairs, for the
    forward and the wgrad (odd stage counts, ragged groups, split calls)."""
    import kernels
    rng = random.Random(9100 + case)
    E = rng.choice([1, 1, 2, 3, 4, 8])
    M = 2 * rng.randrange(64, 4096)
    N = 8 * rng.randrange(16, 384)
    K = 32 * rng.randrange(4, 160)
    offs = _ends(rng, E, M, 1, cover=rng.random() < 0.75)
    Mw = 32 * max(1, M // 32)
    offs_w = _ends(rng, E, Mw, 1, cover=True)
    print(f"rows/pairs fuzz case {case}: E={E} M={M} N={N} K={K} offs={offs} wgrad M={Mw} offs={offs_w}",
          flush=True)
    lay = {"scale_layout": "steps", "data_layout": "pairs"}
    a = randn_bf16((M, K), 1.0, 500 + case).to(gpu)
    w = randn_bf16((E, N, K), 0.05, 600 + case).to(gpu)
    sa, qa = kernels.to_mx(a, scale_layout="steps")
    sw, qw = kernels.to_mx(w, scale_layout="steps")
    _, pa = kernels.to_mx(a, **lay)
    _, pw = kernels.to_mx(w, **lay)
    o = torch.tensor(offs, dtype=torch.int32, device=gpu)
    rows = offs[-1]
    kw = {"BLOCK_M": 256, "BLOCK_N": 256}
    got = kernels.triton_mxfp8_grouped_mm(qa, qw, sa, sw, o, **kw)[:rows]
    ref = kernels.triton_mxfp8_grouped_mm(pa, pw, sa, sw, o, **kw)[:rows]
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), "forward"
    go = randn_bf16((Mw, N), 1.0, 700 + case).to(gpu)
    ia = randn_bf16((Mw, K), 1.0, 800 + case).to(gpu)
    sg, qg = kernels.to_mx_dim0(go, scale_layout="steps")
    si, qi = kernels.to_mx_dim0(ia, scale_layout="steps")
    _, pg = kernels.to_mx_dim0(go, **lay)
    _, pi = kernels.to_mx_dim0(ia, **lay)
    ow = torch.tensor(offs_w, dtype=torch.int32, device=gpu)
    got = kernels.triton_mxfp8_wgrad(qg, sg, qi, si, ow)
    ref = kernels.triton_mxfp8_wgrad(pg, sg, pi, si, ow)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), "wgrad"
