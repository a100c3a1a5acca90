"""Step-major scales end to end (the layout the GEMM kernels read, written by
the quantizers with ``scale_layout="steps"``):

* the quantizers' step-major scales equal ``oracle.step_major`` of the
  oracle's own ``to_mx`` scales byte for byte (bytes past a row's last block
  127), and their data bytes equal the plain-layout call's; ``to_mx_both``
  and ``to_mx_dim0`` are compared with ``oracle.to_mx`` of the transposed
  source directly, special values included;
* the GEMMs given step-major scales (``mxgg_grouped_mm_steps`` /
  ``mxgg_wgrad_steps``, no per-call re-layout) return the same bits as the
  plain-scale entry points, including launches whose last round is split.
"""

import numpy as np
import pytest
import torch

from helpers import bits_u8, bits_u16, seeded_offs
from oracle import mx_oracle as O

pytestmark = pytest.mark.gpu


def _src(shape, dtype, seed, dev, specials=True):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=g) * 3).to(dtype)
    if specials:
        f = x.view(-1)
        f[3], f[70], f[200], f[300], f[301], f[400], f[-1] = (float("inf"), float("-inf"), float("nan"), 0.0, -0.0,
                                                             1e-30, 3.0e4)
    return x.to(dev)


def _oracle_to_mx(x_cpu, elem="e4m3"):
    if x_cpu.dtype == torch.bfloat16:
        return O.to_mx(bits_u16(x_cpu), src="bf16", elem=elem)
    return O.to_mx(x_cpu.float().numpy(), src="f32", elem=elem)


def _words(t):
    return t.contiguous().view(torch.int32).cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(96, 544), (3, 40, 96), (7, 256)])
@pytest.mark.parametrize("elem", ["e4m3", "e2m1"])
def test_to_mx_steps_matches_oracle(gpu, dtype, shape, elem):
    import kernels
    fp = torch.float8_e4m3fn if elem == "e4m3" else torch.float4_e2m1fn_x2
    x = _src(shape, dtype, sum(shape), gpu)
    ss, qs = kernels.to_mx(x, elem_dtype=fp, scale_layout="steps")
    sp, qp = kernels.to_mx(x, elem_dtype=fp)
    assert ss.dtype == torch.int32 and tuple(ss.shape) == shape[:-2] + (-(-shape[-1] // 128), shape[-2])
    assert torch.equal(qs.view(torch.uint8), qp.view(torch.uint8))
    rs, rq = _oracle_to_mx(x.cpu(), elem)
    np.testing.assert_array_equal(bits_u8(qs), rq)
    np.testing.assert_array_equal(_words(ss), O.step_major(rs))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(64, 320), (3, 96, 544), (160, 32)])
def test_to_mx_both_and_dim0_match_oracle(gpu, dtype, shape):
    """Both layouts of to_mx_both, plain and step-major, and to_mx_dim0, against
    oracle.to_mx of the source and of its transpose."""
    import kernels
    x = _src(shape, dtype, sum(shape) + 1, gpu)
    xs = x if x.dim() == 3 else x.unsqueeze(0)
    (s_r, q_r), (s_c, q_c) = kernels.to_mx_both(x)
    (t_r, w_r), (t_c, w_c) = kernels.to_mx_both(x, scale_layout="steps")
    if x.dim() == 2:
        s_r, q_r, s_c, q_c, t_r, w_r, t_c, w_c = (v.unsqueeze(0) for v in (s_r, q_r, s_c, q_c, t_r, w_r, t_c, w_c))
    for b in range(xs.shape[0]):
        xb = xs[b].cpu()
        rs, rq = _oracle_to_mx(xb)
        cs, cq = _oracle_to_mx(xb.t().contiguous())
        np.testing.assert_array_equal(bits_u8(s_r[b]), rs)
        np.testing.assert_array_equal(bits_u8(q_r[b]), rq)
        np.testing.assert_array_equal(bits_u8(s_c[b]), cs)
        np.testing.assert_array_equal(bits_u8(q_c[b]), cq)
        np.testing.assert_array_equal(_words(t_r[b]), O.step_major(rs))
        np.testing.assert_array_equal(_words(t_c[b]), O.step_major(cs))
        assert torch.equal(w_r[b].view(torch.uint8), q_r[b].view(torch.uint8))
        assert torch.equal(w_c[b].view(torch.uint8), q_c[b].view(torch.uint8))
        if dtype != torch.float16:
            d_s, d_q = kernels.to_mx_dim0(xs[b], scale_layout="steps")
            np.testing.assert_array_equal(_words(d_s), O.step_major(cs))
            np.testing.assert_array_equal(bits_u8(d_q), cq)


def _fwd_both_ways(gpu, E, M, N, K, offs, fp4=False, out_dtype=torch.bfloat16, seed=0, tile=None):
    import kernels
    g = torch.Generator(device=gpu).manual_seed(seed)
    a = torch.randn((M, K), device=gpu, generator=g).to(torch.bfloat16)
    w = (torch.randn((E, N, K), device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    fp = torch.float4_e2m1fn_x2 if fp4 else torch.float8_e4m3fn
    sa, qa = kernels.to_mx(a)
    sw, qw = kernels.to_mx(w, elem_dtype=fp)
    ta, _ = kernels.to_mx(a, scale_layout="steps")
    tw, _ = kernels.to_mx(w, elem_dtype=fp, scale_layout="steps")
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    kw = {} if tile is None else {"BLOCK_M": tile, "BLOCK_N": tile}
    plain = kernels.triton_mxfp8_grouped_mm(qa, qw, sa, sw, offs_t, out_dtype=out_dtype, **kw)
    steps = kernels.triton_mxfp8_grouped_mm(qa, qw, ta, tw, offs_t, out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    return plain, steps, (qa, sa, qw, sw)


# Calls that stage nothing, of at most 1.2e11 flop, on plain to_mx scales
# whose rows are 16-byte multiples (K a multiple of 512), run the plain-scale
# kernels (no re-layout launch); the others re-lay the scales step-major.
# The cases cover both, and every case compares with the step-major call bit
# for bit.
@pytest.mark.parametrize("E,M,N,K,fp4,out_dtype,tile", [
    (4, 1024, 512, 544, False, torch.bfloat16, None),      # K % 128 = 32: a padded last step (re-layout)
    (3, 448, 200, 96, False, torch.float32, None),         # ragged N, unaligned output path (re-layout)
    (4, 1024, 512, 512, True, torch.bfloat16, None),       # plain: e2m1 weights, one partial 8-step piece
    (8, 16640, 2048, 5120, False, torch.bfloat16, None),   # re-layout: sweep shape whose last round is split
    (1, 16640, 2048, 2048, False, torch.bfloat16, None),   # re-layout: quarter-tile last round
    (1, 2080, 2048, 2048, False, torch.bfloat16, 128),     # plain: 128 x 128 tiles (expert-parallel shard)
    (2, 4096, 512, 4608, False, torch.float16, None),      # plain: 36 steps, the last 8-step piece half used
    (2, 4096, 1024, 4608, False, torch.bfloat16, 256),     # plain: a lone round of 64-68 tiles, split in
                                                           # pieces that start inside an 8-step piece
    (1, 2304, 7936, 2048, False, torch.bfloat16, 256),     # plain: 279 tiles, a quarter-tile last round
])
def test_fwd_steps_bit_identical(gpu, E, M, N, K, fp4, out_dtype, tile):
    offs = seeded_offs(E, M - M % 32, seed=E + N)
    print(f"fwd steps E={E} M={M} N={N} K={K} fp4={fp4} tile={tile} offs={list(offs)}", flush=True)
    plain, steps, (qa, sa, qw, sw) = _fwd_both_ways(gpu, E, M, N, K, offs, fp4, out_dtype, seed=K, tile=tile)
    rows = int(offs[-1])
    assert torch.equal(plain[:rows].view(torch.int16 if out_dtype != torch.float32 else torch.int32),
                       steps[:rows].view(torch.int16 if out_dtype != torch.float32 else torch.int32))
    if M <= 1024:
        ref = O.grouped_mm(bits_u8(qa), bits_u8(sa), bits_u8(qw), bits_u8(sw), offs,
                           b_elem="e2m1" if fp4 else "e4m3")
        assert O.rel_fro(ref[:rows], steps[:rows].float().cpu().numpy()) <= 3e-3


def test_fwd_plain_scales_padded_strides(gpu):
    """Plain scales in row- and expert-padded buffers (strides 16 bytes past
    the row and 48 bytes past the expert): the same bits as contiguous ones."""
    import kernels
    E, M, N, K = 3, 1536, 640, 2048
    offs = seeded_offs(E, M, seed=5)
    print(f"fwd padded plain scales E={E} M={M} N={N} K={K} offs={list(offs)}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(11)
    a = torch.randn((M, K), device=gpu, generator=g).to(torch.bfloat16)
    w = (torch.randn((E, N, K), device=gpu, generator=g) * 0.02).to(torch.bfloat16)
    sa, qa = kernels.to_mx(a)
    sw, qw = kernels.to_mx(w)
    nb = K // 32
    pa = torch.full((M, nb + 16), 255, dtype=torch.uint8, device=gpu)
    pa[:, :nb] = sa.view(torch.uint8)
    pw = torch.full((E * (N * (nb + 16) + 48),), 255, dtype=torch.uint8, device=gpu)
    pw_v = torch.as_strided(pw, (E, N, nb), (N * (nb + 16) + 48, nb + 16, 1))
    pw_v.copy_(sw.view(torch.uint8))
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    want = kernels.triton_mxfp8_grouped_mm(qa, qw, sa, sw, offs_t)
    got = kernels.triton_mxfp8_grouped_mm(qa, qw, pa[:, :nb].view(sa.dtype), pw_v.view(sw.dtype), offs_t)
    torch.cuda.synchronize()
    assert torch.equal(want.view(torch.int16), got.view(torch.int16))


@pytest.mark.parametrize("E,M,N,K,offs", [
    (4, 1024, 512, 288, None),
    (3, 1024, 320, 288, [7, 500, 1024]),             # bounds off the 16 grid (edge chunks)
    (2, 8192, 256, 256, None),                       # lone under-filled round: device-planned pieces
    (1, 16640, 2048, 2048, None),                    # host-planned split
])
def test_wgrad_steps_bit_identical(gpu, E, M, N, K, offs):
    import kernels
    offs = seeded_offs(E, M, seed=E + K) if offs is None else np.asarray(offs, np.int32)
    print(f"wgrad steps E={E} M={M} N={N} K={K} offs={list(offs)}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(M + N)
    go = torch.randn((M, N), device=gpu, generator=g).to(torch.bfloat16)
    ia = torch.randn((M, K), device=gpu, generator=g).to(torch.bfloat16)
    sg, qg = kernels.to_mx_dim0(go)
    si, qi = kernels.to_mx_dim0(ia)
    tg, _ = kernels.to_mx_dim0(go, scale_layout="steps")
    ti, _ = kernels.to_mx_dim0(ia, scale_layout="steps")
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    plain = kernels.triton_mxfp8_wgrad(qg, sg, qi, si, offs_t)
    steps = kernels.triton_mxfp8_wgrad(qg, tg, qi, ti, offs_t)
    torch.cuda.synchronize()
    assert torch.equal(plain.view(torch.int16), steps.view(torch.int16))
    if M <= 1024:
        ref = O.wgrad(bits_u8(qg), bits_u8(sg), bits_u8(qi), bits_u8(si), offs)
        assert O.rel_fro(ref, steps.float().cpu().numpy()) <= 3e-3


def test_layouts_must_match(gpu):
    """One plain and one step-major scale tensor is an error, not a silent mix."""
    import kernels
    a = torch.randn((256, 256), device=gpu).to(torch.bfloat16)
    sa, qa = kernels.to_mx(a)
    ta, _ = kernels.to_mx(a, scale_layout="steps")
    w = a.view(1, 256, 256)
    sw, qw = kernels.to_mx(w)
    with pytest.raises(TypeError):
        kernels.triton_mxfp8_grouped_mm(qa, qw, ta, sw, torch.tensor([256], dtype=torch.int32, device=gpu))
