"""GPU parity: the HIP MX quantizer is bit-exact with the oracle's ``to_mx``
(utils.py:67-105), including every special case the FLOOR recipe has."""

import numpy as np
import pytest
import torch

from helpers import bits_u8, bits_u16, randn_bf16
from oracle import mx_oracle as O

pytestmark = pytest.mark.gpu


def _check_rows(x_cpu: torch.Tensor, gpu, elem="e4m3"):
    import kernels
    src = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[x_cpu.dtype]
    if src == "bf16":
        ref_s, ref_q = O.to_mx(bits_u16(x_cpu), src="bf16", elem=elem)
    else:
        ref_s, ref_q = O.to_mx(x_cpu.numpy(), src=src, elem=elem)
    fp4 = getattr(torch, "float4_e2m1fn_x2")
    s, q = kernels.to_mx(x_cpu.to(gpu), elem_dtype=torch.float8_e4m3fn if elem == "e4m3" else fp4)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(s), ref_s)
    np.testing.assert_array_equal(bits_u8(q), ref_q)


@pytest.mark.parametrize("shape,std", [((1024, 512), 1.0), ((3, 7, 96), 0.02), ((4, 512, 512), 0.02),
                                       ((1, 32), 5.0), ((257, 160), 1e-3)])
def test_quant_rows_random_bf16(gpu, shape, std):
    _check_rows(randn_bf16(shape, std, seed=sum(shape)), gpu)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_quant_rows_other_dtypes(gpu, dtype):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn((96, 256), generator=g) * 3).to(dtype)
    _check_rows(x, gpu)


def _special_blocks() -> torch.Tensor:
    """Rows of 32-element blocks exercising every branch of the FLOOR recipe."""
    rows = []
    f = np.float32
    z = np.zeros(32, f)
    rows.append(z.copy())                                  # all zero -> scale 0
    r = z.copy(); r[3] = -0.0; rows.append(r)              # negative zero kept
    for amax in (1.0, 448.0, 464.0, 480.0, 511.0, 512.0, 2.0 ** -118, 2.0 ** -119,
                 2.0 ** -126, 2.0 ** -130, 1.5 * 2.0 ** 100, 3.0e38):
        r = np.linspace(-amax, amax, 32).astype(f); rows.append(r)
    r = z.copy(); r[5] = np.nan; r[6] = 1.0; rows.append(r)           # NaN block
    r = z.copy(); r[5] = -np.nan; r[6] = 3.0; rows.append(r)
    r = z.copy(); r[1] = np.inf; r[2] = -7.0; rows.append(r)          # inf block
    r = z.copy(); r[1] = -np.inf; r[2] = np.inf; rows.append(r)
    r = np.full(32, 2.0 ** -133, f); r[0] = 2.0 ** -127; rows.append(r)  # denormal-only
    # ties: values that land exactly half-way on the e4m3 grid after scaling
    r = (np.arange(32, dtype=f) * 0.5 + 256.0).astype(f); rows.append(r)
    r = (np.arange(32, dtype=f) / 64.0).astype(f); rows.append(r)
    return torch.from_numpy(np.stack(rows).astype(np.float32))


def test_quant_special_values(gpu):
    x = _special_blocks()
    _check_rows(x.to(torch.bfloat16), gpu)
    _check_rows(x, gpu)


def test_quant_every_bf16_pattern(gpu):
    """All 65536 bf16 bit patterns, shuffled into blocks, scale 2**k copies."""
    u = np.arange(65536, dtype=np.uint16)
    rng = np.random.default_rng(3)
    for _ in range(2):
        p = rng.permutation(u)
        x = torch.from_numpy(p.view(np.int16).copy()).view(torch.bfloat16).reshape(512, 128)
        _check_rows(x, gpu)


@pytest.mark.parametrize("shape,std", [((1024, 512), 1.0), ((64, 96), 0.02)])
def test_quant_rows_e2m1(gpu, shape, std):
    _check_rows(randn_bf16(shape, std, seed=11), gpu, elem="e2m1")


def test_quant_e2m1_special(gpu):
    _check_rows(_special_blocks().to(torch.bfloat16), gpu, elem="e2m1")


@pytest.mark.parametrize("shape", [(1024, 512), (64, 256), (2048, 40)])
def test_quant_dim0_matches_transposed_rows(gpu, shape):
    import kernels
    x = randn_bf16(shape, 1.0, seed=5)
    ref_s, ref_q = O.to_mx(bits_u16(x.t().contiguous()), src="bf16")
    s, q = kernels.to_mx_dim0(x.to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(s), ref_s)
    np.testing.assert_array_equal(bits_u8(q), ref_q)


def test_quant_dim0_special(gpu):
    import kernels
    x = _special_blocks().t().contiguous().to(torch.bfloat16)   # (32, rows)
    pad = torch.zeros((32, 8 - x.shape[1] % 8), dtype=torch.bfloat16) if x.shape[1] % 8 else None
    if pad is not None:
        x = torch.cat([x, pad], dim=1)
    ref_s, ref_q = O.to_mx(bits_u16(x.t().contiguous()), src="bf16")
    s, q = kernels.to_mx_dim0(x.to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(s), ref_s)
    np.testing.assert_array_equal(bits_u8(q), ref_q)


def test_quant_golden_cfg1(gpu):
    """Replays the committed cfg1 fixture (tests/golden/cfg1.npz)."""
    import os
    import kernels
    path = os.path.join(os.path.dirname(__file__), "golden", "cfg1.npz")
    z = np.load(path)
    a = torch.from_numpy(z["a_bf16"].view(np.int16)).view(torch.bfloat16).to(gpu)
    b = torch.from_numpy(z["b_bf16"].view(np.int16)).view(torch.bfloat16).to(gpu)
    sa, qa = kernels.to_mx(a)
    sb, qb = kernels.to_mx(b)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits_u8(sa), z["a_scales"])
    np.testing.assert_array_equal(bits_u8(qa), z["a_q"])
    np.testing.assert_array_equal(bits_u8(sb), z["b_scales"])
    np.testing.assert_array_equal(bits_u8(qb), z["b_q"])


@pytest.mark.parametrize("shape", [(2080, 256), (96, 544), (4096, 160)])
def test_quant_outputs_on_128_byte_rows(gpu, shape):
    """to_mx_dim0 / to_mx_both return rows on the 128-byte grid (a strided
    view when the row length is not a multiple of 128) holding exactly the
    bytes of the contiguous results, and the weight-gradient GEMM gives the
    same bits on them as on contiguous copies."""
    import kernels
    R, C = shape
    x = randn_bf16((R, C), 1.0, R + C).to(gpu)
    s_d, q_d = kernels.to_mx_dim0(x)
    (s_r, q_r), (s_c, q_c) = kernels.to_mx_both(x)
    for q, length in ((q_d, R), (q_c, R), (q_r, C)):
        assert q.stride(-1) == 1 and q.stride(-2) % 128 == 0 and q.stride(-2) - length < 128
        assert q.data_ptr() % 128 == 0
    rs, rq = O.to_mx(bits_u16(x.cpu()), src="bf16")
    cs, cq = O.to_mx(bits_u16(x.cpu().t().contiguous()), src="bf16")
    np.testing.assert_array_equal(bits_u8(q_r), rq)
    np.testing.assert_array_equal(bits_u8(q_c), cq)
    np.testing.assert_array_equal(bits_u8(q_d), cq)
    np.testing.assert_array_equal(bits_u8(s_c), cs)
    # the GEMM reads the strided operands: same bits as on contiguous copies
    offs = torch.tensor([R // 2 // 32 * 32, R], dtype=torch.int32, device=gpu)
    w_strided = kernels.triton_mxfp8_wgrad(q_c, s_c, q_d, s_d, offs)
    w_contig = kernels.triton_mxfp8_wgrad(q_c.contiguous(), s_c, q_d.contiguous(), s_d, offs)
    torch.cuda.synchronize()
    assert torch.equal(w_strided.view(torch.int16), w_contig.view(torch.int16))
