"""GPU checks of the fused both-ways quantizer and the MXFP8 MoE layer.

* ``to_mx_both`` (``mxgg_quantize_mx_both``) must equal ``to_mx`` and
  ``to_mx_dim0`` byte for byte (both are pinned to the oracle in
  test_gpu_quant.py), for bf16 / f16 / f32 sources with specials, ragged
  tile edges and a batch dimension.
* ``kernels.moe.mxfp8_grouped_mm``: its forward and both gradients must equal,
  bit for bit, the direct GEMM calls on operands quantized along the axes the
  reference's callers use (fwd along K; dgrad grad_out along N and W^T (E, K,
  N) along N, kernels/forward.py:485-488; wgrad along M, kernels/backward.py:
  232-243), and stay within 26 dB SQNR of the fp64 product of the unquantized
  operands (the forward within the reference's 27 dB gate, test_correctness.py:26).
"""

import numpy as np
import pytest
import torch

from helpers import bits_u8, bits_u16, f32, randn_bf16, seeded_offs
from oracle import mx_oracle as O

pytestmark = pytest.mark.gpu


def _with_specials(x):
    flat = x.view(-1)
    flat[3] = float("inf")
    flat[70] = float("-inf")
    flat[200] = float("nan")
    flat[300] = 0.0
    flat[301] = -0.0
    flat[400] = 1e-30
    flat[-1] = 3.0e4
    return x


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", [(64, 320), (3, 96, 544), (32, 32)])
def test_to_mx_both_matches_separate_quantizers(gpu, dtype, shape):
    import kernels
    g = torch.Generator().manual_seed(sum(shape))
    x = _with_specials((torch.randn(shape, generator=g) * 3).to(dtype)).to(gpu)
    (s_r, q_r), (s_c, q_c) = kernels.to_mx_both(x)
    xs = x if x.dim() == 3 else x.unsqueeze(0)
    for b in range(xs.shape[0]):
        rs, rq = kernels.to_mx(xs[b])
        cs, cq = kernels.to_mx_dim0(xs[b])
        gr = (s_r if x.dim() == 3 else s_r.unsqueeze(0))[b]
        gq = (q_r if x.dim() == 3 else q_r.unsqueeze(0))[b]
        hc = (s_c if x.dim() == 3 else s_c.unsqueeze(0))[b]
        hq = (q_c if x.dim() == 3 else q_c.unsqueeze(0))[b]
        assert torch.equal(gr, rs) and torch.equal(gq.view(torch.uint8), rq.view(torch.uint8))
        assert torch.equal(hc, cs) and torch.equal(hq.view(torch.uint8), cq.view(torch.uint8))
        # and directly against the oracle's to_mx, specials included, both layouts
        for t, sc, qq in ((xs[b].cpu(), gr, gq), (xs[b].cpu().t().contiguous(), hc, hq)):
            src = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[t.dtype]
            ref_s, ref_q = O.to_mx(bits_u16(t), src=src) if src == "bf16" else O.to_mx(t.numpy(), src=src)
            np.testing.assert_array_equal(bits_u8(sc), ref_s)
            np.testing.assert_array_equal(bits_u8(qq), ref_q)


def _sqnr(ref, x):
    ref = np.asarray(ref, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    return 20 * np.log10(np.linalg.norm(ref) / np.linalg.norm(ref - x))


@pytest.mark.parametrize("E,M,N,K", [(4, 1024, 512, 768), (1, 512, 256, 1024), (8, 2048, 320, 256)])
def test_moe_layer_forward_and_gradients(gpu, E, M, N, K):
    import kernels
    from kernels.moe import mxfp8_grouped_mm
    offs = [int(v) for v in seeded_offs(E, M, seed=E * 13 + K)]
    offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
    x = randn_bf16((M, K), 1.0, 3 + E).to(gpu).requires_grad_(True)
    w = randn_bf16((E, N, K), 0.05, 4 + E).to(gpu).requires_grad_(True)
    gout = randn_bf16((M, N), 1.0, 5 + E).to(gpu)
    out = mxfp8_grouped_mm(x, w, offs_t)
    out.backward(gout)
    torch.cuda.synchronize()

    # wiring: the same GEMMs on separately quantized operands, bit for bit
    sx, qx = kernels.to_mx(x.detach())
    sw, qw = kernels.to_mx(w.detach())
    assert torch.equal(out, kernels.triton_mxfp8_grouped_mm(qx, qw, sx, sw, offs_t))
    sg, qg = kernels.to_mx(gout)
    swt, qwt = kernels.to_mx(w.detach().transpose(-2, -1).contiguous())
    assert torch.equal(x.grad, kernels.triton_mxfp8_grouped_mm(qg, qwt, sg, swt, offs_t))
    sgt, qgt = kernels.to_mx_dim0(gout)
    sxt, qxt = kernels.to_mx_dim0(x.detach())
    assert torch.equal(w.grad, kernels.triton_mxfp8_wgrad(qgt, sgt, qxt, sxt, offs_t))

    # math: against the fp64 products of the unquantized operands
    xn, wn, gn = (f32(t.detach()).astype(np.float64) for t in (x, w, gout))
    ref_out = np.zeros((M, N))
    ref_gx = np.zeros((M, K))
    ref_gw = np.zeros((E, N, K))
    prev = 0
    for e, end in enumerate(offs):
        ref_out[prev:end] = xn[prev:end] @ wn[e].T
        ref_gx[prev:end] = gn[prev:end] @ wn[e]
        ref_gw[e] = gn[prev:end].T @ xn[prev:end]
        prev = end
    s_out, s_gx, s_gw = _sqnr(ref_out, f32(out.detach())), _sqnr(ref_gx, f32(x.grad)), _sqnr(ref_gw, f32(w.grad))
    print(f"SQNR out {s_out:.2f} dB, grad_x {s_gx:.2f} dB, grad_w {s_gw:.2f} dB")
    assert s_out >= 27.0 and s_gx >= 26.0 and s_gw >= 26.0


def test_moe_module_trains(gpu):
    """A few SGD steps of MXFP8GroupedLinear towards a fixed target reduce the loss."""
    from kernels.moe import MXFP8GroupedLinear
    torch.manual_seed(0)
    E, M, Kin, Nout = 4, 512, 256, 128
    layer = MXFP8GroupedLinear(E, Kin, Nout, device=gpu)
    offs = torch.tensor([128, 256, 384, 512], dtype=torch.int32, device=gpu)
    x = torch.randn((M, Kin), device=gpu).to(torch.bfloat16)
    target = torch.randn((M, Nout), device=gpu).to(torch.bfloat16)
    opt = torch.optim.SGD(layer.parameters(), lr=0.5)
    losses = []
    for _ in range(5):
        opt.zero_grad()
        loss = ((layer(x, offs).float() - target.float()) ** 2).mean()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert all(np.isfinite(losses)) and losses[-1] < losses[0]
