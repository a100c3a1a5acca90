"""MXFP8 grouped linear layer of a mixture-of-experts block, with autograd.

The reference ships the three GEMMs of an MoE layer's expert projection
(forward, dgrad and wgrad: kernels/forward.py:461-606, kernels/backward.py:
217-305) and leaves the training step that chains them to its caller
(README.md:3-12).  This module is that step for ``out[g] = x[g] @ w[g]^T``:

  forward   x (M, K) quantized along K, w (E, N, K) along K
            -> triton_mxfp8_grouped_mm                      out (M, N)
  dgrad     grad_out (M, N) along N, w^T (E, K, N) along N
            -> triton_mxfp8_grouped_mm                      grad_x (M, K)
            (the reference's dgrad form, kernels/forward.py:485-488)
  wgrad     grad_out^T (N, M) and x^T (K, M), both along M
            -> triton_mxfp8_wgrad                           grad_w (E, N, K)
            (the "dim1-quantized" operands, kernels/backward.py:232-243)

Every operand is quantized by ``to_mx_both``, which reads the bf16 tensor once
and writes both the row-wise and the transposed column-wise MX layouts, with
the scales step-major (``scale_layout="steps"``) and the data in row pairs
(``data_layout="pairs"``): the layouts the GEMM kernels read fastest, so none
of the three GEMMs re-lays scales per call and every operand copy moves whole
128-byte lines.  The forward keeps
only the e4m3 layouts the backward needs (x^T along M and w^T along N, with
their scales): half the bytes of keeping x and w in bf16.

Groups are cumulative end offsets (any values; with bounds off the 32 grid a
32-token scale block of the wgrad operands spans two groups and scales both,
as in the reference), and every token must be routed: ``offs[-1] == M``.
Rows past ``offs[-1]`` would get no output and no gradient (the GEMMs leave
them unwritten, as the reference does), so the layer assumes there are none
rather than synchronising to check.
"""

from __future__ import annotations

import math

import torch

from .backward import triton_mxfp8_wgrad
from .forward import triton_mxfp8_grouped_mm
from .quant import to_mx_both


# quantizer output layouts of every operand (M, N, K multiples of 32: even
# row counts, as row pairs need)
_LAYOUTS = {"scale_layout": "steps", "data_layout": "pairs"}


class _MXFP8GroupedMM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, offs, out_dtype):
        (sx, qx), (sxt, qxt) = to_mx_both(x, **_LAYOUTS)   # (M, K) along K; (K, M) along M
        (sw, qw), (swt, qwt) = to_mx_both(w, **_LAYOUTS)   # (E, N, K) along K; (E, K, N) along N
        out = triton_mxfp8_grouped_mm(qx, qw, sx, sw, offs, out_dtype=out_dtype)
        ctx.save_for_backward(qxt, sxt, qwt, swt, offs)
        ctx.x_dtype = x.dtype
        ctx.w_dtype = w.dtype
        return out

    @staticmethod
    def backward(ctx, grad_out):
        qxt, sxt, qwt, swt, offs = ctx.saved_tensors
        (sg, qg), (sgt, qgt) = to_mx_both(grad_out.contiguous(), **_LAYOUTS)   # along N; (N, M) along M
        grad_x = grad_w = None
        if ctx.needs_input_grad[0]:
            grad_x = triton_mxfp8_grouped_mm(qg, qwt, sg, swt, offs, out_dtype=ctx.x_dtype)
        if ctx.needs_input_grad[1]:
            grad_w = triton_mxfp8_wgrad(qgt, sgt, qxt, sxt, offs, out_dtype=torch.bfloat16)
            if grad_w.dtype != ctx.w_dtype:
                grad_w = grad_w.to(ctx.w_dtype)
        return grad_x, grad_w, None, None


def mxfp8_grouped_mm(x: torch.Tensor, w: torch.Tensor, offs: torch.Tensor,
                     out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``out[offs[g-1]:offs[g]] = x[offs[g-1]:offs[g]] @ w[g]^T`` in MXFP8, differentiable
    in ``x`` and ``w``.

    x: ``(M, K)`` bf16/fp16/fp32; w: ``(E, N, K)`` of the same kind; offs: ``(E,)``
    int32 cumulative group ends on the device, ``offs[-1] == M``.
    M, N and K must be multiples of 32.  Returns ``(M, N)`` of ``out_dtype``.
    """
    if x.dim() != 2 or w.dim() != 3 or x.shape[1] != w.shape[2]:
        raise ValueError(f"x must be (M, K) and w (E, N, K); got {tuple(x.shape)} and {tuple(w.shape)}")
    if offs.numel() != w.shape[0]:
        raise ValueError(f"offs has {offs.numel()} entries, w has E={w.shape[0]}")
    if offs.dtype != torch.int32:
        offs = offs.to(torch.int32)
    return _MXFP8GroupedMM.apply(x, w, offs, out_dtype)


class MXFP8GroupedLinear(torch.nn.Module):
    """E expert projections ``in_features -> out_features`` run as one MXFP8 grouped GEMM.

    ``forward(x, offs)`` takes tokens sorted by expert (``x`` is ``(M,
    in_features)``, ``offs`` the cumulative group ends) and returns ``(M,
    out_features)``.  The weight is ``(E, out_features, in_features)``, each
    expert's slice initialised like ``torch.nn.Linear``'s weight.
    """

    def __init__(self, num_experts: int, in_features: int, out_features: int,
                 device=None, dtype=torch.bfloat16, out_dtype=torch.bfloat16):
        super().__init__()
        self.num_experts = num_experts
        self.in_features = in_features
        self.out_features = out_features
        self.out_dtype = out_dtype
        self.weight = torch.nn.Parameter(
            torch.empty((num_experts, out_features, in_features), device=device, dtype=dtype))
        self.reset_parameters()

    def reset_parameters(self) -> None:
        bound = 1.0 / math.sqrt(self.in_features)   # kaiming_uniform_(a=sqrt(5)) of nn.Linear
        with torch.no_grad():
            self.weight.uniform_(-bound, bound)

    def forward(self, x: torch.Tensor, offs: torch.Tensor) -> torch.Tensor:
        return mxfp8_grouped_mm(x, self.weight, offs, self.out_dtype)

    def extra_repr(self) -> str:
        return f"num_experts={self.num_experts}, in_features={self.in_features}, out_features={self.out_features}"
