"""The reference's CPU path in torch ops: MX quantize, dequantize, per-group matmul.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; only
``tests/`` (which pin it to ``mx_oracle``) and ``bench.py``'s ``cpu_baseline``
leg (which times it on the host's cores) use it.

The reference has no CPU GEMM of its own: its correctness script compares the
GPU kernel with an unquantized torch product (test_correctness.py:48-50), and
its quantizer is plain torch (utils.py:67-105).  What a user of the reference
runs on a CPU for this path is therefore ``to_mx`` (which runs on CPU tensors
as written), a dequantize of e4m3 + e8m0 to fp32 and one ``torch.matmul`` per
group.  That is restated here with torch tensors and ops, so that its time on
the GPU box's host cores (torch's intra-op threads) can be reported beside the
HIP path on the same problem.  Pinned by ``tests/test_oracle.py``
(``test_torch_ref_*``): bit-exact with the committed golden fixture and with
``mx_oracle.to_mx`` on special blocks; the GEMM within fp32 accumulation error
of the fp64 oracle.
"""

from __future__ import annotations

import torch

F8E4M3_MAX = 448.0
F8E4M3_MAX_POW2 = 8     # floor(log2(448)); utils.py:63-64
BLOCK = 32


def to_mx(x: torch.Tensor, block: int = BLOCK):
    """(scales uint8, data float8_e4m3fn) of ``x`` along its last dim, FLOOR mode.

    utils.py:84-105: per ``block`` elements, amax in the input dtype taken to
    fp32 and clamped at the smallest normal; its biased exponent e gives the
    scale byte clamp(e - 8, 0, 254); the elements divided by 2**(s - 127)
    (exact), clamped to +-448 and cast to e4m3 with torch's own cast.
    """
    assert x.shape[-1] % block == 0, "last dim must be a multiple of the block"
    shape = x.shape
    xb = x.reshape(-1, shape[-1] // block, block)
    amax = xb.abs().amax(dim=-1, keepdim=True).to(torch.float32)
    amax = torch.clamp(amax, min=torch.finfo(torch.float32).tiny)
    e = (amax.view(torch.int32) >> 23) & 0xFF
    s = torch.clamp(e - F8E4M3_MAX_POW2, 0, 254).to(torch.uint8)
    q = torch.clamp(xb.to(torch.float32) / torch.exp2(s.to(torch.float32) - 127.0), -F8E4M3_MAX, F8E4M3_MAX)
    return s.reshape(*shape[:-1], shape[-1] // block), q.to(torch.float8_e4m3fn).reshape(shape)


def dequant(q: torch.Tensor, s: torch.Tensor, block: int = BLOCK) -> torch.Tensor:
    """fp32 values q * 2**(s - 127), the scale broadcast over its block (exact)."""
    shape = q.shape
    v = q.to(torch.float32).reshape(*shape[:-1], shape[-1] // block, block)
    return (v * torch.exp2(s.to(torch.float32) - 127.0).unsqueeze(-1)).reshape(shape)


def grouped_mm(a_q, a_s, b_q, b_s, offs) -> torch.Tensor:
    """bf16 out[s:e] = deq(A)[s:e] @ deq(B)[g]^T per group (fp32 matmul).

    The forward's mathematics (kernels/forward.py:238-240, 283-294): groups
    are cumulative end offsets, rows past offs[-1] zero here (the reference
    leaves them uninitialised).
    """
    a = dequant(a_q, a_s)
    b = dequant(b_q, b_s)
    out = torch.zeros((a.shape[0], b.shape[1]), dtype=torch.float32)
    prev = 0
    for g, end in enumerate(int(v) for v in offs):
        if end > prev:
            out[prev:end] = torch.matmul(a[prev:end], b[g].t())
        prev = end
    return out.to(torch.bfloat16)
