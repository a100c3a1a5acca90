"""Writes tests/golden/cfg1.npz: BASELINE config 1 inputs and the oracle's
expected outputs (quantized bytes, scales, bf16 GEMM result).

Config 1 (seed 0): A (1024, 512) bf16 ~ N(0, 1); B (4, 512, 512) bf16 ~ N(0, 0.02);
4 groups of random multiples of 32 summing to 1024 (Python random.Random(0));
both quantized along K with the FLOOR MX recipe; out[g] = A[g] @ B[g]^T from
the dequantized operands in float64, stored as bf16.

Run from the repository root:  python tests/golden/make_golden.py
"""

import os
import random
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import mx_oracle as O  # noqa: E402


def main():
    g = torch.Generator().manual_seed(0)
    a = torch.randn((1024, 512), generator=g).to(torch.bfloat16)
    b = (torch.randn((4, 512, 512), generator=g) * 0.02).to(torch.bfloat16)
    a_bits = a.view(torch.int16).numpy().view(np.uint16)
    b_bits = b.view(torch.int16).numpy().view(np.uint16)
    offs = O.generate_jagged_offs(4, 1024, 32, rng=random.Random(0))
    a_s, a_q = O.to_mx(a_bits, src="bf16")
    b_s, b_q = O.to_mx(b_bits, src="bf16")
    out = O.grouped_mm(a_q, a_s, b_q, b_s, offs)
    out_bf16 = O.f32_to_bf16_bits(out.astype(np.float32))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg1.npz")
    np.savez_compressed(path, a_bf16=a_bits, b_bf16=b_bits, offs=offs, a_scales=a_s, a_q=a_q,
                        b_scales=b_s, b_q=b_q, out_bf16=out_bf16)
    print("wrote", path, "offs", offs.tolist())


if __name__ == "__main__":
    main()
