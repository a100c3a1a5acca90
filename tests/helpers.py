"""Shared helpers for the parity tests (tensor <-> numpy bit views, inputs)."""

from __future__ import annotations

import random

import numpy as np
import torch

from oracle import mx_oracle as O


def bits_u16(t: torch.Tensor) -> np.ndarray:
    """bf16 / fp16 tensor -> uint16 bit patterns (CPU numpy)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bits_u8(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def seeded_offs(E: int, M: int, seed: int, multiple_of: int = 32) -> np.ndarray:
    return O.generate_jagged_offs(E, M, multiple_of, rng=random.Random(seed))


def randn_bf16(shape, std: float, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(torch.bfloat16)


def quantize_oracle(x_bf16: torch.Tensor, elem: str = "e4m3"):
    """Oracle to_mx along the last dim of a CPU bf16 tensor -> (scales, q) numpy."""
    return O.to_mx(bits_u16(x_bf16), src="bf16", elem=elem)


def to_dev_u8(a: np.ndarray, device, dtype=torch.uint8) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device).view(dtype)
