"""Drop-in for the reference's ``utils.py`` helpers (utils.py:20-115), MI355X-native.

* ``to_mx``: the on-GPU HIP quantizer (bit-identical to the reference's eager
  torch recipe, utils.py:67-105).  GPU tensors only: there is no CPU path.
* ``generate_jagged_offs``: random sorted cumulative group ends, multiples of
  ``multiple_of``, last = M (utils.py:35-50, same algorithm and the same use of
  Python's ``random`` module, so seeded runs draw the same offsets).
* ``benchmark_cuda_function_in_microseconds``: median device time of a call,
  timed with HIP events around each repetition after flushing the caches
  (the role of ``triton.testing.do_bench`` in utils.py:28-32).
* ``is_MI350``: gfx950 device check (utils.py:108-115).
"""

from __future__ import annotations

import random
import statistics
from typing import Callable

import torch

from kernels.quant import to_mx, to_mx_dim0  # noqa: F401  (re-export)

# MI355X: 4 MB L2 per XCD and a 256 MB Infinity Cache; a flush must exceed both.
_FLUSH_BYTES = 512 * 1024 * 1024
_flush_buf: dict = {}


def _flush(device) -> None:
    buf = _flush_buf.get(device)
    if buf is None:
        buf = torch.empty(_FLUSH_BYTES // 4, dtype=torch.int32, device=device)
        _flush_buf[device] = buf
    buf.zero_()


def benchmark_cuda_function_in_microseconds(fn: Callable, *args, warmup_ms: float = 25.0,
                                            rep_ms: float = 100.0, min_reps: int = 10,
                                            max_reps: int = 1000, flush: bool = True,
                                            **kwargs) -> float:
    """Median runtime of ``fn(*args, **kwargs)`` in microseconds.

    Each repetition is bracketed by events on the current stream, with the
    caches flushed just before it (outside the bracket).
    """
    dev = torch.cuda.current_device()
    fn(*args, **kwargs)
    torch.cuda.synchronize()
    # estimate
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(5):
        fn(*args, **kwargs)
    e.record()
    torch.cuda.synchronize()
    est = max(s.elapsed_time(e) / 5, 1e-3)
    n_warm = max(1, int(warmup_ms / est))
    n_rep = max(min_reps, min(max_reps, int(rep_ms / est)))
    for _ in range(n_warm):
        fn(*args, **kwargs)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    for i in range(n_rep):
        if flush:
            _flush(dev)
        starts[i].record()
        fn(*args, **kwargs)
        ends[i].record()
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in zip(starts, ends)) * 1e3


def generate_jagged_offs(E: int, M: int, multiple_of: int = 32, dtype=torch.int32,
                         device="cuda") -> torch.Tensor:
    """Random sorted cumulative offsets summing to M, each a multiple of
    ``multiple_of``; the last value is always M (utils.py:35-50)."""
    if M % multiple_of != 0:
        raise ValueError(f"M must be divisible by {multiple_of}")
    possible_values = list(range(multiple_of, M + 1, multiple_of))
    if E > len(possible_values):
        raise ValueError("E cannot be larger than the number of possible values")
    selected = sorted(random.sample(possible_values[:-1], E - 1)) + [M]
    return torch.tensor(selected, dtype=dtype).to(device)


def is_MI350() -> bool:
    """Whether the current GPU is a gfx950 part (MI350X / MI355X) under a ROCm
    build of torch (the reference asks the same of device 0, utils.py:108-115).
    Never raises: no GPU, a CUDA or CPU build of torch all answer False."""
    if not getattr(torch.version, "hip", None) or not torch.cuda.is_available():
        return False
    props = torch.cuda.get_device_properties(torch.cuda.current_device())
    return props.gcnArchName.split(":")[0] == "gfx950"
