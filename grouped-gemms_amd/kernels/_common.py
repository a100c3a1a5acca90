"""Availability probe and tensor plumbing shared by the MX operators.

``_rocm_mxfp8_available`` keeps the reference's name and meaning
(kernels/_common.py:17-27): True on a ROCm build of torch when the native
library of this package is present.  Whether the current device is a gfx950
part is checked per call by the library itself (``mxgg_device_supported``).
"""

from __future__ import annotations

import torch

from . import _lib


# A ROCm build of torch (torch.version.hip set) with libmxgg loadable.
_rocm_mxfp8_available = bool(getattr(torch.version, "hip", None)) and _lib.available()

_UNAVAILABLE_MSG = "ROCm MXFP8 kernels require gfx950 and the libmxgg extension"


def _require(t: torch.Tensor, name: str) -> None:
    if not _rocm_mxfp8_available:
        raise NotImplementedError(_UNAVAILABLE_MSG)
    if not t.is_cuda:
        raise TypeError(f"{name} must be a GPU tensor, got device {t.device}")


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _u8(t: torch.Tensor) -> torch.Tensor:
    """View e4m3 / e8m0 / packed-fp4 tensors as uint8 (kernels/forward.py:534-535)."""
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


def _rowmajor(t: torch.Tensor) -> torch.Tensor:
    """Unit stride along the last dim (the MX block dim); other strides kept."""
    if t.dim() == 0 or t.stride(-1) == 1 or t.shape[-1] <= 1:
        return t
    return t.contiguous()


_OUT_CODES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
              torch.float32: _lib.DTYPE_F32}


def _out_code(dtype: torch.dtype, allowed=(torch.bfloat16, torch.float16, torch.float32)) -> int:
    if dtype not in allowed:
        raise ValueError(f"out_dtype {dtype} not supported (allowed: {allowed})")
    return _OUT_CODES[dtype]


def _offsets(offs: torch.Tensor, device: torch.device) -> torch.Tensor:
    """int32, contiguous, on `device` (kernels/forward.py:356-357)."""
    if offs.dim() != 1:
        raise ValueError(f"group_end_offsets must be 1-D, got shape {tuple(offs.shape)}")
    if offs.dtype != torch.int32:
        offs = offs.to(torch.int32)
    if offs.device != device:
        offs = offs.to(device)
    return offs.contiguous()
