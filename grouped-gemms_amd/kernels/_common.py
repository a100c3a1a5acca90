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


def _pair_buffer(batch: tuple, rows: int, length: int, device) -> tuple:
    """Fresh uint8 row-pair storage for ``(*batch, rows, length)`` data.

    Row pairs (``MXGG_DATA_PAIRS``, no counterpart in the reference): with
    ``ld = length`` rounded up to 64, byte k of row r sits at
    ``(r // 2) * 2 * ld + (k // 64) * 128 + (r % 2) * 64 + k % 64``, so the
    64-byte pieces of two adjacent rows that the GEMMs stage together form
    one 128-byte line.  Returned as the strided view
    ``(*batch, rows // 2, 2, ld // 64, 64)`` -- element ``[.., p, h, s, b]`` is
    byte ``64 s + b`` of row ``2 p + h`` -- so ``view.reshape(*batch, rows,
    ld)`` gives the rows back (with the pad bytes past ``length``).  Returns
    ``(view, ld)``."""
    if rows % 2:
        raise ValueError(f"row pairs need an even row count, got {rows}")
    ld = (length + 63) // 64 * 64
    buf = torch.empty(tuple(batch) + (rows // 2, ld // 64, 2, 64), dtype=torch.uint8, device=device)
    return buf.transpose(-3, -2), ld


def _pair_geometry(t: torch.Tensor, nbatch: int):
    """``(rows, padded row bytes, ld)`` when ``t`` is a row-pair view with
    ``nbatch`` leading batch dims (as ``_pair_buffer`` makes them), else
    None (a row-major operand)."""
    if t.dim() != nbatch + 4 or t.shape[-3] != 2 or t.shape[-1] != 64:
        return None
    st = t.stride()
    if st[-1] != 1 or st[-3] != 64 or (t.shape[-2] > 1 and st[-2] != 128):
        return None
    if st[-4] % 128 or st[-4] < 128 * t.shape[-2]:
        return None
    return 2 * t.shape[-4], 64 * t.shape[-2], st[-4] // 2


def to_row_pairs(q: torch.Tensor) -> torch.Tensor:
    """Row-pair copy of row-major e4m3 data ``(*batch, R, L)`` (R even), the
    pad bytes past L zero: what the quantizers write with
    ``data_layout="pairs"``, for operands quantized elsewhere."""
    if q.dim() < 2:
        raise ValueError("to_row_pairs expects (*batch, rows, length) data")
    if q.dtype != torch.float8_e4m3fn:
        raise TypeError(f"row pairs hold float8_e4m3fn data, got {q.dtype}")
    *batch, R, L = q.shape
    batch = tuple(batch)
    view, ld = _pair_buffer(batch, R, L, q.device)
    src = q.view(torch.uint8)
    if ld != L:
        padded = torch.zeros(batch + (R, ld), dtype=torch.uint8, device=q.device)
        padded[..., :L] = src
        src = padded
    view.copy_(src.reshape(batch + (R // 2, 2, ld // 64, 64)))
    return view.view(torch.float8_e4m3fn)


def _offsets(offs: torch.Tensor, device: torch.device) -> torch.Tensor:
    """int32, contiguous, on `device` (kernels/forward.py:356-357)."""
    if offs.dim() != 1:
        raise ValueError(f"group_end_offsets must be 1-D, got shape {tuple(offs.shape)}")
    if offs.dtype != torch.int32:
        offs = offs.to(torch.int32)
    if offs.device != device:
        offs = offs.to(device)
    return offs.contiguous()
