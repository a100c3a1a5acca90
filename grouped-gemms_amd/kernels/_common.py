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


def _staging_enabled() -> bool:
    """False when the environment sets ``MXGG_STAGING=0``: the drop-in calls
    then allocate no room for copying operands into row pairs (less transient
    memory per call -- up to E*N*K + M*K bytes for the forward, (N + K)*M for
    wgrad -- at the cost of the GEMM reading row-major operands; the output
    bits are the same).  Read per call."""
    import os
    return os.environ.get("MXGG_STAGING", "1") != "0"


_OUT_CODES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
              torch.float32: _lib.DTYPE_F32}


def _out_code(dtype: torch.dtype, allowed=(torch.bfloat16, torch.float16, torch.float32)) -> int:
    if dtype not in allowed:
        raise ValueError(f"out_dtype {dtype} not supported (allowed: {allowed})")
    return _OUT_CODES[dtype]


def _pair_buffer(batch: tuple, rows: int, length: int, device, group: int = 2) -> tuple:
    """Fresh uint8 row-group storage for ``(*batch, rows, length)`` data.

    Row pairs (``group`` 2, e4m3: ``MXGG_DATA_PAIRS``) and row quads (4,
    packed e2m1: ``MXGG_DATA_QUADS``), a layout with no counterpart in the
    reference: with pieces of ``P = 128 // group`` bytes (one 64-element
    stage of a row) and ``ld = _row_group_ld(length, P)`` (``length`` rounded
    up to P, plus a pad at some lengths), byte k of row r sits
    at ``(r // group) * group * ld + (k // P) * 128 + (r % group) * P + k % P``,
    so the pieces of the rows of a group that the GEMMs stage together form
    one 128-byte line.  Returned as the strided view
    ``(*batch, rows // group, group, cdiv(length, P), P)`` -- element
    ``[.., g, h, s, b]`` is byte ``P s + b`` of row ``group g + h``, the group
    stride ``group * ld`` -- so ``view.reshape(*batch, rows, -1)`` gives the
    rows back (with the pad bytes past ``length`` up to the piece).  Returns
    ``(view, ld)``."""
    if rows % group:
        raise ValueError(f"row {'pairs' if group == 2 else 'quads'} need a row count divisible by {group}, got {rows}")
    piece = 128 // group
    lv = (length + piece - 1) // piece * piece
    ld = _row_group_ld(length, piece)
    buf = torch.empty(tuple(batch) + (rows // group, ld // piece, group, piece), dtype=torch.uint8, device=device)
    return buf[..., : lv // piece, :, :].transpose(-3, -2), ld


def _row_group_ld(length: int, piece: int) -> int:
    """Row stride of a row-group buffer for rows of ``length`` bytes: the
    length rounded up to the piece, plus 192 bytes (never read) when the
    rows span a multiple of 8 cache lines that is not a power of two (K =
    3072, 5120, 6144, ...).  At those strides the 16 rows of a copy land on
    few cache sets / channels: measured on MI355X, forward kernel-only time
    on row pairs -2 to -7% at K = 5120 and dgrad at N = 5120 over the sweep
    shapes (same bits); power-of-two line counts (2048, 4096, 8192) gain
    nothing from it and keep the tight stride."""
    ld = (length + piece - 1) // piece * piece
    lines = (length + 127) // 128
    return ld + 192 if lines % 8 == 0 and lines & (lines - 1) else ld


def _pair_geometry(t: torch.Tensor, nbatch: int, group: int = 2):
    """``(rows, padded row bytes, ld)`` when ``t`` is a row-group view of
    ``group`` rows (2: pairs, 4: quads) with ``nbatch`` leading batch dims, as
    ``_pair_buffer`` makes them, else None (a row-major operand)."""
    piece = 128 // group
    if t.dim() != nbatch + 4 or t.shape[-3] != group or t.shape[-1] != piece:
        return None
    st = t.stride()
    if st[-1] != 1 or st[-3] != piece or (t.shape[-2] > 1 and st[-2] != 128):
        return None
    if st[-4] % 128 or st[-4] < 128 * t.shape[-2]:
        return None
    return group * t.shape[-4], piece * t.shape[-2], st[-4] // group


def _to_row_groups(q: torch.Tensor, group: int) -> torch.Tensor:
    *batch, R, L = q.shape
    batch = tuple(batch)
    view, _ = _pair_buffer(batch, R, L, q.device, group)
    piece = 128 // group
    lv = view.shape[-2] * piece            # the row's bytes rounded up to a piece
    src = q.view(torch.uint8)
    if lv != L:
        padded = torch.zeros(batch + (R, lv), dtype=torch.uint8, device=q.device)
        padded[..., :L] = src
        src = padded
    view.copy_(src.reshape(batch + (R // group, group, lv // piece, piece)))
    return view.view(q.dtype)


def to_row_pairs(q: torch.Tensor) -> torch.Tensor:
    """Row-pair copy of row-major e4m3 data ``(*batch, R, L)`` (R even), the
    pad bytes past L zero: what the quantizers write with
    ``data_layout="pairs"``, for operands quantized elsewhere."""
    if q.dim() < 2:
        raise ValueError("to_row_pairs expects (*batch, rows, length) data")
    if q.dtype != torch.float8_e4m3fn:
        raise TypeError(f"row pairs hold float8_e4m3fn data, got {q.dtype}")
    return _to_row_groups(q, 2)


def to_row_quads(q: torch.Tensor) -> torch.Tensor:
    """Row-quad copy of row-major packed e2m1 data ``(*batch, R, K/2)``
    (R divisible by 4), the pad zero: what ``to_mx(..., elem_dtype=
    torch.float4_e2m1fn_x2, data_layout="quads")`` writes."""
    if q.dim() < 2:
        raise ValueError("to_row_quads expects (*batch, rows, length) data")
    if q.element_size() != 1 or q.dtype == torch.float8_e4m3fn:
        raise TypeError(f"row quads hold packed e2m1 data (float4_e2m1fn_x2 or uint8), got {q.dtype}")
    return _to_row_groups(q, 4)


def _offsets(offs: torch.Tensor, device: torch.device) -> torch.Tensor:
    """int32, contiguous, on `device` (kernels/forward.py:356-357)."""
    if offs.dim() != 1:
        raise ValueError(f"group_end_offsets must be 1-D, got shape {tuple(offs.shape)}")
    if offs.dtype != torch.int32:
        offs = offs.to(torch.int32)
    if offs.device != device:
        offs = offs.to(device)
    return offs.contiguous()
