"""On-GPU MX quantizer (FLOOR e8m0 scale per 32 elements, e4m3 or packed e2m1).

``to_mx`` is the drop-in for the reference's ``to_mx`` (utils.py:67-105):
same arguments, same ``(scales_uint8, data)`` return order, bit-identical
bytes and scales, computed by one fused HIP kernel (``mxgg_quantize_mx``)
instead of ~10 eager torch kernels.  ``to_mx_dim0`` produces
``to_mx(x.t().contiguous())`` in one pass (``mxgg_quantize_mx_dim0``), the
"dim1-quantized" layout the weight gradient takes (kernels/backward.py:232).
``to_mx_both`` gives both layouts from one read of the source
(``mxgg_quantize_mx_both``), for the backward pass of an MoE layer.

``scale_layout="steps"`` makes any of them write the scales in the layout the
GEMM kernels read (not the reference's: its CDNA4 pre-shuffle,
kernels/forward.py:367-397, is redone on every call): an int32 tensor
``(*batch, T, R)`` for a ``(*batch, R, L)`` result quantized along L,
``T = cdiv(L, 128)``, element ``[t, r]`` holding the scale bytes of elements
``128t .. 128t+127`` of row r (byte j: block 4t+j; bytes past the row 127).
``triton_mxfp8_grouped_mm`` / ``triton_mxfp8_wgrad`` recognise such int32
scales and skip their per-call re-layout.

``data_layout="pairs"`` makes them write the e4m3 data in row pairs: rows 2i
and 2i+1 interleaved in 64-byte pieces, returned as the strided view
``(*batch, R/2, 2, cdiv(L, 64), 64)`` (``_common._pair_buffer``; the pad
bytes past L are zero; the pair stride grows by 192 unread bytes where the
row spans a multiple of 8 cache lines that is not a power of two,
``_common._row_group_ld``).  The GEMMs stage a 64-element slice of two adjacent
rows per step, which is then one 128-byte line instead of halves of two:
13% less time for the forward and 19% for the weight gradient over the
benchmark shapes, same bits.  Packed e2m1 (32 bytes per 64-element step of a
row) goes in row quads the same way (``data_layout="quads"``, the view
``(*batch, R/4, 4, cdiv(L/2, 32), 32)``).  The GEMM wrappers recognise such
views (with step-major scales).
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import _pair_buffer, _require, _stream_handle

_SRC_CODES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16,
              torch.float32: _lib.DTYPE_F32}
_FP4 = getattr(torch, "float4_e2m1fn_x2", None)


def _src_code(t: torch.Tensor) -> int:
    if t.dtype not in _SRC_CODES:
        raise TypeError(f"to_mx input dtype {t.dtype} not one of bf16/fp16/fp32")
    return _SRC_CODES[t.dtype]


def _layout_code(scale_layout: str) -> int:
    if scale_layout == "plain":
        return _lib.SCALES_PLAIN
    if scale_layout == "steps":
        return _lib.SCALES_STEPS
    raise ValueError(f"scale_layout must be 'plain' or 'steps', got {scale_layout!r}")


def _pairs_flag(data_layout: str, allowed=("rows", "pairs")) -> bool:
    """True for a row-group layout ("pairs" / "quads"), False for "rows"."""
    if data_layout not in allowed:
        raise ValueError(f"data_layout must be one of {allowed}, got {data_layout!r}")
    return data_layout != "rows"


def _aligned_rows(batch: tuple, rows: int, length: int, device) -> tuple:
    """Output ``(*batch, rows, length)`` uint8 whose rows start on the
    128-byte grid: a view of a buffer with the row stride rounded up to a
    multiple of 128 when ``length`` is not one (e.g. the token-major operands
    of the weight gradient, whose length is the token count).  The GEMM
    copies operand rows in 64-byte pieces; rows off the 128-byte grid put a
    quarter of them across two cache lines (wgrad at 2080 tokens: 12-16%
    slower).  Returns ``(view, row stride)``."""
    ld = (length + 127) // 128 * 128
    buf = torch.empty(tuple(batch) + (rows, ld), dtype=torch.uint8, device=device)
    return buf[..., :length], ld


def step_scales_shape(batch: tuple, rows: int, length: int) -> tuple:
    """Shape of step-major scales of ``(*batch, rows, length)`` quantized
    along ``length``: ``(*batch, cdiv(length, 128), rows)`` (int32)."""
    return tuple(batch) + ((length + 127) // 128, rows)


def to_mx(data: torch.Tensor, elem_dtype=torch.float8_e4m3fn, block_size: int = 32, *,
          scale_layout: str = "plain", data_layout: str = "rows"):
    """Quantize ``data`` along its last dim; returns ``(scales_u8, data_q)``.

    ``elem_dtype`` float8_e4m3fn gives ``data_q`` of ``data``'s shape;
    ``torch.float4_e2m1fn_x2`` gives packed fp4 with the last dim halved
    (element 2i in the low nibble).  ``scales_u8`` has the last dim divided
    by 32.  Asserts like the reference (utils.py:78-81).  With
    ``scale_layout="steps"`` the scales are step-major int32
    ``(*data.shape[:-2], cdiv(L, 128), data.shape[-2])`` instead.
    ``data_layout="pairs"`` (e4m3, ``data.shape[-2]`` even): ``data_q`` in
    row pairs, the view ``(*data.shape[:-2], R/2, 2, cdiv(L, 64), 64)``;
    ``data_layout="quads"`` (e2m1, ``data.shape[-2]`` divisible by 4): in row
    quads, the view ``(*data.shape[:-2], R/4, 4, cdiv(L/2, 32), 32)``.
    """
    fp4 = _FP4 is not None and elem_dtype is _FP4
    assert elem_dtype is torch.float8_e4m3fn or fp4, "only e4m3fn and e2m1fn_x2 supported"
    assert block_size == 32, "block_size must be 32 (OCP MX)"
    assert data.shape[-1] % block_size == 0, (
        f"last dim {data.shape[-1]} must be divisible by block_size {block_size}"
    )
    _require(data, "data")
    code = _src_code(data)
    shape = tuple(data.shape)
    L = shape[-1]
    x = data.reshape(-1, L) if data.dim() != 2 else data
    if x.stride(-1) != 1 or (x.shape[0] > 1 and (x.stride(0) * x.element_size()) % 16) or x.data_ptr() % 16:
        x = x.contiguous()
    rows = x.shape[0]
    qcols = L // 2 if fp4 else L
    lay = _layout_code(scale_layout)
    pairs = _pairs_flag(data_layout, ("rows", "pairs", "quads"))
    if pairs:
        if data_layout != ("quads" if fp4 else "pairs") or len(shape) < 2:
            raise ValueError("data_layout 'pairs' holds e4m3 output and 'quads' packed e2m1, with at least 2 dims")
        qv, ld_q = _pair_buffer(shape[:-2], shape[-2], qcols, data.device, 4 if fp4 else 2)
        q_ptr = qv.data_ptr()
    else:
        q = torch.empty((rows, qcols), dtype=torch.uint8, device=data.device)
        q_ptr, ld_q = q.data_ptr(), qcols
    if lay == _lib.SCALES_STEPS:
        R = shape[-2] if len(shape) >= 2 else 1
        s = torch.empty(step_scales_shape(shape[:-2], R, L), dtype=torch.int32, device=data.device)
        ld_s = R
    else:
        s = torch.empty((rows, L // 32), dtype=torch.uint8, device=data.device)
        ld_s = L // 32
    lib = _lib.load()
    rc = lib.mxgg_quantize_mx(x.data_ptr(), code, rows, L, x.stride(0) if rows > 1 else L,
                              _lib.FMT_E2M1 if fp4 else _lib.FMT_E4M3,
                              q_ptr, ld_q, s.data_ptr(), ld_s,
                              lay | ((_lib.DATA_QUADS if fp4 else _lib.DATA_PAIRS) if pairs else 0),
                              _stream_handle(data.device))
    _lib.check(rc)
    if pairs:
        q = qv.view(_FP4 if fp4 else torch.float8_e4m3fn)
    else:
        q = q.view(_FP4 if fp4 else torch.float8_e4m3fn).reshape(shape[:-1] + (qcols,))
    if lay == _lib.SCALES_STEPS:
        return s, q
    return s.reshape(shape[:-1] + (L // 32,)), q


def to_mx_dim0(data: torch.Tensor, elem_dtype=torch.float8_e4m3fn, block_size: int = 32, *,
               scale_layout: str = "plain", data_layout: str = "rows"):
    """``to_mx(data.t().contiguous())`` for a 2-D ``(R, C)`` tensor in one pass.

    Returns ``(scales (C, R//32) uint8, data (C, R) float8_e4m3fn)``; with
    ``scale_layout="steps"`` the scales are step-major int32
    ``(cdiv(R, 128), C)``.  When R is not a multiple of 128 the data is a
    view whose row stride is R rounded up to 128 (same values, rows on the
    128-byte grid for the weight-gradient GEMM).  ``data_layout="pairs"``:
    the data in row pairs, the view ``(C/2, 2, cdiv(R, 64), 64)``.
    """
    assert elem_dtype is torch.float8_e4m3fn, "to_mx_dim0 supports e4m3fn only"
    assert block_size == 32, "block_size must be 32 (OCP MX)"
    assert data.dim() == 2, "to_mx_dim0 expects a 2-D tensor"
    R, C = data.shape
    assert R % block_size == 0, f"dim 0 ({R}) must be divisible by block_size {block_size}"
    _require(data, "data")
    code = _src_code(data)
    x = data
    if x.stride(-1) != 1 or (x.stride(0) * x.element_size()) % 16 or x.data_ptr() % 16 \
            or (C * x.element_size()) % 16:
        x = x.contiguous()
    if (C * x.element_size()) % 16:
        raise ValueError(f"to_mx_dim0 needs dim 1 ({C}) to span a multiple of 16 bytes")
    lay = _layout_code(scale_layout)
    pairs = _pairs_flag(data_layout)
    q, ld_q = (_pair_buffer if pairs else _aligned_rows)((), C, R, data.device)
    if lay == _lib.SCALES_STEPS:
        s = torch.empty(step_scales_shape((), C, R), dtype=torch.int32, device=data.device)
        ld_s = C
    else:
        s = torch.empty((C, R // 32), dtype=torch.uint8, device=data.device)
        ld_s = R // 32
    lib = _lib.load()
    rc = lib.mxgg_quantize_mx_dim0(x.data_ptr(), code, R, C, x.stride(0), _lib.FMT_E4M3,
                                   q.data_ptr(), ld_q, s.data_ptr(), ld_s, lay | (_lib.DATA_PAIRS if pairs else 0),
                                   _stream_handle(data.device))
    _lib.check(rc)
    return s, q.view(torch.float8_e4m3fn)


def to_mx_both(data: torch.Tensor, elem_dtype=torch.float8_e4m3fn, block_size: int = 32, *,
               scale_layout: str = "plain", data_layout: str = "rows"):
    """``(to_mx(data), to_mx(data.transpose(-2, -1).contiguous()))`` in one pass.

    ``data`` is ``(R, C)`` or ``(B, R, C)`` with ``R`` and ``C`` multiples of
    32.  Returns ``((scales (.., R, C//32), data (.., R, C)),
    (scales (.., C, R//32), data (.., C, R)))``, e4m3, bit-identical to the
    two separate calls.  ``scale_layout="steps"``: step-major int32 scales
    ``(.., cdiv(C, 128), R)`` and ``(.., cdiv(R, 128), C)``.  Either data
    output whose row length (C, resp. R) is not a multiple of 128 is a view
    with the row stride rounded up to 128 (as in ``to_mx_dim0``).
    ``data_layout="pairs"``: both data outputs in row pairs, the views
    ``(.., R/2, 2, cdiv(C, 64), 64)`` and ``(.., C/2, 2, cdiv(R, 64), 64)``.
    """
    assert elem_dtype is torch.float8_e4m3fn, "to_mx_both supports e4m3fn only"
    assert block_size == 32, "block_size must be 32 (OCP MX)"
    assert data.dim() in (2, 3), "to_mx_both expects a 2-D or 3-D tensor"
    _require(data, "data")
    code = _src_code(data)
    x = data if data.dim() == 3 else data.unsqueeze(0)
    B, R, C = x.shape
    assert R % block_size == 0 and C % block_size == 0, (
        f"both dims ({R}, {C}) must be divisible by block_size {block_size}")
    x = x.contiguous()
    if (C * x.element_size()) % 16:
        raise ValueError(f"to_mx_both needs the last dim ({C}) to span a multiple of 16 bytes")
    dev = data.device
    lay = _layout_code(scale_layout)
    pairs = _pairs_flag(data_layout)
    out = _pair_buffer if pairs else _aligned_rows
    q_r, ld_qr = out((B,), R, C, dev)
    q_c, ld_qc = out((B,), C, R, dev)
    if lay == _lib.SCALES_STEPS:
        s_r = torch.empty(step_scales_shape((B,), R, C), dtype=torch.int32, device=dev)
        s_c = torch.empty(step_scales_shape((B,), C, R), dtype=torch.int32, device=dev)
        ld_r, ld_c = R, C
    else:
        s_r = torch.empty((B, R, C // 32), dtype=torch.uint8, device=dev)
        s_c = torch.empty((B, C, R // 32), dtype=torch.uint8, device=dev)
        ld_r, ld_c = C // 32, R // 32
    lib = _lib.load()
    rc = lib.mxgg_quantize_mx_both(x.data_ptr(), code, B, R, C, C, q_r.data_ptr(), ld_qr, s_r.data_ptr(), ld_r,
                                   q_c.data_ptr(), ld_qc, s_c.data_ptr(), ld_c,
                                   lay | (_lib.DATA_PAIRS if pairs else 0), _stream_handle(dev))
    _lib.check(rc)
    q_r, q_c = q_r.view(torch.float8_e4m3fn), q_c.view(torch.float8_e4m3fn)
    if data.dim() == 2:
        return (s_r[0], q_r[0]), (s_c[0], q_c[0])
    return (s_r, q_r), (s_c, q_c)
