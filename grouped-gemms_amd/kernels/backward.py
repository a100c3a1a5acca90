"""Weight-gradient MX grouped GEMM on gfx950: ``triton_mxfp8_wgrad``.

Drop-in for kernels/backward.py:217-305 of the reference:
``grad_W[g] = grad_output[group_g]^T @ input_act[group_g]`` computed from the
dim-1 quantized operands ``go_t (N, M)`` and ``ia_t (K, M)`` (scales per 32
tokens), one reduction over each group's token range, output ``(E, N, K)``.
As in the reference the stored values are rounded to bf16 whatever
``out_dtype`` is (backward.py:101-104, 214, 251: float32 holds the bf16
value, float16 the bf16 value converted to half) and an empty group yields
zeros.  On plain scales the call's re-layout launch also copies both operands
into row pairs where the GEMM gains more than the copy costs
(``mxgg_wgrad_staging_size``; same bits; ``MXGG_STAGING=0`` in the
environment leaves that room out).  Step-major int32 scales (``(T, N)`` and ``(T, K)``, ``T = cdiv(M, 128)``, as
``to_mx_dim0(..., scale_layout="steps")`` writes them) skip the per-call
re-layout (``mxgg_wgrad_steps``); with them either operand may be in row pairs
(the view ``(N/2, 2, cdiv(M, 64), 64)``, resp. ``(K/2, ...)``, that
``to_mx_dim0`` / ``to_mx_both`` return with ``data_layout="pairs"``).
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import _offsets, _out_code, _pair_geometry, _require, _rowmajor, _staging_enabled, _stream_handle, _u8
from .forward import _split_room


def triton_mxfp8_wgrad(
    go_t: torch.Tensor,
    go_scale: torch.Tensor,
    ia_t: torch.Tensor,
    ia_scale: torch.Tensor,
    group_end_offsets: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    BLOCK_N: int = 256,
    BLOCK_K: int = 256,
    BLOCK_M: int = 64,
    num_warps: int = 8,
    num_stages: int = 2,
) -> torch.Tensor:
    """MX weight gradient: ``grad_W[g] = grad_output[group_g]^T @ input_act[group_g]``.

    Args (kernels/backward.py:238-243):
        go_t: ``(N, M)`` float8_e4m3fn, grad_output quantized along M.
        go_scale: ``(N, M//32)`` e8m0.
        ia_t: ``(K, M)`` float8_e4m3fn, input activations quantized along M.
        ia_scale: ``(K, M//32)`` e8m0.
        group_end_offsets: ``(E,)`` int32 cumulative token counts (any
            nondecreasing values up to M; a 32-token scale block shared by
            two groups scales the tokens of both, as in the reference).
        BLOCK_N / BLOCK_K / BLOCK_M / num_warps / num_stages: accepted for
            signature compatibility; the HIP kernel uses its own tiling.

    Returns ``(E, N, K)`` of ``out_dtype`` (bf16, float16 or float32), the
    bf16-rounded products in each.

    Row-pair operands span M rounded up to 64; with both in row pairs that is
    the M used, which changes nothing: tokens past ``offs[-1]`` are in no
    group, and the step count and plan depend on M only through
    ``cdiv(M, 128)``, which the rounding keeps.
    """
    _require(go_t, "go_t")
    for name, t in (("go_t", go_t), ("ia_t", ia_t)):
        if t.dtype != torch.float8_e4m3fn:
            raise TypeError(f"{name} dtype {t.dtype} is not float8_e4m3fn")
    pg, pi = _pair_geometry(go_t, 0), _pair_geometry(ia_t, 0)
    N, M = (pg[0], pg[1]) if pg else go_t.shape
    K, M2 = (pi[0], pi[1]) if pi else ia_t.shape
    if pg and not pi:
        M, M2 = M2, M
    if (pg is None) != (pi is None):
        if (M + 63) // 64 * 64 != M2:
            raise ValueError(f"token dims differ: {M} tokens and row pairs of {M2}")
    elif M2 != M:
        raise ValueError(f"token dims differ: go_t has {M}, ia_t has {M2}")
    if M % 32:
        raise ValueError(f"M={M} must be a multiple of the MX block size 32")
    steps = go_scale.dtype == torch.int32
    if steps != (ia_scale.dtype == torch.int32):
        raise TypeError("go_scale and ia_scale must both be e8m0 bytes or both step-major int32")
    layout = (_lib.A_PAIRS if pg else 0) | (_lib.B_PAIRS if pi else 0)
    if layout and not steps:
        raise TypeError("row-pair operands need step-major int32 scales (scale_layout='steps')")
    T = (M + 127) // 128
    want_g, want_i = ((T, N), (T, K)) if steps else ((N, M // 32), (K, M // 32))
    if tuple(go_scale.shape) != want_g:
        raise ValueError(f"go_scale shape {tuple(go_scale.shape)} != {want_g}")
    if tuple(ia_scale.shape) != want_i:
        raise ValueError(f"ia_scale shape {tuple(ia_scale.shape)} != {want_i}")
    E = group_end_offsets.shape[0]
    dev = go_t.device
    g = _u8(go_t if pg else _rowmajor(go_t))
    a = _u8(ia_t if pi else _rowmajor(ia_t))
    ld_g = pg[2] if pg else g.stride(0)
    ld_a = pi[2] if pi else a.stride(0)
    offs = _offsets(group_end_offsets, dev)
    code = _out_code(out_dtype)
    out = torch.empty((E, N, K), dtype=out_dtype, device=dev)
    lib = _lib.load()
    ws_bytes = lib.mxgg_wgrad_workspace_size(E, M, N, K)
    if steps:
        gss, iss = go_scale.contiguous(), ia_scale.contiguous()
        ws_bytes = _split_room(ws_bytes, 4 * T * (N + K))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        rc = lib.mxgg_wgrad_steps(
            g.data_ptr(), ld_g, gss.data_ptr(), a.data_ptr(), ld_a, iss.data_ptr(),
            offs.data_ptr(), E, M, N, K,
            out.data_ptr(), code, layout, ws.data_ptr() if ws is not None else None, ws_bytes,
            _stream_handle(dev))
        _lib.check(rc)
        return out
    gs = _u8(_rowmajor(go_scale))
    as_ = _u8(_rowmajor(ia_scale))
    # plus room to stage both operands in row pairs where that pays for its
    # copy (none with MXGG_STAGING=0)
    if _staging_enabled():
        ws_bytes += lib.mxgg_wgrad_staging_size(E, M, N, K)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    rc = lib.mxgg_wgrad(
        g.data_ptr(), g.stride(0), gs.data_ptr(), gs.stride(0),
        a.data_ptr(), a.stride(0), as_.data_ptr(), as_.stride(0),
        offs.data_ptr(), E, M, N, K,
        out.data_ptr(), code, ws.data_ptr() if ws is not None else None, ws_bytes,
        _stream_handle(dev))
    _lib.check(rc)
    return out
