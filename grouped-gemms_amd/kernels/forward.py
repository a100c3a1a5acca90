"""Forward / dgrad MX grouped GEMM on gfx950: ``triton_mxfp8_grouped_mm``.

Drop-in for kernels/forward.py:461-606 of the reference: same name,
positional order, defaults and return value.  ``output[s:e] = A[s:e] @ B[g]^T``
per expert group, MX scales per 32 elements of K, fp32 accumulation, one
rounding to ``out_dtype``.  The work runs in the hand-written HIP kernels of
libmxgg (``mxgg_grouped_mm``): a scale re-layout launch (which also copies an
e4m3 weight and / or the activations into row pairs where the GEMM gains more
than the copy costs, ``mxgg_grouped_mm_staging_size``; same bits), then the
GEMM, which builds the expert->tile routing inside the kernel from
``group_end_offsets`` (no host sync), and, when the last round of tiles is
split along K, the piece and reduce launches.  The per-call workspace (torch's
caching allocator) holds the re-laid scales, up to 128 MiB of fp32 partial
tiles and the staged operands; ``MXGG_STAGING=0`` in the environment leaves
the staging room out.

Beyond the reference, the weight may be MXFP4: ``weight`` of dtype
``torch.float4_e2m1fn_x2`` (or uint8) with last dim K/2, two e2m1 values per
byte (element 2i in the low nibble), scales per 32 elements of K.  And the
scales may come step-major (int32 ``(T, M)`` and ``(E, T, N)``,
``T = cdiv(K, 128)``, as ``to_mx(..., scale_layout="steps")`` writes them):
the call then skips the re-layout launch (``mxgg_grouped_mm_steps``).  With
step-major scales either e4m3 operand may also be in row pairs (the view
``(M/2, 2, cdiv(K, 64), 64)``, resp. ``(E, N/2, 2, cdiv(K, 64), 64)``, that
``to_mx(..., data_layout="pairs")`` returns), and a packed e2m1 weight in row
quads (``(E, N/4, 4, cdiv(K/2, 32), 32)``, ``data_layout="quads"``), which the
kernels copy in whole 128-byte lines.
"""

from __future__ import annotations

import torch

from . import _lib
from ._common import _offsets, _out_code, _pair_geometry, _require, _rowmajor, _staging_enabled, _stream_handle, _u8

# Tile shapes built into libmxgg (BLOCK_M x BLOCK_N); BLOCK_K is fixed at 128.
BUILT_TILES = ((256, 256), (128, 128))

_FP4_DTYPES = tuple(d for d in (getattr(torch, "float4_e2m1fn_x2", None), torch.uint8) if d is not None)


def _split_room(total: int, scale_bytes: int) -> int:
    """Partial-tile room of a workspace of ``total`` bytes whose first
    ``scale_bytes`` (256-byte aligned) hold re-laid scales: what a call on
    step-major scales gets, so that both calls make the same split plan."""
    return max(0, total - ((scale_bytes + 255) // 256) * 256)


def _pick_config(E: int, M: int, N: int, K: int, b_fmt: int = _lib.FMT_E4M3, BLOCK_M: int = 0,
                 BLOCK_N: int = 0, GROUP_M: int = 0, XCD_SWIZZLE: int = 0) -> dict:
    """Launch configuration of one grouped-GEMM call (kernels/forward.py:399-459).

    The reference looks ``(E, N, K)`` up in a table of Triton meta-parameters;
    here libmxgg owns the table (``mxgg_grouped_mm_config``) so that C callers
    get the same choice.  Returns ``{"BLOCK_M", "BLOCK_N", "BLOCK_K",
    "GROUP_M", "XCD_SWIZZLE"}``; requested values are applied when the tile is
    built (``MXGGError`` with code MXGG_ERR_UNSUPPORTED otherwise).
    """
    import ctypes
    bm, bn, gm, xcd = (ctypes.c_int(int(v or 0)) for v in (BLOCK_M, BLOCK_N, GROUP_M, XCD_SWIZZLE))
    rc = _lib.load().mxgg_grouped_mm_config(int(E), int(M), int(N), int(K), int(b_fmt), ctypes.byref(bm),
                                            ctypes.byref(bn), ctypes.byref(gm), ctypes.byref(xcd))
    _lib.check(rc)
    return {"BLOCK_M": bm.value, "BLOCK_N": bn.value, "BLOCK_K": 128, "GROUP_M": gm.value,
            "XCD_SWIZZLE": xcd.value}


def triton_mxfp8_grouped_mm(
    input_act: torch.Tensor,
    weight: torch.Tensor,
    input_act_scales: torch.Tensor,
    weight_scales: torch.Tensor,
    group_end_offsets: torch.Tensor,
    out_dtype: torch.dtype = torch.bfloat16,
    BLOCK_M: int = None,
    BLOCK_N: int = None,
    BLOCK_K: int = None,
    GROUP_M: int = None,
    XCD_SWIZZLE: int = None,
    num_warps: int = None,
    num_stages: int = None,
    matrix_instr_nonkdim: int = None,
    waves_per_eu: int = None,
    kpack: int = 1,
    w_cache_modifier: str = None,
    x_evict_policy: str = None,
) -> torch.Tensor:
    """MX grouped GEMM: ``output[g] = input_act[group_g] @ weight[g]^T``.

    Args (kernels/forward.py:485-497):
        input_act: ``(M, K)`` float8_e4m3fn.
        weight: ``(E, N, K)`` float8_e4m3fn, or ``(E, N, K/2)`` packed e2m1.
        input_act_scales: ``(M, K//32)`` e8m0 (uint8 or float8_e8m0fnu).
        weight_scales: ``(E, N, K//32)`` e8m0.
        group_end_offsets: ``(E,)`` int32 cumulative group ends.
        BLOCK_M / BLOCK_N / GROUP_M / XCD_SWIZZLE: tile-shape and schedule
            requests, honoured when the tile is built (``BUILT_TILES``), else
            the library picks; ``BLOCK_K`` and the Triton
            tunables (num_warps, num_stages, matrix_instr_nonkdim,
            waves_per_eu, kpack, w_cache_modifier, x_evict_policy) are
            accepted for signature compatibility and have no effect.

    Returns ``(M, N)`` of ``out_dtype``; rows at or past ``offs[-1]`` are left
    uninitialised, as in the reference.

    Row-pair operands (see the module doc; step-major scales only) span K
    rounded up to 64.  With one of them row-major its K is used, and the bits
    equal the all-row-major call's.  With both in row pairs the call runs at
    the rounded K: for K % 64 == 32 that adds 32 zeros with scale 2**0 to
    every dot product (the quantizers zero the pad), which the kernels do
    anyway, but the launch configuration is the one chosen for the rounded K.
    """
    _require(input_act, "input_act")
    if input_act.dtype != torch.float8_e4m3fn:
        raise TypeError(f"input_act dtype {input_act.dtype} is not float8_e4m3fn")
    pa = _pair_geometry(input_act, 0)
    pb = _pair_geometry(weight, 1) if weight.dtype == torch.float8_e4m3fn else None
    qb = _pair_geometry(weight, 1, 4) if weight.dtype in _FP4_DTYPES else None   # row quads
    M, Ka = (pa[0], pa[1]) if pa else input_act.shape
    if weight.dtype == torch.float8_e4m3fn:
        b_fmt = _lib.FMT_E4M3
        E, N, Kb = (weight.shape[0], pb[0], pb[1]) if pb else weight.shape
    elif weight.dtype in _FP4_DTYPES:
        b_fmt = _lib.FMT_E2M1
        E = weight.shape[0]
        N, Kb = (qb[0], 2 * qb[1]) if qb else (weight.shape[1], 2 * weight.shape[2])
        pb = qb
    else:
        raise TypeError(f"weight dtype {weight.dtype} is neither float8_e4m3fn nor packed fp4")
    # K: the row-major operand's (row pairs round it up to 64, quads of packed
    # e2m1 likewise: 32 bytes)
    K = Kb if pa and not pb else Ka
    if (pa is None) != (pb is None):
        padded = Ka if pa else Kb
        assert (K + 63) // 64 * 64 == padded, f"K mismatch: {K} and a row-group operand spanning {padded}"
    else:
        assert Ka == Kb, f"K mismatch: A={Ka}, B={Kb}" + (" (packed fp4: K/2 bytes)" if b_fmt else "")
    if K % 32:
        raise ValueError(f"K={K} must be a multiple of the MX block size 32")
    steps = input_act_scales.dtype == torch.int32
    if steps != (weight_scales.dtype == torch.int32):
        raise TypeError("input_act_scales and weight_scales must both be e8m0 bytes or both step-major int32")
    layout = (_lib.A_PAIRS if pa else 0) | ((_lib.B_QUADS if qb else _lib.B_PAIRS) if pb else 0)
    if layout and not steps:
        raise TypeError("row-pair operands need step-major int32 scales (scale_layout='steps')")
    T = (K + 127) // 128
    want_a, want_b = ((T, M), (E, T, N)) if steps else ((M, K // 32), (E, N, K // 32))
    if tuple(input_act_scales.shape) != want_a:
        raise ValueError(f"input_act_scales shape {tuple(input_act_scales.shape)} != {want_a}")
    if tuple(weight_scales.shape) != want_b:
        raise ValueError(f"weight_scales shape {tuple(weight_scales.shape)} != {want_b}")
    if group_end_offsets.numel() != E:
        raise ValueError(f"group_end_offsets has {group_end_offsets.numel()} entries, weight has E={E}")
    # Tile requests are hints: a built tile is used, anything else (e.g. a
    # Triton config copied from the reference's table) falls back to the
    # library's own choice instead of failing.
    bm = BLOCK_M or BLOCK_N or 0
    bn = BLOCK_N or BLOCK_M or 0
    if (bm, bn) not in BUILT_TILES:
        bm = bn = 0
    dev = input_act.device
    a = _u8(input_act if pa else _rowmajor(input_act))
    b = _u8(weight if pb else _rowmajor(weight))
    lda = pa[2] if pa else a.stride(0)
    ldb_n = pb[2] if pb else b.stride(1)
    offs = _offsets(group_end_offsets, dev)
    out = torch.empty((M, N), dtype=out_dtype, device=dev)
    code = _out_code(out_dtype)
    lib = _lib.load()
    # scratch for the scales re-laid step-major and the fp32 partial tiles of a
    # split last round (overwritten by the call; torch's caching allocator
    # makes the per-call allocation cheap)
    ws_bytes = lib.mxgg_grouped_mm_workspace_size(E, M, N, K)
    if steps:
        a_ss, b_ss = input_act_scales.contiguous(), weight_scales.contiguous()
        ws_bytes = _split_room(ws_bytes, 4 * T * (M + E * N))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        rc = lib.mxgg_grouped_mm_steps(
            a.data_ptr(), lda, a_ss.data_ptr(),
            b.data_ptr(), b_fmt, ldb_n, b.stride(0), b_ss.data_ptr(),
            offs.data_ptr(), E, M, N, K,
            out.data_ptr(), code, out.stride(0),
            int(bm), int(bn), int(GROUP_M or 0), int(XCD_SWIZZLE or 0), layout,
            ws.data_ptr() if ws is not None else None, ws_bytes,
            _stream_handle(dev))
        _lib.check(rc)
        return out
    a_s = _u8(_rowmajor(input_act_scales))
    b_s = _u8(_rowmajor(weight_scales))
    # plus room to stage the weight and / or A in row pairs where that pays
    # for its copy (none with MXGG_STAGING=0)
    if _staging_enabled():
        ws_bytes += lib.mxgg_grouped_mm_staging_size(E, M, N, K, b_fmt)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    rc = lib.mxgg_grouped_mm(
        a.data_ptr(), a.stride(0), a_s.data_ptr(), a_s.stride(0),
        b.data_ptr(), b_fmt, b.stride(1), b.stride(0),
        b_s.data_ptr(), b_s.stride(1), b_s.stride(0),
        offs.data_ptr(), E, M, N, K,
        out.data_ptr(), code, out.stride(0),
        int(bm), int(bn), int(GROUP_M or 0), int(XCD_SWIZZLE or 0),
        ws.data_ptr() if ws is not None else None, ws_bytes,
        _stream_handle(dev))
    _lib.check(rc)
    return out
