"""CPU tests of the drop-in boundary: the C-ABI library loads and exports every
symbol include/mxgg.h declares, rejects bad arguments before touching the GPU,
and the Python surface keeps the reference's names, signatures and errors
(kernels/__init__.py:17-25, kernels/forward.py:461-484, kernels/backward.py:217-229,
utils.py:28-115)."""

import ctypes
import inspect
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mxgg.h")


def _declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mxgg_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from kernels import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = _declared_functions()
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"


def test_version_and_error_string():
    from kernels import _lib
    lib = _lib.load()
    assert lib.mxgg_version() == 4001
    assert isinstance(lib.mxgg_last_error_string(), bytes)


def test_pure_size_helpers():
    from kernels import _lib
    lib = _lib.load()
    assert lib.mxgg_routing_words(4, 1024, 128) == 2 * 4 + 1 + 8 + 3
    assert lib.mxgg_routing_words(1, 16640, 256) == 2 + 1 + 65
    assert lib.mxgg_schedule_programs(8, 16640, 8192, 256, 256) == (65 + 7) * 32
    assert lib.mxgg_routing_words(0, 10, 128) == 0


def test_launch_config_query():
    """mxgg_grouped_mm_config (the counterpart of _pick_config) is pure host logic."""
    from kernels import _lib
    from kernels.forward import _pick_config
    # built-in rule (shapes the tuned table does not hold; it is checked in test_tune.py)
    big = _pick_config(8, 16640, 8192, 6144)
    assert (big["BLOCK_M"], big["BLOCK_N"], big["BLOCK_K"]) == (256, 256, 128)
    assert big["GROUP_M"] > 0 and big["XCD_SWIZZLE"] == 8
    # a sweep-sized problem fills the chip with 256 x 256 tiles (65 x 8 of them)
    assert _pick_config(1, 16640, 2048, 3072)["BLOCK_M"] == 256
    # 4 x 2 tiles of 256 would leave most CUs idle: 128 x 128 (7 x 4 expert-padded tiles)
    small = _pick_config(4, 1024, 512, 512)
    assert (small["BLOCK_M"], small["BLOCK_N"]) == (128, 128)
    # ... unless K is long enough for the split of the last round
    assert _pick_config(4, 1024, 512, 8192)["BLOCK_M"] == 256
    assert _pick_config(1, 16640, 2048, 2048, b_fmt=_lib.FMT_E2M1)["BLOCK_M"] == 256
    req = _pick_config(1, 16640, 8192, 8192, BLOCK_M=128, BLOCK_N=128, GROUP_M=4, XCD_SWIZZLE=1)
    assert (req["BLOCK_M"], req["BLOCK_N"], req["GROUP_M"], req["XCD_SWIZZLE"]) == (128, 128, 4, 1)
    with pytest.raises(_lib.MXGGError):
        _pick_config(1, 16640, 2048, 2048, b_fmt=_lib.FMT_E2M1, BLOCK_M=128, BLOCK_N=128)
    with pytest.raises(ValueError):
        _pick_config(1, 16640, 2048, 2048, b_fmt=3)


@pytest.mark.parametrize("args,needle", [
    (dict(b_fmt=3), "weight format"),
    (dict(out_dtype=9), "out_dtype"),
    (dict(E=0), "E=0"),
    (dict(K=48), "multiple of 32"),
    (dict(lda=16), "row stride"),
    (dict(lda=72, K=64), "16-byte aligned"),
])
def test_grouped_mm_validation_without_gpu(args, needle):
    """Invalid requests are rejected (MXGG_ERR_INVALID_ARG) before any HIP call."""
    from kernels import _lib
    lib = _lib.load()
    p = dict(A=16, lda=64, As=16, ldas=2, B=16, b_fmt=0, ldb_n=64, ldb_e=64 * 64, Bs=16, ldbs_n=2,
             ldbs_e=128, offs=16, E=1, M=64, N=64, K=64, out=16, out_dtype=0, ldo=64)
    p.update(args)
    rc = lib.mxgg_grouped_mm(p["A"], p["lda"], p["As"], p["ldas"], p["B"], p["b_fmt"], p["ldb_n"],
                             p["ldb_e"], p["Bs"], p["ldbs_n"], p["ldbs_e"], p["offs"], p["E"], p["M"],
                             p["N"], p["K"], p["out"], p["out_dtype"], p["ldo"], 0, 0, 0, 0, None, 0, None)
    assert rc == _lib.ERR_INVALID_ARG
    assert needle in lib.mxgg_last_error_string().decode()


def test_grouped_mm_workspace_without_gpu():
    """Workspace = the re-laid scales (4 * ceil(red/128) bytes per operand
    row), then, 256-byte aligned, the fp32 partial tiles of a split last round
    when the reduction has >= 32 steps of 128: at most 128 MiB, and no more than
    every tile cut into min(8, steps // 4) pieces (256x256 or 128x128 tiles,
    whichever needs more).  A call without the scale part is rejected
    (MXGG_ERR_WORKSPACE) before any HIP call."""
    from kernels import _lib
    lib = _lib.load()
    MiB = 1 << 20
    # E=8, M=16640, N=8192, K=5120: 40 steps; thousands of tiles -> the 128 MiB cap
    assert lib.mxgg_grouped_mm_workspace_size(8, 16640, 8192, 5120) == 4 * 40 * (16640 + 8 * 8192) + 128 * MiB
    # K=160: 2 steps, K=2048: 16 steps -- too short to split -> scales only, unaligned
    assert lib.mxgg_grouped_mm_workspace_size(1, 100, 64, 160) == 4 * 2 * (100 + 64)
    assert lib.mxgg_grouped_mm_workspace_size(2, 1000, 300, 2048) == 4 * 16 * (1000 + 2 * 300)
    # M=N=256, K=4096: 32 steps -> 8 pieces; one 256x256 tile (8 x 256 KiB) or
    # four 128x128 tiles (32 x 64 KiB): 2 MiB after 65536 bytes of scales
    assert lib.mxgg_grouped_mm_workspace_size(1, 256, 256, 4096) == 4 * 32 * (256 + 256) + 2 * MiB
    # wgrad E=4, M=16640: 33 steps per average group -> 8 pieces; 640 tiles -> cap
    assert lib.mxgg_wgrad_workspace_size(4, 16640, 2048, 5120) == 4 * 130 * (2048 + 5120) + 128 * MiB
    # wgrad E=8, N=K=256: 8 tiles; with several groups the room is sized for one
    # group holding all 130 steps -> 8 pieces of each tile (8 x 8 x 256 KiB)
    assert lib.mxgg_wgrad_workspace_size(8, 16640, 256, 256) == 4 * 130 * (256 + 256) + 16 * MiB
    # wgrad E=1, M=2048: 16 steps -> no split
    assert lib.mxgg_wgrad_workspace_size(1, 2048, 256, 256) == 4 * 16 * (256 + 256)
    # staging an e4m3 weight in row pairs: E * N * K rounded up to 64, plus 256
    # bytes of alignment slack, offered for E <= M / 8192 and K >= 4096 (or
    # K >= 2048 with N >= 4096) only
    E4M3, E2M1 = _lib.FMT_E4M3, _lib.FMT_E2M1
    assert lib.mxgg_grouped_mm_staging_size(1, 16640, 2048, 8192, E4M3) == 2048 * 8192 + 256
    assert lib.mxgg_grouped_mm_staging_size(2, 16640, 5120, 4128, E4M3) == 2 * 5120 * 4160 + 256
    assert lib.mxgg_grouped_mm_staging_size(2, 16384, 5120, 5120, E4M3) == 2 * 5120 * 5120 + 256
    assert lib.mxgg_grouped_mm_staging_size(3, 16384, 5120, 5120, E4M3) == 0     # E > M / 8192
    assert lib.mxgg_grouped_mm_staging_size(1, 16640, 2048, 2048, E4M3) == 0     # K, N < 4096
    # ... plus A (M * K rounded up to 64, plus 256) for N >= 8192, K >= 2048, M even and
    # M * N * K above 6e10 (smaller calls run on plain scales without a re-layout launch)
    assert lib.mxgg_grouped_mm_staging_size(1, 16640, 8192, 2048, E4M3) == 8192 * 2048 + 256 + 16640 * 2048 + 256
    assert lib.mxgg_grouped_mm_staging_size(1, 2080, 8192, 2048, E4M3) == 0       # 3.5e10 multiply-adds
    assert lib.mxgg_grouped_mm_staging_size(1, 3584, 8192, 2048, E4M3) == 3584 * 2048 + 256   # 6.01e10 multiply-adds
    assert lib.mxgg_grouped_mm_staging_size(8, 16640, 8192, 5120, E4M3) == 16640 * 5120 + 256   # A only
    assert lib.mxgg_grouped_mm_staging_size(8, 16641, 8192, 5120, E4M3) == 0                  # odd M
    assert lib.mxgg_grouped_mm_staging_size(1, 16640, 8192, 1024, E4M3) == 0     # K < 2048
    assert lib.mxgg_grouped_mm_staging_size(1, 16640, 8191, 8192, E4M3) == 0     # odd N: no row pairs
    assert lib.mxgg_grouped_mm_staging_size(1, 16640, 8192, 8192, E2M1) == 16640 * 8192 + 256   # A only
    assert lib.mxgg_grouped_mm_staging_size(1, 16640, 4096, 8192, E2M1) == 0     # an e2m1 weight is not staged
    assert lib.mxgg_grouped_mm_staging_size(1, 16640, 8192, 8200, E4M3) == 0     # K % 32
    # wgrad: both operands, (N + K) * M rounded up to 64, plus 512; only at N, K >= 8192, or with
    # E >= 8 at N + K >= 10240; not for odd N or K, or M off the 32 grid
    assert lib.mxgg_wgrad_staging_size(1, 16640, 8192, 8192) == 16384 * 16640 + 512
    assert lib.mxgg_wgrad_staging_size(8, 2080, 5120, 5120) == 10240 * 2112 + 512
    assert lib.mxgg_wgrad_staging_size(8, 16640, 2048, 8192) == 10240 * 16640 + 512
    assert lib.mxgg_wgrad_staging_size(1, 16640, 5120, 5120) == 0
    assert lib.mxgg_wgrad_staging_size(4, 16640, 8192, 5120) == 0
    assert lib.mxgg_wgrad_staging_size(8, 16640, 2048, 5120) == 0
    assert lib.mxgg_wgrad_staging_size(2, 16640, 2048, 2048) == 0
    assert lib.mxgg_wgrad_staging_size(1, 16640, 8191, 8192) == 0
    assert lib.mxgg_wgrad_staging_size(1, 16656, 8192, 8192) == 0
    rc = lib.mxgg_grouped_mm(16, 64, 16, 2, 16, 0, 64, 64 * 64, 16, 2, 128, 16, 1, 64, 64, 64,
                             16, 0, 64, 0, 0, 0, 0, None, 0, None)
    assert rc == _lib.ERR_WORKSPACE and b"workspace" in lib.mxgg_last_error_string()
    rc = lib.mxgg_wgrad(16, 64, 16, 2, 16, 64, 16, 2, 16, 1, 64, 8, 8, 16, 0, None, 0, None)
    assert rc == _lib.ERR_WORKSPACE


def test_wgrad_and_quant_validation_without_gpu():
    from kernels import _lib
    lib = _lib.load()
    rc = lib.mxgg_wgrad(16, 48, 16, 1, 16, 48, 16, 1, 16, 1, 48, 8, 8, 16, 0, None, 0, None)
    assert rc == _lib.ERR_INVALID_ARG and b"multiple of 32" in lib.mxgg_last_error_string()
    rc = lib.mxgg_quantize_mx(16, 0, 4, 40, 40, 0, 16, 40, 16, 2, 0, None)
    assert rc == _lib.ERR_INVALID_ARG and b"divisible by block_size 32" in lib.mxgg_last_error_string()
    rc = lib.mxgg_quantize_mx(16, 5, 4, 64, 64, 0, 16, 64, 16, 2, 0, None)
    assert rc == _lib.ERR_INVALID_ARG
    rc = lib.mxgg_quantize_mx_dim0(16, 0, 40, 64, 64, 0, 16, 40, 16, 1, 0, None)
    assert rc == _lib.ERR_INVALID_ARG
    rc = lib.mxgg_quantize_mx_dim0(16, 0, 64, 64, 64, 4, 16, 64, 16, 2, 0, None)
    assert rc == _lib.ERR_UNSUPPORTED
    # empty problems are valid no-ops that never reach the device
    assert lib.mxgg_quantize_mx(None, 0, 0, 64, 64, 0, None, 64, None, 2, 0, None) == 0
    # both-ways quantizer: both dims must be multiples of 32, strides cover the rows
    rc = lib.mxgg_quantize_mx_both(16, 0, 1, 40, 64, 64, 16, 64, 16, 2, 16, 40, 16, 1, 0, None)
    assert rc == _lib.ERR_INVALID_ARG and b"divisible by block_size 32" in lib.mxgg_last_error_string()
    rc = lib.mxgg_quantize_mx_both(16, 0, 1, 64, 64, 64, 16, 64, 16, 2, 16, 32, 16, 2, 0, None)
    assert rc == _lib.ERR_INVALID_ARG and b"stride" in lib.mxgg_last_error_string()
    rc = lib.mxgg_quantize_mx_both(16, 7, 1, 64, 64, 64, 16, 64, 16, 2, 16, 64, 16, 2, 0, None)
    assert rc == _lib.ERR_INVALID_ARG
    assert lib.mxgg_quantize_mx_both(None, 0, 0, 64, 64, 64, None, 64, None, 2, None, 64, None, 2, 0, None) == 0
    # step-major scales: ld_s is the rows per batch and must divide the rows; unknown layout codes fail
    rc = lib.mxgg_quantize_mx(16, 0, 6, 64, 64, 0, 16, 64, 16, 4, _lib.SCALES_STEPS, None)
    assert rc == _lib.ERR_INVALID_ARG and b"rows per batch" in lib.mxgg_last_error_string()
    rc = lib.mxgg_quantize_mx(16, 0, 6, 64, 64, 0, 16, 64, 16, 2, 9, None)
    assert rc == _lib.ERR_INVALID_ARG and b"layout 9" in lib.mxgg_last_error_string()
    rc = lib.mxgg_quantize_mx_dim0(16, 0, 64, 96, 96, 0, 16, 64, 16, 64, _lib.SCALES_STEPS, None)
    assert rc == _lib.ERR_INVALID_ARG
    # GEMMs on step-major scales: scale words must be 4-byte aligned; wgrad still needs M % 32 == 0
    rc = lib.mxgg_grouped_mm_steps(16, 64, 18, 16, 0, 64, 64 * 64, 16, 16, 1, 64, 64, 64,
                                   16, 0, 64, 0, 0, 0, 0, 0, None, 0, None)
    assert rc == _lib.ERR_INVALID_ARG and b"aligned" in lib.mxgg_last_error_string()
    rc = lib.mxgg_wgrad_steps(16, 48, 16, 16, 48, 16, 16, 1, 48, 8, 8, 16, 0, 0, None, 0, None)
    assert rc == _lib.ERR_INVALID_ARG and b"multiple of 32" in lib.mxgg_last_error_string()


def test_wgrad_out_dtypes_without_gpu():
    """wgrad takes bf16, f16 and f32 outputs (kernels/backward.py:251 allocates
    any out_dtype): a valid f16 call passes every argument check and stops only
    at the missing device; an unknown type code is rejected."""
    from kernels import _lib
    lib = _lib.load()
    ws = 4 * 1 * (64 + 64)
    for code in (_lib.DTYPE_BF16, _lib.DTYPE_F16, _lib.DTYPE_F32):
        rc = lib.mxgg_wgrad(16, 64, 16, 2, 16, 64, 16, 2, 16, 1, 64, 64, 64, 16, code, 256, ws, None)
        assert rc == _lib.ERR_NO_DEVICE, (code, lib.mxgg_last_error_string())
    rc = lib.mxgg_wgrad(16, 64, 16, 2, 16, 64, 16, 2, 16, 1, 64, 64, 64, 16, 7, 256, ws, None)
    assert rc == _lib.ERR_INVALID_ARG and b"out_dtype" in lib.mxgg_last_error_string()


def test_wgrad_config_without_gpu():
    """mxgg_wgrad_config checks its arguments on the host, then needs the
    device (its answer depends on the resident workgroup count)."""
    import ctypes
    from kernels import _lib
    lib = _lib.load()
    b = ctypes.c_int32(0)
    assert lib.mxgg_wgrad_config(2, 16640, 2048, 2048, None) == _lib.ERR_INVALID_ARG
    assert lib.mxgg_wgrad_config(0, 16640, 2048, 2048, ctypes.byref(b)) == _lib.ERR_INVALID_ARG
    assert lib.mxgg_wgrad_config(2, 16640, 0, 2048, ctypes.byref(b)) == _lib.ERR_INVALID_ARG
    assert lib.mxgg_wgrad_config(2, 16640, 2048, 2048, ctypes.byref(b)) == _lib.ERR_NO_DEVICE
    assert b.value == 0


def test_noalloc_rejects_calls_beyond_the_array_without_gpu():
    """mxgg_grouped_mm_noalloc rejects a call whose re-laid scales,
    4 * cdiv(K, 128) * (M + E*N) bytes, exceed its device array with
    MXGG_ERR_WORKSPACE, before anything is launched (the check precedes the
    device lookup: a regression would return MXGG_ERR_NO_DEVICE here, never
    launch).  Fake 16-byte-aligned pointers: nothing is dereferenced."""
    from kernels import _lib
    lib = _lib.load()
    E, M, N, K = 8, 16640, 32768, 8192
    assert 4 * (K // 128) * (M + E * N) > _lib.NOALLOC_SCRATCH_BYTES
    p = 1 << 20
    rc = lib.mxgg_grouped_mm_noalloc(p, K, p, K // 32, p, _lib.FMT_E4M3, K, N * K, p, K // 32, N * K // 32,
                                     p, E, M, N, K, p, _lib.DTYPE_BF16, N, 0, 0, 0, 0, None)
    assert rc == _lib.ERR_WORKSPACE
    assert b"scratch" in lib.mxgg_last_error_string()
    # one just inside the array passes the check and stops at the missing device
    M2, N2, K2 = 4096, 4096, 2048
    assert 4 * (K2 // 128) * (M2 + N2) <= _lib.NOALLOC_SCRATCH_BYTES
    rc = lib.mxgg_grouped_mm_noalloc(p, K2, p, K2 // 32, p, _lib.FMT_E4M3, K2, N2 * K2, p, K2 // 32,
                                     N2 * K2 // 32, p, 1, M2, N2, K2, p, _lib.DTYPE_BF16, N2, 0, 0, 0, 0, None)
    assert rc == _lib.ERR_NO_DEVICE


def test_row_pair_argument_checks():
    """Row-pair and row-quad operands (MXGG_DATA_PAIRS / _QUADS, MXGG_A_PAIRS /
    MXGG_B_PAIRS / MXGG_B_QUADS) are checked before anything launches: row
    counts divisible by 2 (4), strides that hold the rows rounded up to the
    64 (32) byte piece, e4m3 (packed e2m1) only, known flags."""
    from kernels import _lib
    lib = _lib.load()
    P, S = _lib.DATA_PAIRS, _lib.SCALES_STEPS
    err = lib.mxgg_last_error_string
    # quantizers: rows must pair up; the stride a multiple of 64 holding the padded row; e4m3 only
    rc = lib.mxgg_quantize_mx(16, 0, 5, 64, 64, 0, 16, 64, 16, 2, P, None)
    assert rc == _lib.ERR_INVALID_ARG and b"divisible by 2" in err()
    rc = lib.mxgg_quantize_mx(16, 0, 6, 96, 96, 0, 16, 112, 16, 3, P, None)
    assert rc == _lib.ERR_INVALID_ARG and b"multiple of 64" in err()
    rc = lib.mxgg_quantize_mx(16, 0, 6, 96, 96, 0, 16, 96, 16, 3, P, None)
    assert rc == _lib.ERR_INVALID_ARG and b"multiple of 64 and holds 128 bytes" in err()
    rc = lib.mxgg_quantize_mx(16, 0, 6, 64, 64, _lib.FMT_E2M1, 16, 64, 16, 2, P, None)
    assert rc == _lib.ERR_UNSUPPORTED
    assert lib.mxgg_quantize_mx(16, 0, 6, 96, 96, 0, 16, 128, 16, 6, P | S, None) != _lib.ERR_INVALID_ARG
    rc = lib.mxgg_quantize_mx_dim0(16, 0, 96, 64, 64, 0, 16, 96, 16, 64, P | S, None)
    assert rc == _lib.ERR_INVALID_ARG and b"multiple of 64" in err()
    rc = lib.mxgg_quantize_mx_both(16, 0, 1, 96, 64, 64, 16, 64, 16, 96, 16, 112, 16, 64, P | S, None)
    assert rc == _lib.ERR_INVALID_ARG and b"multiple of 64" in err()
    # forward: known flags; e4m3 weights only; M / N even; strides hold K rounded up to 64
    fwd = lambda M, N, K, lda, ldb, fmt, layout: lib.mxgg_grouped_mm_steps(
        16, lda, 16, 16, fmt, ldb, N * ldb, 16, 16, 1, M, N, K, 16, 0, N, 0, 0, 0, 0, layout, None, 0, None)
    assert fwd(64, 64, 64, 64, 64, 0, 8) == _lib.ERR_INVALID_ARG and b"layout flags" in err()
    assert fwd(64, 64, 64, 64, 32, _lib.FMT_E2M1, _lib.B_PAIRS) == _lib.ERR_UNSUPPORTED
    assert fwd(63, 64, 64, 64, 64, 0, _lib.A_PAIRS) == _lib.ERR_INVALID_ARG and b"divisible by 2" in err()
    assert fwd(64, 65, 64, 64, 64, 0, _lib.B_PAIRS) == _lib.ERR_INVALID_ARG and b"divisible by 2" in err()
    assert fwd(63, 65, 64, 64, 64, 0, 0) != _lib.ERR_INVALID_ARG       # odd counts are fine row-major
    assert fwd(64, 64, 96, 112, 128, 0, _lib.A_PAIRS) == _lib.ERR_INVALID_ARG and b"stride" in err()
    assert fwd(64, 64, 96, 128, 112, 0, _lib.B_PAIRS) == _lib.ERR_INVALID_ARG and b"stride" in err()
    # row quads: packed e2m1 weights only, N divisible by 4, stride holding K/2 rounded up to 32
    Q = _lib.DATA_QUADS
    assert fwd(64, 64, 64, 64, 64, 0, _lib.B_QUADS) == _lib.ERR_UNSUPPORTED
    assert fwd(64, 64, 64, 64, 32, _lib.FMT_E2M1, _lib.B_QUADS | _lib.B_PAIRS) == _lib.ERR_INVALID_ARG
    assert fwd(64, 66, 64, 64, 32, _lib.FMT_E2M1, _lib.B_QUADS) == _lib.ERR_INVALID_ARG and b"divisible by" in err()
    assert fwd(64, 64, 96, 128, 48, _lib.FMT_E2M1, _lib.B_QUADS) == _lib.ERR_INVALID_ARG and b"stride" in err()
    assert fwd(64, 68, 96, 128, 64, _lib.FMT_E2M1, _lib.B_QUADS) != _lib.ERR_INVALID_ARG
    rc = lib.mxgg_quantize_mx(16, 0, 8, 64, 64, 0, 16, 64, 16, 2, Q, None)
    assert rc == _lib.ERR_UNSUPPORTED                              # quads hold e2m1, not e4m3
    rc = lib.mxgg_quantize_mx(16, 0, 6, 64, 64, _lib.FMT_E2M1, 16, 32, 16, 2, Q, None)
    assert rc == _lib.ERR_INVALID_ARG and b"divisible by 4" in err()
    rc = lib.mxgg_quantize_mx(16, 0, 8, 96, 96, _lib.FMT_E2M1, 16, 48, 16, 3, Q, None)
    assert rc == _lib.ERR_INVALID_ARG and b"multiple of 32 and holds 64 bytes" in err()
    assert lib.mxgg_quantize_mx(16, 0, 8, 96, 96, _lib.FMT_E2M1, 16, 64, 16, 3, Q, None) != _lib.ERR_INVALID_ARG
    assert lib.mxgg_quantize_mx(16, 0, 8, 64, 64, 0, 16, 64, 16, 2, P | Q, None) == _lib.ERR_INVALID_ARG
    assert lib.mxgg_quantize_mx_dim0(16, 0, 64, 64, 64, 0, 16, 64, 16, 64, Q | S, None) == _lib.ERR_UNSUPPORTED
    # wgrad: the same for go_t (A_PAIRS) and ia_t (B_PAIRS) along the tokens
    wg = lambda M, N, K, ldg, ldi, layout: lib.mxgg_wgrad_steps(
        16, ldg, 16, 16, ldi, 16, 16, 1, M, N, K, 16, 0, layout, None, 0, None)
    assert wg(96, 64, 64, 128, 128, 8) == _lib.ERR_INVALID_ARG and b"layout flags" in err()
    assert wg(96, 63, 64, 128, 128, _lib.A_PAIRS) == _lib.ERR_INVALID_ARG and b"even row count" in err()
    assert wg(96, 64, 65, 128, 128, _lib.B_PAIRS) == _lib.ERR_INVALID_ARG and b"even row count" in err()
    assert wg(96, 64, 64, 128, 128, _lib.B_QUADS) == _lib.ERR_INVALID_ARG and b"layout flags" in err()
    assert wg(96, 64, 64, 112, 128, _lib.A_PAIRS) == _lib.ERR_INVALID_ARG and b"stride" in err()
    assert wg(96, 64, 64, 128, 112, _lib.B_PAIRS) == _lib.ERR_INVALID_ARG and b"stride" in err()


def test_import_surface_matches_reference():
    import kernels
    for name in ("triton_mxfp8_grouped_mm", "triton_mxfp8_wgrad", "_rocm_mxfp8_available"):
        assert hasattr(kernels, name)
    assert isinstance(kernels._rocm_mxfp8_available, bool)
    import utils
    for name in ("to_mx", "generate_jagged_offs", "benchmark_cuda_function_in_microseconds", "is_MI350"):
        assert callable(getattr(utils, name))


def test_forward_signature_matches_reference():
    from kernels import triton_mxfp8_grouped_mm
    sig = inspect.signature(triton_mxfp8_grouped_mm)
    want = ["input_act", "weight", "input_act_scales", "weight_scales", "group_end_offsets", "out_dtype",
            "BLOCK_M", "BLOCK_N", "BLOCK_K", "GROUP_M", "XCD_SWIZZLE", "num_warps", "num_stages",
            "matrix_instr_nonkdim", "waves_per_eu", "kpack", "w_cache_modifier", "x_evict_policy"]
    assert list(sig.parameters) == want
    assert sig.parameters["out_dtype"].default is torch.bfloat16
    assert sig.parameters["kpack"].default == 1
    assert all(sig.parameters[n].default is None for n in want[6:15] if n != "kpack")


def test_wgrad_signature_matches_reference():
    from kernels import triton_mxfp8_wgrad
    sig = inspect.signature(triton_mxfp8_wgrad)
    assert list(sig.parameters) == ["go_t", "go_scale", "ia_t", "ia_scale", "group_end_offsets", "out_dtype",
                                    "BLOCK_N", "BLOCK_K", "BLOCK_M", "num_warps", "num_stages"]
    d = {k: v.default for k, v in sig.parameters.items()}
    assert (d["BLOCK_N"], d["BLOCK_K"], d["BLOCK_M"], d["num_warps"], d["num_stages"]) == (256, 256, 64, 8, 2)


def test_to_mx_signature_matches_reference():
    import utils
    sig = inspect.signature(utils.to_mx)
    # the reference's parameters in its order; additions are keyword-only with defaults
    pos = [n for n, p in sig.parameters.items() if p.kind != p.KEYWORD_ONLY]
    assert pos == ["data", "elem_dtype", "block_size"]
    assert sig.parameters["block_size"].default == 32
    extra = [p for p in sig.parameters.values() if p.kind == p.KEYWORD_ONLY]
    assert [(p.name, p.default) for p in extra] == [("scale_layout", "plain"), ("data_layout", "rows")]


def test_cpu_tensors_fail_loudly():
    """No CPU fallback: the operators refuse host tensors."""
    from kernels import to_mx, triton_mxfp8_grouped_mm
    a = torch.zeros((64, 64), dtype=torch.float8_e4m3fn)
    b = torch.zeros((1, 64, 64), dtype=torch.float8_e4m3fn)
    sa = torch.zeros((64, 2), dtype=torch.uint8)
    sb = torch.zeros((1, 64, 2), dtype=torch.uint8)
    with pytest.raises(TypeError):
        triton_mxfp8_grouped_mm(a, b, sa, sb, torch.tensor([64], dtype=torch.int32))
    with pytest.raises(TypeError):
        to_mx(torch.zeros((4, 64), dtype=torch.bfloat16))
    from kernels import to_mx_both
    from kernels.moe import mxfp8_grouped_mm
    with pytest.raises(TypeError):
        to_mx_both(torch.zeros((64, 64), dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        mxfp8_grouped_mm(torch.zeros((64, 64), dtype=torch.bfloat16), torch.zeros((1, 64, 64), dtype=torch.bfloat16),
                         torch.tensor([64], dtype=torch.int32))


def test_shape_errors_match_reference_types():
    from kernels import triton_mxfp8_grouped_mm
    a = torch.zeros((64, 64), dtype=torch.float8_e4m3fn, device="meta")
    b = torch.zeros((1, 64, 96), dtype=torch.float8_e4m3fn, device="meta")
    with pytest.raises((AssertionError, TypeError)):
        triton_mxfp8_grouped_mm(a, b, None, None, None)


def test_missing_library_raises_not_implemented(tmp_path):
    from kernels import _lib
    with pytest.raises(NotImplementedError):
        _lib.load(str(tmp_path / "missing_libmxgg.so"))


def test_generate_jagged_offs_same_draws_as_reference_algorithm():
    import random
    import utils
    random.seed(123)
    o = utils.generate_jagged_offs(8, 16640, device="cpu")
    random.seed(123)
    want = sorted(random.sample(list(range(32, 16641, 32))[:-1], 7)) + [16640]
    assert o.tolist() == want and o.dtype == torch.int32
    with pytest.raises(ValueError):
        utils.generate_jagged_offs(2, 100, device="cpu")
