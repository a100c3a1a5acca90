"""ctypes binding of libmxgg.so (the C ABI declared in include/mxgg.h).

The library is built in-tree next to this file (``make -C grouped-gemms_amd/csrc``
or ``__graft_entry__.build()``).  There is no fallback: when the library is
missing every operator raises ``NotImplementedError``, like the reference's
stubs when its kernels are unavailable (kernels/forward.py:608-612).
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmxgg.so")

# status codes / enums (include/mxgg.h)
OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_WORKSPACE = -3
ERR_NO_DEVICE = -4
NOALLOC_SCRATCH_BYTES = 48 << 20   # MXGG_NOALLOC_SCRATCH_BYTES
FMT_E4M3 = 0
FMT_E2M1 = 4
DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2
SCALES_PLAIN = 0
SCALES_STEPS = 1
DATA_PAIRS = 2      # quantizer data outputs in row pairs (OR-ed into the scale layout)
DATA_QUADS = 4      # quantizer packed e2m1 outputs in row quads
A_PAIRS = 1         # *_steps GEMMs: A / go_t in row pairs
B_PAIRS = 2         # *_steps GEMMs: B / ia_t in row pairs
B_QUADS = 4         # mxgg_grouped_mm_steps: packed e2m1 B in row quads

_c_i32 = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_sz = ctypes.c_size_t
_c_p = ctypes.c_void_p

# (name, restype, argtypes) for every symbol of include/mxgg.h
SIGNATURES = {
    "mxgg_version": (_c_i32, []),
    "mxgg_last_error_string": (ctypes.c_char_p, []),
    "mxgg_device_supported": (_c_i32, []),
    "mxgg_quantize_mx": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i64,
                                  _c_p, _c_i64, _c_i32, _c_p]),
    "mxgg_quantize_mx_dim0": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i32, _c_p, _c_i64,
                                       _c_p, _c_i64, _c_i32, _c_p]),
    "mxgg_quantize_mx_both": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_i64, _c_i64,
                                       _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_i32, _c_p]),
    "mxgg_routing_words": (_c_i64, [_c_i32, _c_i64, _c_i32]),
    "mxgg_build_routing": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i32, _c_p, _c_p]),
    "mxgg_schedule_programs": (_c_i64, [_c_i32, _c_i64, _c_i64, _c_i32, _c_i32]),
    "mxgg_tile_schedule": (_c_i32, [_c_p, _c_i32, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32,
                                    _c_p, _c_p]),
    "mxgg_grouped_mm_workspace_size": (_c_sz, [_c_i32, _c_i64, _c_i64, _c_i64]),
    "mxgg_grouped_mm_staging_size": (_c_sz, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i32]),
    "mxgg_grouped_mm": (_c_i32, [_c_p, _c_i64, _c_p, _c_i64,
                                 _c_p, _c_i32, _c_i64, _c_i64,
                                 _c_p, _c_i64, _c_i64,
                                 _c_p, _c_i32, _c_i64, _c_i64, _c_i64,
                                 _c_p, _c_i32, _c_i64,
                                 _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_sz, _c_p]),
    "mxgg_grouped_mm_steps": (_c_i32, [_c_p, _c_i64, _c_p,
                                       _c_p, _c_i32, _c_i64, _c_i64, _c_p,
                                       _c_p, _c_i32, _c_i64, _c_i64, _c_i64,
                                       _c_p, _c_i32, _c_i64,
                                       _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_p, _c_sz, _c_p]),
    "mxgg_grouped_mm_noalloc": (_c_i32, [_c_p, _c_i64, _c_p, _c_i64,
                                         _c_p, _c_i32, _c_i64, _c_i64,
                                         _c_p, _c_i64, _c_i64,
                                         _c_p, _c_i32, _c_i64, _c_i64, _c_i64,
                                         _c_p, _c_i32, _c_i64,
                                         _c_i32, _c_i32, _c_i32, _c_i32, _c_p]),
    "mxgg_grouped_mm_config": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, _c_i32,
                                        ctypes.POINTER(_c_i32), ctypes.POINTER(_c_i32),
                                        ctypes.POINTER(_c_i32), ctypes.POINTER(_c_i32)]),
    "mxgg_wgrad_workspace_size": (_c_sz, [_c_i32, _c_i64, _c_i64, _c_i64]),
    "mxgg_wgrad_staging_size": (_c_sz, [_c_i32, _c_i64, _c_i64, _c_i64]),
    "mxgg_wgrad_config": (_c_i32, [_c_i32, _c_i64, _c_i64, _c_i64, ctypes.POINTER(_c_i32)]),
    "mxgg_wgrad": (_c_i32, [_c_p, _c_i64, _c_p, _c_i64,
                            _c_p, _c_i64, _c_p, _c_i64,
                            _c_p, _c_i32, _c_i64, _c_i64, _c_i64,
                            _c_p, _c_i32, _c_p, _c_sz, _c_p]),
    "mxgg_wgrad_steps": (_c_i32, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_p,
                                  _c_p, _c_i32, _c_i64, _c_i64, _c_i64,
                                  _c_p, _c_i32, _c_i32, _c_p, _c_sz, _c_p]),
}

_lock = threading.Lock()
_lib = None


def _open(path: str) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise NotImplementedError(f"{path} not built (run make -C grouped-gemms_amd/csrc)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Return the library with typed entry points (loaded once for LIB_PATH)."""
    global _lib
    if path != LIB_PATH:
        return _open(path)
    with _lock:
        if _lib is None:
            _lib = _open(path)
        return _lib


def available() -> bool:
    try:
        load()
        return True
    except (NotImplementedError, OSError):
        return False


class MXGGError(RuntimeError):
    """A libmxgg entry point returned a nonzero status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"libmxgg error {code}: {msg}")
        self.code = code


def check(rc: int) -> None:
    if rc == OK:
        return
    msg = load().mxgg_last_error_string().decode(errors="replace")
    if rc == ERR_INVALID_ARG:
        raise ValueError(msg)
    if rc == ERR_NO_DEVICE:
        raise NotImplementedError(msg)
    raise MXGGError(rc, msg)
