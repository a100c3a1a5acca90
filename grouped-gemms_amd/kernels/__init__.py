"""MI355X (gfx950) MX-scaled grouped-GEMM kernels, hand-written HIP behind a C ABI.

Drop-in for the reference package ``kernels`` (kernels/__init__.py:17-25):

  - ``triton_mxfp8_grouped_mm``: forward + dgrad grouped GEMM (A @ B^T per group)
  - ``triton_mxfp8_wgrad``: weight-gradient grouped GEMM (A^T @ B per group)
  - ``_rocm_mxfp8_available``: True when the native library is loadable on ROCm

plus the on-GPU quantizers ``to_mx`` / ``to_mx_dim0`` / ``to_mx_both`` (the
reference quantizes with eager torch ops in utils.py:67-105), whose
``data_layout="pairs"`` output (or ``to_row_pairs`` of row-major data) the
GEMMs copy in whole 128-byte lines.
"""

from ._common import _rocm_mxfp8_available, to_row_pairs, to_row_quads
from .backward import triton_mxfp8_wgrad
from .forward import triton_mxfp8_grouped_mm
from .moe import MXFP8GroupedLinear, mxfp8_grouped_mm
from .quant import to_mx, to_mx_both, to_mx_dim0

__all__ = [
    "triton_mxfp8_grouped_mm",
    "triton_mxfp8_wgrad",
    "_rocm_mxfp8_available",
    "to_mx",
    "to_mx_dim0",
    "to_mx_both",
    "to_row_pairs",
    "to_row_quads",
    "mxfp8_grouped_mm",
    "MXFP8GroupedLinear",
]
