"""bench.py's kernel-name handling (no GPU): which launches are whole-tile
or split-piece GEMM launches in a rocprofv3 trace, and name matching against
the committed profile summaries, whose step-major kernels may be listed
without the Cfg's scale-source argument."""

import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import bench  # noqa: E402


def test_gemm_launch_kinds():
    kinds = {
        "mxgg::fwd_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, false>, false, 1>": "whole",
        "mxgg::fwd_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, false>, true, 0>": "piece",
        "mxgg::fwd_kernel<mxgg::Cfg<128, 128, 2, 2, 0, 4, true>, false, 3>": "whole",
        "mxgg::fwd_kernel<mxgg::Cfg<256, 256, 2, 2, 4, 4, true>, true, 0>": "piece",
        "void mxgg::wgrad_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, false>, false, 1>(mxgg::WgradParams)": "whole",
        "mxgg::fwd_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4>, true, 1>": "piece",
        "mxgg::fwd_quad_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, true>, mxgg::Cfg<128, 128, 2, 2, 0, 4, true>, 1>": None,
        "mxgg::fwd_reduce_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, false> >": None,
        "mxgg::scale_relayout_kernel": None,
    }
    for name, kind in kinds.items():
        assert bench.gemm_launch(name) == kind, name


def test_canon_matches_summaries_without_scale_source():
    new = "mxgg::fwd_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, false>, false, 1>"
    old = "mxgg::fwd_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4>, false, 1>"
    plain = "mxgg::fwd_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, true>, false, 1>"
    assert bench.canon(new) == bench.canon(old)
    assert bench.canon(plain) != bench.canon(old)
    assert bench.canon("void mxgg::fwd_reduce_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, false> >(mxgg::FwdParams)") == \
        bench.canon("mxgg::fwd_reduce_kernel<mxgg::Cfg<256,256,2,2,0,4>>")
    assert bench.fwd_kernel_name({"BLOCK_M": 256, "BLOCK_N": 256}) == new
