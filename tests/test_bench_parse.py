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
        "void mxgg::fwd_kernel<mxgg::XLine<mxgg::Cfg<256, 256, 2, 2, 0, 3, false> >, false, 1>(mxgg::FwdParams)":
            "whole",
        "mxgg::fwd_kernel<mxgg::XLine<mxgg::Cfg<256, 256, 2, 2, 0, 3, false> >, true, 0>": "piece",
        "mxgg::fwd_quad_kernel<mxgg::XLine<mxgg::Cfg<256, 256, 2, 2, 0, 3, false> >, "
        "mxgg::Cfg<128, 128, 2, 2, 0, 4, false>, 1>": None,
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


def test_fwd_kernel_names_by_layout():
    # row-major A runs the 256 x 256 tiles as XLine (the demangled name of
    # fwd_kernel<XLine<Cfg<256, 256, 2, 2, 0, 3>>, false, 1>); row pairs, and
    # 128 x 128 tiles on either layout, the one-stage configuration
    xl = "void mxgg::fwd_kernel<mxgg::XLine<mxgg::Cfg<256, 256, 2, 2, 0, 3, false> >, false, 1>(mxgg::FwdParams)"
    assert bench.canon(bench.fwd_kernel_name({"BLOCK_M": 256, "BLOCK_N": 256}, rows=True)) == bench.canon(xl)
    assert bench.fwd_kernel_name({"BLOCK_M": 256, "BLOCK_N": 256}) == bench.FWD_KERNEL
    assert bench.fwd_kernel_name({"BLOCK_M": 128, "BLOCK_N": 128}, rows=True) == \
        "mxgg::fwd_kernel<mxgg::Cfg<128, 128, 2, 2, 0, 4, false>, false, 1>"


def test_summary_lines_parse(tmp_path, monkeypatch):
    # the committed kernel-trace summary's per-call and drop-in lines, as
    # stats_summary writes them, read back by the bench's roofline
    prof = tmp_path / "profiles"
    prof.mkdir()
    fw, xl = bench.FWD_KERNEL, bench.XLINE_KERNEL
    (prof / "kernel_stats_sweep.txt").write_text(
        f"  {xl:62s} all calls   5000: avg    400.00 us;  right after the cache flush   4400: avg    410.00 us;"
        f"  the sweep's first 4320: avg    420.50 us\n"
        f"  {fw:62s} all calls   4600: avg    380.00 us;  right after the cache flush   4320: avg    381.00 us;"
        f"  the native sweep's 4320: avg    382.25 us\n"
        f"  the sweep's 4320 drop-in calls of {fw} and {xl}: GEMM launches 401.02 us = 2175.5 TFLOP/s = 0.435 "
        f"of 5000.0 (dense MXFP8); with the re-layout launch (21.29 us) 2065.8 TFLOP/s = 0.413\n")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    assert bench.read_trace_avg(xl, native=False) == (4320, 420.5)
    assert bench.read_trace_avg(fw, native=True) == (4320, 382.25)
    assert bench.read_trace_avg(fw, native=False) is None
    d = bench.read_dropin_gemm(xl)
    assert d is not None and d["calls"] == 4320 and d["frac"] == 0.435 and d["frac_with_relayout"] == 0.413
    assert bench.read_dropin_gemm(fw)["kernels"] == [fw, xl]
    assert bench.read_dropin_gemm(bench.WGRAD_KERNEL) is None
    # the wgrad family's line: the one-stage kernel where the call stages both
    # operands, XLine on row-major go_t
    wk, wx = bench.WGRAD_KERNEL, bench.WGRAD_XLINE
    assert bench.canon(wx) == bench.canon(
        "void mxgg::wgrad_kernel<mxgg::XLine<mxgg::Cfg<256, 256, 2, 2, 0, 3, false> >, false, 1>(mxgg::WgradParams)")
    with open(prof / "kernel_stats_sweep.txt", "a") as f:
        f.write(f"  the sweep's 2100 drop-in calls of {wk} and {wx}: GEMM launches 300.00 us = 2000.0 TFLOP/s = "
                f"0.400 of 5000.0 (dense MXFP8); with the re-layout launch (20.00 us) 1875.0 TFLOP/s = 0.375\n")
    w = bench.read_dropin_gemm(wx)
    assert w is not None and w["calls"] == 2100 and w["kernels"] == [wk, wx] and w["frac_with_relayout"] == 0.375
    assert bench.read_dropin_gemm(xl)["calls"] == 4320
