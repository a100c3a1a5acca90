"""Benchmark of the MX grouped-GEMM hot path on one MI355X.

Workload (BASELINE.json configs 3 and 4): the reference's 36-shape Llama4
sweep, E in {1,2,4,8}, M = 16640 tokens, N, K in {2048, 5120, 8192}, run as
  * forward  out = A (M,K) @ B[g]^T (E,N,K)            (the headline)
  * dgrad    out = grad_out (M,N) @ W^T[g]^T (E,K,N)
  * wgrad    out[g] = grad_out[g]^T @ A[g]  -> (E,N,K)
with jagged offsets drawn exactly like the reference's bench (random.seed(123),
``generate_jagged_offs`` in config order; bench.py:113-122, 250-257).  Inputs
are synthetic (A, grad_out ~ N(0,1), weights ~ N(0,0.02)), quantized on the GPU
before timing; quantization is outside the timed region, as in the reference
(bench.py:126-130).  Beside the forward, the bf16 arm times torch._grouped_mm
on the unquantized operands (reference bench.py:159-161) for the speedup the
reference's README quotes (1.389x geomean MXFP8 vs bf16, README.md:80).

Timed region per shape: the full drop-in Python call (output allocation, the
C-ABI call, the scale re-layout, the in-kernel routing and the GEMM),
bracketed by HIP events on the current stream after a 512 MB cache flush;
median over ``--steps`` reps after ``--warmup`` reps.  TFLOPs = 2*M*N*K / t
(bench.py:200).  A "step" is one call per shape over all 108 problems;
ms_per_step is the sum of the medians.

Beside it, each call is timed again on step-major scales (the layout the
kernels read, so the call launches no re-layout): between its events lie
only the GEMM launches of the call (the whole-tile kernel, and the piece /
quarter-tile / reduce launches when its last round is split).  The roofline
of the dominant kernel uses that time.  After the sweep, it runs once more on
the operands' native layout (``kernels.quant``: step-major scales and row-pair
data, ``data_layout="pairs"``, written by the quantizers outside the timed
region): kernel-only time again, reported as ``native_geomean_tflops`` and
``roofline_native`` beside the drop-in headline.  Also measured
(e4m3 x e2m1, E=8, M=16640, N=8192, K=5120), the quantizer in GB/s, one
training step (forward + backward) of the MoE layer (kernels/moe.py) and one
GPU's share of the sweep under 8-way expert parallelism (E=1, M=2080).

CPU baseline (``cpu_baseline``): the reference's CPU path -- torch to_mx on
the host, dequantize, one fp32 torch.matmul per group -- on BASELINE config 1
at full size with torch's intra-op threads, beside the GPU drop-in time of the
same quantized operands.

Prints ONE JSON line on stdout, with the per-shape medians of the sweep in its
``rows`` field; progress and the per-shape table also go to stderr and, when
the output folder DETAIL_DIR (below) exists, to bench_detail.json there.
"""

from __future__ import annotations

import argparse
import itertools
import json
import math
import os
import platform
import random
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
DETAIL_DIR = "gpurun_out"   # per-shape detail file goes here when the folder exists
sys.path.insert(0, os.path.join(ROOT, "grouped-gemms_amd"))

PEAK_MXFP8_TFLOPS = 5000.0          # MI355X published dense MXFP8 / FP8 peak
PEAK_MXFP4_TFLOPS = 10100.0         # MI355X published dense MXFP4 peak
PEAK_HBM_GBS = 8000.0               # MI355X HBM3E
REF_FWD_GEOMEAN_TFLOPS = 1498.8     # reference README table, 36-shape fwd geomean (MI355X)
REF_SPEEDUP_VS_BF16 = 1.389         # reference README, geomean MXFP8 / bf16 torch._grouped_mm (MI355X)
REF_BF16_GEOMEAN_TFLOPS = 1079.0    # reference README table, bf16 torch._grouped_mm geomean (MI355X)
M_TOKENS = 16640
SHAPES = [(e, n, k) for e, n, k in itertools.product((1, 2, 4, 8), (2048, 5120, 8192), (2048, 5120, 8192))]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_call(fn, steps: int, warmup: int, flush_buf):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    en = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    for i in range(steps):
        flush_buf.zero_()
        st[i].record()
        fn()
        en[i].record()
    torch.cuda.synchronize()
    ts = [a.elapsed_time(b) for a, b in zip(st, en)]
    return statistics.median(ts), sum(ts) / len(ts)


def fwd_kernel_name(cfg: dict, rows: bool = False) -> str:
    """Device-kernel name (as rocprofv3 lists it) of the whole-tile kernel of an
    e4m3 forward/dgrad launch on step-major scales: Cfg<BLOCK_M, BLOCK_N, waves
    along M, waves along N, B format, LDS stages, plain scales>, pieces=false,
    bf16 epilogue; with ``rows`` (row-major A), the 256 x 256 tiles run as
    XLine (A in two-stage LDS slots, 3 of them).  A call may also launch the
    piece / quarter-tile / reduce kernels of a split last round; the
    kernel-only event time covers those too."""
    if rows and cfg["BLOCK_M"] == 256:
        return XLINE_KERNEL
    return f"mxgg::fwd_kernel<mxgg::Cfg<{cfg['BLOCK_M']}, {cfg['BLOCK_N']}, 2, 2, 0, 4, false>, false, 1>"


# the 256 x 256 e4m3 forward whole-tile kernels: A in row pairs, and row-major A (XLine)
FWD_KERNEL = "mxgg::fwd_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, false>, false, 1>"
XLINE_KERNEL = "mxgg::fwd_kernel<mxgg::XLine<mxgg::Cfg<256, 256, 2, 2, 0, 3, false> >, false, 1>"


# whole-tile kernels with the bf16 epilogue (template argument 1): the bench's outputs are bf16 with aligned rows
WGRAD_KERNEL = "mxgg::wgrad_kernel<mxgg::Cfg<256, 256, 2, 2, 0, 4, false>, false, 1>"
WGRAD_XLINE = "mxgg::wgrad_kernel<mxgg::XLine<mxgg::Cfg<256, 256, 2, 2, 0, 3, false> >, false, 1>"


def wgrad_kernel_name(E: int, M: int, N: int, K: int, rows: bool = False) -> str:
    """Device-kernel name of the whole-tile kernel of a wgrad call of this
    shape: 256 x 256 (WGRAD_KERNEL) or, where the library picks them
    (mxgg_wgrad_config, needs the GPU), 128 x 128 tiles; with ``rows``
    (row-major go_t) the 256 x 256 tiles run as XLine (WGRAD_XLINE)."""
    import ctypes
    from kernels import _lib
    b = ctypes.c_int32(0)
    _lib.check(_lib.load().mxgg_wgrad_config(E, M, N, K, ctypes.byref(b)))
    if rows and b.value == 256:
        return WGRAD_XLINE
    return f"mxgg::wgrad_kernel<mxgg::Cfg<{b.value}, {b.value}, 2, 2, 0, 4, false>, false, 1>"


def canon(kernel: str) -> str:
    """Kernel name without return type, arguments and blanks, for matching
    names across demanglers (``> >`` vs ``>>``), and without the Cfg's scale
    source argument where it is the default step-major one (``false``): the
    names of summaries made before that argument existed match the same
    kernels."""
    k = kernel.replace("void ", "").split("(")[0].replace(" ", "")
    return re.sub(r"(Cfg<\d+,\d+,\d+,\d+,\d+,\d+),false>", r"\1>", k)


def gemm_launch(name: str):
    """'whole' / 'piece' for a whole-tile / split-piece launch of the forward
    or wgrad GEMM kernel (their last two template arguments: pieces, epilogue),
    else None (quarter-tile, reduce and other kernels)."""
    if not ("mxgg::fwd_kernel<" in name or "mxgg::wgrad_kernel<" in name):
        return None
    m = re.search(r">,\s*(true|false),\s*\d+>\s*$", name.replace("void ", "").split("(")[0])
    return None if m is None else ("piece" if m.group(1) == "true" else "whole")


def read_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    (profiles/hbm_traffic_sweep.txt, lines `traffic_bytes_per_launch <kernel> = <bytes>`),
    or None when no measurement of that kernel is recorded."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_sweep.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch ") and "=" in line:
            name, val = line[len("traffic_bytes_per_launch "):].rsplit("=", 1)
            if canon(name) == canon(kernel):
                return float(val)
    return None


def read_trace_avg(kernel: str, native: bool):
    """(calls, average µs) of `kernel`'s kernel-only calls in the committed
    kernel-trace summary (profiles/kernel_stats_sweep.txt: the span of each
    call's GEMM dispatches, the sweep's first cold calls, or the native
    sweep's after them), or None when the summary lacks that kernel."""
    path = os.path.join(ROOT, "profiles", "kernel_stats_sweep.txt")
    if not os.path.exists(path):
        return None
    pat = (r"the native sweep's (\d+)(?: after them)?: avg\s+([\d.]+) us" if native
           else r"the sweep's first (\d+): avg\s+([\d.]+) us")
    for line in open(path):
        head = line.strip().split("all calls")[0].strip()
        if head and canon(head) == canon(kernel):
            m = re.search(pat, line)
            if m:
                return int(m.group(1)), float(m.group(2))
    return None


def read_dropin_gemm(kernel: str):
    """The drop-in calls' figures of `kernel` in the committed kernel-trace
    summary (profiles/kernel_stats_sweep.txt: the GEMM launches the sweep's
    timed drop-in calls make, on operands staged in row pairs where the
    library stages them, without and with their re-layout launch; a line
    may cover several whole-tile kernels, "A and B"), or None."""
    path = os.path.join(ROOT, "profiles", "kernel_stats_sweep.txt")
    if not os.path.exists(path):
        return None
    pat = (r"the sweep's (\d+) drop-in calls of (.+?): GEMM launches ([\d.]+) us = ([\d.]+) TFLOP/s = ([\d.]+) of "
           r".*re-layout launch \(([\d.]+) us\) ([\d.]+) TFLOP/s = ([\d.]+)")
    for line in open(path):
        m = re.search(pat, line)
        if m and canon(kernel) in {canon(n) for n in m.group(2).split(" and ")}:
            return {"calls": int(m.group(1)), "kernels": m.group(2).split(" and "),
                    "gemm_us": float(m.group(3)), "achieved": float(m.group(4)),
                    "frac": float(m.group(5)), "relayout_us": float(m.group(6)),
                    "achieved_with_relayout": float(m.group(7)), "frac_with_relayout": float(m.group(8)),
                    "source": "profiles/kernel_stats_sweep.txt: rocprofv3 kernel-trace spans of the GEMM launches "
                              "inside the sweep's timed drop-in calls of a profiled run of this bench (operands as "
                              "the drop-in call stages them), and of their re-layout launch"}
    return None


def copy_calibration(dev, mib: int = 256, reps: int = 3):
    """A plain device copy of known size, run so that a PMC pass over this
    program can scale FETCH_SIZE / WRITE_SIZE (the copy moves mib MiB each way)."""
    import torch
    src = torch.empty(mib << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: {reps} copies of {mib} MiB")
    del src, dst


def pmc_summary(fetch_csv: str, write_csv: str, steps: int, warmup: int, n_shapes: int,
                kernel_only: bool = False) -> str:
    """HBM bytes per launch of each GEMM kernel from two rocprofv3 --pmc passes
    (FETCH_SIZE, WRITE_SIZE; KiB per dispatch) over
    ``bench.py --steps S --warmup W --no-cpu --no-bf16 --no-extra --copy-calibration``.

    Each counter is scaled so that the calibration copy (256 MiB each way)
    reads 256 MiB; dispatches are matched to sweep shapes by launch order
    (per shape: fwd, dgrad, wgrad, each call timed twice, warmup + steps
    launches each; then the native-layout sweep, each call once) to set the
    algorithmic bytes beside the measured ones.  Kernels of the native sweep
    are listed with the suffix " [row pairs]"."""
    import csv

    def load(path, counter):
        rows = [(int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"]))
                for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
        return sorted(rows)

    out = []
    scaled = {}
    for path, counter in ((fetch_csv, "FETCH_SIZE"), (write_csv, "WRITE_SIZE")):
        rows = load(path, counter)
        cal = [v for _, n, v in rows[:64] if "copyBuffer" in n and v > 1e4][:3]
        if len(cal) != 3:
            raise SystemExit(f"{path}: calibration copies not found")
        factor = (256 * 1024.0) / (sum(cal) / 3)
        out.append(f"{counter}: calibration copy reads {sum(cal) / 3:.1f} KiB per 256 MiB copy -> "
                   f"scale factor {factor:.4f}")
        # whole-tile GEMM kernels only: one per call (piece / reduce kernels of a
        # split last round, when launched, are left out of the per-call match)
        scaled[counter] = [(n, v * factor * 1024.0) for _, n, v in rows
                           if gemm_launch(n) == "whole"]
    f, w = scaled["FETCH_SIZE"], scaled["WRITE_SIZE"]
    # each call is timed twice (plain scales, then step-major; with
    # --kernel-only step-major only), warmup + steps launches each; the
    # native sweep times each call once
    shapes = SHAPES[:n_shapes]
    want = []
    for tag, per in (("", (1 if kernel_only else 2) * (warmup + steps)), (NATIVE_TAG, warmup + steps)):
        for (e, n, k) in shapes:
            for kind in ("fwd", "dgrad", "wgrad"):
                if kind == "wgrad":
                    alg = (n + k) * M_TOKENS * (1 + 1 / 32) + 2 * e * n * k
                else:
                    nn, kk = (n, k) if kind == "fwd" else (k, n)
                    alg = M_TOKENS * kk * (1 + 1 / 32) + e * nn * kk * (1 + 1 / 32) + 2 * M_TOKENS * nn
                want += [(kind, alg, (e, n, k), tag)] * per
    if len(f) != len(w):
        raise SystemExit(f"dispatch count mismatch: fetch {len(f)}, write {len(w)}")
    # a wgrad call whose tiles are all split launches no whole-tile kernel:
    # its entry in `want` has no dispatch and is skipped
    matched = []
    i = 0
    for kind, alg, shape, tag in want:
        if i >= len(f) and tag:
            break                # a run without the native sweep (--no-native)
        if i < len(f) and (("wgrad" in f[i][0]) == (kind == "wgrad")):
            matched.append((f[i], w[i], (kind, alg, shape, tag)))
            i += 1
        elif kind != "wgrad":
            raise SystemExit(f"dispatch {i} ({f[i][0] if i < len(f) else 'none'}) does not match a {kind} call")
    if i != len(f):
        raise SystemExit(f"{len(f) - i} dispatches left unmatched")
    agg, by_shape = {}, {}
    for (nf, vf), (nw, vw), (kind, alg, shape, tag) in matched:
        assert nf == nw and (("wgrad" in nf) == (kind == "wgrad")), (nf, nw, kind)
        name = nf.replace("void ", "").split("(")[0] + tag
        for a in (agg.setdefault(name, [0.0, 0.0, 0.0, 0]), by_shape.setdefault((shape, kind + tag), [0.0, 0.0, 0.0, 0])):
            a[0] += vf
            a[1] += vw
            a[2] += alg
            a[3] += 1
    out.append(f"{'kernel':58s} {'launches':>8s} {'fetch MB':>9s} {'write MB':>9s} {'total MB':>9s} "
               f"{'algorithmic MB':>14s} {'ratio':>6s}")
    for name, (vf, vw, alg, c) in sorted(agg.items()):
        out.append(f"{name:58s} {c:8d} {vf / c / 1e6:9.1f} {vw / c / 1e6:9.1f} {(vf + vw) / c / 1e6:9.1f} "
                   f"{alg / c / 1e6:14.1f} {(vf + vw) / alg:6.2f}")
    for name, (vf, vw, alg, c) in sorted(agg.items()):
        out.append(f"traffic_bytes_per_launch {name} = {(vf + vw) / c:.0f}")
    out += ["", "Per shape (E, N, K) and direction, whole-tile kernel: fetch + write MB per launch / algorithmic MB"]
    for (shape, kind), (vf, vw, alg, c) in sorted(by_shape.items()):
        out.append(f"  {shape[0]} {shape[1]:5d} {shape[2]:5d} {kind:17s} {vf / c / 1e6:8.1f} + {vw / c / 1e6:6.1f}"
                   f" / {alg / c / 1e6:6.1f} = {(vf + vw) / alg:5.2f}")
    return "\n".join(out)


def counter_summary(csv_path: str) -> str:
    """Per-kernel mean of every counter in a ``rocprofv3 --pmc`` counter CSV
    (GEMM kernels only), e.g. MfmaUtil / LdsBankConflict over a bench run."""
    import csv
    acc = {}
    for r in csv.DictReader(open(csv_path)):
        n = r["Kernel_Name"].replace("void ", "").split("(")[0]
        if "mxgg::" not in n or "quant" in n:
            continue
        a = acc.setdefault(n, {}).setdefault(r["Counter_Name"], [0.0, 0])
        a[0] += float(r["Counter_Value"])
        a[1] += 1
    names = sorted({c for v in acc.values() for c in v})
    # full kernel names: the trailing template arguments (pieces, epilogue)
    # tell the launches of one configuration apart
    w = max([62] + [len(n) for n in acc])
    out = [f"{'kernel':{w}s} " + " ".join(f"{c:>16s}" for c in names) + f" {'dispatches':>10s}"]
    for n, v in sorted(acc.items()):
        cells = " ".join(f"{v[c][0] / v[c][1]:16.4f}" if c in v else f"{'-':>16s}" for c in names)
        out.append(f"{n:{w}s} {cells} {max(x[1] for x in v.values()):10d}")
    return "\n".join(out)


GEMM_KERNELS = ("mxgg::fwd_kernel<", "mxgg::fwd_quad_kernel<", "mxgg::fwd_reduce_kernel<", "mxgg::wgrad_kernel<",
                "mxgg::wgrad_reduce_kernel<")


def call_spans(trace_csv: str):
    """GEMM calls in a ``rocprofv3 --kernel-trace`` CSV: each run of
    consecutive GEMM dispatches that starts with a whole-tile kernel (between
    the bench's cache flush, scale re-layout or quantizer kernels) is one
    call.  Returns {whole-tile kernel of the call: [(span ns, cold), ...]},
    span = last end - first start (what the bench's kernel-only events
    bracket); cold: the call directly follows the 512 MB cache flush (a torch
    fill kernel), as the bench's timed kernel-only reps do (its warmup reps
    and the drop-in calls, whose re-layout sits in between, do not)."""
    import csv
    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
                  for r in csv.DictReader(open(trace_csv)))
    spans, cur, prev = {}, None, ""

    def close():
        if cur is not None and cur[2]:
            spans.setdefault(cur[2], []).append((cur[1] - cur[0], cur[3]))
        elif cur is not None and cur[4]:
            # every tile of the call split: pieces and reduce only, counted with
            # the whole-tile kernel of the same configuration (as the bench does)
            spans.setdefault(cur[4], []).append((cur[1] - cur[0], cur[3]))

    for t0, t1, name in rows:
        n = name.replace("void ", "").split("(")[0]
        if any(n.startswith(g) for g in GEMM_KERNELS):
            whole = gemm_launch(n) == "whole"
            if cur is not None and whole and cur[2]:
                close()          # back-to-back calls: a call's whole-tile kernel comes first
                cur = None
            if cur is None:
                cur = [t0, t1, None, "FillFunctor" in prev, None]
            cur[1] = max(cur[1], t1)
            if whole:
                cur[2] = n
            elif gemm_launch(n) == "piece":
                cur[4] = re.sub(r", true, \d+>$", ", false, 1>", n)
        else:
            close()
            cur = None
        prev = n if not any(n.startswith(g) for g in GEMM_KERNELS) else prev
    close()
    return spans


def dropin_spans(trace_csv: str):
    """Drop-in calls in a ``rocprofv3 --kernel-trace`` CSV that directly
    follow the bench's cache flush (its timed drop-in reps): the scale
    re-layout launch (which also stages operands in row pairs where the
    library does), then the call's GEMM dispatches.  Returns {whole-tile
    kernel of the call: [(re-layout ns, GEMM span ns, start ns), ...]} in
    trace order; a call whose every tile is split counts under the whole-tile
    kernel of its configuration."""
    import csv
    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"].replace("void ", "").split("(")[0])
                  for r in csv.DictReader(open(trace_csv)))
    out, i = {}, 0
    while i + 1 < len(rows):
        if "FillFunctor" in rows[i][2] and rows[i + 1][2].startswith("mxgg::scale_relayout_kernel"):
            relayout = rows[i + 1][1] - rows[i + 1][0]
            j, g0, g1, whole, piece, reduced = i + 2, None, None, None, None, False
            while j < len(rows) and any(rows[j][2].startswith(g) for g in GEMM_KERNELS):
                t0, t1, n = rows[j]
                is_whole = gemm_launch(n) == "whole"
                is_piece = gemm_launch(n) == "piece"
                # the next call's GEMM launches (unflushed warmup reps of the bench's next variant follow
                # directly): a second whole-tile launch, or a piece launch after this call's reduce
                if (is_whole and g0 is not None) or (is_piece and reduced):
                    break
                g0 = t0 if g0 is None else g0
                g1 = t1 if g1 is None else max(g1, t1)
                if is_whole:
                    whole = n
                elif is_piece:
                    piece = piece or re.sub(r", true, \d+>$", ", false, 1>", n)
                reduced = reduced or "_reduce_kernel<" in n
                j += 1
            if (whole or piece) and g0 is not None:
                out.setdefault(whole or piece, []).append((relayout, g1 - g0, rows[i][0]))
            i = j
        else:
            i += 1
    return out


def ep_summary(trace_csv: str, ep_json: str) -> str:
    """Per-call timeline of the expert-parallel shard measurement (``bench.py
    --ep-only`` under ``rocprofv3 --kernel-trace``): its timed calls each follow
    the 512 MB cache flush, so every run of kernels between two flushes is one
    call.  The calls come in the measurement's order -- per (N, K): the drop-in
    forward, the drop-in wgrad, then both on the native layout -- and each
    (shape, kind) block is one run of consecutive calls with the same kernel
    signature.  Per block: median span (first start to last end), and the
    median duration of the scale re-layout launch and of each GEMM launch."""
    import csv
    rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"].replace("void ", "").split("(")[0])
                  for r in csv.DictReader(open(trace_csv)))
    calls, cur = [], None
    for t0, t1, n in rows:
        if "FillFunctor" in n:
            if cur:
                calls.append(cur)
            cur = []
        elif cur is not None and n.startswith("mxgg::"):
            cur.append((t0, t1, n))
    if cur:
        calls.append(cur)
    short = lambda n: re.sub(r"mxgg::|\(.*", "", n)
    blocks, sig = [], None
    for c in calls:
        if not c:
            continue
        g = tuple(short(n) for _, _, n in c)
        if g != sig:
            blocks.append([])
            sig = g
        blocks[-1].append(c)
    ep = json.loads(open(ep_json).read().strip().splitlines()[-1])["ep_shard"]["rows"]
    kinds = ("fwd drop-in", "wgrad drop-in", "fwd native", "wgrad native")
    med = lambda xs: statistics.median(xs) if xs else 0.0
    out = ["shape (N, K)   call            calls  span us  re-layout us  GEMM launches (median us each)"]
    # the blocks of short warm-up runs (no flush in between) merge with a neighbour; keep those with most calls
    blocks = [b for b in blocks if len(b) >= 10]
    for i, b in enumerate(blocks):
        shape = ep[i // 4] if i // 4 < len(ep) else {"N": "?", "K": "?"}
        spans = [c[-1][1] - c[0][0] for c in b]
        rl = [t1 - t0 for c in b for t0, t1, n in c if "relayout" in n]
        gemm = {}
        for c in b:
            for t0, t1, n in c:
                if "relayout" not in n:
                    gemm.setdefault(short(n), []).append(t1 - t0)
        g = "; ".join(f"{k} {med(v) / 1e3:.1f}" for k, v in gemm.items())
        out.append(f"({shape['N']}, {shape['K']})  {kinds[i % 4]:14s} {len(b):6d} {med(spans) / 1e3:8.1f} "
                   f"{med(rl) / 1e3 if rl else 0.0:12.1f}  {g}")
    return "\n".join(out)


def stats_summary(stats_csv: str, bench_json: str, trace_csv: str = None) -> str:
    """Per-kernel table of a ``rocprofv3 --kernel-trace --stats`` run over the
    default bench (its ``*_kernel_stats.csv``), the per-call GEMM spans from
    its kernel trace when given, and the same run's own HIP-event figures per
    GEMM kernel (the JSON line bench.py printed)."""
    import csv
    out = [f"{'kernel':78s} {'calls':>6s} {'total ms':>9s} {'avg us':>9s} {'min us':>8s} {'max us':>8s} {'%':>6s}"]
    for r in csv.DictReader(open(stats_csv)):
        name = r["Name"].replace("void ", "").split("(")[0]
        out.append(f"{name[:78]:78s} {int(r['Calls']):6d} {float(r['TotalDurationNs']) / 1e6:9.2f} "
                   f"{float(r['AverageNs']) / 1e3:9.2f} {float(r['MinNs']) / 1e3:8.1f} "
                   f"{float(r['MaxNs']) / 1e3:8.1f} {float(r['Percentage']):6.2f}")
    line = None
    for text in open(bench_json):
        if text.startswith("{"):
            line = json.loads(text)
    bench_calls, native_calls = {}, {}
    if line and line.get("roofline"):
        bench_calls = {canon(k): v["launches"] for k, v in line["roofline"]["by_kernel"].items()}
    if line and line.get("roofline_native"):
        native_calls = {canon(k): v["launches"] for k, v in line["roofline_native"]["by_kernel"].items()}
    if trace_csv:
        out += ["", "Per call, from the kernel trace: the span of each call's GEMM dispatches (whole-tile kernel "
                    "and any split / quarter-tile / reduce launches), by the call's whole-tile kernel; the sweep's "
                    "timed kernel-only calls are the first cold ones, since the sweep runs first:"]
        for name, v in sorted(call_spans(trace_csv).items()):
            cold = [t for t, c in v if c]
            text = (f"  {name:62s} all calls {len(v):6d}: avg {sum(t for t, _ in v) / len(v) / 1e3:9.2f} us;  "
                    f"right after the cache flush {len(cold):6d}: avg "
                    f"{(sum(cold) / len(cold) / 1e3) if cold else float('nan'):9.2f} us")
            nb = bench_calls.get(canon(name), 0)
            if nb and len(cold) >= nb:
                text += f";  the sweep's first {nb}: avg {sum(cold[:nb]) / nb / 1e3:9.2f} us"
            nn = native_calls.get(canon(name))
            if nn and len(cold) >= nb + nn and (nb == 0 or len(cold) >= nb):
                text += (f";  the native sweep's {nn}{' after them' if nb else ''}: avg "
                         f"{sum(cold[nb:nb + nn]) / nn / 1e3:9.2f} us")
            out.append(text)
    if trace_csv and line and line.get("roofline"):
        # the GEMM launches the drop-in calls make, on the operands as the
        # call hands them over (staged in row pairs where the library stages
        # them); the sweep's timed drop-in reps are the first cold ones, and
        # its forward + dgrad (wgrad) calls number what the kernel-only
        # roofline counts, over the same shapes
        rf = line["roofline"]
        spans = dropin_spans(trace_csv)
        out += ["", "Drop-in calls, from the same trace: each timed rep's scale re-layout launch (with any operand "
                    "staging) and the span of its GEMM launches:"]
        for name, v in sorted(spans.items()):
            out.append(f"  {name:62s} calls {len(v):6d}: re-layout avg {sum(x[0] for x in v) / len(v) / 1e3:8.2f} us, "
                       f"GEMM span avg {sum(x[1] for x in v) / len(v) / 1e3:9.2f} us")
        # the kernel-only sweep's row-major forward + dgrad calls all run the
        # XLine kernel, their drop-in twins it or, where the call stages A in
        # row pairs, the one-stage 256 x 256 kernel; the wgrad's likewise (the
        # one-stage kernel where the call stages both operands): each family's
        # calls in trace order
        for fam in ((FWD_KERNEL, XLINE_KERNEL), (WGRAD_KERNEL, WGRAD_XLINE)):
            names = {canon(f) for f in fam}
            v = sorted((x for k, xs in spans.items() if canon(k) in names for x in xs), key=lambda x: x[2])
            key = next((k for k in rf["by_kernel"] if canon(k) in names), None)
            bk = rf["by_kernel"].get(key) if key else None
            if not bk or len(v) < bk["launches"]:
                continue
            nb = bk["launches"]
            flops = bk["tflops"] * 1e12 * bk["avg_launch_us"] * 1e-6
            gem = sum(x[1] for x in v[:nb]) / nb
            rel = sum(x[0] for x in v[:nb]) / nb
            ach = flops / (gem * 1e-9) / 1e12
            whole_call = flops / ((gem + rel) * 1e-9) / 1e12
            label = " and ".join(fam)
            out.append(f"  the sweep's {nb} drop-in calls of {label}: GEMM launches {gem / 1e3:.2f} us = {ach:.1f} "
                       f"TFLOP/s = {ach / PEAK_MXFP8_TFLOPS:.3f} of {PEAK_MXFP8_TFLOPS} (dense MXFP8); with the "
                       f"re-layout launch ({rel / 1e3:.2f} us) {whole_call:.1f} TFLOP/s = "
                       f"{whole_call / PEAK_MXFP8_TFLOPS:.3f}")
    if line and line.get("roofline"):
        out += ["", "Same run, bench.py's own figures (HIP events on the launch stream, timed reps only):"]
        for key, tag in (("roofline", ""), ("roofline_native", NATIVE_TAG)):
            rf = line.get(key)
            if not rf:
                continue
            for name, v in sorted(rf["by_kernel"].items()):
                out.append(f"  {name + tag:70s} avg {v['avg_launch_us']:9.2f} us over {v['launches']:5d} launches, "
                           f"{v['tflops']:7.1f} TFLOP/s")
            out.append(f"  dominant kernel {rf['kernel']}{tag}: achieved {rf['achieved']} TFLOP/s = {rf['frac']} of "
                       f"{rf['peak']} (dense MXFP8), {rf['avg_launch_us']} us per call ({rf.get('scope', '')})")
        out.append(f"  headline: fwd geomean {line['fwd_geomean_tflops']}  dgrad {line['dgrad_geomean_tflops']}  "
                   f"wgrad {line['wgrad_geomean_tflops']} TFLOP/s; kernel-only {line.get('kernel_only_geomean_tflops')}"
                   f"; native layout {line.get('native_geomean_tflops')}")
    return "\n".join(out)


def geomean(xs):
    return math.exp(sum(math.log(x) for x in xs) / len(xs))


def cpu_baseline(budget_s: float, dev, flush, steps: int, warmup: int):
    """The reference's CPU path, timed on this host's cores beside the HIP path
    on the same problem: BASELINE config 1 at full size (E=4, M=1024,
    N=K=512, the config the reference's CPU-runnable pieces cover), quantized
    on the CPU with the torch restatement of to_mx (utils.py:84-105; bits equal
    to the GPU quantizer's), then dequantize -> one fp32 torch.matmul per
    group -> bf16 with torch's intra-op threads (oracle/torch_ref.py), about
    two thirds of `budget_s`.  `gpu_us` is the drop-in forward of the same
    quantized operands on the GPU (median, same flush as the sweep).  The
    numpy port of the oracle on a row slice of config 2's shape is kept as
    `port_sample` for the rest of the budget."""
    import numpy as np
    import torch
    sys.path.insert(0, ROOT)
    from oracle import mx_oracle as O
    from oracle import torch_ref as T
    import kernels

    threads = torch.get_num_threads()
    E, M, N, K = 4, 1024, 512, 512
    g = torch.Generator().manual_seed(0)
    a = torch.randn((M, K), generator=g).to(torch.bfloat16)
    b = (torch.randn((E, N, K), generator=g) * 0.02).to(torch.bfloat16)
    offs = [int(v) for v in O.generate_jagged_offs(E, M, 32, rng=random.Random(0))]
    sa, qa = T.to_mx(a)
    sb, qb = T.to_mx(b)
    flops = 2.0 * M * N * K
    # the HIP path on the same operands
    da, dsa, db, dsb = (t.to(dev) for t in (qa, sa, qb, sb))
    doffs = torch.tensor(offs, dtype=torch.int32, device=dev)
    gpu_ms, _ = time_call(lambda: kernels.triton_mxfp8_grouped_mm(da, db, dsa, dsb, doffs), steps, warmup, flush)
    gpu_out = kernels.triton_mxfp8_grouped_mm(da, db, dsa, dsb, doffs).cpu()
    t_total, reps, out = 0.0, 0, None
    while t_total < budget_s * 2 / 3 or reps < 3:
        t0 = time.perf_counter()
        out = T.grouped_mm(qa, sa, qb, sb, offs)
        t_total += time.perf_counter() - t0
        reps += 1
    per = t_total / reps
    agree = O.rel_fro(out.float().numpy(), gpu_out.float().numpy())

    # the numpy port (oracle) on a slice of config 2's shape
    rng = np.random.default_rng(1)
    rows, N2 = 2048, 2048
    a2 = rng.standard_normal((rows, N2), dtype=np.float32)
    b2 = (rng.standard_normal((1, N2, N2), dtype=np.float32) * 0.02).astype(np.float32)
    s2a, q2a = O.to_mx(a2, src="f32")
    s2b, q2b = O.to_mx(b2, src="f32")
    p_total, p_reps = 0.0, 0
    while p_total < budget_s / 3 or p_reps < 2:
        t0 = time.perf_counter()
        O.f32_to_bf16_bits(O.grouped_mm(q2a, s2a, q2b, s2b, np.array([rows], np.int32), dtype=np.float32))
        p_total += time.perf_counter() - t0
        p_reps += 1
    return {"value": round(flops / per / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "threads": threads,
            "kind": "port",
            "workload": "BASELINE config 1 at full size: E=4, M=1024, N=K=512, offs random.Random(0) "
                        f"{offs}, e4m3 + e8m0 operands (torch to_mx on the CPU, utils.py:84-105)",
            "sample": f"torch CPU path (dequantize -> per-group fp32 torch.matmul -> bf16, oracle/torch_ref.py), "
                      f"{reps} reps in {t_total:.1f}s, torch threads={threads}, "
                      f"cpu={platform.processor() or platform.machine()}, os.cpu_count={os.cpu_count()}",
            "us": round(per * 1e6, 1),
            "gpu_us": round(gpu_ms * 1e3, 2),
            "gpu_tflops": round(flops / (gpu_ms * 1e-3) / 1e12, 2),
            "gpu_over_cpu": round(per / (gpu_ms * 1e-3), 1),
            "gpu_vs_cpu_rel_fro": round(agree, 6),
            "port_sample": {"value": round(2.0 * rows * N2 * N2 / (p_total / p_reps) / 1e12, 5), "unit": "TFLOP/s",
                            "sample": f"numpy oracle fwd (dequantize -> fp32 matmul -> bf16), E=1, M={rows}, "
                                      f"N=K={N2}, {p_reps} reps in {p_total:.1f}s"}}


NATIVE_TAG = " [row pairs]"


def kernel_geomeans(rows, suffix):
    """{fwd, dgrad, wgrad}: geomean TFLOP/s over the rows of the per-call
    times stored under ``<direction><suffix>`` (None when a row lacks one)."""
    return {d: (round(geomean([r["M"] * 2.0 * r["N"] * r["K"] / (r[d + suffix] * 1e-6) / 1e12 for r in rows]), 1)
                if rows and all(d + suffix in r for r in rows) else None)
            for d in ("fwd", "dgrad", "wgrad")}


def make_roofline(stats, tag, scope):
    """Roofline of the dominant device kernel of `stats` (largest summed
    time over the timed reps): algorithmic FLOPs 2*M*N*K per call / the mean
    time of the call's GEMM launches (HIP events on the launch stream; the
    split / quarter-tile tails included).  tag: suffix of the kernel's entry
    in the committed HBM-traffic summary.  Beside it, `profile`: the same
    FLOPs over the mean per-call span the committed kernel-trace summary
    records for those calls (rocprofv3 durations of a profiled run of this
    bench), when it has them."""
    if not stats:
        return None
    kname, k = max(stats.items(), key=lambda kv: kv[1]["ms"])
    achieved = k["flops"] / (k["ms"] * 1e-3) / 1e12
    prof = None
    tr = read_trace_avg(kname, bool(tag))
    if tr:
        p_ach = k["flops"] / k["launches"] / (tr[1] * 1e-6) / 1e12
        prof = {"avg_launch_us": tr[1], "calls": tr[0], "achieved": round(p_ach, 1),
                "frac": round(p_ach / PEAK_MXFP8_TFLOPS, 4),
                "source": "profiles/kernel_stats_sweep.txt: rocprofv3 kernel-trace spans of the same calls in a "
                          "profiled run of this bench (this run's FLOPs per call)"}
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_MXFP8_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_MXFP8_TFLOPS, 4),
            "traffic": read_traffic(kname + tag), "kernel": kname, "scope": scope,
            "avg_launch_us": round(k["ms"] / k["launches"] * 1e3, 2),
            "flops_per_launch": round(k["flops"] / k["launches"]),
            "launches": k["launches"],
            "profile": prof,
            "dropin_gemm": None if tag else read_dropin_gemm(kname),
            "by_kernel": {n: {"avg_launch_us": round(v["ms"] / v["launches"] * 1e3, 2),
                              "tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 1),
                              "launches": v["launches"]} for n, v in stats.items()}}


def native_sweep(dev, args, flush, shapes, offs_by_shape, rows, account):
    """The sweep's calls on the native operand layout: step-major scales and
    row-pair data from the quantizers (``data_layout="pairs"``), GEMM launches
    only between the events.  Stores ``<direction>_native_us`` in the sweep's
    rows and accounts each call to `account`."""
    import torch
    from kernels import to_mx, to_mx_dim0, triton_mxfp8_grouped_mm, triton_mxfp8_wgrad
    from kernels.forward import _pick_config
    lay = {"scale_layout": "steps", "data_layout": "pairs"}
    by_shape = {(r["E"], r["N"], r["K"]): r for r in rows}
    for (E, N, K) in shapes:
        M = M_TOKENS
        offs = offs_by_shape[(E, N, K)]
        flops = 2.0 * M * N * K
        row = by_shape[(E, N, K)]

        def timed(key, fn, kernel):
            med, mean = time_call(fn, args.steps, args.warmup, flush)
            row[key] = med * 1e3
            account(kernel, mean, flops)

        if args.only in ("all", "fwd"):
            ta, pa = to_mx(torch.randn((M, K), device=dev).to(torch.bfloat16), **lay)
            tw, pw = to_mx((torch.randn((E, N, K), device=dev) * 0.02).to(torch.bfloat16), **lay)
            timed("fwd_native_us", lambda: triton_mxfp8_grouped_mm(pa, pw, ta, tw, offs),
                  fwd_kernel_name(_pick_config(E, M, N, K)))
            del ta, pa, tw, pw
        if args.only in ("all", "dgrad"):
            tg, pg = to_mx(torch.randn((M, N), device=dev).to(torch.bfloat16), **lay)
            tt, pt = to_mx((torch.randn((E, K, N), device=dev) * 0.02).to(torch.bfloat16), **lay)
            timed("dgrad_native_us", lambda: triton_mxfp8_grouped_mm(pg, pt, tg, tt, offs),
                  fwd_kernel_name(_pick_config(E, M, K, N)))
            del tg, pg, tt, pt
        if args.only in ("all", "wgrad"):
            tg, pg = to_mx_dim0(torch.randn((M, N), device=dev).to(torch.bfloat16), **lay)
            ti, pi = to_mx_dim0(torch.randn((M, K), device=dev).to(torch.bfloat16), **lay)
            timed("wgrad_native_us", lambda: triton_mxfp8_wgrad(pg, tg, pi, ti, offs), wgrad_kernel_name(E, M, N, K))
            del tg, pg, ti, pi
        torch.cuda.empty_cache()
        log(json.dumps({"E": E, "N": N, "K": K, **{k: round(v, 1) for k, v in row.items() if k.endswith("_native_us")}}))


def extra_measurements(dev, args, flush):
    """BASELINE config 5 (MXFP8 x MXFP4 forward, E=8, M=16640, N=8192,
    K=5120, offsets drawn with random.seed(4)) as a drop-in call, as
    kernel-only time and on the native layout (row pairs / row quads), and
    the quantizer's bandwidth on the sweep's largest
    activation (16640 x 8192 bf16): to_mx (2 + 1 + 1/32 B per element),
    to_mx_dim0 (the same bytes, transposed output) and to_mx_both (both
    layouts from one read: 2 + 2 * (1 + 1/32) B per element)."""
    import torch
    from kernels import to_mx, to_mx_both, to_mx_dim0, triton_mxfp8_grouped_mm
    from utils import generate_jagged_offs
    M, E, N, K = M_TOKENS, 8, 8192, 5120
    random.seed(4)
    offs = generate_jagged_offs(E, M, multiple_of=32, device=dev)
    g = torch.Generator(device=dev).manual_seed(4)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn((E, N, K), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    fp4 = torch.float4_e2m1fn_x2
    sa, qa = to_mx(a)
    sw, qw = to_mx(w, elem_dtype=fp4)
    ta, pa = to_mx(a, scale_layout="steps", data_layout="pairs")
    tw, pw = to_mx(w, elem_dtype=fp4, scale_layout="steps", data_layout="quads")
    del a, w
    flops = 2.0 * M * N * K
    med, _ = time_call(lambda: triton_mxfp8_grouped_mm(qa, qw, sa, sw, offs), args.steps, args.warmup, flush)
    kmed, _ = time_call(lambda: triton_mxfp8_grouped_mm(qa, qw, ta, tw, offs), args.steps, args.warmup, flush)
    nmed, _ = time_call(lambda: triton_mxfp8_grouped_mm(pa, pw, ta, tw, offs), args.steps, args.warmup, flush)
    tf = flops / (med * 1e-3) / 1e12
    cfg5 = {"workload": "BASELINE config 5: e4m3 activations x e2m1 weights, E=8, M=16640, N=8192, K=5120, "
                        "offs random.seed(4)",
            "us": round(med * 1e3, 1), "tflops": round(tf, 1),
            "frac_of_mxfp4_peak": round(tf / PEAK_MXFP4_TFLOPS, 4), "frac_of_mxfp8_peak": round(tf / PEAK_MXFP8_TFLOPS, 4),
            "kernel_only_us": round(kmed * 1e3, 1), "kernel_only_tflops": round(flops / (kmed * 1e-3) / 1e12, 1),
            "native_us": round(nmed * 1e3, 1), "native_tflops": round(flops / (nmed * 1e-3) / 1e12, 1),
            "native_layout": "activations in row pairs, e2m1 weights in row quads, step-major scales"}
    del qa, qw, sa, sw, ta, tw, pa, pw
    torch.cuda.empty_cache()
    x = torch.randn((M, 8192), device=dev).to(torch.bfloat16)
    n = x.numel()
    # what a plain device copy of the same tensor reaches under the same cache
    # flush (the zeroed flush buffer's dirty lines drain during every timed rep)
    y = torch.empty_like(x)
    cmed, _ = time_call(lambda: y.copy_(x), args.steps, args.warmup, flush)
    copy_gbs = 2 * x.numel() * x.element_size() / (cmed * 1e-3) / 1e9
    del y
    quant = {"workload": "bf16 (16640, 8192) -> e4m3 + e8m0 per 32, FLOOR scales (utils.py:67-105)",
             "copy_reference": {"us": round(cmed * 1e3, 1), "gb_s": round(copy_gbs, 1),
                                "what": "torch copy_ of the same bf16 tensor (read + write), same flush"}}
    for name, fn, bpe in (("to_mx", lambda: to_mx(x), 2 + 1 + 1 / 32),
                          ("to_mx_dim0", lambda: to_mx_dim0(x), 2 + 1 + 1 / 32),
                          ("to_mx_both", lambda: to_mx_both(x), 2 + 2 * (1 + 1 / 32))):
        qmed, _ = time_call(fn, args.steps, args.warmup, flush)
        gbs = n * bpe / (qmed * 1e-3) / 1e9
        quant[name] = {"us": round(qmed * 1e3, 1), "bytes_per_elem": round(bpe, 4), "gb_s": round(gbs, 1),
                       "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                       "frac_of_copy_rate": round(gbs / copy_gbs, 4)}
    del x
    torch.cuda.empty_cache()
    moe = moe_layer_measurement(dev, args, flush)
    ep = ep_shard_measurement(dev, args, flush)
    log(json.dumps({"cfg5": cfg5, "quant": quant, "moe_layer": moe, "ep_shard": ep}))
    return {"cfg5": cfg5, "quant": quant, "moe_layer": moe, "ep_shard": ep}


def round_sweep(dev, args, flush):
    """Per-round time of whole forward launches against the reduction length:
    E=1, M=16384, N=8192 is 2048 tiles of 256 x 256, exactly 8 rounds of the
    256 resident workgroups (no split, no quarter-tile tail), at K = 256 ..
    8192, on row-major data and on the native layout (step-major scales both).
    A least-squares line over K >= 1024 (the ring runs at least 6 stages)
    splits a round into a cost per 64-element stage and a fixed cost per tile
    (set-up, the first copies' latency, the epilogue, the dispatch gap)."""
    import torch
    from kernels import to_mx, triton_mxfp8_grouped_mm
    M, N, rounds = 16384, 8192, 8
    offs = torch.tensor([M], dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    rows = []
    for k in (256, 512, 1024, 2048, 4096, 8192):
        a = torch.randn((M, k), device=dev, generator=g).to(torch.bfloat16)
        w = (torch.randn((1, N, k), device=dev, generator=g) * 0.02).to(torch.bfloat16)
        row = {"K": k, "stages": max(6, (k // 64 + 1) & ~1)}
        for lay, kw in (("rows", {"scale_layout": "steps"}), ("pairs", {"scale_layout": "steps", "data_layout": "pairs"})):
            sa, qa = to_mx(a, **kw)
            sw, qw = to_mx(w, **kw)
            med, _ = time_call(lambda: triton_mxfp8_grouped_mm(qa, qw, sa, sw, offs), args.steps, args.warmup, flush)
            row[f"{lay}_round_us"] = round(med * 1e3 / rounds, 2)
            del sa, qa, sw, qw
        rows.append(row)
        del a, w
    torch.cuda.empty_cache()
    fit = {}
    for lay in ("rows", "pairs"):
        pts = [(r["stages"], r[f"{lay}_round_us"]) for r in rows if r["K"] >= 1024]
        n = len(pts)
        mx = sum(x for x, _ in pts) / n
        my = sum(y for _, y in pts) / n
        slope = sum((x - mx) * (y - my) for x, y in pts) / sum((x - mx) ** 2 for x, _ in pts)
        fit[lay] = {"us_per_stage": round(slope, 3), "fixed_us_per_tile": round(my - slope * mx, 2)}
    return {"workload": "E=1, M=16384, N=8192 forward (2048 tiles = 8 rounds of 256), step-major scales, "
                        "cache-flushed calls", "rows": rows, "fit_K_ge_1024": fit}


def ep_shard_measurement(dev, args, flush):
    """One GPU's share of the sweep under 8-way expert parallelism: E=8 over
    8 GPUs leaves one expert and about M/8 = 2080 tokens per GPU, so each
    (N, K) of the sweep becomes an E=1, M=2080 problem (a few hundred tiles,
    where the last round's handling decides the time).  Forward and wgrad,
    drop-in calls, geomean TFLOP/s over the 9 (N, K); beside them the same
    calls on the native layout (step-major scales, row-pair data)."""
    import torch
    from kernels import to_mx, to_mx_dim0, triton_mxfp8_grouped_mm, triton_mxfp8_wgrad
    M = M_TOKENS // 8
    offs = torch.tensor([M], dtype=torch.int32, device=dev)
    g = torch.Generator(device=dev).manual_seed(8)
    rows = []
    for n, k in itertools.product((2048, 5120, 8192), (2048, 5120, 8192)):
        a = torch.randn((M, k), device=dev, generator=g).to(torch.bfloat16)
        w = (torch.randn((1, n, k), device=dev, generator=g) * 0.02).to(torch.bfloat16)
        go = torch.randn((M, n), device=dev, generator=g).to(torch.bfloat16)
        sa, qa = to_mx(a)
        sw, qw = to_mx(w)
        sg, qg = to_mx_dim0(go)
        si, qi = to_mx_dim0(a)
        lay = {"scale_layout": "steps", "data_layout": "pairs"}
        ta, pa = to_mx(a, **lay)
        tw, pw = to_mx(w, **lay)
        tg, pg = to_mx_dim0(go, **lay)
        ti, pi = to_mx_dim0(a, **lay)
        flops = 2.0 * M * n * k
        fmed, _ = time_call(lambda: triton_mxfp8_grouped_mm(qa, qw, sa, sw, offs), args.steps, args.warmup, flush)
        wmed, _ = time_call(lambda: triton_mxfp8_wgrad(qg, sg, qi, si, offs), args.steps, args.warmup, flush)
        fnat, _ = time_call(lambda: triton_mxfp8_grouped_mm(pa, pw, ta, tw, offs), args.steps, args.warmup, flush)
        wnat, _ = time_call(lambda: triton_mxfp8_wgrad(pg, tg, pi, ti, offs), args.steps, args.warmup, flush)
        tf = lambda ms: round(flops / (ms * 1e-3) / 1e12, 1)
        rows.append({"N": n, "K": k, "fwd_us": round(fmed * 1e3, 1), "fwd_tflops": tf(fmed),
                     "wgrad_us": round(wmed * 1e3, 1), "wgrad_tflops": tf(wmed),
                     "fwd_native_tflops": tf(fnat), "wgrad_native_tflops": tf(wnat)})
        del a, w, go, sa, qa, sw, qw, sg, qg, si, qi, ta, pa, tw, pw, tg, pg, ti, pi
    torch.cuda.empty_cache()
    return {"workload": "E=1, M=2080 (16640 tokens / 8 GPUs), N, K in (2048, 5120, 8192): one GPU's expert-parallel "
                        "share of the sweep's E=8 shapes, drop-in calls",
            "fwd_geomean_tflops": round(geomean([r["fwd_tflops"] for r in rows]), 1),
            "wgrad_geomean_tflops": round(geomean([r["wgrad_tflops"] for r in rows]), 1),
            "native_fwd_geomean_tflops": round(geomean([r["fwd_native_tflops"] for r in rows]), 1),
            "native_wgrad_geomean_tflops": round(geomean([r["wgrad_native_tflops"] for r in rows]), 1),
            "rows": rows}


def moe_layer_measurement(dev, args, flush):
    """One training step of the MoE expert projection (kernels/moe.py):
    forward and backward of MXFP8GroupedLinear(E=8, 5120 -> 8192) on 16640
    tokens (offsets random.seed(5)), i.e. to_mx_both of x, w and grad_out, the
    forward GEMM, dgrad and wgrad; 6*M*N*K FLOPs per step.  Beside it, the
    three GEMMs alone on operands in the layer's layouts (step-major scales,
    row-pair data), so the rest of the step (quantization, allocation,
    autograd) is step - GEMMs."""
    import torch
    from kernels import to_mx_both, triton_mxfp8_grouped_mm, triton_mxfp8_wgrad
    from kernels.moe import _LAYOUTS, MXFP8GroupedLinear
    from utils import generate_jagged_offs
    M, E, K, N = M_TOKENS, 8, 5120, 8192
    random.seed(5)
    offs = generate_jagged_offs(E, M, multiple_of=32, device=dev)
    torch.manual_seed(5)
    layer = MXFP8GroupedLinear(E, K, N, device=dev)
    x = torch.randn((M, K), device=dev).to(torch.bfloat16).requires_grad_()
    g = torch.randn((M, N), device=dev).to(torch.bfloat16)

    def fwd():
        with torch.no_grad():
            layer(x, offs)

    def step():
        x.grad = None
        layer.weight.grad = None
        layer(x, offs).backward(g)

    fmed, _ = time_call(fwd, args.steps, args.warmup, flush)
    smed, _ = time_call(step, args.steps, args.warmup, flush)
    x.grad = None
    layer.weight.grad = None
    with torch.no_grad():
        (sx, qx), (sxt, qxt) = to_mx_both(x.detach(), **_LAYOUTS)
        (sw, qw), (swt, qwt) = to_mx_both(layer.weight.detach(), **_LAYOUTS)
        (sg, qg), (sgt, qgt) = to_mx_both(g, **_LAYOUTS)
    gemm = {
        "fwd": time_call(lambda: triton_mxfp8_grouped_mm(qx, qw, sx, sw, offs), args.steps, args.warmup, flush)[0],
        "dgrad": time_call(lambda: triton_mxfp8_grouped_mm(qg, qwt, sg, swt, offs), args.steps, args.warmup,
                           flush)[0],
        "wgrad": time_call(lambda: triton_mxfp8_wgrad(qgt, sgt, qxt, sxt, offs), args.steps, args.warmup, flush)[0],
    }
    del layer, x, g, qx, qw, qxt, qwt, qg, qgt, sx, sw, sxt, swt, sg, sgt
    torch.cuda.empty_cache()
    gsum = sum(gemm.values())
    return {"workload": "MXFP8GroupedLinear E=8, 5120 -> 8192, M=16640 bf16 tokens, offs random.seed(5): "
                        "forward + backward (to_mx_both of x, w, grad_out; fwd, dgrad, wgrad GEMMs)",
            "fwd_us": round(fmed * 1e3, 1), "step_us": round(smed * 1e3, 1),
            "step_tflops": round(6.0 * M * N * K / (smed * 1e-3) / 1e12, 1),
            "gemm_only_us": {k: round(v * 1e3, 1) for k, v in gemm.items()},
            "gemm_share_of_step": round(gsum / smed, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60, help="timed reps per shape")
    ap.add_argument("--warmup", type=int, default=20, help="untimed reps per shape")
    ap.add_argument("--only", choices=("all", "fwd", "dgrad", "wgrad"), default="all")
    ap.add_argument("--shapes", type=int, default=36, help="first N shapes of the sweep")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-bf16", action="store_true",
                    help="skip the bf16 torch._grouped_mm arm of the forward (reference bench.py:159-161)")
    ap.add_argument("--no-native", action="store_true",
                    help="skip the second sweep on row-pair data (the native layout)")
    ap.add_argument("--native-only", action="store_true",
                    help="run only the sweep on row-pair data (for counter passes of that layout)")
    ap.add_argument("--kernel-only", action="store_true",
                    help="time only the calls on step-major scales (the row-major kernel-only figures), not the "
                         "drop-in calls, which may stage operands in row pairs: for counter passes of the "
                         "row-major layout")
    ap.add_argument("--ep-only", action="store_true",
                    help="run only the expert-parallel shard measurement (E=1, M=2080; for kernel traces of it)")
    ap.add_argument("--round-sweep", action="store_true",
                    help="run only the per-round forward timing against K (per-stage and per-tile costs)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the BASELINE config 5 (e4m3 x e2m1) and quantizer measurements")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 3 plain 256 MiB device copies (PMC byte-counter calibration)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarize two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) of "
                         "`bench.py --steps S --warmup W --no-cpu --copy-calibration [--kernel-only]` (same S, W, "
                         "--shapes, --kernel-only) and exit; runs on the CPU")
    ap.add_argument("--ep-summary", nargs=2, metavar=("TRACE_CSV", "EP_JSON"),
                    help="per-call timeline of a rocprofv3 --kernel-trace run of `bench.py --ep-only` (its "
                         "kernel_trace.csv and the JSON line it printed) and exit; runs on the CPU")
    ap.add_argument("--counter-summary", metavar="COUNTER_CSV",
                    help="per-kernel means of a rocprofv3 --pmc counter CSV and exit; runs on the CPU")
    ap.add_argument("--stats-summary", nargs="+", metavar="CSV",
                    help="STATS_CSV BENCH_JSON [TRACE_CSV]: summarize a rocprofv3 --kernel-trace --stats run of "
                         "the default bench (its kernel_stats.csv, the JSON line it printed and, optionally, its "
                         "kernel_trace.csv) and exit; runs on the CPU")
    args = ap.parse_args()
    if args.counter_summary:
        print(counter_summary(args.counter_summary))
        return
    if args.ep_summary:
        print(ep_summary(*args.ep_summary))
        return
    if args.stats_summary:
        print(stats_summary(*args.stats_summary))
        return
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary[0], args.pmc_summary[1], args.steps, args.warmup, args.shapes,
                          args.kernel_only))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import kernels
    from kernels import to_mx, to_mx_dim0, triton_mxfp8_grouped_mm, triton_mxfp8_wgrad
    from kernels.forward import _pick_config
    from utils import generate_jagged_offs

    if not kernels._rocm_mxfp8_available or not torch.cuda.is_available():
        raise SystemExit("libmxgg / GPU unavailable")
    dev = torch.device("cuda:0")
    torch.manual_seed(123)
    random.seed(123)
    flush = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.int32, device=dev)
    shapes = SHAPES[: args.shapes]
    offs_by_shape = {s: generate_jagged_offs(s[0], M_TOKENS, multiple_of=32, device=dev) for s in shapes}
    if args.copy_calibration:
        copy_calibration(dev)
    if args.ep_only:
        print(json.dumps({"ep_shard": ep_shard_measurement(dev, args, flush)}), flush=True)
        return
    if args.round_sweep:
        print(json.dumps({"round_sweep": round_sweep(dev, args, flush)}), flush=True)
        return

    rows = []
    # per device kernel: summed event time (ms), FLOPs and launches of the timed reps
    kstats = {}

    def account(kernel, mean_ms, flops, stats=kstats):
        k = stats.setdefault(kernel, {"ms": 0.0, "flops": 0.0, "launches": 0})
        k["ms"] += mean_ms * args.steps
        k["flops"] += flops * args.steps
        k["launches"] += args.steps

    t_start = time.time()
    def kernel_only(key, fn, kernel, flops, row):
        """Time the same call on step-major scales (only its GEMM launches lie
        between the events) and account it to `kernel`'s roofline."""
        kmed, kmean = time_call(fn, args.steps, args.warmup, flush)
        row[key] = kmed * 1e3
        account(kernel, kmean, flops)

    for (E, N, K) in shapes:
        M = M_TOKENS
        offs = offs_by_shape[(E, N, K)]
        flops = 2.0 * M * N * K
        row = {"E": E, "M": M, "N": N, "K": K}
        if args.native_only:
            rows.append(row)
            continue
        if args.only in ("all", "fwd"):
            a = torch.randn((M, K), device=dev).to(torch.bfloat16)
            w = (torch.randn((E, N, K), device=dev) * 0.02).to(torch.bfloat16)
            sa, qa = to_mx(a)
            sw, qw = to_mx(w)
            ta, _ = to_mx(a, scale_layout="steps")
            tw, _ = to_mx(w, scale_layout="steps")
            if not args.no_bf16:
                # bf16 arm: torch's grouped GEMM on the unquantized operands, as the
                # reference's bench does (bench.py:159-161), but with the weight as a
                # contiguous (E, K, N) tensor: the reference passes a transposed view
                # of (E, N, K), and transposed right operands of torch's bf16 batched
                # products have faulted GPUs of this pool
                wk = w.transpose(-2, -1).contiguous()
                bmed, _ = time_call(lambda: torch._grouped_mm(a, wk, offs, out_dtype=torch.bfloat16),
                                    args.steps, args.warmup, flush)
                row["bf16_us"] = bmed * 1e3
                row["bf16_tflops"] = flops / (bmed * 1e-3) / 1e12
                del wk
            del a, w
            if not args.kernel_only:
                med, mean = time_call(lambda: triton_mxfp8_grouped_mm(qa, qw, sa, sw, offs),
                                      args.steps, args.warmup, flush)
                row["fwd_us"] = med * 1e3
                row["fwd_tflops"] = flops / (med * 1e-3) / 1e12
                if "bf16_us" in row:
                    row["fwd_speedup_vs_bf16"] = row["bf16_us"] / row["fwd_us"]
            kernel_only("fwd_kernel_us", lambda: triton_mxfp8_grouped_mm(qa, qw, ta, tw, offs),
                        fwd_kernel_name(_pick_config(E, M, N, K), rows=True), flops, row)
            del qa, qw, sa, sw, ta, tw
        if args.only in ("all", "dgrad"):
            go = torch.randn((M, N), device=dev).to(torch.bfloat16)
            wt = (torch.randn((E, K, N), device=dev) * 0.02).to(torch.bfloat16)   # W^T (E,K,N)
            sg, qg = to_mx(go)
            st_, qt = to_mx(wt)
            tg, _ = to_mx(go, scale_layout="steps")
            tt, _ = to_mx(wt, scale_layout="steps")
            del go, wt
            if not args.kernel_only:
                med, mean = time_call(lambda: triton_mxfp8_grouped_mm(qg, qt, sg, st_, offs),
                                      args.steps, args.warmup, flush)
                row["dgrad_us"] = med * 1e3
                row["dgrad_tflops"] = flops / (med * 1e-3) / 1e12
            kernel_only("dgrad_kernel_us", lambda: triton_mxfp8_grouped_mm(qg, qt, tg, tt, offs),
                        fwd_kernel_name(_pick_config(E, M, K, N), rows=True), flops, row)
            del qg, qt, sg, st_, tg, tt
        if args.only in ("all", "wgrad"):
            go = torch.randn((M, N), device=dev).to(torch.bfloat16)
            ia = torch.randn((M, K), device=dev).to(torch.bfloat16)
            sg, qg = to_mx_dim0(go)          # (N, M)
            si, qi = to_mx_dim0(ia)          # (K, M)
            tg, _ = to_mx_dim0(go, scale_layout="steps")
            ti, _ = to_mx_dim0(ia, scale_layout="steps")
            del go, ia
            if not args.kernel_only:
                med, mean = time_call(lambda: triton_mxfp8_wgrad(qg, sg, qi, si, offs),
                                      args.steps, args.warmup, flush)
                row["wgrad_us"] = med * 1e3
                row["wgrad_tflops"] = flops / (med * 1e-3) / 1e12
            kernel_only("wgrad_kernel_us", lambda: triton_mxfp8_wgrad(qg, tg, qi, ti, offs),
                        wgrad_kernel_name(E, M, N, K, rows=True), flops, row)
            del qg, qi, sg, si, tg, ti
        torch.cuda.empty_cache()
        rows.append(row)
        log(json.dumps({k: (round(v, 1) if isinstance(v, float) else v) for k, v in row.items()}))

    # the sweep again on row-pair data (after the whole row-major sweep, so
    # that a kernel trace lists the row-major kernel-only calls first)
    nstats = {}
    if not args.no_native or args.native_only:
        native_sweep(dev, args, flush, shapes, offs_by_shape, rows,
                     lambda kernel, mean_ms, flops: account(kernel, mean_ms, flops, nstats))
    extra = None if args.no_extra else extra_measurements(dev, args, flush)

    def gm(key):
        vals = [r[key] for r in rows if key in r]
        return geomean(vals) if vals else None

    fwd_gm, dgrad_gm, wgrad_gm = gm("fwd_tflops"), gm("dgrad_tflops"), gm("wgrad_tflops")
    bf16_gm, speedup_gm = gm("bf16_tflops"), gm("fwd_speedup_vs_bf16")
    ms_per_step = sum(r.get("fwd_us", 0) + r.get("dgrad_us", 0) + r.get("wgrad_us", 0) for r in rows) / 1e3
    per_e = {}
    for e in (1, 2, 4, 8):
        v = [r["fwd_tflops"] for r in rows if r["E"] == e and "fwd_tflops" in r]
        if v:
            per_e[str(e)] = round(geomean(v), 1)

    # roofline of the dominant device kernel (largest summed time over the timed
    # reps): algorithmic FLOPs 2*M*N*K per call / the mean time of the call's
    # GEMM launches on step-major scales (HIP events on the launch stream; no
    # re-layout launch between them, the split / quarter-tile tails included)
    roofline = make_roofline(kstats, "", "GEMM launches of one call on step-major scales and row-major data: "
                                         "the whole-tile kernel, plus the piece / quarter-tile / reduce launches "
                                         "of a split last round")
    roofline_native = make_roofline(nstats, NATIVE_TAG, "the same launches on row-pair data (native layout)")

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_budget, dev, flush, args.steps, args.warmup)
    value = fwd_gm if fwd_gm is not None else (dgrad_gm or wgrad_gm)
    if value is None:            # --kernel-only / --native-only: no drop-in call was timed
        value = next((v for v in list(kernel_geomeans(rows, "_kernel_us").values()) +
                      list(kernel_geomeans(rows, "_native_us").values()) if v), 0.0)
    line = {
        "metric": "geomean MXFP8 grouped-GEMM TFLOPs (% of MXFP8 peak), fwd/dgrad/wgrad, 1 GPU",
        "value": round(value, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(fwd_gm / REF_FWD_GEOMEAN_TFLOPS, 4) if fwd_gm else None,
        "dtype": "mxfp8-e4m3 (e8m0 per-32 scales, fp32 accumulate, bf16 out)",
        "data": "synthetic",
        "config": {"workload": f"{len(rows)}-shape Llama4 MoE sweep, E in (1,2,4,8), M=16640, "
                               f"N,K in (2048,5120,8192); fwd (headline value), dgrad, wgrad",
                   "offs": "generate_jagged_offs, multiples of 32, random.seed(123)"},
        "fwd_geomean_tflops": round(fwd_gm, 1) if fwd_gm else None,
        "dgrad_geomean_tflops": round(dgrad_gm, 1) if dgrad_gm else None,
        "wgrad_geomean_tflops": round(wgrad_gm, 1) if wgrad_gm else None,
        "fwd_pct_of_peak": round(100 * fwd_gm / PEAK_MXFP8_TFLOPS, 2) if fwd_gm else None,
        "bf16_fwd_geomean_tflops": round(bf16_gm, 1) if bf16_gm else None,
        "bf16_arm": "torch._grouped_mm on the unquantized operands, weight as a contiguous (E, K, N) tensor "
                    "(the reference times a transposed (E, N, K) view, not run here), so the same-run speedup "
                    "below is not the README's; fwd_speedup_vs_readme_bf16 divides by the README's own bf16 "
                    "geomean (1079 TFLOP/s, MI355X)",
        "fwd_speedup_vs_bf16_geomean": round(speedup_gm, 3) if speedup_gm else None,
        "fwd_speedup_vs_readme_bf16": round(fwd_gm / REF_BF16_GEOMEAN_TFLOPS, 3) if fwd_gm else None,
        "ref_speedup_vs_bf16_geomean": REF_SPEEDUP_VS_BF16,
        "drop_in_staging": "inside the timed drop-in calls, the re-layout launch also copies an e4m3 weight "
                           "(forward / dgrad, E <= M/8192, K >= 4096 or N >= 4096), A (N >= 8192), or both wgrad "
                           "operands (unless "
                           "N + K < 10240 and E*(N+K) <= 8192) into row pairs, which the GEMM reads in whole "
                           "128-byte lines; same bits as without (mxgg_*_staging_size)",
        "kernel_only_geomean_tflops": kernel_geomeans(rows, "_kernel_us"),
        "native_geomean_tflops": kernel_geomeans(rows, "_native_us"),
        "native_layout": "kernel-only time on the layout the kernels read fastest: step-major scales and row-pair "
                         "e4m3 data (rows 2i, 2i+1 interleaved in 64-byte pieces), both written by the quantizers "
                         "outside the timed region; same bits as the row-major calls",
        "cfg5_mxfp4": extra["cfg5"] if extra else None,
        "quantizer": extra["quant"] if extra else None,
        "moe_layer": extra["moe_layer"] if extra else None,
        "ep_shard": extra["ep_shard"] if extra else None,
        "fwd_geomean_by_E": per_e,
        "baseline_note": "vs_baseline = fwd geomean / 1498.8 TFLOP/s (reference README table, MI355X)",
        "roofline": roofline,
        "roofline_native": roofline_native,
        "cpu_baseline": cpu,
        "rows": {"cols": ["E", "N", "K", "fwd_us", "dgrad_us", "wgrad_us", "fwd_native_us", "dgrad_native_us",
                          "wgrad_native_us"],
                 "what": "per sweep shape (M=16640): drop-in call medians, then kernel-only medians on the "
                         "native layout (row pairs, step-major scales), microseconds",
                 "data": [[r["E"], r["N"], r["K"]] + [round(r[c], 1) if c in r else None for c in
                          ("fwd_us", "dgrad_us", "wgrad_us", "fwd_native_us", "dgrad_native_us", "wgrad_native_us")]
                          for r in rows]},
        "wall_s": round(time.time() - t_start, 1),
    }
    outdir = os.path.join(ROOT, DETAIL_DIR)
    if os.path.isdir(outdir):
        with open(os.path.join(outdir, "bench_detail.json"), "w") as f:
            json.dump({"summary": line, "rows": rows}, f, indent=1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
