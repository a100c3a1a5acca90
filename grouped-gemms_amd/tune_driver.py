"""Forward grouped-GEMM configuration sweep over a shape list, one GPU.

Counterpart of the reference's tune_driver.py (tune_driver.py:1-135): every
shape runs in its own ``tune_worker.py`` process (a failing shape cannot take
the sweep down with it), here one after another on the one visible GPU.
Per-shape results land in ``<out-dir>/<E>_<M>_<N>_<K>[_e2m1].json``; the best
configuration of each shape goes to ``<out-dir>/best.json``.
``--emit-header`` turns best.json into ``csrc/tuned_fwd.h``, the table libmxgg's
launch-configuration pick consults (rebuild the library afterwards).  Only
robust wins go into the table: the best configuration must beat the built-in
default (the worker's first configuration) on every offset draw by at least
``--min-gain``; elsewhere the library keeps its own rule.

    python grouped-gemms_amd/tune_driver.py --out-dir /tmp/mxgg_tune
    python grouped-gemms_amd/tune_driver.py --out-dir /tmp/mxgg_tune --emit-header \\
        grouped-gemms_amd/csrc/tuned_fwd.h

Default shapes: the reference's 36-shape Llama4 sweep (E in 1, 2, 4, 8;
M = 16640; N, K in 2048, 5120, 8192).
"""

from __future__ import annotations

import argparse
import itertools
import json
import os
import subprocess
import sys
import time

_HERE = os.path.dirname(os.path.abspath(__file__))

SHAPES = [(e, 16640, n, k) for e, n, k in itertools.product((1, 2, 4, 8), (2048, 5120, 8192), (2048, 5120, 8192))]

FMT_CODE = {"e4m3": 0, "e2m1": 4}


def result_path(out_dir: str, shape, fmt: str) -> str:
    E, M, N, K = shape
    return os.path.join(out_dir, f"{E}_{M}_{N}_{K}" + ("" if fmt == "e4m3" else f"_{fmt}") + ".json")


def run_one(shape, fmt: str, out_dir: str, timeout_s: float, extra=()) -> dict:
    """One worker process for one shape; returns its exit status and output tails."""
    E, M, N, K = shape
    out_path = os.path.abspath(result_path(out_dir, shape, fmt))
    cmd = [sys.executable, os.path.join(_HERE, "tune_worker.py"), str(E), str(M), str(N), str(K), out_path,
           "--fmt", fmt, *extra]
    env = os.environ.copy()
    env["PYTHONPATH"] = _HERE + (os.pathsep + env["PYTHONPATH"] if env.get("PYTHONPATH") else "")
    t0 = time.time()
    try:
        r = subprocess.run(cmd, cwd=_HERE, env=env, capture_output=True, text=True, timeout=timeout_s)
        rc, so, se = r.returncode, r.stdout, r.stderr
    except subprocess.TimeoutExpired as ex:
        rc, so, se = -9, ex.stdout or "", f"timed out after {timeout_s:.0f} s"
        so = so.decode() if isinstance(so, bytes) else so
    return {"shape": list(shape), "fmt": fmt, "rc": rc, "elapsed_s": time.time() - t0,
            "stdout_tail": so[-500:], "stderr_tail": se[-1000:], "out_path": out_path}


def best_of(data: dict):
    """Fastest successful configuration of one worker result, or None; with
    ``min_draw_gain``, the smallest per-draw speedup over the worker's first
    (built-in default) configuration."""
    ok = [r for r in data.get("results", []) if r.get("us") is not None]
    if not ok:
        return None
    b = min(ok, key=lambda r: r["us"])
    out = {"cfg": b["cfg"], "us": b["us"], "n_ok": len(ok), "n_total": len(data["results"])}
    first = data["results"][0]
    if first.get("us") is not None:
        out["default_cfg"], out["default_us"] = first["cfg"], first["us"]
        fd, bd = first.get("us_draws") or [first["us"]], b.get("us_draws") or [b["us"]]
        if len(fd) == len(bd):
            out["min_draw_gain"] = min(x / y for x, y in zip(fd, bd)) - 1.0
    return out


def aggregate(shapes, fmt: str, out_dir: str, log=print) -> dict:
    """best.json content for the shapes whose result files exist."""
    best = {}
    for shape in shapes:
        path = result_path(out_dir, shape, fmt)
        if not os.path.exists(path):
            log(f"MISSING: {path}")
            continue
        with open(path) as f:
            data = json.load(f)
        b = best_of(data)
        if b is None:
            log(f"NO_OK_CFG: {shape}")
            continue
        E, M, N, K = shape
        key = f"{E}_{M}_{N}_{K}" + ("" if fmt == "e4m3" else f"_{fmt}")
        b["fmt"] = fmt
        b["device"] = data.get("device", "")
        best[key] = b
        tflops = 2.0 * M * N * K / (b["us"] * 1e-6) / 1e12
        log(f"  {key}: {b['us']:.1f} us ({tflops:.1f} TFLOP/s) cfg={b['cfg']} ({b['n_ok']}/{b['n_total']} ok)")
    return best


def emit_header(best: dict, source: str = "", min_gain: float | None = None) -> str:
    """C++ text of tuned_fwd.h for the entries of a best.json (with
    ``min_gain``: only those whose smallest per-draw speedup over the default
    reaches it)."""
    rows = []
    for key, b in best.items():
        if min_gain is not None and b.get("min_draw_gain", -1.0) < min_gain:
            continue
        parts = key.split("_")
        E, M, N, K = (int(x) for x in parts[:4])
        fmt = b.get("fmt", parts[4] if len(parts) > 4 else "e4m3")
        c = b["cfg"]
        rows.append((E, M, N, K, FMT_CODE[fmt], c["BLOCK_M"], c["BLOCK_N"], c["GROUP_M"], c["XCD_SWIZZLE"],
                     1 if c.get("SPLIT", 1) else 0, b["us"]))
    rows.sort()
    lines = [
        "// Tuned forward launch configurations, one per swept shape, consulted by",
        "// pick_fwd (grouped_gemm.hip) before its built-in rule.  Written by",
        "// `python grouped-gemms_amd/tune_driver.py --emit-header` from the sweep's",
        "// best.json; regenerate rather than edit.  An entry applies to calls with",
        "// the same E, N, K and weight format and M within a factor of two of the",
        "// swept M, on every operand layout (the sweep timed the drop-in call's,",
        "// operands staged by the library's rule at the swept shape; the whole entry",
        "// applies elsewhere too, since the tile order can change the bits of a call",
        "// whose last round is split).  Fields: E, M, N, K, b_fmt (0 e4m3, 4 e2m1),",
        "// block_m, block_n,",
        "// group_m, xcd swizzle, split (1: the last round may be split along K when",
        "// the workspace allows it, 0: whole tiles only).",
        f"// sweep: {source or 'none'}",
        "static const TunedFwd kTunedFwd[] = {",
    ]
    for r in rows:
        lines.append("    {%d, %d, %d, %d, %d, %d, %d, %d, %d, %d},   // %.1f us" % r)
    lines.append("    {0, 0, 0, 0, 0, 0, 0, 0, 0, 0},   // end")
    lines.append("};")
    return "\n".join(lines) + "\n"


def parse_shapes(text: str):
    """'E,M,N,K;E,M,N,K' -> list of tuples."""
    out = []
    for item in text.replace(" ", "").split(";"):
        if item:
            v = tuple(int(x) for x in item.split(","))
            if len(v) != 4:
                raise ValueError(f"shape {item!r} is not E,M,N,K")
            out.append(v)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--out-dir", default=os.environ.get("TUNE_OUT_DIR", "/tmp/mxgg_tune"))
    ap.add_argument("--shapes", default=None, help="'E,M,N,K;...' (default: the 36-shape sweep)")
    ap.add_argument("--fmt", choices=tuple(FMT_CODE), default="e4m3")
    ap.add_argument("--limit", type=int, default=None, help="configurations per shape (smoke test)")
    ap.add_argument("--rep-ms", type=float, default=60.0)
    ap.add_argument("--draws", type=int, default=5, help="jagged offset draws per configuration (E > 1)")
    ap.add_argument("--timeout", type=float, default=600.0, help="seconds per shape")
    ap.add_argument("--aggregate-only", action="store_true", help="skip the sweep, rebuild best.json")
    ap.add_argument("--emit-header", default=None, metavar="PATH", help="write tuned_fwd.h from best.json")
    ap.add_argument("--min-gain", type=float, default=0.02,
                    help="table entries need this speedup over the default on every draw")
    args = ap.parse_args()

    shapes = parse_shapes(args.shapes) if args.shapes else SHAPES
    args.out_dir = os.path.abspath(args.out_dir)   # workers run from this file's directory
    os.makedirs(args.out_dir, exist_ok=True)
    failed = 0
    if not args.aggregate_only:
        extra = ["--rep-ms", str(args.rep_ms), "--draws", str(args.draws)] + \
            (["--limit", str(args.limit)] if args.limit else [])
        t_start = time.time()
        print(f"sweeping {len(shapes)} shapes ({args.fmt}) into {args.out_dir}", flush=True)
        for shape in shapes:
            r = run_one(shape, args.fmt, args.out_dir, args.timeout, extra)
            ok = r["rc"] == 0
            failed += 0 if ok else 1
            print(f"[{'OK' if ok else 'FAIL(rc=%d)' % r['rc']}] shape={tuple(shape)} t={r['elapsed_s']:.1f}s",
                  flush=True)
            if not ok:
                print(f"  stderr: {r['stderr_tail']}", flush=True)
                if r["rc"] in (-6, -9, -11, 134, 137, 139):
                    print("  worker crashed: stopping the sweep", flush=True)
                    break
        print(f"total wall time {time.time() - t_start:.1f} s", flush=True)
    best = aggregate(shapes, args.fmt, args.out_dir)
    best_path = os.path.join(args.out_dir, "best.json")
    with open(best_path, "w") as f:
        json.dump(best, f, indent=2)
    print(f"wrote {best_path} with {len(best)} entries", flush=True)
    if args.emit_header:
        dev = next((b.get("device") for b in best.values() if b.get("device")), "")
        kept = sum(1 for b in best.values() if b.get("min_draw_gain", -1.0) >= args.min_gain)
        src = (f"{len(best)} shapes ({args.fmt}, {args.draws} offset draws), {kept} with a gain of at least "
               f"{100 * args.min_gain:g}% on every draw; {dev}")
        with open(args.emit_header, "w") as f:
            f.write(emit_header(best, src, args.min_gain))
        print(f"wrote {args.emit_header}", flush=True)
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
