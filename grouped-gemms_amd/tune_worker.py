"""Per-shape configuration sweep of the forward grouped GEMM (one shape per process).

Counterpart of the reference's tune_worker.py (tune_worker.py:21-109): one
(E, M, N, K) problem, every launch configuration libmxgg has built, each timed
as the median device time of a ``mxgg_grouped_mm`` call (scale re-layout
with the operand staging the drop-in call makes, GEMM, and the piece /
reduce launches of a split last round) with the caches
flushed before every repetition.  The search space is the set of built
instantiations rather than Triton meta-parameters:

  tile (BLOCK_M x BLOCK_N)   256 x 256, 128 x 128 (e4m3 weights; e2m1: 256 only)
  GROUP_M                    1, 4, 8, 12, 16 (m-blocks per band of a group)
  XCD_SWIZZLE                1, 8
  split                      1: full workspace (the library may split the
                             last round along K), 0: scales-only workspace

Group sizes change from batch to batch in an MoE layer, and a configuration
tuned on one draw of jagged offsets can lose several percent on the next, so
each configuration is timed on ``--draws`` seeded offset draws (one for E = 1)
and ranked by the geometric mean (the reference tunes on a single draw).

Invoked as ``python tune_worker.py E M N K out.json [--fmt e4m3|e2m1]
[--limit n] [--rep-ms t] [--draws d]`` with one GPU visible.  Writes
``{"shape": [E, M, N, K], "fmt": ..., "offs": [...], "results": [{"cfg":
{...}, "us": geomean | null, "us_draws": [...], "err": str | null}, ...]}``
(rewritten every 8 configurations, so a crash leaves partial results) and
prints "OK" at the end.
"""

from __future__ import annotations

import argparse
import json
import os
import random
import sys
import time
import traceback

_HERE = os.path.dirname(os.path.abspath(__file__))
if _HERE not in sys.path:
    sys.path.insert(0, _HERE)

TILES = {"e4m3": ((256, 256), (128, 128)), "e2m1": ((256, 256),)}
GROUP_MS = (1, 4, 8, 12, 16)
XCDS = (1, 8)
SPLITS = (1, 0)


def build_search_space(fmt: str = "e4m3") -> list:
    """Every built configuration, library default first (so a truncated sweep
    still has the baseline)."""
    cfgs = [{"BLOCK_M": bm, "BLOCK_N": bn, "GROUP_M": gm, "XCD_SWIZZLE": x, "SPLIT": sp}
            for (bm, bn) in TILES[fmt] for gm in GROUP_MS for x in XCDS for sp in SPLITS]
    default = {"BLOCK_M": 256, "BLOCK_N": 256, "GROUP_M": 12, "XCD_SWIZZLE": 8, "SPLIT": 1}
    cfgs.remove(default)
    return [default] + cfgs


def make_inputs(E: int, M: int, N: int, K: int, fmt: str, device, draws: int = 1):
    """Seeded problem like the reference worker's (tune_worker.py:66-76):
    A ~ N(0, 1), W ~ N(0, 1) * 0.02, quantized along K; ``draws`` jagged
    offset tensors from ``generate_jagged_offs`` after ``random.seed(123)``."""
    import torch

    import kernels
    from utils import generate_jagged_offs

    torch.manual_seed(123)
    random.seed(123)
    a = torch.randn((M, K), device=device).to(torch.bfloat16)
    w = (torch.randn((E, N, K), device=device) * 0.02).to(torch.bfloat16)
    offs = [generate_jagged_offs(E, M, multiple_of=32, device=device) for _ in range(draws if E > 1 else 1)]
    sa, qa = kernels.to_mx(a)
    if fmt == "e2m1":
        sw, qw = kernels.to_mx(w, elem_dtype=torch.float4_e2m1fn_x2)
    else:
        sw, qw = kernels.to_mx(w)
    del a, w
    return qa, sa, qw, sw, offs


def sweep(E: int, M: int, N: int, K: int, fmt: str = "e4m3", limit: int | None = None,
          rep_ms: float = 60.0, out_path: str | None = None, log=None, draws: int = 3) -> dict:
    """Time every configuration of one shape; returns the result dict (and
    keeps ``out_path`` up to date when given)."""
    import math

    import torch

    from kernels import _lib
    from utils import benchmark_cuda_function_in_microseconds

    dev = torch.device("cuda")
    lib = _lib.load()
    qa, sa, qw, sw, offs_list = make_inputs(E, M, N, K, fmt, dev, draws)
    u8 = lambda t: t.view(torch.uint8)
    a, a_s, b, b_s = u8(qa), u8(sa), u8(qw), u8(sw)
    b_fmt = _lib.FMT_E2M1 if fmt == "e2m1" else _lib.FMT_E4M3
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    full = lib.mxgg_grouped_mm_workspace_size(E, M, N, K)
    scales_only = 4 * ((K + 127) // 128) * (M + E * N)
    # plus the operand staging the drop-in call makes (it keeps the split room)
    stage = lib.mxgg_grouped_mm_staging_size(E, M, N, K, b_fmt)
    ws = torch.empty(max(full + stage, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream

    def call(cfg, ws_bytes, offs):
        _lib.check(lib.mxgg_grouped_mm(
            a.data_ptr(), a.stride(0), a_s.data_ptr(), a_s.stride(0),
            b.data_ptr(), b_fmt, b.stride(1), b.stride(0),
            b_s.data_ptr(), b_s.stride(1), b_s.stride(0),
            offs.data_ptr(), E, M, N, K, out.data_ptr(), _lib.DTYPE_BF16, out.stride(0),
            cfg["BLOCK_M"], cfg["BLOCK_N"], cfg["GROUP_M"], cfg["XCD_SWIZZLE"],
            ws.data_ptr(), ws_bytes, stream))

    cfgs = build_search_space(fmt)
    if limit is not None:
        cfgs = cfgs[:limit]
    res = {"shape": [E, M, N, K], "fmt": fmt, "results": [], "n_total": len(cfgs),
           "offs": [o.tolist() for o in offs_list], "device": torch.cuda.get_device_properties(dev).name}
    t0 = time.time()

    def flush_json():
        if out_path:
            res["elapsed_s"] = time.time() - t0
            res["n_done"] = len(res["results"])
            tmp = out_path + ".tmp"
            with open(tmp, "w") as f:
                json.dump(res, f)
            os.replace(tmp, out_path)

    for i, cfg in enumerate(cfgs):
        ws_bytes = (full if cfg["SPLIT"] else (scales_only + 255) // 256 * 256) + stage
        try:
            ts = [float(benchmark_cuda_function_in_microseconds(call, cfg, ws_bytes, o, warmup_ms=10.0,
                                                                rep_ms=rep_ms)) for o in offs_list]
            us = math.exp(sum(map(math.log, ts)) / len(ts))
            res["results"].append({"cfg": cfg, "us": us, "us_draws": ts, "err": None})
        except Exception as ex:   # an unsupported combination is a result, not a crash
            res["results"].append({"cfg": cfg, "us": None, "us_draws": [], "err": f"{type(ex).__name__}: {ex}"})
        if log:
            r = res["results"][-1]
            log(f"  {cfg} -> {r['us'] if r['us'] is not None else r['err']}")
        if (i + 1) % 8 == 0 or i + 1 == len(cfgs):
            flush_json()
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("E", type=int)
    ap.add_argument("M", type=int)
    ap.add_argument("N", type=int)
    ap.add_argument("K", type=int)
    ap.add_argument("out_path")
    ap.add_argument("--fmt", choices=("e4m3", "e2m1"), default="e4m3")
    ap.add_argument("--limit", type=int, default=None, help="first n configurations only (smoke test)")
    ap.add_argument("--rep-ms", type=float, default=60.0, help="timed repetitions per configuration, in ms")
    ap.add_argument("--draws", type=int, default=3, help="jagged offset draws per configuration (E > 1)")
    args = ap.parse_args()
    sweep(args.E, args.M, args.N, args.K, args.fmt, args.limit, args.rep_ms, args.out_path, draws=args.draws)
    print("OK", flush=True)
    return 0


if __name__ == "__main__":
    try:
        sys.exit(main())
    except Exception:
        traceback.print_exc()
        sys.exit(1)
