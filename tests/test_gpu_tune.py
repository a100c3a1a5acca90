"""The sweep worker on the GPU: a few configurations of a small problem, in
this process (the driver runs one worker process per shape; that part is
covered on the CPU)."""

import math

import pytest

pytestmark = pytest.mark.gpu


def test_worker_times_every_configuration(gpu, tmp_path):
    import json

    import tune_worker as W
    out = str(tmp_path / "2_1024_512_512.json")
    print("tune_worker.sweep E=2 M=1024 N=512 K=512 limit=6", flush=True)
    res = W.sweep(2, 1024, 512, 512, "e4m3", limit=6, rep_ms=5.0, out_path=out, draws=2)
    assert res["n_total"] == 6 and len(res["results"]) == 6 and len(res["offs"]) == 2
    for r in res["results"]:
        assert r["err"] is None, r
        assert len(r["us_draws"]) == 2 and all(t > 0 for t in r["us_draws"])
        # geometric mean of the draws (exp of a mean of logs: equal draws may
        # come back an ulp off)
        lo, hi = min(r["us_draws"]), max(r["us_draws"])
        assert math.isfinite(r["us"]) and lo * (1 - 1e-9) <= r["us"] <= hi * (1 + 1e-9)
    with open(out) as f:
        assert json.load(f)["n_done"] == 6
