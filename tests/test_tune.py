"""The configuration sweep (tune_driver.py / tune_worker.py, counterparts of the
reference's tune_driver.py:1-135 and tune_worker.py:21-109) and the tuned
table libmxgg consults.  CPU only: search space, best-of selection, the
emitted header, and that mxgg_grouped_mm_config returns every committed entry
for its shape (and falls back to the built-in rule elsewhere)."""

import ctypes
import json
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TABLE = os.path.join(ROOT, "grouped-gemms_amd", "csrc", "tuned_fwd.h")
ROW = re.compile(r"^\s*\{(-?\d+(?:,\s*-?\d+){9})\},")


def _table_rows(text):
    rows = [tuple(int(x) for x in m.group(1).split(",")) for m in map(ROW.match, text.splitlines()) if m]
    assert rows and rows[-1] == (0,) * 10, "table must end with the all-zero sentinel"
    return rows[:-1]


def test_search_space():
    import tune_worker as W
    s8 = W.build_search_space("e4m3")
    s4 = W.build_search_space("e2m1")
    assert len(s8) == 2 * 5 * 2 * 2 and len(s4) == 5 * 2 * 2
    for s in (s8, s4):
        assert len({json.dumps(c, sort_keys=True) for c in s}) == len(s)
        assert s[0] == {"BLOCK_M": 256, "BLOCK_N": 256, "GROUP_M": 12, "XCD_SWIZZLE": 8, "SPLIT": 1}
    assert {(c["BLOCK_M"], c["BLOCK_N"]) for c in s8} == {(256, 256), (128, 128)}
    assert {(c["BLOCK_M"], c["BLOCK_N"]) for c in s4} == {(256, 256)}


def _write(tmp_path, shape, results, fmt="e4m3"):
    import tune_driver as D
    with open(D.result_path(str(tmp_path), shape, fmt), "w") as f:
        json.dump({"shape": list(shape), "fmt": fmt, "device": "dev0", "results": results}, f)


def test_aggregate_picks_fastest_ok_and_reports_gaps(tmp_path):
    import tune_driver as D
    c = lambda bm, gm, sp: {"BLOCK_M": bm, "BLOCK_N": bm, "GROUP_M": gm, "XCD_SWIZZLE": 8, "SPLIT": sp}
    _write(tmp_path, (1, 16640, 2048, 2048), [
        {"cfg": c(256, 12, 1), "us": 120.0, "us_draws": [110.0, 130.9], "err": None},
        {"cfg": c(128, 8, 0), "us": 99.5, "us_draws": [100.0, 99.0], "err": None},
        {"cfg": c(128, 4, 1), "us": None, "us_draws": [], "err": "MXGGError: boom"},
        {"cfg": c(256, 4, 1), "us": 101.0, "us_draws": [101.0, 101.0], "err": None},
    ])
    _write(tmp_path, (2, 16640, 2048, 2048), [{"cfg": c(256, 12, 1), "us": None, "err": "x"}])
    logs = []
    best = D.aggregate([(1, 16640, 2048, 2048), (2, 16640, 2048, 2048), (4, 16640, 2048, 2048)], "e4m3",
                       str(tmp_path), log=logs.append)
    assert list(best) == ["1_16640_2048_2048"]
    b = best["1_16640_2048_2048"]
    assert b["cfg"] == c(128, 8, 0) and b["us"] == 99.5 and (b["n_ok"], b["n_total"]) == (3, 4)
    assert b["default_us"] == 120.0 and b["device"] == "dev0"
    assert b["min_draw_gain"] == pytest.approx(0.10)    # 110 / 100: the weaker draw counts
    assert any(s.startswith("NO_OK_CFG") for s in logs) and any(s.startswith("MISSING") for s in logs)


def test_emit_header_round_trip():
    import tune_driver as D
    best = {
        "8_16640_8192_2048": {"cfg": {"BLOCK_M": 256, "BLOCK_N": 256, "GROUP_M": 4, "XCD_SWIZZLE": 8,
                                      "SPLIT": 1}, "us": 350.0, "fmt": "e4m3"},
        "1_16640_2048_2048": {"cfg": {"BLOCK_M": 128, "BLOCK_N": 128, "GROUP_M": 16, "XCD_SWIZZLE": 1,
                                      "SPLIT": 0}, "us": 99.0, "fmt": "e4m3"},
        "8_16640_8192_5120_e2m1": {"cfg": {"BLOCK_M": 256, "BLOCK_N": 256, "GROUP_M": 8, "XCD_SWIZZLE": 8,
                                           "SPLIT": 0}, "us": 700.0, "fmt": "e2m1"},
    }
    rows = _table_rows(D.emit_header(best, "test"))
    assert rows == [(1, 16640, 2048, 2048, 0, 128, 128, 16, 1, 0),
                    (8, 16640, 8192, 2048, 0, 256, 256, 4, 8, 1),
                    (8, 16640, 8192, 5120, 4, 256, 256, 8, 8, 0)]
    # only entries that beat the default on every draw by min_gain are kept
    best["1_16640_2048_2048"]["min_draw_gain"] = 0.05
    best["8_16640_8192_2048"]["min_draw_gain"] = 0.01
    rows = _table_rows(D.emit_header(best, "test", min_gain=0.02))
    assert rows == [(1, 16640, 2048, 2048, 0, 128, 128, 16, 1, 0)]
    assert D.emit_header({}, "").count("{0, 0, 0, 0, 0, 0, 0, 0, 0, 0}") == 1


def test_parse_shapes():
    import tune_driver as D
    assert D.parse_shapes("1,16640,2048,2048; 8,1024,512,512;") == [(1, 16640, 2048, 2048), (8, 1024, 512, 512)]
    with pytest.raises(ValueError):
        D.parse_shapes("1,2,3")
    assert len(D.SHAPES) == 36 and len(set(D.SHAPES)) == 36


def _config(lib, E, M, N, K, fmt, req=(0, 0, 0, 0)):
    v = [ctypes.c_int(x) for x in req]
    rc = lib.mxgg_grouped_mm_config(E, M, N, K, fmt, *(ctypes.byref(x) for x in v))
    return rc, tuple(x.value for x in v)


def test_committed_table_is_used_by_the_library():
    from kernels import _lib
    lib = _lib.load()
    rows = _table_rows(open(TABLE).read())
    seen = set()
    for E, M, N, K, fmt, bm, bn, gm, xcd, split in rows:
        assert (E, N, K, fmt) not in seen, "duplicate shape in the tuned table"
        seen.add((E, N, K, fmt))
        assert (bm, bn) in ((256, 256), (128, 128)) and (fmt == 0 or bm == 256)
        assert gm >= 1 and xcd >= 1 and split in (0, 1)
        # the whole entry applies at M within a factor of two of the swept M,
        # whatever the operand layout or staging at that M (the tile order can
        # change the bits of a split call, and every layout gives the same bits)
        for m in (M, M // 2 + 1, 2 * M):
            assert _config(lib, E, m, N, K, fmt) == (0, (bm, bn, gm, xcd))
        # requests still override the table field by field
        assert _config(lib, E, M, N, K, fmt, (0, 0, 3, 1)) == (0, (bm, bn, 3, 1))


def test_untabled_shapes_use_the_built_in_rule():
    from kernels import _lib
    lib = _lib.load()
    rows = _table_rows(open(TABLE).read())
    tabled = {(E, N, K, f) for E, _, N, K, f, *_ in rows}
    # shapes no sweep covers: 256 x 256 tiles, GROUP_M 12, 8-XCD swizzle ...
    if (3, 3072, 8192, 0) not in tabled:
        assert _config(lib, 3, 16640, 3072, 8192, 0) == (0, (256, 256, 12, 8))
    # ... 128 x 128 for small, short e4m3 problems
    if (4, 512, 512, 0) not in tabled:
        assert _config(lib, 4, 1024, 512, 512, 0) == (0, (128, 128, 12, 8))
    # a tabled shape far outside its M range falls back too
    for E, M, N, K, fmt, *_ in rows:
        rc, got = _config(lib, E, 8 * M, N, K, fmt)
        assert rc == 0 and got[:2] == (256, 256)
