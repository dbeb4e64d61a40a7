"""bench.py's line verifier (verify_line) on the CPU: the committed line of the
latest full bench run is consistent with itself and covers every BASELINE
configuration with its timed rounds, and planted inconsistencies are caught
(as the reference's verify_results.py:21-72 recomputes its summaries from
the raw rows)."""
import copy
import importlib.util
import json
import os
import statistics

import pytest

from _util import REPO

LINE = os.path.join(REPO, "profiles", "bench_line.json")
CONFIGS = ("cfg0", "cfg1", "cfg2", "cfg3", "cfg4")


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _line():
    with open(LINE) as f:
        return json.loads(f.read().strip().splitlines()[-1])


def _synthetic(bench):
    """A consistent line built from round times, as bench.py derives it."""
    kvb = 276824064
    us = [42.9, 42.6, 43.1]
    med = statistics.median(us)
    gbps = kvb / (med * 1e-6) / 1e9
    cfg = {"workload": "cfg1", "us_per_step": med, "GB/s": round(gbps, 2), "frac": round(gbps / 8000.0, 4),
           "kv_bytes_per_step": kvb, "max_tol_frac": 0.002, "within_tolerance": True,
           "rounds": {"n": 3, "us_per_step": us, "median": med, "min": min(us), "max": max(us)}}
    return {"value": round(gbps, 2), "ms_per_step": med * 1e-3, "us_per_step": med,
            "pct_hbm_peak": round(100 * gbps / 8000.0, 2), "config": {"kv_bytes_per_step": kvb},
            "rounds": dict(cfg["rounds"]),
            "roofline": {"achieved": round(gbps, 2), "peak": 8000.0, "frac": round(gbps / 8000.0, 4),
                         "bytes_per_launch": kvb},
            "configs": {"cfg1": cfg}}


def test_synthetic_line_is_consistent():
    bench = _bench()
    assert bench.verify_line(_synthetic(bench)) == []


@pytest.mark.parametrize("plant", ["value", "frac", "median", "cfg_gbps", "bytes", "tolerance", "rounds_n"])
def test_planted_inconsistency_is_caught(plant):
    bench = _bench()
    line = _synthetic(bench)
    if plant == "value":
        line["value"] *= 1.05
    elif plant == "frac":
        line["roofline"]["frac"] += 0.02
    elif plant == "median":
        line["rounds"]["median"] = line["rounds"]["max"]
    elif plant == "cfg_gbps":
        line["configs"]["cfg1"]["GB/s"] *= 0.9
    elif plant == "bytes":
        line["roofline"]["bytes_per_launch"] += 1
    elif plant == "tolerance":
        line["configs"]["cfg1"]["max_tol_frac"] = 1.5
    else:
        line["rounds"]["n"] = 5
    assert bench.verify_line(line), plant


@pytest.mark.skipif(not os.path.exists(LINE), reason="no committed bench line")
def test_committed_line():
    """The latest full bench line (profiles/bench_line.json) re-derives from
    its own fields, covers cfg0..cfg4 with 3 timed rounds each, is within the
    parity tolerance everywhere, and its headline is cfg1, BASELINE.json's
    metric configuration."""
    bench = _bench()
    line = _line()
    assert bench.verify_line(line) == [], bench.verify_line(line)
    assert line["config"]["workload"].startswith("cfg1:") and line["metric"] == bench.METRIC
    assert set(CONFIGS) <= set(line["configs"])
    for name in CONFIGS:
        c = line["configs"][name]
        assert c["rounds"]["n"] >= 3, name
        assert c["within_tolerance"], name
        assert c["vs_f64"]["gpu_max_tol_frac"] <= 1.0, name
    assert line["roofline"]["frac"] == line["configs"]["cfg1"]["frac"]
    # A tampered copy no longer verifies.
    bad = copy.deepcopy(line)
    bad["configs"]["cfg2"]["us_per_step"] *= 0.8
    assert bench.verify_line(bad)
