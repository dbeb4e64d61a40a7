"""bench.py and bench_ops.py command-line contract, checked without a GPU:
more than one GPU is refused with a message and a non-zero status before any
device work, and the argument parsers accept every documented option."""
import os
import subprocess
import sys

from _util import REPO


def _run(*args):
    return subprocess.run([sys.executable, *args], cwd=REPO, capture_output=True, text=True, timeout=120)


def test_bench_refuses_several_gpus():
    r = _run("bench.py", "--gpus", "4")
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
    assert not r.stdout.lstrip().startswith("{")  # no JSON line


def test_bench_help_lists_options():
    r = _run("bench.py", "--help")
    assert r.returncode == 0
    for opt in ("--gpus", "--steps", "--warmup", "--settle-ms", "--config", "--splits", "--page-size",
                "--page-order", "--seed", "--no-cpu", "--cpu-budget", "--configs", "--config-steps",
                "--config-cpu-budget", "--placement", "--placement-steps"):
        assert opt in r.stdout, opt


def test_bench_ops_help_lists_options():
    r = _run("bench_ops.py", "--help")
    assert r.returncode == 0
    for opt in ("--op", "--M", "--N", "--d", "--B", "--Hkv", "--L", "--dtype", "--steps", "--warmup"):
        assert opt in r.stdout, opt


def test_traffic_summary_covers_the_decode_configs():
    """profiles/traffic.json (rocprofv3 FETCH_SIZE/WRITE_SIZE, calibrated):
    every BASELINE config's decode launch moves at most 3% more HBM bytes
    than its algorithmic KV bytes -- 5% at cfg2, whose flattened plan writes
    and reads back a partial record per (wave, sequence) segment."""
    import json
    with open(os.path.join(REPO, "profiles", "traffic.json")) as f:
        tr = json.load(f)
    for cfg in ("cfg1", "cfg2", "cfg3", "cfg4"):
        e = tr["configs"][cfg]
        assert e["hbm_bytes_per_launch"] == e["read_bytes_per_launch"] + e["write_bytes_per_launch"]
        bound = 1.05 if cfg == "cfg2" else 1.03
        assert 1.0 <= e["hbm_bytes_per_launch"] / e["algorithmic_bytes_per_launch"] < bound, cfg
        assert os.path.exists(os.path.join(REPO, e["source"]))


def test_bench_helpers_without_gpu():
    """The parity check and provenance helpers of bench.py on host data."""
    import importlib.util
    import numpy as np
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(REPO, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    ref = np.array([[1.0, -2.0, 0.0]], np.float32)
    ok = bench.check_step(ref + np.float32(5e-5), ref)
    assert ok["within_tolerance"] and 0.2 < ok["max_tol_frac"] < 0.6
    bad = bench.check_step(ref + np.float32(1e-2), ref)
    assert not bad["within_tolerance"] and bad["max_tol_frac"] > 1.0
    nan = bench.check_step(np.full_like(ref, np.nan), ref)
    assert nan["within_tolerance"] is False and nan["max_abs_err"] is None
    hi = bench.host_info()
    assert hi["nproc"] >= 1 and hi["os_cpu_count"] >= 1
