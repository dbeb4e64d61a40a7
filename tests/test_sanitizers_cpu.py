"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

- libkvq's host side (C-ABI validation, planners, workspace sizing) is built
  with both sanitizers into tests/sanitize/kvq_host_check, which sweeps the
  public C ABI with device-pointer stand-ins and never launches a kernel; it
  runs once per planner switch (KVQ_FORCE_KERNEL, KVQ_FLAT_PLAN,
  KVQ_SCHEDULE_LAUNCH, KVQ_DEBUG_SYNC).
- The CPU oracle and every planted-mistake variant are built with both
  sanitizers (oracle/Makefile `sanitize`) and tests/test_oracle.py runs against
  them in a child Python with the gcc ASan runtime preloaded.
- Two variants that only the sanitizer builds contain (a read one past the
  score scratch, a signed overflow) show that a report fails the run.

Any report ends the child with a non-zero status (halt_on_error, no UBSan
recovery), and the tests also reject report text in its output.
(The reference's sanitizer leg: benchmarks/selective_scan/run.py:147-164.)
"""
import os
import subprocess
import sys

import pytest

from _util import REPO

SAN_DIR = os.path.join(REPO, "tests", "sanitize")
HOST_CHECK = os.path.join(SAN_DIR, "_build", "kvq_host_check")
REPORTS = ("ERROR: AddressSanitizer", "ERROR: LeakSanitizer", "runtime error:", "UndefinedBehaviorSanitizer")


def _san_env(**extra):
    env = dict(os.environ)
    for k in ("KVQ_FORCE_KERNEL", "KVQ_FLAT_PLAN", "KVQ_SCHEDULE_LAUNCH", "KVQ_DEBUG_SYNC", "LD_PRELOAD"):
        env.pop(k, None)
    env["ASAN_OPTIONS"] = "halt_on_error=1:detect_leaks=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env.update(extra)
    return env


def _gcc_asan_runtime():
    path = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    return path


def _python_env(**extra):
    """A child Python (not itself instrumented) that loads the sanitized oracle."""
    return _san_env(LD_PRELOAD=_gcc_asan_runtime(), ASAN_OPTIONS="halt_on_error=1:detect_leaks=0",
                    KVQ_ORACLE_SANITIZED="1", PYTHONPATH=REPO, **extra)


@pytest.fixture(scope="module")
def host_check():
    subprocess.run(["make", "-s", "-j8", "-C", SAN_DIR], check=True, capture_output=True, timeout=900)
    return HOST_CHECK


@pytest.mark.parametrize("switch", [{}, {"KVQ_FORCE_KERNEL": "valu"}, {"KVQ_FORCE_KERNEL": "generic"},
                                    {"KVQ_FLAT_PLAN": "0"}, {"KVQ_SCHEDULE_LAUNCH": "1"}, {"KVQ_DEBUG_SYNC": "1"}],
                         ids=lambda s: ",".join(f"{k}={v}" for k, v in s.items()) or "default")
def test_host_planner_and_validation_clean(host_check, switch):
    r = subprocess.run([host_check], env=_san_env(**switch), capture_output=True, text=True, timeout=300)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert not any(s in out for s in REPORTS), out[-4000:]
    last = r.stdout.strip().splitlines()[-1]
    assert last.startswith("OK ") and int(last.split()[1]) > 1_000_000, last


def test_oracle_pins_clean_under_sanitizers():
    """tests/test_oracle.py (every pin on the real oracle, every planted
    mistake caught) with the sanitized oracle builds loaded."""
    subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle"), "sanitize"], check=True, capture_output=True,
                   timeout=300)
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(REPO, "tests", "test_oracle.py")],
                       cwd=REPO, env=_python_env(), capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert not any(s in out for s in REPORTS), out[-4000:]
    assert " passed" in r.stdout and " failed" not in r.stdout


_PROBE = """
import sys
import numpy as np
from oracle import oracle as orc
o = orc.Oracle(orc.plant_path(int(sys.argv[1])))
assert orc.SANITIZED and "_asan" in orc.plant_path(1)
rng = np.random.default_rng(0)
H, N, d = 2, 40, 64
Q = rng.standard_normal((H, d), dtype=np.float32)
K = rng.integers(-127, 128, (H, N, d), dtype=np.int8)
V = rng.integers(-127, 128, (H, N, d), dtype=np.int8)
s = np.full((H, N), 0.01, np.float32)
print("sum", float(o.head_f32(Q, K, V, s, s).sum()))
"""


@pytest.mark.parametrize("plant,report", [(12, "heap-buffer-overflow"), (13, "signed integer overflow"),
                                          (0, None)])
def test_sanitizer_report_fails_the_run(plant, report):
    subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle"), "sanitize"], check=True, capture_output=True,
                   timeout=300)
    args = [sys.executable, "-c", _PROBE, str(plant)]
    if plant == 0:  # the real oracle through the same probe: clean
        args = [sys.executable, "-c", _PROBE.replace("orc.plant_path(int(sys.argv[1]))", "orc.LIB_PATH"), "0"]
    r = subprocess.run(args, cwd=REPO, env=_python_env(), capture_output=True, text=True, timeout=120)
    out = r.stdout + r.stderr
    if report is None:
        assert r.returncode == 0 and "sum" in r.stdout, out[-3000:]
        assert not any(s in out for s in REPORTS), out[-3000:]
    else:
        assert r.returncode != 0, out[-3000:]
        assert report in out, out[-3000:]
