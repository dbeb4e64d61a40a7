"""The quantiser's divide-free scale (csrc/kvq_device.hpp quant_scale) equals
the oracle's IEEE quotient amax / 127.0f (oracle/kvq_oracle.c quantize_row)
for every amax the device computes it for; tests/quant_scale_check.c holds the
exhaustive check and the argument for its coverage."""
import os
import re
import subprocess

import pytest

from _util import REPO

SRC = os.path.join(REPO, "tests", "quant_scale_check.c")
DEV = os.path.join(REPO, "cuda-operators_amd", "csrc", "kvq_device.hpp")


def _build(tmp_path, *defs):
    exe = str(tmp_path / "quant_scale_check")
    cmd = ["gcc", "-O2", "-fopenmp", "-ffp-contract=off", *defs, SRC, "-o", exe, "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, timeout=120)
    return exe


def test_device_constants_match_checker():
    dev = open(DEV).read()
    chk = open(SRC).read()
    for name in ("kCh", "kCl"):
        d = re.search(name + r"\s*=\s*(0x[0-9a-fp.+-]+)f", dev).group(1)
        c = re.findall(name + r"\s*=\s*(0x[0-9a-fp.+-]+)f", chk)
        assert d in c, (name, d, c)
    assert "amax < 0x1p-112f" in dev  # the divide below the checked range


def test_scale_matches_ieee_quotient(tmp_path):
    r = subprocess.run([_build(tmp_path)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    m = re.search(r"checked (\d+) mismatches (\d+) below-2\^-112 mismatches (\d+)", r.stdout)
    assert m and int(m.group(1)) > 190_000_000 and int(m.group(2)) == 0 and int(m.group(3)) > 0, r.stdout


def test_planted_low_part_drop_is_caught(tmp_path):
    r = subprocess.run([_build(tmp_path, "-DPLANT_NO_LOW_PART")], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert int(re.search(r"mismatches (\d+)", r.stdout).group(1)) > 0, r.stdout
