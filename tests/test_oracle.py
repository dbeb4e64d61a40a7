"""The CPU oracle against what pins it (CPU only).

The oracle restates cpu_reference (kv_cache/KV_int8_split_optimized.cu:385-437)
and the per-token quantiser spec.  Every pin in _pins.py must hold for the real
oracle, and every planted-mistake build of the oracle must fail at least one
pin -- otherwise the pins could not tell that mistake from the real thing.
"""
import os

import numpy as np
import pytest

from _util import close_report
import _pins
from oracle import oracle as orc


@pytest.fixture(scope="module")
def real():
    orc.build()
    return orc.get()


@pytest.mark.parametrize("pin", _pins.ALL_PINS, ids=lambda p: p.__name__)
def test_real_oracle_passes_pin(real, pin):
    fails = pin(real)
    assert not fails, "\n".join(fails)


PLANTS = {
    1: "score drops k_scale",
    2: "1/d instead of 1/sqrt(d)",
    3: "kv head = hq % Hkv",
    4: "expf(max - s)",
    5: "K transposed",
    6: "ragged length off by one",
    7: "round half away from zero",
    8: "truncation",
    9: "value dequant drops v_scale",
    10: "dense attention: 1/d instead of 1/sqrt(d)",
    11: "dense attention: V transposed",
}


@pytest.fixture(scope="module")
def plants_built():
    orc.build(plants=True)


@pytest.mark.parametrize("plant", sorted(PLANTS), ids=lambda p: PLANTS[p])
def test_planted_mistake_is_caught(plants_built, plant):
    o = orc.Oracle(orc.plant_path(plant))
    assert o.plant == plant
    fails = _pins.run_all(o)
    assert fails, f"planted mistake {plant} ({PLANTS[plant]}) passed every pin"


def test_checker_self_test():
    """The parity gate rejects NaN/Inf and out-of-tolerance values
    (form of benchmarks/selective_scan/bench.cpp:43-53)."""
    ref = np.array([1.0, -2.0, 0.0], np.float32)
    assert close_report(ref, ref)[0]
    assert close_report(ref + np.float32(9e-5), ref)[0]
    assert not close_report(np.array([1.0, -2.0, 2e-4], np.float32), ref)[0]
    assert not close_report(np.array([np.nan, -2.0, 0.0], np.float32), ref)[0]
    assert not close_report(np.array([np.inf, -2.0, 0.0], np.float32), ref)[0]
    assert not close_report(ref[:2], ref)[0]


def test_openmp_threads_do_not_change_results(real):
    """OpenMP over (b, hq) keeps every unit's sequential order: results are
    independent of the thread count (checked via a 1-unit vs many-unit split)."""
    rng = np.random.default_rng(3)
    from _util import make_problem
    p = make_problem(rng, 2, 4, 4, 100, 64, real.quantize_rows)
    full = real.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"])
    for b in range(2):
        one = real.decode_f32(p["q"][b:b + 1], p["k"][b:b + 1], p["v"][b:b + 1],
                              p["ks"][b:b + 1], p["vs"][b:b + 1])
        assert np.array_equal(one, full[b:b + 1])
