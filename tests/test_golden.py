"""Committed golden fixtures (tests/golden/) against the oracle and the float64
textbook (CPU only).  The fixtures are regression anchors for the oracle and
the expected values for the GPU KAT tests; the textbook check pins them."""
import os

import numpy as np
import pytest

from _util import SEEDS, close_report, selftest_inputs, textbook_decode_f64
from oracle import oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KAT_SHAPES = ((4, 128, 64), (8, 1024, 64), (3, 257, 128))


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


@pytest.fixture(scope="module")
def o():
    orc.build()
    return orc.get()


@pytest.mark.parametrize("shape", KAT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_selftest_kat(o, shape):
    H, N, d = shape
    tag = f"{H}x{N}x{d}"
    g = _load("kat_selftest.npz")
    Q, K, V, ks, vs = selftest_inputs(H, N, d)
    got = o.head_f32(Q, K, V, ks, vs)
    assert np.array_equal(got, g[f"out_f32_{tag}"]), "oracle drifted from its golden output"
    tb = textbook_decode_f64(Q[None], K[None], V[None], ks[None], vs[None])[0]
    assert close_report(g[f"out_f64_{tag}"], tb, 1e-12, 1e-10)[0]
    # the reference's own self-test gate: max-abs <= 1e-4 (KV_int8_split_optimized.cu:535)
    assert np.max(np.abs(g[f"out_f32_{tag}"] - tb)) <= 1e-4


@pytest.mark.parametrize("seed", SEEDS)
def test_random_small(o, seed):
    g = _load("random_small.npz")
    q, k, v, ks, vs = (g[f"{n}_{seed}"] for n in ("q", "k", "v", "ks", "vs"))
    got = o.decode_f32(q, k, v, ks, vs)
    assert np.array_equal(got, g[f"out_f32_{seed}"])
    ok, msg = close_report(got, textbook_decode_f64(q, k, v, ks, vs), 2e-5, 2e-4)
    assert ok, msg


def test_quant_fixture(o):
    g = _load("quant.npz")
    qv, sc = o.quantize_rows(g["x"])
    assert np.array_equal(qv, g["q"]) and np.array_equal(sc.view(np.uint32), g["scale"].view(np.uint32))
    # crafted rows: ties to even, negative amax at the last index, zero row, underflow
    assert list(g["q"][0][:8]) == [127, 0, 2, 2, 0, -2, -2, 126] and g["scale"][0] == 1.0
    assert list(g["q"][1][:4]) == [0, -1, 2, -127] and g["scale"][1] == 2.0
    assert g["scale"][2] == 0 and not g["q"][2].any()
    assert g["scale"][3] == 0 and not g["q"][3].any()
