"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

Run from the repo root:  python tests/golden/make_golden.py
The fixtures are data only (inputs and expected outputs), loaded with
numpy.load(allow_pickle=False).  Nothing here comes from running reference code:
the reference ships no recorded outputs for this path, so the expected values
are the oracle's, and tests/test_golden.py re-checks them against the float64
textbook so the fixtures are pinned independently of the oracle.

  kat_selftest.npz  outputs for the reference self-test's patterned inputs
                    (kv_cache/KV_int8_split_optimized.cu:473-486) at the default
                    shape (4,128,64) (:441-443) and two argv-style shapes.
  random_small.npz  seeded N(0,1) problems, seeds 17/29/101, B1 H8 N128 d64.
  quant.npz         quantiser rows (crafted ties, extremes, random) + results.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from _util import SEEDS, make_problem, selftest_inputs  # noqa: E402
from oracle import oracle as orc  # noqa: E402

KAT_SHAPES = ((4, 128, 64), (8, 1024, 64), (3, 257, 128))


def quant_rows():
    rng = np.random.default_rng(41)
    rows = [
        np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5] + [0.0] * 8, np.float32),
        np.array([1.0, -2.0, 3.0, -254.0] + [0.25] * 12, np.float32),
        np.zeros(16, np.float32),
        np.array([1e-44, -2e-44, 0.0, 5e-45] + [0.0] * 12, np.float32),
    ]
    rows += list(rng.standard_normal((12, 16), dtype=np.float32))
    rows += list((rng.standard_normal((4, 16), dtype=np.float32) * np.float32(1e-38)))
    return np.stack(rows).astype(np.float32)


def main():
    orc.build()
    o = orc.get()
    kat = {}
    for (H, N, d) in KAT_SHAPES:
        Q, K, V, ks, vs = selftest_inputs(H, N, d)
        tag = f"{H}x{N}x{d}"
        kat[f"out_f32_{tag}"] = o.head_f32(Q, K, V, ks, vs)
        kat[f"out_f64_{tag}"] = o.decode_f64(Q[None], K[None], V[None], ks[None], vs[None])[0]
    np.savez_compressed(os.path.join(HERE, "kat_selftest.npz"), **kat)

    rnd = {}
    for seed in SEEDS:
        rng = np.random.default_rng(seed)
        p = make_problem(rng, 1, 8, 8, 128, 64, o.quantize_rows)
        for key in ("q", "k", "v", "ks", "vs"):
            rnd[f"{key}_{seed}"] = p[key]
        rnd[f"out_f32_{seed}"] = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"])
    np.savez_compressed(os.path.join(HERE, "random_small.npz"), **rnd)

    x = quant_rows()
    qv, sc = o.quantize_rows(x)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), x=x, q=qv, scale=sc)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
