"""Seeded random sweep over the prefill quantiser's launches: each case draws
the batch, kv heads, new tokens, a tuned or generic head dim, fp32 or bf16
rows and per-sequence or uniform starts that may run before 0 or past the
capacity, so the one-pass grid covers few and many workgroups, partial
blocks of rows and skipped positions.  Bit-exact against the oracle's
quantiser placed by the same start rule (helpers of test_gpu_prefill.py);
no other cache byte may change."""
import numpy as np
import pytest

from _gpu import down, kvq, up
from oracle import oracle as orc
from test_gpu_prefill import _bits, _expected, _inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def o():
    return orc.get()


@pytest.mark.parametrize("case", range(40))
def test_random_prefill(o, case):
    import torch
    rng = np.random.default_rng(11000 + case)
    d = int(rng.choice([32, 64, 128, 256, 96]))
    B = int(rng.choice([1, 2, 5]))
    Hkv = int(rng.choice([1, 3, 8]))
    L = int(rng.choice([1, 7, 64, 300, 1000]))
    while B * Hkv * L * d > 1 << 21:
        L = max(1, L // 2)
    bf16 = bool(rng.integers(0, 2))
    cap = int(rng.choice([L, L + 5, 2 * L + 3]))
    per_seq = bool(rng.integers(0, 2))
    starts = rng.integers(-L // 2, cap - L // 2 + 1, B).astype(np.int32) if per_seq else \
        np.full(B, int(rng.integers(-2, 3)), np.int32)
    xk, kf = _inputs(rng, (B, Hkv, L, d), bf16)
    xv, vf = _inputs(rng, (B, Hkv, L, d), bf16)
    ck = rng.integers(-128, 128, (B, Hkv, cap, d), dtype=np.int8)
    cv = rng.integers(-128, 128, (B, Hkv, cap, d), dtype=np.int8)
    cks = rng.standard_normal((B, Hkv, cap)).astype(np.float32)
    cvs = rng.standard_normal((B, Hkv, cap)).astype(np.float32)
    g = [up(x) for x in (ck, cv, cks, cvs)]
    if per_seq:
        kvq.prefill(xk.cuda(), xv.cuda(), g[0], g[1], g[2], g[3], start=up(starts))
    else:
        kvq.prefill(xk.cuda(), xv.cuda(), g[0], g[1], g[2], g[3], uniform_start=int(starts[0]))
    torch.cuda.synchronize()
    _expected(o, kf, vf, ck, cv, cks, cvs, starts,
              lambda b, pos: None if (pos < 0 or pos >= cap) else (lambda h: (b, h, pos)))
    what = f"case {case}: d={d} B={B} Hkv={Hkv} L={L} cap={cap} bf16={bf16} starts={starts.tolist()}"
    assert np.array_equal(down(g[0]), ck) and np.array_equal(down(g[1]), cv), what
    assert np.array_equal(_bits(down(g[2])), _bits(cks)) and np.array_equal(_bits(down(g[3])), _bits(cvs)), what
