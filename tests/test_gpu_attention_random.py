"""Seeded random sweep over the dense-attention plans: each case draws M, N,
a tuned or generic head dim and a split request, so every kernel the planner
routes to (the few-query VALU kernel, the register-direct kernel, the padded
matrix-core blocks, the generic kernel) runs with and without key splits.
Parity: 1e-4 abs + 1e-3 rel elementwise against the oracle's restatement of
attention/softmax_new.cu."""
import numpy as np
import pytest
import torch

import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _draw(rng):
    d = int(rng.choice([32, 64, 64, 128, 128, 256, 96]))
    M = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 48, 63, 64, 65, 127, 130]))
    N = int(rng.choice([1, 15, 16, 17, 63, 64, 65, 1000, 4096, 4099, 16399, 33000]))
    while M * N * d > 1 << 27:  # keeps the oracle to about a second
        N //= 2
    splits = int(rng.choice([0, 0, 0, 1, 2, 7, 1 << 20]))
    qscale = float(rng.choice([1.0, 1.0, 8.0]))
    return d, M, max(N, 1), splits, qscale


@pytest.mark.parametrize("case", range(60))
def test_random_attention_plan(o, case):
    rng = np.random.default_rng(9000 + case)
    d, M, N, splits, qscale = _draw(rng)
    q = (rng.standard_normal((M, d)) * qscale).astype(np.float32)
    k = rng.standard_normal((N, d)).astype(np.float32)
    v = rng.standard_normal((N, d)).astype(np.float32)
    gq, gk, gv = up(q), up(k), up(v)
    out = _gpu.poisoned((M, d))
    p = kvq.attention_params(gq, gk, gv, out, num_splits=splits)
    info = kvq.attention_plan(p)
    n = kvq.attention_workspace_size(p)
    ws = torch.full((max(n, 1),), 0xFF, dtype=torch.uint8, device="cuda")  # NaN bytes: records need no init
    kvq.attention(gq, gk, gv, out, num_splits=splits, workspace=ws)
    torch.cuda.synchronize()
    what = f"case {case}: d={d} M={M} N={N} splits={splits} q*{qscale} kernel={info.kernel} " \
           f"plan splits={info.splits} qblock={info.query_block}"
    np.testing.assert_allclose(down(out), o.attention_f32(q, k, v), atol=1e-4, rtol=1e-3, err_msg=what)
