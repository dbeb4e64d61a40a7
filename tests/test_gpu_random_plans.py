"""Seeded random sweep over the decode plans: each case draws a batch size,
head counts, head dim, capacity, ragged or uniform lengths (with 0, 1 and the
capacity mixed in), a split request, a contiguous or paged cache and an
optional fused append, so the tuned kernels run under every split plan (the
in-kernel plan, the split schedule in one or several rounds, static splits,
requested splits) with merges of 1 to many splits.

Parity as in test_gpu_decode: out[b, hq] = oracle kvq_ref_decode_f32 over the
first length[b] tokens of kv head hq / G, 1e-4 abs + 1e-3 rel elementwise;
appended int8 values and scales bit-exact, in the contiguous cache or in the
page pool (where every other byte must be unchanged).
"""
import numpy as np
import pytest
import torch

from _util import assert_close, make_problem
import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc
from test_gpu_paged import to_pages

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _draw(rng):
    G = int(rng.choice([1, 2, 4, 8]))
    d = int(rng.choice([64, 128])) if G >= 4 else int(rng.choice([32, 64, 128, 256]))
    Hkv = int(rng.choice([1, 2, 3, 8]))
    B = int(rng.choice([1, 3, 17, 64, 65, 130]))
    cap = int(rng.choice([64, 384, 1500, 4096]))
    while B * Hkv * cap * d > 1 << 25:  # keeps the oracle and input generation to about a second
        cap //= 2
    ragged = bool(rng.integers(0, 4))  # 3 in 4 cases ragged
    if ragged:
        lengths = rng.integers(0, cap + 1, B).astype(np.int32)
        for i, v in enumerate(rng.choice([0, 1, cap, 127, 128, 129], min(B, 3), replace=False)):
            lengths[i] = min(int(v), cap)
    else:
        lengths = None
    splits = int(rng.choice([0, 0, 0, 1, 3, 16]))
    paged = int(rng.choice([0, 0, 32, 64]))
    append = bool(rng.integers(0, 2))
    return G, d, Hkv, B, cap, lengths, splits, paged, append


@pytest.mark.parametrize("case", range(120))
def test_random_plan(o, case):
    rng = np.random.default_rng(7000 + case)
    G, d, Hkv, B, cap, lengths, splits, paged, append = _draw(rng)
    what = f"case {case}: G={G} d={d} Hkv={Hkv} B={B} cap={cap} ragged={lengths is not None} " \
           f"splits={splits} page={paged} append={append}"
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = vn = None
    if append:
        kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
        vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    L = lengths if lengths is not None else np.full(B, cap, np.int32)
    if paged:
        kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], np.full(B, cap), paged)
        g = [up(x) for x in (p["q"], kp, vp, ksp, vsp, table)]
        glen = None if lengths is None else up(lengths)
        gkn = None if kn is None else up(kn)
        gvn = None if vn is None else up(vn)
        out = _gpu.poisoned(p["q"].shape)
        kvq.PagedDecoder(g[0], g[1], g[2], g[3], g[4], g[5], glen, out, max_seq_len=cap, num_splits=splits,
                         k_new=gkn, v_new=gvn)()
        torch.cuda.synchronize()
        got = down(out)
        pool = [down(x) for x in g[1:5]]
    else:
        got, gk, gv, gks, gvs = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths,
                                             max_seq_len=cap, splits=splits, k_new=kn, v_new=vn)
    if append:
        o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=L - 1)
        if not paged:
            assert np.array_equal(gk, p["k"]) and np.array_equal(gv, p["v"]), f"{what}: appended int8 differs"
            assert np.array_equal(_bits(gks), _bits(p["ks"])) and np.array_equal(_bits(gvs), _bits(p["vs"])), what
        else:
            # The page pool after the step: the original pool with each
            # sequence's token length-1 replaced by the oracle's appended row,
            # and no other byte changed.
            want_pool = [x.copy() for x in (kp, vp, ksp, vsp)]
            for b in range(B):
                t = int(L[b]) - 1
                if t < 0:
                    continue
                pg, sl = int(table[b, t // paged]), t % paged
                for wp, src in zip(want_pool, (p["k"], p["v"], p["ks"], p["vs"])):
                    wp[pg, :, sl] = src[b, :, t]
            assert np.array_equal(pool[0], want_pool[0]) and np.array_equal(pool[1], want_pool[1]), \
                f"{what}: paged appended int8 differs"
            assert np.array_equal(_bits(pool[2]), _bits(want_pool[2])) and \
                np.array_equal(_bits(pool[3]), _bits(want_pool[3])), f"{what}: paged appended scales differ"
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=L)
    assert_close(got, want, what=what)
