"""Paged KV cache (include/kvq.h part 3) on the GPU, through the C ABI.

Pinned by equivalence with the contiguous layout: the same tokens scattered
over a page pool in random order must give
  * the oracle's output over the contiguous cache (1e-4 abs + 1e-3 rel), and
  * bit for bit the output of kvq_decode_launch on the contiguous cache when
    both run the same tuned kernel with the same splits (the summation order
    is then identical);
and a fused or separate append must write exactly the bytes the oracle's
append writes into the contiguous cache, at the token's page slot.

Unused pool slots hold random int8 and NaN/Inf scales, and unused block-table
entries hold out-of-range page ids, so any read outside the sequence's own
slots shows up.
"""
import math

import numpy as np
import pytest
import torch

from _util import assert_close, make_problem
import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def to_pages(rng, k, v, ks, vs, lengths, page, spare=5):
    """Scatter the first lengths[b] (at least one page's worth) tokens of each
    sequence into a shuffled page pool.  Returns pool arrays, block table."""
    B, Hkv, cap, d = k.shape
    maxp = math.ceil(cap / page)
    need = [max(1, math.ceil(int(n) / page)) for n in lengths]
    total = sum(need) + spare
    order = rng.permutation(total)
    kp = rng.integers(-128, 128, (total, Hkv, page, d), dtype=np.int8)
    vp = rng.integers(-128, 128, (total, Hkv, page, d), dtype=np.int8)
    ksp = np.full((total, Hkv, page), np.nan, np.float32)
    vsp = np.full((total, Hkv, page), np.inf, np.float32)
    table = np.full((B, maxp), 1 << 30, np.int32)
    at = 0
    for b in range(B):
        for j in range(need[b]):
            pg = int(order[at])
            at += 1
            table[b, j] = pg
            t0, t1 = j * page, min(cap, (j + 1) * page)
            kp[pg, :, : t1 - t0] = k[b, :, t0:t1]
            vp[pg, :, : t1 - t0] = v[b, :, t0:t1]
            ksp[pg, :, : t1 - t0] = ks[b, :, t0:t1]
            vsp[pg, :, : t1 - t0] = vs[b, :, t0:t1]
    return kp, vp, ksp, vsp, table


def from_pages(kp, vp, ksp, vsp, table, lengths, shape):
    """Gather the pages back into contiguous arrays (the first lengths[b] tokens)."""
    B, Hkv, cap, d = shape
    page = kp.shape[2]
    k = np.zeros(shape, np.int8)
    v = np.zeros(shape, np.int8)
    ks = np.zeros(shape[:3], np.float32)
    vs = np.zeros(shape[:3], np.float32)
    for b in range(B):
        for t in range(int(lengths[b])):
            pg, sl = table[b, t // page], t % page
            k[b, :, t], v[b, :, t] = kp[pg, :, sl], vp[pg, :, sl]
            ks[b, :, t], vs[b, :, t] = ksp[pg, :, sl], vsp[pg, :, sl]
    return k, v, ks, vs


def paged_decode(q, kp, vp, ksp, vsp, table, lengths, splits=0, k_new=None, v_new=None, max_seq_len=0):
    g = [up(x) for x in (q, kp, vp, ksp, vsp, table, np.asarray(lengths, np.int32))]
    kn = None if k_new is None else up(k_new)
    vn = None if v_new is None else up(v_new)
    out = _gpu.poisoned(q.shape)
    dec = kvq.PagedDecoder(g[0], g[1], g[2], g[3], g[4], g[5], g[6], out, max_seq_len=max_seq_len,
                           num_splits=splits, k_new=kn, v_new=vn)
    dec()
    torch.cuda.synchronize()
    return down(out), down(g[1]), down(g[2]), down(g[3]), down(g[4]), dec


CASES = [  # (G, d, page): MFMA needs d = 128, G % 4 == 0 and a power-of-two page >= 32;
    (1, 128, 16), (1, 128, 32), (1, 128, 256),  # the VALU kernel a power-of-two page that is a
    (2, 64, 32), (1, 256, 16), (1, 32, 64),     # multiple of its wave tile; anything else runs
    (4, 128, 32), (8, 128, 128), (4, 128, 64),  # the generic kernel.
    (1, 128, 24), (4, 128, 48), (8, 128, 16), (1, 32, 16), (3, 96, 32),
    (4, 64, 32), (8, 64, 128),
]


@pytest.mark.parametrize("G,d,page", CASES)
def test_paged_matches_oracle(o, G, d, page):
    rng = np.random.default_rng(7 * G + d + page)
    B, Hkv, cap = 5, 2, 700
    lengths = np.array([700, 1, 333, 0, 512], np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, dist="student_t", lengths=lengths)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], lengths, page)
    got = paged_decode(p["q"], kp, vp, ksp, vsp, table, lengths)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"paged G={G} d={d} page={page}")


@pytest.mark.parametrize("G,d,page,splits", [(1, 128, 32, 0), (1, 128, 64, 3), (8, 128, 32, 0),
                                             (4, 128, 128, 5), (2, 64, 64, 0), (1, 256, 16, 2), (8, 64, 64, 3)])
def test_paged_bitwise_equals_contiguous(o, G, d, page, splits):
    """Same tuned kernel, same splits: identical bits to the contiguous layout."""
    rng = np.random.default_rng(100 + G + d + page + splits)
    B, Hkv, cap = 6, 2, 1024
    lengths = rng.integers(1, cap + 1, B).astype(np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], lengths, page)
    got = paged_decode(p["q"], kp, vp, ksp, vsp, table, lengths, splits=splits)[0]
    ref = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, splits=splits)[0]
    assert np.array_equal(_bits(got), _bits(ref))


@pytest.mark.parametrize("G,d,page", [(1, 128, 32), (8, 128, 32), (4, 128, 128), (2, 64, 16), (3, 96, 32),
                                      (4, 64, 32)])
def test_paged_fused_append(o, G, d, page):
    """The new token lands in its page slot with the oracle's bits; the output
    attends over it."""
    rng = np.random.default_rng(300 + G + d + page)
    B, Hkv, cap = 4, 2, 600
    lengths = np.array([600, 1, 257, 64], np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], lengths, page)
    got, gkp, gvp, gksp, gvsp, _ = paged_decode(p["q"], kp, vp, ksp, vsp, table, lengths, k_new=kn, v_new=vn)
    o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=lengths - 1)
    k, v, ks, vs = from_pages(gkp, gvp, gksp, gvsp, table, lengths, p["k"].shape)
    for b in range(B):
        n = int(lengths[b])
        assert np.array_equal(k[b, :, :n], p["k"][b, :, :n]) and np.array_equal(v[b, :, :n], p["v"][b, :, :n])
        assert np.array_equal(_bits(ks[b, :, :n]), _bits(p["ks"][b, :, :n]))
        assert np.array_equal(_bits(vs[b, :, :n]), _bits(p["vs"][b, :, :n]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"paged fused append G={G} d={d} page={page}")


def test_paged_append_kernel(o):
    """kvq_paged_append_launch: same bits as kvq_append_launch at the page slot;
    positions past the table are skipped."""
    rng = np.random.default_rng(9)
    B, Hkv, cap, d, page = 3, 2, 256, 128, 32
    lengths = np.array([256, 100, 31], np.int32)
    p = make_problem(rng, B, Hkv, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], lengths, page)
    kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    pos = np.array([255, 99, 300], np.int32)  # the last one is past max_pages * page: skipped
    g = [up(x) for x in (kp, vp, ksp, vsp, table, pos, kn, vn)]
    kvq.paged_append(g[6], g[7], g[0], g[1], g[2], g[3], g[4], positions=g[5])
    torch.cuda.synchronize()
    o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=np.array([255, 99, -1], np.int32))
    k, v, ks, vs = from_pages(down(g[0]), down(g[1]), down(g[2]), down(g[3]), table, lengths, p["k"].shape)
    for b in range(B):
        n = int(lengths[b])
        assert np.array_equal(k[b, :, :n], p["k"][b, :, :n]) and np.array_equal(v[b, :, :n], p["v"][b, :, :n])
        assert np.array_equal(_bits(ks[b, :, :n]), _bits(p["ks"][b, :, :n]))
    # nothing else in the pool changed
    written = {(int(table[b, pos[b] // page]), h, int(pos[b] % page)) for b in range(B) if pos[b] < cap
               for h in range(Hkv)}
    for after, before in ((down(g[0]), kp), (down(g[1]), vp)):
        changed = {tuple(int(i) for i in ix) for ix in np.argwhere((after != before).any(axis=-1))}
        assert changed <= written, sorted(changed - written)[:5]


def test_paged_repeated_launches(o):
    """One workspace, lengths changed between launches (schedule recomputed,
    counters back at zero)."""
    rng = np.random.default_rng(21)
    B, Hkv, G, cap, d, page = 8, 2, 8, 1024, 128, 64
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows)
    full = np.full(B, cap, np.int32)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], full, page)
    g = [up(x) for x in (p["q"], kp, vp, ksp, vsp, table)]
    glen = torch.zeros(B, dtype=torch.int32, device=_gpu.dev())
    out = _gpu.poisoned(p["q"].shape)
    dec = kvq.PagedDecoder(g[0], g[1], g[2], g[3], g[4], g[5], glen, out, max_seq_len=cap)
    for it in range(4):
        lengths = rng.integers(0, cap + 1, B).astype(np.int32)
        glen.copy_(torch.from_numpy(lengths))
        out.fill_(float("nan"))
        dec()
        torch.cuda.synchronize()
        want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
        assert_close(down(out), want, what=f"paged launch {it}")


@pytest.mark.parametrize("G,page", [(1, 32), (8, 64)])
def test_paged_uniform_length(o, G, page):
    """lengths == NULL: every sequence has max_seq_len tokens (static splits,
    no schedule launch); bitwise equal to the contiguous uniform decode, with
    the fused append."""
    rng = np.random.default_rng(40 + G + page)
    B, Hkv, cap, d, L = 3, 2, 512, 128, 448
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows)
    kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], np.full(B, cap), page)
    g = [up(x) for x in (p["q"], kp, vp, ksp, vsp, table, kn, vn)]
    out = _gpu.poisoned(p["q"].shape)
    kvq.PagedDecoder(g[0], g[1], g[2], g[3], g[4], g[5], None, out, max_seq_len=L, k_new=g[6], v_new=g[7])()
    torch.cuda.synchronize()
    ref = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], max_seq_len=L, k_new=kn, v_new=vn)[0]
    assert np.array_equal(_bits(down(out)), _bits(ref))


@pytest.mark.parametrize("page", [32, 128])
def test_paged_in_kernel_schedule_bitwise(o, page):
    """A ragged batch past one round of items (B = 100, 8 work units per
    sequence): the matrix-core kernel derives the split schedule itself and
    fetches each tile's block-table entry one tile ahead; with fused append,
    identical bits to the contiguous layout (same plan), and the oracle."""
    rng = np.random.default_rng(900 + page)
    B, Hkv, G, cap, d = 100, 8, 4, 1024, 64
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[:3] = [cap, 0, 1]
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, dist="student_t", lengths=lengths)
    kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], lengths, page)
    got, gkp, gvp, gksp, gvsp, dec = paged_decode(p["q"], kp, vp, ksp, vsp, table, lengths, k_new=kn, v_new=vn,
                                                  max_seq_len=cap)
    ref, rk, rv, rks, rvs = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, k_new=kn,
                                        v_new=vn)
    assert np.array_equal(_bits(got), _bits(ref))
    k2, v2, ks2, vs2 = from_pages(gkp, gvp, gksp, gvsp, table, lengths, p["k"].shape)
    for x, y in ((k2, rk), (v2, rv)):
        for b in range(B):
            assert np.array_equal(x[b, :, : lengths[b]], y[b, :, : lengths[b]])
    for x, y in ((ks2, rks), (vs2, rvs)):
        for b in range(B):
            assert np.array_equal(_bits(x[b, :, : lengths[b]]), _bits(y[b, :, : lengths[b]]))
    o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=lengths - 1)
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"paged in-kernel schedule page={page}")
