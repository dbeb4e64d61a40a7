"""The flattened tile-stream plan of ragged grouped-query batches
(decode_mfma_flat: at most 64 sequences, matrix-core kernel, num_splits = 0).

Every wave takes an equal range of the sequences' 32-token tiles laid end to
end, so ranges cross sequence boundaries and sequences are split at arbitrary
tiles; records are per wave (mid-range sequence tails) or per run of waves
sharing a last sequence, with empty records filling the ids a run stands for.
The cases aim at each of those paths:

* many short sequences per wave (middle segments written directly);
* one long sequence over nearly every wave (more records than one merge load
  round);
* fewer tiles than waves (one tile per wave, most waves idle);
* consecutive one-tile sequences with the fused append (each wave appends
  several tokens, one loaded while the previous is still being appended);
* empty sequences at the start, middle and end;
* 16 query heads per kv head (two head groups per kv head), d = 64;
* a paged cache; repeated launches with new lengths (counters back at 0).

Parity as in test_gpu_decode: out[b, hq] = oracle kvq_ref_decode_f32 over the
first length[b] tokens of kv head hq / G, 1e-4 abs + 1e-3 rel elementwise;
appended int8 values and scales bit-exact.
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


def _plan(B, Hq, Hkv, d, cap):
    A = 1 << 20
    p = kvq.DecodeParams(B, Hq, Hkv, d, cap, cap, A, A, A, A, A, A, A, 0.0, 0, None, None)
    return kvq.decode_plan(p)


def _check(o, B, Hkv, G, cap, d, lengths, rng, append=False, dist="normal", what=""):
    info = _plan(B, Hkv * G, Hkv, d, cap)
    assert (info.kernel, info.split_plan) == (kvq.KERNEL_DECODE_MFMA, kvq.SPLITS_TILES), what
    # the flattened plan: records for 4 waves per workgroup plus B ids per query head
    units = Hkv * (G // (8 if G % 8 == 0 else 4))
    S = 256 // units
    assert 4 * B >= S, what
    recs = (4 * S + B) * Hkv * G
    ru = lambda x: (x + 255) // 256 * 256
    assert info.workspace_bytes == 256 * 1024 + ru(recs * 8) + ru(recs * d * 4), what
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, dist=dist, lengths=lengths)
    kn = vn = None
    if append:
        kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
        vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    got, gk, gv, gks, gvs = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths,
                                         max_seq_len=cap, k_new=kn, v_new=vn)
    if append:
        pos = np.asarray(lengths) - 1
        o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=pos)
        assert np.array_equal(gk, p["k"]) and np.array_equal(gv, p["v"]), f"{what}: appended int8 differs"
        assert np.array_equal(_bits(gks), _bits(p["ks"])) and np.array_equal(_bits(gvs), _bits(p["vs"]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=what)
    return p, got


@pytest.mark.parametrize("seed", [17, 29, 101])
def test_cfg2_shape_short(o, seed):
    """cfg2's batch (B16 Hq32 Hkv8 d128, lengths U[1024, 8192]) at 1/4 length."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(256, 2049, 16).astype(np.int32)
    _check(o, 16, 8, 4, 2048, 128, lengths, rng, what=f"cfg2/4 seed {seed}")


@pytest.mark.parametrize("G,d", [(4, 128), (8, 128), (8, 64), (16, 64)])
def test_many_short_sequences(o, G, d):
    """64 sequences of 0..300 tokens: most waves hold several whole
    sequences (direct outputs) between a tail and a head."""
    rng = np.random.default_rng(G * 1000 + d)
    B, Hkv, cap = 64, 2, 300
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[:7] = [0, 1, 31, 32, 33, 300, 0]
    lengths[-1] = 0
    _check(o, B, Hkv, G, cap, d, lengths, rng, append=False, what=f"short G={G} d={d}")


@pytest.mark.parametrize("L", [20001, 12000])
def test_one_long_sequence_among_short(o, L):
    """One long sequence over nearly every wave of its work units (a record
    per covering wave: several load rounds of the merge) beside short ones."""
    rng = np.random.default_rng(L)
    B, Hkv, G, d = 8, 8, 4, 128
    lengths = rng.integers(0, 100, B).astype(np.int32)
    lengths[7] = L
    cap = (L + 3) // 4 * 4  # the matrix-core kernel reads scales in aligned quads
    _check(o, B, Hkv, G, cap, d, lengths, rng, append=True, dist="outlier", what=f"L={L}")


def test_fewer_tiles_than_waves(o):
    """5 tiles for 128 waves per work unit: the first waves take one tile each."""
    rng = np.random.default_rng(3)
    lengths = np.array([1, 0, 5, 40, 0, 17, 2, 30], np.int32)
    _check(o, 8, 8, 4, 64, 128, lengths, rng, append=True, what="tiny")


def test_all_sequences_empty(o):
    rng = np.random.default_rng(4)
    lengths = np.zeros(9, np.int32)
    p = make_problem(rng, 9, 16, 4, 64, 128, o.quantize_rows, lengths=lengths)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, max_seq_len=64)[0]
    assert np.array_equal(got, np.zeros_like(got))


@pytest.mark.parametrize("pattern", ["ones", "mixed"])
def test_append_consecutive_one_tile_sequences(o, pattern):
    """Sequence ends on consecutive tiles: a wave appends several tokens, the
    next one's fp32 row loading while the current one is appended."""
    rng = np.random.default_rng(5 if pattern == "ones" else 6)
    if pattern == "ones":
        lengths = np.array([1, 1, 32, 1, 33, 2, 1, 64, 1, 1, 31, 1] * 5, np.int32)
    else:
        lengths = rng.integers(1, 70, 64).astype(np.int32)
    B = len(lengths)
    _check(o, B, 2, 8, 96, 128, lengths, rng, append=True, dist="student_t", what=pattern)


@pytest.mark.parametrize("page", [32, 128])
def test_flat_plan_paged(o, page):
    rng = np.random.default_rng(11 + page)
    B, Hkv, G, cap, d = 20, 4, 4, 2100, 128
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[:4] = [cap, 0, 1, 33]
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], lengths, page)
    g = [up(x) for x in (p["q"], kp, vp, ksp, vsp, table, lengths, kn, vn)]
    out = _gpu.poisoned(p["q"].shape)
    kvq.PagedDecoder(g[0], g[1], g[2], g[3], g[4], g[5], g[6], out, max_seq_len=cap, k_new=g[7], v_new=g[8])()
    torch.cuda.synchronize()
    k, v, ks, vs = p["k"].copy(), p["v"].copy(), p["ks"].copy(), p["vs"].copy()
    o.append(kn, vn, k, v, ks, vs, positions=lengths - 1)
    want = o.decode_f32(p["q"], k, v, ks, vs, lengths=lengths)
    assert_close(down(out), want, what=f"paged {page}")


def test_repeated_launches_new_lengths(o):
    """One workspace; lengths changed between launches (arrival counters are
    back at zero after every launch); each output bitwise repeatable."""
    rng = np.random.default_rng(12)
    B, Hkv, G, cap, d = 33, 8, 4, 3000, 128
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows)
    gq, gk, gv, gks, gvs = up(p["q"]), up(p["k"]), up(p["v"]), up(p["ks"]), up(p["vs"])
    glen = torch.zeros(B, dtype=torch.int32, device=_gpu.dev())
    out = _gpu.poisoned(p["q"].shape)
    dec = kvq.Decoder(gq, gk, gv, gks, gvs, out, lengths=glen, max_seq_len=cap)
    for it in range(4):
        lengths = rng.integers(0, cap + 1, B).astype(np.int32)
        if it == 1:
            lengths[:] = cap
        glen.copy_(torch.from_numpy(lengths))
        out.fill_(float("nan"))
        dec()
        torch.cuda.synchronize()
        first = down(out)
        want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
        assert_close(first, want, what=f"launch {it}")
        dec()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(down(out)), _bits(first)), f"launch {it} not repeatable"


@pytest.mark.parametrize("B,cap", [(65, 256), (256, 64), (1000, 64)])
def test_big_batch_plan(o, B, cap):
    """More than 64 sequences in a small step (at most 16 tiles per wave):
    lengths scanned into LDS, each wave's window of 64 sequences starting at
    its first one (cfg4's head layout at short lengths, with the fused append
    and empty sequences)."""
    rng = np.random.default_rng(B)
    Hkv, G, d = 8, 8, 128
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[:5] = [0, 1, 32, 33, cap]
    _check(o, B, Hkv, G, cap, d, lengths, rng, append=True, dist="student_t", what=f"B={B}")


def test_run_of_empty_sequences(o):
    """1500 sequences of 0-32 tokens with a run of 300 empty ones.  Each empty
    sequence still holds its kFlatSwitchTiles virtual tiles, so the run is
    spread over the waves like any other part of the stream (and no wave's
    range spans 64 sequences: the planner's bound keeps a range below 48
    virtual tiles, which the host checker asserts)."""
    rng = np.random.default_rng(2000)
    B, Hkv, G, cap, d = 1500, 8, 4, 32, 64
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[100:400] = 0  # a run of empty sequences longer than a window
    _check(o, B, Hkv, G, cap, d, lengths, rng, append=True, what="window")


def test_max_batch_plan(o):
    """kFlatMaxSeqs = 4096 sequences of 1-5 tokens."""
    rng = np.random.default_rng(4096)
    B, Hkv, G, cap, d = 4096, 1, 4, 8, 64
    lengths = rng.integers(1, 6, B).astype(np.int32)
    _check(o, B, Hkv, G, cap, d, lengths, rng, what="4096")
