"""Edge cases of the grouped-query decode plans (matrix-core kernel: 4 or 8
query heads per kv head, d in {64, 128}, num_splits = 0), one plan each:

* the in-kernel plan (ragged, at most 64 sequences and 256 / U items per
  work unit): one item per sequence exactly at its limit, empty sequences
  between long ones, a paged cache, lengths changed between launches;
* the device split schedule (more sequences, or more work units per
  sequence than one round holds): a thousand tiny sequences in
  longest-first rounds, more kv heads than CUs;
* static splits (no lengths array) for a batch whose work units do not
  divide the CU count, and a batch too small to split at all.

Parity as in test_gpu_decode: out[b, hq] = oracle kvq_ref_decode_f32 over
the first length[b] tokens of kv head hq / G, 1e-4 abs + 1e-3 rel
elementwise; appended int8 values and scales bit-exact.
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


def _check(o, B, Hkv, G, cap, d, lengths, rng, append=False, dist="normal", what="", max_seq_len=None):
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, dist=dist, lengths=lengths)
    kn = vn = None
    if append:
        kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
        vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    got, gk, gv, gks, gvs = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths,
                                         max_seq_len=max_seq_len, k_new=kn, v_new=vn)
    L = lengths if lengths is not None else np.full(B, max_seq_len or cap, np.int32)
    if append:
        o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=np.asarray(L) - 1)
        assert np.array_equal(gk, p["k"]) and np.array_equal(gv, p["v"]), f"{what}: appended int8 differs"
        assert np.array_equal(_bits(gks), _bits(p["ks"])) and np.array_equal(_bits(gvs), _bits(p["vs"]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=L)
    assert_close(got, want, what=what)
    return p, got


@pytest.mark.parametrize("B", [300, 1025])
def test_schedule_many_tiny_sequences(o, B):
    """Hundreds to a thousand sequences of 0..40 tokens (split schedule,
    longest-first rounds; a tile holds a whole sequence)."""
    rng = np.random.default_rng(B)
    Hkv, G, cap, d = 1, 4, 40, 64
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[:6] = [cap, 0, 1, 31, 32, 33]
    lengths[-1] = cap
    _check(o, B, Hkv, G, cap, d, lengths, rng, append=True, what=f"B={B}")


@pytest.mark.parametrize("G,d", [(8, 128), (4, 64)])
def test_schedule_tiny_sequences_student_t(o, G, d):
    """300 sequences of 1..40 tokens, heavy-tailed values, 2 kv heads; waves
    1-3 of a workgroup have no tile at all."""
    rng = np.random.default_rng(7 * G + d)
    B, Hkv, cap = 300, 2, 40
    lengths = rng.integers(1, cap + 1, B).astype(np.int32)
    _check(o, B, Hkv, G, cap, d, lengths, rng, append=True, dist="student_t", what=f"tiny G={G} d={d}")


@pytest.mark.parametrize("shift", [0, 32, 1])
def test_in_kernel_plan_one_item_per_sequence(o, shift):
    """Hkv = 8, G = 4: 32 items per work unit and 32 sequences, so the
    in-kernel plan gives every sequence exactly one item (no merge); one
    sequence 32 tokens or 1 token shorter than the others."""
    rng = np.random.default_rng(300 + shift)
    B, Hkv, G, cap, d = 32, 8, 4, 1024, 128
    lengths = np.full(B, cap, np.int32)
    lengths[5] -= shift
    _check(o, B, Hkv, G, cap, d, lengths, rng, append=True, what=f"shift={shift}")


@pytest.mark.parametrize("G,d", [(4, 128), (8, 64)])
def test_static_splits_without_lengths(o, G, d):
    """lengths == NULL (every sequence max_seq_len tokens): static splits of
    a batch whose work units do not divide the CU count."""
    rng = np.random.default_rng(40 + G)
    B, Hkv, cap, L = 5, 8, 3072, 3000
    _check(o, B, Hkv, G, cap, d, None, rng, append=True, what=f"uniform G={G} d={d}", max_seq_len=L)


def test_in_kernel_plan_small_batch(o):
    """A few short sequences (one of them empty): the in-kernel plan with
    mostly unsplit items."""
    rng = np.random.default_rng(5)
    B, Hkv, G, cap, d = 4, 2, 8, 256, 128
    lengths = np.array([100, 0, 50, 3], np.int32)
    _check(o, B, Hkv, G, cap, d, lengths, rng, append=True, what="small total")


def test_schedule_more_kv_heads_than_cus(o):
    """260 kv heads x 1 head group: more work units per sequence than one
    round of the in-kernel plan holds, so the split schedule runs."""
    rng = np.random.default_rng(6)
    B, Hkv, G, cap, d = 2, 260, 4, 96, 64
    lengths = np.array([96, 37], np.int32)
    _check(o, B, Hkv, G, cap, d, lengths, rng, what="260 lanes")


def test_in_kernel_plan_empty_between_full(o):
    """Empty sequences between long ones (one empty item each, zero rows);
    the output is bitwise the same on a second launch (the merge order is
    fixed)."""
    rng = np.random.default_rng(8)
    B, Hkv, G, cap, d = 40, 2, 4, 3000, 128
    lengths = rng.integers(1000, cap + 1, B).astype(np.int32)
    lengths[::3] = 0
    lengths[-1] = 0
    p, got = _check(o, B, Hkv, G, cap, d, lengths, rng, what="empties")
    assert np.array_equal(got[lengths == 0], np.zeros_like(got[lengths == 0]))
    again = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)[0]
    assert np.array_equal(_bits(again), _bits(got))


@pytest.mark.parametrize("page", [32, 64])
def test_in_kernel_plan_paged(o, page):
    """Paged cache under the in-kernel plan (items start at multiples of the
    128-token workgroup step, so every wave tile stays inside a page)."""
    rng = np.random.default_rng(9 + page)
    B, Hkv, G, cap, d = 24, 2, 8, 1500, 128
    lengths = rng.integers(1, cap + 1, B).astype(np.int32)
    lengths[:3] = [cap, 1, 33]
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], lengths, page)
    g = [up(x) for x in (p["q"], kp, vp, ksp, vsp, table, lengths, kn, vn)]
    out = _gpu.poisoned(p["q"].shape)
    kvq.PagedDecoder(g[0], g[1], g[2], g[3], g[4], g[5], g[6], out, max_seq_len=cap, k_new=g[7], v_new=g[8])()
    torch.cuda.synchronize()
    o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=lengths - 1)
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(down(out), want, what=f"paged page={page}")


def test_in_kernel_plan_repeated_launches(o):
    """One workspace, lengths changed between launches, one launch with every
    length 0 (the plan is rebuilt from the device lengths each launch;
    counters back at zero)."""
    rng = np.random.default_rng(10)
    B, Hkv, G, cap, d = 50, 4, 4, 2000, 64
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows)
    gq, gk, gv, gks, gvs = up(p["q"]), up(p["k"]), up(p["v"]), up(p["ks"]), up(p["vs"])
    glen = torch.zeros(B, dtype=torch.int32, device=_gpu.dev())
    out = _gpu.poisoned(p["q"].shape)
    dec = kvq.Decoder(gq, gk, gv, gks, gvs, out, lengths=glen, max_seq_len=cap)
    for it in range(4):
        lengths = rng.integers(0, cap + 1, B).astype(np.int32)
        if it == 2:
            lengths[:] = 0
        glen.copy_(torch.from_numpy(lengths))
        out.fill_(float("nan"))
        dec()
        torch.cuda.synchronize()
        want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
        assert_close(down(out), want, what=f"launch {it}")
