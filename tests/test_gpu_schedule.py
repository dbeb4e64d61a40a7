"""Ragged batches under the device split schedule (per-sequence lengths on the
device, num_splits = 0): the schedule kernel picks the chunk from the actual
lengths and orders the work longest first, so every split of every sequence
must be computed exactly once, merged right, and the arrival counters left at
zero for the next launch.

Parity as in test_gpu_decode: out[b, hq] = oracle kvq_ref_decode_f32 over the
first length[b] tokens of kv head hq / G; 1e-4 abs + 1e-3 rel elementwise;
appended int8 values and scales bit-exact.
"""
import numpy as np
import pytest
import torch

from _util import assert_close, lpt_case, make_problem
import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _ragged_lengths(rng, B, cap):
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    edge = np.array([0, 1, cap, 129, 2, cap - 1], np.int32)[:B]
    lengths[: len(edge)] = edge
    return lengths


@pytest.mark.parametrize("append", [False, True])
@pytest.mark.parametrize("G,d", [(1, 128), (2, 64), (4, 128), (8, 128), (1, 256), (4, 32), (4, 64), (8, 64)])
def test_schedule_ragged(o, G, d, append):
    """VALU (G = 1, 2; d 32..256) and matrix-core (G = 4, 8 at d = 128) kernels."""
    rng = np.random.default_rng(1000 * G + d + append)
    B, Hkv, cap = 24, 2, 2048
    lengths = _ragged_lengths(rng, B, cap)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, dist="student_t", lengths=lengths)
    kn = vn = None
    if append:
        kn = rng.standard_t(4, (B, Hkv, d)).astype(np.float32)
        vn = rng.standard_t(4, (B, Hkv, d)).astype(np.float32)
    got, gk, gv, gks, gvs = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths,
                                         k_new=kn, v_new=vn)
    if append:
        o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=lengths - 1)
        assert np.array_equal(gk, p["k"]) and np.array_equal(gv, p["v"]), "appended int8 differs"
        assert np.array_equal(_bits(gks), _bits(p["ks"])) and np.array_equal(_bits(gvs), _bits(p["vs"]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"scheduled G={G} d={d} append={append}")


@pytest.mark.parametrize("G", [1, 4])
def test_schedule_one_long_many_short(o, G):
    """One long sequence among many short ones: the chunk shrinks to the
    batch's mean, so the long one is cut into many splits (more than one
    merge pass can hold for G = 1) while the short ones run whole."""
    rng = np.random.default_rng(55 + G)
    B, Hkv, cap, d = 96, 1, 20000, 128
    lengths = rng.integers(1, 40, B).astype(np.int32)
    lengths[17] = cap
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"one long, many short, G={G}")


def test_schedule_large_batch(o):
    """More sequences than the schedule kernel's threads (several scan rounds)."""
    rng = np.random.default_rng(3)
    B, Hkv, G, cap, d = 2500, 1, 2, 96, 64
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what="large batch")


@pytest.mark.parametrize("G", [1, 8])
def test_schedule_repeated_launches_new_lengths(o, G):
    """One workspace, several launches whose device lengths change in between
    (the schedule is recomputed each launch; counters must be back at zero)."""
    rng = np.random.default_rng(90 + G)
    B, Hkv, cap, d = 12, 2, 1500, 128
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
        want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
        assert_close(down(out), want, what=f"launch {it}")


@pytest.mark.parametrize("G", [1, 4])
def test_schedule_all_empty(o, G):
    """Every length 0 (no tokens at all): one empty item per sequence, zero output rows."""
    rng = np.random.default_rng(7 + G)
    B, Hkv, cap, d = 5, 2, 256, 128
    lengths = np.zeros(B, np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)[0]
    assert np.array_equal(got, np.zeros_like(got))


@pytest.mark.parametrize("B", [255, 256, 257])
def test_schedule_at_the_one_round_limit(o, B):
    """Matrix-core kernel, G = 8, Hkv = 2, sequences too long for the flat
    plan: the schedule launch runs everything in one round while B <= 512 / 2
    sequences; above that the decode kernel derives longest-first rounds
    itself; both sides of the switch are exact."""
    rng = np.random.default_rng(B)
    Hkv, G, cap, d = 2, 8, 1100, 128
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[:3] = [cap, 0, 1]
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    info = kvq.decode_plan(kvq.decode_params(up(p["q"]), up(p["k"]), up(p["v"]), up(p["ks"]), up(p["vs"]),
                                             torch.empty(B, Hkv * G, d, device="cuda"), lengths=up(lengths),
                                             max_seq_len=cap))
    assert info.split_plan == (kvq.SPLITS_SCHEDULE if B <= 256 else kvq.SPLITS_IN_KERNEL)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"B={B}")


@pytest.mark.parametrize("B,G,cap", [(300, 8, 2048), (1100, 8, 512), (300, 4, 2048), (700, 1, 1024)])
def test_schedule_several_passes(o, B, G, cap):
    """One kv head, so one work unit per sequence: the schedule kernel (256
    threads) walks the batch in passes of 256 sequences -- two in one round
    (B = 300 <= 512 items), across rounds five (B = 1100, more sequences than
    the matrix-core kernel derives a schedule for itself) and three (B = 700,
    the VALU kernel)."""
    rng = np.random.default_rng(B + G)
    Hkv, d = 1, 128
    lengths = _ragged_lengths(rng, B, cap)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    info = kvq.decode_plan(kvq.decode_params(up(p["q"]), up(p["k"]), up(p["v"]), up(p["ks"]), up(p["vs"]),
                                             torch.empty(B, Hkv * G, d, device="cuda"), lengths=up(lengths),
                                             max_seq_len=cap))
    assert info.split_plan == kvq.SPLITS_SCHEDULE
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"B={B} G={G}")


@pytest.mark.parametrize("B", [63, 64, 65])
@pytest.mark.parametrize("append", [False, True])
def test_in_kernel_plan_limit(o, B, append):
    """Matrix-core kernel, Hkv = 4, G = 4: a ragged batch of up to 64
    sequences is planned inside the decode kernel (256 / 4 = 64 items per kv
    head, so B = 64 leaves one item per sequence); B = 65 goes back to the
    schedule launch.  Lengths include 0, 1 and the capacity."""
    rng = np.random.default_rng(B + 100 * append)
    Hkv, G, cap, d = 4, 4, 520, 128
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[:4] = [cap, 0, 1, 129]
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = vn = None
    if append:
        kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
        vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    got, gk, _, gks, _ = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, k_new=kn, v_new=vn)
    if append:
        o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=lengths - 1)
        assert np.array_equal(gk, p["k"]) and np.array_equal(_bits(gks), _bits(p["ks"]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"B={B} append={append}")


def test_in_kernel_plan_one_long_sequence(o):
    """A few sequences, one much longer: the in-kernel plan cuts the long one
    into many equal splits (more than one narrowing round of the chunk search)."""
    rng = np.random.default_rng(12)
    B, Hkv, G, cap, d = 6, 2, 8, 70000, 128
    lengths = np.array([70000, 3, 0, 640, 129, 5000], np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what="one long")


_LPT_CHILD = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
from _util import lpt_case
import _gpu
from _gpu import kvq, up
from oracle import oracle as orc
import torch
p = lpt_case(sys.argv[2], orc.get().quantize_rows)
B, Hq, d = p["q"].shape
info = kvq.decode_plan(kvq.decode_params(up(p["q"]), up(p["k"]), up(p["v"]), up(p["ks"]), up(p["vs"]),
                                         torch.empty(B, Hq, d, device="cuda"), lengths=up(p["lengths"]),
                                         max_seq_len=p["k"].shape[2], k_new=up(p["k_new"]), v_new=up(p["v_new"])))
outs = []
for rep in range(2):
    got, gk, gv, gks, gvs = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=p["lengths"],
                                         k_new=p["k_new"], v_new=p["v_new"])
    outs.append(got)
assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "repeat differs"
np.savez(sys.argv[3], out=outs[0], k=gk, v=gv, ks=gks, vs=gvs, plan=np.array([info.split_plan]))
print("child ok")
"""


@pytest.mark.parametrize("name", ["whole", "split", "cfg4_shape"])
def test_in_kernel_schedule_matches_schedule_launch(o, name, tmp_path):
    """Ragged matrix-core batches beyond one round of items (B > 512 / U): the
    decode kernel derives the longest-first schedule itself, with the same
    chunk and splits as the schedule launch (KVQ_SCHEDULE_LAUNCH=1, read once
    per process, hence child processes), so outputs and appended caches are
    bit-identical between the two; both match the oracle.  "whole": every
    sequence one item; "split": one long sequence cut into many chunks among
    short and empty ones."""
    import os
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = {}
    for flag in ("0", "1"):
        f = str(tmp_path / f"out_{flag}.npz")
        env = dict(os.environ, KVQ_SCHEDULE_LAUNCH=flag)
        r = subprocess.run([sys.executable, "-c", _LPT_CHILD, repo, name, f], env=env, capture_output=True,
                           text=True, timeout=110)
        assert r.returncode == 0 and "child ok" in r.stdout, (r.stdout + r.stderr)[-3000:]
        res[flag] = np.load(f)
    assert int(res["0"]["plan"][0]) == kvq.SPLITS_IN_KERNEL
    assert int(res["1"]["plan"][0]) == kvq.SPLITS_SCHEDULE
    for key in ("out", "k", "v", "ks", "vs"):
        assert res["0"][key].tobytes() == res["1"][key].tobytes(), key
    p = lpt_case(name, o.quantize_rows)
    o.append(p["k_new"], p["v_new"], p["k"], p["v"], p["ks"], p["vs"], positions=p["lengths"] - 1)
    assert np.array_equal(res["0"]["k"], p["k"]) and np.array_equal(res["0"]["v"], p["v"])
    assert np.array_equal(_bits(res["0"]["ks"]), _bits(p["ks"])) and np.array_equal(_bits(res["0"]["vs"]), _bits(p["vs"]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=p["lengths"])
    assert_close(res["0"]["out"], want, what=name)


@pytest.mark.parametrize("B,cap,Hkv,G", [(65, 1100, 8, 4), (256, 300, 8, 4), (512, 2048, 4, 16)])
def test_in_kernel_schedule_limits(o, B, cap, Hkv, G):
    """8 work units per sequence: the decode kernel derives the schedule from
    65 sequences (one round of 64 items per work unit exceeded) to 4 rounds
    of items below 2048 tokens of capacity (B = 256) and up to 512 sequences
    (two per thread, 8 rounds) from it; lengths 0, 1 and the capacity
    included, every sequence its own item or split."""
    rng = np.random.default_rng(B + 7)
    d = 64
    lengths = rng.integers(0, cap + 1, B).astype(np.int32)
    lengths[:4] = [cap, 0, 1, 33]
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    info = kvq.decode_plan(kvq.decode_params(up(p["q"]), up(p["k"]), up(p["v"]), up(p["ks"]), up(p["vs"]),
                                             torch.empty(B, Hkv * G, d, device="cuda"), lengths=up(lengths),
                                             max_seq_len=cap))
    assert (info.kernel, info.split_plan) == (kvq.KERNEL_DECODE_MFMA, kvq.SPLITS_IN_KERNEL)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"B={B}")
