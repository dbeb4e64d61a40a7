"""Batched / GQA / ragged / split / fused-append decode on the GPU through
kvq_decode_launch, against the CPU oracle.

The extension has no reference counterpart; its parity is defined by
reduction to the reference math: out[b, hq] = cpu_reference(Q[b, hq],
K[b, hq / g, :len_b], ...) (oracle kvq_ref_decode_f32).  Tolerance: 1e-4 abs +
1e-3 rel elementwise.  Appended int8 values and scales: bit-exact.
"""
import importlib

import numpy as np
import pytest
import torch

from _util import SEEDS, assert_close, make_problem
import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
synth = importlib.import_module("cuda-operators_amd.synth")


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _host(p):
    h = lambda t: None if t is None else down(t)
    return dict(q=h(p.q), k=h(p.k), v=h(p.v), ks=h(p.ks), vs=h(p.vs), k_new=h(p.k_new), v_new=h(p.v_new),
                lengths=p.lengths_host.astype(np.int32))


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _check_config(o, name, seed, scale_len=1.0, splits=0, f64=False):
    p = synth.make(name, seed=seed, scale_len=scale_len)
    h = _host(p)
    out = torch.full(p.q.shape, float("nan"), device=_gpu.dev())
    dec = kvq.Decoder(p.q, p.k, p.v, p.ks, p.vs, out, lengths=p.lengths,
                      max_seq_len=p.max_len if p.lengths is not None else p.cap,
                      num_splits=splits, k_new=p.k_new, v_new=p.v_new)
    dec()
    torch.cuda.synchronize()
    got = down(out)
    if h["k_new"] is not None:
        o.append(h["k_new"], h["v_new"], h["k"], h["v"], h["ks"], h["vs"], positions=h["lengths"] - 1)
        assert np.array_equal(down(p.k), h["k"]) and np.array_equal(down(p.v), h["v"]), "appended int8 differs"
        assert np.array_equal(_bits(down(p.ks)), _bits(h["ks"])), "appended k scale differs"
        assert np.array_equal(_bits(down(p.vs)), _bits(h["vs"])), "appended v scale differs"
    want = o.decode_f32(h["q"], h["k"], h["v"], h["ks"], h["vs"], lengths=h["lengths"])
    assert_close(got, want, what=f"{name} seed {seed} splits {splits}")
    if f64:
        # The float64 oracle as the yardstick for both: the GPU's error may
        # not exceed twice the fp32 oracle's own (sequential fp32 sums).
        w64 = o.decode_f64(h["q"], h["k"], h["v"], h["ks"], h["vs"], lengths=h["lengths"])
        gpu_err = float(np.abs(got.astype(np.float64) - w64).max())
        ref_err = float(np.abs(want.astype(np.float64) - w64).max())
        assert gpu_err <= 2.0 * ref_err, f"{name}: |GPU - f64| {gpu_err:.3e} > 2 x |oracle f32 - f64| {ref_err:.3e}"
    return dec


@pytest.mark.parametrize("seed", SEEDS)
@pytest.mark.parametrize("name", ["cfg0", "cfg1", "cfg2", "cfg3", "cfg4"])
def test_config_small(o, name, seed):
    """Every config's shape family at reduced lengths (all seeds)."""
    _check_config(o, name, seed, scale_len=1 / 16)


@pytest.mark.parametrize("name", ["cfg0", "cfg1", "cfg2", "cfg3", "cfg4"])
def test_config_full_size(o, name):
    """Every config at its full BASELINE size (seed 17)."""
    _check_config(o, name, 17)


@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg4"])
def test_config_full_size_against_f64(o, name):
    """The grouped-query configs (matrix-core kernel: q as int8 limbs, PV
    weights as f16 hi/lo pairs) at full size against the float64 oracle: the
    GPU's largest error is at most twice the fp32 oracle's, so an accuracy
    loss in the matrix-core path shows up inside the 1e-4 + 1e-3 band."""
    _check_config(o, name, 17, f64=True)


@pytest.mark.parametrize("seed", [29, 101])
@pytest.mark.parametrize("name", ["cfg2", "cfg4"])
def test_ragged_config_full_size_other_seeds(o, name, seed):
    """The ragged configs at full size with the other seeds' lengths: other
    tile-stream ranges and sequence switches for cfg2's flattened plan, other
    schedules for cfg4."""
    _check_config(o, name, seed)


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16, 64, 1000])
def test_split_counts_agree(o, splits):
    """Split + log-sum-exp merge == unsplit, for every split count (incl. more splits than tiles)."""
    rng = np.random.default_rng(splits)
    lengths = np.array([2000, 1, 1999, 777], np.int32)
    p = make_problem(rng, 4, 8, 2, 2000, 128, o.quantize_rows, dist="outlier", lengths=lengths)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, splits=splits)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"splits={splits}")


@pytest.mark.parametrize("splits,L", [(17, 2100), (24, 3000), (31, 3900), (32, 4000)])
def test_merge_of_17_to_32_splits(o, splits, L):
    """17..32 splits: the last split's workgroup merges with two lanes per output
    column (splits of one parity each), every sequence length split differently."""
    rng = np.random.default_rng(splits + L)
    lengths = np.array([L, 1, L - 1, (2 * L) // 5], np.int32)
    p = make_problem(rng, 4, 8, 2, L, 128, o.quantize_rows, dist="outlier", lengths=lengths)
    prm = kvq.DecodeParams(batch=4, num_q_heads=8, num_kv_heads=2, head_dim=128, capacity=L, max_seq_len=L,
                           lengths=4096, q=4096, k_cache=4096, v_cache=4096, k_scale=4096, v_scale=4096,
                           out=4096, num_splits=splits)
    info = kvq.decode_plan(prm)
    assert (info.kernel, info.splits) == (kvq.KERNEL_DECODE_MFMA, splits)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, splits=splits)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"splits={splits} L={L}")


@pytest.mark.parametrize("splits", [33, 48, 100, 257])
def test_merge_past_32_splits(o, splits):
    """More than 32 splits: the last split's workgroup merges with the
    two-phase group merge ((m, l) pairs into LDS, then the accumulators, 16
    in flight per thread), every sequence length split differently; 257
    splits is past that merge's limit of 256 and takes the per-element merge."""
    L = splits * 128 - 28
    rng = np.random.default_rng(splits)
    lengths = np.array([L, 1, L - 1, (2 * L) // 5], np.int32)
    p = make_problem(rng, 4, 8, 2, L, 128, o.quantize_rows, dist="outlier", lengths=lengths)
    prm = kvq.DecodeParams(batch=4, num_q_heads=8, num_kv_heads=2, head_dim=128, capacity=L, max_seq_len=L,
                           lengths=4096, q=4096, k_cache=4096, v_cache=4096, k_scale=4096, v_scale=4096,
                           out=4096, num_splits=splits)
    info = kvq.decode_plan(prm)
    assert info.kernel == kvq.KERNEL_DECODE_MFMA and info.splits > 32, (info.kernel, info.splits)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, splits=splits)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"splits={splits} L={L}")


@pytest.mark.parametrize("G", [1, 2, 3, 4, 6, 8, 12, 16])
@pytest.mark.parametrize("d", [64, 128])
def test_group_sizes(o, G, d):
    """Query heads per kv head: 1 (MHA) .. 16, incl. groups the kernel tiles as 4+4 or 1+1+1."""
    rng = np.random.default_rng(G * 10 + d)
    Hkv = 2
    lengths = np.array([513, 64], np.int32)
    p = make_problem(rng, 2, Hkv * G, Hkv, 600, d, o.quantize_rows, lengths=lengths)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, max_seq_len=600)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"G={G} d={d}")


def test_gqa_equals_replicated_mha(o):
    """GQA over Hkv heads gives the same numbers as MHA over replicated kv heads."""
    rng = np.random.default_rng(7)
    p = make_problem(rng, 2, 16, 4, 900, 128, o.quantize_rows)
    rep = lambda a: np.repeat(a, 4, axis=1)
    a = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"])[0]
    b = _gpu.decode(p["q"], rep(p["k"]), rep(p["v"]), rep(p["ks"]), rep(p["vs"]))[0]
    assert_close(a, b, atol=1e-6, rtol=1e-5, what="gqa vs replicated")


def test_ragged_edges(o):
    """Length 0 (zero row), 1, capacity, and lengths above capacity (clamped)."""
    rng = np.random.default_rng(3)
    cap = 300
    lengths = np.array([0, 1, cap, 150, cap + 50], np.int32)
    p = make_problem(rng, 5, 4, 4, cap, 64, o.quantize_rows)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, max_seq_len=cap)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=np.minimum(lengths, cap))
    assert np.all(got[0] == 0.0)
    assert_close(got, want, what="ragged edges")


def test_softmax_scale_override(o):
    rng = np.random.default_rng(4)
    p = make_problem(rng, 1, 4, 4, 200, 64, o.quantize_rows)
    s = 0.5
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], softmax_scale=s)[0]
    # scaling q by s*sqrt(d) turns the default 1/sqrt(d) into s
    want = o.decode_f32(p["q"] * np.float32(s * np.sqrt(64.0)), p["k"], p["v"], p["ks"], p["vs"])
    assert_close(got, want, what="softmax_scale")


@pytest.mark.parametrize("d,G", [(64, 2), (128, 2), (256, 2), (96, 2), (128, 4), (128, 8), (128, 16), (64, 4),
                                 (64, 8)])
def test_fused_append_matches_separate_append(o, d, G):
    """Fused append inside the decode kernel == kvq_append_launch followed by decode:
    bit-for-bit in the cache; the outputs agree to fp32 rounding (the new token
    enters the online softmax at a different point of the summation order)."""
    rng = np.random.default_rng(d + G)
    B, Hkv, cap = 3, 2, 700
    Hq = Hkv * G
    lengths = np.array([700, 1, 389], np.int32)
    p = make_problem(rng, B, Hq, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = rng.standard_normal((B, Hkv, d), dtype=np.float32) * np.float32(3)
    vn = rng.standard_normal((B, Hkv, d), dtype=np.float32)
    fused = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, k_new=kn, v_new=vn)
    gk, gv, gks, gvs = up(p["k"]), up(p["v"]), up(p["ks"]), up(p["vs"])
    kvq.append(up(kn), up(vn), gk, gv, gks, gvs, positions=up(lengths - 1))
    torch.cuda.synchronize()
    sep = _gpu.decode(p["q"], down(gk), down(gv), down(gks), down(gvs), lengths=lengths)
    for name, a, b in zip(("k", "v", "ks", "vs"), fused[1:], (down(gk), down(gv), down(gks), down(gvs))):
        assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8)), name
    assert_close(fused[0], sep[0], atol=1e-6, rtol=1e-5, what="fused vs separate output")
    # and both equal the oracle
    o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=lengths - 1)
    assert np.array_equal(fused[1], p["k"]) and np.array_equal(_bits(fused[3]), _bits(p["ks"]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(fused[0], want, what=f"fused append d={d} G={G}")


def test_misaligned_pointers_use_generic_path(o):
    """Caches not 16-byte aligned still decode correctly (generic kernel)."""
    rng = np.random.default_rng(8)
    B, Hq, Hkv, cap, d = 2, 4, 2, 257, 128
    p = make_problem(rng, B, Hq, Hkv, cap, d, o.quantize_rows)
    n = B * Hkv * cap * d
    kbuf = torch.zeros(n + 1, dtype=torch.int8, device=_gpu.dev())
    vbuf = torch.zeros(n + 1, dtype=torch.int8, device=_gpu.dev())
    k = kbuf[1:].view(B, Hkv, cap, d)
    v = vbuf[1:].view(B, Hkv, cap, d)
    k.copy_(up(p["k"]))
    v.copy_(up(p["v"]))
    out = torch.empty((B, Hq, d), device=_gpu.dev())
    gq, gks, gvs = up(p["q"]), up(p["ks"]), up(p["vs"])  # keep alive across the launch
    params = kvq.decode_params(gq, k, v, gks, gvs, out, max_seq_len=cap)
    ws = kvq.new_workspace(params)
    kvq.decode_launch(params, ws)
    torch.cuda.synchronize()
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"])
    assert_close(down(out), want, what="misaligned")


def test_workspace_left_zeroed_and_reusable(o):
    """Arrival counters return to zero after each launch, so a workspace is reusable."""
    rng = np.random.default_rng(9)
    p = make_problem(rng, 2, 8, 2, 3000, 128, o.quantize_rows)
    g = [up(p[k]) for k in ("q", "k", "v", "ks", "vs")]
    out = torch.empty((2, 8, 128), device=_gpu.dev())
    dec = kvq.Decoder(*g, out, max_seq_len=3000, num_splits=6)
    assert dec.ws_bytes > 0
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"])
    for _ in range(3):
        out.fill_(float("nan"))
        dec()
        torch.cuda.synchronize()
        assert_close(down(out), want, what="reuse")
        counters = down(dec.ws[:64].view(torch.int32))
        assert not counters.any(), counters


def test_side_stream(o):
    rng = np.random.default_rng(10)
    p = make_problem(rng, 3, 8, 8, 1500, 64, o.quantize_rows)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], stream=s)[0]
    assert_close(got, o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"]), what="side stream")


@pytest.mark.parametrize("splits", [1, 3, 8])
@pytest.mark.parametrize("G", [4, 8])
@pytest.mark.parametrize("d", [64, 128])
def test_mfma_splits_with_fused_append(o, d, G, splits):
    """Grouped-query (matrix-core) path: fused append in the last split, split merge."""
    rng = np.random.default_rng(100 * G + splits + d)
    B, Hkv, cap = 3, 2, 1500
    lengths = np.array([1500, 33, 1025], np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, dist="student_t", lengths=lengths)
    kn = rng.standard_t(4, (B, Hkv, d)).astype(np.float32)
    vn = rng.standard_t(4, (B, Hkv, d)).astype(np.float32)
    got, gk, gv, gks, gvs = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, splits=splits,
                                         k_new=kn, v_new=vn)
    o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=lengths - 1)
    assert np.array_equal(gk, p["k"]) and np.array_equal(gv, p["v"])
    assert np.array_equal(_bits(gks), _bits(p["ks"])) and np.array_equal(_bits(gvs), _bits(p["vs"]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"mfma d={d} G={G} splits={splits}")


@pytest.mark.parametrize("d", [64, 128])
def test_mfma_extreme_scales(o, d):
    """Tiny, huge and zero per-token scales and a large |q| on the matrix-core path."""
    rng = np.random.default_rng(77 + d)
    B, Hkv, G, cap = 1, 2, 8, 300
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows)
    p["vs"][0, 0, :50] = np.float32(1e-30)
    p["vs"][0, 0, 50:60] = np.float32(0.0)
    p["vs"][0, 1, :40] = np.float32(3e4)
    p["ks"][0, 1, 100:120] = np.float32(1e-6)
    p["q"][0, 3] *= np.float32(50.0)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"])[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"])
    assert_close(got, want, what="mfma extreme scales")


@pytest.mark.parametrize("splits", [1, 5])
@pytest.mark.parametrize("d", [64, 128])
def test_mfma_ignores_slots_past_length(o, d, splits):
    """Cache slots past each sequence's length hold NaN/Inf scales and the last
    tile of a wave reaches into them (and past the capacity): they must get no
    weight.  Also negative v scales, which the weight normalisation takes by
    magnitude."""
    rng = np.random.default_rng(31 + splits + d)
    B, Hkv, G, cap = 4, 2, 4, 1028
    lengths = np.array([1028, 1, 161, 700], np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    for b, n in enumerate(lengths):
        p["ks"][b, :, n:] = np.float32(np.nan)
        p["vs"][b, :, n:] = np.float32(np.inf)
    p["vs"][2, 1, :100] *= np.float32(-1.0)
    got = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, splits=splits)[0]
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert np.isfinite(got).all()
    assert_close(got, want, what=f"mfma slots past length, splits {splits}")
