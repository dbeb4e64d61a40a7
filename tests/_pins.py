"""Checks that pin the CPU oracle to the mathematics of the reference's path.

Each pin takes an oracle.Oracle (the real build or a planted-mistake build)
and returns a list of failure strings (empty = pin holds).  tests/test_oracle.py
asserts that the real oracle passes every pin and that every planted mistake
fails at least one, so a pin that cannot tell a plausible bug from the real
thing shows up as a failing test.

None of these retypes the oracle's formula: the attention pins compare against
a float64 textbook (scipy softmax + matrix products) or against closed forms,
and the quantiser pins are properties that determine round-to-nearest-even.
"""
from __future__ import annotations

import numpy as np

from _util import SEEDS, close_report, make_problem, selftest_inputs, textbook_decode_f64

# The fp32 oracle against the float64 textbook: fp32 rounding only.
TIGHT_ATOL = 2e-5
TIGHT_RTOL = 2e-4


def _q(oracle):
    return oracle.quantize_rows


def pin_textbook_mha(oracle):
    fails = []
    for seed in SEEDS:
        rng = np.random.default_rng(seed)
        p = make_problem(rng, 1, 8, 8, 1024, 64, _q(oracle))          # cfg0 shape
        got = oracle.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"])
        ref = textbook_decode_f64(p["q"], p["k"], p["v"], p["ks"], p["vs"])
        ok, msg = close_report(got, ref, TIGHT_ATOL, TIGHT_RTOL)
        if not ok:
            fails.append(f"textbook mha seed {seed}: {msg}")
        got64 = oracle.decode_f64(p["q"], p["k"], p["v"], p["ks"], p["vs"])
        ok, msg = close_report(got64, ref, 1e-12, 1e-10)
        if not ok:
            fails.append(f"textbook mha f64 seed {seed}: {msg}")
    return fails


def pin_textbook_gqa_ragged(oracle):
    fails = []
    for seed, dist in zip(SEEDS, ("normal", "student_t", "outlier")):
        rng = np.random.default_rng(seed)
        lengths = np.array([1, 77, 300, 129], np.int32)
        p = make_problem(rng, 4, 8, 2, 300, 128, _q(oracle), dist=dist, lengths=lengths)
        got = oracle.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
        ref = textbook_decode_f64(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
        ok, msg = close_report(got, ref, TIGHT_ATOL, TIGHT_RTOL)
        if not ok:
            fails.append(f"textbook gqa ragged {dist} seed {seed}: {msg}")
    return fails


def pin_selftest_kat(oracle):
    """The reference self-test's patterned inputs against the float64 textbook."""
    fails = []
    for (H, N, d) in ((4, 128, 64), (8, 1024, 64), (3, 257, 128)):
        Q, K, V, ks, vs = selftest_inputs(H, N, d)
        got = oracle.head_f32(Q, K, V, ks, vs)
        ref = textbook_decode_f64(Q[None], K[None], V[None], ks[None], vs[None])[0]
        ok, msg = close_report(got, ref, TIGHT_ATOL, TIGHT_RTOL)
        if not ok:
            fails.append(f"selftest KAT {(H, N, d)}: {msg}")
    return fails


def pin_closed_forms(oracle):
    fails = []
    rng = np.random.default_rng(5)
    d = 64
    # N = 1: the output is the single dequantised V row (prob is exactly 1).
    q = rng.standard_normal((3, d), dtype=np.float32)
    k = rng.integers(-127, 128, (3, 1, d), dtype=np.int8)
    v = rng.integers(-127, 128, (3, 1, d), dtype=np.int8)
    ks = rng.uniform(0.001, 0.05, (3, 1)).astype(np.float32)
    vs = rng.uniform(0.001, 0.05, (3, 1)).astype(np.float32)
    got = oracle.head_f32(q, k, v, ks, vs)
    want = v[:, 0, :].astype(np.float32) * vs
    if not np.array_equal(got, want):
        fails.append("N=1 output is not the dequantised V row")
    # K = 0: all scores equal, output is the mean of dequantised V rows.
    N = 50
    k0 = np.zeros((3, N, d), np.int8)
    v = rng.integers(-127, 128, (3, N, d), dtype=np.int8)
    ks = rng.uniform(0.001, 0.05, (3, N)).astype(np.float32)
    vs = rng.uniform(0.001, 0.05, (3, N)).astype(np.float32)
    got = oracle.head_f32(q, k0, v, ks, vs)
    want = (v.astype(np.float64) * vs[..., None]).mean(axis=1)
    ok, msg = close_report(got, want, 1e-6, 1e-5)
    if not ok:
        fails.append(f"K=0 mean: {msg}")
    # Constant V rows: the output equals that row whatever the weights.
    row = rng.integers(-127, 128, (3, 1, d), dtype=np.int8)
    vc = np.repeat(row, N, axis=1)
    vsc = np.full((3, N), 0.02, np.float32)
    k = rng.integers(-127, 128, (3, N, d), dtype=np.int8)
    got = oracle.head_f32(q, k, vc, ks, vsc)
    want = row[:, 0, :].astype(np.float64) * 0.02
    ok, msg = close_report(got, want, 1e-6, 1e-5)
    if not ok:
        fails.append(f"constant V: {msg}")
    # One dominating score: K row 7 aligned with q and huge; output -> V row 7.
    qd = np.ones((1, d), np.float32)
    kd = np.zeros((1, N, d), np.int8)
    kd[0, 7, :] = 127
    ksd = np.full((1, N), 1.0, np.float32)
    vd = rng.integers(-127, 128, (1, N, d), dtype=np.int8)
    vsd = np.full((1, N), 0.01, np.float32)
    got = oracle.head_f32(qd, kd, vd, ksd, vsd)
    want = vd[0, 7].astype(np.float64) * 0.01
    ok, msg = close_report(got[0], want, 1e-6, 1e-6)
    if not ok:
        fails.append(f"dominating score: {msg}")
    # Token permutation invariance and convexity (output inside per-dim range).
    k = rng.integers(-127, 128, (2, N, d), dtype=np.int8)
    v = rng.integers(-127, 128, (2, N, d), dtype=np.int8)
    ks = rng.uniform(0.001, 0.05, (2, N)).astype(np.float32)
    vs = rng.uniform(0.001, 0.05, (2, N)).astype(np.float32)
    q2 = q[:2]
    base = oracle.head_f32(q2, k, v, ks, vs)
    perm = rng.permutation(N)
    permd = oracle.head_f32(q2, k[:, perm], v[:, perm], ks[:, perm], vs[:, perm])
    ok, msg = close_report(permd, base, 1e-6, 1e-5)
    if not ok:
        fails.append(f"permutation: {msg}")
    deq = v.astype(np.float64) * vs[..., None]
    lo, hi = deq.min(axis=1) - 1e-6, deq.max(axis=1) + 1e-6
    if not (np.all(base >= lo) and np.all(base <= hi)):
        fails.append("output outside the convex hull of dequantised V")
    return fails


def pin_gqa_equals_replicated(oracle):
    """GQA over Hkv heads == MHA over KV heads replicated g times (bit-exact)."""
    fails = []
    rng = np.random.default_rng(11)
    B, Hq, Hkv, cap, d = 2, 8, 2, 40, 64
    p = make_problem(rng, B, Hq, Hkv, cap, d, _q(oracle))
    g = Hq // Hkv
    rep = lambda a: np.repeat(a, g, axis=1)
    got = oracle.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"])
    want = oracle.decode_f32(p["q"], rep(p["k"]), rep(p["v"]), rep(p["ks"]), rep(p["vs"]))
    if not np.array_equal(got, want):
        fails.append("GQA differs from replicated MHA")
    return fails


def pin_ragged_equals_truncated(oracle):
    """lengths[b] == running the uniform path on the first lengths[b] tokens."""
    fails = []
    rng = np.random.default_rng(12)
    B, Hq, Hkv, cap, d = 3, 4, 4, 64, 32
    p = make_problem(rng, B, Hq, Hkv, cap, d, _q(oracle))
    lengths = np.array([64, 1, 33], np.int32)
    got = oracle.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    for b in range(B):
        L = int(lengths[b])
        sl = lambda a: np.ascontiguousarray(a[b:b + 1, :, :L])
        want = oracle.decode_f32(p["q"][b:b + 1], sl(p["k"]), sl(p["v"]), sl(p["ks"]), sl(p["vs"]))
        if not np.array_equal(got[b:b + 1], want):
            fails.append(f"ragged b={b} L={L} differs from truncated")
    return fails


# ---------------------------------------------------------------------------
# quantiser: properties that fix round-to-nearest-even per-row quantisation
# ---------------------------------------------------------------------------
def quant_rows_for_pins():
    rng = np.random.default_rng(23)
    rows = [rng.standard_normal((64, 128), dtype=np.float32),
            (rng.standard_t(4, (64, 128))).astype(np.float32),
            rng.standard_normal((32, 64), dtype=np.float32).repeat(2, axis=1) * np.float32(1e-30),
            # scales in the fp32 subnormal range
            rng.standard_normal((16, 64), dtype=np.float32) * np.float32(1e-38)]
    out = []
    for r in rows:
        out.extend(list(r))
    return out


def pin_quantizer_properties(oracle):
    fails = []
    for x in quant_rows_for_pins():
        x = x.astype(np.float32)
        q, s = oracle.quantize_rows(x[None])
        q, s = q[0], s[0]
        amax = np.float32(np.max(np.abs(x)))
        if s != np.float32(amax / np.float32(127.0)):
            fails.append("scale != amax/127 (IEEE fp32)")
            break
        if np.any(np.abs(q.astype(np.int32)) > 127):
            fails.append("|q| > 127")
            break
        if s > 0:
            r = x.astype(np.float64) / np.float64(s)
            # round-to-nearest: the integer is within half a step of x/scale
            # (x/scale itself is rounded once to fp32, hence the 1e-5 slack)
            if np.any(np.abs(r - q) > 0.5 + 1e-5):
                fails.append("round-to-nearest violated")
                break
            i = int(np.argmax(np.abs(x)))
            if abs(int(q[i])) != 127:
                fails.append("max element does not map to +-127")
                break
    # Exact ties: amax = 127 gives scale = 1.0 exactly, so x/scale = x.
    x = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -3.5, 4.5], np.float32)
    q, s = oracle.quantize_rows(x[None])
    if s[0] != np.float32(1.0) or list(q[0]) != [127, 0, 2, 2, 0, -2, -2, 126, -4, 4]:
        fails.append(f"ties-to-even: got {list(q[0])} scale {s[0]}")
    # amax carried by a negative element at the last index.
    x = np.array([1.0, -2.0, 3.0, -254.0], np.float32)
    q, s = oracle.quantize_rows(x[None])
    if s[0] != np.float32(2.0) or list(q[0]) != [0, -1, 2, -127]:
        fails.append(f"negative amax: got {list(q[0])} scale {s[0]}")
    # Zero row.
    q, s = oracle.quantize_rows(np.zeros((1, 16), np.float32))
    if s[0] != 0 or np.any(q != 0):
        fails.append("zero row")
    # amax so small that amax/127 underflows to 0: defined as the zero row.
    x = np.array([1e-44, -2e-44, 0.0, 5e-45], np.float32)
    q, s = oracle.quantize_rows(x[None])
    if s[0] != 0 or np.any(q != 0):
        fails.append(f"underflowing scale: got {list(q[0])} scale {s[0]}")
    return fails


def pin_append(oracle):
    """append writes quantise_rows(new) at positions[b] and touches nothing else."""
    fails = []
    rng = np.random.default_rng(31)
    B, Hkv, cap, d = 3, 2, 8, 16
    k = rng.integers(-127, 128, (B, Hkv, cap, d), dtype=np.int8)
    v = rng.integers(-127, 128, (B, Hkv, cap, d), dtype=np.int8)
    ks = rng.uniform(0.01, 0.1, (B, Hkv, cap)).astype(np.float32)
    vs = rng.uniform(0.01, 0.1, (B, Hkv, cap)).astype(np.float32)
    kn = rng.standard_normal((B, Hkv, d), dtype=np.float32)
    vn = rng.standard_normal((B, Hkv, d), dtype=np.float32)
    pos = np.array([0, 7, 3], np.int32)
    k2, v2, ks2, vs2 = k.copy(), v.copy(), ks.copy(), vs.copy()
    oracle.append(kn, vn, k2, v2, ks2, vs2, positions=pos)
    qk, sk = oracle.quantize_rows(kn)
    qv, sv = oracle.quantize_rows(vn)
    for b in range(B):
        p = pos[b]
        if not (np.array_equal(k2[b, :, p], qk[b]) and np.array_equal(v2[b, :, p], qv[b])
                and np.array_equal(ks2[b, :, p], sk[b]) and np.array_equal(vs2[b, :, p], sv[b])):
            fails.append(f"append b={b} wrong token")
        mask = np.ones(cap, bool)
        mask[p] = False
        if not (np.array_equal(k2[b][:, mask], k[b][:, mask]) and np.array_equal(ks2[b][:, mask], ks[b][:, mask])):
            fails.append(f"append b={b} touched other tokens")
    return fails


def textbook_attention_f64(Q, K, V):
    """softmax(Q K^T / sqrt(d)) V in float64 with scipy's softmax."""
    from scipy.special import softmax
    Q, K, V = (np.asarray(x, np.float64) for x in (Q, K, V))
    return softmax(Q @ K.T / np.sqrt(Q.shape[1]), axis=1) @ V


def pin_attention_textbook(oracle):
    """Dense fp32 attention (attention/softmax_new.cu) against the float64
    textbook on random and heavy-tailed data, several shapes."""
    fails = []
    for seed, (M, N, d) in zip(SEEDS, ((7, 300, 64), (33, 129, 128), (5, 1000, 96))):
        rng = np.random.default_rng(seed)
        Q = rng.standard_normal((M, d)).astype(np.float32)
        K = (rng.standard_t(4, (N, d)) * 0.7).astype(np.float32)
        V = rng.standard_normal((N, d)).astype(np.float32)
        got = oracle.attention_f32(Q, K, V)
        ok, msg = close_report(got, textbook_attention_f64(Q, K, V), TIGHT_ATOL, TIGHT_RTOL)
        if not ok:
            fails.append(f"attention textbook {(M, N, d)}: {msg}")
    return fails


def pin_attention_closed_forms(oracle):
    fails = []
    rng = np.random.default_rng(8)
    M, N, d = 4, 60, 32
    Q = rng.standard_normal((M, d)).astype(np.float32)
    V = rng.standard_normal((N, d)).astype(np.float32)
    # N = 1: every output row is the V row.
    got = oracle.attention_f32(Q, rng.standard_normal((1, d)).astype(np.float32), V[:1])
    if not np.array_equal(got, np.repeat(V[:1], M, axis=0)):
        fails.append("attention N=1 is not the V row")
    # K = 0: uniform weights, the mean of V.
    got = oracle.attention_f32(Q, np.zeros((N, d), np.float32), V)
    ok, msg = close_report(got, np.repeat(V.astype(np.float64).mean(0, keepdims=True), M, 0), 1e-6, 1e-5)
    if not ok:
        fails.append(f"attention K=0 mean: {msg}")
    # One dominating key: output -> that V row.
    K = np.zeros((N, d), np.float32)
    K[11] = 40.0
    got = oracle.attention_f32(np.abs(Q) + 1.0, K, V)
    ok, msg = close_report(got, np.repeat(V[11:12].astype(np.float64), M, 0), 1e-6, 1e-6)
    if not ok:
        fails.append(f"attention dominating key: {msg}")
    # Key permutation invariance.
    K = rng.standard_normal((N, d)).astype(np.float32)
    perm = rng.permutation(N)
    ok, msg = close_report(oracle.attention_f32(Q, K[perm], V[perm]), oracle.attention_f32(Q, K, V), 1e-6, 1e-5)
    if not ok:
        fails.append(f"attention permutation: {msg}")
    return fails


ALL_PINS = (pin_textbook_mha, pin_textbook_gqa_ragged, pin_selftest_kat, pin_closed_forms,
            pin_gqa_equals_replicated, pin_ragged_equals_truncated, pin_quantizer_properties,
            pin_append, pin_attention_textbook, pin_attention_closed_forms)


def run_all(oracle):
    fails = []
    for pin in ALL_PINS:
        fails.extend(f"{pin.__name__}: {f}" for f in pin(oracle))
    return fails
