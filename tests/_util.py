"""Shared helpers for the test suite: data generators, an independent float64
textbook reference, and the parity checker.

Nothing here is product code.  The float64 textbook reference is written from
the mathematics of softmax attention (scipy.special.softmax + matrix products),
not from the oracle, so it can pin the oracle.
"""
from __future__ import annotations

import os
import sys

import numpy as np
from scipy.special import softmax

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

# Parity bar for the HIP path against the fp32 oracle (task tolerance).
ATOL = 1e-4
RTOL = 1e-3

SEEDS = (17, 29, 101)


# ---------------------------------------------------------------------------
# checker
# ---------------------------------------------------------------------------
def close_report(got, ref, atol=ATOL, rtol=RTOL):
    """Elementwise |got-ref| <= atol + rtol*|ref|, rejecting NaN/Inf in got.

    Same form as the reference's scan harness gate
    (benchmarks/selective_scan/bench.cpp:29-41).  Returns (ok, message)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if got.shape != ref.shape:
        return False, f"shape {got.shape} != {ref.shape}"
    if not np.all(np.isfinite(got)):
        bad = np.argwhere(~np.isfinite(got))[0]
        return False, f"non-finite output at {tuple(bad)}: {got[tuple(bad)]}"
    if not np.all(np.isfinite(ref)):
        return False, "non-finite reference"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    ok = bool(np.all(err <= bound))
    if err.size == 0:
        return True, "empty"
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    msg = (f"max_abs_err={err.max():.3e} worst@{tuple(int(i) for i in worst)} "
           f"got={got[worst]:.8g} ref={ref[worst]:.8g} bound={bound[worst]:.3e}")
    return ok, msg


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    ok, msg = close_report(got, ref, atol, rtol)
    assert ok, f"{what}: {msg}"


# ---------------------------------------------------------------------------
# the reference self-test's patterned inputs (kv_cache/KV_int8_split_optimized.cu:473-486)
# ---------------------------------------------------------------------------
def selftest_inputs(H, N, d):
    i = np.arange(H * d, dtype=np.int64)
    Q = ((i % 17) - 8).astype(np.float32) * np.float32(0.125)
    j = np.arange(H * N * d, dtype=np.int64)
    K = ((j % 23) - 11).astype(np.int8)
    V = (((j * 3) % 29) - 14).astype(np.int8)
    s = np.arange(H * N, dtype=np.int64)
    ks = np.float32(0.015625) + (s % 5).astype(np.float32) * np.float32(0.001)
    vs = np.float32(0.03125) + (s % 7).astype(np.float32) * np.float32(0.001)
    return (Q.reshape(H, d), K.reshape(H, N, d), V.reshape(H, N, d),
            ks.astype(np.float32).reshape(H, N), vs.astype(np.float32).reshape(H, N))


# ---------------------------------------------------------------------------
# independent float64 textbook reference
# ---------------------------------------------------------------------------
def textbook_decode_f64(q, k, v, ks, vs, lengths=None, uniform_len=None):
    """softmax(q . dequant(K)^T / sqrt(d)) @ dequant(V), float64, per (b, hq).

    q[B,Hq,d], k/v[B,Hkv,cap,d] int8, ks/vs[B,Hkv,cap]; query head hq reads
    kv head hq // (Hq // Hkv) over the first lengths[b] tokens."""
    q = np.asarray(q, np.float64)
    B, Hq, d = q.shape
    _, Hkv, cap, _ = k.shape
    g = Hq // Hkv
    out = np.zeros((B, Hq, d), np.float64)
    for b in range(B):
        L = int(lengths[b]) if lengths is not None else int(uniform_len if uniform_len else cap)
        L = min(L, cap)
        if L <= 0:
            continue
        for h in range(Hkv):
            Kd = k[b, h, :L].astype(np.float64) * ks[b, h, :L, None].astype(np.float64)
            Vd = v[b, h, :L].astype(np.float64) * vs[b, h, :L, None].astype(np.float64)
            Qg = q[b, h * g:(h + 1) * g]
            P = softmax(Qg @ Kd.T / np.sqrt(d), axis=-1)
            out[b, h * g:(h + 1) * g] = P @ Vd
    return out


# ---------------------------------------------------------------------------
# synthetic data (numpy, seeded) for CPU-side tests
# ---------------------------------------------------------------------------
def normal(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32)


def student_t4(rng, shape):
    z = rng.standard_normal(shape, dtype=np.float32)
    chi = np.zeros(shape, np.float32)
    for _ in range(4):
        chi += rng.standard_normal(shape, dtype=np.float32) ** 2
    return (z / np.sqrt(chi / np.float32(4.0))).astype(np.float32)


def outlier_k(rng, shape, frac=0.01, factor=20.0):
    """N(0,1) K with ceil(frac*d) seeded outlier channels per kv head scaled by factor."""
    x = rng.standard_normal(shape, dtype=np.float32)
    B, H, L, d = shape
    n_out = max(1, int(np.ceil(frac * d)))
    for b in range(B):
        for h in range(H):
            ch = rng.choice(d, n_out, replace=False)
            x[b, h, :, ch] *= np.float32(factor)
    return x


def make_problem(rng, B, Hq, Hkv, cap, d, quantize, dist="normal", lengths=None):
    """Random q plus a quantised cache; `quantize` maps fp32 rows -> (int8, scale)."""
    q = normal(rng, (B, Hq, d))
    if dist == "normal":
        kf, vf = normal(rng, (B, Hkv, cap, d)), normal(rng, (B, Hkv, cap, d))
    elif dist == "student_t":
        kf, vf = student_t4(rng, (B, Hkv, cap, d)), student_t4(rng, (B, Hkv, cap, d))
    elif dist == "outlier":
        kf, vf = outlier_k(rng, (B, Hkv, cap, d)), normal(rng, (B, Hkv, cap, d))
    else:
        raise ValueError(dist)
    k, ks = quantize(kf)
    v, vs = quantize(vf)
    return dict(q=q, k=k, v=v, ks=ks, vs=vs, lengths=lengths)


# ---------------------------------------------------------------------------
# ragged batches for the matrix-core kernel's in-kernel split schedule
# ---------------------------------------------------------------------------
LPT_CASES = {
    # B, Hq, Hkv, d, cap: 8 work units per sequence, so more than 512 / 8 = 64
    # sequences take longest-first rounds.  "whole": lengths in [cap/2, cap],
    # every sequence one item; "split": one sequence of cap tokens among short
    # ones (and an empty one), cut into many chunks.
    "whole": (100, 32, 8, 64, 1024),
    "split": (80, 64, 4, 64, 4096),
    "cfg4_shape": (65, 64, 8, 128, 1024),
}


def lpt_case(name, quantize):
    """Seeded problem (dict of make_problem plus k_new / v_new) for LPT_CASES[name]."""
    B, Hq, Hkv, d, cap = LPT_CASES[name]
    rng = np.random.default_rng(sum(map(ord, name)))
    if name == "split":
        lengths = rng.integers(1, 100, B).astype(np.int32)
        lengths[:3] = [cap, 0, 1]
    else:
        lengths = rng.integers(cap // 2, cap + 1, B).astype(np.int32)
        lengths[:2] = [cap, cap // 2]
    p = make_problem(rng, B, Hq, Hkv, cap, d, quantize, dist="student_t", lengths=lengths)
    p["k_new"] = student_t4(rng, (B, Hkv, d))
    p["v_new"] = student_t4(rng, (B, Hkv, d))
    return p
