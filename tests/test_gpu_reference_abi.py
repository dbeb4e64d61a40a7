"""The reference ABI on the GPU: solve, kv_int8_split_launch, kv_int8_simple_launch
against the CPU oracle (restated cpu_reference, kv_cache/KV_int8_split_optimized.cu:385-437).

Tolerance: 1e-4 abs + 1e-3 rel elementwise (task bar), plus the reference
self-test's own gate (max-abs <= 1e-4, KV_int8_split_optimized.cu:535) on its
patterned inputs.  Outputs are poisoned with NaN before every call.
"""
import os

import numpy as np
import pytest
import torch

from _util import ATOL, RTOL, SEEDS, assert_close, selftest_inputs
import _gpu
from _gpu import down, kvq, poisoned, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KAT_SHAPES = ((4, 128, 64), (8, 1024, 64), (3, 257, 128))


def _run(entry, Q, K, V, ks, vs, stream=None, scratch_fill=float("nan")):
    H, N, d = K.shape
    gQ, gK, gV, gks, gvs = up(Q), up(K), up(V), up(ks), up(vs)
    out = poisoned((H, d))
    if entry == "solve":
        kvq.solve(gQ, gK, gV, gks, gvs, out)
    else:
        S = torch.full((H * N,), scratch_fill, dtype=torch.float32, device=_gpu.dev())
        rc = kvq.kv_int8_split_launch(gQ, gK, gV, gks, gvs, out, S, stream=stream, simple=(entry == "simple"))
        assert rc == 0, f"{entry} returned {rc}"
    torch.cuda.synchronize()
    return down(out)


@pytest.mark.parametrize("entry", ["solve", "split", "simple"])
@pytest.mark.parametrize("shape", KAT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_selftest_kat(entry, shape):
    H, N, d = shape
    g = np.load(os.path.join(GOLD, "kat_selftest.npz"), allow_pickle=False)
    Q, K, V, ks, vs = selftest_inputs(H, N, d)
    got = _run(entry, Q, K, V, ks, vs)
    want = g[f"out_f32_{H}x{N}x{d}"]
    assert np.max(np.abs(got - want)) <= 1e-4  # the reference self-test's gate
    assert_close(got, want, what=f"{entry} KAT {shape}")


SWEEP_N = (1, 2, 63, 127, 128, 129, 1023, 1024, 1025, 4097)
SWEEP_D = (32, 64, 128, 256, 96, 100, 17)


@pytest.mark.parametrize("d", SWEEP_D)
@pytest.mark.parametrize("N", SWEEP_N)
def test_shape_sweep(N, d):
    """Boundary sequence lengths x head dims (tuned kernel for d in {32,64,128,256},
    generic kernel otherwise); solve and the stream launch agree with the oracle."""
    rng = np.random.default_rng(1000 * N + d)
    H = 3
    Q, K, V, ks, vs = _gpu.reference_problem(H, N, d, rng)
    want = orc.get().head_f32(Q, K, V, ks, vs)
    for entry in ("solve", "split"):
        assert_close(_run(entry, Q, K, V, ks, vs), want, what=f"{entry} H{H} N{N} d{d}")


@pytest.mark.parametrize("seed", SEEDS)
def test_cfg0_reference_shape(seed):
    """Config 0 (B1 H8 d64 L1024) through all three reference entry points."""
    rng = np.random.default_rng(seed)
    Q, K, V, ks, vs = _gpu.reference_problem(8, 1024, 64, rng)
    want = orc.get().head_f32(Q, K, V, ks, vs)
    for entry in ("solve", "split", "simple"):
        assert_close(_run(entry, Q, K, V, ks, vs), want, what=f"cfg0 {entry} seed {seed}")


def test_cfg1_folded_reference_shape():
    """Config 1 folded into the reference ABI: H = B*H = 256, N = 4096, d = 128."""
    rng = np.random.default_rng(17)
    Q, K, V, ks, vs = _gpu.reference_problem(256, 4096, 128, rng)
    want = orc.get().head_f32(Q, K, V, ks, vs)
    for entry in ("solve", "split"):
        assert_close(_run(entry, Q, K, V, ks, vs), want, what=f"cfg1 folded {entry}")


def test_split_launch_on_side_stream_with_garbage_scratch():
    rng = np.random.default_rng(29)
    Q, K, V, ks, vs = _gpu.reference_problem(16, 3000, 128, rng, dist="student_t")
    want = orc.get().head_f32(Q, K, V, ks, vs)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        got = _run("split", Q, K, V, ks, vs, stream=s, scratch_fill=1e30)
    assert_close(got, want, what="side stream")


def test_solve_twice_reuses_workspace():
    """solve's library-owned workspace (arrival counters) is reusable across calls and shapes."""
    o = orc.get()
    for seed, (H, N, d) in enumerate(((4, 5000, 128), (2, 9000, 64), (4, 5000, 128), (8, 700, 256))):
        rng = np.random.default_rng(seed)
        Q, K, V, ks, vs = _gpu.reference_problem(H, N, d, rng)
        assert_close(_run("solve", Q, K, V, ks, vs), o.head_f32(Q, K, V, ks, vs), what=f"solve #{seed}")


def test_tolerance_constants():
    assert (ATOL, RTOL) == (1e-4, 1e-3)


@pytest.mark.parametrize("H,N,d", [(1, 576, 256), (1, 516, 256), (16, 774, 256), (1, 769, 128), (1, 1025, 96)])
def test_split_launch_stays_inside_scratch(H, N, d):
    """kv_int8_split_launch writes only the first H*N floats of S: shapes where
    the record layout fills S (or would overrun it without the bound) run with
    a canary tail after S that must come back unchanged."""
    info = kvq.reference_plan(H, N, d)
    assert info.workspace_bytes <= 4 * H * N
    rng = np.random.default_rng(H * 100000 + N * 10 + d)
    Q, K, V, ks, vs = _gpu.reference_problem(H, N, d, rng)
    want = orc.get().head_f32(Q, K, V, ks, vs)
    gQ, gK, gV, gks, gvs = up(Q), up(K), up(V), up(ks), up(vs)
    tail = 4096
    buf = torch.full((H * N + tail,), float("nan"), dtype=torch.float32, device=_gpu.dev())
    canary = torch.arange(tail, dtype=torch.float32, device=_gpu.dev()) * 0.5 + 12345.0
    buf[H * N:] = canary
    S = buf[: H * N]
    for simple in (False, True):
        out = poisoned((H, d))
        assert kvq.kv_int8_split_launch(gQ, gK, gV, gks, gvs, out, S, simple=simple) == 0
        torch.cuda.synchronize()
        assert_close(down(out), want, what=f"H{H} N{N} d{d} splits {info.splits}")
        assert torch.equal(buf[H * N:], canary), "kv_int8_split_launch wrote past S"


SELFTEST_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "selftest")


@pytest.mark.parametrize("argv", [[], ["8", "1024", "64"], ["3", "257", "128"], ["256", "4096", "128"],
                                  ["2", "5000", "96"]], ids=lambda a: "x".join(a) or "default")
def test_cpp_selftest_program(argv):
    """The C++ self-test (tests/selftest/kvq_selftest.cpp) -- the reference's
    main() of kv_cache/KV_int8_split_optimized.cu:439-543 on its patterned
    inputs, linked against libkvq.so through include/kvq.h -- exits 0 after
    solve, kv_int8_split_launch and kv_int8_simple_launch pass its 1e-4 gate."""
    import subprocess
    exe = os.path.join(SELFTEST_DIR, "kvq_selftest")
    if not os.path.exists(exe):
        subprocess.run(["make", "-C", SELFTEST_DIR, "all"], check=True, capture_output=True)
    r = subprocess.run([exe, *argv], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, f"kvq_selftest {' '.join(argv)} exited {r.returncode}:\n{r.stdout}\n{r.stderr}"
    for entry in ("solve", "kv_int8_split_launch", "kv_int8_simple_launch"):
        assert entry in r.stdout, f"{entry} not exercised:\n{r.stdout}"
