"""Dense fp32 attention (attention_online_launch / kvq_attention_launch) on the
GPU, through the C ABI, against the oracle's restatement of
attention/softmax_new.cu (kvq_ref_attention_f32, pinned in test_oracle.py).

Tolerance: |gpu - oracle| <= 1e-4 + 1e-3 * |oracle| per element (fp32 with a
different summation order and exp2 of log2-scaled scores).  Cases: the
matrix-core head dims (32, 64, 128, 256) with query counts around the
128-query block and key counts around the 64-key tile (32 at d = 256), split and unsplit plans,
explicit split requests, untuned head dims and misaligned pointers (generic
kernel), peaked and flat softmax, workspace reuse across calls, a side
stream, and at full prefill size a float64 check of sampled rows."""
import math

import numpy as np
import pytest
import torch

import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
ATOL, RTOL = 1e-4, 1e-3


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _problem(rng, M, N, d, qscale=1.0):
    q = (rng.standard_normal((M, d)) * qscale).astype(np.float32)
    k = rng.standard_normal((N, d)).astype(np.float32)
    v = rng.standard_normal((N, d)).astype(np.float32)
    return q, k, v


def _close(got, ref, what=""):
    np.testing.assert_allclose(got, ref, atol=ATOL, rtol=RTOL, err_msg=what)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 12, 16])
@pytest.mark.parametrize("N", [1, 13, 4099, 65536])
def test_attention_few_queries(o, d, M, N):
    """Few queries: the VALU kernel (up to 4 queries at d = 128, 2 at d = 64,
    8 at d = 32 and 256, and 9-16 as 8-query blocks at d = 32 and 256 from
    65536 keys) with key splits of whole 4096/d-key steps, a tail step past N
    and merged records; the rest take attention_direct or the padded
    matrix-core block."""
    rng = np.random.default_rng(M * 131 + N * 7 + d)
    q, k, v = _problem(rng, M, N, d)
    out = _gpu.poisoned((M, d))
    kvq.attention_online(up(q), up(k), up(v), out)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"M={M} N={N} d={d}")


@pytest.mark.parametrize("N,splits", [(32768, 0), (40001, 0), (131072, 0), (140000, 0), (65536, 128), (65536, 512),
                                      (20000, 100)])
@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_attention_one_query_split_sizes(o, d, N, splits):
    """One query: splits of 128-512 keys run 8 waves per workgroup, others 4
    (the window's edges, a ragged last split, explicit split requests on
    both sides of it)."""
    rng = np.random.default_rng(N + d + splits)
    q, k, v = _problem(rng, 1, N, d)
    gq, gk, gv = up(q), up(k), up(v)
    out = _gpu.poisoned((1, d))
    p = kvq.attention_params(gq, gk, gv, out, num_splits=splits)
    info = kvq.attention_plan(p)
    assert info.kernel == kvq.KERNEL_ATTENTION_ROWS and info.query_block == 1, (info.kernel, info.query_block)
    kvq.attention(gq, gk, gv, out, num_splits=splits)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"N={N} d={d} splits={splits} chunk={info.chunk}")


@pytest.mark.parametrize("splits", [1, 2, 5, 1 << 20])
@pytest.mark.parametrize("M", [4, 6])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_attention_few_queries_peaked_and_splits(o, d, M, splits):
    """Large logits (frequent rescales) under any split request, and
    identical keys (the output is the mean of V): at d = 256 M = 4 runs the
    few-query kernel's 4-query block and M = 6 its 8-query block (a key row
    over d/8 lanes with 8 dims each); at d = 128 M = 4 the 4-query block; the
    others attention_direct."""
    rng = np.random.default_rng(d + splits + 1000 * M)
    N = 3000
    q, k, v = _problem(rng, M, N, d, qscale=8.0)
    gq, gk, gv = up(q), up(k), up(v)
    out = _gpu.poisoned((M, d))
    p = kvq.attention_params(gq, gk, gv, out, num_splits=splits)
    n = kvq.attention_workspace_size(p)
    ws = torch.full((max(n, 1),), 0xFF, dtype=torch.uint8, device="cuda")  # NaN bytes: records need no init
    kvq.attention(gq, gk, gv, out, num_splits=splits, workspace=ws)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"peaked, splits={splits}")
    kf = np.repeat(rng.standard_normal((1, d)).astype(np.float32), N, axis=0)
    out = kvq.attention_online(gq, up(kf), gv)
    torch.cuda.synchronize()
    _close(down(out), np.broadcast_to(v.astype(np.float64).mean(0), (M, d)), "flat")


@pytest.mark.parametrize("d,M,N", [(128, M, N) for M in (5, 8, 9, 16, 17, 32) for N in (1, 15, 17, 4099, 65536)]
                         + [(128, M, N) for M in (33, 64) for N in (16399, 65536)]
                         + [(64, M, N) for M in (3, 8) for N in (1, 17, 4099)]
                         + [(64, M, N) for M in (9, 16, 33, 64) for N in (32785, 65536)])
def test_attention_direct_kernel(o, d, M, N):
    """attention_direct (16 queries per wave, keys straight from memory in
    16-key blocks) where the planner picks it -- d = 128 with 5-32 queries
    at any N or 33-64 from 16384 keys, d = 64 with 3-8 queries at any N or
    up to 64 from 32768 keys: a single key, blocks cut short by N, the plan's
    key splits, rows past M in the last wave."""
    rng = np.random.default_rng(M * 17 + N * 3 + d)
    q, k, v = _problem(rng, M, N, d)
    gq, gk, gv = up(q), up(k), up(v)
    out = _gpu.poisoned((M, d))
    info = kvq.attention_plan(kvq.attention_params(gq, gk, gv, out))
    assert info.kernel == kvq.KERNEL_ATTENTION_DIRECT
    kvq.attention_online(gq, gk, gv, out)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"M={M} N={N} d={d}")


@pytest.mark.parametrize("d,M", [(128, 8), (128, 16), (128, 40), (64, 16)])
def test_attention_direct_long_keys(o, d, M):
    """attention_direct over 2^18 + 5 keys: 253 splits of 1040 keys (the
    plan aims at 256 in whole 16-key blocks), each walked by 4 key parts (1
    beyond 32 queries), the last split short."""
    rng = np.random.default_rng(7 * M + d)
    N = (1 << 18) + 5
    q, k, v = _problem(rng, M, N, d)
    gq, gk, gv = up(q), up(k), up(v)
    out = _gpu.poisoned((M, d))
    info = kvq.attention_plan(kvq.attention_params(gq, gk, gv, out))
    assert info.kernel == kvq.KERNEL_ATTENTION_DIRECT and (info.splits, info.chunk) == (253, 1040)
    kvq.attention_online(gq, gk, gv, out)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"M={M} N={N} d={d}")


@pytest.mark.parametrize("splits", [1, 2, 5, 1 << 20])
@pytest.mark.parametrize("d,M,N", [(128, 12, 3000), (128, 40, 20000), (64, 40, 33000)])
def test_attention_direct_peaked_and_splits(o, d, M, N, splits):
    """attention_direct under any split request with large logits (frequent
    rescales) and a NaN-filled workspace, and with identical keys (the
    output is the mean of V)."""
    rng = np.random.default_rng(d + splits + 100 * M)
    q, k, v = _problem(rng, M, N, d, qscale=8.0)
    gq, gk, gv = up(q), up(k), up(v)
    out = _gpu.poisoned((M, d))
    p = kvq.attention_params(gq, gk, gv, out, num_splits=splits)
    assert kvq.attention_plan(p).kernel == kvq.KERNEL_ATTENTION_DIRECT
    n = kvq.attention_workspace_size(p)
    ws = torch.full((max(n, 1),), 0xFF, dtype=torch.uint8, device="cuda")
    kvq.attention(gq, gk, gv, out, num_splits=splits, workspace=ws)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"peaked, splits={splits}")
    kf = np.repeat(rng.standard_normal((1, d)).astype(np.float32), N, axis=0)
    out = kvq.attention_online(gq, up(kf), gv)
    torch.cuda.synchronize()
    _close(down(out), np.broadcast_to(v.astype(np.float64).mean(0), (M, d)), "flat")


@pytest.mark.parametrize("d", [32, 64, 128, 256])
@pytest.mark.parametrize("M,N", [(1, 1), (1, 4099), (7, 64), (128, 65), (129, 300), (200, 1000), (256, 4096),
                                 (1000, 127), (513, 2048), (63, 1024), (65, 700), (191, 256)])
def test_attention_online_tuned(o, d, M, N):
    """Query blocks of 128 (8 waves) where they fill the GPU -- (256, 4096)
    -- and of 64 (4 waves, d <= 128) where they do not: the other shapes,
    with rows past M in the last block."""
    rng = np.random.default_rng(M * 7919 + N * 31 + d)
    q, k, v = _problem(rng, M, N, d)
    out = _gpu.poisoned((M, d))
    kvq.attention_online(up(q), up(k), up(v), out)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"M={M} N={N} d={d}")


@pytest.mark.parametrize("d", [1, 17, 96, 512, 1024])
def test_attention_online_generic_dims(o, d):
    rng = np.random.default_rng(d)
    M, N = 37, 301
    q, k, v = _problem(rng, M, N, d)
    out = _gpu.poisoned((M, d))
    kvq.attention_online(up(q), up(k), up(v), out)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"d={d}")


@pytest.mark.parametrize("which", ["q", "k", "v", "out"])
@pytest.mark.parametrize("M,N,d", [(150, 333, 64), (4, 5000, 128), (1, 65536, 256), (300, 2000, 32)])
def test_attention_misaligned_takes_generic_path(o, which, M, N, d):
    """A 4-byte-aligned q, k, v or out at a tuned head dim runs
    attention_generic, unsplit (kvq_attention_plan says so), and matches."""
    rng = np.random.default_rng(11 + M + d)
    q, k, v = _problem(rng, M, N, d)
    t = {"q": up(q), "k": up(k), "v": up(v), "out": _gpu.poisoned((M, d))}
    aligned = kvq.attention_plan(kvq.attention_params(t["q"], t["k"], t["v"], t["out"]))
    assert aligned.kernel != kvq.KERNEL_ATTENTION_GENERIC
    base = torch.full((t[which].numel() + 1,), float("nan"), dtype=torch.float32, device="cuda")
    shifted = base[1:].view(t[which].shape)
    shifted.copy_(t[which])
    t[which] = shifted
    info = kvq.attention_plan(kvq.attention_params(t["q"], t["k"], t["v"], t["out"]))
    assert (info.kernel, info.splits, info.workspace_bytes) == (kvq.KERNEL_ATTENTION_GENERIC, 1, 0)
    kvq.attention_online(t["q"], t["k"], t["v"], t["out"])
    torch.cuda.synchronize()
    _close(down(t["out"]), o.attention_f32(q, k, v), which)


@pytest.mark.parametrize("M,N,d", [(1, 65536, 128), (37, 301, 96), (200, 1000, 64)])
def test_attention_compat_solve(o, M, N, d):
    """The reference's `solve(Q, K, V, output, M, N, d)`
    (attention/softmax_new.cu:283-287) from libkvq_attention.so: asynchronous
    on the null stream, same result as attention_online_launch."""
    rng = np.random.default_rng(M + N + d)
    q, k, v = _problem(rng, M, N, d)
    out = _gpu.poisoned((M, d))
    kvq.attention_solve(up(q), up(k), up(v), out)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"solve M={M} N={N} d={d}")


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 64, 1 << 20])
def test_attention_split_requests(o, splits):
    """Any split request (clamped to whole key tiles) gives the same result
    within tolerance; the workspace is reused by a second, smaller problem."""
    rng = np.random.default_rng(splits)
    M, N, d = 300, 2500, 128
    q, k, v = _problem(rng, M, N, d)
    gq, gk, gv = up(q), up(k), up(v)
    out = _gpu.poisoned((M, d))
    p = kvq.attention_params(gq, gk, gv, out, num_splits=splits)
    n = kvq.attention_workspace_size(p)
    assert (n == 0) == (splits == 1)
    ws = torch.full((max(n, 1),), 0xFF, dtype=torch.uint8, device="cuda")  # NaN bytes: records need no init
    kvq.attention(gq, gk, gv, out, num_splits=splits, workspace=ws)
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), f"splits={splits}")
    q2, k2, v2 = _problem(rng, 200, 1300, 128)
    out2 = _gpu.poisoned((200, 128))
    kvq.attention(up(q2), up(k2), up(v2), out2, num_splits=splits, workspace=ws)
    torch.cuda.synchronize()
    _close(down(out2), o.attention_f32(q2, k2, v2), f"second call, splits={splits}")


@pytest.mark.parametrize("d", [64, 128, 256])
def test_attention_peaked_and_flat(o, d):
    """Large logits (running max changes often, rescales taken) and identical
    keys (uniform weights: the output is the mean of V)."""
    rng = np.random.default_rng(d + 3)
    M, N = 140, 1500
    q, k, v = _problem(rng, M, N, d, qscale=8.0)
    out = kvq.attention_online(up(q), up(k), up(v))
    torch.cuda.synchronize()
    _close(down(out), o.attention_f32(q, k, v), "peaked")
    kf = np.repeat(rng.standard_normal((1, d)).astype(np.float32), N, axis=0)
    out = kvq.attention_online(up(q), up(kf), up(v))
    torch.cuda.synchronize()
    _close(down(out), np.broadcast_to(v.astype(np.float64).mean(0), (M, d)), "flat")


def test_attention_scale_and_side_stream(o):
    rng = np.random.default_rng(5)
    M, N, d = 130, 777, 128
    q, k, v = _problem(rng, M, N, d)
    s = torch.cuda.Stream()
    gq, gk, gv = up(q), up(k), up(v)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        out = kvq.attention(gq, gk, gv, softmax_scale=0.25)
        out_ref_abi = kvq.attention_online(gq, gk, gv)
    s.synchronize()
    # softmax(q k^T * 0.25) is the default-scale attention of q * 0.25 * sqrt(d).
    _close(down(out), o.attention_f32(q * np.float32(0.25 * math.sqrt(d)), k, v), "scale 0.25")
    _close(down(out_ref_abi), o.attention_f32(q, k, v), "side stream")


def test_attention_prefill_size_sampled_rows():
    """M = N = 4096, d = 128 (one prefill head): 96 sampled rows checked in
    float64 on the CPU; the output is finite everywhere and each row lies in
    the per-dim range of V (softmax weights are a convex combination)."""
    M = N = 4096
    d = 128
    gen = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn((M, d), generator=gen, device="cuda")
    k = torch.randn((N, d), generator=gen, device="cuda")
    v = torch.randn((N, d), generator=gen, device="cuda")
    out = kvq.attention_online(q, k, v)
    torch.cuda.synchronize()
    rows = torch.randperm(M, generator=torch.Generator().manual_seed(1))[:96]
    qc, kc, vc = q.cpu().double(), k.cpu().double(), v.cpu().double()
    s = (qc[rows] @ kc.T) / math.sqrt(d)
    ref = torch.softmax(s, dim=1) @ vc
    got = out.cpu()[rows].double()
    assert torch.allclose(got, ref, atol=ATOL, rtol=RTOL), (got - ref).abs().max()
    oc = out.cpu()
    assert torch.isfinite(oc).all()
    assert (oc <= vc.max(0).values.float() + 1e-5).all() and (oc >= vc.min(0).values.float() - 1e-5).all()
