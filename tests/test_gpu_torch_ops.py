"""torch.ops.kvq.* on the GPU: each operator gives the same bits as the
direct C-ABI call it wraps (itself checked against the oracle elsewhere),
passes torch.library.opcheck's schema and fake-tensor checks, and a decode
step captured into a CUDA (HIP) graph replays correctly: every replay, with
eager updates and synchronisations between replays, equals an eager call."""
import importlib

import numpy as np
import pytest
import torch

from _util import make_problem
import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc

torch_ops = importlib.import_module("cuda-operators_amd.torch_ops")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("G,append", [(1, False), (4, True), (8, False), (2, True)])
def test_decode_op_matches_c_abi(o, G, append):
    rng = np.random.default_rng(G + 10 * append)
    B, Hkv, cap, d = 4, 2, 700, 128
    lengths = np.array([700, 5, 0, 333], np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = rng.standard_normal((B, Hkv, d)).astype(np.float32) if append else None
    vn = rng.standard_normal((B, Hkv, d)).astype(np.float32) if append else None
    ref, rk, _, rks, _ = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, k_new=kn, v_new=vn)
    g = [up(x) for x in (p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths)]
    gkn = None if kn is None else up(kn)
    gvn = None if vn is None else up(vn)
    out = torch.ops.kvq.decode(g[0], g[1], g[2], g[3], g[4], g[5], cap, 0.0, 0, gkn, gvn)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(down(out)), _bits(ref))
    assert np.array_equal(down(g[1]), rk) and np.array_equal(_bits(down(g[3])), _bits(rks))


def test_paged_decode_op_matches_c_abi(o):
    rng = np.random.default_rng(3)
    B, Hkv, G, d, page, maxp = 3, 2, 8, 128, 32, 10
    npages = B * maxp
    q = rng.standard_normal((B, Hkv * G, d)).astype(np.float32)
    kp = rng.integers(-127, 128, (npages, Hkv, page, d), dtype=np.int8)
    vp = rng.integers(-127, 128, (npages, Hkv, page, d), dtype=np.int8)
    ksp = rng.uniform(0.001, 0.05, (npages, Hkv, page)).astype(np.float32)
    vsp = rng.uniform(0.001, 0.05, (npages, Hkv, page)).astype(np.float32)
    table = rng.permutation(npages).reshape(B, maxp).astype(np.int32)
    lengths = np.array([320, 77, 1], np.int32)
    g = [up(x) for x in (q, kp, vp, ksp, vsp, table, lengths)]
    ref = _gpu.poisoned(q.shape)
    kvq.PagedDecoder(g[0], g[1], g[2], g[3], g[4], g[5], g[6], ref)()
    out = torch.ops.kvq.paged_decode(g[0], g[1], g[2], g[3], g[4], g[5], g[6], 0, 0.0, 0, None, None)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(down(out)), _bits(down(ref)))


def test_append_and_prefill_ops(o):
    rng = np.random.default_rng(4)
    B, Hkv, cap, d, L = 2, 2, 64, 128, 9
    k = np.zeros((B, Hkv, cap, d), np.int8)
    s = np.zeros((B, Hkv, cap), np.float32)
    x = rng.standard_normal((B, Hkv, L, d)).astype(np.float32)
    gk, gv, gks, gvs = up(k), up(k), up(s), up(s)
    torch.ops.kvq.prefill(up(x), up(x), gk, gv, gks, gvs, None, 3, None)
    xn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    pos = up(np.array([12, 0], np.int32))
    torch.ops.kvq.append(up(xn), up(xn), gk, gv, gks, gvs, pos, 0)
    torch.cuda.synchronize()
    qx, sx = o.quantize_rows(x)
    qn, sn = o.quantize_rows(xn)
    k[:, :, 3:3 + L], s[:, :, 3:3 + L] = qx, sx
    k[0, :, 12], s[0, :, 12] = qn[0], sn[0]
    k[1, :, 0], s[1, :, 0] = qn[1], sn[1]
    assert np.array_equal(down(gk), k) and np.array_equal(down(gv), k)
    assert np.array_equal(_bits(down(gks)), _bits(s))


def test_opcheck_decode(o):
    rng = np.random.default_rng(5)
    B, Hkv, G, cap, d = 2, 2, 4, 256, 128
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows)
    g = [up(x) for x in (p["q"], p["k"], p["v"], p["ks"], p["vs"])]
    lengths = up(np.array([256, 100], np.int32))
    torch.library.opcheck(torch.ops.kvq.decode.default, (g[0], g[1], g[2], g[3], g[4], lengths, cap, 0.0, 0,
                                                          None, None),
                          test_utils=("test_schema", "test_faketensor"))


@pytest.mark.parametrize("G,B", [(1, 4), (1, 80), (8, 4), (8, 80), (8, 300), (8, 600)])
def test_decode_graph_capture_replays(o, G, B):
    """One ragged decode step captured once and replayed three times; q
    changes eagerly between replays.  4 sequences: one launch that plans its
    splits itself; 80: the split-schedule launch, then the FMA decode (G = 1),
    or the flattened tile plan (matrix-core kernel, G = 8); 300: the
    matrix-core kernel derives the split schedule itself (one launch); 600:
    the schedule launch, then the matrix-core decode."""
    rng = np.random.default_rng(6 + G + B)
    Hkv, cap, d = 2, 1024, 128
    lengths = rng.integers(1, cap + 1, B).astype(np.int32)
    lengths[:4] = [1024, 517, 33, 800]
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    g = [up(x) for x in (p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths)]
    args = lambda: (g[0], g[1], g[2], g[3], g[4], g[5], cap, 0.0, 0, None, None)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        torch.ops.kvq.decode(*args())  # workspace exists before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = torch.ops.kvq.decode(*args())
    info = kvq.decode_plan(kvq.decode_params(g[0], g[1], g[2], g[3], g[4], out, lengths=g[5], max_seq_len=cap))
    want = {(1, 4): kvq.SPLITS_IN_KERNEL, (1, 80): kvq.SPLITS_SCHEDULE, (8, 4): kvq.SPLITS_IN_KERNEL,
            (8, 80): kvq.SPLITS_TILES, (8, 300): kvq.SPLITS_IN_KERNEL, (8, 600): kvq.SPLITS_SCHEDULE}
    assert info.split_plan == want[(G, B)]
    for rep in range(3):
        g[0].copy_(up(rng.standard_normal(p["q"].shape).astype(np.float32)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = torch.ops.kvq.decode(*args())
        torch.cuda.synchronize()
        assert np.array_equal(_bits(down(out)), _bits(down(eager))), f"replay {rep}"


@pytest.mark.parametrize("M,N,splits", [(300, 2000, 0), (4096, 256, 0), (200, 1000, 5)])
def test_attention_op_matches_c_abi(o, M, N, splits):
    rng = np.random.default_rng(M + N)
    d = 128
    q, k, v = (rng.standard_normal(s).astype(np.float32) for s in ((M, d), (N, d), (N, d)))
    g = [up(x) for x in (q, k, v)]
    ref = kvq.attention(g[0], g[1], g[2], num_splits=splits)
    out = torch.ops.kvq.attention(g[0], g[1], g[2], 0.0, splits)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(down(out)), _bits(down(ref)))
    np.testing.assert_allclose(down(out), o.attention_f32(q, k, v), atol=1e-4, rtol=1e-3)
    torch.library.opcheck(torch.ops.kvq.attention.default, (g[0], g[1], g[2], 0.0, splits),
                          test_utils=("test_schema", "test_faketensor"))


def test_attention_graph_capture_replays(o):
    """Split attention (main + merge launches) captured once, replayed three
    times with eager q updates between replays; each replay equals eager."""
    rng = np.random.default_rng(9)
    M, N, d = 256, 3000, 64
    g = [up(rng.standard_normal(s).astype(np.float32)) for s in ((M, d), (N, d), (N, d))]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        torch.ops.kvq.attention(g[0], g[1], g[2], 0.0, 0)  # workspace exists before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = torch.ops.kvq.attention(g[0], g[1], g[2], 0.0, 0)
    for rep in range(3):
        g[0].copy_(up(rng.standard_normal((M, d)).astype(np.float32)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = torch.ops.kvq.attention(g[0], g[1], g[2], 0.0, 0)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(down(out)), _bits(down(eager))), f"replay {rep}"


def test_graph_replay_after_workspace_growth(o):
    """Capture a split decode step on stream s, then run a larger eager
    problem on s (its workspace grows), then replay: the graph still owns
    the workspace it was captured with (the superseded one is kept, not
    freed), so the replay is correct and tensors allocated after the growth
    are not overwritten."""
    rng = np.random.default_rng(77)
    Hkv, G, d = 2, 4, 128
    B1, cap1 = 4, 1024
    lengths = np.array([1024, 517, 33, 800], np.int32)
    p = make_problem(rng, B1, Hkv * G, Hkv, cap1, d, o.quantize_rows, lengths=lengths)
    g = [up(x) for x in (p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths)]
    args = lambda: (g[0], g[1], g[2], g[3], g[4], g[5], cap1, 0.0, 0, None, None)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        torch.ops.kvq.decode(*args())
    s.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = torch.ops.kvq.decode(*args())
    # A larger problem on the same stream grows the cached workspace (200
    # sequences: the split-schedule plan, 2.2 MB against 0.8 MB).
    B2, cap2 = 200, 1024
    l2 = rng.integers(1, cap2 + 1, B2).astype(np.int32)
    p2 = make_problem(rng, B2, Hkv * G, Hkv, cap2, d, o.quantize_rows, lengths=l2)
    g2 = [up(x) for x in (p2["q"], p2["k"], p2["v"], p2["ks"], p2["vs"], l2)]
    with torch.cuda.stream(s):
        big = torch.ops.kvq.decode(g2[0], g2[1], g2[2], g2[3], g2[4], g2[5], cap2, 0.0, 0, None, None)
    s.synchronize()
    key = ("decode", 0, s.cuda_stream)
    assert torch_ops._workspaces[key].numel() >= 2179840 and len(torch_ops._retired) >= 1
    np.testing.assert_allclose(down(big), o.decode_f32(p2["q"], p2["k"], p2["v"], p2["ks"], p2["vs"], lengths=l2),
                               atol=1e-4, rtol=1e-3)
    guards = [torch.full((794624 // 4,), 7.0, device="cuda") for _ in range(16)]  # the old workspace's size
    for rep in range(3):
        g[0].copy_(up(rng.standard_normal(p["q"].shape).astype(np.float32)))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = o.decode_f32(down(g[0]), p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
        np.testing.assert_allclose(down(out), want, atol=1e-4, rtol=1e-3, err_msg=f"replay {rep}")
        assert all(bool((t == 7.0).all()) for t in guards), f"replay {rep} wrote into freed memory"


def test_capture_time_workspace_stays_with_its_graph(o):
    """A decode step captured on a fresh stream with no eager call before
    (its workspace is created inside the capture, zero-filled only when the
    graph replays), then an eager call on the same stream before the first
    replay: the eager call must not use the capture's workspace, whose
    arrival counters were never zeroed.  Both the eager result and every
    replay equal the oracle."""
    rng = np.random.default_rng(91)
    Hkv, G, d, B, cap = 2, 4, 128, 4, 1024
    lengths = np.array([1024, 517, 33, 800], np.int32)
    p = make_problem(rng, B, Hkv * G, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    g = [up(x) for x in (p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths)]
    args = lambda: (g[0], g[1], g[2], g[3], g[4], g[5], cap, 0.0, 0, None, None)
    s = torch.cuda.Stream()
    key = ("decode", 0, s.cuda_stream)
    assert key not in torch_ops._workspaces
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = torch.ops.kvq.decode(*args())
    assert key not in torch_ops._workspaces  # the capture's workspace is the graph's own
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    with torch.cuda.stream(s):
        eager = torch.ops.kvq.decode(*args())
    s.synchronize()
    np.testing.assert_allclose(down(eager), want, atol=1e-4, rtol=1e-3)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_allclose(down(out), want, atol=1e-4, rtol=1e-3, err_msg=f"replay {rep}")
        with torch.cuda.stream(s):
            eager = torch.ops.kvq.decode(*args())
        s.synchronize()
        assert np.array_equal(_bits(down(out)), _bits(down(eager))), f"replay {rep}"
