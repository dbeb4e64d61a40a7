"""kvq_decode_launch_noalloc through the C ABI: the same plan and kernels as
kvq_decode_launch with the library's fixed device scratch array in place of a
workspace, so its output must equal kvq_decode_launch's bit for bit (which the
other GPU tests hold to the oracle; here it is checked against the oracle as
well).  Two calls in a row, the second with a smaller problem, so the second
reads scratch the first left behind; then a problem whose workspace exceeds
the array is rejected before any device work."""
import ctypes

import numpy as np
import pytest
import torch

from _util import assert_close, make_problem
import _gpu
from _gpu import down, kvq, poisoned, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _pair(o, rng, B, Hq, Hkv, cap, d, lengths, splits=0, append=False, check_alloc=True):
    """(noalloc output, kvq_decode_launch output, oracle) for one problem; the
    fused append writes separate cache copies for each path."""
    p = make_problem(rng, B, Hq, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = rng.standard_normal((B, Hkv, d)).astype(np.float32) if append else None
    vn = rng.standard_normal((B, Hkv, d)).astype(np.float32) if append else None
    outs = {}
    # kvq_decode_launch first: the HIP runtime loads each kernel's code object
    # on its first launch (device memory of its own), so the allocation check
    # of the no-alloc call sees only what that call does.
    for path in ("workspace", "noalloc"):
        g = [up(x) for x in (p["q"], p["k"], p["v"], p["ks"], p["vs"])]
        gl = None if lengths is None else up(np.asarray(lengths, np.int32))
        gkn = None if kn is None else up(kn)
        gvn = None if vn is None else up(vn)
        out = poisoned((B, Hq, d))
        msl = 0 if lengths is not None else cap
        params = kvq.decode_params(g[0], g[1], g[2], g[3], g[4], out, gl, msl, 0.0, splits, gkn, gvn)
        if path == "noalloc":
            free0 = torch.cuda.mem_get_info()[0]
            assert kvq.decode_launch_noalloc(params) == 0
            torch.cuda.synchronize()
            if check_alloc:
                assert torch.cuda.mem_get_info()[0] == free0, "the no-alloc launch allocated device memory"
        else:
            ws = kvq.new_workspace(params, g[0].device)
            kvq.decode_launch(params, ws)
            torch.cuda.synchronize()
        outs[path] = (down(out), down(g[1]), down(g[3]))
    k, ks = p["k"].copy(), p["ks"].copy()
    v, vs = p["v"].copy(), p["vs"].copy()
    L = np.asarray(lengths if lengths is not None else np.full(B, cap), np.int32)
    if append:
        o.append(kn, vn, k, v, ks, vs, positions=L - 1)
    ref = o.decode_f32(p["q"], k, v, ks, vs, lengths=L)
    return outs["noalloc"], outs["workspace"], ref, (k, ks)


CASES = ["gqa_ragged_then_smaller", "mha_splits_then_smaller", "append_then_smaller"]


@pytest.fixture(scope="module", autouse=True)
def scratch_loaded():
    """One tiny split call first: the code object holding the scratch array
    is loaded (by the HIP runtime, once per process) on the first lookup of its
    address, so the allocation check below starts from the second call."""
    o = orc.get()
    rng = np.random.default_rng(5)
    _pair(o, rng, 1, 2, 2, 4096, 64, None, splits=4, check_alloc=False)


@pytest.mark.parametrize("case", CASES)
def test_noalloc_matches_workspace_launch(case):
    o = orc.get()
    rng = np.random.default_rng(100 + CASES.index(case))
    if case == "gqa_ragged_then_smaller":
        # in-kernel split plan (matrix-core kernel), then a smaller one
        probs = [dict(B=12, Hq=32, Hkv=8, cap=4096, d=128, lengths=rng.integers(1, 4097, 12)),
                 dict(B=3, Hq=16, Hkv=4, cap=1024, d=128, lengths=np.array([1024, 7, 600]))]
    elif case == "mha_splits_then_smaller":
        # static splits with the last-arrival merge (FMA kernel), then fewer heads and tokens
        probs = [dict(B=2, Hq=8, Hkv=8, cap=16384, d=128, lengths=None, splits=16),
                 dict(B=1, Hq=4, Hkv=4, cap=2048, d=64, lengths=None, splits=4)]
    else:
        # split schedule (80 sequences) with the fused append, then a small ragged batch with append
        probs = [dict(B=80, Hq=16, Hkv=2, cap=1024, d=128, lengths=rng.integers(1, 1025, 80), append=True),
                 dict(B=4, Hq=8, Hkv=2, cap=512, d=128, lengths=np.array([512, 1, 300, 45]), append=True)]
    for i, pr in enumerate(probs):
        lengths = None if pr["lengths"] is None else np.asarray(pr["lengths"], np.int32)
        (na, nak, naks), (ws, wsk, wsks), ref, (k, ks) = _pair(
            o, rng, pr["B"], pr["Hq"], pr["Hkv"], pr["cap"], pr["d"], lengths, pr.get("splits", 0),
            pr.get("append", False))
        assert np.array_equal(_bits(na), _bits(ws)), f"{case} call {i}: noalloc differs from kvq_decode_launch"
        assert_close(na, ref, what=f"{case} call {i}")
        assert np.array_equal(nak, wsk) and np.array_equal(_bits(naks), _bits(wsks))
        if pr.get("append", False):
            assert np.array_equal(nak, k) and np.array_equal(_bits(naks), _bits(ks))


def test_noalloc_rejects_beyond_scratch():
    """A problem whose workspace exceeds KVQ_NOALLOC_SCRATCH_BYTES is rejected
    (hipErrorInvalidValue) before any device work; the output stays poisoned."""
    B, Hq, Hkv, d, cap = 4096, 64, 8, 128, 1024
    A = 1 << 20
    lengths = torch.full((B,), cap, dtype=torch.int32, device="cuda")
    q = torch.zeros((B, Hq, d), device="cuda")
    out = poisoned((B, Hq, d))
    p = kvq.DecodeParams(B, Hq, Hkv, d, cap, 0, lengths.data_ptr(), q.data_ptr(), A, A, A, A, out.data_ptr(),
                         0.0, 0, None, None)
    assert kvq.workspace_size(p) > kvq.NOALLOC_SCRATCH_BYTES
    assert kvq.decode_launch_noalloc(p) == kvq.HIP_ERROR_INVALID_VALUE
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
