"""GPU-side helpers for the parity tests: move numpy problems to the device,
call the operator through its C ABI (ctypes binding), bring results back."""
from __future__ import annotations

import importlib

import numpy as np
import torch

kvq = importlib.import_module("cuda-operators_amd").kvq


def dev():
    return torch.device("cuda:0")


def up(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def down(t):
    return t.detach().cpu().numpy()


def poisoned(shape, dtype=torch.float32):
    """Output buffer pre-filled with NaN: every element must be overwritten."""
    return torch.full(shape, float("nan"), dtype=dtype, device=dev())


def decode(q, k, v, ks, vs, lengths=None, max_seq_len=None, splits=0, k_new=None, v_new=None,
           softmax_scale=0.0, stream=None):
    """Batched decode through kvq_decode_launch.  Returns (out, k, v, ks, vs) as numpy
    (the caches come back because a fused append writes them)."""
    gq, gk, gv, gks, gvs = up(q), up(k), up(v), up(ks), up(vs)
    gl = None if lengths is None else up(np.asarray(lengths, np.int32))
    gkn = None if k_new is None else up(k_new)
    gvn = None if v_new is None else up(v_new)
    out = poisoned(q.shape)
    cap = k.shape[2]
    msl = max_seq_len if max_seq_len is not None else (cap if lengths is not None else cap)
    d = kvq.Decoder(gq, gk, gv, gks, gvs, out, lengths=gl, max_seq_len=msl, num_splits=splits,
                    k_new=gkn, v_new=gvn, softmax_scale=softmax_scale, stream=stream)
    d(stream)
    torch.cuda.synchronize()
    return down(out), down(gk), down(gv), down(gks), down(gvs)


def reference_problem(H, N, d, rng, dist="normal"):
    """Random problem in the reference ABI layout Q[H,d], K/V[H,N,d], scales[H,N]."""
    from oracle import oracle as orc
    o = orc.get()
    Q = rng.standard_normal((H, d), dtype=np.float32)
    if dist == "normal":
        kf = rng.standard_normal((H, N, d), dtype=np.float32)
        vf = rng.standard_normal((H, N, d), dtype=np.float32)
    else:
        kf = rng.standard_t(4, (H, N, d)).astype(np.float32)
        vf = rng.standard_t(4, (H, N, d)).astype(np.float32)
    K, ks = o.quantize_rows(kf)
    V, vs = o.quantize_rows(vf)
    return Q, K, V, ks, vs
