"""Prefill quantiser (kvq_prefill_quantize_launch) on the GPU, through the C ABI.

Bit-exact against the oracle's quantiser (oracle kvq_ref_quantize_rows, the
rule of the append): every input row (b, h, t) must appear, int8 values and
fp32 scale bits, at cache position start_b + t, and no other cache byte may
change.  bf16 inputs are compared against the oracle on their exact fp32
widening.  Contiguous and paged caches, per-sequence and uniform starts,
positions falling outside the cache (skipped), the tuned head dims and a
generic one, misaligned inputs (generic kernel).
"""
import math

import numpy as np
import pytest
import torch

import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def _inputs(rng, shape, bf16):
    x = (rng.standard_t(4, shape) * rng.uniform(0.01, 50.0, shape[:-1] + (1,))).astype(np.float32)
    x[..., 0, :] = 0.0  # an all-zero row per (b, h)
    if bf16:
        xt = torch.from_numpy(x).to(torch.bfloat16)
        return xt, xt.to(torch.float32).numpy()
    return torch.from_numpy(x), x


def _expected(o, kf, vf, cache_k, cache_v, cache_ks, cache_vs, starts, where):
    """Apply the oracle's quantiser to every row and place it via where(b, h, pos)."""
    B, Hkv, L, d = kf.shape
    qk, sk = o.quantize_rows(kf)
    qv, sv = o.quantize_rows(vf)
    for b in range(B):
        for t in range(L):
            loc = where(b, int(starts[b]) + t)
            if loc is None:
                continue
            for h in range(Hkv):
                i = loc(h)
                cache_k[i], cache_v[i] = qk[b, h, t], qv[b, h, t]
                cache_ks[i], cache_vs[i] = sk[b, h, t], sv[b, h, t]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("d", [32, 64, 128, 256, 96])
def test_prefill_contiguous(o, d, bf16):
    rng = np.random.default_rng(d + 1000 * bf16)
    B, Hkv, L, cap = 3, 2, 37, 80
    xk, kf = _inputs(rng, (B, Hkv, L, d), bf16)
    xv, vf = _inputs(rng, (B, Hkv, L, d), bf16)
    starts = np.array([0, 43, 60], np.int32)  # the last sequence runs past cap: 17 rows skipped
    ck = rng.integers(-128, 128, (B, Hkv, cap, d), dtype=np.int8)
    cv = rng.integers(-128, 128, (B, Hkv, cap, d), dtype=np.int8)
    cks = rng.standard_normal((B, Hkv, cap)).astype(np.float32)
    cvs = rng.standard_normal((B, Hkv, cap)).astype(np.float32)
    g = [up(x) for x in (ck, cv, cks, cvs, starts)]
    kvq.prefill(xk.cuda(), xv.cuda(), g[0], g[1], g[2], g[3], start=g[4])
    torch.cuda.synchronize()
    _expected(o, kf, vf, ck, cv, cks, cvs, starts,
              lambda b, pos: None if pos >= cap else (lambda h: (b, h, pos)))
    assert np.array_equal(down(g[0]), ck) and np.array_equal(down(g[1]), cv)
    assert np.array_equal(_bits(down(g[2])), _bits(cks)) and np.array_equal(_bits(down(g[3])), _bits(cvs))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("d,page", [(128, 16), (128, 64), (64, 32), (96, 16)])
def test_prefill_paged(o, d, page, bf16):
    rng = np.random.default_rng(7 * d + page + bf16)
    B, Hkv, L = 3, 2, 50
    maxp = 8
    npages = B * maxp + 3
    table = rng.permutation(npages)[: B * maxp].reshape(B, maxp).astype(np.int32)
    xk, kf = _inputs(rng, (B, Hkv, L, d), bf16)
    xv, vf = _inputs(rng, (B, Hkv, L, d), bf16)
    ck = rng.integers(-128, 128, (npages, Hkv, page, d), dtype=np.int8)
    cv = rng.integers(-128, 128, (npages, Hkv, page, d), dtype=np.int8)
    cks = rng.standard_normal((npages, Hkv, page)).astype(np.float32)
    cvs = rng.standard_normal((npages, Hkv, page)).astype(np.float32)
    start = 5
    g = [up(x) for x in (ck, cv, cks, cvs, table)]
    kvq.prefill(xk.cuda(), xv.cuda(), g[0], g[1], g[2], g[3], uniform_start=start, block_table=g[4])
    torch.cuda.synchronize()

    def where(b, pos):
        if pos >= maxp * page:
            return None
        return lambda h: (table[b, pos // page], h, pos % page)

    _expected(o, kf, vf, ck, cv, cks, cvs, np.full(B, start), where)
    assert np.array_equal(down(g[0]), ck) and np.array_equal(down(g[1]), cv)
    assert np.array_equal(_bits(down(g[2])), _bits(cks)) and np.array_equal(_bits(down(g[3])), _bits(cvs))


def test_prefill_negative_start_and_misaligned(o):
    """Rows before position 0 are skipped; inputs at an odd 4-byte offset
    take the generic kernel and give the same bits."""
    rng = np.random.default_rng(5)
    B, Hkv, L, d, cap = 2, 3, 20, 128, 32
    xk, kf = _inputs(rng, (B, Hkv, L, d), False)
    xv, vf = _inputs(rng, (B, Hkv, L, d), False)
    starts = np.array([-7, 4], np.int32)
    for misalign in (False, True):
        ck = np.zeros((B, Hkv, cap, d), np.int8)
        cv = np.zeros((B, Hkv, cap, d), np.int8)
        cks = np.zeros((B, Hkv, cap), np.float32)
        cvs = np.zeros((B, Hkv, cap), np.float32)
        g = [up(x) for x in (ck, cv, cks, cvs, starts)]
        if misalign:
            bk = torch.empty(xk.numel() + 1, dtype=torch.float32, device="cuda")
            bv = torch.empty(xv.numel() + 1, dtype=torch.float32, device="cuda")
            gk, gv = bk[1:].view(xk.shape), bv[1:].view(xv.shape)
            gk.copy_(xk.cuda())
            gv.copy_(xv.cuda())
        else:
            gk, gv = xk.cuda(), xv.cuda()
        kvq.prefill(gk, gv, g[0], g[1], g[2], g[3], start=g[4])
        torch.cuda.synchronize()
        _expected(o, kf, vf, ck, cv, cks, cvs, starts,
                  lambda b, pos: None if (pos < 0 or pos >= cap) else (lambda h: (b, h, pos)))
        assert np.array_equal(down(g[0]), ck) and np.array_equal(_bits(down(g[2])), _bits(cks)), misalign


@pytest.mark.parametrize("bf16", [False, True])
def test_prefill_large_matches_row_quantiser(bf16):
    """cfg4-like volume (64 x 8 heads x 1024 tokens x d 128): the tuned prefill
    equals kvq_quantize_rows_launch (checked bit-exact against the oracle
    elsewhere) on every row."""
    B, Hkv, L, d = 64, 8, 1024, 128
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn((B, Hkv, L, d), generator=gen, device="cuda") * 3.0
    if bf16:
        x = x.to(torch.bfloat16)
    k = torch.zeros((B, Hkv, L, d), dtype=torch.int8, device="cuda")
    v = torch.zeros_like(k)
    ks = torch.zeros((B, Hkv, L), dtype=torch.float32, device="cuda")
    vs = torch.zeros_like(ks)
    kvq.prefill(x, x, k, v, ks, vs, uniform_start=0)
    qr, sr = kvq.quantize_rows(x.to(torch.float32).contiguous())
    torch.cuda.synchronize()
    assert torch.equal(k, qr) and torch.equal(v, qr)
    assert torch.equal(ks.view(torch.int32), sr.view(torch.int32)) and torch.equal(vs.view(torch.int32),
                                                                                   sr.view(torch.int32))
