"""Caches beyond 4 GiB: 64-bit row and page addressing.

A contiguous cache [5, 8, 2^20, 128] int8 (5.4 GB per K and V) whose one
non-empty sequence starts at byte 2^32, and a page pool whose pages lie past
byte 2^32, each decoded by the FMA kernel (MHA) and the matrix-core kernel
(4 query heads per kv head), with and without the fused append (whose int8
row and scale are written past 2^32).  Only the touched slices are filled;
the empty sequences' rows stay uninitialised, as the kernels never read them.

Parity as in test_gpu_decode: the oracle's kvq_ref_decode_f32 over the
non-empty sequence's slice, 1e-4 abs + 1e-3 rel; appended bytes bit-exact.
"""
import numpy as np
import pytest
import torch

from _util import assert_close
import _gpu
from _gpu import down, kvq, up
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

HKV, D, L = 8, 128, 3000
B, CAP = 5, 1 << 20        # sequence 4 starts at byte 4 * 8 * 2^20 * 128 = 2^32
PAGE, POOL = 64, (1 << 16) + 640   # page 2^16 starts at byte 2^32


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _slice(rng, o, n):
    """Quantised K/V rows for one sequence: int8 [HKV, n, D] and scales [HKV, n]."""
    k, ks = o.quantize_rows(rng.standard_normal((HKV, n, D)).astype(np.float32))
    v, vs = o.quantize_rows(rng.standard_normal((HKV, n, D)).astype(np.float32))
    return k, v, ks, vs


def _want(o, q_last, k, v, ks, vs, kn, vn):
    """Oracle output of the non-empty sequence, after the append when kn is given."""
    if kn is not None:
        o.append(kn, vn, k[None], v[None], ks[None], vs[None], positions=np.array([L - 1], np.int32))
    return o.decode_f32(q_last[None], k[None], v[None], ks[None], vs[None], lengths=np.array([L], np.int32))[0]


def _empty_rows(o, q):
    """Oracle output for zero-length sequences."""
    n = q.shape[0]
    z8 = np.zeros((n, HKV, 4, D), np.int8)
    zs = np.zeros((n, HKV, 4), np.float32)
    return o.decode_f32(q, z8, z8, zs, zs, lengths=np.zeros(n, np.int32))


@pytest.mark.parametrize("append", [False, True])
@pytest.mark.parametrize("G", [1, 4])
def test_contiguous_past_4gib(o, G, append):
    rng = np.random.default_rng(9100 + 10 * G + append)
    dev = _gpu.dev()
    print(f"contiguous [{B},{HKV},{CAP},{D}] G={G} append={append}", flush=True)
    gk = torch.empty((B, HKV, CAP, D), dtype=torch.int8, device=dev)
    gv = torch.empty_like(gk)
    gks = torch.empty((B, HKV, CAP), dtype=torch.float32, device=dev)
    gvs = torch.empty_like(gks)
    try:
        assert gk[B - 1].data_ptr() - gk.data_ptr() == 1 << 32
        k, v, ks, vs = _slice(rng, o, L)
        gk[B - 1, :, :L].copy_(torch.from_numpy(k))
        gv[B - 1, :, :L].copy_(torch.from_numpy(v))
        gks[B - 1, :, :L].copy_(torch.from_numpy(ks))
        gvs[B - 1, :, :L].copy_(torch.from_numpy(vs))
        q = rng.standard_normal((B, HKV * G, D)).astype(np.float32)
        lengths = np.array([0] * (B - 1) + [L], np.int32)
        kn = vn = None
        if append:
            kn = rng.standard_normal((B, HKV, D)).astype(np.float32)
            vn = rng.standard_normal((B, HKV, D)).astype(np.float32)
        out = _gpu.poisoned(q.shape)
        kvq.Decoder(up(q), gk, gv, gks, gvs, out, lengths=up(lengths), max_seq_len=L,
                    k_new=None if kn is None else up(kn), v_new=None if vn is None else up(vn))()
        torch.cuda.synchronize()
        got = down(out)
        want = _want(o, q[B - 1], k, v, ks, vs, None if kn is None else kn[B - 1:], None if vn is None else vn[B - 1:])
        if append:
            assert np.array_equal(down(gk[B - 1, :, L - 1]), k[:, L - 1]), "appended K row past 4 GiB differs"
            assert np.array_equal(down(gv[B - 1, :, L - 1]), v[:, L - 1]), "appended V row past 4 GiB differs"
            assert np.array_equal(down(gks[B - 1, :, L - 1]).view(np.uint32), ks[:, L - 1].view(np.uint32))
            assert np.array_equal(down(gvs[B - 1, :, L - 1]).view(np.uint32), vs[:, L - 1].view(np.uint32))
        assert_close(got[B - 1], want, what=f"sequence at 4 GiB, G={G} append={append}")
        assert_close(got[:B - 1], _empty_rows(o, q[:B - 1]), what="empty sequences")
    finally:
        del gk, gv, gks, gvs
        torch.cuda.empty_cache()


@pytest.mark.parametrize("append", [False, True])
@pytest.mark.parametrize("G", [1, 4])
def test_paged_past_4gib(o, G, append):
    rng = np.random.default_rng(9200 + 10 * G + append)
    dev = _gpu.dev()
    npg = -(-L // PAGE)
    print(f"paged pool {POOL} x [{HKV},{PAGE},{D}] G={G} append={append}", flush=True)
    kp = torch.empty((POOL, HKV, PAGE, D), dtype=torch.int8, device=dev)
    vp = torch.empty_like(kp)
    ksp = torch.empty((POOL, HKV, PAGE), dtype=torch.float32, device=dev)
    vsp = torch.empty_like(ksp)
    try:
        assert kp[1 << 16].data_ptr() - kp.data_ptr() == 1 << 32
        # The sequence's pages: shuffled, all but the first two past byte 2^32.
        pages = np.concatenate([[5, (1 << 15) + 3], rng.choice(np.arange(1 << 16, POOL), npg - 2, replace=False)])
        pages = pages[rng.permutation(npg)].astype(np.int32)
        k, v, ks, vs = _slice(rng, o, npg * PAGE)
        for j, pg in enumerate(pages.tolist()):
            sl = slice(j * PAGE, (j + 1) * PAGE)
            kp[pg].copy_(torch.from_numpy(np.ascontiguousarray(k[:, sl])))
            vp[pg].copy_(torch.from_numpy(np.ascontiguousarray(v[:, sl])))
            ksp[pg].copy_(torch.from_numpy(np.ascontiguousarray(ks[:, sl])))
            vsp[pg].copy_(torch.from_numpy(np.ascontiguousarray(vs[:, sl])))
        k, v, ks, vs = (np.ascontiguousarray(x[:, :L]) for x in (k, v, ks, vs))
        q = rng.standard_normal((1, HKV * G, D)).astype(np.float32)
        kn = vn = None
        if append:
            kn = rng.standard_normal((1, HKV, D)).astype(np.float32)
            vn = rng.standard_normal((1, HKV, D)).astype(np.float32)
        out = _gpu.poisoned(q.shape)
        kvq.PagedDecoder(up(q), kp, vp, ksp, vsp, up(pages[None]), up(np.array([L], np.int32)), out,
                         max_seq_len=L, k_new=None if kn is None else up(kn),
                         v_new=None if vn is None else up(vn))()
        torch.cuda.synchronize()
        got = down(out)
        want = _want(o, q[0], k, v, ks, vs, kn, vn)
        if append:
            pg, slot = int(pages[(L - 1) // PAGE]), (L - 1) % PAGE
            assert np.array_equal(down(kp[pg, :, slot]), k[:, L - 1]), "appended K row differs"
            assert np.array_equal(down(vp[pg, :, slot]), v[:, L - 1]), "appended V row differs"
            assert np.array_equal(down(ksp[pg, :, slot]).view(np.uint32), ks[:, L - 1].view(np.uint32))
            assert np.array_equal(down(vsp[pg, :, slot]).view(np.uint32), vs[:, L - 1].view(np.uint32))
        assert_close(got[0], want, what=f"pages past 4 GiB, G={G} append={append}")
    finally:
        del kp, vp, ksp, vsp
        torch.cuda.empty_cache()


def test_prefill_and_append_past_4gib(o):
    """The prefill quantiser and the standalone append write rows of a
    [5, 8, 2^20, 128] cache up to its last slot (which ends at byte 5 * 2^30),
    bit-exact against the oracle's quantiser; positions -1 and cap are skipped."""
    rng = np.random.default_rng(9300)
    dev = _gpu.dev()
    n = 256
    print(f"prefill + append into [{B},{HKV},{CAP},{D}]", flush=True)
    gk = torch.empty((B, HKV, CAP, D), dtype=torch.int8, device=dev)
    gv = torch.empty_like(gk)
    gks = torch.empty((B, HKV, CAP), dtype=torch.float32, device=dev)
    gvs = torch.empty_like(gks)
    try:
        xk = rng.standard_normal((B, HKV, n, D)).astype(np.float32)
        xv = rng.standard_normal((B, HKV, n, D)).astype(np.float32)
        start = np.array([0, 1 << 19, 3, (1 << 20) - 2 * n, CAP - n - 1], np.int32)
        kvq.prefill(up(xk), up(xv), gk, gv, gks, gvs, start=up(start))
        kn = rng.standard_normal((B, HKV, D)).astype(np.float32)
        vn = rng.standard_normal((B, HKV, D)).astype(np.float32)
        pos = np.array([-1, 5, -1, CAP, CAP - 1], np.int32)  # -1 and CAP are skipped
        kvq.append(up(kn), up(vn), gk, gv, gks, gvs, positions=up(pos))
        torch.cuda.synchronize()
        wk, wks = o.quantize_rows(xk)
        wv, wvs = o.quantize_rows(xv)
        for b in range(B):
            sl = slice(int(start[b]), int(start[b]) + n)
            assert np.array_equal(down(gk[b, :, sl]), wk[b]), f"prefill K rows of sequence {b}"
            assert np.array_equal(down(gv[b, :, sl]), wv[b]), f"prefill V rows of sequence {b}"
            assert np.array_equal(down(gks[b, :, sl]).view(np.uint32), wks[b].view(np.uint32)), f"K scales {b}"
            assert np.array_equal(down(gvs[b, :, sl]).view(np.uint32), wvs[b].view(np.uint32)), f"V scales {b}"
        ak, aks = o.quantize_rows(kn)
        av, avs = o.quantize_rows(vn)
        for b in (1, 4):
            p = int(pos[b])
            assert np.array_equal(down(gk[b, :, p]), ak[b]) and np.array_equal(down(gv[b, :, p]), av[b]), b
            assert np.array_equal(down(gks[b, :, p]).view(np.uint32), aks[b].view(np.uint32)), b
            assert np.array_equal(down(gvs[b, :, p]).view(np.uint32), avs[b].view(np.uint32)), b
        # The rows next to the appended slot of sequence 4 are the prefill's, untouched.
        assert np.array_equal(down(gk[4, :, CAP - 2]), wk[4, :, n - 1])
    finally:
        del gk, gv, gks, gvs
        torch.cuda.empty_cache()
