"""The quantisers on the GPU, bit-exact against the CPU oracle.

The reference has no quantiser (kv_cache/new_kvint8.cu:83-84); the rule is
the task spec (scale = max|x|/127, int8 = round(x/scale) clamped to +-127) with
the decisions fixed in the oracle: IEEE division, round half to even, zero or
underflowing scale -> zero row.  Int8 values and scale bits must match exactly.
"""
import os

import numpy as np
import pytest
import torch

import _gpu
from _gpu import down, kvq, up
from _util import student_t4
from oracle import oracle as orc

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def crafted_rows(d):
    rng = np.random.default_rng(d)
    rows = []
    r = np.zeros(d, np.float32)
    r[:8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]  # exact ties (scale 1.0)
    rows.append(r)
    r = np.full(d, 0.25, np.float32)
    r[-1] = -254.0                                           # amax negative, last index
    rows.append(r)
    rows.append(np.zeros(d, np.float32))                     # zero row
    r = np.zeros(d, np.float32)
    r[:3] = [1e-44, -2e-44, 5e-45]                           # scale underflows to 0
    rows.append(r)
    rows.append(rng.standard_normal(d, dtype=np.float32) * np.float32(1e-38))  # subnormal scale
    r = rng.standard_normal(d, dtype=np.float32)
    r[0] = 1e30                                              # huge outlier at index 0
    rows.append(r)
    # ties at a non-unit scale: amax = 254 -> scale = 2.0, x = 2*(k + 0.5)
    r = np.zeros(d, np.float32)
    r[0] = 254.0
    r[1:6] = [1.0, 3.0, 5.0, -7.0, 9.0]
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("d", [16, 64, 100, 128, 256])
def test_quantize_rows_bit_exact(d):
    o = orc.get()
    rng = np.random.default_rng(d + 1)
    x = np.concatenate([crafted_rows(d), rng.standard_normal((500, d), dtype=np.float32),
                        student_t4(rng, (300, d)), rng.standard_normal((50, d), dtype=np.float32) * np.float32(1e4)])
    gq, gs = kvq.quantize_rows(up(x))
    torch.cuda.synchronize()
    wq, ws = o.quantize_rows(x)
    assert np.array_equal(down(gq), wq)
    assert np.array_equal(_bits(down(gs)), _bits(ws))


def test_quantize_golden_fixture():
    g = np.load(os.path.join(GOLD, "quant.npz"), allow_pickle=False)
    gq, gs = kvq.quantize_rows(up(g["x"]))
    torch.cuda.synchronize()
    assert np.array_equal(down(gq), g["q"]) and np.array_equal(_bits(down(gs)), _bits(g["scale"]))


def near_tie_rows(rng, d, rows):
    """Rows whose elements sit at, and one or two ulps either side of, the
    rounding boundaries (k + 1/2) * scale of their own scale: element 0 sets
    amax, so scale = fl(amax / 127); the rest are fl((k + 1/2) * scale) moved
    by -2..2 ulps, for k across the int8 range, at varied magnitudes.  These
    are the elements whose product with 1/scale can round differently from
    the IEEE quotient."""
    out = np.empty((rows, d), np.float32)
    for r in range(rows):
        amax = np.float32(np.exp(rng.uniform(-30.0, 30.0)))
        scale = np.float32(amax / np.float32(127.0))
        k = rng.integers(-127, 127, d - 1).astype(np.float32)
        x = ((k + np.float32(0.5)) * scale).astype(np.float32)
        for _ in range(2):
            step = rng.integers(-1, 2, d - 1)
            x = np.where(step > 0, np.nextafter(x, np.float32(np.inf)),
                         np.where(step < 0, np.nextafter(x, np.float32(-np.inf)), x)).astype(np.float32)
        x = np.clip(x, -amax, amax)
        out[r, 0] = amax if r % 2 == 0 else -amax
        out[r, 1:] = x
    return out


@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_quantize_near_ties_bit_exact(d):
    """The quantiser's multiply-by-reciprocal path must give the IEEE
    division's integers on elements next to rounding boundaries (the oracle
    divides), fp32 and bf16 inputs, through the prefill kernel."""
    o = orc.get()
    rng = np.random.default_rng(100 + d)
    x = near_tie_rows(rng, d, 2048)
    gq, gs = kvq.quantize_rows(up(x))
    torch.cuda.synchronize()
    wq, ws = o.quantize_rows(x)
    assert np.array_equal(_bits(down(gs)), _bits(ws))
    diff = np.argwhere(down(gq) != wq)
    assert diff.size == 0, f"{len(diff)} elements differ, first {diff[:5].tolist()}"
    xb = torch.from_numpy(x).to(torch.bfloat16)
    xbf = xb.to(torch.float32).numpy()
    k = torch.zeros((1, 1, x.shape[0], d), dtype=torch.int8, device="cuda")
    ks = torch.zeros((1, 1, x.shape[0]), dtype=torch.float32, device="cuda")
    kvq.prefill(xb.view(1, 1, -1, d).cuda(), xb.view(1, 1, -1, d).cuda(), k, k.clone(), ks, ks.clone())
    torch.cuda.synchronize()
    bq, bs = o.quantize_rows(xbf)
    assert np.array_equal(down(k)[0, 0], bq) and np.array_equal(_bits(down(ks)[0, 0]), _bits(bs))


def threshold_rows(rng, d, rows):
    """Rows whose quotients x / scale sit near half-integers at distances
    around 2^-15, where the prefill quantiser switches from its reciprocal
    product to the IEEE quotient: delta in {2^-17, 2^-16, 2^-15 * (1 +- 1/8),
    2^-14, 2^-12} either side of k + 1/2, for k across the int8 range."""
    deltas = np.array([2.0 ** -17, 2.0 ** -16, 2.0 ** -15 * 0.875, 2.0 ** -15, 2.0 ** -15 * 1.125,
                       2.0 ** -14, 2.0 ** -12])
    out = np.empty((rows, d), np.float32)
    for r in range(rows):
        amax = np.float32(np.exp(rng.uniform(-20.0, 20.0)))
        scale = np.float64(np.float32(amax / np.float32(127.0)))
        k = rng.integers(-127, 127, d - 1).astype(np.float64)
        sgn = rng.choice([-1.0, 1.0], d - 1)
        dl = rng.choice(deltas, d - 1)
        x = np.clip(((k + 0.5 + sgn * dl) * scale).astype(np.float32), -amax, amax)
        out[r, 0] = amax if r % 2 == 0 else -amax
        out[r, 1:] = x
    return out


@pytest.mark.parametrize("d", [32, 128, 256])
def test_quantize_fast_path_threshold(d):
    """Bit-exact on both sides of the reciprocal path's exactness test, fp32
    and bf16 inputs."""
    o = orc.get()
    rng = np.random.default_rng(300 + d)
    x = threshold_rows(rng, d, 1024)
    gq, gs = kvq.quantize_rows(up(x))
    torch.cuda.synchronize()
    wq, ws = o.quantize_rows(x)
    assert np.array_equal(_bits(down(gs)), _bits(ws))
    diff = np.argwhere(down(gq) != wq)
    assert diff.size == 0, f"{len(diff)} elements differ, first {diff[:5].tolist()}"
    xb = torch.from_numpy(x).to(torch.bfloat16)
    k = torch.zeros((1, 1, x.shape[0], d), dtype=torch.int8, device="cuda")
    ks = torch.zeros((1, 1, x.shape[0]), dtype=torch.float32, device="cuda")
    kvq.prefill(xb.view(1, 1, -1, d).cuda(), xb.view(1, 1, -1, d).cuda(), k, k.clone(), ks, ks.clone())
    torch.cuda.synchronize()
    bq, bs = o.quantize_rows(xb.to(torch.float32).numpy())
    assert np.array_equal(down(k)[0, 0], bq) and np.array_equal(_bits(down(ks)[0, 0]), _bits(bs))


def test_quantize_many_rows():
    """A bulk prefill-sized tensor (grid-stride path) stays bit-exact."""
    o = orc.get()
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 8, 4096, 128), dtype=np.float32)
    gq, gs = kvq.quantize_rows(up(x))
    torch.cuda.synchronize()
    wq, ws = o.quantize_rows(x)
    assert np.array_equal(down(gq), wq) and np.array_equal(_bits(down(gs)), _bits(ws))


@pytest.mark.parametrize("d", [64, 128, 100])
def test_append_bit_exact_and_positions(d):
    o = orc.get()
    rng = np.random.default_rng(d)
    B, Hkv, cap = 4, 3, 50
    k = rng.integers(-127, 128, (B, Hkv, cap, d), dtype=np.int8)
    v = rng.integers(-127, 128, (B, Hkv, cap, d), dtype=np.int8)
    ks = rng.uniform(0.01, 0.1, (B, Hkv, cap)).astype(np.float32)
    vs = rng.uniform(0.01, 0.1, (B, Hkv, cap)).astype(np.float32)
    kn = np.concatenate([crafted_rows(d)[:Hkv][None], rng.standard_normal((B - 1, Hkv, d), dtype=np.float32)])
    vn = student_t4(rng, (B, Hkv, d))
    pos = np.array([0, cap - 1, cap, 17], np.int32)  # cap is out of range: skipped
    gk, gv, gks, gvs = up(k), up(v), up(ks), up(vs)
    kvq.append(up(kn), up(vn), gk, gv, gks, gvs, positions=up(pos))
    torch.cuda.synchronize()
    o.append(kn, vn, k, v, ks, vs, positions=pos)
    assert np.array_equal(down(gk), k) and np.array_equal(down(gv), v)
    assert np.array_equal(_bits(down(gks)), _bits(ks)) and np.array_equal(_bits(down(gvs)), _bits(vs))
    # uniform position
    kvq.append(up(kn), up(vn), gk, gv, gks, gvs, positions=None, uniform_position=5)
    torch.cuda.synchronize()
    o.append(kn, vn, k, v, ks, vs, positions=None, uniform_pos=5)
    assert np.array_equal(down(gk), k) and np.array_equal(_bits(down(gvs)), _bits(vs))


def test_append_cfg4_shape():
    """One appended token per (b, kv head) at config 4's shape (B256, Hkv8, d128)."""
    o = orc.get()
    rng = np.random.default_rng(44)
    B, Hkv, cap, d = 256, 8, 8, 128
    k = np.zeros((B, Hkv, cap, d), np.int8)
    v = np.zeros_like(k)
    ks = np.zeros((B, Hkv, cap), np.float32)
    vs = np.zeros_like(ks)
    kn, vn = student_t4(rng, (B, Hkv, d)), student_t4(rng, (B, Hkv, d))
    pos = rng.integers(0, cap, B).astype(np.int32)
    gk, gv, gks, gvs = up(k), up(v), up(ks), up(vs)
    kvq.append(up(kn), up(vn), gk, gv, gks, gvs, positions=up(pos))
    torch.cuda.synchronize()
    o.append(kn, vn, k, v, ks, vs, positions=pos)
    assert np.array_equal(down(gk), k) and np.array_equal(down(gv), v)
    assert np.array_equal(_bits(down(gks)), _bits(ks)) and np.array_equal(_bits(down(gvs)), _bits(vs))


def tiny_scale_rows(rng, d, rows):
    """Rows whose amax spans 2^-126 .. 2^-80 (denser around 2^-112, below
    which the device's scale takes the IEEE divide, and up to 2^-90, where
    amax * Cl of its divide-free scale is subnormal), random significands."""
    e = np.concatenate([rng.uniform(-126.0, -80.0, rows // 2), rng.uniform(-114.0, -110.0, rows - rows // 2)])
    amax = (np.float32(2.0) ** e.astype(np.float32)) * rng.uniform(1.0, 2.0, rows).astype(np.float32)
    x = rng.uniform(-1.0, 1.0, (rows, d)).astype(np.float32) * amax[:, None]
    x[np.arange(rows), rng.integers(0, d, rows)] = amax * np.where(np.arange(rows) % 2 == 0, 1, -1)
    return x.astype(np.float32)


@pytest.mark.parametrize("d", [64, 128])
def test_quantize_tiny_scales_bit_exact(d):
    """Scales near and below the range of the divide-free scale computation:
    scale bits and int8 values equal the oracle's, fp32 rows through
    quantize_rows and bf16 rows through prefill."""
    o = orc.get()
    x = tiny_scale_rows(np.random.default_rng(300 + d), d, 4096)
    gq, gs = kvq.quantize_rows(up(x))
    torch.cuda.synchronize()
    wq, ws = o.quantize_rows(x)
    assert np.array_equal(_bits(down(gs)), _bits(ws))
    assert np.array_equal(down(gq), wq)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    k = torch.zeros((1, 1, x.shape[0], d), dtype=torch.int8, device="cuda")
    ks = torch.zeros((1, 1, x.shape[0]), dtype=torch.float32, device="cuda")
    kvq.prefill(xb.view(1, 1, -1, d).cuda(), xb.view(1, 1, -1, d).cuda(), k, k.clone(), ks, ks.clone())
    torch.cuda.synchronize()
    bq, bs = o.quantize_rows(xb.to(torch.float32).numpy())
    assert np.array_equal(_bits(down(ks)[0, 0]), _bits(bs)) and np.array_equal(down(k)[0, 0], bq)


_STRIDE_CHILD = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
from _gpu import down, kvq, up
from oracle import oracle as orc
o = orc.get()
rng = np.random.default_rng(11)
for dt in (torch.float32, torch.bfloat16):
    for d in (64, 128):
        x = (rng.standard_normal((3, 2, 1000, d), dtype=np.float32) * 3).astype(np.float32)
        xt = torch.from_numpy(x).to(dt)
        k = torch.zeros((3, 2, 1000, d), dtype=torch.int8, device="cuda")
        ks = torch.zeros((3, 2, 1000), dtype=torch.float32, device="cuda")
        v, vs = k.clone(), ks.clone()
        kvq.prefill(xt.cuda(), (-xt).cuda(), k, v, ks, vs)
        torch.cuda.synchronize()
        xf = xt.to(torch.float32).numpy().reshape(-1, d)
        wq, ws = o.quantize_rows(xf)
        nq, ns = o.quantize_rows(-xf)
        assert np.array_equal(down(k).reshape(-1, d), wq) and np.array_equal(down(ks).reshape(-1), ws)
        assert np.array_equal(down(v).reshape(-1, d), nq) and np.array_equal(down(vs).reshape(-1), ns)
print("stride ok")
"""


def test_prefill_grid_stride_loop():
    """The prefill quantiser with its grid capped at 3 workgroups per plane
    (KVQ_PREFILL_MAX_GROUPS, read once per process, hence a child process):
    every workgroup walks the rows of both planes in strides, bit-exact."""
    import subprocess
    import sys
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, KVQ_PREFILL_MAX_GROUPS="3")
    r = subprocess.run([sys.executable, "-c", _STRIDE_CHILD, repo], env=env, capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0 and "stride ok" in r.stdout, (r.stdout + r.stderr)[-3000:]
