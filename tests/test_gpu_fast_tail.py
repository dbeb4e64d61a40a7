"""decode_fast's rebalanced tail: in a range of 8 or more workgroup blocks
(SG = 1) the last block goes to waves 0-3, two 16-token steps each (d = 128;
32-token steps at d = 64).  Ranges whose last block holds from 1 token to a
whole block, with and without the fused append, one or two splits, against
the oracle; the paged layout gives the same bits."""
import numpy as np
import pytest

from _util import assert_close, make_problem
import _gpu
from _gpu import kvq, up, down
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

# Block = 8 waves x one step: 128 tokens at d = 128, 256 at d = 64.  Lengths
# around 8 blocks: exactly 8, 8 + 1 token, partial steps, a whole last block,
# just under 8 (still 8 blocks), 7 blocks (no rebalance).
LENGTHS = {128: [1024, 1025, 1040, 1072, 1087, 1151, 1152, 1023, 896, 1700],
           64: [2048, 2049, 2080, 2111, 2300, 2303, 2047, 1792, 3001, 2560]}


@pytest.fixture(scope="module")
def o():
    return orc.get()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("append", [False, True])
@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("d", [64, 128])
def test_rebalanced_tail_matches_oracle(o, d, splits, append):
    rng = np.random.default_rng(d * 10 + splits * 2 + append)
    lengths = np.array(LENGTHS[d], np.int32)
    B, Hkv = len(lengths), 2
    cap = int(lengths.max())
    prm = kvq.DecodeParams(batch=B, num_q_heads=Hkv, num_kv_heads=Hkv, head_dim=d, capacity=cap,
                           max_seq_len=cap, lengths=4096, q=4096, k_cache=4096, v_cache=4096, k_scale=4096,
                           v_scale=4096, out=4096, num_splits=splits)
    info = kvq.decode_plan(prm)
    assert (info.kernel, info.heads_per_group, info.splits) == (kvq.KERNEL_DECODE_VALU, 1, splits)
    p = make_problem(rng, B, Hkv, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kn = vn = None
    if append:
        kn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
        vn = rng.standard_normal((B, Hkv, d)).astype(np.float32)
    got, gk, gv, gks, gvs = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, splits=splits,
                                        k_new=kn, v_new=vn)
    if append:
        o.append(kn, vn, p["k"], p["v"], p["ks"], p["vs"], positions=lengths - 1)
        assert np.array_equal(gk, p["k"]) and np.array_equal(gv, p["v"])
        assert np.array_equal(_bits(gks), _bits(p["ks"])) and np.array_equal(_bits(gvs), _bits(p["vs"]))
    want = o.decode_f32(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths)
    assert_close(got, want, what=f"d={d} splits={splits} append={append}")


@pytest.mark.parametrize("d,page", [(128, 32), (64, 64)])
def test_rebalanced_tail_paged_bits(o, d, page):
    """The paged layout walks the same token order (its page entries are
    prefetched along it): the same bits as the contiguous layout."""
    from test_gpu_paged import paged_decode, to_pages
    rng = np.random.default_rng(d + page)
    lengths = np.array(LENGTHS[d], np.int32)
    B, Hkv = len(lengths), 2
    cap = int(lengths.max())
    p = make_problem(rng, B, Hkv, Hkv, cap, d, o.quantize_rows, lengths=lengths)
    kp, vp, ksp, vsp, table = to_pages(rng, p["k"], p["v"], p["ks"], p["vs"], lengths, page)
    got = paged_decode(p["q"], kp, vp, ksp, vsp, table, lengths, splits=1)[0]
    ref = _gpu.decode(p["q"], p["k"], p["v"], p["ks"], p["vs"], lengths=lengths, splits=1)[0]
    assert np.array_equal(_bits(got), _bits(ref))
