// kvq_attention.hip -- dense fp32 attention forward on gfx950 matrix cores:
// out = softmax(Q K^T / sqrt(d)) V for Q[M,d], K/V[N,d] (one head), the math
// of the reference's attention_online_launch (attention/softmax_new.cu:87-281).
//
// attention_mfma<D> (d in {32, 64, 128, 256}): a workgroup of 8 waves owns
// 128 queries (16 per wave) and one split of the keys, which it streams
// through LDS in 64-key tiles (32 at d = 256) shared by all its waves (two
// LDS buffers: one barrier per tile; 135 KB of LDS at d = 128).  Both products run on
// v_mfma_f32_16x16x4_f32 (fp32 in, fp32 accumulate: the same arithmetic as
// fp32 FMAs, in another order):
//   * S^T = K Q^T per 16-key block: A = K rows from LDS, B = this wave's q
//     (held in registers, pre-scaled by softmax_scale * log2 e); the k index
//     g = lane / 16 of step s is dim g * D/4 + s, so each lane reads its K
//     operands as contiguous 16-byte LDS loads.  C leaves lane l with keys
//     4g + i of query l % 16.
//   * online softmax per query: max and sum over the lane's 16 keys of the
//     tile and across the 4 lane groups (shuffles); exp2 of log2-unit scores.
//   * O^T += V^T P^T: the P values stay in the registers the QK product left
//     them in -- step i of a key block takes register i of every lane, i.e.
//     keys {4g + i}, and the A operand reads V rows 4g + i to match.  Output
//     rows (dims) of block c are dims (D/16) * m + c, so each lane's V
//     operands are contiguous too.
// Keys are split over the grid's second dimension when the query blocks alone
// cannot fill the GPU; splits write partial (m, l, acc) records and a second
// launch, attention_merge, combines them over the whole grid (a merge by the
// last split to arrive would leave the records of a query block to one CU,
// whose far reads then dominate the launch).
//
// attention_generic: any d <= 1024 (one wave per query row, VALU), the
// correctness path for other head dims.
#include <math.h>

#include "kvq_device.hpp"
#include "kvq_internal.hpp"

namespace kvq {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Waves per workgroup (16 queries each): kAttnBlockWide / 16, or
// kAttnBlockNarrow / 16 when the wide blocks cannot fill the GPU.
// Keys per LDS tile: 64, or 32 at d = 256 (two double-buffered K/V tiles of
// 64 x 256 floats would not fit in LDS).
template <int D>
constexpr int attention_tile() {
    return D >= 256 ? 32 : 64;
}
constexpr int kAttnMaxSplits = 1024;    // key splits per launch (the merge loops over them)

// Merge of the split records: a group of 2^glog lanes (within one wave) per
// (query, 16-byte output column), lane j of the group taking splits j, j + G,
// ...  The weights of a query's splits, w_s = 2^(m_s - max m), come from its
// (m, l) records (read by every column group of the query: cache hits after
// the first); out = sum_s w_s acc_s / sum_s w_s l_s, reduced over the group
// with shuffles.  The host picks G so that a lane sees at most 8 splits (up
// to 512 splits), so the records and accumulators arrive in one round trip.
constexpr int kMergeThreads = 256;
template <int D>
__global__ __launch_bounds__(kMergeThreads) void attention_merge(const AttnArgs a, int glog) {
    constexpr int C4 = D / 4;
    const int G = 1 << glog;
    const int j = threadIdx.x & (G - 1);
    const int e = (blockIdx.x * kMergeThreads + threadIdx.x) >> glog;
    if (e >= a.M * C4) return;  // whole groups leave together
    const int q = e / C4;
    const int S = a.splits;
    const float2* ml = reinterpret_cast<const float2*>(a.part_ml) + q;
    const float4* acc = reinterpret_cast<const float4*>(a.part_acc) + e;
    const size_t ml_stride = static_cast<size_t>(a.M);
    const size_t acc_stride = static_cast<size_t>(a.M) * C4;
    // One pass: each chunk's records and accumulators are loaded together
    // (one round trip per 8 splits a lane takes; one in all when the splits
    // fit), the lane keeps a running max mr and rescales, then the group
    // combines its lanes by their maxima.
    float mr = -INFINITY, L = 0.0f;
    float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = j; s0 < S; s0 += 8 * G) {
        float4 x[8];
        float2 y[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const size_t sp = static_cast<size_t>(min(s0 + u * G, S - 1));
            x[u] = acc[sp * acc_stride];
            y[u] = ml[sp * ml_stride];
        }
        float cm = mr;
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (s0 + u * G < S) cm = fmaxf(cm, y[u].x);
        const float c = cm == mr ? 1.0f : fast_exp2(mr - cm);
        L *= c;
        A.x *= c;
        A.y *= c;
        A.z *= c;
        A.w *= c;
        mr = cm;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float w = s0 + u * G < S && cm != -INFINITY ? fast_exp2(y[u].x - cm) : 0.0f;
            L = fmaf(y[u].y, w, L);
            A.x = fmaf(x[u].x, w, A.x);
            A.y = fmaf(x[u].y, w, A.y);
            A.z = fmaf(x[u].z, w, A.z);
            A.w = fmaf(x[u].w, w, A.w);
        }
    }
    float mx = mr;
    for (int off = 1; off < G; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    {
        const float c = mr == -INFINITY ? 0.0f : fast_exp2(mr - mx);
        L *= c;
        A.x *= c;
        A.y *= c;
        A.z *= c;
        A.w *= c;
    }
    for (int off = 1; off < G; off <<= 1) {
        L += __shfl_xor(L, off);
        A.x += __shfl_xor(A.x, off);
        A.y += __shfl_xor(A.y, off);
        A.z += __shfl_xor(A.z, off);
        A.w += __shfl_xor(A.w, off);
    }
    if (j == 0) {
        const float inv = 1.0f / L;
        reinterpret_cast<float4*>(a.out)[e] = make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
    }
}

template <int D, int W>
__global__ __launch_bounds__(W* kWave) void attention_mfma(const AttnArgs a) {
    constexpr int DQ = D / 4;   // contraction dims per lane group in QK
    constexpr int NB = D / 16;  // 16-dim output blocks; block c row m = dim NB * m + c
    static_assert(NB % 4 == 0 || NB == 2, "V operand / output vector width");
    constexpr int KS = D + 4;   // LDS row stride in floats (16-byte pad: conflict-free row reads)
    constexpr int AK = attention_tile<D>();  // keys per tile
    constexpr int KB = AK / 16;              // 16-key blocks per tile
    constexpr int NL = AK * D / 4 / (W * kWave);  // float4 per thread per tile per tensor
    static_assert(NL >= 1 && AK % 16 == 0, "tile load shape");
    __shared__ __align__(16) float s_kv[2][2 * AK * KS];  // two (K tile, V tile) buffers
    int cur = 0;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int split = blockIdx.y;
    const int q0 = blockIdx.x * (16 * W) + wave * 16;
    const int k0 = split * a.chunk;
    const int k1 = min(a.N, k0 + a.chunk);

    // This wave's q^T operand: lane holds q[q0 + r][g * DQ + s], scaled.
    float qv[DQ];
    {
        const float* qp = a.q + static_cast<size_t>(min(q0 + r, a.M - 1)) * D + g * DQ;
#pragma unroll
        for (int j = 0; j < DQ / 4; j++) {
            const float4 x = *reinterpret_cast<const float4*>(qp + 4 * j);
            qv[4 * j] = x.x * a.scale_log2;
            qv[4 * j + 1] = x.y * a.scale_log2;
            qv[4 * j + 2] = x.z * a.scale_log2;
            qv[4 * j + 3] = x.w * a.scale_log2;
        }
    }
    f32x4 o[NB];
#pragma unroll
    for (int c = 0; c < NB; c++) o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    // Tile loads: float4 f = threadIdx.x + j * (64 W) of the AK x D tile.
    float4 pk[NL], pv[NL];
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int j = 0; j < NL; j++) {
            const int f = threadIdx.x + j * W * kWave;
            const int row = f / (D / 4);
            const int c4 = f - row * (D / 4);
            const int key = t0 + row;
            // Rows past the split's end read its last row (in bounds) and are
            // zeroed by a select.
            const size_t kr = static_cast<size_t>(min(key, k1 - 1)) * D + 4 * c4;
            const float keep = key < k1 ? 1.0f : 0.0f;
            const float4 x = *reinterpret_cast<const float4*>(a.k + kr);
            const float4 y = *reinterpret_cast<const float4*>(a.v + kr);
            pk[j] = make_float4(x.x * keep, x.y * keep, x.z * keep, x.w * keep);
            pv[j] = make_float4(y.x * keep, y.y * keep, y.z * keep, y.w * keep);
        }
    };
    auto store_tile = [&](int buf) {
        float* const s_k = s_kv[buf];
        float* const s_v = s_kv[buf] + AK * KS;
#pragma unroll
        for (int j = 0; j < NL; j++) {
            const int f = threadIdx.x + j * W * kWave;
            const int row = f / (D / 4);
            const int c4 = f - row * (D / 4);
            *reinterpret_cast<float4*>(s_k + row * KS + 4 * c4) = pk[j];
            *reinterpret_cast<float4*>(s_v + row * KS + 4 * c4) = pv[j];
        }
    };

    // Tile t is computed from LDS buffer t % 2 while tile t + 1 waits in
    // registers (loaded during tile t - 1) and tile t + 2 is loading.
    if (k0 < k1) {
        load_tile(k0);
        store_tile(0);
        if (k0 + AK < k1) load_tile(k0 + AK);
        __syncthreads();
    }
    for (int t0 = k0; t0 < k1; t0 += AK) {
        const float* const s_k = s_kv[cur];
        const float* const s_v = s_kv[cur] + AK * KS;

        // S^T for the KB key blocks: sv[4 kb + i] = score of key t0 + 16 kb + 4 g + i, query r.
        float sv[4 * KB];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
            f32x4 c = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            const float* kr = s_k + (16 * kb + r) * KS + g * DQ;
#pragma unroll
            for (int s4 = 0; s4 < DQ; s4 += 4) {
                const float4 kk = *reinterpret_cast<const float4*>(kr + s4);
                c = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.x, qv[s4], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.y, qv[s4 + 1], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.z, qv[s4 + 2], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.w, qv[s4 + 3], c, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = t0 + 16 * kb + 4 * g + i;
                sv[4 * kb + i] = key < k1 ? c[i] : -INFINITY;
            }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < 4 * KB; j++) mt = fmaxf(mt, sv[j]);
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        const float ms = mn == -INFINITY ? 0.0f : mn;
        const float alpha = fast_exp2(m - ms);
        m = mn;
        l *= alpha;
#pragma unroll
        for (int j = 0; j < 4 * KB; j++) {
            sv[j] = fast_exp2(sv[j] - ms);
            l += sv[j];
        }
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int c = 0; c < NB; c++) o[c] *= alpha;
        }
        // O^T += V^T P^T: step (kb, i) contracts keys 16 kb + 4 g + i (k index g).
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float* vr = s_v + (16 * kb + 4 * g + i) * KS + NB * r;
                float vv[NB];
                if constexpr (NB % 4 == 0) {
#pragma unroll
                    for (int c4 = 0; c4 < NB; c4 += 4) {
                        const float4 x = *reinterpret_cast<const float4*>(vr + c4);
                        vv[c4] = x.x;
                        vv[c4 + 1] = x.y;
                        vv[c4 + 2] = x.z;
                        vv[c4 + 3] = x.w;
                    }
                } else {
                    const float2 x = *reinterpret_cast<const float2*>(vr);
                    vv[0] = x.x;
                    vv[1] = x.y;
                }
#pragma unroll
                for (int c = 0; c < NB; c++)
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[c], sv[4 * kb + i], o[c], 0, 0, 0);
            }
        }
        // The next tile (in registers since the previous iteration) goes to the
        // idle buffer, which every wave finished reading before the last
        // barrier; the tile after it starts loading.  One barrier per tile.
        if (t0 + AK < k1) {
            store_tile(cur ^ 1);
            if (t0 + 2 * AK < k1) load_tile(t0 + 2 * AK);
        }
        __syncthreads();
        cur ^= 1;
    }
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);

    // One split: the normalised output.  Several: the partial record of
    // (split, query) -- unnormalised acc, and (m, l) -- for attention_merge.
    const int q = q0 + r;
    if (q < a.M) {
        const bool whole = a.splits == 1;
        const float inv = whole ? 1.0f / l : 1.0f;
        float* const row = whole ? a.out + static_cast<size_t>(q) * D
                                 : a.part_acc + (static_cast<size_t>(split) * a.M + q) * D;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float* op = row + NB * (4 * g + i);
            if constexpr (NB % 4 == 0) {
#pragma unroll
                for (int c4 = 0; c4 < NB; c4 += 4)
                    *reinterpret_cast<float4*>(op + c4) = make_float4(o[c4][i] * inv, o[c4 + 1][i] * inv,
                                                                      o[c4 + 2][i] * inv, o[c4 + 3][i] * inv);
            } else {
                *reinterpret_cast<float2*>(op) = make_float2(o[0][i] * inv, o[1][i] * inv);
            }
        }
        if (!whole && g == 0)
            *reinterpret_cast<float2*>(a.part_ml + (static_cast<size_t>(split) * a.M + q) * 2) = make_float2(m, l);
    }
}

// attention_direct<D, W, KW>: 9 to 64 queries (16 per wave, W query blocks)
// on the same v_mfma_f32_16x16x4_f32 products as attention_mfma, but with no
// LDS tile and no padded 64-query block: each wave streams keys from global
// memory straight into its MFMA operands, 16 keys per block, the next block
// loading while the current one is computed.  KW waves share a query block's
// split, taking every KW-th block of it, and meet in LDS at the end (part 0
// rescales and adds the others' (m, l, o)), so the grid has KW times the waves
// for the same split records.  Per block a lane loads
//   K[t + r][g * D/4 + s], s < D/4   (its A operand of S^T = K q^T), and
//   V[t + 4 g + i][NB * r + c]        (its A operand of O^T += V^T P^T),
// so every byte of the block is read once per wave, in 16-byte loads that
// cover whole rows per lane group.  The W query blocks of a workgroup read
// the same keys (L2 hits after the first).  Keys past the split's end read its last
// row (in bounds); their scores are -inf and their V values zero.  Splits
// write the (m, l, acc) records attention_merge combines, as attention_mfma.
constexpr int kDirectBlock = 16;  // keys per block
template <int D, int W, int KW>
__global__ __launch_bounds__(W* KW* kWave) void attention_direct(const AttnArgs a) {
    constexpr int DQ = D / 4;
    constexpr int NB = D / 16;
    static_assert(NB % 4 == 0, "V operand width");
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int wq = wave % W;  // query block of this wave
    const int kw = wave / W;  // key part: blocks kw, kw + KW, ... of the split
    const int r = lane & 15;
    const int g = lane >> 4;
    const int split = blockIdx.y;
    const int q0 = blockIdx.x * (16 * W) + wq * 16;
    const int k0 = split * a.chunk;
    const int k1 = min(a.N, k0 + a.chunk);

    float qv[DQ];
    {
        const float* qp = a.q + static_cast<size_t>(min(q0 + r, a.M - 1)) * D + g * DQ;
#pragma unroll
        for (int j = 0; j < DQ / 4; j++) {
            const float4 x = *reinterpret_cast<const float4*>(qp + 4 * j);
            qv[4 * j] = x.x * a.scale_log2;
            qv[4 * j + 1] = x.y * a.scale_log2;
            qv[4 * j + 2] = x.z * a.scale_log2;
            qv[4 * j + 3] = x.w * a.scale_log2;
        }
    }
    f32x4 o[NB];
#pragma unroll
    for (int c = 0; c < NB; c++) o[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    struct Block {
        float4 k[DQ / 4];
        float4 v[4][NB / 4];
    };
    auto load_block = [&](int t, Block& b) {
        const float* kr = a.k + static_cast<size_t>(min(t + r, k1 - 1)) * D + g * DQ;
#pragma unroll
        for (int j = 0; j < DQ / 4; j++) b.k[j] = *reinterpret_cast<const float4*>(kr + 4 * j);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float* vr = a.v + static_cast<size_t>(min(t + 4 * g + i, k1 - 1)) * D + NB * r;
#pragma unroll
            for (int j = 0; j < NB / 4; j++) b.v[i][j] = *reinterpret_cast<const float4*>(vr + 4 * j);
        }
    };

    Block cur;
    load_block(k0 + kw * kDirectBlock, cur);
    for (int t = k0 + kw * kDirectBlock; t < k1; t += KW * kDirectBlock) {
        Block nxt;
        load_block(t + KW * kDirectBlock, nxt);  // unconditional: past k1 it rereads the last row
        f32x4 c = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < DQ / 4; j++) {
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.k[j].x, qv[4 * j], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.k[j].y, qv[4 * j + 1], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.k[j].z, qv[4 * j + 2], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.k[j].w, qv[4 * j + 3], c, 0, 0, 0);
        }
        // sv[i]: score of key t + 4 g + i for query r.
        float sv[4];
        bool live[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            live[i] = t + 4 * g + i < k1;
            sv[i] = live[i] ? c[i] : -INFINITY;
        }
        float mt = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        const float ms = mn == -INFINITY ? 0.0f : mn;
        const float alpha = fast_exp2(m - ms);
        m = mn;
        l *= alpha;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            sv[i] = fast_exp2(sv[i] - ms);
            l += sv[i];
        }
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int cc = 0; cc < NB; cc++) o[cc] *= alpha;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int j = 0; j < NB / 4; j++) {
                const float4 x = cur.v[i][j];
                const float vv[4] = {live[i] ? x.x : 0.0f, live[i] ? x.y : 0.0f, live[i] ? x.z : 0.0f,
                                     live[i] ? x.w : 0.0f};
#pragma unroll
                for (int e = 0; e < 4; e++)
                    o[4 * j + e] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[e], sv[i], o[4 * j + e], 0, 0, 0);
            }
        }
        cur = nxt;
    }
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if constexpr (KW > 1) {
        // The key parts of a query block meet in LDS: parts 1.. store their
        // (m, l, o) lane by lane, part 0 rescales and adds them.
        __shared__ float s_part[(KW - 1) * W][4 * NB + 2][kWave];
        if (kw > 0) {
            float(*const sp)[kWave] = s_part[(kw - 1) * W + wq];
#pragma unroll
            for (int c = 0; c < NB; c++)
#pragma unroll
                for (int i = 0; i < 4; i++) sp[4 * c + i][lane] = o[c][i];
            sp[4 * NB][lane] = m;
            sp[4 * NB + 1][lane] = l;
        }
        __syncthreads();
        if (kw > 0) return;
#pragma unroll
        for (int p = 0; p < KW - 1; p++) {
            float(*const sp)[kWave] = s_part[p * W + wq];
            const float mp = sp[4 * NB][lane];
            const float mn = fmaxf(m, mp);
            const float ms = mn == -INFINITY ? 0.0f : mn;
            const float a0 = fast_exp2(m - ms), a1 = fast_exp2(mp - ms);
            l = l * a0 + sp[4 * NB + 1][lane] * a1;
#pragma unroll
            for (int c = 0; c < NB; c++)
#pragma unroll
                for (int i = 0; i < 4; i++) o[c][i] = o[c][i] * a0 + sp[4 * c + i][lane] * a1;
            m = mn;
        }
    }

    const int q = q0 + r;
    if (q < a.M) {
        const bool whole = a.splits == 1;
        const float inv = whole ? 1.0f / l : 1.0f;
        float* const row = whole ? a.out + static_cast<size_t>(q) * D
                                 : a.part_acc + (static_cast<size_t>(split) * a.M + q) * D;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float* op = row + NB * (4 * g + i);
#pragma unroll
            for (int c4 = 0; c4 < NB; c4 += 4)
                *reinterpret_cast<float4*>(op + c4) =
                    make_float4(o[c4][i] * inv, o[c4 + 1][i] * inv, o[c4 + 2][i] * inv, o[c4 + 3][i] * inv);
        }
        if (!whole && g == 0)
            *reinterpret_cast<float2*>(a.part_ml + (static_cast<size_t>(split) * a.M + q) * 2) = make_float2(m, l);
    }
}

// attention_rows<D, QM>: up to QM <= 8 queries (decode-shaped attention) on
// the VALU, with no LDS tiles and no padded query block.  A key row is held by
// a group of L lanes, each with E = D/L of its dims: float4 number j·L + lane
// of the row, for j < E/4, so each load instruction reads 16·L contiguous
// bytes per group.  A wave covers 64/L keys per load and keeps 4 loads of K
// and 4 of V in flight per lane (8 KB per wave at any D), so a wave step is
// 1024/D keys whatever L is.  Each key group keeps its own online-softmax
// state per query; its scores are sums over the group's lanes (DPP within a
// 16-lane row, ds_bpermute across rows).  L = D/4 (4 dims per lane), except
// D/8 (8 dims per lane) at d >= 128 with 4-8 queries: there the per-key
// cross-row sums dominated the ALU time (N = 65536, d = 128, M = 8: 31.7 ->
// 23.4 us; d = 256, M = 4: 45.0 -> 29.0 us); with 1-2 queries 4 dims per lane
// ran faster, and 16 dims per lane (one key per lane and step) slower still.
// The epilogue merges the groups of a wave (shuffles), then the waves
// (LDS), and writes the output, or the split's (m, l, acc) record for
// attention_merge.
// Waves per workgroup: 4 (one per SIMD; about 32 KB of K/V in flight per
// CU, the streaming optimum), or 8 for one query over short splits, where two
// waves per SIMD hide more of each split's start (M = 1, N = 65536: d = 128
// 13.52 against 13.74 us, d = 64 8.63 against 9.10 us; at 1024 keys per split
// and more 8 waves ran slower, N = 2^20: 157.2 against 151.9 us, and at 32-64
// keys per split no faster).
constexpr int kRowsWaves = 4;
constexpr int kRowsWavesShort = 8;
constexpr int kRowsShortMin = 128, kRowsShortMax = 512;  // keys per split that take kRowsWavesShort waves (one query)
constexpr int kRowsLoads = 4;  // float4 loads of K (and of V) in flight per lane
constexpr int kRowsMaxQueries = kAttnRowsBlock;
template <int D, int QM, int W = kRowsWaves>
struct RowsShape {
    static constexpr int L = QM >= 4 && D >= 128 ? D / 8 : D / 4;  // lanes per key row
    static constexpr int E = D / L;                              // dims per lane
    static constexpr int NV = E / 4;                             // float4 loads per row per lane
    static constexpr int U = kRowsLoads / NV;                    // keys per lane per step
    static constexpr int KW = kWave / L;                         // keys per wave load
    static constexpr int T = W * KW * U;                         // keys per workgroup step
    static_assert(T == W * 1024 / D, "a wave step is 1024/D keys at any group width");
};
template <int D, int QM>
constexpr int rows_tile() {
    return RowsShape<D, QM>::T;  // the 4-wave step, which sizes the splits
}

template <int L>
__device__ __forceinline__ float key_sum(float x) {
    if constexpr (L <= 16) {
        return group_sum<L>(x);
    } else {
        x = group_sum<16>(x);
        x += __shfl_xor(x, 16);
        if constexpr (L == 64) x += __shfl_xor(x, 32);
        return x;
    }
}

typedef float f32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 load_row16(const float* p) {
    const f32x4v t = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(p));
    return make_float4(t.x, t.y, t.z, t.w);
}

template <int D, int QM, int W>
__global__ __launch_bounds__(W* kWave) void attention_rows(const AttnArgs a) {
    using S = RowsShape<D, QM, W>;
    constexpr int L = S::L, E = S::E, NV = S::NV, U = S::U, KW = S::KW, T = S::T;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int kg = lane / L;
    const int ds = lane % L;
    const int q0 = blockIdx.x * QM;
    const int split = blockIdx.y;
    const int k0 = split * a.chunk;
    const int k1 = min(a.N, k0 + a.chunk);

    // Element 4j + i of a lane's dims is dim 4(jL + ds) + i.
    float qv[QM][E], acc[QM][E], m[QM], l[QM];
#pragma unroll
    for (int qi = 0; qi < QM; qi++) {
        const int q = q0 + qi;
#pragma unroll
        for (int j = 0; j < NV; j++) {
            const float4 x = q < a.M ? *reinterpret_cast<const float4*>(a.q + static_cast<size_t>(q) * D + 4 * (j * L + ds))
                                     : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            qv[qi][4 * j] = x.x * a.scale_log2;
            qv[qi][4 * j + 1] = x.y * a.scale_log2;
            qv[qi][4 * j + 2] = x.z * a.scale_log2;
            qv[qi][4 * j + 3] = x.w * a.scale_log2;
        }
        m[qi] = -INFINITY;
        l[qi] = 0.0f;
#pragma unroll
        for (int e = 0; e < E; e++) acc[qi][e] = 0.0f;
    }

    for (int base = k0 + wave * KW * U; base < k1; base += T) {
        float kr[U][E], vr[U][E];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int t = base + u * KW + kg;
            ok[u] = t < k1;
            const size_t row = static_cast<size_t>(ok[u] ? t : k1 - 1) * D + 4 * ds;
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const float4 x = load_row16(a.k + row + 4 * L * j);
                const float4 y = load_row16(a.v + row + 4 * L * j);
                kr[u][4 * j] = x.x; kr[u][4 * j + 1] = x.y; kr[u][4 * j + 2] = x.z; kr[u][4 * j + 3] = x.w;
                vr[u][4 * j] = y.x; vr[u][4 * j + 1] = y.y; vr[u][4 * j + 2] = y.z; vr[u][4 * j + 3] = y.w;
            }
        }
#pragma unroll
        for (int qi = 0; qi < QM; qi++) {
            float s[U];
            float mx = m[qi];
#pragma unroll
            for (int u = 0; u < U; u++) {
                float dot = qv[qi][0] * kr[u][0];
#pragma unroll
                for (int e = 1; e < E; e++) dot = fmaf(qv[qi][e], kr[u][e], dot);
                s[u] = key_sum<L>(dot);
                if (ok[u]) mx = fmaxf(mx, s[u]);
            }
            // mx stays -inf only while the group has seen no key; then every
            // weight below is 0 and the state is unchanged.
            const float c = mx == m[qi] ? 1.0f : fast_exp2(m[qi] - mx);
            l[qi] *= c;
#pragma unroll
            for (int e = 0; e < E; e++) acc[qi][e] *= c;
            m[qi] = mx;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float pw = ok[u] ? fast_exp2(s[u] - mx) : 0.0f;
                l[qi] += pw;
#pragma unroll
                for (int e = 0; e < E; e++) acc[qi][e] = fmaf(pw, vr[u][e], acc[qi][e]);
            }
        }
    }

    // The wave's key groups: lanes ds of every group hold the same dims.
#pragma unroll
    for (int qi = 0; qi < QM; qi++) {
        float mw = m[qi];
#pragma unroll
        for (int off = L; off < kWave; off <<= 1) mw = fmaxf(mw, __shfl_xor(mw, off));
        const float c = m[qi] == -INFINITY ? 0.0f : fast_exp2(m[qi] - mw);
        l[qi] *= c;
#pragma unroll
        for (int e = 0; e < E; e++) acc[qi][e] *= c;
#pragma unroll
        for (int off = L; off < kWave; off <<= 1) {
            l[qi] += __shfl_xor(l[qi], off);
#pragma unroll
            for (int e = 0; e < E; e++) acc[qi][e] += __shfl_xor(acc[qi][e], off);
        }
        m[qi] = mw;
    }

    // The workgroup's waves, through LDS (float4 column c4 = jL + ds).
    __shared__ float2 s_ml[W][QM];
    __shared__ float4 s_acc[W][QM][D / 4];
    if (kg == 0) {
#pragma unroll
        for (int qi = 0; qi < QM; qi++) {
#pragma unroll
            for (int j = 0; j < NV; j++)
                s_acc[wave][qi][j * L + ds] =
                    make_float4(acc[qi][4 * j], acc[qi][4 * j + 1], acc[qi][4 * j + 2], acc[qi][4 * j + 3]);
            if (ds == 0) s_ml[wave][qi] = make_float2(m[qi], l[qi]);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < QM * (D / 4); i += W * kWave) {
        const int qi = i / (D / 4);
        const int c4 = i - qi * (D / 4);
        const int q = q0 + qi;
        if (q >= a.M) continue;
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; w++) mm = fmaxf(mm, s_ml[w][qi].x);
        float ls = 0.0f;
        float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float2 ml = s_ml[w][qi];
            const float c = ml.x == -INFINITY ? 0.0f : fast_exp2(ml.x - mm);
            const float4 x = s_acc[w][qi][c4];
            ls = fmaf(c, ml.y, ls);
            A.x = fmaf(c, x.x, A.x);
            A.y = fmaf(c, x.y, A.y);
            A.z = fmaf(c, x.z, A.z);
            A.w = fmaf(c, x.w, A.w);
        }
        if (a.splits == 1) {
            const float inv = 1.0f / ls;
            *reinterpret_cast<float4*>(a.out + static_cast<size_t>(q) * D + 4 * c4) =
                make_float4(A.x * inv, A.y * inv, A.z * inv, A.w * inv);
        } else {
            const size_t rec = static_cast<size_t>(split) * a.M + q;
            *reinterpret_cast<float4*>(a.part_acc + rec * D + 4 * c4) = A;
            if (c4 == 0) *reinterpret_cast<float2*>(a.part_ml + rec * 2) = make_float2(mm, ls);
        }
    }
}

// Any d <= 1024: one wave per query row; scores of 64 keys per step, one per
// lane (dot over d), online softmax over the steps, accumulator in LDS.
constexpr int kGenWaves = 4;
__global__ __launch_bounds__(kGenWaves* kWave) void attention_generic(const AttnArgs a) {
    extern __shared__ float sh[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int row = blockIdx.x * kGenWaves + wave;
    const int d = a.d;
    float* acc = sh + wave * d;
    if (row >= a.M) return;
    for (int j = lane; j < d; j += kWave) acc[j] = 0.0f;
    const float* q = a.q + static_cast<size_t>(row) * d;
    float m = -INFINITY, l = 0.0f;
    for (int t0 = 0; t0 < a.N; t0 += kWave) {
        const int t = t0 + lane;
        float s = -INFINITY;
        if (t < a.N) {
            const float* k = a.k + static_cast<size_t>(t) * d;
            float dot = 0.0f;
            for (int j = 0; j < d; j++) dot = fmaf(q[j], k[j], dot);
            s = dot * a.scale_log2;
        }
        const float mn = fmaxf(m, wave_max(s));
        const float alpha = fast_exp2(m - mn);
        const float p = fast_exp2(s - mn);
        l = l * alpha + wave_sum(p);
        m = mn;
        const int nt = min(kWave, a.N - t0);
        // Dims in passes of 64 with every lane active, so the shuffles read
        // live lanes; lanes past d carry zeros and store nothing.
        for (int j0 = 0; j0 < d; j0 += kWave) {
            const int j = j0 + lane;
            const bool in = j < d;
            float x = in ? acc[j] * alpha : 0.0f;
            for (int u = 0; u < nt; u++) {
                const float pu = __shfl(p, u);
                x = fmaf(pu, in ? a.v[static_cast<size_t>(t0 + u) * d + j] : 0.0f, x);
            }
            if (in) acc[j] = x;
        }
    }
    for (int j = lane; j < d; j += kWave) a.out[static_cast<size_t>(row) * d + j] = acc[j] / l;
}

}  // namespace

int attention_tuned_dim(int d) { return d == 32 || d == 64 || d == 128 || d == 256; }
int attention_key_tile(int d) { return d >= 256 ? attention_tile<256>() : attention_tile<128>(); }
int attention_max_splits(int) { return kAttnMaxSplits; }
int attention_direct_dim(int d) { return d == 64 || d == 128; }
int attention_rows_queries(int M) {
    if (M <= 1) return 1;
    if (M <= 2) return 2;
    if (M <= 4) return 4;
    return M <= kRowsMaxQueries ? kRowsMaxQueries : 0;
}
template <int D>
int rows_tile_d(int qm) {
    switch (qm) {
        case 1: return rows_tile<D, 1>();
        case 2: return rows_tile<D, 2>();
        case 4: return rows_tile<D, 4>();
        default: return rows_tile<D, kRowsMaxQueries>();
    }
}
int attention_rows_tile(int d, int qm) {
    switch (d) {
        case 32: return rows_tile_d<32>(qm);
        case 64: return rows_tile_d<64>(qm);
        case 128: return rows_tile_d<128>(qm);
        default: return rows_tile_d<256>(qm);
    }
}

namespace {
template <int D, int W>
void launch_mfma_attention(const AttnArgs& a, int glog, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.M + 16 * W - 1) / (16 * W)), static_cast<unsigned>(a.splits));
    hipLaunchKernelGGL((attention_mfma<D, W>), grid, dim3(W * kWave), 0, stream, a);
    if (a.splits > 1) {
        const dim3 mgrid(static_cast<unsigned>(
            ((static_cast<long long>(a.M) * (D / 4) << glog) + kMergeThreads - 1) / kMergeThreads));
        hipLaunchKernelGGL(attention_merge<D>, mgrid, dim3(kMergeThreads), 0, stream, a, glog);
    }
}
template <int D, int QM>
void launch_rows_attention(const AttnArgs& a, int glog, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.M + QM - 1) / QM), static_cast<unsigned>(a.splits));
    // (and at least one 8-wave step per split, so no wave idles: d = 32 from 256 keys)
    if (QM == 1 && a.chunk >= kRowsShortMin && a.chunk >= RowsShape<D, QM, kRowsWavesShort>::T &&
        a.chunk <= kRowsShortMax)
        hipLaunchKernelGGL((attention_rows<D, QM, kRowsWavesShort>), grid, dim3(kRowsWavesShort * kWave), 0, stream, a);
    else
        hipLaunchKernelGGL((attention_rows<D, QM, kRowsWaves>), grid, dim3(kRowsWaves * kWave), 0, stream, a);
    if (a.splits > 1) {
        const dim3 mgrid(static_cast<unsigned>(
            ((static_cast<long long>(a.M) * (D / 4) << glog) + kMergeThreads - 1) / kMergeThreads));
        hipLaunchKernelGGL(attention_merge<D>, mgrid, dim3(kMergeThreads), 0, stream, a, glog);
    }
}
template <int D>
void launch_rows_attention_d(const AttnArgs& a, int glog, hipStream_t stream) {
    switch (a.qblock) {
        case 1: launch_rows_attention<D, 1>(a, glog, stream); break;
        case 2: launch_rows_attention<D, 2>(a, glog, stream); break;
        case 4: launch_rows_attention<D, 4>(a, glog, stream); break;
        default: launch_rows_attention<D, kRowsMaxQueries>(a, glog, stream); break;
    }
}
template <int D, int W, int KW>
void launch_direct_attention(const AttnArgs& a, int glog, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((a.M + 16 * W - 1) / (16 * W)), static_cast<unsigned>(a.splits));
    hipLaunchKernelGGL((attention_direct<D, W, KW>), grid, dim3(W * KW * kWave), 0, stream, a);
    if (a.splits > 1) {
        const dim3 mgrid(static_cast<unsigned>(
            ((static_cast<long long>(a.M) * (D / 4) << glog) + kMergeThreads - 1) / kMergeThreads));
        hipLaunchKernelGGL(attention_merge<D>, mgrid, dim3(kMergeThreads), 0, stream, a, glog);
    }
}
template <int D>
void launch_mfma_attention_d(const AttnArgs& a, int glog, hipStream_t stream) {
    if (a.qblock <= kRowsMaxQueries) {
        launch_rows_attention_d<D>(a, glog, stream);
        return;
    }
    if constexpr (D == 64 || D == 128) {
        if (a.direct) {
            // Up to 32 queries four waves share a query block's split; 33-64
            // queries run as four query blocks of one wave each.
            if (a.qblock == 16) launch_direct_attention<D, 1, 4>(a, glog, stream);
            else if (a.qblock == 32) launch_direct_attention<D, 2, 4>(a, glog, stream);
            else launch_direct_attention<D, 4, 1>(a, glog, stream);
            return;
        }
    }
    if constexpr (D <= 128) {  // at d = 256 a 4-wave block would need over 256 VGPRs
        if (a.qblock == kAttnBlockNarrow) {
            launch_mfma_attention<D, kAttnBlockNarrow / 16>(a, glog, stream);
            return;
        }
    }
    launch_mfma_attention<D, kAttnBlockWide / 16>(a, glog, stream);
}
}  // namespace

hipError_t launch_attention(const AttnArgs& a, hipStream_t stream) {
    if (a.tuned && attention_tuned_dim(a.d)) {
        int glog = 0;  // lanes per merge group: at most 8 splits per lane, at most a wave
        while (glog < 6 && ((a.splits - 1) >> glog) >= 8) glog++;
        switch (a.d) {
            case 32: launch_mfma_attention_d<32>(a, glog, stream); break;
            case 64: launch_mfma_attention_d<64>(a, glog, stream); break;
            case 128: launch_mfma_attention_d<128>(a, glog, stream); break;
            default: launch_mfma_attention_d<256>(a, glog, stream); break;
        }
        return hipGetLastError();
    }
    const dim3 grid(static_cast<unsigned>((a.M + kGenWaves - 1) / kGenWaves));
    const size_t lds = sizeof(float) * kGenWaves * static_cast<size_t>(a.d);
    hipLaunchKernelGGL(attention_generic, grid, dim3(kGenWaves * kWave), lds, stream, a);
    return hipGetLastError();
}

}  // namespace kvq
