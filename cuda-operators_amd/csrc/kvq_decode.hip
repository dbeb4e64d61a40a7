// kvq_decode.hip -- gfx950 decode-attention kernels over an int8 K/V cache.
//
// Math (per query head, the reference's cpu_reference,
// kv_cache/KV_int8_split_optimized.cu:385-437): s_t = (q . K_t) * k_scale_t *
// softmax_scale, p = softmax(s), out = sum_t p_t * V_t * v_scale_t.  Scores are
// kept in log2 units (softmax_scale * log2 e folded into one multiplier) so
// every exponential is one v_exp_f32.
//
// decode_fast<D, SG>: one workgroup (8 waves) per (sequence split, batch,
//   kv head, group of SG query heads).  A token's D-byte K row is read by D/16
//   lanes with one 16-byte load each, so one wave load covers 64*16 contiguous
//   bytes (several whole rows).  Each lane dequantises its 16 bytes in
//   registers (SDWA sign-extended byte converts), forms 16-element partial dots
//   for its SG query heads and finishes them with DPP row sums over the token's
//   lane group.  Every lane group keeps its own online-softmax state (max, sum,
//   16 accumulators per head) with no cross-lane traffic per token; states are
//   merged across lane groups (ds_bpermute), then across waves (LDS), once per
//   workgroup.  Each K/V byte is read once per kv head: the SG query heads of a
//   group share the loads.
//   A sequence longer than one chunk is split; each split writes a partial
//   (max, sum, acc[D]) record, and the last split to finish (device-scope
//   arrival counter) merges the records with a log-sum-exp reduction, so the
//   whole decode is a single kernel.  Without counters (caller scratch of
//   unknown contents) merge_kernel does the merge instead.
//   Optionally wave 0 of the workgroup owning a sequence's last token
//   quantises that token from fp32 (append) after its tiles, with no
//   workgroup barrier, and attends to it from registers.
//
// decode_generic: any head dim up to KVQ_MAX_HEAD_DIM and any alignment; one
//   wave per (split, batch, query head), q and the accumulators in LDS.  It is
//   the correctness path for shapes the tuned kernel does not cover.
#include <math.h>

#include "kvq_device.hpp"
#include "kvq_internal.hpp"
#include "kvq_split.hpp"

namespace kvq {
namespace {

// Ranges of at least this many workgroup blocks give their last block to the
// first wave of each SIMD (see the tile loop of decode_fast).
constexpr int kRebalanceBlocks = 8;
#ifndef KVQ_FAST_WAVES
#define KVQ_FAST_WAVES 8
#endif
constexpr int kFastWaves = KVQ_FAST_WAVES;  // waves per workgroup

// Tile geometry: D/16 lanes share a token (16 bytes each); U tokens per lane
// group per loop iteration.  U = 2 keeps ~32 KB of K/V loads in flight per CU
// (8 waves x 2 x 2 KB), which measured fastest on MI355X: at U = 4 (64 KB) the
// same kernel streams ~4% slower, at U = 8 ~15% slower, at U = 1 too little
// is in flight.
template <int D, int SG>
struct FastGeom {
    static constexpr int LPT = D / 16;                // lanes per token
    static constexpr int TPL = kWave / LPT;           // tokens per wave load
    static constexpr int U = 2;                       // tokens per lane group per iteration
    // Software pipelining (next tile's loads in flight during compute) pays
    // for SG = 4; at SG <= 2 the extra registers cost more than it hides.
    static constexpr bool PIPE = SG >= 4;
    static constexpr int WSTEP = TPL * U;             // tokens per wave iteration
    static constexpr int BSTEP = WSTEP * kFastWaves;  // tokens per workgroup iteration
};

// Online-softmax update of one lane group's state with U tokens (one per load).
template <int SG, int U, int LPT>
__device__ __forceinline__ void attend(const float (&qr)[SG][16], const int4 (&kk)[U],
                                       const int4 (&vv)[U], const float (&kscl)[U],
                                       const float (&vscl)[U], const bool (&ok)[U],
                                       float scale_log2, float (&m)[SG], float (&l)[SG],
                                       float (&acc)[SG][16]) {
    float s[SG][U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        float kf[16];
        unpack16(kk[u], kf);
#pragma unroll
        for (int h = 0; h < SG; h++) {
            float dot = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++) dot = fmaf(qr[h][j], kf[j], dot);
            dot = group_sum<LPT>(dot);
            s[h][u] = ok[u] ? (dot * kscl[u]) * scale_log2 : -INFINITY;
        }
    }
    float w[SG][U];
#pragma unroll
    for (int h = 0; h < SG; h++) {
        float mx = m[h];
#pragma unroll
        for (int u = 0; u < U; u++) mx = fmaxf(mx, s[h][u]);
        const float ms = (mx == -INFINITY) ? 0.0f : mx;
        const float alpha = fast_exp2(m[h] - ms);
        l[h] *= alpha;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {  // the max moved in some lane group
#pragma unroll
            for (int j = 0; j < 16; j++) acc[h][j] *= alpha;
        }
        m[h] = mx;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float p = fast_exp2(s[h][u] - ms);
            l[h] += p;
            w[h][u] = p * vscl[u];
        }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        float vf[16];
        unpack16(vv[u], vf);
#pragma unroll
        for (int h = 0; h < SG; h++) {
#pragma unroll
            for (int j = 0; j < 16; j++) acc[h][j] = fmaf(w[h][u], vf[j], acc[h][j]);
        }
    }
}

template <int D, int SG, bool PAGED, bool FIT>
__global__ __launch_bounds__(kFastWaves* kWave) void decode_fast(const DecodeArgs a) {
    using Geo = FastGeom<D, SG>;
    constexpr int LPT = Geo::LPT;
    constexpr int U = Geo::U;
    constexpr int NE = (2 * D + kWave - 1) / kWave;  // appended K+V elements per lane of wave 0
    __shared__ float s_ml[kFastWaves][SG][2];
    __shared__ float s_acc[kFastWaves][SG][D];
    __shared__ __align__(16) int s_newq[2][D / 4];  // appended K and V rows, packed int8
    __shared__ int s_last;
    __shared__ MergeScratch s_merge;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int tg = lane / LPT;  // token slot within a wave load
    const int ds = lane % LPT;  // 16-element slice of the head dim

    SplitWork w;
    if constexpr (FIT) {
        if (!locate_fit(a, w)) return;
    } else {
        if (!locate_work(a, w)) return;
    }
    const int unit = w.unit;
    const int bh = unit / a.nsg;
    const int sgi = unit - bh * a.nsg;
    const int b = bh / a.Hkv;
    const int kvh = bh - b * a.Hkv;
    const int hq0 = kvh * a.G + sgi * SG;
    const size_t bhq0 = static_cast<size_t>(b) * a.Hq + hq0;
    const int len = w.len;
    const int split = w.split;
    const int nsplit = w.nsplit;

    if (len == 0) {
        for (int i = threadIdx.x; i < SG * D; i += blockDim.x) a.out[bhq0 * D + i] = 0.0f;
        return;
    }

    const int t0 = w.t0;
    const int t1 = w.t1;
    const bool app = (a.k_new != nullptr) && (t1 == len);
    const int tend = app ? t1 - 1 : t1;  // tokens read from the cache

    // Fused append, part 1: wave 0 fetches the new token (element e = lane +
    // 64 j of the K row then the V row) first, so the loads overlap the rest.
    float xnew[NE];
#pragma unroll
    for (int j = 0; j < NE; j++) {
        const int e = lane + j * kWave;
        xnew[j] = 0.0f;
        if (app && wave == 0 && e < 2 * D)
            xnew[j] = (e < D ? a.k_new : a.v_new)[static_cast<size_t>(bh) * D + (e < D ? e : e - D)];
    }

    float qr[SG][16];
#pragma unroll
    for (int h = 0; h < SG; h++) {
        const float4* qp = reinterpret_cast<const float4*>(a.q + (bhq0 + h) * D + ds * 16);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 x = qp[j];
            qr[h][4 * j + 0] = x.x;
            qr[h][4 * j + 1] = x.y;
            qr[h][4 * j + 2] = x.z;
            qr[h][4 * j + 3] = x.w;
        }
    }
    float m[SG], l[SG], acc[SG][16];
#pragma unroll
    for (int h = 0; h < SG; h++) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) acc[h][j] = 0.0f;
    }

    // Cache rows (K/V row at byte row * D, scale at element row).  A wave
    // tile's WSTEP tokens are consecutive rows in either layout: paged caches
    // run here only with power-of-two pages that are a multiple of WSTEP.
    const size_t row0 = static_cast<size_t>(bh) * a.cap;

    // Main loop.  Lane group tg owns the U consecutive tokens base + tg*U + u,
    // so each 16-byte K/V load instruction still covers whole 128-byte rows
    // and the U scales of a lane group come in one 16-byte load per scale
    // array.  With PIPE the loads of a wave's next tile are in flight while
    // the current tile is computed.
    struct Tile {
        int4 k[U], v[U];
        float ks[U], vs[U];
    };
    auto load_tile = [&](Tile& T, int base, size_t r) {  // r: row of token `base`
        const int8_t* kp = a.k + r * D + ds * 16;
        const int8_t* vp = a.v + r * D + ds * 16;
        const float* ksp = a.ks + r;
        const float* vsp = a.vs + r;
        const int t_first = base + tg * U;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int tc = min(t_first + u, tend - 1) - base;
            T.k[u] = load16_stream(kp + static_cast<ptrdiff_t>(tc) * D);
            T.v[u] = load16_stream(vp + static_cast<ptrdiff_t>(tc) * D);
        }
        const float* ksu = ksp + (t_first - base);
        const float* vsu = vsp + (t_first - base);
        const bool vec_ok = ((reinterpret_cast<uintptr_t>(ksu) | reinterpret_cast<uintptr_t>(vsu)) &
                             (sizeof(float) * U - 1)) == 0;
        if (t_first + U <= tend && vec_ok) {
            load_scales<U>(ksu, T.ks);
            load_scales<U>(vsu, T.vs);
        } else {
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int tc = min(t_first + u, tend - 1) - base;
                T.ks[u] = ksp[tc];
                T.vs[u] = vsp[tc];
            }
        }
    };
    auto run_tile = [&](const Tile& T, int base) {
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; u++) ok[u] = base + tg * U + u < tend;
        attend<SG, U, LPT>(qr, T.k, T.v, T.ks, T.vs, ok, a.scale_log2, m, l, acc);
    };
    int base = t0 + __builtin_amdgcn_readfirstlane(wave) * Geo::WSTEP;  // wave-uniform
    // In a paged cache (power-of-two pages here) the next tile's block-table
    // entry is fetched one tile ahead and only turned into a row when that tile
    // loads, so the load's latency stays off the load path.  It is a vector
    // load: vector loads complete in order, so the wait for it leaves the
    // tile loads issued after it in flight (a scalar load shares its counter
    // with LDS traffic and comes back out of order).  The index is clamped to
    // this sequence's last token: the table is never read past the sequence's
    // own entries.
    const buf_rsrc tabr =
        make_rsrc(PAGED ? a.pages.table + static_cast<size_t>(b) * a.pages.max_pages : nullptr,
                  PAGED ? static_cast<unsigned>(a.pages.max_pages) * 4u : 0u);
    auto page_entry = [&](int t) -> int {
        if constexpr (PAGED)
            return __builtin_amdgcn_raw_buffer_load_b32(tabr, (min(t, tend - 1) >> a.pages.shift) * 4, 0, 0);
        else return 0;
    };
    int pg_next = page_entry(base);
    auto row_of = [&](int tb, int nb) -> size_t {  // row of the tile at tb; prefetch the entry of nb
        if constexpr (PAGED) {
            const int page = min(max(__builtin_amdgcn_readfirstlane(pg_next), 0), a.pages.num_pages - 1);
            pg_next = page_entry(nb);
            return (static_cast<size_t>(page) * a.Hkv + kvh) * a.pages.size + (tb & (a.pages.size - 1));
        } else {
            return row0 + tb;
        }
    };
    auto next_row = [&](int nb) -> size_t { return row_of(nb - Geo::BSTEP, nb); };
    if constexpr (!Geo::PIPE) {
        // The two waves that share a SIMD do not stream at the same rate: the
        // first one dispatched (waves 0 .. kFastWaves/2 - 1) wins issue
        // arbitration and ends its tile loop ~1.6 us before its partner at
        // cfg1.  In ranges of kRebalanceBlocks blocks or more, the last block
        // therefore goes to the first waves alone, two steps each (a fixed
        // assignment: outputs stay bit-reproducible); shorter ranges keep
        // every wave busy instead.  Measured and applied at SG = 1 only (at
        // SG = 2 the extra code took some instantiations past 128 VGPRs).
        const int nblk = (tend - t0 + Geo::BSTEP - 1) / Geo::BSTEP;
        const int lastb = SG == 1 && nblk >= kRebalanceBlocks ? t0 + (nblk - 1) * Geo::BSTEP : tend;
        for (; base < lastb; base += Geo::BSTEP) {
            Tile tt;
            load_tile(tt, base, next_row(base + Geo::BSTEP));
            run_tile(tt, base);
        }
        const int wvu = __builtin_amdgcn_readfirstlane(wave);
        if (lastb < tend && wvu < kFastWaves / 2) {
            // base == lastb + wvu * WSTEP, whose page entry the loop prefetched
            const int b1 = base + (kFastWaves / 2) * Geo::WSTEP;
            if (base < tend) {
                Tile tt;
                load_tile(tt, base, row_of(base, b1));
                run_tile(tt, base);
            }
            if (b1 < tend) {
                Tile tt;
                load_tile(tt, b1, row_of(b1, b1 + Geo::BSTEP));
                run_tile(tt, b1);
            }
        }
    } else {
        Tile ta, tb;
        if (base < tend) load_tile(ta, base, next_row(base + Geo::BSTEP));
        while (base < tend) {
            int nb = base + Geo::BSTEP;
            if (nb < tend) load_tile(tb, nb, next_row(nb + Geo::BSTEP));
            run_tile(ta, base);
            base = nb;
            if (base >= tend) break;
            nb = base + Geo::BSTEP;
            if (nb < tend) load_tile(ta, nb, next_row(nb + Geo::BSTEP));
            run_tile(tb, base);
            base = nb;
        }
    }

    if (app && wave == 0) {
        // Fused append, part 2 (wave 0 alone, no workgroup barrier): per-row
        // max|x|, the scale, the quantised elements (same rule and bits as
        // append_kernel) into LDS, read back in the attend layout; one store
        // of the token per kv head, and lane group 0 attends to it.
        float mk = 0.0f, mv = 0.0f;
#pragma unroll
        for (int j = 0; j < NE; j++) {
            const int e = lane + j * kWave;
            if (e < D) mk = fmaxf(mk, fabsf(xnew[j]));
            else if (e < 2 * D) mv = fmaxf(mv, fabsf(xnew[j]));
        }
        const float sk = quant_scale(wave_max(mk)), sv = quant_scale(wave_max(mv));
#pragma unroll
        for (int j = 0; j < NE; j++) {
            const int e = lane + j * kWave;
            if (e < 2 * D) {
                const int row = e < D ? 0 : 1;
                reinterpret_cast<int8_t*>(s_newq[row])[e - row * D] =
                    static_cast<int8_t>(quant_one(xnew[j], row ? sv : sk));
            }
        }
        int4 kk1[1], vv1[1];
        kk1[0] = *reinterpret_cast<const int4*>(&s_newq[0][ds * 4]);
        vv1[0] = *reinterpret_cast<const int4*>(&s_newq[1][ds * 4]);
        const float sk1[1] = {sk}, sv1[1] = {sv};
        const int tnew = len - 1;
        if (sgi == 0 && tg == 0) {
            const size_t rn = PAGED ? cache_row(a.pages, a.Hkv, a.cap, b, kvh, tnew) : row0 + tnew;
            *reinterpret_cast<int4*>(a.k + rn * D + ds * 16) = kk1[0];
            *reinterpret_cast<int4*>(a.v + rn * D + ds * 16) = vv1[0];
            if (ds == 0) {
                a.ks[rn] = sk;
                a.vs[rn] = sv;
            }
        }
        const bool ok1[1] = {tg == 0};
        attend<SG, 1, LPT>(qr, kk1, vv1, sk1, sv1, ok1, a.scale_log2, m, l, acc);
    }

    // Merge the lane groups of this wave (lanes that share ds).
#pragma unroll
    for (int off = LPT; off < kWave; off <<= 1) {
#pragma unroll
        for (int h = 0; h < SG; h++) {
            const float mo = __shfl_xor(m[h], off);
            const float lo = __shfl_xor(l[h], off);
            const float mx = fmaxf(m[h], mo);
            const float ms = (mx == -INFINITY) ? 0.0f : mx;
            const float a1 = fast_exp2(m[h] - ms), a2 = fast_exp2(mo - ms);
            l[h] = l[h] * a1 + lo * a2;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float ao = __shfl_xor(acc[h][j], off);
                acc[h][j] = acc[h][j] * a1 + ao * a2;
            }
            m[h] = mx;
        }
    }
    if (tg == 0) {
#pragma unroll
        for (int h = 0; h < SG; h++) {
#pragma unroll
            for (int j = 0; j < 16; j++) s_acc[wave][h][ds * 16 + j] = acc[h][j];
            if (ds == 0) {
                s_ml[wave][h][0] = m[h];
                s_ml[wave][h][1] = l[h];
            }
        }
    }
    __syncthreads();

    // Merge the waves; one thread per (head, element).
    RecMap map{0, 0, 0};
    if (nsplit > 1) {
        map = rec_map(a, w, bhq0);
    }
    for (int i = threadIdx.x; i < SG * D; i += blockDim.x) {
        const int h = i / D;
        const int dim = i - h * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kFastWaves; w++) M = fmaxf(M, s_ml[w][h][0]);
        const float Ms = (M == -INFINITY) ? 0.0f : M;
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kFastWaves; w++) {
            const float f = fast_exp2(s_ml[w][h][0] - Ms);
            L = fmaf(s_ml[w][h][1], f, L);
            A = fmaf(s_acc[w][h][dim], f, A);
        }
        store_result(a, map, bhq0, h, dim, split, nsplit, M, L, A);
    }
    finish_split(a, unit, map, bhq0, SG, nsplit, &s_last, s_merge);
}

// Log-sum-exp merge of one element over nsplit records, 8 splits' (m, l, acc)
// loaded together per step with a running max (one round trip per 8 splits,
// where a load-max-then-accumulate loop waits on every record in turn).
// Every split holds at least one token, so every record's m is finite.
__device__ inline float merge_dim_pipelined(const DecodeArgs& a, const RecMap& map, int dim, int nsplit) {
    constexpr int kStep = 8;
    float M = -INFINITY, L = 0.0f, A = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += kStep) {
        float m[kStep], l[kStep], x[kStep];
#pragma unroll
        for (int u = 0; u < kStep; u++) {
            const size_t rec = map.r0 + static_cast<size_t>(min(s0 + u, nsplit - 1)) * map.ss;
            m[u] = get_coherent(a.part_ml + rec * 2);
            l[u] = get_coherent(a.part_ml + rec * 2 + 1);
            x[u] = get_coherent(a.part_acc + rec * a.d + dim);
        }
        float cm = M;
#pragma unroll
        for (int u = 0; u < kStep; u++)
            if (s0 + u < nsplit) cm = fmaxf(cm, m[u]);
        const float c = fast_exp2(M - cm);  // 0 on the first step (M = -inf)
        L *= c;
        A *= c;
        M = cm;
#pragma unroll
        for (int u = 0; u < kStep; u++) {
            const float w = s0 + u < nsplit ? fast_exp2(m[u] - cm) : 0.0f;
            L = fmaf(l[u], w, L);
            A = fmaf(x[u], w, A);
        }
    }
    return A / L;
}

__global__ __launch_bounds__(256) void merge_kernel(const DecodeArgs a) {
    const int bhq = blockIdx.x;
    const int b = bhq / a.Hq;
    const int len = seq_len_of(a, b);
    const int nsplit = (len + a.chunk - 1) / a.chunk;
    if (nsplit <= 1) return;  // written directly by the decode kernel
    const RecMap map = rec_map_static(a, bhq);
    for (int dim = threadIdx.x; dim < a.d; dim += blockDim.x)
        a.out[static_cast<size_t>(bhq) * a.d + dim] = merge_dim_pipelined(a, map, dim, nsplit);
}

__global__ __launch_bounds__(kWave) void decode_generic(const DecodeArgs a) {
    extern __shared__ float sh[];
    float* qs = sh;
    float* accs = sh + a.d;
    const int lane = threadIdx.x;
    const int bhqn = a.B * a.Hq;
    const int split = blockIdx.x / bhqn;
    const int bhq = blockIdx.x - split * bhqn;
    const int b = bhq / a.Hq;
    const int hq = bhq - b * a.Hq;
    const int kvh = hq / a.G;
    const int d = a.d;
    const int len = seq_len_of(a, b);
    const int nsplit = (len + a.chunk - 1) / a.chunk;
    float* outp = a.out + static_cast<size_t>(bhq) * d;
    if (len == 0) {
        if (split == 0)
            for (int i = lane; i < d; i += kWave) outp[i] = 0.0f;
        return;
    }
    if (split >= nsplit) return;
    const int t0 = split * a.chunk;
    const int t1 = min(len, t0 + a.chunk);

    for (int i = lane; i < d; i += kWave) {
        qs[i] = a.q[static_cast<size_t>(bhq) * d + i];
        accs[i] = 0.0f;
    }
    __syncthreads();

    float m = -INFINITY, l = 0.0f;
    for (int t = t0; t < t1; t++) {
        const size_t row = cache_row(a.pages, a.Hkv, a.cap, b, kvh, t);
        const int8_t* kr = a.k + row * d;
        const int8_t* vr = a.v + row * d;
        float dot = 0.0f;
        for (int i = lane; i < d; i += kWave) dot = fmaf(qs[i], static_cast<float>(kr[i]), dot);
        dot = wave_sum(dot);
        const float s = (dot * a.ks[row]) * a.scale_log2;
        const float mx = fmaxf(m, s);
        const float alpha = fast_exp2(m - mx);
        const float p = fast_exp2(s - mx);
        l = l * alpha + p;
        const float w = p * a.vs[row];
        for (int i = lane; i < d; i += kWave) accs[i] = fmaf(w, static_cast<float>(vr[i]), accs[i] * alpha);
        m = mx;
    }
    if (nsplit == 1) {
        for (int i = lane; i < d; i += kWave) outp[i] = accs[i] / l;
    } else {
        const size_t rec = static_cast<size_t>(bhq) * a.splits + split;
        for (int i = lane; i < d; i += kWave) a.part_acc[rec * d + i] = accs[i];
        if (lane == 0) {
            a.part_ml[rec * 2] = m;
            a.part_ml[rec * 2 + 1] = l;
        }
    }
}

template <int D, int SG>
void launch_fast_sg(const DecodeArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
    // The in-kernel split plan (locate_fit) is built for SG <= 2 only: with
    // more heads per group the matrix-core kernel takes d = 128.
    if constexpr (SG <= 2) {
        if (a.fit_items > 0) {
            if (a.pages.table) hipLaunchKernelGGL((decode_fast<D, SG, true, true>), grid, block, 0, stream, a);
            else hipLaunchKernelGGL((decode_fast<D, SG, false, true>), grid, block, 0, stream, a);
            return;
        }
    }
    if (a.pages.table) hipLaunchKernelGGL((decode_fast<D, SG, true, false>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((decode_fast<D, SG, false, false>), grid, block, 0, stream, a);
}

template <int D>
hipError_t launch_fast_d(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(decode_grid(a, p)));
    const dim3 block(kFastWaves * kWave);
    switch (p.sg) {
        case 1: launch_fast_sg<D, 1>(a, grid, block, stream); break;
        case 2: launch_fast_sg<D, 2>(a, grid, block, stream); break;
        case 4: launch_fast_sg<D, 4>(a, grid, block, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

template <int SG>
int tile_tokens_sg(int d) {
    switch (d) {
        case 32: return FastGeom<32, SG>::BSTEP;
        case 64: return FastGeom<64, SG>::BSTEP;
        case 128: return FastGeom<128, SG>::BSTEP;
        case 256: return FastGeom<256, SG>::BSTEP;
        default: return 0;
    }
}

int fast_tile_tokens(int d, int sg) {
    switch (sg) {
        case 1: return tile_tokens_sg<1>(d);
        case 2: return tile_tokens_sg<2>(d);
        case 4: return tile_tokens_sg<4>(d);
        default: return 0;
    }
}

int fast_wave_tokens(int d, int sg) { return fast_tile_tokens(d, sg) / kFastWaves; }

int fast_heads_per_group(int G) {
    if (G % 4 == 0) return 4;
    if (G % 2 == 0) return 2;
    return 1;
}

hipError_t launch_merge(const DecodeArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(merge_kernel, dim3(static_cast<unsigned>(a.B * a.Hq)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

long decode_grid(const DecodeArgs& a, const DecodePlan& p) {
    const long units = static_cast<long>(a.Hkv) * p.nsg;
    if (p.fit) return units * p.sched_items;
    return p.scheduled ? units * p.sched_items : units * a.B * p.splits;
}

hipError_t launch_decode(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
    hipError_t err;
    if (p.scheduled && !p.lpt) {
        err = launch_schedule(a.lengths, a.B, a.max_len, a.Hkv * p.nsg, p.sched_target, p.sched_gran,
                              p.sched_items, const_cast<int*>(a.sched), stream);
        if (err != hipSuccess) return err;
    }
    if (p.kernel == Kernel::Mfma) {
        err = launch_decode_mfma(a, p, stream);
        if (err != hipSuccess) return err;
        if (a.counters == nullptr && p.splits > 1) return launch_merge(a, stream);
        return hipSuccess;
    }
    if (p.kernel == Kernel::Valu) {
        switch (a.d) {
            case 32: err = launch_fast_d<32>(a, p, stream); break;
            case 64: err = launch_fast_d<64>(a, p, stream); break;
            case 128: err = launch_fast_d<128>(a, p, stream); break;
            case 256: err = launch_fast_d<256>(a, p, stream); break;
            default: return hipErrorInvalidValue;
        }
        if (err != hipSuccess) return err;
        if (a.counters == nullptr && p.splits > 1) return launch_merge(a, stream);
        return hipSuccess;
    }
    DecodeArgs g = a;
    if (a.k_new != nullptr) {
        // Generic path: append first (token length-1 of each sequence), then attend.
        err = launch_append(a.k_new, a.v_new, a.k, a.v, a.ks, a.vs, a.lengths,
                            min(max(a.uniform_len, 0), a.max_len) - 1, true, a.B, a.Hkv, a.max_len,
                            a.cap, a.d, a.pages, stream);
        if (err != hipSuccess) return err;
        g.k_new = g.v_new = nullptr;
    }
    g.counters = nullptr;
    const dim3 grid(static_cast<unsigned>(a.B * a.Hq * p.splits));
    const size_t lds = sizeof(float) * 2 * static_cast<size_t>(a.d);
    hipLaunchKernelGGL(decode_generic, grid, dim3(kWave), lds, stream, g);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (p.splits > 1) return launch_merge(g, stream);
    return hipSuccess;
}

}  // namespace kvq
