// kvq_append.hip -- gfx950 quantiser kernels of libkvq.so.
//
// The reference has no quantiser (kv_cache/new_kvint8.cu:83-84).  The rule
// implemented here is the per-token symmetric scheme of the task spec:
// scale = max|x| / 127.0f, q = clamp(rintf(x / scale), -127, 127), zero scale
// -> all-zero row.  kvq_device.hpp holds the one definition shared with the
// fused append inside decode_fast, so both paths write identical bits.
#include "kvq_device.hpp"
#include "kvq_internal.hpp"

namespace kvq {
namespace {

// One wave quantises one row of d values (lanes stride over the row).
__device__ void quantize_row_wave(const float* x, int d, int8_t* q, float* scale_out, int lane) {
    float amax = 0.0f;
    for (int i = lane; i < d; i += kWave) amax = fmaxf(amax, fabsf(x[i]));
    amax = wave_max(amax);
    const float s = quant_scale(amax);
    for (int i = lane; i < d; i += kWave) q[i] = static_cast<int8_t>(quant_one(x[i], s));
    if (lane == 0) *scale_out = s;
}

// grid = B*Hkv workgroups of 2 waves: wave 0 quantises the K row, wave 1 the V row.
__global__ __launch_bounds__(2 * kWave) void append_kernel(const float* k_new, const float* v_new,
                                                           int8_t* k, int8_t* v, float* ks, float* vs,
                                                           const int32_t* positions, int uniform_pos,
                                                           int from_lengths, int max_len, int Hkv, int cap,
                                                           int d, const PageMap pages) {
    const int bh = blockIdx.x;
    const int b = bh / Hkv;
    const int kvh = bh - b * Hkv;
    int pos;
    if (positions == nullptr) pos = uniform_pos;
    else if (from_lengths) pos = min(max(positions[b], 0), max_len) - 1;
    else pos = positions[b];
    if (pos < 0 || pos >= cap) return;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const size_t tok = cache_row(pages, Hkv, cap, b, kvh, pos);
    if (wave == 0) quantize_row_wave(k_new + static_cast<size_t>(bh) * d, d, k + tok * d, ks + tok, lane);
    else quantize_row_wave(v_new + static_cast<size_t>(bh) * d, d, v + tok * d, vs + tok, lane);
}

constexpr int kQuantWaves = 4;

__global__ __launch_bounds__(kQuantWaves* kWave) void quantize_rows_kernel(const float* x, int64_t rows,
                                                                          int d, int8_t* q, float* scale) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kQuantWaves;
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * kQuantWaves + threadIdx.x / kWave; r < rows; r += stride)
        quantize_row_wave(x + r * d, d, q + r * d, scale + r, lane);
}

// ---------------------------------------------------------------------------
// Prefill quantiser: L new K and V rows per (b, kv head) into the cache.
// ---------------------------------------------------------------------------

// Element e of an input row as fp32 (bf16 is widened exactly).
template <bool BF16>
__device__ __forceinline__ float load_elem(const void* row, int e) {
    if constexpr (BF16) return __uint_as_float(static_cast<unsigned>(static_cast<const uint16_t*>(row)[e]) << 16);
    else return static_cast<const float*>(row)[e];
}

// Max over aligned groups of N lanes (N a power of two <= 64) of the lanes'
// |x| maxima (non-negative; fmaxf drops NaN elements, so never NaN).
template <int N>
__device__ __forceinline__ float lanes_max(float x) {
    if constexpr (N <= 16) {
        return group_max_nonneg<N>(x);
    } else {
        x = group_max_nonneg<16>(x);
        x = fmaxf(x, __shfl_xor(x, 16));
        if constexpr (N == 64) x = fmaxf(x, __shfl_xor(x, 32));
        return x;
    }
}

// Tuned path: LPR lanes read one row with a 16-byte load each (fp32: 4
// elements, bf16: 8), so one wave load covers 64 / LPR whole rows; U wave
// loads are in flight per lane (fp32: 8, bf16: 4).  Each lane packs its
// quantised elements into one 4- or 8-byte store, so a row's int8 bytes go
// out contiguous.  The grid covers all rows in one pass up to
// kPrefillMaxGroups workgroups: a workgroup takes one contiguous block of
// rows, so the resident workgroups read and write one moving window of the
// input and the cache (a grid-stride loop over 8192 workgroups, every
// workgroup a quarter of the rows apart, was 10% slower for fp32).
constexpr int kPrefillWaves = 4;
constexpr unsigned kPrefillMaxGroups = 1u << 20;
template <bool BF16>
constexpr int prefill_unroll() { return BF16 ? 4 : 8; }

template <int D, bool BF16>
__global__ __launch_bounds__(kPrefillWaves* kWave) void prefill_kernel(const PrefillArgs a) {
    constexpr int EPL = BF16 ? 8 : 4;
    constexpr int LPR = D / EPL;
    constexpr int RPW = kWave / LPR;
    constexpr int kPrefillU = prefill_unroll<BF16>();
    static_assert(LPR >= 1 && LPR <= kWave && (kWave % LPR) == 0, "row geometry");
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int slot = lane / LPR;  // row within a wave load
    const int ls = lane % LPR;    // 16-byte piece of the row
    const int kv = blockIdx.y;    // 0: K rows, 1: V rows
    const char* x = static_cast<const char*>(kv ? a.v_new : a.k_new);
    int8_t* qo = kv ? a.v : a.k;
    float* so = kv ? a.vs : a.ks;
    constexpr int ESZ = BF16 ? 2 : 4;
    const unsigned step = gridDim.x * kPrefillWaves * RPW * kPrefillU;
    const buf_rsrc srs = make_rsrc(a.start, a.start ? static_cast<unsigned>(a.nseq) * 4u : 0u);
    const int start0 = a.start ? 0 : a.uniform_start;
    const bool paged = a.pages.table != nullptr;
    // Both fit in 2^31 bytes (the launcher sends larger tables to the generic kernel).
    const buf_rsrc trs = make_rsrc(a.pages.table, paged ? static_cast<unsigned>(a.nseq) * a.pages.max_pages * 4u : 0u);
    for (unsigned r0 = (blockIdx.x * kPrefillWaves + wave) * RPW * kPrefillU; r0 < a.rows; r0 += step) {
        // The kPrefillU row loads go out together and unconditionally (a row
        // past the end rereads the last row and is dropped below), so no
        // load waits for another.
        int4 raw[kPrefillU];
        unsigned row[kPrefillU];
#pragma unroll
        for (int u = 0; u < kPrefillU; u++) {
            row[u] = r0 + u * RPW + slot;
            const unsigned rc = min(row[u], a.rows - 1);
            raw[u] = *reinterpret_cast<const int4*>(x + (static_cast<size_t>(rc) * D + ls * EPL) * ESZ);
        }
        // Each row's destination: (b, kv head, token) from the row index,
        // then the cache row.  start[b] and the page-table entries come
        // through buffer resources (a null start, or an index outside the
        // table, reads 0), so the loads of all kPrefillU rows are
        // unconditional and in flight together.  -1: the row is skipped.
        int pos[kPrefillU], bb[kPrefillU], hh[kPrefillU];
#pragma unroll
        for (int u = 0; u < kPrefillU; u++) {
            const unsigned rc = min(row[u], a.rows - 1);
            const unsigned bh = fastdiv(rc, a.divL);
            bb[u] = static_cast<int>(fastdiv(bh, a.divH));
            hh[u] = static_cast<int>(bh - static_cast<unsigned>(bb[u]) * a.Hkv);
            pos[u] = static_cast<int>(rc - bh * a.L) + start0 + buffer_load4(srs, bb[u] * 4, 0);
        }
        long long orow[kPrefillU];
        if (paged) {
            int page[kPrefillU], pi[kPrefillU];
#pragma unroll
            for (int u = 0; u < kPrefillU; u++) {
                pi[u] = a.pages.shift >= 0 ? pos[u] >> a.pages.shift : pos[u] / a.pages.size;
                page[u] = buffer_load4(trs, (bb[u] * a.pages.max_pages + pi[u]) * 4, 0);
            }
#pragma unroll
            for (int u = 0; u < kPrefillU; u++) {
                const int pg = min(max(page[u], 0), a.pages.num_pages - 1);
                orow[u] = (static_cast<long long>(pg) * a.Hkv + hh[u]) * a.pages.size + (pos[u] - pi[u] * a.pages.size);
            }
        } else {
#pragma unroll
            for (int u = 0; u < kPrefillU; u++)
                orow[u] = (static_cast<long long>(bb[u]) * a.Hkv + hh[u]) * a.cap + pos[u];
        }
#pragma unroll
        for (int u = 0; u < kPrefillU; u++)
            if (!(row[u] < a.rows && pos[u] >= 0 && pos[u] < a.cap)) orow[u] = -1;
#pragma unroll
        for (int u = 0; u < kPrefillU; u++) {
            float e[EPL];
            const int w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
            for (int i = 0; i < EPL; i++) {
                if constexpr (BF16) e[i] = __uint_as_float((i & 1) ? (static_cast<unsigned>(w[i >> 1]) & 0xffff0000u)
                                                                 : (static_cast<unsigned>(w[i >> 1]) << 16));
                else e[i] = __int_as_float(w[i]);
            }
            float am = 0.0f;
#pragma unroll
            for (int i = 0; i < EPL; i++) am = fmaxf(am, fabsf(e[i]));
            const float scale = quant_scale(lanes_max<LPR>(am));
            if (orow[u] < 0) continue;
            const size_t o = static_cast<size_t>(orow[u]);
            int qv[EPL];
            quant_row<EPL>(e, scale, qv);
            if constexpr (BF16) {
                const int2 pk = make_int2(pack4(qv[0], qv[1], qv[2], qv[3]), pack4(qv[4], qv[5], qv[6], qv[7]));
                *reinterpret_cast<int2*>(qo + o * D + ls * EPL) = pk;
            } else {
                *reinterpret_cast<int*>(qo + o * D + ls * EPL) = pack4(qv[0], qv[1], qv[2], qv[3]);
            }
            if (ls == 0) so[o] = scale;
        }
    }
}

// Any head dim / alignment: one wave per row, lanes striding over it.
template <bool BF16>
__global__ __launch_bounds__(kPrefillWaves* kWave) void prefill_generic_kernel(const PrefillArgs a, int d) {
    const int lane = threadIdx.x & (kWave - 1);
    const int kv = blockIdx.y;
    const char* x = static_cast<const char*>(kv ? a.v_new : a.k_new);
    int8_t* qo = kv ? a.v : a.k;
    float* so = kv ? a.vs : a.ks;
    const unsigned step = gridDim.x * kPrefillWaves;
    for (unsigned row = blockIdx.x * kPrefillWaves + threadIdx.x / kWave; row < a.rows; row += step) {
        const void* xr = x + static_cast<size_t>(row) * d * (BF16 ? 2 : 4);
        const unsigned bh = fastdiv(row, a.divL);
        const int t = static_cast<int>(row - bh * a.L);
        const int b = static_cast<int>(fastdiv(bh, a.divH));
        const int h = static_cast<int>(bh - static_cast<unsigned>(b) * a.Hkv);
        const int pos = (a.start ? a.start[b] : a.uniform_start) + t;
        if (pos < 0 || pos >= a.cap) continue;
        const size_t orow = cache_row(a.pages, a.Hkv, a.cap, b, h, pos);
        float am = 0.0f;
        for (int i = lane; i < d; i += kWave) am = fmaxf(am, fabsf(load_elem<BF16>(xr, i)));
        const float scale = quant_scale(wave_max(am));
        for (int i = lane; i < d; i += kWave) qo[orow * d + i] = static_cast<int8_t>(quant_one(load_elem<BF16>(xr, i), scale));
        if (lane == 0) so[orow] = scale;
    }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(uint8_t* p, size_t bytes) {
    const size_t words = bytes / 4;
    uint32_t* w = reinterpret_cast<uint32_t*>(p);
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride) w[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x < (bytes & 3)) p[words * 4 + threadIdx.x] = 0;
}

}  // namespace

hipError_t launch_append(const float* k_new, const float* v_new, int8_t* k, int8_t* v, float* ks,
                         float* vs, const int32_t* positions, int uniform_pos, bool from_lengths,
                         int B, int Hkv, int max_len, int cap, int d, const PageMap& pages,
                         hipStream_t stream) {
    hipLaunchKernelGGL(append_kernel, dim3(static_cast<unsigned>(B * Hkv)), dim3(2 * kWave), 0, stream,
                       k_new, v_new, k, v, ks, vs, positions, uniform_pos, from_lengths ? 1 : 0, max_len,
                       Hkv, cap, d, pages);
    return hipGetLastError();
}

hipError_t launch_quantize_rows(const float* x, int64_t rows, int d, int8_t* q, float* scale,
                                hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const int64_t wgs = (rows + kQuantWaves - 1) / kQuantWaves;
    const unsigned grid = static_cast<unsigned>(wgs < 65536 ? wgs : 65536);
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(grid), dim3(kQuantWaves * kWave), 0, stream, x, rows,
                       d, q, scale);
    return hipGetLastError();
}

template <bool BF16>
hipError_t launch_prefill_t(const PrefillArgs& a, int d, bool vec_ok, hipStream_t stream) {
    const unsigned want_rows = static_cast<unsigned>(a.rows);
    auto grid_for = [&](unsigned rows_per_wg) {
        const unsigned wgs = (want_rows + rows_per_wg - 1) / rows_per_wg;
        const unsigned cap = a.max_groups ? min(a.max_groups, kPrefillMaxGroups) : kPrefillMaxGroups;
        return dim3(wgs < cap ? (wgs ? wgs : 1) : cap, static_cast<unsigned>(a.planes));
    };
    const dim3 block(kPrefillWaves * kWave);
    constexpr int EPL = BF16 ? 8 : 4;
    if (vec_ok) {
        switch (d) {
#define KVQ_PREFILL_CASE(DD)                                                                        \
    case DD:                                                                                        \
        hipLaunchKernelGGL((prefill_kernel<DD, BF16>),                                              \
                           grid_for(kPrefillWaves * (kWave / (DD / EPL)) * prefill_unroll<BF16>()), block, 0, \
                           stream, a);                                                              \
        return hipGetLastError();
            KVQ_PREFILL_CASE(32)
            KVQ_PREFILL_CASE(64)
            KVQ_PREFILL_CASE(128)
            KVQ_PREFILL_CASE(256)
#undef KVQ_PREFILL_CASE
            default: break;
        }
    }
    hipLaunchKernelGGL((prefill_generic_kernel<BF16>), grid_for(kPrefillWaves), block, 0, stream, a, d);
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a, int d, bool bf16, bool vec_ok, hipStream_t stream) {
    if (a.rows == 0) return hipSuccess;
    return bf16 ? launch_prefill_t<true>(a, d, vec_ok, stream) : launch_prefill_t<false>(a, d, vec_ok, stream);
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    const size_t words = (bytes + 3) / 4;
    const size_t wgs = (words + 255) / 256;
    const unsigned grid = static_cast<unsigned>(wgs < 4096 ? wgs : 4096);
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, stream, static_cast<uint8_t*>(p), bytes);
    return hipGetLastError();
}

}  // namespace kvq
