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

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    const size_t words = (bytes + 3) / 4;
    const size_t wgs = (words + 255) / 256;
    const unsigned grid = static_cast<unsigned>(wgs < 4096 ? wgs : 4096);
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid), dim3(256), 0, stream, static_cast<uint8_t*>(p), bytes);
    return hipGetLastError();
}

}  // namespace kvq
