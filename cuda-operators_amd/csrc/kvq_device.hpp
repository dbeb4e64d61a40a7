// kvq_device.hpp -- device helpers shared by the gfx950 kernels of libkvq.so.
//
// Wave64 throughout.  Cross-lane sums inside a token's lane group use DPP row
// permutations (no LDS traffic); wider exchanges use ds_bpermute (__shfl_xor).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvq {

constexpr int kWave = 64;

// DPP control words (GCN/CDNA DPP encoding).
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141; // lane i <- 7-i within each 8 lanes
constexpr int kDppRowMirror = 0x140;     // lane i <- 15-i within each 16 lanes

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of N lanes (N in {1,2,4,8,16}); every lane of the
// group receives the group total.  After the two quad steps each quad holds its
// sum, so a half-row mirror adds the neighbouring quad and a row mirror adds
// the other half of the 16-lane row.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
    if constexpr (N >= 2) x += dpp<kDppQuadXor1>(x);
    if constexpr (N >= 4) x += dpp<kDppQuadXor2>(x);
    if constexpr (N >= 8) x += dpp<kDppRowHalfMirror>(x);
    if constexpr (N >= 16) x += dpp<kDppRowMirror>(x);
    return x;
}

template <int N>
__device__ __forceinline__ float group_max(float x) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
    if constexpr (N >= 2) x = fmaxf(x, dpp<kDppQuadXor1>(x));
    if constexpr (N >= 4) x = fmaxf(x, dpp<kDppQuadXor2>(x));
    if constexpr (N >= 8) x = fmaxf(x, dpp<kDppRowHalfMirror>(x));
    if constexpr (N >= 16) x = fmaxf(x, dpp<kDppRowMirror>(x));
    return x;
}

// Max over aligned groups of N lanes of non-negative, non-NaN floats.  Their
// bit patterns order as unsigned integers, so the steps run as v_max_u32 with
// the DPP operand folded in (the float max needs a quieting step per stage).
template <int N>
__device__ __forceinline__ float group_max_nonneg(float x) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "group size");
    unsigned u = __float_as_uint(x);
    if constexpr (N >= 2) u = max(u, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), kDppQuadXor1, 0xF, 0xF, false)));
    if constexpr (N >= 4) u = max(u, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), kDppQuadXor2, 0xF, 0xF, false)));
    if constexpr (N >= 8) u = max(u, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), kDppRowHalfMirror, 0xF, 0xF, false)));
    if constexpr (N >= 16) u = max(u, static_cast<unsigned>(__builtin_amdgcn_update_dpp(0, static_cast<int>(u), kDppRowMirror, 0xF, 0xF, false)));
    return __uint_as_float(u);
}

// Inclusive prefix sum over the wave: Hillis-Steele steps within each
// 16-lane row (DPP row_shr 1, 2, 4, 8; lanes shifted in from outside the row
// add 0), then the row broadcasts of GFX9 DPP: lane 15 of rows 0 and 2 into
// rows 1 and 3 (row_bcast:15), lane 31 into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ int wave_inclusive_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return v;
}

// Inclusive prefix max over the wave of non-negative ints (the steps of
// wave_inclusive_scan with max; lanes shifted in from outside a row give 0).
__device__ __forceinline__ int wave_inclusive_max_nonneg(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false));
    return v;
}

// Size class of a sequence's last chunk under a split schedule (0: a whole
// chunk, kClasses - 1: nearly empty): kClasses (chunk - last) / (chunk + 1)
// in fp32 (no 64-bit divide).  Longest-first order dispatches class 0 first.
template <int kClasses>
__device__ __forceinline__ int last_chunk_class(int chunk, int last) {
    const float f =
        static_cast<float>(chunk - last) * (static_cast<float>(kClasses) / static_cast<float>(chunk + 1));
    return min(max(static_cast<int>(f), 0), kClasses - 1);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}

// Signed byte b of a dword as float: one v_cvt_f32_i32 with an SDWA
// sign-extended byte select on gfx950.
__device__ __forceinline__ float sbyte(int w, int b) {
    return static_cast<float>(static_cast<int8_t>(w >> (8 * b)));
}

// 16 int8 values (one int4 load) -> 16 floats.
__device__ __forceinline__ void unpack16(const int4& x, float (&f)[16]) {
    const int w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int b = 0; b < 4; b++) f[4 * j + b] = sbyte(w[j], b);
    }
}

#ifndef KVQ_NT_LOADS
#define KVQ_NT_LOADS 1
#endif
typedef int v4i_t __attribute__((ext_vector_type(4)));

// 16-byte load of streamed cache data (read once per decode step).  The
// non-temporal hint keeps the stream from displacing reusable lines and
// measured ~13% more read bandwidth on MI355X (6.9 vs 6.1 TB/s).
__device__ __forceinline__ int4 load16_stream(const int8_t* p) {
#if KVQ_NT_LOADS
    const v4i_t t = __builtin_nontemporal_load(reinterpret_cast<const v4i_t*>(p));
    return make_int4(t.x, t.y, t.z, t.w);
#else
    return *reinterpret_cast<const int4*>(p);
#endif
}

// Raw buffer resource over [base, base + bytes) (gfx9 descriptor word 3 =
// 0x00020000: 32-bit data format, no swizzle, stride 0).  A load through it
// adds a per-lane byte offset (VGPR), a wave-uniform byte offset (SGPR) and an
// immediate, so a tile loop advances one scalar instead of 64-bit lane
// addresses; bytes at or past `bytes` read as 0.
typedef __amdgpu_buffer_rsrc_t buf_rsrc;

__device__ __forceinline__ buf_rsrc make_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}

// 16 bytes of streamed cache data (non-temporal, as load16_stream).
__device__ __forceinline__ v4i_t buffer_load16_stream(buf_rsrc r, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, KVQ_NT_LOADS ? 2 : 0);
}

// 4 consecutive fp32 values (16 bytes).
__device__ __forceinline__ v4i_t buffer_load16(buf_rsrc r, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

// One 32-bit word.
__device__ __forceinline__ int buffer_load4(buf_rsrc r, int voff, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

// v_exp_f32: 2^x, exp2(-inf) == 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------
// Per-token symmetric int8 quantiser.  scale = amax / 127.0f with IEEE division
// (HIP's default correctly rounded fp32 divide), q = clamp(rintf(x / scale),
// -127, 127) with rintf = round half to even (v_rndne_f32); a zero scale (amax
// == 0, or amax so small that the quotient underflows) stores q = 0.
// ---------------------------------------------------------------------------
// RN(amax / 127) without the divide: with C = 1/127 split as Ch = RN(C) and
// Cl = RN(C - Ch), fma(amax, Ch, RN(amax * Cl)) is the correctly rounded
// quotient for every amax >= 2^-112 (Brisebarre and Muller, "Correctly rounded
// multiplication by arbitrary precision constants", IEEE TC 57(2), 2008; for
// this C checked over all such floats by tests/quant_scale_check.c).  Smaller
// amax (a subnormal or near-subnormal quotient) takes the divide.
__device__ __forceinline__ float quant_scale(float amax) {
    constexpr float kCh = 0x1.020408p-7f;
    constexpr float kCl = 0x1.020408p-35f;
    if (__builtin_expect(amax < 0x1p-112f, 0)) return amax / 127.0f;
    return __builtin_fmaf(amax, kCh, amax * kCl);
}

__device__ __forceinline__ int quant_one(float x, float scale) {
    if (scale == 0.0f) return 0;
    float y = __builtin_rintf(x / scale);
    y = fminf(fmaxf(y, -127.0f), 127.0f);
    return static_cast<int>(y);
}

// The same quantisation of N elements of one row, with the quotient taken as
// x * rcp(scale) instead of the IEEE divide (a standard division by a
// reciprocal with an error-bounded exactness test; e.g. Muller et al.,
// Handbook of Floating-Point Arithmetic, 2nd ed., sec. 4.9 / 5.3).  The result
// is bit-identical to quant_one for every input:
// * |x| <= amax and scale = RN(amax / 127), so |x / scale| < 128.
// * v_rcp_f32 is within 1 ulp (relative 2^-23) of 1 / scale and the product
//   rounds once (2^-24), so the fast quotient q is within 1.5 * 2^-23 * 128 =
//   1.5 * 2^-16 of x / scale; the IEEE quotient Q is within 2^-24 * 128 =
//   2^-17 of it; hence |q - Q| <= 2^-15.
// * rintf changes value only at half-integers, so rintf(q) == rintf(Q)
//   whenever q is more than 2^-15 from every half-integer (then Q lies on
//   the same side and is not itself a tie).  The test also holds when the
//   compiler fuses y - n into fma(x, rinv, -n): then it measures the exact
//   product P, with |P - Q| <= 1.5 * 2^-16 and |y - P| <= 2^-17, both below
//   the margin, so q, P and Q round alike.  An element within 2^-15 of a
//   half-integer takes quant_one: about one in 16000 for fp32 data, but about
//   one in 600 for bf16 inputs, whose 8-bit significands often make x / scale
//   an exact tie.  So does every element of a row whose scale is outside
//   [2^-100, 2^100] (zero, subnormal or non-finite scales included).
// * No clamp is needed on the fast path: |x| <= amax gives |q| < 127.001, so
//   rintf(q) is within [-127, 127].
// Cost per element: multiply, rint, fused subtract, compare, convert --
// against the IEEE divide's ten instructions.
template <int N>
__device__ __forceinline__ void quant_row(const float (&x)[N], float scale, int (&q)[N]) {
    if (!(scale >= 0x1p-100f && scale <= 0x1p100f)) {
#pragma unroll
        for (int i = 0; i < N; i++) q[i] = quant_one(x[i], scale);
        return;
    }
    const float rinv = __builtin_amdgcn_rcpf(scale);
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float y = x[i] * rinv;
        const float n = __builtin_rintf(y);
        q[i] = static_cast<int>(n);
        // One branch per element, so a wave runs the divide only for the
        // element positions that some lane flags.  A NaN element fails the
        // test and takes quant_one too.
        if (!(fabsf(y - n) < 0.5f - 0x1p-15f)) q[i] = quant_one(x[i], scale);
    }
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
    return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | (static_cast<int>(static_cast<unsigned>(d & 0xff) << 24));
}

}  // namespace kvq
