// kvq_split.hpp -- sequence-split plumbing shared by the decode kernels:
// lengths, device-coherent partial records, the log-sum-exp merge and the
// last-arrival handshake.
#pragma once

#include <math.h>

#include "kvq_device.hpp"
#include "kvq_internal.hpp"

namespace kvq {

__device__ __forceinline__ int seq_len_of(const DecodeArgs& a, int b) {
    const int len = a.lengths ? a.lengths[b] : a.uniform_len;
    return min(max(len, 0), a.max_len);
}

// U consecutive per-token scales (U in {1,2,4,8}); p is U*4-byte aligned when
// the token index is a multiple of U (tiles start at multiples of U tokens).
template <int U>
__device__ __forceinline__ void load_scales(const float* p, float (&out)[U]) {
    if constexpr (U % 4 == 0) {
#pragma unroll
        for (int i = 0; i < U; i += 4) {
            const float4 x = *reinterpret_cast<const float4*>(p + i);
            out[i] = x.x;
            out[i + 1] = x.y;
            out[i + 2] = x.z;
            out[i + 3] = x.w;
        }
    } else if constexpr (U == 2) {
        const float2 x = *reinterpret_cast<const float2*>(p);
        out[0] = x.x;
        out[1] = x.y;
    } else {
#pragma unroll
        for (int i = 0; i < U; i++) out[i] = p[i];
    }
}

// Partial records cross workgroups (and XCDs, whose L2s are not coherent with
// each other) inside one launch.  They are written and read with agent-scope
// relaxed atomics, i.e. device-coherent global_store/global_load sc1, so no
// L2-wide writeback/invalidate fence is needed; the producer waits for its
// stores to complete (s_waitcnt 0) before it bumps the arrival counter.
__device__ __forceinline__ void put_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float get_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Log-sum-exp merge of the nsplit partial records of output row bhq, element dim.
__device__ inline float merge_dim(const DecodeArgs& a, size_t bhq, int dim, int nsplit) {
    const float* ml = a.part_ml + bhq * a.splits * 2;
    const float* acc = a.part_acc + bhq * a.splits * a.d;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, get_coherent(ml + 2 * s));
    float L = 0.0f, A = 0.0f;
    for (int s = 0; s < nsplit; s++) {
        const float w = fast_exp2(get_coherent(ml + 2 * s) - M);
        L = fmaf(get_coherent(ml + 2 * s + 1), w, L);
        A = fmaf(get_coherent(acc + static_cast<size_t>(s) * a.d + dim), w, A);
    }
    return A / L;
}

// One output element of a workgroup's result: the final value when the
// sequence has one split, otherwise this split's partial record.
__device__ __forceinline__ void store_result(const DecodeArgs& a, size_t bhq, int dim, int split, int nsplit,
                                             float M, float L, float A) {
    if (nsplit == 1) {
        a.out[bhq * a.d + dim] = A / L;
    } else {
        const size_t rec = bhq * a.splits + split;
        put_coherent(a.part_acc + rec * a.d + dim, A);
        if (dim == 0) {
            put_coherent(a.part_ml + rec * 2, M);
            put_coherent(a.part_ml + rec * 2 + 1, L);
        }
    }
}

// Merge of one sequence group's records by a whole workgroup (nthreads
// threads, nheads <= kMergeHeads, nsplit <= kMergeSplits): per head the max
// and the weights exp2(m_s - M) are computed once, in parallel over splits,
// then every output element sums its nsplit accumulators with 8 loads in
// flight.
constexpr int kMergeHeads = 8;
constexpr int kMergeSplits = 256;

__device__ inline void merge_group(const DecodeArgs& a, size_t bhq0, int nheads, int nsplit) {
    __shared__ float s_w[kMergeHeads][kMergeSplits];
    __shared__ float s_red[kMergeHeads][16];
    __shared__ float s_inv[kMergeHeads];
    const int nthreads = blockDim.x;
    const int nw = nthreads / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    for (int h = 0; h < nheads; h++) {
        const float* ml = a.part_ml + (bhq0 + h) * a.splits * 2;
        float mx = -INFINITY;
        for (int sp = threadIdx.x; sp < nsplit; sp += nthreads) {
            const float mv = get_coherent(ml + 2 * sp);
            s_w[h][sp] = mv;
            mx = fmaxf(mx, mv);
        }
        mx = wave_max(mx);
        if (lane == 0) s_red[h][wave] = mx;
    }
    __syncthreads();
    for (int h = 0; h < nheads; h++) {
        const float* ml = a.part_ml + (bhq0 + h) * a.splits * 2;
        float M = -INFINITY;
        for (int w = 0; w < nw; w++) M = fmaxf(M, s_red[h][w]);
        float lsum = 0.0f;
        for (int sp = threadIdx.x; sp < nsplit; sp += nthreads) {
            const float w = fast_exp2(s_w[h][sp] - M);
            s_w[h][sp] = w;
            lsum = fmaf(get_coherent(ml + 2 * sp + 1), w, lsum);
        }
        lsum = wave_sum(lsum);
        __syncthreads();  // every wave has read s_red[h] before it is reused
        if (lane == 0) s_red[h][wave] = lsum;
    }
    __syncthreads();
    if (threadIdx.x < nheads) {
        float L = 0.0f;
        for (int w = 0; w < nw; w++) L += s_red[threadIdx.x][w];
        s_inv[threadIdx.x] = L;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nheads * a.d; i += nthreads) {
        const int h = i / a.d;
        const int dim = i - h * a.d;
        const float* acc = a.part_acc + (bhq0 + h) * a.splits * a.d + dim;
        float A = 0.0f;
        int sp = 0;
        for (; sp + 8 <= nsplit; sp += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = get_coherent(acc + static_cast<size_t>(sp + j) * a.d);
#pragma unroll
            for (int j = 0; j < 8; j++) A = fmaf(v[j], s_w[h][sp + j], A);
        }
        for (; sp < nsplit; sp++) A = fmaf(get_coherent(acc + static_cast<size_t>(sp) * a.d), s_w[h][sp], A);
        a.out[(bhq0 + h) * a.d + dim] = A / s_inv[h];
    }
}

// Called by every thread of a workgroup after its store_result calls: counts
// the split's arrival and, in the last workgroup of the sequence group, merges
// the records of heads [bhq0, bhq0 + nheads).  s_last: one int of LDS.
__device__ __forceinline__ void finish_split(const DecodeArgs& a, int unit, size_t bhq0, int nheads, int nsplit,
                                             int* s_last) {
    if (nsplit <= 1 || a.counters == nullptr) return;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's record stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(a.counters + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_last = (prev == nsplit - 1);
    }
    __syncthreads();
    if (*s_last) {
        if (nheads <= kMergeHeads && nsplit <= kMergeSplits) {
            merge_group(a, bhq0, nheads, nsplit);
        } else {
            for (int i = threadIdx.x; i < nheads * a.d; i += blockDim.x) {
                const int h = i / a.d;
                const int dim = i - h * a.d;
                a.out[(bhq0 + h) * a.d + dim] = merge_dim(a, bhq0 + h, dim, nsplit);
            }
        }
        if (threadIdx.x == 0)  // ready for the next launch
            __hip_atomic_store(a.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace kvq
