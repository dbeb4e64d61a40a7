// kvq_schedule.hip -- device-side split schedule of a ragged decode batch.
//
// With per-sequence lengths on the device, a static split grid (every
// sequence cut into the same number of chunks of the longest sequence's
// length) leaves most workgroups of short sequences idle and the longest ones
// finishing last.  One small workgroup instead reads the lengths and writes a
// schedule (layout at kSchedHeader in kvq_internal.hpp) that the decode launch
// right after it on the same stream follows.  `target` is the number of
// workgroups the decode grid can run at once (S = target / units items):
//
// * one round (B <= S, every sequence can have its own items): the smallest
//   chunk c (a multiple of the tile granularity) with
//   sum_b ceil(len_b / c) <= S, so every item runs in the first round and the
//   launch takes as long as its largest item.  The candidates lie in
//   [total / S, total / (S - B)] (sum ceil(len / c) < total / c + B); one
//   thread tests each.  Sequence b then splits into n_b = ceil(len_b / c)
//   equal chunks of round_up(ceil(len_b / n_b), gran) <= c tokens, so its
//   last split is not a small remainder.
// * several rounds (B > S): chunk = total tokens x units / target, rounded
//   up to the granularity: about `target` equal chunks over the whole batch.
//   Whole chunks are dispatched first and each sequence's last (partial)
//   chunk after them, longest first (64 size classes, a counting sort), so
//   the work left at the end of the launch is small -- list scheduling in
//   longest-processing-time order.
// * partial records are numbered per sequence (rec_base) so the workspace
//   holds records only for splits that exist: at most B + target / units.
#include <limits.h>

#include "kvq_device.hpp"
#include "kvq_internal.hpp"

namespace kvq {
namespace {

// 256 threads: at B256 the 1024-thread version took 5.9 us per launch and
// this one 4.8 us (fewer waves in every barrier and scan); 64 and 128
// threads, which loop more, took 8.7 and 6.4 us.
constexpr int kSchedThreads = 256;
constexpr int kSchedLen = 1024;  // lengths kept in LDS
constexpr int kSchedWaves = kSchedThreads / kWave;

// Exclusive prefix sum of x over the workgroup (thread order); *total gets
// the sum.  s_tmp: kSchedWaves ints of LDS, reusable after the call.
__device__ int block_exclusive_scan(int x, int* s_tmp, int* total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int v = wave_inclusive_scan(x);
    if (lane == kWave - 1) s_tmp[wave] = v;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kSchedWaves; w++) {
        const int t = s_tmp[w];
        before += w < wave ? t : 0;
        all += t;
    }
    *total = all;
    __syncthreads();
    return before + v - x;
}

// The same class function in both passes that use it.
__device__ __forceinline__ int size_class(int chunk, int last) { return last_chunk_class<kSizeClasses>(chunk, last); }

__device__ __forceinline__ int clamped_len(const int32_t* lengths, int b, int max_len) {
    return min(max(lengths[b], 0), max_len);
}

// Work item pos: split s of sequence b (n splits of chunk tokens, first
// record rec, len tokens), in the layout at kSchedHeader (kvq_internal.hpp).
__device__ __forceinline__ void put_item(int* items, int pos, int b, int s, int n, int rec, int chunk, int len) {
    int4* it = reinterpret_cast<int4*>(items + kSchedItemInts * pos);
    it[0] = make_int4(b, s, n, rec);
    it[1] = make_int4(chunk, len, 0, 0);
}

__global__ __launch_bounds__(kSchedThreads) void schedule_kernel(const int32_t* lengths, int B, int max_len,
                                                                 int units, int target, int gran, int items_cap,
                                                                 int* sched) {
    __shared__ int s_tmp[kSchedWaves];
    __shared__ long long s_sum[kSchedWaves];
    __shared__ int s_class[kSizeClasses];
    __shared__ int s_len[kSchedLen];  // the first kSchedLen clamped lengths
    __shared__ int s_best;
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    // Length of sequence b: from LDS after the first pass (one read of the
    // lengths for batches up to kSchedLen), from memory beyond that.
    auto len_of = [&](int b) { return b < kSchedLen ? s_len[b] : clamped_len(lengths, b, max_len); };

    long long sum = 0;
    for (int b = t; b < B; b += kSchedThreads) {
        const int len = clamped_len(lengths, b, max_len);
        sum += len;
        if (b < kSchedLen) s_len[b] = len;
    }
    // The wave's sum in two 32-bit halves by DPP (a lane's sum is below 2^43:
    // at most 2^12 lengths below 2^31 each for batches up to 2^20; the
    // halves' wave sums stay below 2^32), else by 64-bit shuffles.
    if (B <= (1 << 20)) {
        const unsigned lo = wave_inclusive_scan(static_cast<int>(sum & 0xFFFFF));
        const unsigned hi = wave_inclusive_scan(static_cast<int>(sum >> 20));
        sum = (static_cast<long long>(__builtin_amdgcn_readlane(static_cast<int>(hi), kWave - 1)) << 20) +
              static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(lo), kWave - 1));
    } else {
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    }
    if (lane == 0) s_sum[wave] = sum;
    if (t < kSizeClasses) s_class[t] = 0;
    if (t == 0) s_best = INT_MAX;
    __syncthreads();
    long long total = 0;
#pragma unroll
    for (int w = 0; w < kSchedWaves; w++) total += s_sum[w];

    int* items = sched + kSchedHeader;
    int2* seq = reinterpret_cast<int2*>(items + kSchedItemInts * items_cap);  // (rec_base, chunk) per sequence
    // (At most INT_MAX rounded down to the granularity: a chunk is an int.)
    const long long cmax = min((static_cast<long long>(max(max_len, 1)) + gran - 1) / gran * gran,
                               static_cast<long long>(INT_MAX) / gran * gran);
    const int S = target / units;

    if (B <= S && B <= kSchedLen) {
        // One round: the smallest chunk whose items all fit.
        const long long lo = min(cmax, max(static_cast<long long>(gran), (total + S - 1) / S + gran - 1) / gran * gran);
        const long long hi =
            S > B ? max(lo, min(cmax, ((total + (S - B) - 1) / (S - B) + gran - 1) / gran * gran)) : cmax;
        for (long long c = lo + static_cast<long long>(t) * gran; c <= hi; c += static_cast<long long>(kSchedThreads) * gran) {
            long long n = 0;
            for (int b = 0; b < B; b++) n += s_len[b] == 0 ? 1 : (s_len[b] + c - 1) / c;
            if (n <= S || c == hi) atomicMin(&s_best, static_cast<int>(c));
        }
        __syncthreads();
        const int chunk = s_best;
        int carry = 0;
        for (int b0 = 0; b0 < B; b0 += kSchedThreads) {
            const int b = b0 + t;
            int n = 0, cb = gran;
            if (b < B) {
                const int len = s_len[b];
                n = len == 0 ? 1 : (len + chunk - 1) / chunk;
                cb = len == 0 ? gran : ((len + n - 1) / n + gran - 1) / gran * gran;
            }
            int tot = 0;
            const int pre = carry + block_exclusive_scan(n, s_tmp, &tot);
            if (b < B) {
                seq[b] = make_int2(pre, cb);
                for (int s = 0; s < n; s++) {
                    if (pre + s < items_cap) put_item(items, pre + s, b, s, n, pre, cb, s_len[b]);
                }
            }
            carry += tot;
        }
        if (t == 0) {
            sched[0] = chunk;
            sched[1] = min(carry, items_cap);
        }
        return;
    }

    const long long want = (total * units + target - 1) / target;
    const long long c = (want + gran - 1) / gran * gran;
    const int chunk = static_cast<int>(min(cmax, max(static_cast<long long>(gran), c)));
    int rec_carry = 0, full_carry = 0;
    for (int b0 = 0; b0 < B; b0 += kSchedThreads) {
        const int b = b0 + t;
        int len = 0, n = 0;
        if (b < B) {
            len = len_of(b);
            n = len == 0 ? 1 : (len + chunk - 1) / chunk;
        }
        const int full = n > 0 ? n - 1 : 0;
        // Every b < B has n >= 1, so the prefix of the full chunks is the
        // prefix of n less the sequences before b in this pass.
        int tot_n = 0;
        const int pre_n = block_exclusive_scan(n, s_tmp, &tot_n);
        const int valid = min(B - b0, kSchedThreads);
        const int pre_f = pre_n - t;
        const int tot_f = tot_n - valid;
        if (b < B) {
            seq[b] = make_int2(rec_carry + pre_n, chunk);
            for (int s = 0; s < full; s++) {
                const int pos = full_carry + pre_f + s;
                if (pos < items_cap) put_item(items, pos, b, s, n, rec_carry + pre_n, chunk, len);
            }
            const int last = len - (n - 1) * chunk;  // in [0, chunk]
            const int cls = size_class(chunk, last);
            atomicAdd(&s_class[cls], 1);
        }
        rec_carry += tot_n;
        full_carry += tot_f;
    }
    __syncthreads();
    // Size classes -> first item position of each class (longest first).
    if (wave == 0) {
        const int cnt = s_class[lane];
        s_class[lane] = full_carry + wave_inclusive_scan(cnt) - cnt;
    }
    __syncthreads();
    for (int b = t; b < B; b += kSchedThreads) {
        const int len = len_of(b);
        const int n = len == 0 ? 1 : (len + chunk - 1) / chunk;
        const int last = len - (n - 1) * chunk;
        const int cls = size_class(chunk, last);
        const int pos = atomicAdd(&s_class[cls], 1);
        if (pos < items_cap) put_item(items, pos, b, n - 1, n, seq[b].x, chunk, len);
    }
    if (t == 0) {
        sched[0] = chunk;
        sched[1] = min(full_carry + B, items_cap);
    }
}

}  // namespace

hipError_t launch_schedule(const int32_t* lengths, int B, int max_len, int units_per_seq, int target_wgs,
                           int gran, int items_cap, int* sched, hipStream_t stream) {
    hipLaunchKernelGGL(schedule_kernel, dim3(1), dim3(kSchedThreads), 0, stream, lengths, B, max_len,
                       units_per_seq, target_wgs, gran, items_cap, sched);
    return hipGetLastError();
}

}  // namespace kvq
