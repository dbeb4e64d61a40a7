// kvq_split.hpp -- sequence-split plumbing shared by the decode kernels:
// lengths, device-coherent partial records, the log-sum-exp merge and the
// last-arrival handshake.
#pragma once

#include <limits.h>
#include <math.h>

#include "kvq_device.hpp"
#include "kvq_internal.hpp"

namespace kvq {

__device__ __forceinline__ int seq_len_of(const DecodeArgs& a, int b) {
    const int len = a.lengths ? a.lengths[b] : a.uniform_len;
    return min(max(len, 0), a.max_len);
}

// What one decode workgroup computes: work unit `unit` (index (b * Hkv + kvh)
// * nsg + sgi of (sequence, kv head, head group)) over tokens [t0, t1), split
// `split` of the sequence's nsplit.  A length-0 sequence has one split with
// t0 = t1 = 0 (its workgroup writes the zero output).
struct SplitWork {
    int unit, b, split, nsplit, len, t0, t1;
    int rec;  // in-kernel plan: the sequence's first partial record (see locate_fit)
};

// Work of workgroup blockIdx.x, from the static split grid (split-major:
// blockIdx = split * units + unit) or the device split schedule; false: the
// workgroup has nothing to do.
__device__ __forceinline__ bool locate_work(const DecodeArgs& a, SplitWork& w) {
    const int U = a.Hkv * a.nsg;
    int chunk;
    if (a.sched) {
        // The count and the item (in bounds: the grid has sched_items items)
        // load together, one round trip before the workgroup's first tile.
        const int item = blockIdx.x / U;
        const int count = a.sched[1];
        const int4* it = reinterpret_cast<const int4*>(a.sched + kSchedHeader + kSchedItemInts * item);
        const int4 i0 = it[0];
        const int4 i1 = it[1];
        if (item >= count) return false;
        w.b = i0.x;
        w.split = i0.y;
        w.nsplit = i0.z;
        w.rec = i0.w;
        chunk = i1.x;
        w.len = i1.y;
        w.unit = w.b * U + (blockIdx.x - item * U);
    } else {
        const int units = a.B * U;
        w.split = blockIdx.x / units;
        w.unit = blockIdx.x - w.split * units;
        w.b = w.unit / U;
        chunk = a.chunk;
        w.len = seq_len_of(a, w.b);
        w.nsplit = w.len == 0 ? 1 : (w.len + chunk - 1) / chunk;
    }
    if (w.split >= w.nsplit) return false;
    w.t0 = w.split * chunk;
    w.t1 = min(w.len, w.t0 + chunk);
    return true;
}

// In-kernel one-round split plan of a ragged batch (a.fit_items > 0; at most
// kFitMaxSeqs sequences, one per lane).  The decode grid has fit_items x U
// workgroups.  Each wave derives the same plan from the device lengths with
// lane operations only, so it needs no LDS, no barrier and no separate
// schedule launch:
// * chunk = the smallest multiple c of the tile granularity with
//   sum_b max(1, ceil(len_b / c)) <= fit_items, i.e. every item runs in the
//   first round and the launch takes as long as its largest item.  Lanes test
//   64 candidates at a time between total / S and total / (S - B) (the sum is
//   below total / c + B, so the upper end always fits), narrowing until the
//   candidates are one granule apart.
// * sequence b splits into n_b = max(1, ceil(len_b / c)) equal chunks of
//   round_up(ceil(len_b / n_b), gran) <= c tokens (its last split is not a
//   small remainder); items are numbered sequence by sequence, and the items
//   before sequence b are also its first partial record (rec).
__device__ __forceinline__ int fit_items_for(int len_sgpr, int c) {
    return len_sgpr == 0 ? 1 : static_cast<int>((static_cast<unsigned>(len_sgpr) + c - 1) / static_cast<unsigned>(c));
}

__device__ inline bool locate_fit(const DecodeArgs& a, SplitWork& w) {
    const int lane = threadIdx.x & (kWave - 1);
    const int B = a.B;
    const int S = a.fit_items;
    const int gran = a.fit_gran;
    const int len = lane < B ? seq_len_of(a, lane) : 0;
    long long total = len;
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) total += __shfl_xor(total, off);
    auto round_g = [&](long long x) { return (x + gran - 1) / gran * gran; };
    auto clamp_ll = [](long long x, long long l, long long h) { return x < l ? l : (x > h ? h : x); };
    const int cmax = static_cast<int>(round_g(max(a.max_len, 1)));
    const int lo0 = static_cast<int>(clamp_ll(round_g((total + S - 1) / S), gran, cmax));
    int lo = lo0;
    int hi = S > B ? static_cast<int>(clamp_ll(round_g((total + (S - B) - 1) / (S - B)), lo0, cmax)) : cmax;
    int chunk = hi;
    for (;;) {
        const int step = max(gran, static_cast<int>(round_g((hi - lo + kWave - 2) / (kWave - 1))));
        const int c = min(hi, lo + lane * step);
        int n = 0;
        for (int j = 0; j < B; j++) n += fit_items_for(__builtin_amdgcn_readlane(len, j), c);
        int best = n <= S ? c : INT_MAX;
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) best = min(best, __shfl_xor(best, off));
        chunk = best;  // hi always fits
        if (step == gran) break;
        lo = max(lo, best - step + gran);
        hi = best;
    }
    const int nb = lane < B ? fit_items_for(len, chunk) : 0;
    const int cb = lane < B && len > 0 ? static_cast<int>(round_g((len + nb - 1) / nb)) : gran;
    const int incl = wave_inclusive_scan(nb);
    const int count = __builtin_amdgcn_readlane(incl, kWave - 1);
    const int U = a.Hkv * a.nsg;
    const int item = blockIdx.x / U;
    if (item >= count) return false;
    const int excl = incl - nb;
    const int b = __builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < B && excl <= item)) - 1;
    w.b = b;
    w.rec = __builtin_amdgcn_readlane(excl, b);
    w.split = item - w.rec;
    w.unit = b * U + (blockIdx.x - item * U);
    w.len = __builtin_amdgcn_readlane(len, b);
    w.nsplit = __builtin_amdgcn_readlane(nb, b);
    const int cs = __builtin_amdgcn_readlane(cb, b);
    w.t0 = w.split * cs;
    w.t1 = min(w.len, w.t0 + cs);
    return true;
}

// In-kernel longest-first schedule (a.lpt_target > 0): a ragged batch of
// S < B <= kLptMaxSeqs sequences, S = a.lpt_target / U items per round.
// Every workgroup derives the multi-round schedule of schedule_kernel from the
// lengths and takes its own item, so the decode step needs no schedule
// launch:
// * chunk = the tokens of all sequences times U over the target, rounded up
//   to the granularity, at most the longest possible sequence;
// * items: the whole chunks of every sequence first (sequence order, split
//   order), then each sequence's last chunk, longest first (kSizeClasses
//   size classes, sequence order within a class) -- list scheduling in
//   longest-processing-time order; split s of sequence b covers tokens
//   [s * chunk, (s + 1) * chunk), its first record is the splits of the
//   sequences before b.
// When no sequence is longer than the chunk (every sequence one item) the
// workgroup orders the sequences by their whole lengths, counted while the
// chunk is still being summed, and skips the scans of whole chunks and
// records.  Two sequences per thread (b = 2t + k) of a 256-thread
// workgroup; scratch in LDS that the kernel reuses after the call (no read of
// it follows the last barrier), and pick: 5 ints of LDS that stay.
constexpr int kLptThreads = 256;
constexpr int kLptPerThread = kLptMaxSeqs / kLptThreads;
constexpr int kLptWaves = kLptThreads / kWave;
constexpr int kLptGroups = kLptMaxSeqs / kWave;
struct LptScratch {
    unsigned long long bits[kSizeClasses][kLptGroups];  // sequences 64 g + i whose last chunk has class c
    int len[kLptMaxSeqs];
    int rec[kLptMaxSeqs];  // first record of each sequence (when some sequence splits)
    int hist[kSizeClasses];
    unsigned long long total;  // length sum, counted by one atomic per wave
    int longest;               // longest length, likewise
    int red[2][kLptWaves];     // per wave: splits, whole chunks
};

// Lowest set lane of a wave mask, 0 for an empty mask (index clamp).
__device__ __forceinline__ int first_lane(unsigned long long m) { return m ? __builtin_ctzll(m) : 0; }

// Sequence b of the j-th last chunk in longest-first order (wave 0; j below
// the class counts' sum, B, so every mask below has a lane; the clamps only
// keep indices in range).
__device__ __forceinline__ int lpt_select(const LptScratch& s, int j, int lane, int B) {
    const int c = s.hist[lane];
    const int incl = wave_inclusive_scan(c);
    const int cls = first_lane(__builtin_amdgcn_ballot_w64(incl > j));
    j -= __builtin_amdgcn_readlane(incl - c, cls);
    const int p = lane < kLptGroups ? __builtin_popcountll(s.bits[cls][lane]) : 0;
    const int incl2 = wave_inclusive_scan(p);
    const int grp = min(first_lane(__builtin_amdgcn_ballot_w64(incl2 > j)), kLptGroups - 1);
    j -= __builtin_amdgcn_readlane(incl2 - p, grp);
    const unsigned long long word = s.bits[cls][grp];
    const bool hit = ((word >> lane) & 1ull) && __builtin_popcountll(word & ((1ull << lane) - 1ull)) == j;
    return min(grp * kWave + first_lane(__builtin_amdgcn_ballot_w64(hit)), B - 1);
}

__device__ inline bool locate_lpt(const DecodeArgs& a, SplitWork& w, LptScratch& s, int* pick) {
    const int U = a.Hkv * a.nsg;
    const int item = blockIdx.x / U;
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const int B = a.B;
    const int gran = a.fit_gran;
    // The device lengths (never null under this plan), loaded unconditionally
    // at in-bounds indices so that the loads are in flight together,
    // while the class counts are cleared.
    int len[kLptPerThread];
#pragma unroll
    for (int k = 0; k < kLptPerThread; k++) len[k] = a.lengths[min(kLptPerThread * t + k, B - 1)];
    auto clear_classes = [&]() {
        unsigned long long* const bits = &s.bits[0][0];
#pragma unroll
        for (int i = 0; i < kSizeClasses * kLptGroups / kLptThreads; i++) bits[t + i * kLptThreads] = 0ull;
        if (t < kSizeClasses) s.hist[t] = 0;
    };
    if (t == 0) {
        s.total = 0ull;
        s.longest = 0;
    }
    auto add_class = [&](int b, int c) {
        atomicAdd(&s.hist[c], 1);
        atomicOr(&s.bits[c][b / kWave], 1ull << (b % kWave));
    };
    clear_classes();
    __syncthreads();
    // The classes as whole sequences (chunk = cmax), which order the items
    // longest first whenever no sequence splits, whatever the chunk.
    const unsigned gm = static_cast<unsigned>(gran) - 1u;
    const int cmax = static_cast<int>((static_cast<unsigned>(max(a.max_len, 1)) + gm) & ~gm);
    long long sum = 0;
    int mx = 0;
#pragma unroll
    for (int k = 0; k < kLptPerThread; k++) {
        const int b = kLptPerThread * t + k;
        len[k] = b < B ? min(max(len[k], 0), a.max_len) : 0;
        sum += len[k];
        mx = max(mx, len[k]);
        if (b < B) {
            s.len[b] = len[k];
            add_class(b, last_chunk_class<kSizeClasses>(cmax, len[k]));
        }
    }
    // Lane sums are below 2^32: the wave sums of their low 20 bits and of the
    // rest stay below 2^26 and 2^18.
    const int lo = wave_inclusive_scan(static_cast<int>(sum & 0xFFFFF));
    const int hi = wave_inclusive_scan(static_cast<int>(sum >> 20));
    const int wm = wave_inclusive_max_nonneg(mx);
    if (lane == kWave - 1) {
        atomicAdd(&s.total, (static_cast<unsigned long long>(static_cast<unsigned>(hi)) << 20) + static_cast<unsigned>(lo));
        atomicMax(&s.longest, wm);
    }
    __syncthreads();
    const long long total = static_cast<long long>(s.total);
    const int longest = s.longest;
    // chunk = min(cmax, max(gran, round_up(ceil(total * U / target), gran)))
    // without divides: gran and the target are powers of two.
    const long long num = total * U;
    int chunk = cmax;
    if (num < (static_cast<long long>(cmax) << a.lpt_target_log2)) {
        const int want = static_cast<int>((num + (1ll << a.lpt_target_log2) - 1) >> a.lpt_target_log2);
        chunk = min(cmax, max(gran, static_cast<int>((static_cast<unsigned>(want) + gm) & ~gm)));
    }

    if (longest <= chunk) {
        // Every sequence is one item: item j is the j-th longest.
        if (item >= B) return false;
        if (wave == 0) {
            const int b = lpt_select(s, item, lane, B);
            if (lane == 0) {
                pick[0] = b;
                pick[1] = 0;
                pick[2] = 1;
                pick[3] = b;
                pick[4] = s.len[b];
            }
        }
    } else {
        // Some sequence splits: the classes of the last chunks replace those
        // of the whole sequences.
        clear_classes();
        __syncthreads();
        int n[kLptPerThread], full[kLptPerThread];
        int nt = 0, ft = 0;
#pragma unroll
        for (int k = 0; k < kLptPerThread; k++) {
            const int b = kLptPerThread * t + k;
            n[k] = b < B ? (len[k] == 0 ? 1 : (len[k] + chunk - 1) / chunk) : 0;
            full[k] = b < B ? n[k] - 1 : 0;
            if (b < B) add_class(b, last_chunk_class<kSizeClasses>(chunk, len[k] - full[k] * chunk));
            nt += n[k];
            ft += full[k];
        }
        const int in = wave_inclusive_scan(nt);
        const int inf = wave_inclusive_scan(ft);
        if (lane == kWave - 1) {
            s.red[0][wave] = in;
            s.red[1][wave] = inf;
        }
        __syncthreads();
        int r = in - nt, f = inf - ft, whole = 0;
#pragma unroll
        for (int v = 0; v < kLptWaves; v++) {
            r += v < wave ? s.red[0][v] : 0;
            f += v < wave ? s.red[1][v] : 0;
            whole += s.red[1][v];
        }
        if (item >= whole + B) return false;
#pragma unroll
        for (int k = 0; k < kLptPerThread; k++) {
            const int b = kLptPerThread * t + k;
            if (b < B) {
                s.rec[b] = r;
                if (item >= f && item < f + full[k]) {
                    pick[0] = b;
                    pick[1] = item - f;
                    pick[2] = n[k];
                    pick[3] = r;
                    pick[4] = len[k];
                }
            }
            r += n[k];
            f += full[k];
        }
        __syncthreads();
        if (item >= whole && wave == 0) {
            const int b = lpt_select(s, item - whole, lane, B);
            if (lane == 0) {
                const int lb = s.len[b];
                const int nb = lb == 0 ? 1 : (lb + chunk - 1) / chunk;
                pick[0] = b;
                pick[1] = nb - 1;
                pick[2] = nb;
                pick[3] = s.rec[b];
                pick[4] = lb;
            }
        }
    }
    __syncthreads();
    w.b = pick[0];
    w.split = pick[1];
    w.nsplit = pick[2];
    w.rec = pick[3];
    w.len = pick[4];
    w.unit = w.b * U + (blockIdx.x - item * U);
    w.t0 = w.split * chunk;
    w.t1 = min(w.len, w.t0 + chunk);
    return true;
}

// Partial record of row bhq0 + h, split s: r0 + h * hs + s * ss (records of
// 2 floats in part_ml, d floats in part_acc).
struct RecMap {
    size_t r0;
    int hs, ss;
};

// Records of static splits: [B, Hq, splits].
__device__ __forceinline__ RecMap rec_map_static(const DecodeArgs& a, size_t bhq0) {
    return {bhq0 * a.splits, a.splits, 1};
}

// Records of workgroup w's sequence: under the in-kernel plans (locate_fit,
// locate_lpt) or the split schedule, split s of sequence b owns records
// (w.rec + s) * Hq + hq;
// otherwise static splits.
__device__ __forceinline__ RecMap rec_map(const DecodeArgs& a, const SplitWork& w, size_t bhq0) {
    if (a.fit_items > 0 || a.sched || a.lpt_target > 0)
        return {static_cast<size_t>(w.rec) * a.Hq + (bhq0 - static_cast<size_t>(w.b) * a.Hq), 1, a.Hq};
    return rec_map_static(a, bhq0);
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

// Log-sum-exp merge of the nsplit partial records of row bhq0 + h, element dim.
__device__ inline float merge_dim(const DecodeArgs& a, const RecMap& map, int h, int dim, int nsplit) {
    const size_t r = map.r0 + static_cast<size_t>(h) * map.hs;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, get_coherent(a.part_ml + (r + static_cast<size_t>(s) * map.ss) * 2));
    float L = 0.0f, A = 0.0f;
    for (int s = 0; s < nsplit; s++) {
        const size_t rec = r + static_cast<size_t>(s) * map.ss;
        const float w = fast_exp2(get_coherent(a.part_ml + rec * 2) - M);
        L = fmaf(get_coherent(a.part_ml + rec * 2 + 1), w, L);
        A = fmaf(get_coherent(a.part_acc + rec * a.d + dim), w, A);
    }
    return A / L;
}

// One output element of a workgroup's result, row bhq0 + h: the final value
// when the sequence has one split, otherwise this split's partial record.
__device__ __forceinline__ void store_result(const DecodeArgs& a, const RecMap& map, size_t bhq0, int h, int dim,
                                             int split, int nsplit, float M, float L, float A) {
    if (nsplit == 1) {
        a.out[(bhq0 + h) * a.d + dim] = A / L;
    } else {
        const size_t rec = map.r0 + static_cast<size_t>(h) * map.hs + static_cast<size_t>(split) * map.ss;
        put_coherent(a.part_acc + rec * a.d + dim, A);
        if (dim == 0) {
            put_coherent(a.part_ml + rec * 2, M);
            put_coherent(a.part_ml + rec * 2 + 1, L);
        }
    }
}

// Merge of one sequence group's records by a whole workgroup (nheads <=
// kMergeHeads, nsplit <= kMergeSplits, nheads * nsplit <= 8 per thread, d % 4
// == 0, the group's records below 2 GiB; merge_group_fits).  Every load is issued with as many others in flight as registers
// allow, since the merge runs after the rest of the launch has drained and
// its latency adds directly to the step time:
// 1. one coherent 8-byte load per (head, split) for (m, l), into LDS;
// 2. per head (one wave each): M = max m, the weights exp2(m - M) and
//    L = sum l * weight;
// 3. the accumulators as coherent 16-byte loads, 16 in flight per thread,
//    threads splitting the splits of a column when there are fewer columns
//    than threads; out = (sum acc * weight) / L.
constexpr int kMergeHeads = 8;
constexpr int kMergeSplits = 256;
constexpr int kMergeMaxThreads = 512;
constexpr int kMergePairsPerThread = 8;  // (m, l) loads per thread in phase 1
constexpr int kCoherent = 16;  // buffer-load cache policy: sc1, device-coherent (as get_coherent)

// Records spanned by the group's merge (relative to map.r0).
__device__ __forceinline__ long merge_span(const RecMap& map, int nheads, int nsplit) {
    return static_cast<long>(nheads - 1) * map.hs + static_cast<long>(nsplit - 1) * map.ss + 1;
}

__device__ inline bool merge_group_fits(const DecodeArgs& a, const RecMap& map, int nheads, int nsplit) {
    return nheads <= kMergeHeads && nsplit <= kMergeSplits && (a.d & 3) == 0 &&
           merge_span(map, nheads, nsplit) * a.d < (1L << 29) && blockDim.x <= kMergeMaxThreads &&
           nheads * nsplit <= kMergePairsPerThread * static_cast<int>(blockDim.x);
}

// merge_group's LDS, provided by the kernel (which may overlay it on LDS it is
// done with by the time finish_split's first barrier has passed).
struct MergeScratch {
    float w[kMergeHeads][kMergeSplits];  // m, then the weights
    float L[kMergeHeads];
    union {
        float l[kMergeHeads][kMergeSplits];  // phases 1-2
        float4 part[kMergeMaxThreads];       // phase 3
    } x;
};

__device__ inline void merge_group(const DecodeArgs& a, const RecMap& map, size_t bhq0, int nheads, int nsplit,
                                   MergeScratch& ms) {
    auto& s_w = ms.w;
    auto& s_L = ms.L;
    auto& s_x = ms.x;
    const int T = blockDim.x;
    const int t = threadIdx.x;
    const int lane = t & (kWave - 1);
    const int wave = t / kWave;
    const int nw = T / kWave;
    const int d = a.d;
    const int hs = map.hs, ss = map.ss;
    const unsigned span = static_cast<unsigned>(merge_span(map, nheads, nsplit));
    const buf_rsrc mlr = make_rsrc(a.part_ml + map.r0 * 2, span * 8u);
    const buf_rsrc accr = make_rsrc(a.part_acc + map.r0 * d, span * static_cast<unsigned>(d) * 4u);

    const int npairs = nheads * nsplit;  // <= kMergePairsPerThread * T (merge_group_fits)
#pragma unroll
    for (int k = 0; k < kMergePairsPerThread; k++) {
        const int i = t + k * T;
        if (i < npairs) {
            const int h = i / nsplit;
            const int sp = i - h * nsplit;
            typedef int v2i_t __attribute__((ext_vector_type(2)));
            const v2i_t x = __builtin_amdgcn_raw_buffer_load_b64(mlr, (h * hs + sp * ss) * 8, 0, kCoherent);
            s_w[h][sp] = __int_as_float(x.x);
            s_x.l[h][sp] = __int_as_float(x.y);
        }
    }
    __syncthreads();
    for (int h = wave; h < nheads; h += nw) {
        float mx = -INFINITY;
        for (int sp = lane; sp < nsplit; sp += kWave) mx = fmaxf(mx, s_w[h][sp]);
        mx = wave_max(mx);
        const float M = mx == -INFINITY ? 0.0f : mx;
        float L = 0.0f;
        for (int sp = lane; sp < nsplit; sp += kWave) {
            const float w = fast_exp2(s_w[h][sp] - M);
            s_w[h][sp] = w;
            L = fmaf(s_x.l[h][sp], w, L);
        }
        L = wave_sum(L);
        if (lane == 0) s_L[h] = L;
    }
    __syncthreads();
    const int cpr = d >> 2;  // 16-byte columns per head
    const int ncols = nheads * cpr;
    const int groups = max(1, min(T / ncols, nsplit));
    for (int item = t; item < ncols * groups; item += T) {
        const int j = item / ncols;
        const int c = item - j * ncols;
        const int h = c / cpr;
        const int off0 = (h * hs * d + 4 * (c - h * cpr)) * 4;
        float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int sp0 = j; sp0 < nsplit; sp0 += 16 * groups) {
            v4i_t v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const int sp = sp0 + k * groups;
                v[k] = sp < nsplit ? __builtin_amdgcn_raw_buffer_load_b128(accr, off0 + sp * ss * d * 4, 0, kCoherent)
                                   : v4i_t{0, 0, 0, 0};
            }
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const int sp = sp0 + k * groups;
                const float w = sp < nsplit ? s_w[h][sp] : 0.0f;
                A.x = fmaf(__int_as_float(v[k].x), w, A.x);
                A.y = fmaf(__int_as_float(v[k].y), w, A.y);
                A.z = fmaf(__int_as_float(v[k].z), w, A.z);
                A.w = fmaf(__int_as_float(v[k].w), w, A.w);
            }
        }
        if (groups > 1) {
            s_x.part[item] = A;
        } else {
            float* o = a.out + (bhq0 + h) * d + 4 * (c - h * cpr);
            const float L = s_L[h];
            o[0] = A.x / L, o[1] = A.y / L, o[2] = A.z / L, o[3] = A.w / L;
        }
    }
    if (groups > 1) {
        __syncthreads();
        for (int c = t; c < ncols; c += T) {
            float4 A = s_x.part[c];
            for (int j = 1; j < groups; j++) {
                const float4 x = s_x.part[j * ncols + c];
                A.x += x.x, A.y += x.y, A.z += x.z, A.w += x.w;
            }
            const int h = c / cpr;
            float* o = a.out + (bhq0 + h) * d + 4 * (c - h * cpr);
            const float L = s_L[h];
            o[0] = A.x / L, o[1] = A.y / L, o[2] = A.z / L, o[3] = A.w / L;
        }
    }
}

// Merge of at most kFlatSplits splits in one round trip: one thread per
// (head, 16-byte output column) loads that head's (m, l) and its accumulator
// column of every split together, then combines them in registers -- no LDS,
// no barrier, against merge_group's two load phases and three barriers (cfg2:
// 36.6 -> 34.1 us).  Same conditions as merge_group otherwise.
constexpr int kFlatSplits = 16;

__device__ inline void merge_flat(const DecodeArgs& a, const RecMap& map, size_t bhq0, int nheads, int nsplit) {
    const int d = a.d;
    const int cpr = d >> 2;
    const unsigned span = static_cast<unsigned>(merge_span(map, nheads, nsplit));
    const buf_rsrc mlr = make_rsrc(a.part_ml + map.r0 * 2, span * 8u);
    const buf_rsrc accr = make_rsrc(a.part_acc + map.r0 * d, span * static_cast<unsigned>(d) * 4u);
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    for (int c = threadIdx.x; c < nheads * cpr; c += blockDim.x) {
        const int h = c / cpr;
        const int col = c - h * cpr;
        v2i_t ml[kFlatSplits];
        v4i_t acc[kFlatSplits];
#pragma unroll
        for (int k = 0; k < kFlatSplits; k++) {
            const int rec = h * map.hs + k * map.ss;
            if (k < nsplit) {
                ml[k] = __builtin_amdgcn_raw_buffer_load_b64(mlr, rec * 8, 0, kCoherent);
                acc[k] = __builtin_amdgcn_raw_buffer_load_b128(accr, (rec * d + 4 * col) * 4, 0, kCoherent);
            }
        }
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < kFlatSplits; k++)
            if (k < nsplit) M = fmaxf(M, __int_as_float(ml[k].x));
        const float Ms = M == -INFINITY ? 0.0f : M;
        float L = 0.0f;
        float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < kFlatSplits; k++) {
            if (k < nsplit) {
                const float w = fast_exp2(__int_as_float(ml[k].x) - Ms);
                L = fmaf(__int_as_float(ml[k].y), w, L);
                A.x = fmaf(__int_as_float(acc[k].x), w, A.x);
                A.y = fmaf(__int_as_float(acc[k].y), w, A.y);
                A.z = fmaf(__int_as_float(acc[k].z), w, A.z);
                A.w = fmaf(__int_as_float(acc[k].w), w, A.w);
            }
        }
        float* o = a.out + (bhq0 + h) * d + 4 * col;
        o[0] = A.x / L, o[1] = A.y / L, o[2] = A.z / L, o[3] = A.w / L;
    }
}

// Merge of 17 to 2 * kFlatSplits splits in one round trip: two adjacent
// lanes per (head, 16-byte output column), lane half j taking splits j,
// j + 2, ...; the pair exchanges its maxima, then its sums and accumulators,
// with lane shuffles (no LDS, no barrier), as merge_flat does for one lane.
__device__ inline void merge_flat_pairs(const DecodeArgs& a, const RecMap& map, size_t bhq0, int nheads,
                                        int nsplit) {
    const int d = a.d;
    const int cpr = d >> 2;
    const unsigned span = static_cast<unsigned>(merge_span(map, nheads, nsplit));
    const buf_rsrc mlr = make_rsrc(a.part_ml + map.r0 * 2, span * 8u);
    const buf_rsrc accr = make_rsrc(a.part_acc + map.r0 * d, span * static_cast<unsigned>(d) * 4u);
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    const int half = threadIdx.x & 1;
    // Every lane of a wave runs the same number of iterations (blockDim is a
    // multiple of 64), so the shuffles below always have their partner.
    for (int c0 = threadIdx.x >> 1; c0 < ((nheads * cpr + kWave / 2 - 1) / (kWave / 2)) * (kWave / 2);
         c0 += blockDim.x >> 1) {
        const bool live = c0 < nheads * cpr;
        const int c = live ? c0 : 0;
        const int h = c / cpr;
        const int col = c - h * cpr;
        v2i_t ml[kFlatSplits];
        v4i_t acc[kFlatSplits];
#pragma unroll
        for (int k = 0; k < kFlatSplits; k++) {
            const int sp = 2 * k + half;
            const int rec = h * map.hs + sp * map.ss;
            if (sp < nsplit) {
                ml[k] = __builtin_amdgcn_raw_buffer_load_b64(mlr, rec * 8, 0, kCoherent);
                acc[k] = __builtin_amdgcn_raw_buffer_load_b128(accr, (rec * d + 4 * col) * 4, 0, kCoherent);
            }
        }
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < kFlatSplits; k++)
            if (2 * k + half < nsplit) M = fmaxf(M, __int_as_float(ml[k].x));
        M = fmaxf(M, __shfl_xor(M, 1));
        const float Ms = M == -INFINITY ? 0.0f : M;
        float L = 0.0f;
        float4 A = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < kFlatSplits; k++) {
            if (2 * k + half < nsplit) {
                const float w = fast_exp2(__int_as_float(ml[k].x) - Ms);
                L = fmaf(__int_as_float(ml[k].y), w, L);
                A.x = fmaf(__int_as_float(acc[k].x), w, A.x);
                A.y = fmaf(__int_as_float(acc[k].y), w, A.y);
                A.z = fmaf(__int_as_float(acc[k].z), w, A.z);
                A.w = fmaf(__int_as_float(acc[k].w), w, A.w);
            }
        }
        L += __shfl_xor(L, 1);
        A.x += __shfl_xor(A.x, 1);
        A.y += __shfl_xor(A.y, 1);
        A.z += __shfl_xor(A.z, 1);
        A.w += __shfl_xor(A.w, 1);
        if (live && half == 0) {
            float* o = a.out + (bhq0 + h) * d + 4 * col;
            o[0] = A.x / L, o[1] = A.y / L, o[2] = A.z / L, o[3] = A.w / L;
        }
    }
}

// Called by every thread of a workgroup after its store_result calls: counts
// the split's arrival and, in the last workgroup of the work unit, merges the
// records of rows [bhq0, bhq0 + nheads).  s_last: one int of LDS; ms: LDS
// that nothing reads or writes after finish_split's first barrier.  FLAT: up
// to kFlatSplits splits merge with merge_flat, up to twice that with
// merge_flat_pairs (their registers are not worth taking from the FMA
// kernel, whose ragged batches rarely split).
template <bool FLAT = false>
__device__ __forceinline__ void finish_split(const DecodeArgs& a, int unit, const RecMap& map, size_t bhq0,
                                             int nheads, int nsplit, int* s_last, MergeScratch& ms) {
    if (nsplit <= 1 || a.counters == nullptr) return;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's record stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(a.counters + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *s_last = (prev == nsplit - 1);
    }
    __syncthreads();
    if (*s_last) {
        if (FLAT && nsplit <= kFlatSplits && merge_group_fits(a, map, nheads, nsplit)) {
            merge_flat(a, map, bhq0, nheads, nsplit);
        } else if (FLAT && nsplit <= 2 * kFlatSplits && merge_group_fits(a, map, nheads, nsplit)) {
            merge_flat_pairs(a, map, bhq0, nheads, nsplit);
        } else if (merge_group_fits(a, map, nheads, nsplit)) {
            merge_group(a, map, bhq0, nheads, nsplit, ms);
        } else {
            for (int i = threadIdx.x; i < nheads * a.d; i += blockDim.x) {
                const int h = i / a.d;
                const int dim = i - h * a.d;
                a.out[(bhq0 + h) * a.d + dim] = merge_dim(a, map, h, dim, nsplit);
            }
        }
        if (threadIdx.x == 0)  // ready for the next launch
            __hip_atomic_store(a.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace kvq
