// kvq_capi.cpp -- the extern "C" surface of libkvq.so (declared in include/kvq.h).
//
// Every entry point validates its arguments before making any HIP call, so the
// error paths (null pointers, bad shapes, undersized workspace) are testable on
// a machine without a GPU, as in kv_cache/KV_int8_split_optimized.cu:272-273.
#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <functional>
#include <map>
#include <mutex>
#include <vector>

#include "../../include/kvq.h"
#include "kvq_internal.hpp"

namespace {

using kvq::DecodeArgs;
using kvq::DecodePlan;

constexpr float kLog2e = 1.4426950408889634f;
constexpr size_t kAlign = 256;
// Arrival counters live in a fixed-size prefix of every workspace, so a
// workspace zero-filled once stays valid for any later problem shape: the
// counters are only ever written as counters (and left at zero), partial
// records always start after the prefix.  Problems with more sequence groups
// than counters use the separate merge kernel instead.
constexpr size_t kCounterBytes = 256 * 1024;
constexpr long kMaxCounters = static_cast<long>(kCounterBytes / sizeof(int));
// Workgroups a decode launch aims for when it picks the split count itself
// (MI355X: 256 CUs).  An 8-wave VALU workgroup fills a CU's issue slots on its
// own.  A 4-wave MFMA workgroup streams faster alone on a CU than two sharing
// one (cfg3: 48.0 us at 256 workgroups, 52.0 us at 512, 62.3 us at 384), and
// its split count rounds down so the grid stays within one round.
constexpr int kTargetWorkgroupsValu = 256;
#ifndef KVQ_TARGET_WG_MFMA
#define KVQ_TARGET_WG_MFMA 256
#endif
constexpr int kTargetWorkgroupsMfma = KVQ_TARGET_WG_MFMA;
// Below this many K/V bytes per (sequence, kv head) a chosen split count is 1:
// a split's merge (record stores, arrival atomic, far reads) costs more than
// the parallelism saves (B1 H8 d64 L1024: 7.65 us unsplit, 9.8 us in 4
// splits; from 264 KB per unit the split plans win).
constexpr long kMinSplitUnitBytes = 192 * 1024;
// The same for the device split schedule of a ragged batch (work items of
// equal size, so the target is the number of chunks over the whole batch).
#ifndef KVQ_SCHED_TARGET_VALU
#define KVQ_SCHED_TARGET_VALU 512
#endif
// Items per work unit of a ragged batch planned inside the matrix-core kernel
// (one round): one 4-wave workgroup per CU streams faster than two (cfg2:
// 36.7 us at 256, 38.5 us at 512, 47.8 us at 768).
// The same for the 8-wave FMA kernel, two of which share a CU (a ragged
// B8 H32 d128 MHA batch: 59.8 us, against 63.7 us with the schedule launch).
#ifndef KVQ_FIT_TARGET_VALU
#define KVQ_FIT_TARGET_VALU 512
#endif
// Workgroups of the few-query attention kernel: one 4-wave workgroup per CU
// streams best for one query (M = 1, N = 65536, d = 128: 15.6 us at 256,
// 17.0 at 512), two per CU hide the ALU work of more (M = 2: 21.1 us at 256;
// M = 8: 44.5 us at 256, 31.4 at 512, 37.3 at 1024).
#ifndef KVQ_ATTN_ROWS_TARGET
#define KVQ_ATTN_ROWS_TARGET(qm) ((qm) <= 1 ? 256 : 512)
#endif
#ifndef KVQ_FIT_TARGET_MFMA
#define KVQ_FIT_TARGET_MFMA 256
#endif
#ifndef KVQ_SCHED_TARGET_MFMA
#define KVQ_SCHED_TARGET_MFMA 512
#endif

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Diagnostic switches, read once from the environment on first use:
// * KVQ_DEBUG_SYNC: on ("1", "true", "yes", "on"), every launching entry point
//   synchronises its stream after its launches and returns the first error,
//   so an asynchronous fault is reported by the call that caused it (the
//   reference's compile-time KV_CUDA_DEBUG_SYNC,
//   kv_cache/KV_int8_split_optimized.cu:16-18,253-264).  Skipped while the
//   stream is being captured into a graph.
// * KVQ_FORCE_KERNEL: "valu" keeps decode plans off the matrix-core kernel,
//   "generic" off both tuned kernels, so one problem can be profiled on either
//   kernel.  Any other value changes nothing.
// * KVQ_PREFILL_MAX_GROUPS: a positive integer caps the prefill quantiser's
//   workgroups per plane (default and maximum 2^20), so tests can run its
//   grid-stride loop on small inputs.
bool env_on(const char* name) {
    const char* s = getenv(name);
    if (!s) return false;
    static const char* const kOn[] = {"1", "true", "yes", "on", "TRUE", "YES", "ON", "True", "Yes", "On"};
    for (const char* o : kOn)
        if (strcmp(s, o) == 0) return true;
    return false;
}

bool debug_sync() {
    static const bool on = env_on("KVQ_DEBUG_SYNC");
    return on;
}

enum ForcedKernel { kForceNone = 0, kForceValu = 1, kForceGeneric = 2 };

// KVQ_FLAT_PLAN=0 keeps ragged matrix-core batches on the per-sequence item
// plan (locate_fit), for comparison.
bool flat_enabled() {
    static const bool on = [] {
        const char* s = getenv("KVQ_FLAT_PLAN");
        return !(s && strcmp(s, "0") == 0);
    }();
    return on;
}

// KVQ_SCHEDULE_LAUNCH=1 keeps the separate schedule launch for the ragged
// matrix-core batches whose schedule the decode kernel derives itself
// (locate_lpt), for comparison.
bool lpt_enabled() {
    static const bool on = !env_on("KVQ_SCHEDULE_LAUNCH");
    return on;
}

unsigned prefill_max_groups() {
    static const unsigned g = [] {
        const char* s = getenv("KVQ_PREFILL_MAX_GROUPS");
        if (!s || !*s) return 0u;
        char* end = nullptr;
        const long v = strtol(s, &end, 10);
        return (*end == '\0' && v > 0 && v <= (1L << 20)) ? static_cast<unsigned>(v) : 0u;
    }();
    return g;
}

int forced_kernel() {
    static const int k = [] {
        const char* s = getenv("KVQ_FORCE_KERNEL");
        if (s && strcmp(s, "valu") == 0) return static_cast<int>(kForceValu);
        if (s && strcmp(s, "generic") == 0) return static_cast<int>(kForceGeneric);
        return static_cast<int>(kForceNone);
    }();
    return k;
}

// The library's code objects are built for gfx950 only.  Checked once per
// device before its first launch, as the reference warns once about an
// untuned architecture (kv_cache/KV_int8_split_optimized.cu:57-65); here
// another architecture cannot run the kernels at all, so the call fails with
// hipErrorInvalidDevice after one stderr line.
std::mutex g_arch_mutex;
signed char g_arch_state[64];  // 0 unknown, 1 gfx950, -1 other

hipError_t arch_check() {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_arch_mutex);
    if (g_arch_state[dev] == 0) {
        hipDeviceProp_t prop;
        err = hipGetDeviceProperties(&prop, dev);
        if (err != hipSuccess) return err;
        const bool ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
                        (prop.gcnArchName[6] == '\0' || prop.gcnArchName[6] == ':');
        g_arch_state[dev] = ok ? 1 : -1;
        if (!ok)
            fprintf(stderr, "[kvq] device %d is %s; libkvq is built for gfx950 (MI355X) only\n", dev,
                    prop.gcnArchName);
    }
    return g_arch_state[dev] > 0 ? hipSuccess : hipErrorInvalidDevice;
}

// Every launching entry point returns through here: the device check, the
// launches, then (KVQ_DEBUG_SYNC) the stream's completion status.
hipError_t finish_call(hipError_t err, hipStream_t stream);
template <class Launch>
hipError_t checked_call(hipStream_t stream, Launch&& launch) {
    const hipError_t err = arch_check();
    if (err != hipSuccess) return err;
    return finish_call(launch(), stream);
}

hipError_t finish_call(hipError_t err, hipStream_t stream) {
    if (err != hipSuccess || !debug_sync()) return err;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    err = hipStreamIsCapturing(stream, &st);
    if (err != hipSuccess || st != hipStreamCaptureStatusNone) return err;
    // The launchers already returned their launch status; the caller's own
    // pending error (hipGetLastError) is left for the caller.
    return hipStreamSynchronize(stream);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Split count and workspace layout for one decode problem.
// aligned: q, caches and new rows are 16-byte aligned (vector loads);
// quads: the matrix-core kernel's layout needs hold (scale arrays 16-byte
// aligned, capacity a multiple of 4 and below 2^24);
// page: tokens per page of a paged cache (0: contiguous); a tuned kernel runs
// a paged cache only when no wave tile straddles a page;
// ragged: per-sequence lengths on the device;
// max_splits bounds the splits (scratch capacity of the reference ABI);
// fused selects the arrival-counter merge (workspace holds counters).
DecodePlan make_plan(int B, int Hq, int Hkv, int d, int max_len, bool aligned, bool quads, int page,
                     bool ragged, int requested, int max_splits, bool fused) {
    DecodePlan p{};
    const int G = Hq / Hkv;
    const int sg_m = kvq::mfma_heads_per_group(G, d);
    const int sg_v = kvq::fast_heads_per_group(G);
    const bool pow2 = page > 0 && (page & (page - 1)) == 0;
    const int wave_tokens = kvq::fast_wave_tokens(d, sg_v);
    const bool valu_pages = page == 0 || (pow2 && wave_tokens > 0 && page % wave_tokens == 0);
    const bool mfma_pages = page == 0 || (pow2 && page % 32 == 0 && page < (1 << 24));
    int tile = 0;
    const int force = forced_kernel();
    if (force == kForceGeneric) aligned = false;
    if (force == kForceValu) quads = false;
    if (aligned && quads && mfma_pages && sg_m > 0) {
        p.kernel = kvq::Kernel::Mfma;
        p.sg = sg_m;
        tile = kvq::mfma_tile_tokens();
    } else if (aligned && valu_pages && kvq::fast_tile_tokens(d, sg_v) > 0) {
        p.kernel = kvq::Kernel::Valu;
        p.sg = sg_v;
        tile = kvq::fast_tile_tokens(d, sg_v);
    } else {
        p.kernel = kvq::Kernel::Generic;
        p.sg = 1;
    }
    p.fast = p.kernel != kvq::Kernel::Generic;
    p.tile = tile;
    p.nsg = p.fast ? G / p.sg : G;
    const long units = p.fast ? static_cast<long>(B) * Hkv * p.nsg : static_cast<long>(B) * Hq;
    const int gran = p.fast ? tile : 64;
    max_len = std::max(max_len, 1);
    const int U = Hkv * p.nsg;
    const bool fit_kernel = p.kernel == kvq::Kernel::Mfma || (p.kernel == kvq::Kernel::Valu && p.sg <= 2);
    const int fit_items = (p.kernel == kvq::Kernel::Mfma ? KVQ_FIT_TARGET_MFMA : KVQ_FIT_TARGET_VALU) / U;
    // Flattened tile plan (decode_mfma_flat): the workgroups' waves take
    // equal ranges of the sequences' tiles laid end to end.
    // * A sequence covering w waves is merged from w records by one wave, so
    //   batches averaging over 16 waves per sequence (4 * fit_items waves,
    //   B < fit_items / 4) keep the per-sequence item plan below (two
    //   sequences of 30-60K tokens: 53 us flat, 42 us itemised; B = 8,
    //   4K-32K tokens: 57 / 56 us; B = 16, cfg2: 33.1 / 34.0 us).
    // * Up to 64 sequences it replaces the one-round item plan or schedule
    //   (B64 Hq32/Hkv8 L 1K-8K: 101 us flat, 143 us scheduled; with 8 heads
    //   per kv head and append, L 512-4K: 69 / 83 us).
    // * Beyond 64 the schedule's longest-first rounds balance long steps
    //   better than one static split, whose waves' rate differences add up
    //   (cfg4: 222 us flat, 203 us scheduled -- per-wave stamps: 141 tiles
    //   per wave at 1.46-1.52 us, loop ends 10-14 us apart; B128 L 512-2K:
    //   66 / 62 us), so
    //   the flat plan keeps only small steps, at most 16 tiles per wave for
    //   full-length sequences (B300 L 1-40: 26 / 34 us; B1000 L 0-256: 122 /
    //   125 us).
    // Record ids run to waves + B per query head.
    // The kernel counts the virtual stream (every tile at full length plus
    // kFlatSwitchTiles per sequence) in 32-bit integers.
    const long flat_tiles = static_cast<long>(B) * ((static_cast<long>(max_len) + kvq::kMfmaTile - 1) / kvq::kMfmaTile);
    const bool flat_shape = B <= kvq::kFitMaxSeqs || flat_tiles <= 16L * kvq::kMfmaWaves * fit_items;
    const bool flat_counts = flat_tiles + static_cast<long>(kvq::kFlatSwitchTiles) * B <= INT_MAX;
    if (ragged && requested == 0 && fused && p.kernel == kvq::Kernel::Mfma && fit_items >= 1 &&
        B <= kvq::kFlatMaxSeqs && 4 * B >= fit_items && flat_shape && flat_counts &&
        static_cast<long>(B) * U <= kMaxCounters && max_len <= KVQ_MAX_SEQ_LEN && flat_enabled()) {
        p.fit = true;
        p.flat = true;
        p.counters = true;
        p.sched_items = fit_items;
        p.sched_gran = gran;
        p.splits = 0;
        p.chunk = 0;
        const size_t recs = (static_cast<size_t>(fit_items) * kvq::kMfmaWaves + B) * Hq;
        p.counter_bytes = kCounterBytes;
        p.ml_bytes = round_up(recs * 2 * sizeof(float), kAlign);
        p.acc_bytes = round_up(recs * static_cast<size_t>(d) * sizeof(float), kAlign);
        return p;
    }
    if (ragged && requested == 0 && fused && fit_kernel && units <= kMaxCounters && B <= kvq::kFitMaxSeqs &&
        B <= fit_items && max_len <= KVQ_MAX_SEQ_LEN) {
        // Small ragged batch: every workgroup plans the batch itself from the
        // lengths (one round of at most fit_items items per work unit; no
        // schedule launch).
        p.fit = true;
        p.counters = true;
        p.sched_items = fit_items;
        p.sched_gran = gran;
        p.splits = 0;
        p.chunk = 0;
        const size_t recs = static_cast<size_t>(fit_items) * Hq;
        p.counter_bytes = kCounterBytes;
        p.ml_bytes = round_up(recs * 2 * sizeof(float), kAlign);
        p.acc_bytes = round_up(recs * static_cast<size_t>(d) * sizeof(float), kAlign);
        return p;
    }
    if (ragged && requested == 0 && fused && p.fast && units <= kMaxCounters) {
        // Ragged batch: the split schedule is computed on the device from the
        // lengths.  Items (and records) <= B + target / units per sequence.
        p.scheduled = true;
        p.counters = true;
        p.sched_target = p.kernel == kvq::Kernel::Mfma ? KVQ_SCHED_TARGET_MFMA : KVQ_SCHED_TARGET_VALU;
        p.sched_gran = gran;
        p.sched_items = B + (p.sched_target + U - 1) / U + 1;
        p.splits = 0;
        p.chunk = 0;
        // Beyond one round of items (B > target / U), up to kLptMaxSeqs
        // sequences and a few rounds of B items, the matrix-core kernel
        // derives the schedule itself (locate_lpt): one launch per step
        // instead of two (one box: cfg4 200.9 against 202.9-203.3 us; B128
        // Hq32/Hkv8 L 512-2K 61.3 / 63.0 us; B512 Hq64/Hkv8 L 256-2K 230.5 /
        // 232.6 us; B300 Hq64/Hkv8 L 1-8K 404.8 / 408.2 us).
        p.lpt = p.kernel == kvq::Kernel::Mfma && B > p.sched_target / U && B <= kvq::kLptMaxSeqs &&
                static_cast<long>(B) * U <=
                    static_cast<long>(max_len >= kvq::kLptLongTokens ? kvq::kLptMaxRounds : kvq::kLptMaxRounds / 2) *
                        p.sched_target &&
                (gran & (gran - 1)) == 0 && (p.sched_target & (p.sched_target - 1)) == 0 && max_len <= KVQ_MAX_SEQ_LEN &&
                lpt_enabled();
        const size_t recs = static_cast<size_t>(p.sched_items) * Hq;
        p.counter_bytes = kCounterBytes;
        p.sched_bytes =
            p.lpt ? 0
                  : round_up((kvq::kSchedHeader + kvq::kSchedItemInts * static_cast<size_t>(p.sched_items) +
                              2 * static_cast<size_t>(B)) *
                                 sizeof(int),
                             kAlign);
        p.ml_bytes = round_up(recs * 2 * sizeof(float), kAlign);
        p.acc_bytes = round_up(recs * static_cast<size_t>(d) * sizeof(float), kAlign);
        return p;
    }
    long splits;
    int chunk;
    if (requested > 0) {
        splits = std::min<long>(requested, max_len);
        splits = std::min<long>(splits, std::max(max_splits, 1));
        chunk = static_cast<int>((max_len + splits - 1) / splits);
        // Tuned kernels get chunks of whole workgroup tiles: matrix-core tiles
        // must start at multiples of 4 tokens (aligned scale quads), and in a
        // paged cache no wave tile may straddle a page.  So fewer splits than
        // requested may run.
        if (p.fast && splits > 1) chunk = static_cast<int>(round_up(static_cast<size_t>(chunk), gran));
    } else {
        if (static_cast<long>(max_len) * (2 * d + 8) < kMinSplitUnitBytes)
            splits = 1;
        else if (p.kernel == kvq::Kernel::Mfma)
            splits = std::max<long>(1, kTargetWorkgroupsMfma / units);
        else
            splits = (kTargetWorkgroupsValu + units - 1) / units;
        splits = std::min<long>(splits, (static_cast<long>(max_len) + gran - 1) / gran);
        splits = std::max<long>(1, std::min<long>(splits, std::max(max_splits, 1)));
        chunk = static_cast<int>((max_len + splits - 1) / splits);
        if (splits > 1) chunk = static_cast<int>(round_up(static_cast<size_t>(chunk), gran));
    }
    p.chunk = chunk;
    p.splits = static_cast<int>((static_cast<long>(max_len) + chunk - 1) / chunk);
    if (p.splits > 1) {
        const size_t recs = static_cast<size_t>(B) * Hq * p.splits;
        // A workspace in fused layout always reserves the counter prefix, even
        // for a plan that merges with the separate kernel, so partial records
        // can never land on another plan's counters.
        p.counter_bytes = fused ? kCounterBytes : 0;
        p.counters = fused && p.fast && units <= kMaxCounters;
        p.ml_bytes = round_up(recs * 2 * sizeof(float), kAlign);
        p.acc_bytes = round_up(recs * static_cast<size_t>(d) * sizeof(float), kAlign);
    }
    return p;
}

size_t plan_bytes(const DecodePlan& p) { return p.counter_bytes + p.sched_bytes + p.ml_bytes + p.acc_bytes; }

// Workspace: [counters][split schedule][partial (m, l)][partial accumulators].
void bind_workspace(DecodeArgs& a, const DecodePlan& p, void* ws) {
    char* base = static_cast<char*>(ws);
    a.counters = p.counters ? reinterpret_cast<int*>(base) : nullptr;
    a.sched = p.scheduled && !p.lpt ? reinterpret_cast<const int*>(base + p.counter_bytes) : nullptr;
    a.lpt_target = p.lpt ? p.sched_target : 0;
    a.lpt_target_log2 = p.lpt ? __builtin_ctz(static_cast<unsigned>(p.sched_target)) : 0;
    a.sched_items = p.sched_items;
    a.fit_items = p.fit ? p.sched_items : 0;
    a.flat = p.flat ? 1 : 0;
    a.fit_gran = p.sched_gran;
    const size_t ml = p.counter_bytes + p.sched_bytes;
    a.part_ml = p.ml_bytes ? reinterpret_cast<float*>(base + ml) : nullptr;
    a.part_acc = p.acc_bytes ? reinterpret_cast<float*>(base + ml + p.ml_bytes) : nullptr;
}

bool shape_ok(int H, int N, int d) {
    return H > 0 && N > 0 && N <= KVQ_MAX_SEQ_LEN && d > 0 && d <= KVQ_MAX_HEAD_DIM;
}

// Reference-ABI problem ([H,N,d], one query per head) as a batched problem.
DecodeArgs reference_args(const float* Q, const int8_t* K, const int8_t* V, const float* ks,
                          const float* vs, float* out, int H, int N, int d) {
    DecodeArgs a{};
    a.q = Q;
    a.k = const_cast<int8_t*>(K);
    a.v = const_cast<int8_t*>(V);
    a.ks = const_cast<float*>(ks);
    a.vs = const_cast<float*>(vs);
    a.out = out;
    a.B = 1;
    a.Hq = a.Hkv = H;
    a.G = 1;
    a.cap = N;
    a.d = d;
    a.uniform_len = N;
    a.max_len = N;
    a.scale_log2 = (1.0f / sqrtf(static_cast<float>(d))) * kLog2e;
    return a;
}

bool reference_aligned(const void* Q, const void* K, const void* V, int d) {
    return aligned16(Q) && aligned16(K) && aligned16(V) && (d % 16) == 0;
}

// Plan of kv_int8_split_launch / kv_int8_simple_launch, whose workspace is the
// caller's S of H*N floats.  A split needs (d + 2) floats of records per head,
// but the (m, l) region is padded to kAlign bytes before the accumulators, so
// N / (d + 2) splits can still overrun S by up to kAlign bytes at small H
// (H = 1, N = 516, d = 256: 2 splits need 2304 bytes of a 2064-byte S).  The
// split count therefore steps down until the whole layout fits.
DecodePlan reference_plan(int H, int N, int d, bool aligned) {
    const size_t cap = static_cast<size_t>(H) * static_cast<size_t>(N) * sizeof(float);
    int max_splits = std::max(1, N / (d + 2));
    DecodePlan p = make_plan(1, H, H, d, N, aligned, false, 0, false, 0, max_splits, false);
    while (p.splits > 1 && plan_bytes(p) > cap) {
        max_splits = p.splits - 1;
        p = make_plan(1, H, H, d, N, aligned, false, 0, false, 0, max_splits, false);
    }
    return p;
}

hipError_t reference_launch(const float* Q, const int8_t* K, const int8_t* V, const float* ks,
                            const float* vs, float* out, int H, int N, int d, float* S,
                            hipStream_t stream) {
    if (!Q || !K || !V || !ks || !vs || !out || !S || !shape_ok(H, N, d)) return hipErrorInvalidValue;
    if (static_cast<long long>(H) * N > INT_MAX) return hipErrorInvalidValue;
    DecodeArgs a = reference_args(Q, K, V, ks, vs, out, H, N, d);
    const DecodePlan p = reference_plan(H, N, d, reference_aligned(Q, K, V, d));
    a.splits = p.splits;
    a.chunk = p.chunk;
    a.nsg = p.nsg;
    bind_workspace(a, p, S);
    return checked_call(stream, [&] { return kvq::launch_decode(a, p, stream); });
}

// Library-owned, per-device split workspace for the legacy `solve` ABI.  Grown
// on demand (hipFree waits for in-flight work) and zero-filled on allocation;
// completed launches leave the arrival counters at zero.  `launch(ptr)` is
// enqueued while the lock is held, so a concurrent call that grows the
// workspace frees it only after this launch is on the null stream.
struct SolveWorkspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mutex;
SolveWorkspace g_ws[64];

template <class Launch>
hipError_t with_solve_workspace(size_t need, Launch&& launch) {
    if (need == 0) return launch(nullptr);
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    SolveWorkspace& w = g_ws[dev];
    if (w.bytes < need) {
        if (w.ptr) {
            err = hipFree(w.ptr);
            w.ptr = nullptr;
            w.bytes = 0;
            if (err != hipSuccess) return err;
        }
        const size_t bytes = round_up(need, 1 << 20);
        err = hipMalloc(&w.ptr, bytes);
        if (err != hipSuccess) return err;
        err = kvq::launch_fill_zero(w.ptr, bytes, nullptr);
        if (err != hipSuccess) return err;
        w.bytes = bytes;
    }
    return launch(w.ptr);
}

kvq_plan_info decode_info(const DecodePlan& p) {
    kvq_plan_info r{};
    r.kernel = p.kernel == kvq::Kernel::Mfma   ? KVQ_KERNEL_DECODE_MFMA
               : p.kernel == kvq::Kernel::Valu ? KVQ_KERNEL_DECODE_VALU
                                               : KVQ_KERNEL_DECODE_GENERIC;
    r.heads_per_group = p.sg;
    r.split_plan = p.flat           ? KVQ_SPLITS_TILES
                   : p.fit || p.lpt ? KVQ_SPLITS_IN_KERNEL
                   : p.scheduled    ? KVQ_SPLITS_SCHEDULE
                                    : KVQ_SPLITS_STATIC;
    r.splits = r.split_plan == KVQ_SPLITS_STATIC ? p.splits : 0;
    r.chunk = r.split_plan == KVQ_SPLITS_STATIC ? p.chunk : 0;
    r.query_block = 0;
    r.workspace_bytes = plan_bytes(p);
    r.tile_tokens = p.tile;
    return r;
}

bool decode_params_ok(const kvq_decode_params* p) {
    if (!p) return false;
    if (p->batch <= 0 || p->num_q_heads <= 0 || p->num_kv_heads <= 0) return false;
    if (p->num_q_heads % p->num_kv_heads != 0) return false;
    if (p->head_dim <= 0 || p->head_dim > KVQ_MAX_HEAD_DIM || p->capacity <= 0) return false;
    if (p->max_seq_len < 0 || p->num_splits < 0) return false;
    if (!p->lengths && p->max_seq_len == 0) return false;
    if (p->max_seq_len > p->capacity) return false;
    if ((p->max_seq_len > 0 ? p->max_seq_len : p->capacity) > KVQ_MAX_SEQ_LEN) return false;
    if (!p->q || !p->k_cache || !p->v_cache || !p->k_scale || !p->v_scale || !p->out) return false;
    if ((p->k_new == nullptr) != (p->v_new == nullptr)) return false;
    const long long units = static_cast<long long>(p->batch) * p->num_q_heads;
    if (units > INT_MAX / 4) return false;
    return true;
}

int decode_max_len(const kvq_decode_params* p) { return p->max_seq_len > 0 ? p->max_seq_len : p->capacity; }

// Launches a validated decode problem under `plan` with a workspace of at
// least plan_bytes(plan) (zero-filled counter prefix).
hipError_t decode_run(const kvq_decode_params* p, const DecodePlan& plan, void* workspace, hipStream_t stream) {
    DecodeArgs a{};
    a.q = p->q;
    a.k = p->k_cache;
    a.v = p->v_cache;
    a.ks = p->k_scale;
    a.vs = p->v_scale;
    a.out = p->out;
    a.lengths = p->lengths;
    a.k_new = p->k_new;
    a.v_new = p->v_new;
    a.B = p->batch;
    a.Hq = p->num_q_heads;
    a.Hkv = p->num_kv_heads;
    a.G = p->num_q_heads / p->num_kv_heads;
    a.cap = p->capacity;
    a.d = p->head_dim;
    a.uniform_len = decode_max_len(p);
    a.max_len = decode_max_len(p);
    a.splits = plan.splits;
    a.chunk = plan.chunk;
    a.nsg = plan.nsg;
    const float scale = p->softmax_scale > 0.0f ? p->softmax_scale : 1.0f / sqrtf(static_cast<float>(p->head_dim));
    a.scale_log2 = scale * kLog2e;
    bind_workspace(a, plan, workspace);
    return kvq::launch_decode(a, plan, stream);
}

// Workspace of kvq_decode_launch_noalloc: a fixed device array in place of a
// caller's allocation.  Each GPU holds its own copy at its own address until
// the process ends; the host name `scratch` is not a device address, so the
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and only that pointer is ever passed to kernels.  The arrival
// counters at its start are zero-filled (by a kernel) on the first call on
// each device; every completed launch leaves them at zero again, as for any
// workspace.  All calls on one GPU share the array, so calls that overlap in
// time on one GPU race.
static __device__ __align__(256) unsigned char scratch[KVQ_NOALLOC_SCRATCH_BYTES];
std::mutex g_scratch_mutex;
void* g_scratch_ptr[64];

hipError_t noalloc_scratch(hipStream_t stream, void** out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return err;
        if (ptr == nullptr) return hipErrorInvalidSymbol;
        err = kvq::launch_fill_zero(ptr, kCounterBytes, stream);
        if (err != hipSuccess) return err;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

bool decode_aligned(const kvq_decode_params* p) {
    return aligned16(p->q) && aligned16(p->k_cache) && aligned16(p->v_cache) && (p->head_dim % 16) == 0 &&
           (!p->k_new || (aligned16(p->k_new) && aligned16(p->v_new)));
}

// The matrix-core kernel reads 4 consecutive scales as one 16-byte load and
// addresses a (batch, kv head) cache row through a buffer resource with 32-bit
// byte offsets (capacity * head_dim < 2^31).
bool decode_mfma_layout(const kvq_decode_params* p) {
    return aligned16(p->k_scale) && aligned16(p->v_scale) && (p->capacity % 4) == 0 && p->capacity < (1 << 24);
}

DecodePlan decode_plan(const kvq_decode_params* p) {
    return make_plan(p->batch, p->num_q_heads, p->num_kv_heads, p->head_dim, decode_max_len(p),
                     decode_aligned(p), decode_mfma_layout(p), 0, p->lengths != nullptr, p->num_splits, INT_MAX,
                     true);
}

bool paged_params_ok(const kvq_paged_decode_params* p) {
    if (!p) return false;
    if (p->batch <= 0 || p->num_q_heads <= 0 || p->num_kv_heads <= 0) return false;
    if (p->num_q_heads % p->num_kv_heads != 0) return false;
    if (p->head_dim <= 0 || p->head_dim > KVQ_MAX_HEAD_DIM) return false;
    if (p->page_size <= 0 || p->num_pages <= 0 || p->max_pages_per_seq <= 0) return false;
    const long long cap = static_cast<long long>(p->max_pages_per_seq) * p->page_size;
    if (cap > INT_MAX || p->max_seq_len < 0 || p->max_seq_len > cap || p->num_splits < 0) return false;
    if (!p->lengths && p->max_seq_len == 0) return false;
    if ((p->max_seq_len > 0 ? p->max_seq_len : cap) > KVQ_MAX_SEQ_LEN) return false;
    if (!p->block_table || !p->q || !p->k_pages || !p->v_pages || !p->k_scale_pages || !p->v_scale_pages ||
        !p->out)
        return false;
    if ((p->k_new == nullptr) != (p->v_new == nullptr)) return false;
    if (static_cast<long long>(p->batch) * p->num_q_heads > INT_MAX / 4) return false;
    if (static_cast<long long>(p->batch) * p->max_pages_per_seq > INT_MAX) return false;
    return true;
}

int paged_cap(const kvq_paged_decode_params* p) { return p->max_pages_per_seq * p->page_size; }
int paged_max_len(const kvq_paged_decode_params* p) { return p->max_seq_len > 0 ? p->max_seq_len : paged_cap(p); }

kvq::PageMap page_map(const int32_t* table, int size, int max_pages, int num_pages) {
    int shift = -1;
    if ((size & (size - 1)) == 0)
        for (shift = 0; (1 << shift) < size; shift++) {
        }
    return kvq::PageMap{table, size, max_pages, num_pages, shift};
}

DecodePlan paged_plan(const kvq_paged_decode_params* p) {
    const bool aligned = aligned16(p->q) && aligned16(p->k_pages) && aligned16(p->v_pages) &&
                         (p->head_dim % 16) == 0 && (!p->k_new || (aligned16(p->k_new) && aligned16(p->v_new)));
    const bool quads = aligned16(p->k_scale_pages) && aligned16(p->v_scale_pages);
    return make_plan(p->batch, p->num_q_heads, p->num_kv_heads, p->head_dim, paged_max_len(p), aligned, quads,
                     p->page_size, p->lengths != nullptr, p->num_splits, INT_MAX, true);
}

// ---- dense attention ------------------------------------------------------

// Workgroups the attention grid should reach before keys are split: one
// round of resident matrix-core workgroups (8 waves each; at d = 128 the
// register file holds one per CU, below that two).
int attention_target_workgroups(int d) { return d >= 128 ? 256 : 512; }

// The register-direct attention kernel (up to 64 queries, d = 64 or 128):
// key splits per launch, KVQ_ATTN_DIRECT_SPLITS(M), but at least
// min(blocks, 128) and at most half the 16-key blocks; up to 32 queries four
// waves per query block share a split.  On one box (d = 128, N = 65536):
// M = 16 ran 23.3 us with 512 splits of one wave, 20.9 with 256 of 4 waves,
// 26.7 with 128 of 4, 21.4 with 256 of 8; M = 32 33.9 (256 x 1) against 25.1
// (256 x 4); M = 64 36.8 (256 x 1) against 38.0 (256 x 2).
#ifndef KVQ_ATTN_DIRECT_SPLITS
#define KVQ_ATTN_DIRECT_SPLITS(M) 256
#endif

struct AttnPlan {
    bool tuned = false;
    bool direct = false;
    int splits = 1, chunk = 0;
    int qblock = kvq::kAttnBlockWide;
    size_t ml_bytes = 0, acc_bytes = 0;
    size_t bytes() const { return ml_bytes + acc_bytes; }
};

bool attention_args_ok(int M, int N, int d, const void* q, const void* k, const void* v, const void* out) {
    if (!q || !k || !v || !out) return false;
    if (M <= 0 || N <= 0 || d <= 0 || d > 1024) return false;
    // Key loops step 64 keys past N; keep those indices in int range.
    return N <= INT_MAX - 1024 && M <= INT_MAX - 1024;
}

AttnPlan attention_plan(int M, int N, int d, bool aligned, int requested) {
    AttnPlan p;
    p.tuned = kvq::attention_tuned_dim(d) && aligned;
    p.chunk = N;
    if (!p.tuned) return p;  // the generic kernel runs unsplit
    // 9-16 queries over long key ranges at d = 32 or 256 also run the VALU
    // kernel, as 8-query blocks (M = 16, N = 65536, d = 256: 65.9 us against
    // 83.3 us in a padded matrix-core block); at d = 64 and 128 the
    // register-direct kernel below takes them.
    int qm = kvq::attention_rows_queries(M);
    // 5-8 queries at d = 64 and 128, and 3-4 at d = 64, go to the
    // register-direct kernel below (M = 8, N = 65536: 20.0 against 21.5 us at
    // d = 128, 11.2 against 16.2 at d = 64; M = 4, N = 65536, d = 64: 10.8
    // against 14.2 us); 1-4 queries at d = 128 stay here (M = 1, 2, 4: 14.0,
    // 15.9, 17.6 us against 19.5-19.7).
    if (kvq::attention_direct_dim(d) && (qm == kvq::kAttnRowsBlock || (d == 64 && qm == 4))) qm = 0;
    // Up to 64 queries the register-direct kernel takes what the few-query
    // kernel above left, where it beat the padded matrix-core block (one box):
    // at d = 128 from 16384 keys or with up to 32 queries, at d = 64 from
    // 32768 keys or with up to 8 queries.
    const bool direct_ok = M <= 64 && kvq::attention_direct_dim(d) && (d == 128 ? (N >= 16384 || M <= 32) : (N >= 32768 || M <= 8));
    if (qm == 0 && M <= 2 * kvq::kAttnRowsBlock && N >= 65536 && !direct_ok) qm = kvq::kAttnRowsBlock;
    if (qm > 0) {
        // A few queries: the VALU kernel, query blocks of qm, key splits to
        // fill KVQ_ATTN_ROWS_TARGET(qm) workgroups per query block.
        p.qblock = qm;
        const long long rt = kvq::attention_rows_tile(d, qm);
        const long long rtiles = (static_cast<long long>(N) + rt - 1) / rt;
        const long long want = std::max(1LL, std::min({requested > 0 ? static_cast<long long>(requested)
                                                                     : static_cast<long long>(KVQ_ATTN_ROWS_TARGET(qm)),
                                                      rtiles, static_cast<long long>(kvq::attention_max_splits(d))}));
        p.chunk = static_cast<int>(std::min<long long>((rtiles + want - 1) / want * rt, N));
        p.splits = static_cast<int>((N + static_cast<long long>(p.chunk) - 1) / p.chunk);
        if (p.splits > 1) {
            p.ml_bytes = round_up(static_cast<size_t>(p.splits) * M * 2 * sizeof(float), kAlign);
            p.acc_bytes = round_up(static_cast<size_t>(p.splits) * M * d * sizeof(float), kAlign);
        }
        return p;
    }
    if (direct_ok) {
        // 16 queries per wave; 1, 2 or 4 query blocks times the key parts per workgroup.
        p.direct = true;
        p.qblock = M <= 16 ? 16 : M <= 32 ? 32 : 64;
        const long long blocks = (static_cast<long long>(N) + 15) / 16;
        const long long cap = std::min<long long>(blocks, kvq::attention_max_splits(d));
        const long long want =
            requested > 0 ? std::min<long long>(requested, cap)
                          : std::min(cap, std::max(std::min(blocks, 128LL),
                                                   std::min<long long>(KVQ_ATTN_DIRECT_SPLITS(M), (blocks + 1) / 2)));
        p.chunk = static_cast<int>(std::min<long long>((blocks + want - 1) / want * 16, N));
        p.splits = static_cast<int>((N + static_cast<long long>(p.chunk) - 1) / p.chunk);
        if (p.splits > 1) {
            p.ml_bytes = round_up(static_cast<size_t>(p.splits) * M * 2 * sizeof(float), kAlign);
            p.acc_bytes = round_up(static_cast<size_t>(p.splits) * M * d * sizeof(float), kAlign);
        }
        return p;
    }
    const int tile = kvq::attention_key_tile(d);
    const long long tiles = (static_cast<long long>(N) + tile - 1) / tile;
    const long long target = attention_target_workgroups(d);
    // Splits for query blocks of qb: enough to fill the target, in whole key
    // tiles, within the merge's limit.
    auto splits_for = [&](int qb) {
        const long long qblocks = (static_cast<long long>(M) + qb - 1) / qb;
        const long long w = requested > 0 ? requested : (target + qblocks - 1) / qblocks;
        return std::max(1LL, std::min({w, tiles, static_cast<long long>(kvq::attention_max_splits(d))}));
    };
    long long want = splits_for(kvq::kAttnBlockWide);
    const long long wide_wgs = (static_cast<long long>(M) + kvq::kAttnBlockWide - 1) / kvq::kAttnBlockWide * want;
    if (requested == 0 && wide_wgs < target && d <= 128) {
        // The wide blocks leave CUs idle: narrow blocks double the grid.
        p.qblock = kvq::kAttnBlockNarrow;
        want = splits_for(kvq::kAttnBlockNarrow);
    }
    // The merge runs up to 64 lanes per 16-byte output column, indexed in int.
    if (static_cast<long long>(M) * (d / 4) * 64 >= INT_MAX) want = 1;
    const long long chunk_tiles = (tiles + want - 1) / want;
    p.chunk = static_cast<int>(std::min<long long>(chunk_tiles * tile, N));
    p.splits = static_cast<int>((N + static_cast<long long>(p.chunk) - 1) / p.chunk);
    if (p.splits > 1) {
        p.ml_bytes = round_up(static_cast<size_t>(p.splits) * M * 2 * sizeof(float), kAlign);
        p.acc_bytes = round_up(static_cast<size_t>(p.splits) * M * d * sizeof(float), kAlign);
    }
    return p;
}

bool attention_aligned(const float* q, const float* k, const float* v, const float* out) {
    return aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
}

hipError_t attention_run(int M, int N, int d, const float* q, const float* k, const float* v, float* out,
                         float scale, const AttnPlan& p, void* ws, hipStream_t stream) {
    kvq::AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.out = out;
    a.M = M;
    a.N = N;
    a.d = d;
    a.splits = p.splits;
    a.chunk = p.chunk;
    a.qblock = p.qblock;
    a.tuned = p.tuned;
    a.direct = p.direct;
    a.scale_log2 = scale * 1.4426950408889634f;
    if (p.splits > 1) {
        char* base = static_cast<char*>(ws);
        a.part_ml = reinterpret_cast<float*>(base);
        a.part_acc = reinterpret_cast<float*>(base + p.ml_bytes);
    }
    return kvq::launch_attention(a, stream);
}

// Library-owned attention workspaces, one per (device, stream): launches on
// one stream are ordered and may share one; different streams must not.  The
// split records need no initial contents.  Grown on demand to at least twice
// the old size; a superseded workspace is never freed, because a graph
// captured from an earlier call on this stream still writes to it on every
// replay (so the retired bytes stay below the live ones).  Growing needs
// hipMalloc, which a capturing stream does not allow: run one eager call of
// the largest problem before capturing.  As for `solve`, `launch(ptr)` is
// enqueued under the lock.
struct AttnWorkspaceKey {
    int device;
    hipStream_t stream;
    bool operator<(const AttnWorkspaceKey& o) const {
        return device != o.device ? device < o.device : std::less<hipStream_t>()(stream, o.stream);
    }
};
std::mutex g_attn_ws_mutex;
std::map<AttnWorkspaceKey, SolveWorkspace> g_attn_ws;
std::vector<void*> g_attn_retired;

template <class Launch>
hipError_t with_attention_workspace(size_t need, hipStream_t stream, Launch&& launch) {
    if (need == 0) return launch(nullptr);
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    std::lock_guard<std::mutex> lock(g_attn_ws_mutex);
    SolveWorkspace& w = g_attn_ws[AttnWorkspaceKey{dev, stream}];
    if (w.bytes < need) {
        const size_t bytes = round_up(std::max(need, 2 * w.bytes), 1 << 20);
        void* ptr = nullptr;
        err = hipMalloc(&ptr, bytes);
        if (err != hipSuccess) return err;
        if (w.ptr) g_attn_retired.push_back(w.ptr);  // still referenced by any graph captured before
        w.ptr = ptr;
        w.bytes = bytes;
    }
    return launch(w.ptr);
}

}  // namespace

extern "C" {

void solve(const float* Q, const int8_t* K_int8, const int8_t* V_int8, const float* k_scale,
           const float* v_scale, float* output, int num_heads, int seq_len, int head_dim) {
    if (!Q || !K_int8 || !V_int8 || !k_scale || !v_scale || !output) {
        fprintf(stderr, "[kvq] solve: null pointer input: Q=%p K_int8=%p V_int8=%p k_scale=%p v_scale=%p output=%p\n",
                static_cast<const void*>(Q), static_cast<const void*>(K_int8), static_cast<const void*>(V_int8),
                static_cast<const void*>(k_scale), static_cast<const void*>(v_scale), static_cast<void*>(output));
        return;
    }
    if (!shape_ok(num_heads, seq_len, head_dim) || static_cast<long long>(num_heads) * seq_len > INT_MAX) {
        fprintf(stderr,
                "[kvq] solve: invalid shape: num_heads=%d, seq_len=%d, head_dim=%d (head_dim <= %d, seq_len <= %d)\n",
                num_heads, seq_len, head_dim, KVQ_MAX_HEAD_DIM, KVQ_MAX_SEQ_LEN);
        return;
    }
    DecodeArgs a = reference_args(Q, K_int8, V_int8, k_scale, v_scale, output, num_heads, seq_len, head_dim);
    const DecodePlan p = make_plan(1, num_heads, num_heads, head_dim, seq_len,
                                   reference_aligned(Q, K_int8, V_int8, head_dim), false, 0, false, 0, INT_MAX, true);
    a.splits = p.splits;
    a.chunk = p.chunk;
    a.nsg = p.nsg;
    const hipError_t err = checked_call(nullptr, [&] {
        return with_solve_workspace(plan_bytes(p), [&](void* ws) {
            bind_workspace(a, p, ws);
            return kvq::launch_decode(a, p, nullptr);
        });
    });
    if (err != hipSuccess) fprintf(stderr, "[kvq] solve: HIP error: %s (%s)\n", hipGetErrorName(err), hipGetErrorString(err));
}

hipError_t kv_int8_split_launch(const float* Q, const int8_t* K_int8, const int8_t* V_int8,
                                const float* k_scale, const float* v_scale, float* output,
                                int num_heads, int seq_len, int head_dim, float* S, hipStream_t stream) {
    return reference_launch(Q, K_int8, V_int8, k_scale, v_scale, output, num_heads, seq_len, head_dim, S, stream);
}

hipError_t kv_int8_simple_launch(const float* Q, const int8_t* K_int8, const int8_t* V_int8,
                                 const float* k_scale, const float* v_scale, float* output,
                                 int num_heads, int seq_len, int head_dim, float* S, hipStream_t stream) {
    return reference_launch(Q, K_int8, V_int8, k_scale, v_scale, output, num_heads, seq_len, head_dim, S, stream);
}

size_t kvq_decode_workspace_size(const kvq_decode_params* p) {
    if (!decode_params_ok(p)) return 0;
    return plan_bytes(decode_plan(p));
}

hipError_t kvq_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (workspace_bytes == 0) return hipSuccess;
    if (!workspace) return hipErrorInvalidValue;
    return checked_call(stream, [&] { return kvq::launch_fill_zero(workspace, workspace_bytes, stream); });
}

hipError_t kvq_decode_launch(const kvq_decode_params* p, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
    if (!decode_params_ok(p)) return hipErrorInvalidValue;
    const DecodePlan plan = decode_plan(p);
    const size_t need = plan_bytes(plan);
    if (need > 0 && (!workspace || workspace_bytes < need)) return hipErrorInvalidValue;
    return checked_call(stream, [&] { return decode_run(p, plan, workspace, stream); });
}

hipError_t kvq_decode_launch_noalloc(const kvq_decode_params* p, hipStream_t stream) {
    if (!decode_params_ok(p)) return hipErrorInvalidValue;
    const DecodePlan plan = decode_plan(p);
    const size_t need = plan_bytes(plan);
    if (need > KVQ_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;  // beyond the fixed scratch array
    return checked_call(stream, [&] {
        void* ws = nullptr;
        if (need > 0) {
            const hipError_t err = noalloc_scratch(stream, &ws);
            if (err != hipSuccess) return err;
        }
        return decode_run(p, plan, ws, stream);
    });
}

hipError_t kvq_append_launch(const kvq_append_params* p, hipStream_t stream) {
    if (!p || p->batch <= 0 || p->num_kv_heads <= 0 || p->head_dim <= 0 || p->head_dim > KVQ_MAX_HEAD_DIM ||
        p->capacity <= 0 || !p->k_new || !p->v_new || !p->k_cache || !p->v_cache || !p->k_scale || !p->v_scale)
        return hipErrorInvalidValue;
    if (static_cast<long long>(p->batch) * p->num_kv_heads > INT_MAX) return hipErrorInvalidValue;
    return checked_call(stream, [&] {
        return kvq::launch_append(p->k_new, p->v_new, p->k_cache, p->v_cache, p->k_scale, p->v_scale, p->positions,
                                  p->uniform_position, false, p->batch, p->num_kv_heads, p->capacity, p->capacity,
                                  p->head_dim, kvq::PageMap{nullptr, 0, 0, 0, -1}, stream);
    });
}

hipError_t kvq_quantize_rows_launch(const float* x, int64_t rows, int head_dim, int8_t* q, float* scale,
                                    hipStream_t stream) {
    if (rows < 0 || head_dim <= 0 || head_dim > KVQ_MAX_HEAD_DIM) return hipErrorInvalidValue;
    if (rows > 0 && (!x || !q || !scale)) return hipErrorInvalidValue;
    const bool tuned_d = head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256;
    if (rows > 0 && rows < (1LL << 31) && tuned_d && aligned16(x) && (reinterpret_cast<uintptr_t>(q) & 7u) == 0) {
        // The prefill kernel over one plane of `rows` tokens at positions 0..rows-1.
        kvq::PrefillArgs a{};
        a.k_new = a.v_new = x;
        a.k = a.v = q;
        a.ks = a.vs = scale;
        a.Hkv = 1;
        a.L = static_cast<int>(rows);
        a.divL = kvq::make_fastdiv(static_cast<uint32_t>(std::max<int64_t>(rows, 1)));
        a.divH = kvq::make_fastdiv(1);
        a.cap = static_cast<int>(rows);
        a.rows = static_cast<unsigned>(rows);
        a.planes = 1;
        a.nseq = 1;
        a.pages = kvq::PageMap{nullptr, 0, 0, 0, -1};
        a.max_groups = prefill_max_groups();
        return checked_call(stream, [&] { return kvq::launch_prefill(a, head_dim, false, true, stream); });
    }
    return checked_call(stream, [&] { return kvq::launch_quantize_rows(x, rows, head_dim, q, scale, stream); });
}

size_t kvq_paged_decode_workspace_size(const kvq_paged_decode_params* p) {
    if (!paged_params_ok(p)) return 0;
    return plan_bytes(paged_plan(p));
}

hipError_t kvq_paged_decode_launch(const kvq_paged_decode_params* p, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
    if (!paged_params_ok(p)) return hipErrorInvalidValue;
    const DecodePlan plan = paged_plan(p);
    const size_t need = plan_bytes(plan);
    if (need > 0 && (!workspace || workspace_bytes < need)) return hipErrorInvalidValue;
    DecodeArgs a{};
    a.q = p->q;
    a.k = p->k_pages;
    a.v = p->v_pages;
    a.ks = p->k_scale_pages;
    a.vs = p->v_scale_pages;
    a.out = p->out;
    a.lengths = p->lengths;
    a.k_new = p->k_new;
    a.v_new = p->v_new;
    a.pages = page_map(p->block_table, p->page_size, p->max_pages_per_seq, p->num_pages);
    a.B = p->batch;
    a.Hq = p->num_q_heads;
    a.Hkv = p->num_kv_heads;
    a.G = p->num_q_heads / p->num_kv_heads;
    a.cap = paged_cap(p);
    a.d = p->head_dim;
    a.uniform_len = paged_max_len(p);
    a.max_len = paged_max_len(p);
    a.splits = plan.splits;
    a.chunk = plan.chunk;
    a.nsg = plan.nsg;
    const float scale = p->softmax_scale > 0.0f ? p->softmax_scale : 1.0f / sqrtf(static_cast<float>(p->head_dim));
    a.scale_log2 = scale * kLog2e;
    bind_workspace(a, plan, workspace);
    return checked_call(stream, [&] { return kvq::launch_decode(a, plan, stream); });
}

hipError_t kvq_paged_append_launch(const kvq_paged_append_params* p, hipStream_t stream) {
    if (!p || p->batch <= 0 || p->num_kv_heads <= 0 || p->head_dim <= 0 || p->head_dim > KVQ_MAX_HEAD_DIM ||
        p->page_size <= 0 || p->num_pages <= 0 || p->max_pages_per_seq <= 0 || !p->block_table || !p->k_new ||
        !p->v_new || !p->k_pages || !p->v_pages || !p->k_scale_pages || !p->v_scale_pages)
        return hipErrorInvalidValue;
    const long long cap = static_cast<long long>(p->max_pages_per_seq) * p->page_size;
    if (cap > INT_MAX || static_cast<long long>(p->batch) * p->num_kv_heads > INT_MAX ||
        static_cast<long long>(p->batch) * p->max_pages_per_seq > INT_MAX)
        return hipErrorInvalidValue;
    return checked_call(stream, [&] {
        return kvq::launch_append(p->k_new, p->v_new, p->k_pages, p->v_pages, p->k_scale_pages, p->v_scale_pages,
                                  p->positions, p->uniform_position, false, p->batch, p->num_kv_heads,
                                  static_cast<int>(cap), static_cast<int>(cap), p->head_dim,
                                  page_map(p->block_table, p->page_size, p->max_pages_per_seq, p->num_pages), stream);
    });
}

hipError_t kvq_prefill_quantize_launch(const kvq_prefill_params* p, hipStream_t stream) {
    if (!p || p->batch <= 0 || p->num_kv_heads <= 0 || p->head_dim <= 0 || p->head_dim > KVQ_MAX_HEAD_DIM ||
        p->tokens < 0 || (p->dtype != KVQ_DTYPE_F32 && p->dtype != KVQ_DTYPE_BF16))
        return hipErrorInvalidValue;
    if (!p->k_new || !p->v_new || !p->k_cache || !p->v_cache || !p->k_scale || !p->v_scale)
        return hipErrorInvalidValue;
    const long long rows = static_cast<long long>(p->batch) * p->num_kv_heads * p->tokens;
    if (rows >= (1LL << 31)) return hipErrorInvalidValue;
    kvq::PrefillArgs a{};
    if (p->block_table) {
        if (p->page_size <= 0 || p->num_pages <= 0 || p->max_pages_per_seq <= 0) return hipErrorInvalidValue;
        const long long cap = static_cast<long long>(p->max_pages_per_seq) * p->page_size;
        if (cap > INT_MAX || static_cast<long long>(p->batch) * p->max_pages_per_seq > INT_MAX)
            return hipErrorInvalidValue;
        a.cap = static_cast<int>(cap);
        a.pages = page_map(p->block_table, p->page_size, p->max_pages_per_seq, p->num_pages);
    } else {
        if (p->capacity <= 0) return hipErrorInvalidValue;
        a.cap = p->capacity;
        a.pages = kvq::PageMap{nullptr, 0, 0, 0, -1};
    }
    a.k_new = p->k_new;
    a.v_new = p->v_new;
    a.k = p->k_cache;
    a.v = p->v_cache;
    a.ks = p->k_scale;
    a.vs = p->v_scale;
    a.start = p->start;
    a.uniform_start = p->uniform_start;
    a.nseq = p->batch;
    a.Hkv = p->num_kv_heads;
    a.L = p->tokens;
    a.divL = kvq::make_fastdiv(static_cast<uint32_t>(std::max(p->tokens, 1)));
    a.divH = kvq::make_fastdiv(static_cast<uint32_t>(p->num_kv_heads));
    a.rows = static_cast<unsigned>(rows);
    a.planes = 2;
    a.max_groups = prefill_max_groups();
    // The tuned kernel reads start[] and the block table through buffer
    // resources with 32-bit byte offsets; larger tables take the generic one.
    const bool tables_fit = static_cast<long long>(p->batch) * 4 < (1LL << 31) &&
                            (!p->block_table ||
                             static_cast<long long>(p->batch) * p->max_pages_per_seq * 4 < (1LL << 31));
    const bool vec_ok = tables_fit && aligned16(p->k_new) && aligned16(p->v_new) &&
                        ((reinterpret_cast<uintptr_t>(p->k_cache) | reinterpret_cast<uintptr_t>(p->v_cache)) & 7u) == 0;
    return checked_call(stream,
                        [&] { return kvq::launch_prefill(a, p->head_dim, p->dtype == KVQ_DTYPE_BF16, vec_ok, stream); });
}

hipError_t attention_online_launch(const float* Q, const float* K, const float* V, float* output, int M, int N,
                                   int d, hipStream_t stream) {
    if (!attention_args_ok(M, N, d, Q, K, V, output)) return hipErrorInvalidValue;
    const AttnPlan p = attention_plan(M, N, d, attention_aligned(Q, K, V, output), 0);
    return checked_call(stream, [&] {
        return with_attention_workspace(p.bytes(), stream, [&](void* ws) {
            return attention_run(M, N, d, Q, K, V, output, 1.0f / sqrtf(static_cast<float>(d)), p, ws, stream);
        });
    });
}

size_t kvq_attention_workspace_size(const kvq_attention_params* p) {
    if (!p || !attention_args_ok(p->M, p->N, p->d, p->q, p->k, p->v, p->out) || p->num_splits < 0) return 0;
    return attention_plan(p->M, p->N, p->d, attention_aligned(p->q, p->k, p->v, p->out), p->num_splits).bytes();
}

hipError_t kvq_attention_launch(const kvq_attention_params* p, void* workspace, size_t workspace_bytes,
                                hipStream_t stream) {
    if (!p || !attention_args_ok(p->M, p->N, p->d, p->q, p->k, p->v, p->out) || p->num_splits < 0)
        return hipErrorInvalidValue;
    const AttnPlan plan =
        attention_plan(p->M, p->N, p->d, attention_aligned(p->q, p->k, p->v, p->out), p->num_splits);
    if (plan.bytes() > 0 && (!workspace || workspace_bytes < plan.bytes() || !aligned16(workspace)))
        return hipErrorInvalidValue;
    const float scale = p->softmax_scale != 0.0f ? p->softmax_scale : 1.0f / sqrtf(static_cast<float>(p->d));
    return checked_call(stream, [&] {
        return attention_run(p->M, p->N, p->d, p->q, p->k, p->v, p->out, scale, plan, workspace, stream);
    });
}

const char* kvq_version(void) { return "kvq 0.2.0 gfx950"; }

hipError_t kvq_reference_plan(const float* Q, const int8_t* K_int8, const int8_t* V_int8, int num_heads,
                              int seq_len, int head_dim, kvq_plan_info* info) {
    if (!info || !Q || !K_int8 || !V_int8 || !shape_ok(num_heads, seq_len, head_dim) ||
        static_cast<long long>(num_heads) * seq_len > INT_MAX)
        return hipErrorInvalidValue;
    *info = decode_info(reference_plan(num_heads, seq_len, head_dim, reference_aligned(Q, K_int8, V_int8, head_dim)));
    return hipSuccess;
}

hipError_t kvq_decode_plan(const kvq_decode_params* p, kvq_plan_info* info) {
    if (!info || !decode_params_ok(p)) return hipErrorInvalidValue;
    *info = decode_info(decode_plan(p));
    return hipSuccess;
}

hipError_t kvq_paged_decode_plan(const kvq_paged_decode_params* p, kvq_plan_info* info) {
    if (!info || !paged_params_ok(p)) return hipErrorInvalidValue;
    *info = decode_info(paged_plan(p));
    return hipSuccess;
}

hipError_t kvq_attention_plan(const kvq_attention_params* p, kvq_plan_info* info) {
    if (!info || !p || !attention_args_ok(p->M, p->N, p->d, p->q, p->k, p->v, p->out) || p->num_splits < 0)
        return hipErrorInvalidValue;
    const AttnPlan plan = attention_plan(p->M, p->N, p->d, attention_aligned(p->q, p->k, p->v, p->out), p->num_splits);
    kvq_plan_info r{};
    if (!plan.tuned) r.kernel = KVQ_KERNEL_ATTENTION_GENERIC;
    else if (plan.qblock <= kvq::kAttnRowsBlock) r.kernel = KVQ_KERNEL_ATTENTION_ROWS;
    else if (plan.direct) r.kernel = KVQ_KERNEL_ATTENTION_DIRECT;
    else r.kernel = KVQ_KERNEL_ATTENTION_MFMA;
    r.heads_per_group = 1;
    r.splits = plan.splits;
    r.chunk = plan.chunk;
    r.split_plan = KVQ_SPLITS_STATIC;
    r.query_block = plan.tuned ? plan.qblock : 0;
    r.workspace_bytes = plan.bytes();
    *info = r;
    return hipSuccess;
}

int kvq_diagnostics(void) { return (debug_sync() ? 1 : 0) | (forced_kernel() << 4); }

}  // extern "C"
