// kvq_internal.hpp -- host/device shared definitions of libkvq.so (not installed).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "kvq_fastdiv.hpp"

namespace kvq {

// Paged cache: k/v are page pools [num_pages, Hkv, size, d], their scales
// [num_pages, Hkv, size]; token t of sequence b is slot t % size of page
// table[b * max_pages + t / size].  table == null: contiguous layout.
struct PageMap {
    const int32_t* table;
    int size, max_pages, num_pages;
    int shift;  // log2(size) when size is a power of two, else -1
};

// Row index of token t of (sequence b, kv head kvh): its K/V row starts at
// byte row * d, its scale is element row.  Page ids are clamped into
// [0, num_pages), so a bad table entry cannot address outside the pool.
__device__ __forceinline__ size_t cache_row(const PageMap& pm, int Hkv, int cap, int b, int kvh, int t) {
    if (pm.table == nullptr) return (static_cast<size_t>(b) * Hkv + kvh) * cap + t;
    const int pi = pm.shift >= 0 ? t >> pm.shift : t / pm.size;
    const int page = min(max(pm.table[static_cast<size_t>(b) * pm.max_pages + pi], 0), pm.num_pages - 1);
    return (static_cast<size_t>(page) * Hkv + kvh) * pm.size + (t - pi * pm.size);
}

// Everything one decode launch needs; passed to the kernels by value.
struct DecodeArgs {
    const float* q;          // [B, Hq, d]
    int8_t* k;               // [B, Hkv, cap, d]
    int8_t* v;
    float* ks;               // [B, Hkv, cap]
    float* vs;
    float* out;              // [B, Hq, d]
    const int32_t* lengths;  // [B] or null
    const float* k_new;      // fused append source [B, Hkv, d] or null
    const float* v_new;
    float* part_ml;          // partial records (max in log2 units, sum): [B, Hq, splits, 2],
                             // or [records, Hq, 2] under a split schedule
    float* part_acc;         // unnormalised accumulators, same order, d floats per record
    int* counters;           // [B * Hkv * nsg] arrival counters, or null (merge kernel)
    const int* sched;        // split schedule written by schedule_kernel, or null (static splits)
    int sched_items;         // capacity of the schedule's item list
    int fit_items;           // > 0: the matrix-core kernel plans a ragged batch itself (locate_fit), this many items
    int fit_gran;            // chunk granularity of that plan (tokens)
    int flat;                // matrix-core kernel, ragged batch: fit_items workgroups per work unit take
                             // equal ranges of the sequences' tiles laid end to end (decode_mfma_flat)
    PageMap pages;           // paged layout, or pages.table == null (contiguous rows of cap tokens)
    int B, Hq, Hkv, G, cap, d;
    int uniform_len;         // used when lengths == null
    int max_len;             // every length is clamped to [0, max_len], max_len <= cap
    int splits;              // grid splits per sequence (static splits)
    int chunk;               // tokens per split (static splits)
    int nsg;                 // head groups per kv head (G / heads per workgroup)
    int lpt_target;          // > 0: the matrix-core kernel derives the split schedule itself (locate_lpt)
                             // for this many workgroups per round (the schedule kernel's target) ...
    int lpt_target_log2;     // ... a power of two, 2^lpt_target_log2
    float scale_log2;        // softmax_scale * log2(e)
};

// Split schedule of a ragged batch, computed on the device from the lengths
// by schedule_kernel before the decode launch (int words):
//   [0] chunk: the largest tokens per split;  [1] item count;  [2], [3] unused
//   items  [kSchedHeader, + kSchedItemInts * sched_items): per work item
//          (batch index b, split index s, splits of b, first record of b,
//          chunk of b, length of b, 0, 0) -- everything a decode workgroup
//          needs in two 16-byte loads; every split of every sequence once
//          (a length-0 sequence has one empty item that writes its zero
//          output).  Split s covers tokens [s * chunk, (s + 1) * chunk) and
//          owns records (first record + s) * Hq + hq;
//   seq [B] int2 after the items: (first record, chunk) of sequence b, for
//          the schedule kernel's own passes.
// Workgroup i of the decode grid takes item i / U, work unit i % U of that
// sequence (U = Hkv * nsg).
constexpr int kSchedHeader = 4;
constexpr int kSchedItemInts = 8;

// Most sequences of a ragged batch the matrix-core kernel plans itself (one
// per lane of a wave).
constexpr int kFitMaxSeqs = 64;
// Waves per workgroup of the matrix-core decode kernels, and tokens per wave tile.
constexpr int kMfmaWaves = 4;
constexpr int kMfmaTile = 32;
// Most sequences of a ragged batch under the flattened tile plan of the
// matrix-core kernel (their first tiles and lengths are scanned into LDS).
constexpr int kFlatMaxSeqs = 4096;
// Virtual tiles of no work before each sequence in the flattened tile plan
// (the cost of a wave's switch into a sequence, in tiles).
#ifndef KVQ_FLAT_SWITCH_TILES
#define KVQ_FLAT_SWITCH_TILES 2
#endif
constexpr int kFlatSwitchTiles = KVQ_FLAT_SWITCH_TILES;
// Most sequences of a ragged batch whose multi-round split schedule the
// matrix-core kernel derives itself (locate_lpt) instead of reading it from a
// schedule launch: two per thread of its 256.  Every workgroup pays for the
// derivation at its start, so larger batches (B1024 Hq32/Hkv8 L 64-1K: 257
// against 245 us) and many rounds of short items keep the launch: at most
// kLptMaxRounds rounds of B items, half that below kLptLongTokens tokens of
// capacity (B512 Hq32/Hkv8 L 64-1K, 8 rounds: 124.9 against 123.1 us).
constexpr int kLptMaxSeqs = 512;
constexpr int kLptMaxRounds = 8;
constexpr int kLptLongTokens = 2048;
// Size classes of a sequence's last chunk in the longest-first order.
constexpr int kSizeClasses = 64;

// Which decode kernel a plan runs.
enum class Kernel {
    Generic,  // any head dim / alignment (decode_generic)
    Valu,     // decode_fast: d in {32,64,128,256}, per-lane FMAs
    Mfma,     // decode_mfma: d = 128, 4 or 8 query heads per kv head group
};

// Launch plan chosen on the host.
struct DecodePlan {
    Kernel kernel;
    bool fast;       // a tuned kernel (Valu or Mfma): 16-byte aligned rows
    int sg;          // query heads per workgroup (tuned kernels)
    int tile;        // tokens one workgroup iteration covers (tuned kernels; 0: generic)
    int nsg;         // G / sg
    int splits;      // splits per sequence (grid dimension)
    int chunk;       // tokens per split
    bool counters;   // last-arriving split merges (fast path with a zeroed counter prefix)
    bool scheduled;  // ragged batch: the split schedule is computed on the device
    bool fit;        // ragged batch planned inside the matrix-core kernel (one round, no schedule launch)
    bool flat;       // with fit: the flattened tile-stream plan (decode_mfma_flat)
    bool lpt;        // with scheduled: the matrix-core kernel derives the schedule (no schedule launch)
    int sched_items;     // schedule item capacity (scheduled)
    int sched_target;    // workgroups the schedule aims for (scheduled)
    int sched_gran;      // chunk granularity in tokens (scheduled)
    size_t counter_bytes, sched_bytes, ml_bytes, acc_bytes;  // workspace regions
};

// Kernel launchers (kvq_decode.hip / kvq_append.hip).  They do no argument
// validation; the C ABI layer (kvq_capi.cpp) validates before calling them.
hipError_t launch_decode(const DecodeArgs& a, const DecodePlan& plan, hipStream_t stream);
// Workgroups of a tuned decode kernel's grid.
long decode_grid(const DecodeArgs& a, const DecodePlan& plan);
hipError_t launch_merge(const DecodeArgs& a, hipStream_t stream);
// Writes the split schedule of a ragged batch (see kSchedHeader) to sched.
hipError_t launch_schedule(const int32_t* lengths, int B, int max_len, int units_per_seq, int target_wgs,
                           int gran, int items_cap, int* sched, hipStream_t stream);
// Append one token per (b, kv head).  Position: positions[b] (or uniform_pos
// when positions is null); with from_lengths, positions holds sequence lengths
// and the token goes to clamp(lengths[b], 0, max_len) - 1.  Positions outside
// [0, cap) are skipped (paged: cap = max_pages * page size).
hipError_t launch_append(const float* k_new, const float* v_new, int8_t* k, int8_t* v, float* ks,
                         float* vs, const int32_t* positions, int uniform_pos, bool from_lengths,
                         int B, int Hkv, int max_len, int cap, int d, const PageMap& pages, hipStream_t stream);
hipError_t launch_quantize_rows(const float* x, int64_t rows, int d, int8_t* q, float* scale,
                                hipStream_t stream);

// Prefill: rows = B * Hkv * L input rows of K and of V ([B, Hkv, L, d], fp32
// or bf16), row (b, h, t) to cache position start_b + t (skipped outside
// [0, cap)).
struct PrefillArgs {
    const void* k_new;
    const void* v_new;
    int8_t* k;
    int8_t* v;
    float* ks;
    float* vs;
    const int32_t* start;
    int uniform_start;
    int Hkv, L, cap;
    FastDiv divL, divH;  // division of row indices by L and Hkv
    unsigned rows;
    int planes;  // 2: K and V; 1: K only
    int nseq;    // sequences (entries of start, rows of the page table)
    PageMap pages;
    unsigned max_groups;  // grid cap per plane (0: the default); beyond it workgroups stride
};
// vec_ok: 16-byte aligned inputs and 8-byte aligned caches (tuned kernel for
// d in {32, 64, 128, 256}).
hipError_t launch_prefill(const PrefillArgs& a, int d, bool bf16, bool vec_ok, hipStream_t stream);
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t stream);

// Dense fp32 attention (kvq_attention.hip): out = softmax(q k^T * scale) v.
// Queries per matrix-core attention workgroup (16 per wave): 8 waves, or 4
// when the wide blocks times the key splits cannot fill one round of
// workgroups (few queries, or few keys to split).
constexpr int kAttnBlockWide = 128;
constexpr int kAttnBlockNarrow = 64;
constexpr int kAttnRowsBlock = 8;     // queries per workgroup of the few-query kernel, at most

struct AttnArgs {
    const float* q;    // [M, d]
    const float* k;    // [N, d]
    const float* v;    // [N, d]
    float* out;        // [M, d]
    float* part_ml;    // [splits, M, 2] partial (max in log2 units, sum)
    float* part_acc;   // [splits, M, d] unnormalised partial accumulators
    int M, N, d;
    int splits, chunk;  // key splits (grid y) and keys per split (a multiple of the key tile)
    int qblock;         // queries per workgroup: kAttnBlockWide or kAttnBlockNarrow (matrix cores),
                        // or 1, 2, 4, 8 (few-query kernel, attention_rows)
    bool direct;        // attention_direct: qblock 16, 32 or 64 queries (16 per wave), no LDS tiles;
                        // up to 32 queries four waves share each query block's split
    float scale_log2;   // softmax scale * log2(e)
    bool tuned;         // a tuned kernel runs (tuned head dim and 16-byte aligned q, k, v, out);
                        // otherwise attention_generic, unsplit
};
int attention_tuned_dim(int d);   // the matrix-core kernel handles head dim d
int attention_key_tile(int d);    // keys per LDS tile of the matrix-core kernel at head dim d
int attention_max_splits(int d);  // most key splits per matrix-core launch (tuned d)
int attention_direct_dim(int d);  // attention_direct handles head dim d
int attention_rows_queries(int M);  // queries per workgroup of the few-query kernel (0: M too large)
int attention_rows_tile(int d, int qm);  // keys per workgroup step of the few-query kernel (tuned d, qm queries)
hipError_t launch_attention(const AttnArgs& a, hipStream_t stream);

// Tokens one workgroup iteration of the fast kernel covers for head dim d and
// sg query heads per workgroup; 0 when the fast kernel does not support d.
int fast_tile_tokens(int d, int sg);
// Tokens one wave of the fast kernel covers per iteration (its tile).
int fast_wave_tokens(int d, int sg);
int fast_heads_per_group(int G);
// decode_mfma: query heads per workgroup for group size G and head dim d (0:
// not applicable), tokens per workgroup iteration, launcher.
int mfma_heads_per_group(int G, int d);
int mfma_tile_tokens();
hipError_t launch_decode_mfma(const DecodeArgs& a, const DecodePlan& plan, hipStream_t stream);

}  // namespace kvq
