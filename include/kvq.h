/*
 * kvq.h -- C ABI of libkvq.so, the MI355X (gfx950) INT8 KV-cache
 * decode-attention operator.
 *
 * Part 1 is the drop-in boundary: the exact extern "C" symbols of the
 * reference's kv_cache/ path (Murmurwkk/cuda-operators), with HIP types in
 * place of CUDA ones (hipSuccess == cudaSuccess == 0,
 * hipErrorInvalidValue == cudaErrorInvalidValue == 1).  One library exports
 * one `solve`; the reference's four kv_cache .cu files each export their own
 * and cannot be linked together.
 *
 * Part 2 is the extension the reference lacks (batch, grouped-query heads,
 * ragged lengths, sequence splits with a log-sum-exp merge, appending a
 * quantised token).  Each query head hq of batch b computes exactly the
 * reference's single-head math over kv head hq / (Hq/Hkv) and the first
 * lengths[b] tokens.
 *
 * Layouts (row-major, contiguous; all pointers are device pointers):
 *   reference ABI:  Q[H,d] fp32, K/V[H,N,d] int8, k/v_scale[H,N] fp32, out[H,d]
 *   extension:      q[B,Hq,d], k/v cache[B,Hkv,cap,d] int8,
 *                   k/v scale[B,Hkv,cap] fp32, out[B,Hq,d], lengths[B] int32
 *
 * Math (both parts): s_t = (sum_i q_i * K[t,i]) * k_scale[t] * softmax_scale,
 * p = softmax(s), out_i = sum_t p_t * (V[t,i] * v_scale[t]); softmax_scale
 * defaults to 1/sqrtf(d) as in the reference.
 */
#ifndef KVQ_H
#define KVQ_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Largest head_dim any entry point accepts (head_dim in {32,64,128,256} runs
 * the tuned kernels; any other value up to this bound runs a generic kernel). */
#define KVQ_MAX_HEAD_DIM 4096

/* Longest sequence any decode entry point attends to, in tokens: seq_len of
 * the reference entry points, and the effective max_seq_len of the extension
 * (max_seq_len, or the capacity when it is 0).  The kernels count tokens and
 * tiles in 32-bit integers; beyond this bound the call is rejected with
 * hipErrorInvalidValue (solve: one stderr line).  Capacities and page tables
 * may be larger. */
#define KVQ_MAX_SEQ_LEN (1 << 30)

/* ===================== Part 1: reference entry points ===================== */

/* Replaces `solve`, kv_cache/KV_int8.cu:306-316 (also KV_int8_single_buffer.cu:260-270,
 * KV_int8_split_optimized.cu:294-304, new_kvint8.cu:102-104).
 * Legacy void ABI: invalid arguments print one line to stderr and return
 * without device work (as KV_int8_split_optimized.cu:306-324).  Runs
 * asynchronously on the null stream.  Split workspace comes from a per-device
 * cache owned by the library (allocated on first use, grown when needed). */
#ifndef KVQ_OMIT_DECODE_SOLVE /* defined by code that declares the attention `solve` (kvq_attention.h) */
void solve(const float* Q, const int8_t* K_int8, const int8_t* V_int8,
           const float* k_scale, const float* v_scale, float* output,
           int num_heads, int seq_len, int head_dim);
#endif

/* Replaces `kv_int8_split_launch`, kv_cache/KV_int8_split_optimized.cu:266-292.
 * S is caller-owned scratch of at least num_heads*seq_len floats; it holds the
 * per-split partial (max, sum, acc[d]) records, so at most seq_len/(head_dim+2)
 * splits per head are used (1 split needs no scratch at all).
 * Returns hipErrorInvalidValue, before any HIP call, for a null pointer,
 * num_heads/seq_len/head_dim <= 0, head_dim > KVQ_MAX_HEAD_DIM or
 * seq_len > KVQ_MAX_SEQ_LEN; otherwise the launch status.  Asynchronous on `stream`; the caller checks completion. */
hipError_t kv_int8_split_launch(const float* Q, const int8_t* K_int8, const int8_t* V_int8,
                                const float* k_scale, const float* v_scale, float* output,
                                int num_heads, int seq_len, int head_dim, float* S,
                                hipStream_t stream);

/* Replaces `kv_int8_simple_launch`, kv_cache/new_kvint8.cu:83-100 (identical
 * signature and contract to kv_int8_split_launch; same kernels here). */
hipError_t kv_int8_simple_launch(const float* Q, const int8_t* K_int8, const int8_t* V_int8,
                                 const float* k_scale, const float* v_scale, float* output,
                                 int num_heads, int seq_len, int head_dim, float* S,
                                 hipStream_t stream);

/* ============== Part 2: extension (no counterpart in the reference) ============== */

typedef struct kvq_decode_params {
    int batch;             /* B  >= 1 */
    int num_q_heads;       /* Hq >= 1, a multiple of num_kv_heads */
    int num_kv_heads;      /* Hkv >= 1 */
    int head_dim;          /* d in [1, KVQ_MAX_HEAD_DIM] */
    int capacity;          /* token stride of one (b, kv_head) cache row block, >= 1 */
    int max_seq_len;       /* uniform length when lengths == NULL; otherwise an upper
                              bound on every lengths[b] (0 means capacity) */
    const int32_t* lengths;/* device [B] or NULL; each clamped on device to
                              [0, max_seq_len] (max_seq_len 0: capacity);
                              a sequence of length 0 yields a zero output row */
    const float* q;        /* [B, Hq, d] */
    int8_t* k_cache;       /* [B, Hkv, capacity, d]; written only by a fused append */
    int8_t* v_cache;
    float* k_scale;        /* [B, Hkv, capacity] */
    float* v_scale;
    float* out;            /* [B, Hq, d], fully overwritten */
    float softmax_scale;   /* <= 0 selects 1/sqrtf(d) */
    int num_splits;        /* 0 = choose; otherwise the split count per sequence (the
                              tuned kernels round chunks up to whole tiles, so fewer
                              splits may run) */
    /* Fused append (both NULL = off).  When set, token length_b - 1 of every
     * (b, kv_head) is first quantised from k_new/v_new [B, Hkv, d] fp32 into the
     * cache (int8 values + scale, the same bits as kvq_append_launch), then
     * attended over; the caller's lengths already count the new token. */
    const float* k_new;
    const float* v_new;
} kvq_decode_params;

/* Bytes of workspace kvq_decode_launch needs for `p` (0 when one split
 * suffices).  The workspace holds per-split partials and one arrival counter
 * per (b, kv_head, head group); it must be zero-filled once after allocation
 * (kvq_workspace_init) and is left zeroed by every completed launch.  Calls
 * that overlap in time must not share a workspace. */
size_t kvq_decode_workspace_size(const kvq_decode_params* p);

/* Zero-fills a workspace on `stream` with a fill kernel (no hipMemset). */
hipError_t kvq_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Decode attention (plus the optional fused append) in one kernel launch:
 * splits write partial (max, sum, acc) records and the last split of each
 * sequence to finish merges them with a log-sum-exp reduction.
 * Returns hipErrorInvalidValue before any HIP call on a bad argument or a
 * workspace smaller than kvq_decode_workspace_size(p). */
hipError_t kvq_decode_launch(const kvq_decode_params* p, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* Size of the fixed device scratch array of kvq_decode_launch_noalloc. */
#define KVQ_NOALLOC_SCRATCH_BYTES (16u << 20)

/* No counterpart in the reference.  kvq_decode_launch without a workspace
 * argument and without any allocation, for callers that cannot allocate device
 * memory (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split records and arrival counters live in a fixed
 * KVQ_NOALLOC_SCRATCH_BYTES device array that each GPU holds until the process
 * ends (its counters are zero-filled by a kernel on the first call on each
 * device and left at zero by every completed launch).  Same plan, kernels and
 * result bits as kvq_decode_launch.  hipErrorInvalidValue for the arguments
 * kvq_decode_launch rejects and when kvq_decode_workspace_size(p) exceeds
 * KVQ_NOALLOC_SCRATCH_BYTES.  All calls on one GPU share the array: calls that
 * overlap in time on one GPU (different streams, or host threads) race. */
hipError_t kvq_decode_launch_noalloc(const kvq_decode_params* p, hipStream_t stream);

typedef struct kvq_append_params {
    int batch, num_kv_heads, head_dim, capacity;
    const int32_t* positions; /* device [B] write position per sequence, or NULL */
    int uniform_position;     /* used when positions == NULL */
    const float* k_new;       /* [B, Hkv, d] fp32 */
    const float* v_new;
    int8_t* k_cache;          /* [B, Hkv, capacity, d] */
    int8_t* v_cache;
    float* k_scale;           /* [B, Hkv, capacity] */
    float* v_scale;
} kvq_append_params;

/* Quantises one new K and V token per (b, kv_head): scale = max|x|/127.0f
 * (IEEE division), q = clamp(rintf(x/scale), -127, 127); a zero (or
 * underflowing) scale stores 0 and all-zero int8.  Positions outside
 * [0, capacity) are skipped.  lengths are not modified. */
hipError_t kvq_append_launch(const kvq_append_params* p, hipStream_t stream);

/* Bulk (prefill) quantiser: x[rows, d] fp32 -> q[rows, d] int8 + scale[rows],
 * the same per-row rule as kvq_append_launch. */
hipError_t kvq_quantize_rows_launch(const float* x, int64_t rows, int head_dim, int8_t* q,
                                    float* scale, hipStream_t stream);

/* ============ Part 3: paged KV cache (no counterpart in the reference) ============
 *
 * The cache lives in a pool of pages instead of one contiguous row block per
 * (b, kv_head):
 *   k/v_pages        [num_pages, Hkv, page_size, d] int8
 *   k/v_scale_pages  [num_pages, Hkv, page_size]    fp32
 *   block_table      [batch, max_pages_per_seq]     int32 page ids
 * Token t of sequence b is slot t % page_size of page
 * block_table[b * max_pages_per_seq + t / page_size]; within a page each kv
 * head's page_size rows are contiguous (page_size * d bytes).  Page ids
 * outside [0, num_pages) are clamped into it on the device (no fault; the
 * result is then meaningless).  Everything else -- math, lengths, splits,
 * fused append, workspace rules -- is as for kvq_decode_params, and a paged
 * cache holding the same tokens gives the same output. */

typedef struct kvq_paged_decode_params {
    int batch;              /* B >= 1 */
    int num_q_heads;        /* Hq >= 1, a multiple of num_kv_heads */
    int num_kv_heads;       /* Hkv >= 1 */
    int head_dim;           /* d in [1, KVQ_MAX_HEAD_DIM] */
    int page_size;          /* tokens per page, >= 1 (a multiple of 16 runs the tuned kernels) */
    int num_pages;          /* pages in the pool, >= 1 */
    int max_pages_per_seq;  /* row stride of block_table, >= 1 */
    int max_seq_len;        /* uniform length when lengths == NULL; otherwise a bound on
                               every lengths[b] (0: max_pages_per_seq * page_size) */
    const int32_t* block_table; /* device [B, max_pages_per_seq] */
    const int32_t* lengths; /* device [B] or NULL; clamped on device to [0, max_seq_len] */
    const float* q;         /* [B, Hq, d] */
    int8_t* k_pages;        /* [num_pages, Hkv, page_size, d]; written only by a fused append */
    int8_t* v_pages;
    float* k_scale_pages;   /* [num_pages, Hkv, page_size] */
    float* v_scale_pages;
    float* out;             /* [B, Hq, d], fully overwritten */
    float softmax_scale;    /* <= 0 selects 1/sqrtf(d) */
    int num_splits;         /* 0 = choose; otherwise the split count per sequence */
    const float* k_new;     /* fused append as in kvq_decode_params (both NULL = off) */
    const float* v_new;
} kvq_paged_decode_params;

/* Workspace bytes for kvq_paged_decode_launch (same rules as
 * kvq_decode_workspace_size). */
size_t kvq_paged_decode_workspace_size(const kvq_paged_decode_params* p);

/* Decode attention over a paged cache, plus the optional fused append.
 * Returns hipErrorInvalidValue before any HIP call on a bad argument or a
 * workspace smaller than kvq_paged_decode_workspace_size(p). */
hipError_t kvq_paged_decode_launch(const kvq_paged_decode_params* p, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream);

typedef struct kvq_paged_append_params {
    int batch, num_kv_heads, head_dim, page_size, num_pages, max_pages_per_seq;
    const int32_t* block_table; /* device [B, max_pages_per_seq] */
    const int32_t* positions;   /* device [B] token position per sequence, or NULL */
    int uniform_position;       /* used when positions == NULL */
    const float* k_new;         /* [B, Hkv, d] fp32 */
    const float* v_new;
    int8_t* k_pages;            /* [num_pages, Hkv, page_size, d] */
    int8_t* v_pages;
    float* k_scale_pages;       /* [num_pages, Hkv, page_size] */
    float* v_scale_pages;
} kvq_paged_append_params;

/* kvq_append_launch for a paged cache: the token goes to its position's page
 * slot; positions outside [0, max_pages_per_seq * page_size) are skipped. */
hipError_t kvq_paged_append_launch(const kvq_paged_append_params* p, hipStream_t stream);

/* ============ Part 4: prefill quantiser (no counterpart in the reference) ============
 *
 * Writes L new tokens per (b, kv head) into a contiguous or paged cache:
 * K and V rows x[B, Hkv, L, d] (fp32 or bf16) are quantised with the rule of
 * kvq_append_launch and stored at token positions start_b .. start_b + L - 1
 * (start_b = start[b], or uniform_start when start is NULL).  Positions
 * outside [0, capacity) -- paged: [0, max_pages_per_seq * page_size) -- are
 * skipped.  bf16 inputs are widened to fp32 exactly before the same rule. */

#define KVQ_DTYPE_F32 0
#define KVQ_DTYPE_BF16 1

typedef struct kvq_prefill_params {
    int batch, num_kv_heads, head_dim;
    int tokens;               /* L >= 0 new tokens per (b, kv head) */
    int dtype;                /* KVQ_DTYPE_F32 or KVQ_DTYPE_BF16 */
    const void* k_new;        /* [B, Hkv, L, d] */
    const void* v_new;
    const int32_t* start;     /* device [B] first position per sequence, or NULL */
    int uniform_start;        /* used when start == NULL */
    int capacity;             /* contiguous cache: tokens per (b, kv head) row block */
    int8_t* k_cache;          /* contiguous [B, Hkv, capacity, d] or pages [num_pages, Hkv, page_size, d] */
    int8_t* v_cache;
    float* k_scale;           /* [B, Hkv, capacity] or [num_pages, Hkv, page_size] */
    float* v_scale;
    const int32_t* block_table; /* NULL: contiguous cache; else paged (as kvq_paged_decode_params) */
    int page_size, num_pages, max_pages_per_seq;
} kvq_prefill_params;

/* One launch quantises all B*Hkv*L K and V rows. */
hipError_t kvq_prefill_quantize_launch(const kvq_prefill_params* p, hipStream_t stream);

/* ============ Part 5: dense fp32 attention (prefill-shaped) ============
 *
 * out[M, d] = softmax(Q K^T * scale) V for Q[M, d], K/V[N, d] fp32, one head,
 * no mask; the operator of attention/softmax_new.cu:87-281.  Inputs must be
 * finite (as the reference requires, attention/softmax_new.cu:237). */

/* Replaces attention_online_launch (attention/softmax_new.cu:239-281): same
 * arguments, scale 1/sqrtf(d), hipErrorInvalidValue for a NULL pointer,
 * M, N or d <= 0, or d > 1024 (the reference's limit, :252).  When the
 * queries alone cannot fill the GPU the keys are split over workgroups; the
 * partial results then live in a workspace the library owns, one per (device,
 * stream), allocated on first use and grown on demand (hipMalloc).  Callers
 * that must not allocate use kvq_attention_launch with their own workspace.
 * The reference's compatibility `solve(Q, K, V, output, M, N, d)`
 * (attention/softmax_new.cu:283-287) is not exported: its symbol is the
 * decode `solve` above. */
hipError_t attention_online_launch(const float* Q, const float* K, const float* V, float* output, int M, int N,
                                   int d, hipStream_t stream);

typedef struct kvq_attention_params {
    int M, N, d;              /* queries, keys, head dim (1 <= d <= 1024) */
    const float* q;           /* [M, d] */
    const float* k;           /* [N, d] */
    const float* v;           /* [N, d] */
    float* out;               /* [M, d] */
    float softmax_scale;      /* 0 -> 1/sqrtf(d) */
    int num_splits;           /* 0 -> chosen by the library; else a request (clamped) */
} kvq_attention_params;

/* Workspace bytes kvq_attention_launch needs for p (0: none, or invalid p):
 * the split records, which need no initial contents. */
size_t kvq_attention_workspace_size(const kvq_attention_params* p);

/* attention_online_launch with an explicit scale, split request and
 * caller-owned workspace (16-byte aligned, at least
 * kvq_attention_workspace_size(p) bytes); allocates nothing.  With splits, a
 * second kernel merges the records.  Launches that share a workspace must be
 * ordered (one stream).  hipErrorInvalidValue, before any HIP call, for the
 * checks of attention_online_launch, M or N above INT_MAX - 1024, a negative
 * num_splits, or a workspace too small, NULL or misaligned when one is
 * needed. */
hipError_t kvq_attention_launch(const kvq_attention_params* p, void* workspace, size_t workspace_bytes,
                                hipStream_t stream);

/* Library version string, e.g. "kvq 0.1.0 gfx950". */
const char* kvq_version(void);

/* ============ Part 6: plan queries and diagnostics (no counterpart in the reference) ============
 *
 * Host-only: these read no device memory and make no HIP call, so pointers
 * may be any values with the alignment of the real ones.  They report what
 * the matching launch would do. */

#define KVQ_KERNEL_DECODE_GENERIC 0   /* decode_generic: any head dim or alignment */
#define KVQ_KERNEL_DECODE_VALU 1      /* decode_fast: per-lane FMAs */
#define KVQ_KERNEL_DECODE_MFMA 2      /* decode_mfma: grouped-query heads on matrix cores */
#define KVQ_KERNEL_ATTENTION_MFMA 3   /* attention_mfma: query blocks on matrix cores */
#define KVQ_KERNEL_ATTENTION_ROWS 4   /* attention_rows: up to 8 queries per workgroup */
#define KVQ_KERNEL_ATTENTION_GENERIC 5 /* attention_generic: any head dim or alignment */
#define KVQ_KERNEL_ATTENTION_DIRECT 6  /* attention_direct: 9-64 queries, 16 per wave, no LDS tiles */

#define KVQ_SPLITS_STATIC 0     /* splits and chunk fixed on the host */
#define KVQ_SPLITS_IN_KERNEL 1  /* ragged batch planned inside the decode kernel */
#define KVQ_SPLITS_SCHEDULE 2   /* ragged batch planned by a schedule launch */
#define KVQ_SPLITS_TILES 3      /* ragged batch as one tile stream, split evenly over the
                                   matrix-core kernel's waves inside the kernel */

typedef struct kvq_plan_info {
    int kernel;             /* KVQ_KERNEL_* */
    int heads_per_group;    /* query heads one workgroup computes */
    int splits;             /* static plans: splits per sequence (1 = unsplit); 0 otherwise */
    int chunk;              /* static plans: tokens (keys) per split */
    int split_plan;         /* KVQ_SPLITS_* */
    int query_block;        /* attention: queries per workgroup; decode: 0 */
    size_t workspace_bytes; /* workspace (or scratch S) bytes the launch uses */
    int tile_tokens;        /* decode: tokens one workgroup iteration of the tuned kernel covers
                               (0: generic kernel); attention: 0 */
} kvq_plan_info;

/* The plan of kv_int8_split_launch / kv_int8_simple_launch for these
 * arguments; workspace_bytes is the part of S it uses (<= 4*num_heads*seq_len).
 * hipErrorInvalidValue for arguments the launch rejects. */
hipError_t kvq_reference_plan(const float* Q, const int8_t* K_int8, const int8_t* V_int8, int num_heads,
                              int seq_len, int head_dim, kvq_plan_info* info);
/* The plan of kvq_decode_launch for p. */
hipError_t kvq_decode_plan(const kvq_decode_params* p, kvq_plan_info* info);
/* The plan of kvq_paged_decode_launch for p. */
hipError_t kvq_paged_decode_plan(const kvq_paged_decode_params* p, kvq_plan_info* info);
/* The plan of kvq_attention_launch for p (attention_online_launch: p with
 * softmax_scale 0 and num_splits 0). */
hipError_t kvq_attention_plan(const kvq_attention_params* p, kvq_plan_info* info);

/* Diagnostic switches in force, read once from the environment:
 * bit 0: KVQ_DEBUG_SYNC ("1", "true", "yes" or "on"): every launching entry
 *        point synchronises its stream after its launches and returns the first
 *        error (not while the stream is being captured);
 * bits 4-7: KVQ_FORCE_KERNEL: 1 = "valu" (decode plans avoid the matrix-core
 *        kernel), 2 = "generic" (decode plans avoid both tuned kernels). */
int kvq_diagnostics(void);

#ifdef __cplusplus
}
#endif

#endif /* KVQ_H */
