/*
 * kvq_oracle.c -- CPU oracle for the INT8 KV-cache decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py
 * may load the library built from it.  The shipped operator (libkvq.so) never
 * links, loads or falls back to it.
 *
 * What it restates (citations are into the read-only reference tree):
 *   kvq_ref_head_f32      cpu_reference, kv_cache/KV_int8_split_optimized.cu:385-437
 *                         (fp32, same operation order: fmaf dot over d :405-411,
 *                         score=(dot*k_scale)*inv_sqrt :412, running max :414,
 *                         expf(s-max) and sequential denom :417-422,
 *                         fmaf(prob, v*v_scale, sum) sequential over t :424-435).
 *   kvq_ref_head_f64      the same formula in double precision (error yardstick).
 *   kvq_ref_decode_f32    batch / GQA / ragged reduction to kvq_ref_head_f32:
 *                         out[b,hq] = head(Q[b,hq], K[b,hq/g,:len_b], ...), g=Hq/Hkv.
 *                         The reference has no batched entry point; its single
 *                         head loop is kv_cache/KV_int8_split_optimized.cu:400.
 *   kvq_ref_decode_f64    same reduction over kvq_ref_head_f64.
 *   kvq_ref_quantize_rows per-token symmetric int8 quantiser.  The reference has
 *                         no quantiser (kv_cache/new_kvint8.cu:83-84 says so); the
 *                         spec is the task's config text: scale = max|x|/127,
 *                         int8 = round(x/scale) clamped to +-127.  Decisions fixed
 *                         here: IEEE fp32 division for both divisions, rintf
 *                         (round half to even), amax == 0 (or a scale that
 *                         underflows to 0) gives scale 0 and all-zero int8.
 *   kvq_ref_append        writes one quantised token per (b, kv_head) at
 *                         positions[b] into the cache (layout [B,Hkv,cap,d]).
 *   kvq_ref_attention_f32 dense fp32 attention softmax(Q K^T / sqrt(d)) V, the
 *                         math of attention/softmax_new.cu:87-281.
 *
 * Pinning (what checks this oracle, in tests/test_oracle.py):
 *   - float64 textbook softmax attention (numpy/scipy) on random inputs,
 *   - closed forms: N=1, K=0 (uniform weights), constant V, one dominating
 *     score, token-permutation invariance, convexity of the output,
 *   - GQA == MHA over explicitly replicated KV heads, ragged == truncated,
 *   - the reference self-test's patterned inputs (KV_int8_split_optimized.cu:473-486)
 *     against the float64 textbook and the committed golden outputs,
 *   - quantiser: |x - q*scale| <= scale/2, ties to even, extreme elements map
 *     to +-127, scale == amax/127 exactly, zero row,
 *   - planted mistakes (PLANT below) must each fail at least one of these.
 *
 * Build: see oracle/Makefile (gcc -O3 -fopenmp -ffp-contract=off, no -ffast-math).
 */
#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Planted-mistake builds (tests only): each value breaks one thing a plausible
 * implementation bug would break.  0 = the real oracle. */
#ifndef PLANT
#define PLANT 0
#endif
#define PLANT_NO_KSCALE 1   /* score drops k_scale                         */
#define PLANT_INV_D 2       /* 1/d instead of 1/sqrt(d)                     */
#define PLANT_GQA_MOD 3     /* kv head = hq % Hkv instead of hq / g         */
#define PLANT_EXP_SIGN 4    /* expf(max - s) instead of expf(s - max)       */
#define PLANT_TRANSPOSE 5   /* K indexed [d][t] instead of [t][d]           */
#define PLANT_LEN_M1 6      /* ragged length off by one                     */
#define PLANT_ROUND_AWAY 7  /* roundf (half away from zero) instead of rintf */
#define PLANT_TRUNC 8       /* truncation instead of rounding               */
#define PLANT_NO_VSCALE 9   /* value dequant drops v_scale                  */
#define PLANT_ATT_INV_D 10  /* dense attention: 1/d instead of 1/sqrt(d)     */
#define PLANT_ATT_V_T 11    /* dense attention: V indexed [d][n]             */
/* Memory and undefined-behaviour faults, built only by the sanitizer target
 * (oracle/Makefile `sanitize`) to show that a sanitizer report fails the run: */
#define PLANT_OOB_READ 12   /* softmax loop runs one past the score scratch */
#define PLANT_INT_OVF 13    /* signed int overflow                          */

int kvq_ref_plant_id(void) { return PLANT; }

int kvq_ref_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* One head, fp32, same operation order as the reference's cpu_reference.
 * scores: caller scratch of n floats. */
static void head_f32(const float* q, const int8_t* k, const int8_t* v,
                     const float* ks, const float* vs, float* out,
                     int n, int d, float* scores) {
    const float inv_sqrt = 1.0f / sqrtf((float)d);
    float max_score = -FLT_MAX;
    for (int t = 0; t < n; t++) {
        float dot = 0.0f;
        for (int i = 0; i < d; i++) {
#if PLANT == PLANT_TRANSPOSE
            const float kv = (float)k[(size_t)i * n + t];
#else
            const float kv = (float)k[(size_t)t * d + i];
#endif
            dot = fmaf(q[i], kv, dot);
        }
#if PLANT == PLANT_NO_KSCALE
        float score = dot * inv_sqrt;
#elif PLANT == PLANT_INV_D
        float score = dot * ks[t] * (1.0f / (float)d);
#else
        float score = dot * ks[t] * inv_sqrt;
#endif
        scores[t] = score;
        max_score = fmaxf(max_score, score);
    }
    float denom = 0.0f;
#if PLANT == PLANT_OOB_READ
    for (int t = 0; t <= n; t++) {
#else
    for (int t = 0; t < n; t++) {
#endif
#if PLANT == PLANT_EXP_SIGN
        scores[t] = expf(max_score - scores[t]);
#else
        scores[t] = expf(scores[t] - max_score);
#endif
        denom += scores[t];
    }
    for (int i = 0; i < d; i++) {
        float sum = 0.0f;
        for (int t = 0; t < n; t++) {
            const float prob = scores[t] / denom;
#if PLANT == PLANT_NO_VSCALE
            const float val = (float)v[(size_t)t * d + i];
#else
            const float val = (float)v[(size_t)t * d + i] * vs[t];
#endif
            sum = fmaf(prob, val, sum);
        }
        out[i] = sum;
    }
}

/* Same formula in double precision. */
static void head_f64(const float* q, const int8_t* k, const int8_t* v,
                     const float* ks, const float* vs, double* out,
                     int n, int d, double* scores) {
    const double inv_sqrt = 1.0 / sqrt((double)d);
    double max_score = -DBL_MAX;
    for (int t = 0; t < n; t++) {
        double dot = 0.0;
        for (int i = 0; i < d; i++) dot += (double)q[i] * (double)k[(size_t)t * d + i];
        const double score = dot * (double)ks[t] * inv_sqrt;
        scores[t] = score;
        if (score > max_score) max_score = score;
    }
    double denom = 0.0;
    for (int t = 0; t < n; t++) {
        scores[t] = exp(scores[t] - max_score);
        denom += scores[t];
    }
    for (int i = 0; i < d; i++) {
        double sum = 0.0;
        for (int t = 0; t < n; t++)
            sum += (scores[t] / denom) * ((double)v[(size_t)t * d + i] * (double)vs[t]);
        out[i] = sum;
    }
}

/* Reference ABI shape: Q[H,d], K/V[H,N,d], scales[H,N], out[H,d]. */
void kvq_ref_head_f32(const float* Q, const int8_t* K, const int8_t* V,
                      const float* ks, const float* vs, float* out,
                      int num_heads, int seq_len, int head_dim) {
    float* scores = (float*)malloc(sizeof(float) * (size_t)seq_len);
#if PLANT == PLANT_INT_OVF
    volatile int big = INT_MAX;
    const int wrapped = big + num_heads;
    if (wrapped == 0) num_heads = 0;
#endif
    for (int h = 0; h < num_heads; h++) {
        const size_t kv = (size_t)h * seq_len * head_dim;
        head_f32(Q + (size_t)h * head_dim, K + kv, V + kv, ks + (size_t)h * seq_len,
                 vs + (size_t)h * seq_len, out + (size_t)h * head_dim, seq_len, head_dim, scores);
    }
    free(scores);
}

static int kv_head_of(int hq, int Hq, int Hkv) {
#if PLANT == PLANT_GQA_MOD
    (void)Hq;
    return hq % Hkv;
#else
    return hq / (Hq / Hkv);
#endif
}

static int length_of(const int32_t* lengths, int b, int uniform_len, int cap) {
    int len = lengths ? lengths[b] : uniform_len;
#if PLANT == PLANT_LEN_M1
    if (lengths) len -= 1;
#endif
    if (len > cap) len = cap;
    return len;
}

/* Batched / GQA / ragged decode, fp32.
 * q[B,Hq,d]  k,v[B,Hkv,cap,d]  ks,vs[B,Hkv,cap]  lengths[B] (or NULL: uniform_len)
 * out[B,Hq,d].  A sequence with length <= 0 produces zeros.
 * OpenMP over (b, hq); every unit keeps the reference's sequential order. */
void kvq_ref_decode_f32(const float* q, const int8_t* k, const int8_t* v,
                        const float* ks, const float* vs, const int32_t* lengths,
                        int B, int Hq, int Hkv, int cap, int d, int uniform_len,
                        float* out) {
    const int units = B * Hq;
#pragma omp parallel
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)(cap > 0 ? cap : 1));
#pragma omp for schedule(dynamic, 1)
        for (int u = 0; u < units; u++) {
            const int b = u / Hq, hq = u % Hq;
            const int kvh = kv_head_of(hq, Hq, Hkv);
            const int len = length_of(lengths, b, uniform_len, cap);
            float* o = out + (size_t)u * d;
            if (len <= 0) {
                memset(o, 0, sizeof(float) * (size_t)d);
                continue;
            }
            const size_t row = (size_t)b * Hkv + kvh;
            head_f32(q + (size_t)u * d, k + row * cap * d, v + row * cap * d,
                     ks + row * cap, vs + row * cap, o, len, d, scores);
        }
        free(scores);
    }
}

void kvq_ref_decode_f64(const float* q, const int8_t* k, const int8_t* v,
                        const float* ks, const float* vs, const int32_t* lengths,
                        int B, int Hq, int Hkv, int cap, int d, int uniform_len,
                        double* out) {
    const int units = B * Hq;
#pragma omp parallel
    {
        double* scores = (double*)malloc(sizeof(double) * (size_t)(cap > 0 ? cap : 1));
#pragma omp for schedule(dynamic, 1)
        for (int u = 0; u < units; u++) {
            const int b = u / Hq, hq = u % Hq;
            const int kvh = hq / (Hq / Hkv);
            int len = lengths ? lengths[b] : uniform_len;
            if (len > cap) len = cap;
            double* o = out + (size_t)u * d;
            if (len <= 0) {
                for (int i = 0; i < d; i++) o[i] = 0.0;
                continue;
            }
            const size_t row = (size_t)b * Hkv + kvh;
            head_f64(q + (size_t)u * d, k + row * cap * d, v + row * cap * d,
                     ks + row * cap, vs + row * cap, o, len, d, scores);
        }
        free(scores);
    }
}

/* Per-token symmetric int8 quantiser (one row of d values). */
static void quantize_row(const float* x, int d, int8_t* qo, float* scale_out) {
    float amax = 0.0f;
    for (int i = 0; i < d; i++) amax = fmaxf(amax, fabsf(x[i]));
    const float scale = amax / 127.0f;
    *scale_out = scale;
    if (scale == 0.0f) {
        memset(qo, 0, (size_t)d);
        return;
    }
    for (int i = 0; i < d; i++) {
        const float r = x[i] / scale;
#if PLANT == PLANT_ROUND_AWAY
        float y = roundf(r);
#elif PLANT == PLANT_TRUNC
        float y = truncf(r);
#else
        float y = rintf(r);
#endif
        if (y > 127.0f) y = 127.0f;
        if (y < -127.0f) y = -127.0f;
        qo[i] = (int8_t)y;
    }
}

void kvq_ref_quantize_rows(const float* x, int64_t rows, int d, int8_t* q, float* scale) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        quantize_row(x + r * d, d, q + r * d, scale + r);
}

/* Append one token per (b, kv_head) at positions[b] (or uniform_pos when
 * positions is NULL).  Positions outside [0, cap) are skipped. */
void kvq_ref_append(const float* k_new, const float* v_new, int8_t* k, int8_t* v,
                    float* ks, float* vs, const int32_t* positions, int uniform_pos,
                    int B, int Hkv, int cap, int d) {
    for (int b = 0; b < B; b++) {
        const int pos = positions ? positions[b] : uniform_pos;
        if (pos < 0 || pos >= cap) continue;
        for (int h = 0; h < Hkv; h++) {
            const size_t row = (size_t)b * Hkv + h;
            const size_t tok = row * cap + (size_t)pos;
            quantize_row(k_new + row * d, d, k + tok * d, ks + tok);
            quantize_row(v_new + row * d, d, v + tok * d, vs + tok);
        }
    }
}

/* Dense fp32 attention, one query row per call: the math of the reference's
 * attention_online_launch (attention/softmax_new.cu:87-203, launch :239-281):
 * s_t = (sum_i fmaf(q_i, K[t,i])) * (1/sqrtf(d)), m = max_t s_t,
 * e_t = expf(s_t - m), l = sum_t e_t, out_j = (sum_t fmaf(e_t, V[t,j])) * (1/l)
 * (the reference scales the accumulator by a reciprocal of l, :192-200).
 * Sums are sequential in t and i. */
static void attention_row_f32(const float* q, const float* K, const float* V, float* out, int N, int d,
                              float* e) {
#if PLANT == PLANT_ATT_INV_D
    const float scale = 1.0f / (float)d;
#else
    const float scale = 1.0f / sqrtf((float)d);
#endif
    float m = -FLT_MAX;
    for (int t = 0; t < N; t++) {
        float dot = 0.0f;
        for (int i = 0; i < d; i++) dot = fmaf(q[i], K[(size_t)t * d + i], dot);
        e[t] = dot * scale;
        m = fmaxf(m, e[t]);
    }
    float l = 0.0f;
    for (int t = 0; t < N; t++) {
        e[t] = expf(e[t] - m);
        l += e[t];
    }
    const float inv_l = 1.0f / l;
    for (int j = 0; j < d; j++) {
        float acc = 0.0f;
        for (int t = 0; t < N; t++) {
#if PLANT == PLANT_ATT_V_T
            acc = fmaf(e[t], V[(size_t)j * N + t], acc);
#else
            acc = fmaf(e[t], V[(size_t)t * d + j], acc);
#endif
        }
        out[j] = acc * inv_l;
    }
}

/* Q[M,d], K[N,d], V[N,d] fp32 -> out[M,d]; OpenMP over query rows. */
void kvq_ref_attention_f32(const float* Q, const float* K, const float* V, float* out, int M, int N, int d) {
#pragma omp parallel
    {
        float* e = (float*)malloc(sizeof(float) * (size_t)(N > 0 ? N : 1));
#pragma omp for schedule(static)
        for (int r = 0; r < M; r++) attention_row_f32(Q + (size_t)r * d, K, V, out + (size_t)r * d, N, d, e);
        free(e);
    }
}
