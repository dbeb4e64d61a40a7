/*
 * kvq_attention.h -- C ABI of libkvq_attention.so, the dense-attention
 * compatibility library.
 *
 * The reference's attention/softmax_new.cu exports its own `solve`, whose
 * symbol is also the decode `solve` of libkvq.so (include/kvq.h part 1).  As
 * the reference ships one library per .cu file, this one ships the attention
 * `solve` in a library of its own; it runs attention_online_launch of
 * libkvq.so (include/kvq.h part 5), which it links.  A caller of
 * softmax_new.cu links -lkvq_attention in its place, unchanged.
 */
#ifndef KVQ_ATTENTION_H
#define KVQ_ATTENTION_H

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces `solve`, attention/softmax_new.cu:283-287: out[M, d] =
 * softmax(Q K^T / sqrtf(d)) V for Q[M, d], K/V[N, d] fp32 device pointers.
 * Compatibility only, as in the reference: asynchronous on the null stream,
 * errors are not reported (attention_online_launch reports them). */
void solve(const float* Q, const float* K, const float* V, float* output, int M, int N, int d);

#ifdef __cplusplus
}
#endif

#endif /* KVQ_ATTENTION_H */
