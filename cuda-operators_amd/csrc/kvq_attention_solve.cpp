// kvq_attention_solve.cpp -- libkvq_attention.so: the dense-attention `solve`
// of attention/softmax_new.cu:283-287, in a library of its own because
// libkvq.so already exports the decode `solve` (include/kvq_attention.h).
#include "../../include/kvq_attention.h"

#define KVQ_OMIT_DECODE_SOLVE  // this library's `solve` is the attention one
#include "../../include/kvq.h"

extern "C" void solve(const float* Q, const float* K, const float* V, float* output, int M, int N, int d) {
    // As the reference: the launch status is dropped; callers that need it use
    // attention_online_launch.
    (void)attention_online_launch(Q, K, V, output, M, N, d, nullptr);
}
