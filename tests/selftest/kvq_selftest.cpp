// kvq_selftest -- C++ self-test of libkvq.so through its C ABI, mirroring the
// reference's only test of this path (kv_cache/KV_int8_split_optimized.cu:439-543):
// the same patterned inputs (:473-486), the default shape heads=4 seq_len=128
// head_dim=64 or one from argv (:441-450), solve() then a host check with a
// max-abs gate of 1e-4 (:535).  Adds the stream-aware launches with a NaN
// poisoned output and caller scratch.  The host check is the CPU oracle
// (oracle/kvq_oracle.c, linked into this test program only).
//
// usage: kvq_selftest [num_heads seq_len head_dim]     exit 0 = pass
#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "kvq.h"

extern "C" void kvq_ref_head_f32(const float* Q, const int8_t* K, const int8_t* V, const float* ks,
                                 const float* vs, float* out, int num_heads, int seq_len, int head_dim);

#define CHECK(x)                                                                                   \
    do {                                                                                           \
        hipError_t e_ = (x);                                                                       \
        if (e_ != hipSuccess) {                                                                    \
            fprintf(stderr, "[kvq_selftest] %s failed: %s\n", #x, hipGetErrorString(e_));          \
            return 1;                                                                              \
        }                                                                                          \
    } while (0)

static float max_abs_err(const std::vector<float>& a, const std::vector<float>& b) {
    float m = 0.0f;
    for (size_t i = 0; i < a.size(); i++) {
        const float e = fabsf(a[i] - b[i]);
        if (!(e <= m)) m = e;  // NaN propagates as a failure
    }
    return m;
}

int main(int argc, char** argv) {
    int H = 4, N = 128, d = 64;
    if (argc >= 4) {
        H = atoi(argv[1]);
        N = atoi(argv[2]);
        d = atoi(argv[3]);
    }
    if (H <= 0 || N <= 0 || d <= 0) {
        fprintf(stderr, "usage: %s [num_heads seq_len head_dim]\n", argv[0]);
        return 1;
    }
    printf("[kvq_selftest] %s  shape: heads=%d seq_len=%d head_dim=%d\n", kvq_version(), H, N, d);
    const size_t nq = (size_t)H * d, nkv = (size_t)H * N * d, ns = (size_t)H * N;
    std::vector<float> Q(nq), ks(ns), vs(ns), out(nq), ref(nq);
    std::vector<int8_t> K(nkv), V(nkv);
    for (size_t i = 0; i < nq; i++) Q[i] = (float)((int)(i % 17) - 8) * 0.125f;
    for (size_t i = 0; i < nkv; i++) {
        K[i] = (int8_t)((int)(i % 23) - 11);
        V[i] = (int8_t)((int)((i * 3) % 29) - 14);
    }
    for (size_t i = 0; i < ns; i++) {
        ks[i] = 0.015625f + (float)(i % 5) * 0.001f;
        vs[i] = 0.03125f + (float)(i % 7) * 0.001f;
    }
    kvq_ref_head_f32(Q.data(), K.data(), V.data(), ks.data(), vs.data(), ref.data(), H, N, d);

    float *dQ, *dks, *dvs, *dout, *dS;
    int8_t *dK, *dV;
    CHECK(hipMalloc(&dQ, nq * 4));
    CHECK(hipMalloc(&dK, nkv));
    CHECK(hipMalloc(&dV, nkv));
    CHECK(hipMalloc(&dks, ns * 4));
    CHECK(hipMalloc(&dvs, ns * 4));
    CHECK(hipMalloc(&dout, nq * 4));
    CHECK(hipMalloc(&dS, ns * 4));
    CHECK(hipMemcpy(dQ, Q.data(), nq * 4, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dK, K.data(), nkv, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dV, V.data(), nkv, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dks, ks.data(), ns * 4, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(dvs, vs.data(), ns * 4, hipMemcpyHostToDevice));

    std::vector<float> nan_fill(nq, NAN), s_fill(ns, 1e30f);
    int fails = 0;
    const char* names[3] = {"solve", "kv_int8_split_launch", "kv_int8_simple_launch"};
    hipStream_t st;
    CHECK(hipStreamCreate(&st));
    for (int entry = 0; entry < 3; entry++) {
        CHECK(hipMemcpy(dout, nan_fill.data(), nq * 4, hipMemcpyHostToDevice));
        CHECK(hipMemcpy(dS, s_fill.data(), ns * 4, hipMemcpyHostToDevice));
        if (entry == 0) {
            solve(dQ, dK, dV, dks, dvs, dout, H, N, d);
        } else {
            hipError_t e = entry == 1 ? kv_int8_split_launch(dQ, dK, dV, dks, dvs, dout, H, N, d, dS, st)
                                      : kv_int8_simple_launch(dQ, dK, dV, dks, dvs, dout, H, N, d, dS, st);
            CHECK(e);
            CHECK(hipStreamSynchronize(st));
        }
        CHECK(hipDeviceSynchronize());
        CHECK(hipMemcpy(out.data(), dout, nq * 4, hipMemcpyDeviceToHost));
        const float err = max_abs_err(out, ref);
        const bool ok = err <= 1e-4f;
        printf("[kvq_selftest] %-22s max_abs_err = %.8g  first outputs: %.6f %.6f %.6f %.6f  %s\n", names[entry],
               err, out[0], out[1], out[2], out[3], ok ? "passed" : "FAILED");
        fails += !ok;
    }
    // argument errors come back before any device work
    if (kv_int8_split_launch(nullptr, dK, dV, dks, dvs, dout, H, N, d, dS, st) != hipErrorInvalidValue ||
        kv_int8_split_launch(dQ, dK, dV, dks, dvs, dout, 0, N, d, dS, st) != hipErrorInvalidValue) {
        printf("[kvq_selftest] invalid-argument check FAILED\n");
        fails++;
    }
    CHECK(hipStreamDestroy(st));
    void* bufs[] = {dQ, dK, dV, dks, dvs, dout, dS};
    for (void* b : bufs) (void)hipFree(b);
    printf("[kvq_selftest] validation %s\n", fails ? "FAILED" : "passed");
    return fails ? 1 : 0;
}
