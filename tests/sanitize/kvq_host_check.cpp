// kvq_host_check -- drives the host side of libkvq (argument validation,
// planners, workspace sizing) through the public C ABI of include/kvq.h over
// a sweep of shapes, with no GPU and no HIP call: every call either is a plan
// query or is rejected before the library touches the runtime.  Built with
// AddressSanitizer + UndefinedBehaviorSanitizer from host-only objects
// (tests/sanitize/Makefile) and run by tests/test_sanitizers_cpu.py, so an
// out-of-bounds access, a signed overflow in a size computation or a host-side
// dereference of a device pointer ends the run with a report.
//
// Besides the sanitizers it checks the invariants the planners promise:
//   * kv_int8_split_launch's records fit the caller's scratch S (H*N floats,
//     kv_cache/KV_int8_split_optimized.cu:266-267), splits <= N / (d + 2);
//   * kvq_*_workspace_size equals the plan query's workspace_bytes, and is 0
//     exactly when the parameters are rejected;
//   * a workspace one byte short is rejected with hipErrorInvalidValue;
//   * lengths above KVQ_MAX_SEQ_LEN are rejected, and every accepted plan's
//     32-bit token and tile counts stay in range (paged_bounds).
// Exit status 0 and a last line "OK <checks>" when everything holds.
#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "kvq.h"
#include "kvq_device.hpp"    // kWave
#include "kvq_internal.hpp"  // kMfmaTile, kFlatSwitchTiles: the tile-stream plan's geometry

namespace {

long g_checks = 0;
long g_fails = 0;

void expect(bool ok, const char* what, long a = 0, long b = 0, long c = 0, long d = 0) {
    g_checks++;
    if (!ok) {
        g_fails++;
        if (g_fails <= 50) std::printf("FAIL %s (%ld %ld %ld %ld)\n", what, a, b, c, d);
    }
}

// Device-pointer stand-ins: 16-byte aligned (or offset by 4) addresses that
// host code must never dereference.
const uintptr_t kA = uintptr_t(1) << 20;
template <class T>
T* fake(uintptr_t off = 0) {
    return reinterpret_cast<T*>(kA + off);
}

void reference_abi() {
    kvq_plan_info info;
    const int dims[] = {1, 16, 32, 64, 96, 128, 256, 512, 1024, 4096};
    const int heads[] = {1, 2, 3, 5, 16, 256};
    std::vector<int> lens;
    for (int n = 1; n <= 1100; n += 3) lens.push_back(n);
    for (int n : {2047, 2048, 4096, 4097, 16384, 131072, 1 << 22}) lens.push_back(n);
    for (int d : dims) {
        for (int H : heads) {
            for (int N : lens) {
                const hipError_t e =
                    kvq_reference_plan(fake<float>(), fake<int8_t>(), fake<int8_t>(), H, N, d, &info);
                expect(e == hipSuccess, "reference plan accepted", H, N, d);
                if (e != hipSuccess) continue;
                expect(info.workspace_bytes <= 4ull * H * N, "reference plan fits S", H, N, d,
                       static_cast<long>(info.workspace_bytes));
                expect(info.splits >= 1, "reference plan splits >= 1", H, N, d, info.splits);
                if (info.splits > 1) expect(info.splits <= N / (d + 2), "splits <= N/(d+2)", H, N, d, info.splits);
            }
        }
    }
    // Misaligned inputs plan too (the generic kernel).
    for (uintptr_t off : {uintptr_t(4), uintptr_t(8), uintptr_t(12)}) {
        expect(kvq_reference_plan(fake<float>(off), fake<int8_t>(), fake<int8_t>(), 4, 1000, 128, &info) ==
                   hipSuccess,
               "misaligned reference plan");
    }
    struct Bad {
        bool nq, nk, nv, nks, nvs, nout, ns;
        int H, N, d;
    };
    const Bad bad[] = {{true, false, false, false, false, false, false, 4, 128, 64},
                       {false, true, false, false, false, false, false, 4, 128, 64},
                       {false, false, true, false, false, false, false, 4, 128, 64},
                       {false, false, false, true, false, false, false, 4, 128, 64},
                       {false, false, false, false, true, false, false, 4, 128, 64},
                       {false, false, false, false, false, true, false, 4, 128, 64},
                       {false, false, false, false, false, false, true, 4, 128, 64},
                       {false, false, false, false, false, false, false, 0, 128, 64},
                       {false, false, false, false, false, false, false, 4, 0, 64},
                       {false, false, false, false, false, false, false, 4, 128, 0},
                       {false, false, false, false, false, false, false, -1, 128, 64},
                       {false, false, false, false, false, false, false, 4, -5, 64},
                       {false, false, false, false, false, false, false, 4, 128, -1},
                       {false, false, false, false, false, false, false, 4, 128, 4097},
                       {false, false, false, false, false, false, false, INT_MIN, INT_MIN, INT_MIN}};
    for (const Bad& b : bad) {
        const float* Q = b.nq ? nullptr : fake<float>();
        const int8_t* K = b.nk ? nullptr : fake<int8_t>();
        const int8_t* V = b.nv ? nullptr : fake<int8_t>();
        const float* ks = b.nks ? nullptr : fake<float>();
        const float* vs = b.nvs ? nullptr : fake<float>();
        float* out = b.nout ? nullptr : fake<float>();
        float* S = b.ns ? nullptr : fake<float>();
        expect(kv_int8_split_launch(Q, K, V, ks, vs, out, b.H, b.N, b.d, S, nullptr) == hipErrorInvalidValue,
               "split launch rejects", b.H, b.N, b.d);
        expect(kv_int8_simple_launch(Q, K, V, ks, vs, out, b.H, b.N, b.d, S, nullptr) == hipErrorInvalidValue,
               "simple launch rejects", b.H, b.N, b.d);
        if (!b.ns) solve(Q, K, V, ks, vs, out, b.H, b.N, b.d);  // prints and returns
    }
    expect(kvq_reference_plan(fake<float>(), fake<int8_t>(), fake<int8_t>(), 4, 4, 64, nullptr) ==
               hipErrorInvalidValue,
           "reference plan without info");
}

kvq_decode_params decode_params(int B, int Hq, int Hkv, int d, int cap, int max_len, bool ragged, int splits,
                                bool append, uintptr_t misalign) {
    kvq_decode_params p{};
    p.batch = B;
    p.num_q_heads = Hq;
    p.num_kv_heads = Hkv;
    p.head_dim = d;
    p.capacity = cap;
    p.max_seq_len = max_len;
    p.lengths = ragged ? fake<int32_t>() : nullptr;
    p.q = fake<float>(misalign);
    p.k_cache = fake<int8_t>();
    p.v_cache = fake<int8_t>();
    p.k_scale = fake<float>();
    p.v_scale = fake<float>();
    p.out = fake<float>();
    p.softmax_scale = 0.0f;
    p.num_splits = splits;
    p.k_new = append ? fake<float>() : nullptr;
    p.v_new = append ? fake<float>() : nullptr;
    return p;
}

void decode_plans() {
    const int batches[] = {1, 2, 3, 7, 16, 63, 64, 65, 256, 512, 513, 1000, 1024, 1025, 4096, 4097, 65536};
    const int groups[][2] = {{1, 1}, {8, 8}, {32, 32}, {32, 8}, {64, 8}, {32, 2}, {16, 1}, {12, 3}, {5, 5}, {128, 1}};
    const int dims[] = {1, 3, 32, 64, 96, 128, 256, 512, 1024};
    const int lens[] = {1, 31, 32, 33, 1000, 4096, 1 << 17, 1 << 24, INT_MAX};
    const int splits[] = {0, 1, 3, 1000, INT_MAX};
    kvq_plan_info info;
    for (int B : batches) {
        for (const auto& g : groups) {
            for (int d : dims) {
                for (int L : lens) {
                    for (int s : splits) {
                        for (int variant = 0; variant < 4; variant++) {
                            const bool ragged = variant & 1;
                            const bool append = variant & 2;
                            for (uintptr_t mis : {uintptr_t(0), uintptr_t(4)}) {
                                kvq_decode_params p = decode_params(B, g[0], g[1], d, L, L, ragged, s, append, mis);
                                const hipError_t e = kvq_decode_plan(&p, &info);
                                const size_t need = kvq_decode_workspace_size(&p);
                                expect(e == hipSuccess || e == hipErrorInvalidValue, "decode plan status", B, d, L,
                                       s);
                                if (e != hipSuccess) {
                                    expect(need == 0, "rejected decode needs no workspace", B, d, L, s);
                                    continue;
                                }
                                expect(need == info.workspace_bytes, "decode workspace == plan", B, d, L, s);
                                expect(info.kernel >= KVQ_KERNEL_DECODE_GENERIC &&
                                           info.kernel <= KVQ_KERNEL_DECODE_MFMA,
                                       "decode kernel id", B, d, info.kernel);
                                if (info.split_plan == KVQ_SPLITS_TILES && B > kvq::kWave) {
                                    // Beyond one wave of sequences no wave range may span 64
                                    // sequences (each holds kFlatSwitchTiles virtual tiles).
                                    const long U = static_cast<long>(g[1]) * (g[0] / g[1] / info.heads_per_group);
                                    const long waves = kvq::kMfmaWaves * (256 / U);
                                    const long stream = static_cast<long>(B) * ((L + kvq::kMfmaTile - 1) / kvq::kMfmaTile) +
                                                        static_cast<long>(kvq::kFlatSwitchTiles) * B;
                                    expect((stream + waves - 1) / waves < static_cast<long>(kvq::kWave) * kvq::kFlatSwitchTiles,
                                           "tile-stream ranges span fewer than 64 sequences", B, d, L, stream);
                                }
                                if (need > 0) {
                                    expect(kvq_decode_launch(&p, fake<void>(), need - 1, nullptr) ==
                                               hipErrorInvalidValue,
                                           "short decode workspace rejected", B, d, L, s);
                                    expect(kvq_decode_launch(&p, nullptr, need, nullptr) == hipErrorInvalidValue,
                                           "null decode workspace rejected", B, d, L, s);
                                }
                            }
                        }
                    }
                }
            }
        }
    }
    // Rejections of single bad fields (as the ctypes tests, here under the sanitizers).
    for (int which = 0; which < 14; which++) {
        kvq_decode_params p = decode_params(2, 8, 2, 128, 4096, 4096, false, 0, false, 0);
        switch (which) {
            case 0: p.batch = 0; break;
            case 1: p.num_q_heads = 7; break;
            case 2: p.num_kv_heads = 0; break;
            case 3: p.head_dim = 0; break;
            case 4: p.head_dim = 5000; break;
            case 5: p.capacity = 0; break;
            case 6: p.max_seq_len = 5000; break;
            case 7: p.max_seq_len = 0; break;
            case 8: p.q = nullptr; break;
            case 9: p.out = nullptr; break;
            case 10: p.k_cache = nullptr; break;
            case 11: p.v_scale = nullptr; break;
            case 12: p.k_new = fake<float>(); break;
            default: p.num_splits = -1; break;
        }
        expect(kvq_decode_workspace_size(&p) == 0, "bad decode field: no workspace", which);
        expect(kvq_decode_plan(&p, &info) == hipErrorInvalidValue, "bad decode field: plan", which);
        expect(kvq_decode_launch(&p, fake<void>(), size_t(1) << 30, nullptr) == hipErrorInvalidValue,
               "bad decode field: launch", which);
        expect(kvq_decode_launch_noalloc(&p, nullptr) == hipErrorInvalidValue, "bad decode field: noalloc", which);
    }
    expect(kvq_decode_plan(nullptr, &info) == hipErrorInvalidValue, "decode plan null params");
    expect(kvq_decode_workspace_size(nullptr) == 0, "decode workspace null params");
}

void paged_plans() {
    const int pages[] = {1, 16, 32, 48, 64, 128, 1 << 20};
    const int batches[] = {1, 3, 64, 256, 4096};
    const int dims[] = {64, 96, 128, 256};
    for (int ps : pages) {
        for (int B : batches) {
            for (int d : dims) {
                for (int mpp : {1, 4, 4096}) {
                    for (int s : {0, 1, 5}) {
                        kvq_paged_decode_params p{};
                        p.batch = B;
                        p.num_q_heads = 32;
                        p.num_kv_heads = 8;
                        p.head_dim = d;
                        p.page_size = ps;
                        p.num_pages = 1 << 16;
                        p.max_pages_per_seq = mpp;
                        p.max_seq_len = static_cast<int>(std::min<long>(INT_MAX, static_cast<long>(ps) * mpp));
                        p.block_table = fake<int32_t>();
                        p.lengths = fake<int32_t>();
                        p.q = fake<float>();
                        p.k_pages = fake<int8_t>();
                        p.v_pages = fake<int8_t>();
                        p.k_scale_pages = fake<float>();
                        p.v_scale_pages = fake<float>();
                        p.out = fake<float>();
                        p.num_splits = s;
                        const size_t need = kvq_paged_decode_workspace_size(&p);
                        if (need > 0) {
                            expect(kvq_paged_decode_launch(&p, fake<void>(), need - 1, nullptr) ==
                                       hipErrorInvalidValue,
                                   "short paged workspace rejected", B, ps, d, mpp);
                        }
                    }
                }
            }
        }
    }
    expect(kvq_paged_decode_workspace_size(nullptr) == 0, "paged workspace null params");
    expect(kvq_paged_decode_launch(nullptr, fake<void>(), 1 << 20, nullptr) == hipErrorInvalidValue,
           "paged launch null params");
}

// Paged caches may span up to INT_MAX tokens per sequence, but a decode call
// attends to at most KVQ_MAX_SEQ_LEN.  Every accepted plan must keep the
// counts its kernel holds in 32-bit integers in range:
//   * the flattened tile stream (KVQ_SPLITS_TILES): every sequence's tiles at
//     the longest length plus kFlatSwitchTiles virtual tiles per sequence;
//   * static splits: the last split's end, splits * chunk;
//   * every plan: the longest length itself.
void paged_bounds() {
    const int batches[] = {1, 2, 16, 33, 63, 64};
    const int groups[][2] = {{32, 8}, {64, 8}, {8, 2}, {32, 32}};
    const int pages[] = {32, 128, 4096, 1 << 16, 1 << 20};
    const long long wants[] = {1 << 20, (1LL << 30) - 32, 1LL << 30, (1LL << 30) + 1, 1LL << 31};
    kvq_plan_info info;
    long flat_seen = 0;
    for (int B : batches) {
        for (const auto& g : groups) {
            for (int d : {64, 128}) {
                for (int ps : pages) {
                    for (long long want : wants) {
                        // Table row long enough for `want` tokens, capped at INT_MAX tokens.
                        const long long mpp_ll = std::min<long long>((want + ps - 1) / ps, INT_MAX / ps);
                        const int mpp = static_cast<int>(mpp_ll);
                        const long long cap = static_cast<long long>(mpp) * ps;
                        for (int msl_kind = 0; msl_kind < 2; msl_kind++) {
                            for (int s : {0, 2, 7}) {
                                kvq_paged_decode_params p{};
                                p.batch = B;
                                p.num_q_heads = g[0];
                                p.num_kv_heads = g[1];
                                p.head_dim = d;
                                p.page_size = ps;
                                p.num_pages = 1 << 16;
                                p.max_pages_per_seq = mpp;
                                p.max_seq_len = msl_kind == 0 ? 0 : static_cast<int>(std::min<long long>(want, cap));
                                p.block_table = fake<int32_t>();
                                p.lengths = fake<int32_t>();
                                p.q = fake<float>();
                                p.k_pages = fake<int8_t>();
                                p.v_pages = fake<int8_t>();
                                p.k_scale_pages = fake<float>();
                                p.v_scale_pages = fake<float>();
                                p.out = fake<float>();
                                p.num_splits = s;
                                const long long eff = p.max_seq_len > 0 ? p.max_seq_len : cap;
                                const hipError_t e = kvq_paged_decode_plan(&p, &info);
                                const bool table_ok = static_cast<long long>(B) * mpp <= INT_MAX;
                                expect((e == hipSuccess) == (eff <= KVQ_MAX_SEQ_LEN && table_ok),
                                       "paged plan accepted iff length <= KVQ_MAX_SEQ_LEN", B, ps, eff, e);
                                expect(kvq_paged_decode_workspace_size(&p) == (e == hipSuccess ? info.workspace_bytes : 0),
                                       "paged workspace == plan", B, ps, eff);
                                if (e != hipSuccess) continue;
                                if (info.split_plan == KVQ_SPLITS_TILES) {
                                    flat_seen++;
                                    const long long stream =
                                        B * ((eff + kvq::kMfmaTile - 1) / kvq::kMfmaTile) +
                                        static_cast<long long>(kvq::kFlatSwitchTiles) * B;
                                    expect(stream <= INT_MAX, "tile stream fits int32", B, ps, eff, stream >> 20);
                                }
                                if (info.split_plan == KVQ_SPLITS_STATIC && info.splits > 1) {
                                    expect(static_cast<long long>(info.splits) * info.chunk <= INT_MAX,
                                           "last split end fits int32", B, ps, eff, info.splits);
                                }
                            }
                        }
                    }
                }
            }
        }
    }
    // Unless a planner switch keeps it off (KVQ_FORCE_KERNEL, KVQ_FLAT_PLAN=0).
    const char* flat_env = std::getenv("KVQ_FLAT_PLAN");
    const bool flat_on = (kvq_diagnostics() >> 4) == 0 && !(flat_env && std::strcmp(flat_env, "0") == 0);
    expect(flat_seen > 0 || !flat_on, "the sweep reaches the tile-stream plan", flat_seen);
    expect(kvq_paged_decode_plan(nullptr, &info) == hipErrorInvalidValue, "paged plan null params");
}

void attention_plans() {
    const int Ms[] = {1, 2, 3, 4, 5, 8, 9, 15, 16, 17, 63, 64, 65, 128, 1000, 1 << 17};
    const int Ns[] = {1, 31, 32, 33, 64, 4096, 65536, 1 << 20};
    const int dims[] = {1, 16, 32, 33, 64, 96, 128, 256, 1024};
    kvq_plan_info info;
    for (int M : Ms) {
        for (int N : Ns) {
            for (int d : dims) {
                for (int s : {0, 1, 7, 1 << 20}) {
                    for (uintptr_t mis : {uintptr_t(0), uintptr_t(4)}) {
                        kvq_attention_params p{M, N, d, fake<float>(), fake<float>(mis), fake<float>(),
                                               fake<float>(), 0.0f, s};
                        const hipError_t e = kvq_attention_plan(&p, &info);
                        const size_t need = kvq_attention_workspace_size(&p);
                        expect(e == hipSuccess, "attention plan accepted", M, N, d, s);
                        expect(need == info.workspace_bytes, "attention workspace == plan", M, N, d, s);
                        if (mis) {
                            expect(info.kernel == KVQ_KERNEL_ATTENTION_GENERIC && need == 0,
                                   "misaligned attention is generic", M, N, d, info.kernel);
                        }
                        if (need > 0) {
                            expect(kvq_attention_launch(&p, fake<void>(), need - 1, nullptr) == hipErrorInvalidValue,
                                   "short attention workspace rejected", M, N, d, s);
                        }
                    }
                }
            }
        }
    }
    const int bad[][3] = {{0, 4, 64}, {4, 0, 64}, {4, 4, 0}, {-1, 4, 64}, {4, -3, 64}, {4, 4, -8}, {4, 4, 1025}};
    for (const auto& b : bad) {
        kvq_attention_params p{b[0], b[1], b[2], fake<float>(), fake<float>(), fake<float>(), fake<float>(), 0.0f, 0};
        expect(kvq_attention_plan(&p, &info) == hipErrorInvalidValue, "bad attention plan", b[0], b[1], b[2]);
        expect(kvq_attention_workspace_size(&p) == 0, "bad attention workspace", b[0], b[1], b[2]);
        expect(attention_online_launch(fake<float>(), fake<float>(), fake<float>(), fake<float>(), b[0], b[1], b[2],
                                       nullptr) == hipErrorInvalidValue,
               "bad attention_online_launch", b[0], b[1], b[2]);
    }
}

void writers() {
    // Append / paged append / prefill / quantize: single bad fields.
    for (int which = 0; which < 6; which++) {
        kvq_append_params a{2, 2, 128, 64, nullptr, 0, fake<float>(), fake<float>(), fake<int8_t>(), fake<int8_t>(),
                            fake<float>(), fake<float>()};
        switch (which) {
            case 0: a.batch = 0; break;
            case 1: a.head_dim = 0; break;
            case 2: a.head_dim = 5000; break;
            case 3: a.capacity = 0; break;
            case 4: a.k_new = nullptr; break;
            default: a.v_scale = nullptr; break;
        }
        expect(kvq_append_launch(&a, nullptr) == hipErrorInvalidValue, "bad append", which);
    }
    expect(kvq_append_launch(nullptr, nullptr) == hipErrorInvalidValue, "append null params");
    for (int which = 0; which < 7; which++) {
        kvq_paged_append_params a{2, 2, 128, 32, 10, 4, fake<int32_t>(), nullptr, 0, fake<float>(), fake<float>(),
                                  fake<int8_t>(), fake<int8_t>(), fake<float>(), fake<float>()};
        switch (which) {
            case 0: a.block_table = nullptr; break;
            case 1: a.k_new = nullptr; break;
            case 2: a.page_size = 0; break;
            case 3: a.num_pages = 0; break;
            case 4: a.max_pages_per_seq = 0; break;
            case 5: a.head_dim = 0; break;
            default: a.v_scale_pages = nullptr; break;
        }
        expect(kvq_paged_append_launch(&a, nullptr) == hipErrorInvalidValue, "bad paged append", which);
    }
    expect(kvq_paged_append_launch(nullptr, nullptr) == hipErrorInvalidValue, "paged append null params");
    for (int which = 0; which < 11; which++) {
        kvq_prefill_params p{};
        p.batch = 2;
        p.num_kv_heads = 2;
        p.head_dim = 128;
        p.tokens = 16;
        p.dtype = KVQ_DTYPE_F32;
        p.k_new = fake<void>();
        p.v_new = fake<void>();
        p.capacity = 64;
        p.k_cache = fake<int8_t>();
        p.v_cache = fake<int8_t>();
        p.k_scale = fake<float>();
        p.v_scale = fake<float>();
        switch (which) {
            case 0: p.batch = 0; break;
            case 1: p.head_dim = 0; break;
            case 2: p.head_dim = 5000; break;
            case 3: p.tokens = -1; break;
            case 4: p.dtype = 2; break;
            case 5: p.k_new = nullptr; break;
            case 6: p.v_scale = nullptr; break;
            case 7: p.capacity = 0; break;
            case 8: p.block_table = fake<int32_t>(); break;
            case 9:
                p.block_table = fake<int32_t>();
                p.page_size = 16;
                p.num_pages = 4;
                break;
            default:
                p.batch = 1 << 16;
                p.num_kv_heads = 1 << 8;
                p.tokens = 1 << 8;
                break;
        }
        expect(kvq_prefill_quantize_launch(&p, nullptr) == hipErrorInvalidValue, "bad prefill", which);
    }
    expect(kvq_prefill_quantize_launch(nullptr, nullptr) == hipErrorInvalidValue, "prefill null params");
    expect(kvq_quantize_rows_launch(nullptr, 4, 128, fake<int8_t>(), fake<float>(), nullptr) == hipErrorInvalidValue,
           "quantize null input");
    expect(kvq_quantize_rows_launch(fake<float>(), -1, 128, fake<int8_t>(), fake<float>(), nullptr) ==
               hipErrorInvalidValue,
           "quantize negative rows");
    expect(kvq_quantize_rows_launch(fake<float>(), 4, 0, fake<int8_t>(), fake<float>(), nullptr) ==
               hipErrorInvalidValue,
           "quantize zero head dim");
    expect(kvq_workspace_init(nullptr, 64, nullptr) == hipErrorInvalidValue, "workspace init null");
}

}  // namespace

int main() {
    const char* v = kvq_version();
    expect(v != nullptr && v[0] == 'k', "version string");
    expect(kvq_diagnostics() >= 0, "diagnostics");
    reference_abi();
    decode_plans();
    paged_plans();
    paged_bounds();
    attention_plans();
    writers();
    if (g_fails) {
        std::printf("FAILED %ld of %ld checks\n", g_fails, g_checks);
        return 1;
    }
    std::printf("OK %ld\n", g_checks);
    return 0;
}
