// kvq_decode_mfma.hip -- grouped-query decode attention on gfx950 matrix cores.
//
// For G query heads sharing a kv head the per-token work is a small dense
// contraction (QK: [G x D] x [D x T], PV: [G x T] x [T x D]), so with G = 4
// or 8 it runs on MFMA instead of per-lane FMAs.  Same math and result
// contract as decode_fast (the reference's cpu_reference per query head,
// kv_cache/KV_int8_split_optimized.cu:385-437); head dim D = 64 or 128.
//
// One workgroup (4 waves) per (sequence split, batch, kv head, group of G
// query heads); each wave walks 32-token tiles with its own online-softmax
// state, merged across waves through LDS at the end.  Per tile:
//
// * QK on v_mfma_i32_16x16x64_i8.  The int8 K rows go from memory straight
//   into the A operand (lane l: token l%16, dims 16*(l/16) + [0,16) of each
//   64-dim block); no dequantisation instruction touches K.  q is held as three
//   balanced int8 limbs of a 22-bit fixed-point value per head (q*2^E rounded
//   once, |error| <= 2^-23 * max|q|), one MFMA column block per limb; the int32
//   products are exact, and dot = ((C0*2^16 + C1*2^8) + C2) * 2^-E.
//   MFMA rows n = 0..15 all carry head n % G (duplicates are free).
// * softmax: the running max m of s = (dot * k_scale) * softmax_scale * log2 e
//   gives p = exp2(s - m) and the denominator; the PV weights are
//   w = p * v_scale * 2^15 / vref, with vref the running max of |v_scale|, so
//   |w| <= 2^15 whatever the scale magnitudes.  A tile that raises m or vref
//   rescales the accumulator once (skipped when no row of the wave changed).
// * PV on v_mfma_f32_16x16x32_f16 computing O^T[dim, row] += V^T P: the
//   weights are split into f16 hi + lo rows (rows n < G.. hold hi, the next G
//   rows lo), so the product keeps ~22 bits; int8 V is exact in f16.
//   V tiles are staged in LDS (rows XOR-swizzled in 16-byte pieces, conflict
//   free) and read back transposed with ds_read_b64_tr_b8: within each 16-lane
//   group, lanes 2r and 2r+1 address the two 8-byte halves of row r and lane i
//   receives byte i of each row -- 8 tokens of one dim, the A operand layout.
//   The token order of a lane group's k-slots (4g..4g+3, 16+4g..16+4g+3)
//   matches where the QK C layout left that lane's probabilities, so P needs
//   no data movement.
// * fused append: the new token is quantised by the one wave whose last tile
//   holds token length-1 (its fp32 loads were issued at kernel start) and
//   substituted from LDS into that tile.
#include <math.h>

#include "kvq_device.hpp"
#include "kvq_internal.hpp"
#include "kvq_split.hpp"

namespace kvq {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

constexpr int kMWaves = kMfmaWaves;  // waves per workgroup
constexpr int kMTile = kMfmaTile;  // tokens per wave tile
constexpr float kPScale = 32768.0f;  // PV weights are formed in [-2^15, 2^15] before the f16 split
constexpr int kMBStep = kMTile * kMWaves;

// 8 signed bytes -> 8 f16 (exact): bias each byte to unsigned, place it under
// the f16 exponent of 1024 (0x64xx = 1024 + u), subtract 1152 = 1024 + 128.
__device__ __forceinline__ f16x8 i8x8_to_f16(i32x2 v) {
    const unsigned x0 = static_cast<unsigned>(v.x) ^ 0x80808080u;
    const unsigned x1 = static_cast<unsigned>(v.y) ^ 0x80808080u;
    const unsigned w0 = __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u);
    const unsigned w1 = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u);
    const unsigned w2 = __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u);
    const unsigned w3 = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u);
    const f16x2 bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    const f16x2 h0 = __builtin_bit_cast(f16x2, w0) - bias;
    const f16x2 h1 = __builtin_bit_cast(f16x2, w1) - bias;
    const f16x2 h2 = __builtin_bit_cast(f16x2, w2) - bias;
    const f16x2 h3 = __builtin_bit_cast(f16x2, w3) - bias;
    return f16x8{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
}

__device__ __forceinline__ int pack_bytes(const int* b) {
    return (b[0] & 0xff) | ((b[1] & 0xff) << 8) | ((b[2] & 0xff) << 16) |
           static_cast<int>(static_cast<unsigned>(b[3] & 0xff) << 24);
}

// Piece slot of 16-byte piece p of V row rw in an LDS tile (rows of D / 16
// pieces).  LDS serves 256 bytes (64 banks of 4 bytes) per cycle, and a
// transposed read takes 32 lanes per cycle: 16 rows (4g .. 4g+3 and
// 16+4g .. 16+4g+3 for the two 16-lane groups g of the half wave) of 16
// bytes each.  A row's 16-byte bank group is (row bytes / 16 * rw + slot)
// mod 16, so rows that share a bank half (D = 128: equal parity; D = 64:
// equal rw mod 4) must get distinct slots.  Tile stores write whole rows, so
// any per-row permutation keeps them conflict-free.
template <int D>
__device__ __forceinline__ int v_slot(int p, int rw) {
    if constexpr (D == 128) return p ^ (((rw >> 1) & 3) | ((rw >> 2) & 4));
    else return p ^ (((rw >> 2) & 1) | ((rw >> 3) & 2));
}

template <int D, int G, bool PAGED, bool FIT>
__global__ __launch_bounds__(kMWaves* kWave) __attribute__((amdgpu_waves_per_eu(2))) void decode_mfma(
    const DecodeArgs a) {
    static_assert(G == 4 || G == 8, "heads per workgroup");
    static_assert(D == 64 || D == 128, "head dims of the matrix-core decode kernel");
    constexpr int NJ = D / 64;            // 64-dim blocks of a K row (QK k-steps, q limb blocks)
    constexpr int NB = D / 16;            // 16-byte pieces of a row (PV blocks)
    constexpr int RPLV = kWave / NB;      // V rows one tile load instruction covers
    constexpr int NV = kMTile / RPLV;     // V load instructions per tile
    constexpr int NE = 2 * D / kWave;     // appended K+V elements per lane of the owning wave
    // V tile buffers during the tile loop; the waves' results afterwards
    // (rows padded by one float, so the lanes of one result column, 16 rows
    // apart, hit different banks).
    // (Before the tile loop, the in-kernel schedule's scratch; at the end, the
    // merge's.)
    union TileOrResult {
        int8_t v[kMWaves][2][kMTile * D];
        float acc[kMWaves][16][D + 1];
        LptScratch lpt;
        MergeScratch merge;  // finish_split, after s_acc's last read
    };
    static_assert(kMWaves * kWave == kLptThreads, "locate_lpt's workgroup size");
    __shared__ __align__(16) TileOrResult s_u;
    auto& s_v = s_u.v;
    auto& s_acc = s_u.acc;
    __shared__ float s_ml[kMWaves][G][2];
    __shared__ __align__(16) int8_t s_newq[2][D];
    __shared__ int s_last;
    __shared__ int s_pick[5];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r = lane & 15;   // MFMA row / token-in-subtile index
    const int g = lane >> 4;   // 16-lane group

    SplitWork w;
    if constexpr (FIT) {
        if (!locate_fit(a, w)) return;
    } else if (a.lpt_target > 0) {
        if (!locate_lpt(a, w, s_u.lpt, s_pick)) return;
    } else {
        if (!locate_work(a, w)) return;
    }
    const int unit = w.unit;
    const int bh = unit / a.nsg;
    const int sgi = unit - bh * a.nsg;
    const int b = bh / a.Hkv;
    const int kvh = bh - b * a.Hkv;
    const int hq0 = kvh * a.G + sgi * G;
    const size_t bhq0 = static_cast<size_t>(b) * a.Hq + hq0;
    const int len = w.len;
    const int split = w.split;
    const int nsplit = w.nsplit;

    if (len == 0) {
        for (int i = threadIdx.x; i < G * D; i += blockDim.x) a.out[bhq0 * D + i] = 0.0f;
        return;
    }

    const int t0 = w.t0;
    const int tend = w.t1;
    const bool app = (a.k_new != nullptr) && (tend == len);
    const int tnew = len - 1;
    const size_t row0 = static_cast<size_t>(bh) * a.cap;

    // Fused append: the wave whose tiles include token len-1 (wave w's tiles
    // start at t0 + 32 w + 128 i) quantises the new token on its own; its fp32
    // row is fetched first (element lane + 64 j: j < NJ of K, j >= NJ of V).
    const bool own_new = app && ((tnew - t0) / kMTile) % kMWaves == wave;
    float xnew[NE];
#pragma unroll
    for (int j = 0; j < NE; j++)
        xnew[j] = own_new ? (j < NJ ? a.k_new : a.v_new)[static_cast<size_t>(bh) * D + ((lane + kWave * j) & (D - 1))]
                          : 0.0f;

    // q of head (r % G) as int8 limbs in the QK B operand layout:
    // qb[j][limb] holds dims 64j + 16g + [0,16).
    const int hrow = r % G;
    float qv[16 * NJ];
    {
        const float* qp = a.q + (bhq0 + hrow) * D + 16 * g;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
#pragma unroll
            for (int i4 = 0; i4 < 4; i4++) {
                const float4 x = *reinterpret_cast<const float4*>(qp + 64 * j + 4 * i4);
                qv[16 * j + 4 * i4] = x.x;
                qv[16 * j + 4 * i4 + 1] = x.y;
                qv[16 * j + 4 * i4 + 2] = x.z;
                qv[16 * j + 4 * i4 + 3] = x.w;
            }
        }
    }
    // The limbs are formed after the first tile's loads are issued (their
    // latency overlaps this work); qs turns an integer dot into a score in
    // log2 units (after x k_scale).
    i32x4 qb[NJ][3];
    float qs = 0.0f;
    auto prepare_q = [&]() {
        float qmax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16 * NJ; i++) qmax = fmaxf(qmax, fabsf(qv[i]));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
        int qexp = 0;
        frexpf(qmax, &qexp);  // qmax < 2^qexp
        const int E = qmax > 0.0f ? min(max(22 - qexp, -100), 126) : 0;
        qs = ldexpf(1.0f, -E) * a.scale_log2;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            int limb[3][16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int Q = static_cast<int>(__builtin_rintf(ldexpf(qv[16 * j + i], E)));
                const int l2 = ((Q + 128) & 255) - 128;
                const int Q1 = (Q - l2) >> 8;
                const int l1 = ((Q1 + 128) & 255) - 128;
                limb[0][i] = (Q1 - l1) >> 8;
                limb[1][i] = l1;
                limb[2][i] = l2;
            }
#pragma unroll
            for (int lb = 0; lb < 3; lb++)
                qb[j][lb] = i32x4{pack_bytes(&limb[lb][0]), pack_bytes(&limb[lb][4]), pack_bytes(&limb[lb][8]),
                                  pack_bytes(&limb[lb][12])};
        }
    };

    // Online-softmax state of head hrow (identical in every lane of that
    // row): the score max m (log2 units), the denominator lsum, and vref, the
    // running max of |v_scale| that keeps the PV weights p * v_scale / vref in
    // [-1, 1].  acc[c] holds O^T[16c + 4g + i][row r] in units of
    // vref / kPScale.
    float m = -INFINITY, lsum = 0.0f, vref = 0.0f;
    f32x4 acc[NB];
#pragma unroll
    for (int c = 0; c < NB; c++) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const bool lo_row = ((r / G) & 1) != 0;

    // This (batch, kv head)'s cache rows as buffer resources: tile loads add a
    // fixed per-lane offset to a wave-uniform tile offset, and a tail tile's
    // reads past the capacity return 0.  A paged cache gets resources per
    // tile instead (below).
    const unsigned cap = static_cast<unsigned>(a.cap);
    const buf_rsrc kres = make_rsrc(a.k + row0 * D, cap * D);
    const buf_rsrc vres = make_rsrc(a.v + row0 * D, cap * D);
    const buf_rsrc ksres = make_rsrc(a.ks + row0, cap * 4u);
    const buf_rsrc vsres = make_rsrc(a.vs + row0, cap * 4u);

    // The transposed V reads: lanes 2rr + h2 of group g address row R(rr),
    // half h2, of each 16-dim piece.
    const int rr = (lane & 15) >> 1;
    const int h2 = lane & 1;
    const int vrow = rr < 4 ? 4 * g + rr : 16 + 4 * g + (rr - 4);

    // Fused append, part 2 (the owning wave, no workgroup barrier): per-row
    // max|x|, the scale, the quantised elements -- same rule and bits as
    // append_kernel.  The rows land in LDS for the final tile and in the cache
    // for later steps (once per kv head).
    float newks = 0.0f, newvs = 0.0f;
    auto append_new = [&]() {
        const size_t rnew = PAGED ? cache_row(a.pages, a.Hkv, a.cap, b, kvh, tnew) : row0 + tnew;
        float amk = fabsf(xnew[0]), amv = fabsf(xnew[NJ]);
#pragma unroll
        for (int j = 1; j < NJ; j++) {
            amk = fmaxf(amk, fabsf(xnew[j]));
            amv = fmaxf(amv, fabsf(xnew[NJ + j]));
        }
        newks = quant_scale(wave_max(amk));
        newvs = quant_scale(wave_max(amv));
#pragma unroll
        for (int j = 0; j < NE; j++)
            s_newq[j / NJ][lane + kWave * (j % NJ)] = static_cast<int8_t>(quant_one(xnew[j], j < NJ ? newks : newvs));
        if (sgi == 0) {
            if (lane < 2 * NB) {
                const int row = lane / NB, piece = lane % NB;
                *reinterpret_cast<int4*>((row ? a.v : a.k) + rnew * D + 16 * piece) =
                    *reinterpret_cast<const int4*>(&s_newq[row][16 * piece]);
            }
            if (lane == 0) {
                a.ks[rnew] = newks;
                a.vs[rnew] = newvs;
            }
        }
    };

    // One tile's global data in registers: K sub-tiles (A operand of QK), the
    // 32 V rows (16 bytes per lane) and the scales of tokens base+16s+4g+i.
    struct Tile {
        i32x4 ka[2][NJ];
        int4 v[NV];
        float ks[2][4], vs[2][4];
    };
    const int wbase = t0 + __builtin_amdgcn_readfirstlane(wave) * kMTile;  // wave-uniform
    const int ntiles = wbase < tend ? (tend - wbase + kMBStep - 1) / kMBStep : 0;
    // Lane byte offsets within a tile: K row r, dims 16g.. (+64 for the second
    // 64-dim block, +16 rows for sub-tile 1); V row lane/8, 16-byte piece
    // lane%8 (+8 rows per c); scales of tokens 4g..4g+3 (+16 tokens for s = 1).
    const int kvo = r * D + 16 * g;
    const int vvo = (lane / NB) * D + 16 * (lane % NB);
    const int svo = 16 * g;
    // Paged: each tile's page id comes from the block table one tile ahead,
    // by a vector load issued before the previous tile's K/V loads, so a
    // tile's loads wait only for that id (in-order vector-memory counter),
    // never for a table round trip of their own (cfg3 with 128-token pages
    // ran 61.9 us against 46.7 contiguous with the lookup inside the tile).
    // Page sizes are powers of two here; indices past the table's row are
    // clamped into it.
    const buf_rsrc tabr =
        make_rsrc(PAGED ? a.pages.table + static_cast<size_t>(b) * a.pages.max_pages : nullptr,
                  PAGED ? static_cast<unsigned>(a.pages.max_pages) * 4u : 0u);
    auto fetch_page = [&](int it) {
        const int pi = min((wbase + it * kMBStep) >> a.pages.shift, a.pages.max_pages - 1);
        return __builtin_amdgcn_raw_buffer_load_b32(tabr, pi * 4, 0, 0);
    };
    int pg_next = 0;
    if constexpr (PAGED) pg_next = fetch_page(0);
    auto load_tile = [&](Tile& T, int it) {
        const int base = wbase + it * kMBStep;
        int ko = base * D;
        int so = base * 4;
        buf_rsrc kr = kres, vr = vres, ksr = ksres, vsr = vsres;
        if constexpr (PAGED) {
            // The tile lies in one page (page size a multiple of 32): resources
            // from its first token to the end of that page.
            const int page = min(max(__builtin_amdgcn_readfirstlane(pg_next), 0), a.pages.num_pages - 1);
            pg_next = fetch_page(it + 1);
            const size_t rp = (static_cast<size_t>(page) * a.Hkv + kvh) * a.pages.size + (base & (a.pages.size - 1));
            const unsigned rem = static_cast<unsigned>(a.pages.size - (base & (a.pages.size - 1)));
            kr = make_rsrc(a.k + rp * D, rem * D);
            vr = make_rsrc(a.v + rp * D, rem * D);
            ksr = make_rsrc(a.ks + rp, rem * 4u);
            vsr = make_rsrc(a.vs + rp, rem * 4u);
            ko = so = 0;
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
#pragma unroll
            for (int j = 0; j < NJ; j++) T.ka[s][j] = buffer_load16_stream(kr, kvo + s * 16 * D + 64 * j, ko);
        }
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const v4i_t x = buffer_load16_stream(vr, vvo + c * RPLV * D, ko);
            T.v[c] = make_int4(x.x, x.y, x.z, x.w);
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const v4i_t xk = buffer_load16(ksr, svo + 64 * s, so);
            const v4i_t xv = buffer_load16(vsr, svo + 64 * s, so);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                T.ks[s][i] = __int_as_float(xk[i]);
                T.vs[s][i] = __int_as_float(xv[i]);
            }
        }
    };
    // V rows into an LDS tile buffer: 16-byte piece p of row rw is stored at
    // slot v_slot(p, rw), which keeps the transposed reads conflict-free.
    auto stage_v = [&](const Tile& T, int8_t* vt) {
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const int rw = RPLV * c + lane / NB;
            const int p = lane % NB;
            *reinterpret_cast<int4*>(vt + rw * D + (v_slot<D>(p, rw) << 4)) = T.v[c];
        }
    };
    // The appended token replaces what the cache held at position len-1 (only
    // the workgroup's final tile can contain it): K and scales in registers,
    // the V row in the tile's LDS buffer.
    auto substitute_new = [&](Tile& T, int base, int8_t* vt) {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            if (base + 16 * s + r == tnew) {
#pragma unroll
                for (int j = 0; j < NJ; j++) T.ka[s][j] = *reinterpret_cast<const i32x4*>(&s_newq[0][64 * j + 16 * g]);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (base + 16 * s + 4 * g + i == tnew) {
                    T.ks[s][i] = newks;
                    T.vs[s][i] = newvs;
                }
        }
        const int rw = tnew - base;
        if (rw >= 0 && rw < kMTile && lane < NB)
            *reinterpret_cast<int4*>(vt + rw * D + (v_slot<D>(lane, rw) << 4)) =
                *reinterpret_cast<const int4*>(&s_newq[1][16 * lane]);
    };
    // check_tail: the tile may reach past tend (only a wave's last tile can).
    auto compute = [&](const Tile& T, int base, const int8_t* vt, bool check_tail) {
        // QK: C[token 4g + i][row r] per sub-tile and limb.
        i32x4 cq[2][3];
#pragma unroll
        for (int s = 0; s < 2; s++) {
#pragma unroll
            for (int lb = 0; lb < 3; lb++) {
                i32x4 c = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < NJ; j++) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(T.ka[s][j], qb[j][lb], c, 0, 0, 0);
                cq[s][lb] = c;
            }
        }
        // Scores in log2 units, k-slot order s*4 + i: the low limbs combine
        // exactly in int32 ((C1 << 8) + C2 < 2^30), the top limb in fp32.
        float sc[8], vsv[8];
        float mt = -INFINITY, vmax = 0.0f;
#pragma unroll
        for (int s = 0; s < 2; s++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int low = (cq[s][1][i] << 8) + cq[s][2][i];
                const float dot = static_cast<float>(cq[s][0][i]) * 65536.0f + static_cast<float>(low);
                sc[4 * s + i] = (dot * T.ks[s][i]) * qs;
                vsv[4 * s + i] = T.vs[s][i];
            }
        }
        if (check_tail && base + kMTile > tend) {
            // Tail tile: tokens past tend (the next split's, or whatever the
            // cache holds past the sequence) get no weight, whatever their
            // scales hold.
#pragma unroll
            for (int s = 0; s < 2; s++) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (base + 16 * s + 4 * g + i >= tend) {
                        sc[4 * s + i] = -INFINITY;
                        vsv[4 * s + i] = 0.0f;
                    }
            }
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            mt = fmaxf(mt, sc[k]);
            vmax = fmaxf(vmax, fabsf(vsv[k]));
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        vmax = fmaxf(vmax, __shfl_xor(vmax, 16));
        vmax = fmaxf(vmax, __shfl_xor(vmax, 32));
        const float mn = fmaxf(m, mt);
        const float ms = mn == -INFINITY ? 0.0f : mn;
        const float alpha = fast_exp2(m - ms);
        const float vn = fmaxf(vref, vmax);
        const float rvn = vn > 0.0f ? __builtin_amdgcn_rcpf(vn) : 0.0f;  // v_rcp_f32, 1 ulp
        const float f = vn > 0.0f ? alpha * (vref * rvn) : alpha;
        const float winv = kPScale * rvn;
        m = mn;
        vref = vn;
        if (__builtin_amdgcn_ballot_w64(f != 1.0f) != 0) {  // a row's max or vref moved
#pragma unroll
            for (int c = 0; c < NB; c++) acc[c] *= f;
        }
        // P^T as the PV B operand: row r takes the hi or lo f16 part of
        // w = p * v_scale * kPScale / vref.
        float ps = 0.0f;
        f16x8 pb;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float p = fast_exp2(sc[k] - ms);
            ps += p;
            const float w = p * (vsv[k] * winv);
            const _Float16 hi = static_cast<_Float16>(w);
            const _Float16 lo = static_cast<_Float16>(w - static_cast<float>(hi));
            pb[k] = lo_row ? lo : hi;
        }
        lsum = lsum * alpha + ps;
        // PV: D / 16 blocks of 16 dims.
#pragma unroll
        for (int c = 0; c < NB; c++) {
            const int8_t* src = vt + vrow * D + (v_slot<D>(c, vrow) << 4) + 8 * h2;
            const i32x2 vb = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(const_cast<int8_t*>(src)));
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(i8x8_to_f16(vb), pb, acc[c], 0, 0, 0);
        }
    };

    // Software-pipelined tile loop: tile i+1's global loads are in flight
    // while tile i is computed; its V rows go to LDS buffer (i+1) % 2 at the
    // end of the iteration.  Two register tiles alternate (the loop body is
    // written out twice), so no tile is copied.
    Tile ta, tb;
    auto inner = [&](Tile& T, Tile& N, int it) {  // any tile but the last
        load_tile(N, it + 1);
        compute(T, wbase + it * kMBStep, s_v[wave][it & 1], false);
        stage_v(N, s_v[wave][(it + 1) & 1]);
    };
    if (ntiles > 0) {
        load_tile(ta, 0);
        prepare_q();
        stage_v(ta, s_v[wave][0]);
        int it = 0;
        for (; it + 2 < ntiles; it += 2) {
            inner(ta, tb, it);
            inner(tb, ta, it + 1);
        }
        if (it + 1 < ntiles) {
            inner(ta, tb, it);
            ta = tb;
            it++;
        }
        const int base = wbase + it * kMBStep;
        int8_t* vt = s_v[wave][it & 1];
        if (own_new) {
            append_new();
            substitute_new(ta, base, vt);
        }
        compute(ta, base, vt, true);
    }

    // Wave results to LDS: the softmax sum over the 4 lane groups, and the
    // accumulator in output units (relative to the score max m).
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    __syncthreads();  // every wave is done with its V tiles (s_acc reuses them)
    const float fct = vref * (1.0f / kPScale);
#pragma unroll
    for (int c = 0; c < NB; c++) {
#pragma unroll
        for (int i = 0; i < 4; i++) s_acc[wave][r][16 * c + 4 * g + i] = acc[c][i] * fct;
    }
    if (g == 0 && r < G) {
        s_ml[wave][r][0] = m;
        s_ml[wave][r][1] = lsum;
    }
    __syncthreads();

    // Merge the waves and the hi/lo rows; one thread per (head, element).
    RecMap map{0, 0, 0};
    if (nsplit > 1) {
        map = rec_map(a, w, bhq0);
    }
    for (int i = threadIdx.x; i < G * D; i += blockDim.x) {
        const int h = i / D;
        const int dim = i - h * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kMWaves; w++) M = fmaxf(M, s_ml[w][h][0]);
        const float Ms = M == -INFINITY ? 0.0f : M;
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kMWaves; w++) {
            const float f = fast_exp2(s_ml[w][h][0] - Ms);
            L = fmaf(s_ml[w][h][1], f, L);
            A = fmaf(s_acc[w][h][dim] + s_acc[w][h + G][dim], f, A);
        }
        store_result(a, map, bhq0, h, dim, split, nsplit, M, L, A);
    }
    finish_split<true>(a, unit, map, bhq0, G, nsplit, &s_last, s_u.merge);
}


// ---------------------------------------------------------------------------
// decode_mfma_flat: a ragged batch of at most kFlatMaxSeqs sequences, balanced
// over waves rather than over whole work items.
//
// For one work unit (kv head, head group) the sequences' 32-token tiles are
// laid end to end: sequence b owns tiles [E_b, E_b + n_b), n_b = ceil(len_b /
// 32), T tiles in all.  The W = 4 * fit_items waves of the unit's workgroups
// take equal contiguous ranges of that stream (tile counts differ by at most
// one), whatever the lengths, where a plan of whole items per sequence waits
// for its largest item (cfg2: 1.26-1.36x the mean).  A wave's range may cross
// sequence boundaries: the tile loads run one tile ahead across the switch
// (the next sequence's q is loaded with its first tile), so a switch costs no
// pipeline drain.  Per wave, straight from registers (no LDS, no barrier):
// * a segment that covers a whole sequence writes its output;
// * any other segment writes a partial record with id gw + b (gw: the
//   wave's index in the unit).  Ids gw + b are distinct for distinct (wave,
//   sequence) pairs because both grow along the stream.
// Each record counts one arrival on its sequence's counter; the arrival that
// completes the count of waves covering b (known from the plan) merges b's
// records (merge_wave_records, one wave) and resets the counter.  A wave's
// first segment, when it is a sequence's tail, arrives as soon as its stores
// have drained, inside the tile loop, so that merge overlaps other waves'
// streaming.  Every wave computes the same plan from the device lengths:
// with lane operations up to 64 sequences (lane b holds sequence b), and
// beyond that from a block-wide scan of the lengths into LDS, through a
// window of 64 sequences that moves along the wave's range.
// ---------------------------------------------------------------------------

// A stream of T tiles over W waves: with q = T / W and r = T % W, wave j
// takes q + 1 tiles if j < r, else q, starting at tile j * q + min(j, r)
// (32-bit arithmetic only).  With T < W the first T waves take one tile each,
// so every wave of a covering range holds tiles.
struct FlatSplit {
    int q, r;
};
__device__ __forceinline__ FlatSplit flat_split(int T, int W) {
    const unsigned q = static_cast<unsigned>(T) / static_cast<unsigned>(W);
    return {static_cast<int>(q), T - static_cast<int>(q) * W};
}
__device__ __forceinline__ int flat_start(const FlatSplit& f, int j) { return j * f.q + min(j, f.r); }
__device__ __forceinline__ int flat_wave_of(const FlatSplit& f, int t) {  // the wave holding tile t < T
    const int big = f.r * (f.q + 1);  // tiles of the waves that take q + 1
    if (t < big) return static_cast<int>(static_cast<unsigned>(t) / static_cast<unsigned>(f.q + 1));
    return f.r + static_cast<int>(static_cast<unsigned>(t - big) / static_cast<unsigned>(f.q));
}

// Log-sum-exp merge, by one wave, of sequence b's records for query heads
// hq0 .. + G - 1 under the flattened plan: one record per wave covering b,
// ids w0 + b .. w0 + b + nrec - 1, record id r of head hq at row r * Hq + hq.
// kWave / G lanes per head, each with D / 4 / (kWave / G) 16-byte columns:
// a record's (m, l) load serves all of a lane's columns, and KR records per
// round are loaded together with device-coherent buffer loads.
template <int D, int G>
__device__ inline void merge_wave_records(const DecodeArgs& a, int b, int w0, int nrec, int hq0, int lane) {
    constexpr int LPH = kWave / G;        // lanes per head
    constexpr int NC = D / 4 / LPH;       // 16-byte columns per lane
    constexpr int KR = NC <= 2 ? 16 : 8;  // records per round
    const int h = lane / LPH;
    const int c0 = lane - h * LPH;        // columns c0, c0 + LPH, ...
    const size_t r0 = (static_cast<size_t>(w0) + b) * a.Hq + hq0;
    const unsigned span = static_cast<unsigned>((nrec - 1) * a.Hq + G);
    const buf_rsrc mlr = make_rsrc(a.part_ml + r0 * 2, span * 8u);
    const buf_rsrc accr = make_rsrc(a.part_acc + r0 * D, span * static_cast<unsigned>(D) * 4u);
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    float M = -INFINITY, L = 0.0f;
    f32x4 A[NC];
#pragma unroll
    for (int j = 0; j < NC; j++) A[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = 0; k0 < nrec; k0 += KR) {
        v2i_t ml[KR];
        v4i_t acc[KR][NC];
#pragma unroll
        for (int k = 0; k < KR; k++) {
            if (k0 + k < nrec) {
                const int rec = (k0 + k) * a.Hq + h;
                ml[k] = __builtin_amdgcn_raw_buffer_load_b64(mlr, rec * 8, 0, kCoherent);
#pragma unroll
                for (int j = 0; j < NC; j++)
                    acc[k][j] = __builtin_amdgcn_raw_buffer_load_b128(accr, (rec * D + 4 * (c0 + j * LPH)) * 4, 0,
                                                                      kCoherent);
            }
        }
        float cm = M;
#pragma unroll
        for (int k = 0; k < KR; k++)
            if (k0 + k < nrec) cm = fmaxf(cm, __int_as_float(ml[k].x));
        const float f = fast_exp2(M - cm);  // 0 on the first round (M = -inf); every record is finite
        L *= f;
#pragma unroll
        for (int j = 0; j < NC; j++) A[j] *= f;
        M = cm;
#pragma unroll
        for (int k = 0; k < KR; k++) {
            if (k0 + k < nrec) {
                const float w = fast_exp2(__int_as_float(ml[k].x) - cm);
                L = fmaf(__int_as_float(ml[k].y), w, L);
#pragma unroll
                for (int j = 0; j < NC; j++) A[j] += __builtin_bit_cast(f32x4, acc[k][j]) * w;
            }
        }
    }
    const float rl = 1.0f / L;
    float* o = a.out + (static_cast<size_t>(b) * a.Hq + hq0 + h) * D;
#pragma unroll
    for (int j = 0; j < NC; j++) {
#pragma unroll
        for (int i = 0; i < 4; i++) o[4 * (c0 + j * LPH) + i] = A[j][i] * rl;
    }
}

template <int D, int G, bool PAGED, bool APPEND>
__global__ __launch_bounds__(kMWaves* kWave) __attribute__((amdgpu_waves_per_eu(APPEND ? 1 : 2, APPEND ? 1 : 2))) void decode_mfma_flat(
    const DecodeArgs a) {
    static_assert(G == 4 || G == 8, "heads per workgroup");
    static_assert(D == 64 || D == 128, "head dims of the matrix-core decode kernel");
    constexpr int NJ = D / 64;
    constexpr int NB = D / 16;
    constexpr int RPLV = kWave / NB;
    constexpr int NV = kMTile / RPLV;
    constexpr int NE = 2 * D / kWave;
    __shared__ __align__(16) int8_t s_v[kMWaves][2][kMTile * D];  // V tiles, per wave
    __shared__ __align__(16) int8_t s_newq[kMWaves][2][D];
    __shared__ int s_E[kFlatMaxSeqs + 1];  // big batches: first tile of each sequence, then T
    __shared__ int s_len[kFlatMaxSeqs];    // and its length
    __shared__ int s_wsum[kMWaves];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r = lane & 15;
    const int g = lane >> 4;

    const int U = a.Hkv * a.nsg;
    const int item = blockIdx.x / U;
    const int unit = blockIdx.x - item * U;
    const int kvh = unit / a.nsg;
    const int sgi = unit - kvh * a.nsg;
    const int hq0 = kvh * a.G + sgi * G;
    const int Wn = a.fit_items * kMWaves;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int gw = item * kMWaves + wv;

    // The plan.  A window of 64 sequences lives in lanes: lane j holds
    // sequence wb0 + j's length, tiles and first tile.  Up to 64 sequences
    // the window is the whole batch, scanned in lanes; beyond that the
    // workgroup scans the lengths into LDS (first tiles and lengths of up to
    // kFlatMaxSeqs sequences) and each wave's window starts at its first
    // sequence, moving on when its range runs past 64 sequences.
    const int B = a.B;
    int wb0 = 0, wcount = 0, wend = 0;  // window base, size, and the tile where it ends
    int len_l = 0, n_l = 0, e_l = 0;
    int T = 0;
    const bool big = B > kWave;
    if (!big) {
        len_l = lane < B ? seq_len_of(a, lane) : 0;
        n_l = (len_l + kMTile - 1) / kMTile;
        const int incl = wave_inclusive_scan(n_l);
        e_l = incl - n_l;
        T = __builtin_amdgcn_readlane(incl, kWave - 1);
        wcount = B;
        wend = T;
    } else {
        // Thread t scans sequences [t * per, (t + 1) * per), then the block.
        constexpr int kPer = kFlatMaxSeqs / (kMWaves * kWave);
        const int per = (B + blockDim.x - 1) / blockDim.x;
        const int s0 = threadIdx.x * per;
        int lens[kPer];
        int tot = 0;
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            lens[k] = (k < per && s0 + k < B) ? seq_len_of(a, s0 + k) : 0;
            tot += (lens[k] + kMTile - 1) / kMTile;
        }
        const int incl = wave_inclusive_scan(tot);
        if (lane == kWave - 1) s_wsum[wv] = incl;
        __syncthreads();
        int base = incl - tot;
        for (int w = 0; w < wv; w++) base += s_wsum[w];
        T = 0;
#pragma unroll
        for (int w = 0; w < kMWaves; w++) T += s_wsum[w];
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            if (k < per && s0 + k < B) {
                s_E[s0 + k] = base;
                s_len[s0 + k] = lens[k];
                base += (lens[k] + kMTile - 1) / kMTile;
            }
        }
        if (threadIdx.x == 0) s_E[B] = T;
        __syncthreads();
    }
    // Window at sequence b0 (big batches).
    auto win_load = [&](int b0) {
        wb0 = b0;
        wcount = min(kWave, B - b0);
        const bool in = lane < wcount;
        e_l = in ? s_E[b0 + lane] : T;
        n_l = in ? s_E[b0 + lane + 1] - e_l : 0;
        len_l = in ? s_len[b0 + lane] : 0;
        wend = s_E[b0 + wcount];
    };
    // The sequence holding tile t < T, by two rounds of 64-way search in LDS (big batches).
    auto find_seq = [&](int t) {
        const int step = (B + kWave - 1) / kWave;
        const int i1 = min(B - 1, lane * step);
        const int j1 = static_cast<int>(__builtin_popcountll(__builtin_amdgcn_ballot_w64(s_E[i1] <= t &&
                                                                                       lane * step < B))) - 1;
        const int lo = j1 * step;
        const int i2 = min(B - 1, lo + lane);
        return lo + static_cast<int>(__builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < step && s_E[i2] <= t &&
                                                                                    lo + lane < B))) - 1;
    };
    // The waves split a virtual stream in which every sequence is preceded by
    // kFlatSwitchTiles tiles of no work: sequence b's real tiles E_b + i sit at
    // virtual position E_b + i + kFlatSwitchTiles * (b + 1).  A wave whose
    // range crosses into a sequence gets that many fewer real tiles, which
    // pays for the switch (the next sequence's q, the record of the one it
    // leaves): ~2 us, by per-wave timestamps at cfg2.
    const int P = kFlatSwitchTiles;
    const FlatSplit fs = flat_split(T + P * B, Wn);
    // The real tile at or after virtual position v (T at the end).
    auto real_of = [&](int v) {
        if (v >= T + P * B) return T;
        int b, e, n;
        if (!big) {
            b = static_cast<int>(__builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < B && e_l + P * lane <= v))) - 1;
            e = __builtin_amdgcn_readlane(e_l, b);
            n = __builtin_amdgcn_readlane(n_l, b);
        } else {
            const int step = (B + kWave - 1) / kWave;
            const int i1 = min(B - 1, lane * step);
            const int j1 = static_cast<int>(__builtin_popcountll(
                               __builtin_amdgcn_ballot_w64(s_E[i1] + P * i1 <= v && lane * step < B))) - 1;
            const int lo = j1 * step;
            const int i2 = min(B - 1, lo + lane);
            b = lo + static_cast<int>(__builtin_popcountll(__builtin_amdgcn_ballot_w64(
                         lane < step && s_E[i2] + P * i2 <= v && lo + lane < B))) - 1;
            e = s_E[b];
            n = s_E[b + 1] - e;
        }
        return e + min(max(v - e - P * (b + 1), 0), n);
    };
    // The wave holding real tile t of sequence b.
    auto wave_of = [&](int t, int b) { return flat_wave_of(fs, t + P * (b + 1)); };
    const int tb = real_of(flat_start(fs, gw));
    const int te = real_of(flat_start(fs, gw + 1));
    if (big) win_load(tb < T ? find_seq(tb) : 0);
    // The sequence holding tile t < T; moves the window when t is past it.
    // With kFlatSwitchTiles >= 1 the planner's bound (at most 16 tiles per
    // wave at full length beyond 64 sequences) keeps every range below
    // 16 * (1 + kFlatSwitchTiles) virtual tiles, fewer than 64 sequences
    // need, so the move is a safeguard that no planned launch takes.
    static_assert(kFlatSwitchTiles >= 1, "switch tiles bound the sequences one wave range spans");
    auto seq_of = [&](int t) {
        if (big && t >= wend) win_load(find_seq(t));
        return wb0 + static_cast<int>(__builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < wcount && e_l <= t))) -
               1;
    };
    // Plan entries of sequence b in the window.
    auto plan_e = [&](int b) { return __builtin_amdgcn_readlane(e_l, b - wb0); };
    auto plan_n = [&](int b) { return __builtin_amdgcn_readlane(n_l, b - wb0); };
    auto plan_len = [&](int b) { return __builtin_amdgcn_readlane(len_l, b - wb0); };

    // Zero rows of empty sequences, once per work unit.
    if (item == 0 && wv == 0) {
        for (int c0 = 0; c0 < B; c0 += kWave) {
            const int b = c0 + lane;
            const int len = b < B ? (big ? s_len[b] : len_l) : 1;
            unsigned long long empty = __builtin_amdgcn_ballot_w64(len == 0);
            while (empty) {
                const int be = c0 + __builtin_ctzll(empty);
                empty &= empty - 1;
                for (int i = lane; i < G * D; i += kWave) a.out[(static_cast<size_t>(be) * a.Hq + hq0) * D + i] = 0.0f;
            }
        }
    }

    constexpr bool app = APPEND;  // a.k_new != nullptr
    // q of head (r % G) of sequence b, dims 16g.. of each 64-dim block.
    const int hrow = r % G;
    float qv[16 * NJ];
    auto load_q = [&](int b) {
        const float* qp = a.q + (static_cast<size_t>(b) * a.Hq + hq0 + hrow) * D + 16 * g;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
#pragma unroll
            for (int i4 = 0; i4 < 4; i4++) {
                const float4 x = *reinterpret_cast<const float4*>(qp + 64 * j + 4 * i4);
                qv[16 * j + 4 * i4] = x.x;
                qv[16 * j + 4 * i4 + 1] = x.y;
                qv[16 * j + 4 * i4 + 2] = x.z;
                qv[16 * j + 4 * i4 + 3] = x.w;
            }
        }
    };
    i32x4 qb[NJ][3];
    float qs = 0.0f;
    auto prepare_q = [&]() {
        float qmax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16 * NJ; i++) qmax = fmaxf(qmax, fabsf(qv[i]));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 16));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
        int qexp = 0;
        frexpf(qmax, &qexp);
        const int E = qmax > 0.0f ? min(max(22 - qexp, -100), 126) : 0;
        qs = ldexpf(1.0f, -E) * a.scale_log2;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            int limb[3][16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int Q = static_cast<int>(__builtin_rintf(ldexpf(qv[16 * j + i], E)));
                const int l2 = ((Q + 128) & 255) - 128;
                const int Q1 = (Q - l2) >> 8;
                const int l1 = ((Q1 + 128) & 255) - 128;
                limb[0][i] = (Q1 - l1) >> 8;
                limb[1][i] = l1;
                limb[2][i] = l2;
            }
#pragma unroll
            for (int lb = 0; lb < 3; lb++)
                qb[j][lb] = i32x4{pack_bytes(&limb[lb][0]), pack_bytes(&limb[lb][4]), pack_bytes(&limb[lb][8]),
                                  pack_bytes(&limb[lb][12])};
        }
    };

    float m = -INFINITY, lsum = 0.0f, vref = 0.0f;
    f32x4 acc[NB];
#pragma unroll
    for (int c = 0; c < NB; c++) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const bool lo_row = ((r / G) & 1) != 0;
    const int rr = (lane & 15) >> 1;
    const int h2 = lane & 1;
    const int vrow = rr < 4 ? 4 * g + rr : 16 + 4 * g + (rr - 4);
    const unsigned cap = static_cast<unsigned>(a.cap);

    struct Tile {
        i32x4 ka[2][NJ];
        int4 v[NV];
        float ks[2][4], vs[2][4];
    };
    const int kvo = r * D + 16 * g;
    const int vvo = (lane / NB) * D + 16 * (lane % NB);
    const int svo = 16 * g;
    // Tile loads of sequence b at token `base` (a multiple of 32).  `none`:
    // past the wave's range -- the same loads through empty resources (they
    // read zeros and touch no memory), so that every iteration issues the
    // same loads and the waits for the current tile can leave the next one in
    // flight.
    // The load cursor's sequence as buffer resources (contiguous layout;
    // rebuilt only when the cursor moves to another sequence).
    buf_rsrc lkr, lvr, lksr, lvsr;
    auto set_load_seq = [&](int b) {
        if constexpr (!PAGED) {
            const size_t row0 = (static_cast<size_t>(b) * a.Hkv + kvh) * a.cap;
            lkr = make_rsrc(a.k + row0 * D, cap * D);
            lvr = make_rsrc(a.v + row0 * D, cap * D);
            lksr = make_rsrc(a.ks + row0, cap * 4u);
            lvsr = make_rsrc(a.vs + row0, cap * 4u);
        }
    };
    // Paged: the page id of the cursor's next tile in the same sequence is
    // fetched with each tile's loads (a vector load issued before them, so
    // waiting for it leaves them in flight) and used when that tile loads; a
    // move to another sequence looks its first page up at once.  Page sizes
    // are powers of two here; indices past a row are clamped into it.
    int pf_b = -1, pf_base = 0, pf_page = 0;
    auto table_load = [&](int b, int base) {
        const buf_rsrc tabr = make_rsrc(a.pages.table + static_cast<size_t>(b) * a.pages.max_pages,
                                        static_cast<unsigned>(a.pages.max_pages) * 4u);
        return __builtin_amdgcn_raw_buffer_load_b32(tabr, min(base >> a.pages.shift, a.pages.max_pages - 1) * 4, 0, 0);
    };
    auto load_tile = [&](Tile& Tt, int b, int base, bool none) {
        buf_rsrc kr, vr, ksr, vsr;
        int ko, so;
        if (none) {
            kr = vr = ksr = vsr = make_rsrc(a.k, 0u);
            ko = so = 0;
        } else if constexpr (PAGED) {
            int id = pf_page;
            if (b != pf_b || base != pf_base) id = table_load(b, base);
            const int page = min(max(__builtin_amdgcn_readfirstlane(id), 0), a.pages.num_pages - 1);
            pf_b = b;
            pf_base = base + kMTile;
            pf_page = table_load(b, pf_base);
            const size_t rp = (static_cast<size_t>(page) * a.Hkv + kvh) * a.pages.size + (base & (a.pages.size - 1));
            const unsigned rem = static_cast<unsigned>(a.pages.size - (base & (a.pages.size - 1)));
            kr = make_rsrc(a.k + rp * D, rem * D);
            vr = make_rsrc(a.v + rp * D, rem * D);
            ksr = make_rsrc(a.ks + rp, rem * 4u);
            vsr = make_rsrc(a.vs + rp, rem * 4u);
            ko = so = 0;
        } else {
            kr = lkr;
            vr = lvr;
            ksr = lksr;
            vsr = lvsr;
            ko = base * D;
            so = base * 4;
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
#pragma unroll
            for (int j = 0; j < NJ; j++) Tt.ka[s][j] = buffer_load16_stream(kr, kvo + s * 16 * D + 64 * j, ko);
        }
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const v4i_t x = buffer_load16_stream(vr, vvo + c * RPLV * D, ko);
            Tt.v[c] = make_int4(x.x, x.y, x.z, x.w);
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const v4i_t xk = buffer_load16(ksr, svo + 64 * s, so);
            const v4i_t xv = buffer_load16(vsr, svo + 64 * s, so);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                Tt.ks[s][i] = __int_as_float(xk[i]);
                Tt.vs[s][i] = __int_as_float(xv[i]);
            }
        }
    };
    auto stage_v = [&](const Tile& Tt, int8_t* vt) {
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const int rw = RPLV * c + lane / NB;
            const int p = lane % NB;
            *reinterpret_cast<int4*>(vt + rw * D + (v_slot<D>(p, rw) << 4)) = Tt.v[c];
        }
    };

    // Fused append of sequence b's token len-1 (its last tile is in this
    // wave's range): the fp32 rows are loaded one tile ahead, quantised with
    // the rule and bits of append_kernel, written to the cache once per kv head
    // and substituted into the tile.
    // Two banks: the next sequence's row may be loaded in the step that
    // appends the current one (a one-tile sequence after a sequence end).
    float xnew0[NE], xnew1[NE];
    int x_issue = 0, x_use = 0;  // rows loaded / appended so far (bank = count & 1)
    float newks = 0.0f, newvs = 0.0f;
    auto load_new = [&](int b) {
        const size_t bh = static_cast<size_t>(b) * a.Hkv + kvh;
        if (x_issue & 1) {
#pragma unroll
            for (int j = 0; j < NE; j++)
                xnew1[j] = (j < NJ ? a.k_new : a.v_new)[bh * D + ((lane + kWave * j) & (D - 1))];
        } else {
#pragma unroll
            for (int j = 0; j < NE; j++)
                xnew0[j] = (j < NJ ? a.k_new : a.v_new)[bh * D + ((lane + kWave * j) & (D - 1))];
        }
        x_issue++;
    };
    auto append_new = [&](int b, int tnew) {
        float xnew[NE];
#pragma unroll
        for (int j = 0; j < NE; j++) xnew[j] = (x_use & 1) ? xnew1[j] : xnew0[j];
        x_use++;
        const size_t rnew = cache_row(a.pages, a.Hkv, a.cap, b, kvh, tnew);
        float amk = fabsf(xnew[0]), amv = fabsf(xnew[NJ]);
#pragma unroll
        for (int j = 1; j < NJ; j++) {
            amk = fmaxf(amk, fabsf(xnew[j]));
            amv = fmaxf(amv, fabsf(xnew[NJ + j]));
        }
        newks = quant_scale(wave_max(amk));
        newvs = quant_scale(wave_max(amv));
#pragma unroll
        for (int j = 0; j < NE; j++)
            s_newq[wv][j / NJ][lane + kWave * (j % NJ)] =
                static_cast<int8_t>(quant_one(xnew[j], j < NJ ? newks : newvs));
        if (sgi == 0) {
            if (lane < 2 * NB) {
                const int row = lane / NB, piece = lane % NB;
                *reinterpret_cast<int4*>((row ? a.v : a.k) + rnew * D + 16 * piece) =
                    *reinterpret_cast<const int4*>(&s_newq[wv][row][16 * piece]);
            }
            if (lane == 0) {
                a.ks[rnew] = newks;
                a.vs[rnew] = newvs;
            }
        }
    };
    auto substitute_new = [&](Tile& Tt, int base, int tnew, int8_t* vt) {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            if (base + 16 * s + r == tnew) {
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    Tt.ka[s][j] = *reinterpret_cast<const i32x4*>(&s_newq[wv][0][64 * j + 16 * g]);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (base + 16 * s + 4 * g + i == tnew) {
                    Tt.ks[s][i] = newks;
                    Tt.vs[s][i] = newvs;
                }
        }
        const int rw = tnew - base;
        if (rw >= 0 && rw < kMTile && lane < NB)
            *reinterpret_cast<int4*>(vt + rw * D + (v_slot<D>(lane, rw) << 4)) =
                *reinterpret_cast<const int4*>(&s_newq[wv][1][16 * lane]);
    };

    // One tile of the current sequence (tokens [base, base + 32) of len).
    auto compute = [&](const Tile& Tt, int base, int len, const int8_t* vt) {
        i32x4 cq[2][3];
#pragma unroll
        for (int s = 0; s < 2; s++) {
#pragma unroll
            for (int lb = 0; lb < 3; lb++) {
                i32x4 c = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < NJ; j++) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(Tt.ka[s][j], qb[j][lb], c, 0, 0, 0);
                cq[s][lb] = c;
            }
        }
        float sc[8], vsv[8];
        float mt = -INFINITY, vmax = 0.0f;
#pragma unroll
        for (int s = 0; s < 2; s++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int low = (cq[s][1][i] << 8) + cq[s][2][i];
                const float dot = static_cast<float>(cq[s][0][i]) * 65536.0f + static_cast<float>(low);
                sc[4 * s + i] = (dot * Tt.ks[s][i]) * qs;
                vsv[4 * s + i] = Tt.vs[s][i];
            }
        }
        if (base + kMTile > len) {
#pragma unroll
            for (int s = 0; s < 2; s++) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (base + 16 * s + 4 * g + i >= len) {
                        sc[4 * s + i] = -INFINITY;
                        vsv[4 * s + i] = 0.0f;
                    }
            }
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            mt = fmaxf(mt, sc[k]);
            vmax = fmaxf(vmax, fabsf(vsv[k]));
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        vmax = fmaxf(vmax, __shfl_xor(vmax, 16));
        vmax = fmaxf(vmax, __shfl_xor(vmax, 32));
        const float mn = fmaxf(m, mt);
        const float ms = mn == -INFINITY ? 0.0f : mn;
        const float alpha = fast_exp2(m - ms);
        const float vn = fmaxf(vref, vmax);
        const float rvn = vn > 0.0f ? __builtin_amdgcn_rcpf(vn) : 0.0f;
        const float f = vn > 0.0f ? alpha * (vref * rvn) : alpha;
        const float winv = kPScale * rvn;
        m = mn;
        vref = vn;
        if (__builtin_amdgcn_ballot_w64(f != 1.0f) != 0) {
#pragma unroll
            for (int c = 0; c < NB; c++) acc[c] *= f;
        }
        float ps = 0.0f;
        f16x8 pb;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float p = fast_exp2(sc[k] - ms);
            ps += p;
            const float w = p * (vsv[k] * winv);
            const _Float16 hi = static_cast<_Float16>(w);
            const _Float16 lo = static_cast<_Float16>(w - static_cast<float>(hi));
            pb[k] = lo_row ? lo : hi;
        }
        lsum = lsum * alpha + ps;
#pragma unroll
        for (int c = 0; c < NB; c++) {
            const int8_t* src = vt + vrow * D + (v_slot<D>(c, vrow) << 4) + 8 * h2;
            const i32x2 vb = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(const_cast<int8_t*>(src)));
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(i8x8_to_f16(vb), pb, acc[c], 0, 0, 0);
        }
    };

    // A finished segment of sequence b from registers (no LDS, no barrier):
    // the output when it covers the whole sequence, else record gw + b.
    auto emit_segment = [&](int b, bool complete) {
        float lt = lsum;
        lt += __shfl_xor(lt, 16);
        lt += __shfl_xor(lt, 32);
        const float fct = vref * (1.0f / kPScale);
        const bool writer = r < G;
        const size_t row = static_cast<size_t>(b) * a.Hq + hq0 + r;
        const size_t rec = (static_cast<size_t>(gw) + b) * a.Hq + hq0 + r;
        const float sc = complete ? fct / lt : fct;
        const buf_rsrc recr = make_rsrc(a.part_acc + (static_cast<size_t>(gw) + b) * a.Hq * D, a.Hq * D * 4u);
#pragma unroll
        for (int c = 0; c < NB; c++) {
            f32x4 o;
            // Row r < G (hi part) adds row r + G (lo part): a DPP row shift left by G.
#pragma unroll
            for (int i = 0; i < 4; i++)
                o[i] = (acc[c][i] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(acc[c][i]),
                                                                                 0x100 + G, 0xF, 0xF, false))) * sc;
            if (writer) {
                if (complete) {
#pragma unroll
                    for (int i = 0; i < 4; i++) a.out[row * D + 16 * c + 4 * g + i] = o[i];
                } else {
                    // Device-coherent 16-byte store (sc1), as put_coherent.
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i_t, o), recr,
                                                           ((hq0 + r) * D + 16 * c + 4 * g) * 4, 0, kCoherent);
                }
            }
        }
        if (!complete && writer && g == 0) {
            put_coherent(a.part_ml + rec * 2, m);
            put_coherent(a.part_ml + rec * 2 + 1, lt);
        }
    };
    auto reset_state = [&]() {
        m = -INFINITY;
        lsum = 0.0f;
        vref = 0.0f;
#pragma unroll
        for (int c = 0; c < NB; c++) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };

    // One wave's arrival for sequence b, in two halves so that the wave does
    // not wait for the atomic's return: arrive_issue (lane 0; after the
    // wave's record stores have completed) bumps the counter and keeps the
    // count it reached; arrive_resolve, after the tile loop, returns b when
    // that count completes the number of waves covering b -- this wave then
    // owns b's merge, and puts the counter back to 0 for the next launch.
    auto arrive_issue = [&](int b) {
        int reached = 0;
        if (lane == 0) {
            int* ctr = a.counters + static_cast<size_t>(b) * U + unit;
            reached = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
        }
        return reached;
    };
    auto arrive_resolve = [&](int b, int bE, int bn, int reached) {
        int done = -1;
        if (lane == 0) {
            const int cover = wave_of(bE + bn - 1, b) - wave_of(bE, b) + 1;
            if (reached == cover) {
                __hip_atomic_store(a.counters + static_cast<size_t>(b) * U + unit, 0, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                done = b;
            }
        }
        return __builtin_amdgcn_readfirstlane(__shfl(done, 0));
    };

    // Compute cursor (sequence of the tile being computed) and load cursor
    // (sequence of the tile being loaded, one ahead); wave-uniform.
    int pend = -1, pend_e = 0, pend_n = 0;  // this wave's partial first-segment record, not yet counted
    bool pend_aged = false;                 // ... written at least one tile ago
    int pm = -1, pm_e = 0, pm_n = 0, pm_reached = 0;  // that record's arrival, issued mid-range
    int cb = -1, cE = 0, cn = 0, clen = 0;
    int from = tb;  // first tile of the current segment
    const int ntiles = te - tb;
    if (ntiles > 0) {
        cb = seq_of(tb);
        cE = plan_e(cb);
        cn = plan_n(cb);
        clen = plan_len(cb);
        int lb = cb, lE = cE, ln = cn;  // load cursor
        Tile ta, tb_;
        set_load_seq(cb);
        load_tile(ta, cb, (tb - cE) * kMTile, false);
        load_q(cb);
        if (app && tb == cE + cn - 1) load_new(cb);
        prepare_q();
        stage_v(ta, s_v[wv][0]);
        // One iteration: tile it (in Tc, LDS buffer it & 1) is computed while
        // tile it + 1 loads into Tn.
        auto step = [&](Tile& Tc, Tile& Tn, int it) {
            const int t = tb + it;
            const bool more = it + 1 < ntiles;
            // Tile t ends its sequence; the next tile starts the next non-empty one.
            const bool switched = more && t + 1 == lE + ln;
            if (switched) {
                lb = seq_of(t + 1);
                lE = plan_e(lb);
                ln = plan_n(lb);
                set_load_seq(lb);
            }
            load_tile(Tn, lb, (t + 1 - lE) * kMTile, !more);
            if constexpr (PAGED) {
                // Tile t + 2 starts the next sequence: its first page instead.
                // Looked up without moving the window, which must keep the
                // compute cursor's sequence for its length below.
                if (more && t + 2 < te && t + 2 == lE + ln) {
                    pf_b = (big && t + 2 >= wend) ? find_seq(t + 2) : seq_of(t + 2);
                    pf_base = 0;
                    pf_page = table_load(pf_b, 0);
                }
            }
            if (switched) load_q(lb);
            if (app && more && t + 1 == lE + ln - 1) load_new(lb);
            int8_t* vt = s_v[wv][it & 1];
            const int base = (t - cE) * kMTile;
            if (app && t == cE + cn - 1) {
                append_new(cb, clen - 1);
                substitute_new(Tc, base, clen - 1, vt);
            }
            compute(Tc, base, clen, vt);
            if (more && t == cE + cn - 1) {
                // The segment ends inside the range: a middle segment is a
                // whole sequence, the first one may be a sequence's tail.
                // The next sequence's q limbs come first: their loads went out
                // with the next tile's, so that wait covers loads only.  After
                // the segment's stores it would also wait for them to complete
                // (the compiler cannot count loads past pending stores), which
                // cost each switching wave ~2 us.
                const bool complete = from == cE;
                prepare_q();
                emit_segment(cb, complete);
                if (!complete) pend = cb, pend_e = cE, pend_n = cn;
                cb = lb;
                cE = lE;
                cn = ln;
                clen = plan_len(cb);
                from = t + 1;
                reset_state();
            }
            if (more) stage_v(Tn, s_v[wv][(it + 1) & 1]);
            if (pend >= 0) {
                // Count the tail record one tile after it was written: by then
                // its stores have completed and the wait below only covers
                // loads the tile just staged has drained, so the tile pipeline
                // does not stall (counting it at once cost such a wave ~3 us).
                if (pend_aged) {
                    __builtin_amdgcn_s_waitcnt(0);
                    pm_reached = arrive_issue(pend);
                    pm = pend;
                    pm_e = pend_e;
                    pm_n = pend_n;
                    pend = -1;
                } else {
                    pend_aged = true;
                }
            }
        };
        int it = 0;
        for (; it + 1 < ntiles; it += 2) {
            step(ta, tb_, it);
            step(tb_, ta, it + 1);
        }
        if (it < ntiles) step(ta, tb_, it);
    }

    // The last segment: output or record straight from registers, then its
    // arrival (one wave), and the merge of any sequence whose count this wave
    // completed (here, or mid-range for its first-segment tail).  No LDS and
    // no barrier: waves finish independently.
    if (ntiles == 0) return;
    const bool last_done = from == cE && te == cE + cn;
    emit_segment(cb, last_done);
    if (!last_done || pend >= 0) __builtin_amdgcn_s_waitcnt(0);  // this wave's record stores have completed
    if (pend >= 0) {  // a tail record written at the range's second-to-last tile
        pm_reached = arrive_issue(pend);
        pm = pend;
        pm_e = pend_e;
        pm_n = pend_n;
    }
    const int last_reached = last_done ? 0 : arrive_issue(cb);
    if (pm >= 0) pm = arrive_resolve(pm, pm_e, pm_n, pm_reached);
    const int done1 = last_done ? -1 : arrive_resolve(cb, cE, cn, last_reached);
    if (pm < 0 && done1 < 0) return;
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int b = k == 0 ? pm : done1;
        if (b < 0) continue;
        const int bE = k == 0 ? pm_e : cE;
        const int bn = k == 0 ? pm_n : cn;
        const int w0 = wave_of(bE, b);
        const int w1 = wave_of(bE + bn - 1, b);
        merge_wave_records<D, G>(a, b, w0, w1 - w0 + 1, hq0, lane);
    }
}

}  // namespace

int mfma_tile_tokens() { return kMBStep; }

int mfma_heads_per_group(int G, int d) {
    if (d != 64 && d != 128) return 0;
    if (G % 8 == 0) return 8;
    if (G % 4 == 0) return 4;
    return 0;
}

namespace {
template <int D, int G>
void launch_mfma_dg(const DecodeArgs& a, dim3 grid, dim3 block, hipStream_t stream) {
    const bool paged = a.pages.table != nullptr;
    if (a.flat) {
        const bool app = a.k_new != nullptr;
        if (paged && app) hipLaunchKernelGGL((decode_mfma_flat<D, G, true, true>), grid, block, 0, stream, a);
        else if (paged) hipLaunchKernelGGL((decode_mfma_flat<D, G, true, false>), grid, block, 0, stream, a);
        else if (app) hipLaunchKernelGGL((decode_mfma_flat<D, G, false, true>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((decode_mfma_flat<D, G, false, false>), grid, block, 0, stream, a);
    } else if (a.fit_items > 0) {
        if (paged) hipLaunchKernelGGL((decode_mfma<D, G, true, true>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((decode_mfma<D, G, false, true>), grid, block, 0, stream, a);
    } else {
        if (paged) hipLaunchKernelGGL((decode_mfma<D, G, true, false>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((decode_mfma<D, G, false, false>), grid, block, 0, stream, a);
    }
}
}  // namespace

hipError_t launch_decode_mfma(const DecodeArgs& a, const DecodePlan& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(decode_grid(a, p)));
    const dim3 block(kMWaves * kWave);
    if (a.d == 128 && p.sg == 4) launch_mfma_dg<128, 4>(a, grid, block, stream);
    else if (a.d == 128 && p.sg == 8) launch_mfma_dg<128, 8>(a, grid, block, stream);
    else if (a.d == 64 && p.sg == 4) launch_mfma_dg<64, 4>(a, grid, block, stream);
    else if (a.d == 64 && p.sg == 8) launch_mfma_dg<64, 8>(a, grid, block, stream);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace kvq
