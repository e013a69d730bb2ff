// Ragged MoE prefill on gfx950: the layer of QwenCPUModel.moeForward
// (QwenCPUModel.swift:500-569) applied to S tokens at once.  The (token,
// expert) pairs are grouped by expert, so each expert's weights are read once
// per tile of up to 64 of its tokens and contracted on the bf16 matrix cores.
// The grouping follows mlx's _gather_sort / gather_qmm / _scatter_unsort
// (switch_layers.py:12-24, 75-90, 176-199); the arithmetic follows the CPU
// path, which loops the same per-token computation (QwenCPUModel.swift:544-567).
//
// Launches, all on the caller's stream:
//   1. router GEMM: partial logits [slice][T, E], 16-token tiles x K slices
//      of 4 groups; its first column block also writes x in the layout
//      gate/up reads (bf16 planes) and the group sums of x;
//   2. route: softmax, top-k (ties to the lower id), renormalisation and
//      the shared-expert gate logit per token;
//   2b. group: one workgroup of 1024 threads counts the pairs per expert and
//      builds the sorted pair order and the table of 64-row tiles (routed
//      experts, then the shared expert over all tokens);
//   3. gate/up GEMM over the tile table with the SwiGLU epilogue: h in
//      sorted pair order, as bf16 hi + lo planes;
//   4. down GEMM over the same tiles: y rows (f32) in sorted pair order;
//   5. combine: out[t] = sum_k w_tk y[pos(t,k)] in pick order, then
//      + sigmoid(sg_t) y_shared[t] (QwenCPUModel.swift:556, :566).
//
// Quantised contraction on the matrix cores.  For output n, input group g
// (64 inputs) and activation row m, with w = s*q + b:
//   y[m,n] = sum_g s[n,g] * C_g[m,n] + sum_g b'[n,g] * X_g[m]
//   C_g[m,n] = sum_{i in g} c_i * a[m,i],   X_g[m] = sum_{i in g} a[m,i]
// where c = 16 + q, b' = b - 16 s for 4-bit codes (the bf16 bit pattern
// 0x4180 | q << 3 is 16 + q, built two codes per shift and and-or; the small
// offset keeps the cancellation between the two terms to a few bits), and
// c = q, b' = b for 8-bit codes.  The codes are exact in bf16; activations are bf16 (exact)
// or split into bf16 hi + lo (fp32 inputs, the SwiGLU output), one MFMA per
// part.  Every product is exact and accumulates in fp32, the scale applies
// per group in fp32, and the bias term is one more MFMA chain over the group
// axis with both factors split hi + lo.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/swq_bench.h"
#include "moe_host.hpp"
#include "route.hpp"

namespace swq {
namespace {

constexpr int kPfThreads = 256;  // 4 waves
constexpr int kGroupK = 64;      // the quantisation group: one MFMA pair of k = 32
constexpr int kLdsPitch = 72;    // bf16 per staged row: 64 + 8 (144 B rows, conflict-free b128 reads)
constexpr int kMaxGroups = 64;   // inputs per row <= 4096
constexpr int kXsPitch = kMaxGroups + 36;  // a K slice's bias term reads up to 31 groups past its first
constexpr int kTileRows = 64;    // rows of a routed / shared tile
constexpr int kRouterRows = 16;  // rows of a router tile
constexpr int kRouteWaves = 1;   // tokens per route workgroup, one wave each (512 workgroups at 512 tokens)
constexpr int kXcds = 8;         // XCDs of the device: workgroup b runs on XCD b % 8

// Workgroups covering `tiles` tiles of `nblk` column blocks under the XCD
// mapping of pf_gemm (tiles rounded up to a multiple of 8).
int gemm_blocks(int tiles, int nblk) { return ((tiles + kXcds - 1) / kXcds) * kXcds * nblk; }

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4_t;

enum { kSrcBF16 = 0, kSrcF32 = 1, kSrcSplit = 2 };
enum { kEpiRows = 0, kEpiSwiGLU = 1 };
enum { kSumStage = 0, kSumLoad = 1 };  // group sums: computed while staging / read from xs_in

struct Tile {
    int32_t expert;  // 0..E-1, or E for the shared expert
    int32_t row0;    // first row in sorted pair order
    int32_t rows;    // 1..64
    int32_t pad;
};

struct GemmArgs {
    QMat m[2];                // routed matrices of B operands 0 and 1 (stacked over experts)
    QMat sh[2];               // shared-expert matrices (tiles with expert == E)
    const void *a0;           // activation rows: x, or the h hi plane
    const void *a1;           // the h lo plane
    const int32_t *row_src;   // tile row -> activation row; null: the tile row itself
    const Tile *tiles;        // null: dense tiles of 16*MT rows over rows_total
    const int32_t *n_tiles;
    void *o0, *o1;            // outputs: rows (f32), or h hi / lo planes (bf16)
    int64_t a_ld, o_ld;       // elements per activation / output row
    int32_t K, Ksh;           // inputs of the routed / shared matrices
    int32_t N, Nsh;           // outputs of the routed / shared matrices
    int32_t E;                // tiles with this expert id use `sh` (-1: none)
    int32_t rows_total;       // dense tiles: rows; table tiles: rows of the sorted order
    int32_t a_rows;           // rows of the activation source
    int32_t nblk;             // column blocks per tile
    int32_t col_block, col_wave, col_op;  // output column of block / wave / operand steps
    // Group sums X_g of the activation rows, [rows][xs_ld] f32.  The router
    // computes those of x while staging it and writes them (xs_out, by
    // token); gate/up reads them by token and writes those of h (by sorted
    // row, one group per 64-column block); down reads those.
    const float *xs_in;
    float *xs_out;
    int32_t xs_ld, xs_ld_out;
    int32_t o_perm;           // SwiGLU output in nibble_order within each 8 columns (4-bit down)
    int32_t max_tiles;        // entries of the tile table
    // pf_gemm: K split over blockIdx.y into kslices slices of kgroups groups
    // (the last may be shorter); rows outputs of slice s at o0 + s * o_slice
    int32_t kslices, kgroups;
    int64_t o_slice;
    // pf_gemm (the router, first column block): x as the bf16 planes gate/up
    // reads ([rows][a_ld]: hi, and lo for f32 x; in nibble_order within each
    // 8 for 4-bit gate/up codes), or null
    uint16_t *pl0, *pl1;
    int32_t pl_perm;
};

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x4_t mfma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Scales and biases of dtype ST (SWQ_F32 / SWQ_F16 / SWQ_BF16), fixed per
// kernel instance so that the K loop has no branches: a branch around a
// load or its use makes the compiler wait for every load in flight.
template <int ST>
__device__ __forceinline__ float scale_of(uint32_t raw) {
    if constexpr (ST == SWQ_F16) return f16_to_f32(static_cast<uint16_t>(raw));
    else if constexpr (ST == SWQ_BF16) return bf16_to_f32(static_cast<uint16_t>(raw));
    else return __uint_as_float(raw);
}

template <int ST>
__device__ __forceinline__ uint32_t scale_raw(const uint8_t *base, int64_t idx) {
    if constexpr (ST == SWQ_F32) return *reinterpret_cast<const uint32_t *>(base + idx * 4);
    else return *reinterpret_cast<const uint16_t *>(base + idx * 2);
}

// Eight natural-order bf16 (pairs d0 = {x0,x1} .. d3 = {x6,x7}) reordered to
// {x0,x4},{x1,x5},{x2,x6},{x3,x7}: the order in which a 4-bit code word
// yields its codes two at a time (nibbles j and j+4 of `v >> 4j`).  One
// v_perm_b32 per pair: selector bytes 0-3 pick from the second operand,
// 4-7 from the first.
__device__ __forceinline__ u32x4_t nibble_order(u32x4_t d) {
    u32x4_t o;
    o[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);
    o[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);
    o[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);
    o[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);
    return o;
}

// 8 codes of one 4-bit word as bf16 (16 + q: the code in the top four
// mantissa bits of 16.0), in nibble_order.
__device__ __forceinline__ u32x4_t codes_q4(uint32_t w) {
    u32x4_t o;
    o[0] = and_or(w << 3, 0x00780078u, 0x41804180u);
    o[1] = and_or(w >> 1, 0x00780078u, 0x41804180u);
    o[2] = and_or(w >> 5, 0x00780078u, 0x41804180u);
    o[3] = and_or(w >> 9, 0x00780078u, 0x41804180u);
    return o;
}

// Two bytes of an 8-bit word as a bf16 pair (exact: q < 256 has 8 bits).
__device__ __forceinline__ uint32_t byte_pair_bf16(uint32_t w, int b0) {
    const float f0 = static_cast<float>((w >> (8 * b0)) & 0xFFu);
    const float f1 = static_cast<float>((w >> (8 * b0 + 8)) & 0xFFu);
    return (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
}

// 8 codes of two 8-bit words as bf16, natural order.
__device__ __forceinline__ u32x4_t codes_q8(uint32_t w0, uint32_t w1) {
    u32x4_t o;
    o[0] = byte_pair_bf16(w0, 0);
    o[1] = byte_pair_bf16(w0, 2);
    o[2] = byte_pair_bf16(w1, 0);
    o[3] = byte_pair_bf16(w1, 2);
    return o;
}

__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// Eight fp32 values as bf16 hi and lo pairs (natural order).
__device__ __forceinline__ void split8(const float (&v)[8], u32x4_t &hi, u32x4_t &lo) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t h, l;
        split_pair(v[2 * i], v[2 * i + 1], h, l);
        hi[i] = h;
        lo[i] = l;
    }
}

// Eight fp32 values as three bf16 parts hi + mid + lo (24 significant bits):
// the group sums of the bias term, which cancels against the scaled codes.
__device__ __forceinline__ void split8x3(const float (&v)[8], u32x4_t &hi, u32x4_t &mid, u32x4_t &lo) {
    float r[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t h, m;
        split_pair(v[2 * i], v[2 * i + 1], h, m);
        hi[i] = h;
        r[2 * i] = v[2 * i] - bf16_lo(h);
        r[2 * i + 1] = v[2 * i + 1] - bf16_hi(h);
    }
    split8(r, mid, lo);
}

// ---------------------------------------------------------------------------
// the grouped quantised GEMM

// One staged group (64 inputs) of this thread's pieces: piece p = tid + 256 i
// is row p / 8, inputs 8 (p % 8) .. +7 of the group.
template <int SRC, int PPT>
struct AStage {
    u32x4_t v[PPT][SRC == kSrcBF16 ? 1 : 2];
};

template <int BITS>
struct BSlot {
    uint32_t w[2][BITS == 4 ? 2 : 4];  // operand j: the lane's code words of the group
    uint32_t s[2];                     // operand j: the raw scale of (row, group)
};

// Eight consecutive group sums of one activation row, zeros past NG (the
// row holds at least g + 8 entries; g is a multiple of 4).
__device__ __forceinline__ void load_sums8(const float *row, int g, int NG, float (&v)[8]) {
    const float4 x0 = *reinterpret_cast<const float4 *>(row + g);
    const float4 x1 = *reinterpret_cast<const float4 *>(row + g + 4);
    const float t[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = g + i < NG ? t[i] : 0.f;
}

// Raw biases (and 4-bit: scales) of one 32-group block of the bias term:
// this lane's groups g0 + 8 kg .. +7 of both operands.
template <int ST>
struct BiasRaw {
    uint32_t b[2][8], s[2][8];
};

// The bias term sum_g b'[n,g] X_g[m] over the block's groups below ge, on the
// group axis, added to acc.  b' is exact as bf16 hi + lo (an fp16 bias less
// 16 fp16 scales); X_g as hi + mid + lo; the five products above 2^-24
// relative are accumulated.  xrow[mt]: the group sums of this lane's A row
// (16 mt + n); entries up to g0 + 31 are readable.
template <int BITS, int ST, int MT>
__device__ __forceinline__ void bias_apply(f32x4_t (&acc)[MT][2], const BiasRaw<ST> &r,
                                           const float *const (&xrow)[MT], int g0, int ge, int rows, int kg) {
    float xv[MT][8];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) load_sums8(xrow[mt], g0 + 8 * kg, ge, xv[mt]);
    u32x4_t bh[2], bl[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float bp = scale_of<ST>(r.b[j][i]);
            if constexpr (BITS == 4) bp = fmaf(-16.f, scale_of<ST>(r.s[j][i]), bp);
            v[i] = g0 + 8 * kg + i < ge ? bp : 0.f;
        }
        split8(v, bh[j], bl[j]);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if (16 * mt >= rows) break;
        u32x4_t xh, xm, xl;
        split8x3(xv[mt], xh, xm, xl);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[mt][j] = mfma(xl, bh[j], acc[mt][j]);
            acc[mt][j] = mfma(xm, bl[j], acc[mt][j]);
            acc[mt][j] = mfma(xm, bh[j], acc[mt][j]);
            acc[mt][j] = mfma(xh, bl[j], acc[mt][j]);
            acc[mt][j] = mfma(xh, bh[j], acc[mt][j]);
        }
    }
}

// Biases and scales of the bias term (one 32-group block: rows of at most
// 2048 inputs): this lane's groups 8 kg .. +7 of both operands, raw (fp16 or
// bf16 in pairs, or f32), loaded before the K loop so they arrive during it.
template <int ST>
struct BiasBS {
    uint32_t b[2][ST == SWQ_F32 ? 8 : 4];
    uint32_t s[2][ST == SWQ_F32 ? 8 : 4];
};

template <int ST>
__device__ __forceinline__ void load_bias_bs(BiasBS<ST> &bi, const uint8_t *const (&sbase)[2],
                                             const uint8_t *const (&bbase)[2], const int64_t (&srow)[2], int NG,
                                             int kg) {
    constexpr int W = ST == SWQ_F32 ? 8 : 4;
    constexpr int EB = ST == SWQ_F32 ? 4 : 2;
    // scale words first: the K loop reads them (see the register pass after
    // the first ring wait), the bias words only after it
    auto gi = [&](int i) {
        // group index of the word, clamped into the row (rows hold an even number of groups)
        return min(8 * kg + (ST == SWQ_F32 ? i : 2 * i), NG - (ST == SWQ_F32 ? 1 : 2));
    };
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < W; ++i) bi.s[j][i] = *reinterpret_cast<const uint32_t *>(sbase[j] + (srow[j] + gi(i)) * EB);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < W; ++i) bi.b[j][i] = *reinterpret_cast<const uint32_t *>(bbase[j] + (srow[j] + gi(i)) * EB);
}

// bias_term from preloaded biases/scales and the lane's group sums xv[mt]
// (NG <= 32).
template <int BITS, int ST, int MT>
__device__ __forceinline__ void bias_term_bs(f32x4_t (&acc)[MT][2], const BiasBS<ST> &bi, const float (&xv)[MT][8],
                                             int NG, int rows, int kg) {
    u32x4_t bh[2], bl[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t rb, rs;
            if constexpr (ST == SWQ_F32) {
                rb = bi.b[j][i];
                rs = bi.s[j][i];
            } else {
                rb = (i & 1) ? bi.b[j][i >> 1] >> 16 : bi.b[j][i >> 1] & 0xFFFFu;
                rs = (i & 1) ? bi.s[j][i >> 1] >> 16 : bi.s[j][i >> 1] & 0xFFFFu;
            }
            float bp = scale_of<ST>(rb);
            if constexpr (BITS == 4) bp = fmaf(-16.f, scale_of<ST>(rs), bp);
            v[i] = 8 * kg + i < NG ? bp : 0.f;
        }
        split8(v, bh[j], bl[j]);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        if (16 * mt >= rows) break;
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 8 * kg + i < NG ? xv[mt][i] : 0.f;
        u32x4_t xh, xm, xl;
        split8x3(x, xh, xm, xl);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[mt][j] = mfma(xl, bh[j], acc[mt][j]);
            acc[mt][j] = mfma(xm, bl[j], acc[mt][j]);
            acc[mt][j] = mfma(xm, bh[j], acc[mt][j]);
            acc[mt][j] = mfma(xh, bl[j], acc[mt][j]);
            acc[mt][j] = mfma(xh, bh[j], acc[mt][j]);
        }
    }
}

// The 2-byte scales of group g (g < NG <= 32) for this lane's columns of
// both operands, from the words load_bias_bs preloaded: lane (n, kg) holds
// groups 8 kg .. 8 kg + 7, so they come from lane (n, g / 8), both operands'
// halves packed into one ds_bpermute.  g is wave-uniform; the word index is
// picked by selects (no register indexing).
template <int ST>
__device__ __forceinline__ void scales_from_bs(const BiasBS<ST> &bi, int g, int n, float (&sc)[2]) {
    static_assert(ST != SWQ_F32, "2-byte scales");
    auto pick4 = [](uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, int i) {
        return (i & 2) ? ((i & 1) ? w3 : w2) : ((i & 1) ? w1 : w0);
    };
    const int i = (g & 7) >> 1;
    const uint32_t w0 = pick4(bi.s[0][0], bi.s[0][1], bi.s[0][2], bi.s[0][3], i);
    const uint32_t w1 = pick4(bi.s[1][0], bi.s[1][1], bi.s[1][2], bi.s[1][3], i);
    // {operand 0, operand 1} halves of group g: bytes 0-1 or 2-3 of each word
    const uint32_t both = __builtin_amdgcn_perm(w1, w0, (g & 1) ? 0x07060302u : 0x05040100u);
    const uint32_t r = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(((g >> 3) * 16 + n) * 4, static_cast<int>(both)));
    sc[0] = scale_of<ST>(r & 0xFFFFu);
    sc[1] = scale_of<ST>(r >> 16);
}

// Position of column c in a row stored in nibble_order (within each 8).
__device__ __forceinline__ int nibble_pos(int c) {
    const int i = c & 7;
    return (c & ~7) | (i < 4 ? 2 * i : 2 * i - 7);
}

// Epilogue: lane holds column n of rows 16 mt + 4 kg + r.  kEpiRows stores
// f32 rows; kEpiSwiGLU stores h = silu(g) * u as bf16 hi + lo planes and the
// group sum of h over the workgroup's 64 columns (one group of the down
// projection's input).  Every thread of the workgroup calls it.
template <int EPI, int MT, int WAVES = 4>
__device__ __forceinline__ void epilogue(const f32x4_t (&acc)[MT][2], const GemmArgs &a, const int (&col)[2], int N,
                                         bool active, int row0, int rows, int nb, float *s_red, int64_t obase = 0) {
    constexpr int ROWS = 16 * MT;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 15, kg = lane >> 4;
    if constexpr (EPI == kEpiSwiGLU) {
        const bool cok = active && col[0] < N;
        const int pc = a.o_perm ? nibble_pos(col[0]) : col[0];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if (16 * mt >= rows) break;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * mt + 4 * kg + r;
                const float h = swiglu(acc[mt][0][r], acc[mt][1][r]);
                uint32_t hi, lo;
                split_pair(h, 0.f, hi, lo);
                if (cok && row < rows) {
                    const int64_t o = static_cast<int64_t>(row0 + row) * a.o_ld + pc;
                    static_cast<uint16_t *>(a.o0)[o] = static_cast<uint16_t>(hi);
                    static_cast<uint16_t *>(a.o1)[o] = static_cast<uint16_t>(lo);
                }
                const float hv = cok ? bf16_lo(hi) + bf16_lo(lo) : 0.f;
                const float rs = segment_reduce(hv, 4);  // the wave's 16 columns
                if (n == 0) s_red[wave * ROWS + row] = rs;
            }
        }
        __syncthreads();
        // waves 4 q .. 4 q + 3 cover group (nb * col_block / 64 + q) of h (16 columns each)
        constexpr int NQ = WAVES / 4;
        for (int i = tid; i < rows * NQ; i += 64 * WAVES) {
            const int gq = i / rows, r = i - gq * rows;
            const float *sr = s_red + 4 * gq * ROWS + r;
            const float t = (sr[0] + sr[ROWS]) + (sr[2 * ROWS] + sr[3 * ROWS]);
            a.xs_out[static_cast<int64_t>(row0 + r) * a.xs_ld_out + nb * (a.col_block / 64) + gq] = t;
        }
    } else if (active) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if (16 * mt >= rows) break;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = 16 * mt + 4 * kg + r;
                if (row >= rows) continue;
                const int64_t o = obase + static_cast<int64_t>(row0 + row) * a.o_ld;
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    if (col[j] < N) static_cast<float *>(a.o0)[o + col[j]] = acc[mt][j][r];
            }
        }
    }
}

constexpr int kBlockG = 4;  // pf_gemm: K groups staged per round trip

// The grouped quantised GEMM: one workgroup computes a tile of up to 16*MT
// activation rows against 4 waves x 2 operands x 16 matrix rows (output
// columns); see the file comment for the arithmetic.  Rows past the tile
// (`rows`) are staged from row 0 and never stored: the matrix cores keep rows
// apart, so they cannot disturb the others.
template <int BITS, int ST, int SRC, int MT, int EPI, int SUM>
__global__ __launch_bounds__(kPfThreads) void pf_gemm(const GemmArgs a) {
    constexpr int ROWS = 16 * MT;
    constexpr int NPL = SRC == kSrcBF16 ? 1 : 2;
    constexpr int PIECES = ROWS * 8;
    constexpr int PPT = (PIECES + kPfThreads - 1) / kPfThreads;
    __shared__ __attribute__((aligned(16))) uint16_t s_a[kBlockG][NPL][ROWS * kLdsPitch];
    __shared__ __attribute__((aligned(16))) float s_xs[SUM == kSumStage ? ROWS * kXsPitch : 1];
    __shared__ float s_red[EPI == kEpiSwiGLU ? 4 * ROWS : 1];
    // raw scales and biases of the slice's groups for the workgroup's
    // columns: [operand][scales, biases][wave * 16 + n][group - gb], one
    // u32 per element (f32) or a u16 pair per word
    __shared__ uint32_t s_tab[2 * 2 * 64 * kBlockG];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, kg = lane >> 4;

    // Workgroup b runs on XCD b % 8 (round-robin dispatch).  XCD x takes
    // tiles x, x + 8, ...; the column blocks of one tile follow each other
    // on the same XCD, so its activation rows come from HBM once and from
    // that XCD's L2 afterwards.
    const int xcd = blockIdx.x & (kXcds - 1), q = blockIdx.x >> 3;
    const int ti = (q / a.nblk) * kXcds + xcd, nb = q % a.nblk;
    int expert = 0, row0, rows;
    if (a.tiles) {
        if (ti >= *a.n_tiles) return;
        const Tile t = a.tiles[ti];
        expert = t.expert;
        row0 = t.row0;
        rows = t.rows;
        // a table from a workspace that skipped swq_moe_workspace_init
        if (expert < 0 || expert > a.E || rows <= 0 || rows > ROWS || row0 < 0 || row0 + rows > a.rows_total)
            return;
    } else {
        row0 = ti * ROWS;
        if (row0 >= a.rows_total) return;
        rows = min(ROWS, a.rows_total - row0);
    }
    const bool shared = expert == a.E;
    const int K = shared ? a.Ksh : a.K;
    const int N = shared ? a.Nsh : a.N;
    const int NG = K / kGroupK;
    // this workgroup's K slice (blockIdx.y of kslices): groups [gb, ge), an
    // even count of at most kBlockG
    const int gb = static_cast<int>(blockIdx.y) * a.kgroups, ge = min(gb + a.kgroups, NG);
    if (gb >= ge) return;
    const int wcol = nb * a.col_block + wave * a.col_wave;
    const bool active = wcol < N;

    // ---- B operands: matrix row R_j of this lane, clamped into the matrix
    const uint8_t *wrow[2];
    const uint8_t *sbase[2];
    const uint8_t *bbase[2];
    int64_t srow[2];
    int col[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const QMat &m = shared ? a.sh[j] : a.m[j];
        col[j] = wcol + j * a.col_op + n;
        const int R = min(col[j], N - 1);
        const int64_t eoff_w = shared ? 0 : static_cast<int64_t>(expert) * m.stride_w;
        const int64_t eoff_s = shared ? 0 : static_cast<int64_t>(expert) * m.stride_sb;
        wrow[j] = m.w + eoff_w + static_cast<int64_t>(R) * m.row_bytes + (BITS == 4 ? 8 : 16) * kg;
        sbase[j] = m.s + eoff_s;
        bbase[j] = m.b + eoff_s;
        srow[j] = static_cast<int64_t>(R) * m.gpr;
    }

    auto load_b = [&](BSlot<BITS> &sl, int g) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if constexpr (BITS == 4) {
                const uint2 v = *reinterpret_cast<const uint2 *>(wrow[j] + 32 * g);
                sl.w[j][0] = v.x;
                sl.w[j][1] = v.y;
            } else {
                const uint4 v = *reinterpret_cast<const uint4 *>(wrow[j] + 64 * g);
                sl.w[j][0] = v.x;
                sl.w[j][1] = v.y;
                sl.w[j][2] = v.z;
                sl.w[j][3] = v.w;
            }
        }
    };

    // ---- the slice's scales and biases into s_tab, every load at once
    // (4-byte words of an even group count per row; 2-byte entries may
    // start 2 bytes past a word boundary, and are then taken from the two
    // aligned words around them with a byte shift: no branch around the loads)
    {
        constexpr int ES = ST == SWQ_F32 ? 4 : 2;
        constexpr int WPE = kBlockG * ES / 4;  // words per (operand, array, column)
        constexpr int WORDS = 2 * 2 * 64 * WPE;
        constexpr int PER = WORDS / kPfThreads;
        const int valid = (ge - gb) * ES / 4;  // words holding the slice's groups
        uint32_t v[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int w = tid + u * kPfThreads;
            const int q = w % WPE, lc = (w / WPE) % 64, arr = (w / (WPE * 64)) % 2, j = w / (WPE * 128);
            const int c = min(nb * a.col_block + (lc >> 4) * a.col_wave + j * a.col_op + (lc & 15), N - 1);
            const uint8_t *base = arr ? (j ? bbase[1] : bbase[0]) : (j ? sbase[1] : sbase[0]);
            const int64_t byte = (static_cast<int64_t>(c) * (K / kGroupK) + gb) * ES + 4 * min(q, valid - 1);
            if constexpr (ES == 4) {
                v[u] = *reinterpret_cast<const uint32_t *>(base + byte);
            } else {
                // mis = 0 or 2; the second word is read only when the entries
                // straddle it (it lies in the same aligned word as their end)
                const uintptr_t pa = reinterpret_cast<uintptr_t>(base + byte);
                const uint32_t mis = static_cast<uint32_t>(pa & 3u);
                const uint32_t *w = reinterpret_cast<const uint32_t *>(pa & ~static_cast<uintptr_t>(3));
                const uint32_t w0 = w[0], w1 = w[mis ? 1 : 0];
                v[u] = __builtin_amdgcn_alignbyte(w1, w0, mis);
            }
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) s_tab[tid + u * kPfThreads] = v[u];
    }
    // raw scale (arr 0) or bias (arr 1) of operand j, this lane's column, group g
    auto tab = [&](int j, int arr, int g) -> uint32_t {
        const int e = ((j * 2 + arr) * 64 + wave * 16 + n) * kBlockG + (g - gb);
        if constexpr (ST == SWQ_F32) return s_tab[e];
        else return reinterpret_cast<const uint16_t *>(s_tab)[e];
    };

    // ---- A staging (rows past the tile stage row 0)
    int64_t src[PPT];
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
        const int p = tid + kPfThreads * i;
        const int r = p >> 3;
        const int rr = p < PIECES && r < rows ? r : 0;
        const int64_t s = min(max(a.row_src ? a.row_src[row0 + rr] : row0 + rr, 0), a.a_rows - 1);
        src[i] = s * a.a_ld + 8 * (p & 7);
    }

    auto load_a = [&](AStage<SRC, PPT> &st, int g) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int64_t e = src[i] + kGroupK * g;
            if constexpr (SRC == kSrcBF16) {
                st.v[i][0] = *reinterpret_cast<const u32x4_t *>(static_cast<const uint16_t *>(a.a0) + e);
            } else if constexpr (SRC == kSrcF32) {
                const float *p = static_cast<const float *>(a.a0) + e;
                st.v[i][0] = *reinterpret_cast<const u32x4_t *>(p);
                st.v[i][1] = *reinterpret_cast<const u32x4_t *>(p + 4);
            } else {
                st.v[i][0] = *reinterpret_cast<const u32x4_t *>(static_cast<const uint16_t *>(a.a0) + e);
                st.v[i][1] = *reinterpret_cast<const u32x4_t *>(static_cast<const uint16_t *>(a.a1) + e);
            }
        }
    };

    auto store_a = [&](const AStage<SRC, PPT> &st, int buf, int g) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int p = tid + kPfThreads * i;
            if (p >= PIECES) continue;  // whole waves
            const int r = p >> 3, c8 = p & 7;
            u32x4_t hi, lo = {0u, 0u, 0u, 0u};
            if constexpr (SRC == kSrcBF16) {
                hi = st.v[i][0];
            } else if constexpr (SRC == kSrcF32) {
                float v[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[q] = __uint_as_float(st.v[i][0][q]);
                    v[4 + q] = __uint_as_float(st.v[i][1][q]);
                }
                split8(v, hi, lo);
            } else {
                hi = st.v[i][0];
                lo = st.v[i][1];
            }
            if constexpr (SUM == kSumStage) {
                float t[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if constexpr (SRC == kSrcBF16) t[q] = bf16_lo(hi[q]) + bf16_hi(hi[q]);
                    else t[q] = (bf16_lo(hi[q]) + bf16_lo(lo[q])) + (bf16_hi(hi[q]) + bf16_hi(lo[q]));
                }
                const float sum = segment_reduce((t[0] + t[1]) + (t[2] + t[3]), 3);  // 8 lanes of (row, group)
                // the last column is a sink for the redundant groups the
                // loop's tail stages (the bias term reads columns < 64)
                if (c8 == 0) s_xs[r * kXsPitch + (g < ge ? g : kXsPitch - 1)] = sum;
            }
            // the activation planes of gate/up (one column block writes them)
            if (a.pl0 && nb == 0 && g < ge && r < rows) {
                const int64_t e = static_cast<int64_t>(row0 + r) * a.a_ld + kGroupK * g + 8 * c8;
                *reinterpret_cast<u32x4_t *>(a.pl0 + e) = a.pl_perm ? nibble_order(hi) : hi;
                if (a.pl1) *reinterpret_cast<u32x4_t *>(a.pl1 + e) = a.pl_perm ? nibble_order(lo) : lo;
            }
            if constexpr (BITS == 4) {
                hi = nibble_order(hi);
                if constexpr (NPL == 2) lo = nibble_order(lo);
            }
            *reinterpret_cast<u32x4_t *>(&s_a[buf][0][r * kLdsPitch + 8 * c8]) = hi;
            if constexpr (NPL == 2) *reinterpret_cast<u32x4_t *>(&s_a[buf][1][r * kLdsPitch + 8 * c8]) = lo;
        }
    };

    f32x4_t acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const BSlot<BITS> &sl, int buf, int g) {
        u32x4_t bq[2][2];
        float sc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if constexpr (BITS == 4) {
                bq[j][0] = codes_q4(sl.w[j][0]);
                bq[j][1] = codes_q4(sl.w[j][1]);
            } else {
                bq[j][0] = codes_q8(sl.w[j][0], sl.w[j][1]);
                bq[j][1] = codes_q8(sl.w[j][2], sl.w[j][3]);
            }
            sc[j] = scale_of<ST>(tab(j, 0, g));
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if (16 * mt >= rows) break;
            const uint16_t *ar = &s_a[buf][0][(16 * mt + n) * kLdsPitch + 16 * kg];
            const u32x4_t a_0 = *reinterpret_cast<const u32x4_t *>(ar);
            const u32x4_t a_1 = *reinterpret_cast<const u32x4_t *>(ar + 8);
            u32x4_t l_0, l_1;
            if constexpr (NPL == 2) {
                const uint16_t *lr = &s_a[buf][1][(16 * mt + n) * kLdsPitch + 16 * kg];
                l_0 = *reinterpret_cast<const u32x4_t *>(lr);
                l_1 = *reinterpret_cast<const u32x4_t *>(lr + 8);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                f32x4_t c = mfma(a_0, bq[j][0], f32x4_t{0.f, 0.f, 0.f, 0.f});
                c = mfma(a_1, bq[j][1], c);
                if constexpr (NPL == 2) {
                    c = mfma(l_0, bq[j][0], c);
                    c = mfma(l_1, bq[j][1], c);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[mt][j][r] = fmaf(sc[j], c[r], acc[mt][j][r]);
            }
        }
    };

    // ---- the K loop over the slice, kBlockG groups at a time: every load
    // of a block is issued at once (A into registers, then LDS; B into
    // registers), so a slice of up to kBlockG groups costs one round trip.
    // Loads past the slice repeat group ge-1 (staged into the sink column,
    // never computed).  Waves whose columns lie past N compute on clamped
    // rows and store nothing.
#pragma unroll 1
    for (int g0 = gb; g0 < ge; g0 += kBlockG) {
        AStage<SRC, PPT> st[kBlockG];
        BSlot<BITS> bs[kBlockG];
#pragma unroll
        for (int u = 0; u < kBlockG; ++u) {
            const int g = min(g0 + u, ge - 1);
            load_a(st[u], g);
            load_b(bs[u], g);
        }
#pragma unroll
        for (int u = 0; u < kBlockG; ++u) store_a(st[u], u, g0 + u);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kBlockG; ++u)
            if (g0 + u < ge) compute(bs[u], u, g0 + u);
        __syncthreads();  // the buffers are restaged by the next block
    }

    // the router hands the group sums of x to gate/up (one column block does)
    if constexpr (SUM == kSumStage) {
        if (a.xs_out && nb == 0) {
            const int gs = ge - gb;
            for (int i = tid; i < rows * gs; i += kPfThreads) {
                const int r = i / gs, g = gb + (i - r * gs);
                a.xs_out[static_cast<int64_t>(row0 + r) * a.xs_ld_out + g] = s_xs[r * kXsPitch + g];
            }
        }
    }

    if (active) {
        const float *xrow[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int rr = min(16 * mt + n, rows - 1);
            if constexpr (SUM == kSumLoad) {
                const int64_t xr = a.row_src ? a.row_src[row0 + rr] : row0 + rr;
                xrow[mt] = a.xs_in + xr * a.xs_ld;
            } else {
                xrow[mt] = &s_xs[(16 * mt + n) * kXsPitch];
            }
        }
        // the slice's biases (and 4-bit scales) from s_tab: lane kg holds
        // groups gb + 8 kg .. (only kg = 0 has any: a slice has at most
        // kBlockG groups)
        BiasRaw<ST> braw;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int g = min(gb + 8 * kg + i, ge - 1);
                braw.b[j][i] = tab(j, 1, g);
                braw.s[j][i] = tab(j, 0, g);
            }
        bias_apply<BITS, ST, MT>(acc, braw, xrow, gb, ge, rows, kg);
    }
    epilogue<EPI, MT>(acc, a, col, N, active, row0, rows, nb, s_red, static_cast<int64_t>(blockIdx.y) * a.o_slice);
}

// ---------------------------------------------------------------------------
// the grouped GEMM on an LDS DMA ring (gate/up, down)

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// LDS DMA: lane L copies 16 (4) bytes from src to LDS byte address lds + 16 L
// (4 L); M0 carries lds.  These writes are invisible to the compiler: the
// kernel orders them by hand (vmcnt waits and barriers in ring_wait), and no
// other code in these kernels uses M0.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void *src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" : : "v"(src), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// Wait until at most N of this wave's memory loads are in flight, then meet
// the other waves: every wave's loads but its newest N have landed.
template <int N>
__device__ __forceinline__ void ring_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}

// ring_wait<Cn>() for the wave's count n of live activation copies per
// group (wave-uniform, 0..4): one branch per count, each with its immediate.
template <int C0, int C1, int C2, int C3, int C4>
__device__ __forceinline__ void ring_wait_sel(int n) {
    if (n <= 0) ring_wait<C0>();
    else if (n == 1) ring_wait<C1>();
    else if (n == 2) ring_wait<C2>();
    else if (n == 3) ring_wait<C3>();
    else ring_wait<C4>();
}

// The grouped quantised GEMM of pf_gemm (same tile, lanes and arithmetic) fed
// by an LDS ring D groups deep: per group, each wave's DMA brings in its
// share of the 64 activation rows (NPL bf16 planes, already in the order the
// codes need) and its 2 x 16 code rows (f32 scales: and their scales); a
// group is used D - 1 groups after its loads were issued.  2-byte scales come
// from registers: the bias term's scale preload holds every group's, handed
// between lanes per group.  Activation rows are 128 B; row r
// keeps its 16 B chunk c in slot c ^ (r & 7) so the matrix-core reads of 16
// rows at one chunk hit distinct banks.
template <int BITS, int ST, int NPL, int EPI, int DA, int DB, int WAVES>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(4))) void pf_gemm_dma(const GemmArgs a) {
    // B(g) must be issued before A(g) for the wait on A(g) to cover it
    static_assert(DA >= 2 && DB > DA, "ring depths");
    static_assert(WAVES == 4 || WAVES == 8, "waves per workgroup");
    constexpr int MT = 4, ROWS = 64;
    constexpr int AW = 8 / WAVES;                    // 8-row slabs each wave brings in per plane
    constexpr int A_SLOT = NPL * ROWS * 128;         // activation rows of one group
    constexpr int B_WAVE = BITS == 4 ? 1024 : 2048;  // code bytes per wave per group
    constexpr bool kScaleDma = ST == SWQ_F32;        // f32 scales ride the ring
    constexpr int B_SLOT = WAVES * (B_WAVE + (kScaleDma ? 256 : 0));  // codes (+ scales) of one group
    // DMA instructions per wave per group: activations, codes (+ scales)
    constexpr int LA = AW * NPL, LB = B_WAVE / 1024 + (kScaleDma ? 1 : 0), L = LA + LB;
    __shared__ __attribute__((aligned(16))) uint8_t s_ring_a[DA * A_SLOT];
    __shared__ __attribute__((aligned(16))) uint8_t s_ring_b[DB * B_SLOT];
    __shared__ __attribute__((aligned(16))) uint8_t s_xs[ROWS * 128];  // group sums of the rows
    __shared__ float s_red[EPI == kEpiSwiGLU ? WAVES * ROWS : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, kg = lane >> 4;

    const int xcd = blockIdx.x & (kXcds - 1), q = blockIdx.x >> 3;
    const int ti = (q / a.nblk) * kXcds + xcd, nb = q % a.nblk;
    // the count and the entry in one round trip
    const int n_tiles = *a.n_tiles;
    const Tile t = a.tiles[min(ti, a.max_tiles - 1)];
    if (ti >= n_tiles) return;
    const int expert = t.expert, row0 = t.row0, rows = t.rows;
    // a table from a workspace that skipped swq_moe_workspace_init
    if (expert < 0 || expert > a.E || rows <= 0 || rows > ROWS || row0 < 0 || row0 + rows > a.rows_total) return;
    const bool shared = expert == a.E;
    const int K = shared ? a.Ksh : a.K;
    const int N = shared ? a.Nsh : a.N;
    const int NG = K / kGroupK;
    const int wcol = nb * a.col_block + wave * a.col_wave;
    const bool active = wcol < N;

    // ---- matrices of the two operands (this lane's compute row n, clamped)
    const uint8_t *wbase[2];
    const uint8_t *sbase[2];
    const uint8_t *bbase[2];
    int64_t srow[2];
    int col[2];
    int row_bytes = 0, gpr = 0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const QMat &m = shared ? a.sh[j] : a.m[j];
        col[j] = wcol + j * a.col_op + n;
        const int64_t eoff_w = shared ? 0 : static_cast<int64_t>(expert) * m.stride_w;
        const int64_t eoff_s = shared ? 0 : static_cast<int64_t>(expert) * m.stride_sb;
        wbase[j] = m.w + eoff_w;
        sbase[j] = m.s + eoff_s;
        bbase[j] = m.b + eoff_s;
        srow[j] = static_cast<int64_t>(min(col[j], N - 1)) * m.gpr;
        row_bytes = m.row_bytes;
        gpr = m.gpr;
    }

    // ---- DMA sources: activation rows 8 (AW wave + i) + lane / 8 and their
    // group sums (128 B rows, chunks swizzled like the activations), code
    // rows and scale pairs of this wave's columns
    const uint8_t *asrc[NPL][AW];
    const uint8_t *xsrc[AW];
    // rows past the tile are not fetched (their LDS rows hold stale values,
    // which stay in those rows of the matrix-core results, never stored):
    // a wave issues the copies of its slabs that hold tile rows (`live`, the
    // same count every group; the ring waits use it), and within a partial
    // slab lane 0 always fetches so that no copy is empty
    const int live = min(AW, max(0, (rows + 7) / 8 - AW * wave));
    bool afetch[AW];
#pragma unroll
    for (int i = 0; i < AW; ++i) {
        const int r = 8 * (AW * wave + i) + (lane >> 3);
        afetch[i] = r < rows || lane == 0;
        const int c = (lane & 7) ^ (r & 7);
        const int rr = r < rows ? r : 0;
        const int64_t sr = min(max(a.row_src ? a.row_src[row0 + rr] : row0 + rr, 0), a.a_rows - 1);
        const int64_t e = sr * a.a_ld + 8 * c;
        asrc[0][i] = static_cast<const uint8_t *>(a.a0) + 2 * e;
        if constexpr (NPL == 2) asrc[1][i] = static_cast<const uint8_t *>(a.a1) + 2 * e;
        xsrc[i] = reinterpret_cast<const uint8_t *>(a.xs_in + sr * a.xs_ld) + 16 * c;
    }
    const uint8_t *bsrc[BITS == 4 ? 1 : 2];
    if constexpr (BITS == 4) {
        const int j = lane >> 5, r = min(wcol + j * a.col_op + ((lane >> 1) & 15), N - 1);
        bsrc[0] = (j ? wbase[1] : wbase[0]) + static_cast<int64_t>(r) * row_bytes + 16 * (lane & 1);
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = min(wcol + j * a.col_op + (lane >> 2), N - 1);
            bsrc[j] = wbase[j] + static_cast<int64_t>(r) * row_bytes + 16 * (lane & 3);
        }
    }
    const uint8_t *ssrc = nullptr;
    if constexpr (kScaleDma) {
        const int j = lane >> 5, r = min(wcol + j * a.col_op + (lane & 15), N - 1);
        ssrc = (j ? sbase[1] : sbase[0]) + static_cast<int64_t>(r) * gpr * 4;
    }
    const uint32_t ring_a = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_ring_a));
    const uint32_t ring_b = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_ring_b));

    // the bias term's biases and scales (the K loop takes its scales from
    // them), issued before every ring load
    BiasBS<ST> bi;
    load_bias_bs<ST>(bi, sbase, bbase, srow, NG, kg);

    // group g's activation rows into A slot sa (LA instructions per wave)
    auto issue_a = [&](int sa, int g) {
        const uint32_t base = ring_a + sa * A_SLOT;
#pragma unroll
        for (int p = 0; p < NPL; ++p)
#pragma unroll
            for (int i = 0; i < AW; ++i)
                if (i < live) {
                    // the LDS address in a scalar register before the branch
                    const uint32_t d = __builtin_amdgcn_readfirstlane(base + p * ROWS * 128 + 8 * (AW * wave + i) * 128);
                    if (afetch[i]) dma16(asrc[p][i] + kGroupK * 2 * g, d);
                }
    };
    // group g's code rows (and f32 scales) into B slot sb (LB instructions per wave)
    auto issue_b = [&](int sb, int g) {
        const uint32_t base = ring_b + sb * B_SLOT;
        if constexpr (BITS == 4) {
            dma16(bsrc[0] + 32 * g, base + wave * B_WAVE);
        } else {
            dma16(bsrc[0] + 64 * g, base + wave * B_WAVE);
            dma16(bsrc[1] + 64 * g, base + wave * B_WAVE + 1024);
        }
        if constexpr (kScaleDma) dma4(ssrc + 4 * g, base + WAVES * B_WAVE + wave * 256);
    };

    f32x4_t acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int sa, int sb, int g) {
        const uint8_t *sl = s_ring_a + sa * A_SLOT;
        const uint8_t *bl = s_ring_b + sb * B_SLOT;
        u32x4_t bq[2][2];
        float sc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            if constexpr (BITS == 4) {
                const uint2 w = *reinterpret_cast<const uint2 *>(bl + wave * B_WAVE + (j * 32 + n * 2) * 16 + 8 * kg);
                bq[j][0] = codes_q4(w.x);
                bq[j][1] = codes_q4(w.y);
            } else {
                const uint4 w = *reinterpret_cast<const uint4 *>(bl + wave * B_WAVE + (j * 64 + n * 4 + kg) * 16);
                bq[j][0] = codes_q8(w.x, w.y);
                bq[j][1] = codes_q8(w.z, w.w);
            }
            if constexpr (kScaleDma)
                sc[j] = __uint_as_float(*reinterpret_cast<const uint32_t *>(bl + WAVES * B_WAVE + wave * 256 + (j * 32 + n) * 4));
        }
        if constexpr (!kScaleDma) scales_from_bs<ST>(bi, g, n, sc);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if (16 * mt >= rows) break;
            const int m = 16 * mt + n;
            const uint8_t *ar = sl + m * 128;
            const int c0 = ((2 * kg) ^ (m & 7)) * 16, c1 = ((2 * kg + 1) ^ (m & 7)) * 16;
            const u32x4_t a_0 = *reinterpret_cast<const u32x4_t *>(ar + c0);
            const u32x4_t a_1 = *reinterpret_cast<const u32x4_t *>(ar + c1);
            u32x4_t l_0, l_1;
            if constexpr (NPL == 2) {
                l_0 = *reinterpret_cast<const u32x4_t *>(ar + ROWS * 128 + c0);
                l_1 = *reinterpret_cast<const u32x4_t *>(ar + ROWS * 128 + c1);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                f32x4_t c = mfma(a_0, bq[j][0], f32x4_t{0.f, 0.f, 0.f, 0.f});
                c = mfma(a_1, bq[j][1], c);
                if constexpr (NPL == 2) {
                    c = mfma(l_0, bq[j][0], c);
                    c = mfma(l_1, bq[j][1], c);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[mt][j][r] = fmaf(sc[j], c[r], acc[mt][j][r]);
            }
        }
    };

    // ---- the bias term's inputs (biases and scales in registers, group
    // sums by DMA into LDS), issued before the ring so that they are older
    // than every ring load (ring_wait's counts stay exact) and arrive during
    // the loop
    {
        const uint32_t xb = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(s_xs));
#pragma unroll
        for (int i = 0; i < AW; ++i) {
            const uint32_t d = __builtin_amdgcn_readfirstlane(xb + 8 * (AW * wave + i) * 128);
            if (afetch[i]) dma16(xsrc[i], d);
        }
    }

    // ---- the rings: codes DB-1 groups ahead, activation rows
    // (mostly L2 hits) DA-1 groups ahead.  Before the loop: B groups 0..DB-2,
    // then A groups 0..DA-2.  At group g: wait until A(g) has landed (B(g)
    // is older), then refill the slots group g-1 used with A(g+DA-1) and
    // B(g+DB-1) (past NG: group NG-1 again, never read), then compute g.
    // Loads return in order, so "at most N of this wave's loads in flight"
    // with N = the loads issued after A(g) means A(g) and everything before
    // it have landed; N is the same for every group from DA-1 on, and the
    // first DA-1 groups are peeled with their own counts.  The counts depend
    // on the wave's live copies n = NPL * live per group: with none, the same
    // formula counts the loads after B(g) (issued one step before A(g)
    // would be, DB = DA + 1) exactly in the loop and too few in the peeled
    // groups (a stricter wait).
#pragma unroll
    for (int s = 0; s < DB - 1; ++s) issue_b(s, min(s, NG - 1));
#pragma unroll
    for (int s = 0; s < DA - 1; ++s) issue_a(s, min(s, NG - 1));
    auto step = [&](int g, int sa, int sb) {
        issue_a(sa == 0 ? DA - 1 : sa - 1, min(g + DA - 1, NG - 1));
        issue_b(sb == 0 ? DB - 1 : sb - 1, min(g + DB - 1, NG - 1));
        compute(sa, sb, g);
    };
    static_assert(DA <= 4 && DB == DA + 1 && LA <= 4, "peeled prologue, wait counts");
    const int nl = NPL * live;
    // the wait counts for n live copies per group (n <= LA)
    constexpr auto w0 = [](int n) constexpr { return (DA - 2) * n; };
    constexpr auto w1 = [](int n) constexpr { return (DA - 3) * n + (n + LB); };
    constexpr auto w2 = [](int n) constexpr { return (DA - 4) * n + 2 * (n + LB); };
    constexpr auto wl = [](int n) constexpr { return LB + (DA - 2) * (n + LB); };
    constexpr auto cl = [](int n) constexpr { return n < LA ? n : LA; };
    if (0 < NG) ring_wait_sel<w0(0), w0(cl(1)), w0(cl(2)), w0(cl(3)), w0(cl(4))>(nl);
    // The scale words were loaded before every ring load, so the wait above
    // has landed them; the compiler cannot know that (it does not count the
    // DMA loads) and would wait for them at their first use in the loop, on
    // every pass and with a count that ignores the ring: vmcnt(0) for the
    // last words loaded, a drain of the whole ring every other pair of
    // groups.  Passing them through an empty asm here makes its outputs the
    // values the loop reads, so the compiler's one wait for them is here,
    // with a count of eight (the bias words were loaded after them).
    if constexpr (!kScaleDma)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(bi.s[j][i]));
    if (0 < NG) step(0, 0, 0);
    if constexpr (DA >= 3)
        if (1 < NG) {
            ring_wait_sel<w1(0), w1(cl(1)), w1(cl(2)), w1(cl(3)), w1(cl(4))>(nl);
            step(1, 1, 1);
        }
    if constexpr (DA >= 4)
        if (2 < NG) {
            ring_wait_sel<w2(0), w2(cl(1)), w2(cl(2)), w2(cl(3)), w2(cl(4))>(nl);
            step(2, 2, 2);
        }
    {
        int sa = (DA - 1) % DA, sb = (DA - 1) % DB;
#pragma unroll 1
        for (int g = DA - 1; g < NG; ++g) {
            ring_wait_sel<wl(0), wl(cl(1)), wl(cl(2)), wl(cl(3)), wl(cl(4))>(nl);
            step(g, sa, sb);
            sa = sa + 1 == DA ? 0 : sa + 1;
            sb = sb + 1 == DB ? 0 : sb + 1;
        }
    }

    if (active) {
        float xv[MT][8];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = 16 * mt + n;
            const uint8_t *xr = s_xs + m * 128;
            const float4 x0 = *reinterpret_cast<const float4 *>(xr + 16 * ((2 * kg) ^ (m & 7)));
            const float4 x1 = *reinterpret_cast<const float4 *>(xr + 16 * ((2 * kg + 1) ^ (m & 7)));
            xv[mt][0] = x0.x; xv[mt][1] = x0.y; xv[mt][2] = x0.z; xv[mt][3] = x0.w;
            xv[mt][4] = x1.x; xv[mt][5] = x1.y; xv[mt][6] = x1.z; xv[mt][7] = x1.w;
        }
        bias_term_bs<BITS, ST, MT>(acc, bi, xv, NG, rows, kg);
    }
    epilogue<EPI, MT, WAVES>(acc, a, col, N, active, row0, rows, nb, s_red);
}

// ---------------------------------------------------------------------------
// routing and grouping

constexpr int kMaxLogitSlices = 16;  // router K slices (partial logit rows per token): H <= 4096

struct RouteArgs {
    QMat seg;                 // shared_expert_gate [1, H]
    const void *x;
    const float *logits;      // [lslices][T, E] partial logits, summed in slice order
    const float *bias;        // [E] added to the logits, or null
    int32_t *ids;             // [T, K]
    float *wts;               // [T, K]
    int32_t *user_ids;
    float *user_w;
    float *sg;                // [T]
    int32_t *pos;             // [T, K]: sorted index of pair (t, k)
    int32_t *tok;             // [P + T]: token of each sorted row
    Tile *tiles;
    int32_t *n_tiles;
    int32_t T, E, K, H, norm, has_shared;
    int32_t lslices;
    int64_t lslice;           // elements between slices
};

// <w_sg, x_t> over one row of any vector-path format (QwenCPUModel.swift:559).
// Lane l sums chunks l, l + 64, ... in that order; two chunks' loads go out
// before either is used.
template <int XDT, int BITS>
__device__ float row_dot(const QMat &m, const void *x, int64_t x0, int lane) {
    constexpr int CPC = 128 / BITS;  // codes per 16-byte chunk
    float acc = 0.f;
    for (int c0 = lane; c0 < m.chunks; c0 += 2 * kWave) {
        const bool has1 = c0 + kWave < m.chunks;
        const int c1 = has1 ? c0 + kWave : c0;
        const uint4 w0 = *reinterpret_cast<const uint4 *>(m.w + 16 * static_cast<int64_t>(c0));
        const uint4 w1 = *reinterpret_cast<const uint4 *>(m.w + 16 * static_cast<int64_t>(c1));
        const int g0 = (c0 * CPC) / m.group, g1 = (c1 * CPC) / m.group;
        const float s0 = load_scale(m.s, g0, m.stype), b0 = load_scale(m.b, g0, m.stype);
        const float s1 = load_scale(m.s, g1, m.stype), b1 = load_scale(m.b, g1, m.stype);
        float xv0[CPC], xv1[CPC];
        load_x<XDT, CPC>(xv0, x, x0 + static_cast<int64_t>(c0) * CPC);
        load_x<XDT, CPC>(xv1, x, x0 + static_cast<int64_t>(c1) * CPC);
        float xs0 = 0.f, xs1 = 0.f;
#pragma unroll
        for (int i = 0; i < CPC; ++i) {
            xs0 += xv0[i];
            xs1 += xv1[i];
        }
        float d0, d1;
        if constexpr (BITS == 4) {
            d0 = dot_chunk_q4(w0, xv0);
            d1 = dot_chunk_q4(w1, xv1);
        } else {
            d0 = dot_chunk_q8(w0, xv0);
            d1 = dot_chunk_q8(w1, xv1);
        }
        acc += s0 * d0 + b0 * xs0;
        if (has1) acc += s1 * d1 + b1 * xs1;
    }
    return wave_sum(acc);
}

// Inclusive prefix sum over the lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int u = __shfl_up(v, d, kWave);
        if (lane >= d) v += u;
    }
    return v;
}

// The grouping workgroup (NT threads): per-expert pair counts (LDS atomics
// over the ids), exclusive scans of the pair counts and of the tile counts,
// the tile table (by decreasing row count), and the sorted pair order (a
// second pass hands out the slots; the order of pairs within an expert does
// not matter, every row is computed on its own).  The first kHeldIds * NT
// ids are loaded at once and kept in registers for the second pass.
template <int NT>
__device__ void group_pairs(const RouteArgs &a) {
    __shared__ int32_t s_cnt[kMaxExperts];  // counts, then the next free slot
    __shared__ int32_t s_wsum[2][NT / kWave];
    __shared__ int32_t s_rows[kTileRows + 1];  // tiles of each row count, then their next slot
    static_assert(NT <= kMaxExperts && NT <= 4096, "at least one expert and one held id per thread");
    constexpr int kHeldIds = 4096 / NT;  // every id of 512 tokens x top-8
    constexpr int kBatch = 8;  // ids per thread per pass past the held ones, all in flight at once
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int P = a.T * a.K;
    int held[kHeldIds];
#pragma unroll
    for (int u = 0; u < kHeldIds; ++u) held[u] = a.ids[min(tid + u * NT, P - 1)];
    for (int e = tid; e < a.E; e += NT) s_cnt[e] = 0;
    for (int r = tid; r <= kTileRows; r += NT) s_rows[r] = 0;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kHeldIds; ++u)
        if (tid + u * NT < P) atomicAdd(&s_cnt[held[u]], 1);
    for (int p0 = tid + kHeldIds * NT; p0 < P; p0 += kBatch * NT) {
        int e[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) e[u] = a.ids[min(p0 + u * NT, P - 1)];
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (p0 + u * NT < P) atomicAdd(&s_cnt[e[u]], 1);
    }
    __syncthreads();
    constexpr int EPT = kMaxExperts / NT;  // experts per thread
    int cnt[EPT], tl[EPT];
    int csum = 0, tsum = 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid * EPT + i;
        cnt[i] = e < a.E ? s_cnt[e] : 0;
        tl[i] = (cnt[i] + kTileRows - 1) / kTileRows;
        csum += cnt[i];
        tsum += tl[i];
    }
    // exclusive scans over the threads' pair and tile counts: wave scans,
    // then the wave totals
    const int cinc = wave_incl_scan(csum, lane), tinc = wave_incl_scan(tsum, lane);
    if (lane == kWave - 1) {
        s_wsum[0][wave] = cinc;
        s_wsum[1][wave] = tinc;
    }
    // The tile table in decreasing row count (the GEMMs start the heaviest
    // tiles first, so the light ones fill in at the end): tiles per row
    // count, their first slots, then each tile into the next slot of its count.
    const int sh_tiles = a.has_shared ? (a.T + kTileRows - 1) / kTileRows : 0;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        if (tid * EPT + i < a.E && cnt[i] > 0) {
            if (cnt[i] >= kTileRows) atomicAdd(&s_rows[kTileRows], cnt[i] / kTileRows);
            if (cnt[i] % kTileRows) atomicAdd(&s_rows[cnt[i] % kTileRows], 1);
        }
    }
    if (tid == 0 && sh_tiles > 0) {
        if (a.T >= kTileRows) atomicAdd(&s_rows[kTileRows], a.T / kTileRows);
        if (a.T % kTileRows) atomicAdd(&s_rows[a.T % kTileRows], 1);
    }
    __syncthreads();
    int c0 = cinc - csum, routed_tiles = 0;
#pragma unroll
    for (int w = 0; w < NT / kWave; ++w) {
        if (w < wave) c0 += s_wsum[0][w];
        routed_tiles += s_wsum[1][w];
    }
    static_assert(kTileRows == kWave, "one lane per tile row count");
    if (wave == 0) {
        // first slot of each row count, counts 64 .. 1 in that order (lane l: 64 - l)
        const int r = kTileRows - lane;
        const int n = s_rows[r];
        s_rows[r] = wave_incl_scan(n, lane) - n;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
        const int e = tid * EPT + i;
        if (e < a.E) {
            s_cnt[e] = c0;  // each thread rewrites only its own experts
            for (int q = 0; q < tl[i]; ++q) {
                const int rows = min(kTileRows, cnt[i] - q * kTileRows);
                a.tiles[atomicAdd(&s_rows[rows], 1)] = Tile{e, c0 + q * kTileRows, rows, 0};
            }
        }
        c0 += cnt[i];
    }
    for (int q = tid; q < sh_tiles; q += NT) {
        const int rows = min(kTileRows, a.T - q * kTileRows);
        a.tiles[atomicAdd(&s_rows[rows], 1)] = Tile{a.E, P + q * kTileRows, rows, 0};
    }
    if (tid == 0) *a.n_tiles = routed_tiles + sh_tiles;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kHeldIds; ++u) {
        const int p = tid + u * NT;
        if (p < P) {
            const int q = atomicAdd(&s_cnt[held[u]], 1);
            a.pos[p] = q;
            a.tok[q] = p / a.K;
        }
    }
    for (int p0 = tid + kHeldIds * NT; p0 < P; p0 += kBatch * NT) {
        int e[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) e[u] = a.ids[min(p0 + u * NT, P - 1)];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int p = p0 + u * NT;
            if (p >= P) continue;
            const int q = atomicAdd(&s_cnt[e[u]], 1);
            a.pos[p] = q;
            a.tok[q] = p / a.K;
        }
    }
    if (a.has_shared)
        for (int t = tid; t < a.T; t += NT) a.tok[P + t] = t;
}

// One token's routing on one wave: the logits of the lane's experts
// l*M .. l*M+M-1, summed over the router's K slices in slice order (every
// slice's load in flight at once) plus the bias; top-k by the rounds of
// route.hpp; the shared-expert gate logit, whose loads go out with the
// logits'.
// The lane's M consecutive entries l*M .. of a row of E floats (vector loads
// when E is a multiple of M, so that the row and lane offsets are aligned;
// entries past E repeat the last).
template <int M>
__device__ __forceinline__ void load_lane_m(const float *row, int E, int lane, bool vec, float (&v)[M]) {
    if (vec && M >= 4) {
#pragma unroll
        for (int q = 0; q < M / 4; ++q) {
            const float4 f = *reinterpret_cast<const float4 *>(row + lane * M + 4 * q);
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
    } else if (vec && M == 2) {
        const float2 f = *reinterpret_cast<const float2 *>(row + lane * M);
        v[0] = f.x;
        v[1 % M] = f.y;
    } else {
#pragma unroll
        for (int j = 0; j < M; ++j) v[j] = row[min(lane * M + j, E - 1)];
    }
}

// One token's routing on one wave: the logits of the lane's experts
// l*M .. l*M+M-1, summed over the router's K slices in slice order (eight
// slices' loads in flight at once) plus the bias; top-k by the rounds of
// route.hpp; the shared-expert gate logit, whose loads go out with the
// logits'.
template <int XDT, int M>
__device__ __forceinline__ void route_token(const RouteArgs &a, int t, int lane, int32_t *s_pick) {
    constexpr int kBatch = 8;
    const float *lg = a.logits + static_cast<int64_t>(t) * a.E;
    // lanes past E (M * 64 > E) read in bounds when E is a multiple of M
    const bool vec = a.E % M == 0 && lane * M < a.E;
    float v[M];
    float sg = 0.f;
    for (int k0 = 0; k0 < a.lslices; k0 += kBatch) {
        float part[kBatch][M];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) load_lane_m<M>(lg + min(k0 + k, a.lslices - 1) * a.lslice, a.E, lane, vec, part[k]);
        if (k0 == 0 && a.has_shared) {
            if (a.seg.bits == 4) sg = row_dot<XDT, 4>(a.seg, a.x, static_cast<int64_t>(t) * a.H, lane);
            else sg = row_dot<XDT, 8>(a.seg, a.x, static_cast<int64_t>(t) * a.H, lane);
        }
#pragma unroll
        for (int j = 0; j < M; ++j) {
            float acc = k0 == 0 ? part[0][j] : v[j] + part[0][j];
#pragma unroll
            for (int k = 1; k < kBatch; ++k)
                if (k0 + k < a.lslices) acc += part[k][j];
            v[j] = acc;
        }
    }
    if (a.bias) {
#pragma unroll
        for (int j = 0; j < M; ++j) v[j] += a.bias[min(lane * M + j, a.E - 1)];
    }
    Rounds<M> rd;
    rounds_init(rd, v, a.E, lane);
    rounds_run(rd, a.K, lane, s_pick);
    const float w = rounds_weight(rd, a.K, a.norm, lane);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < a.K) {
        const int32_t id = s_pick[lane];
        const int64_t p = static_cast<int64_t>(t) * a.K + lane;
        a.ids[p] = id;
        a.wts[p] = w;
        if (a.user_ids) a.user_ids[p] = id;
        if (a.user_w) a.user_w[p] = w;
    }
    if (a.has_shared && lane == 0) a.sg[t] = sg;
}

template <int XDT>
__global__ __launch_bounds__(kRouteWaves * kWave) void pf_route(const RouteArgs a) {
    __shared__ int32_t s_pick[kRouteWaves][SWQ_MAX_TOPK];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * kRouteWaves + wave;
    if (t < a.T) {
        const int M = (a.E + kWave - 1) / kWave;
        if (M <= 1) route_token<XDT, 1>(a, t, lane, s_pick[wave]);
        else if (M <= 2) route_token<XDT, 2>(a, t, lane, s_pick[wave]);
        else if (M <= 4) route_token<XDT, 4>(a, t, lane, s_pick[wave]);
        else if (M <= 8) route_token<XDT, 8>(a, t, lane, s_pick[wave]);
        else route_token<XDT, 16>(a, t, lane, s_pick[wave]);
    }
}

// The pairs grouped by expert once every token is routed: its own launch, so
// the kernel boundary orders the routing's stores before the grouping's
// loads (an arrival count with a release per routing workgroup cost more).
constexpr int kGroupThreads = 1024;
__global__ __launch_bounds__(kGroupThreads) void pf_group(const RouteArgs a) { group_pairs<kGroupThreads>(a); }

// ---------------------------------------------------------------------------
// combine

struct CombineArgs {
    const float *y;        // [P + T, H] in sorted pair order
    const int32_t *pos;    // [T, K]
    const float *wts;      // [T, K]
    const float *sg;       // [T]
    void *out;
    int32_t T, K, H, odt, accumulate, has_shared;
};

__global__ __launch_bounds__(kPfThreads) void pf_combine(const CombineArgs a) {
    __shared__ int32_t s_pos[SWQ_MAX_TOPK];
    __shared__ float s_w[SWQ_MAX_TOPK];
    const int t = blockIdx.x;
    const int64_t P = static_cast<int64_t>(a.T) * a.K;
    if (threadIdx.x < static_cast<unsigned>(a.K)) {
        s_pos[threadIdx.x] = min(max(a.pos[t * a.K + threadIdx.x], 0), static_cast<int32_t>(P) - 1);
        s_w[threadIdx.x] = a.wts[t * a.K + threadIdx.x];
    }
    __syncthreads();
    const float gate = a.has_shared ? sigmoidf_ref(a.sg[t]) : 0.f;
    for (int c = 4 * threadIdx.x; c < a.H; c += 4 * kPfThreads) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < a.K; ++k) {
            const float4 v = *reinterpret_cast<const float4 *>(a.y + static_cast<int64_t>(s_pos[k]) * a.H + c);
            acc[0] += s_w[k] * v.x;
            acc[1] += s_w[k] * v.y;
            acc[2] += s_w[k] * v.z;
            acc[3] += s_w[k] * v.w;
        }
        if (a.has_shared) {
            const float4 v = *reinterpret_cast<const float4 *>(a.y + (P + t) * a.H + c);
            acc[0] += gate * v.x;
            acc[1] += gate * v.y;
            acc[2] += gate * v.z;
            acc[3] += gate * v.w;
        }
        const int64_t o = static_cast<int64_t>(t) * a.H + c;
        if (a.odt == SWQ_BF16) {
            uint16_t *out = static_cast<uint16_t *>(a.out) + o;
#pragma unroll
            for (int i = 0; i < 4; ++i) out[i] = f32_to_bf16_rne(acc[i]);
        } else {
            float *out = static_cast<float *>(a.out) + o;
#pragma unroll
            for (int i = 0; i < 4; ++i) out[i] = a.accumulate ? out[i] + acc[i] : acc[i];
        }
    }
}

// ---------------------------------------------------------------------------
// host side

// K slices of the router GEMM: kBlockG groups each (the last one 2 when the
// group count is not a multiple of 4), so that 16-token tiles x 128-column
// blocks x slices fill the device and a slice's loads are one round trip.
int router_kslices(int H) { return (H / kGroupK + kBlockG - 1) / kBlockG; }

struct PfLayout {
    size_t header, logits, sg, ids, wts, pos, tok, tiles, xs_x, xs_h, xa0, xa1, h_hi, h_lo, y, total;
    int max_tiles, Ih, xs_ld_x, xs_ld_h, kslices;
};

PfLayout pf_layout(const swq_moe_layer *l, int T) {
    PfLayout w{};
    size_t off = 0;
    auto take = [&](size_t n) {
        const size_t o = off;
        off = align256(off + n);
        return o;
    };
    const size_t P = static_cast<size_t>(T) * l->top_k;
    const size_t rows = P + (l->has_shared ? T : 0);
    const int U = static_cast<int>(std::min<size_t>(P, static_cast<size_t>(l->num_experts)));
    w.max_tiles = static_cast<int>((P + static_cast<size_t>(kTileRows - 1) * U) / kTileRows) +
                  (l->has_shared ? (T + kTileRows - 1) / kTileRows : 0);
    w.Ih = std::max(l->moe_intermediate, l->has_shared ? l->shared_intermediate : 0);
    w.header = take(256);  // [1] tile count
    w.kslices = router_kslices(l->hidden);
    w.logits = take(static_cast<size_t>(w.kslices) * T * l->num_experts * 4);  // [slice][T][E] partial logits
    w.sg = take(static_cast<size_t>(T) * 4);
    w.ids = take(P * 4);
    w.wts = take(P * 4);
    w.pos = take(P * 4);
    w.tok = take(rows * 4);
    w.tiles = take(static_cast<size_t>(w.max_tiles) * sizeof(Tile));
    w.xs_ld_x = ((l->hidden / kGroupK) + 31) & ~31;  // whole 32-group blocks (the bias MFMA's k)
    w.xs_ld_h = ((w.Ih / kGroupK) + 31) & ~31;
    w.xs_x = take(static_cast<size_t>(T) * w.xs_ld_x * 4);
    w.xs_h = take(rows * w.xs_ld_h * 4);
    w.xa0 = take(static_cast<size_t>(T) * l->hidden * 2);  // x planes for gate/up
    w.xa1 = take(static_cast<size_t>(T) * l->hidden * 2);
    w.h_hi = take(rows * w.Ih * 2);
    w.h_lo = take(rows * w.Ih * 2);
    w.y = take(rows * l->hidden * 4);
    w.total = off;
    return w;
}

// A matrix on the MFMA path: 4/8-bit codes, group 64, rows of whole 128-input
// blocks (an even number of groups), at most 4096 inputs, 16 B aligned rows.
int check_mfma(const swq_qlinear *l, int out_dim, int in_dim, bool stacked, int E, bool dma = true) {
    int st = check_linear_shape(l);
    if (st != SWQ_OK) return st;
    if (l->out_dim != out_dim || l->in_dim != in_dim) return SWQ_ERR_BAD_SHAPE;
    if (l->bits != 4 && l->bits != 8) return SWQ_ERR_UNSUPPORTED_BITS;
    if (l->group_size != kGroupK) return SWQ_ERR_LIMIT;
    if (in_dim % (2 * kGroupK) != 0 || in_dim > kGroupK * kMaxGroups) return SWQ_ERR_LIMIT;
    if (!vector_path_ok(l, 0, 0, 0)) return SWQ_ERR_MISALIGNED;
    // the LDS DMA kernels fetch 2-byte scales and biases as aligned 4-byte
    // pairs, and take the bias term over one block of 32 groups
    if (dma && in_dim > 32 * kGroupK) return SWQ_ERR_LIMIT;
    if (dma && (((reinterpret_cast<uintptr_t>(l->scales) + l->s_off) % 4 != 0) ||
                ((reinterpret_cast<uintptr_t>(l->biases) + l->b_off) % 4 != 0) || l->expert_stride_sb % 4 != 0))
        return SWQ_ERR_MISALIGNED;
    if (stacked && E > 1 && (l->expert_stride_w == 0 || l->expert_stride_sb == 0)) return SWQ_ERR_INVALID_ARGUMENT;
    return SWQ_OK;
}

int check_prefill_layer(const swq_moe_layer *l, int T) {
    if (!l) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->reserved != 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (T <= 0 || l->hidden <= 0 || l->num_experts <= 0 || l->moe_intermediate <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->top_k <= 0 || l->top_k > l->num_experts) return SWQ_ERR_EXPERT_RANGE;
    if (l->top_k > SWQ_MAX_TOPK || l->num_experts > kMaxExperts) return SWQ_ERR_LIMIT;
    if (static_cast<int64_t>(T) * l->top_k > (1 << 24)) return SWQ_ERR_LIMIT;
    const int H = l->hidden, E = l->num_experts, I = l->moe_intermediate;
    int st;
    if ((st = check_mfma(&l->router, E, H, false, E, false)) != SWQ_OK) return st;
    // the router GEMM stages f32 scales and biases as aligned 4-byte words
    // (2-byte ones at any even offset)
    if (l->router.scales_type == SWQ_F32 &&
        (((reinterpret_cast<uintptr_t>(l->router.scales) + l->router.s_off) % 4 != 0) ||
         ((reinterpret_cast<uintptr_t>(l->router.biases) + l->router.b_off) % 4 != 0)))
        return SWQ_ERR_MISALIGNED;
    if ((st = check_mfma(&l->gate, I, H, true, E)) != SWQ_OK) return st;
    if ((st = check_mfma(&l->up, I, H, true, E)) != SWQ_OK) return st;
    if ((st = check_mfma(&l->down, H, I, true, E)) != SWQ_OK) return st;
    // one kernel instance per launch: one code width and one scale dtype
    if (l->gate.bits != l->up.bits || l->gate.scales_type != l->up.scales_type) return SWQ_ERR_LIMIT;
    if (l->has_shared) {
        const int Is = l->shared_intermediate;
        if (Is <= 0) return SWQ_ERR_INVALID_ARGUMENT;
        if ((st = check_mfma(&l->shared_gate, Is, H, false, 1)) != SWQ_OK) return st;
        if ((st = check_mfma(&l->shared_up, Is, H, false, 1)) != SWQ_OK) return st;
        if ((st = check_mfma(&l->shared_down, H, Is, false, 1)) != SWQ_OK) return st;
        if ((st = check_linear_shape(&l->shared_expert_gate)) != SWQ_OK) return st;
        const swq_qlinear &sg = l->shared_expert_gate;
        if (sg.out_dim != 1 || sg.in_dim != H) return SWQ_ERR_BAD_SHAPE;
        if (sg.bits != 4 && sg.bits != 8) return SWQ_ERR_UNSUPPORTED_BITS;
        if ((static_cast<int64_t>(H) * sg.bits) % 128 != 0 || (static_cast<int64_t>(sg.group_size) * sg.bits) % 128 != 0)
            return SWQ_ERR_BAD_SHAPE;
        if (!vector_path_ok(&sg, 0, 0, 0)) return SWQ_ERR_MISALIGNED;
        if (l->shared_gate.bits != l->gate.bits || l->shared_up.bits != l->gate.bits ||
            l->shared_down.bits != l->down.bits)
            return SWQ_ERR_LIMIT;
        if (l->shared_gate.scales_type != l->gate.scales_type || l->shared_up.scales_type != l->gate.scales_type ||
            l->shared_down.scales_type != l->down.scales_type)
            return SWQ_ERR_LIMIT;
    }
    return SWQ_OK;
}

template <int BITS, int SRC, int MT, int EPI, int SUM>
void launch_gemm_st(int stype, const GemmArgs &a, int blocks, hipStream_t s) {
    const dim3 grid(blocks, a.kslices);
    if (stype == SWQ_F16)
        hipLaunchKernelGGL((pf_gemm<BITS, SWQ_F16, SRC, MT, EPI, SUM>), grid, dim3(kPfThreads), 0, s, a);
    else if (stype == SWQ_BF16)
        hipLaunchKernelGGL((pf_gemm<BITS, SWQ_BF16, SRC, MT, EPI, SUM>), grid, dim3(kPfThreads), 0, s, a);
    else
        hipLaunchKernelGGL((pf_gemm<BITS, SWQ_F32, SRC, MT, EPI, SUM>), grid, dim3(kPfThreads), 0, s, a);
}

template <int SRC, int MT, int EPI, int SUM>
int launch_gemm(const swq_qlinear &lin, const GemmArgs &a, int blocks, hipStream_t s) {
    if (blocks <= 0) return SWQ_OK;
    // slices of kBlockG groups cover the rows' groups (an even count), the
    // scale table covers the column block; tiled rows hold one slice
    const int NG = a.K / kGroupK;
    if (a.kgroups != std::min(kBlockG, NG) || a.kslices != (NG + kBlockG - 1) / kBlockG || a.col_block > 128 ||
        a.col_wave != 32 || a.col_op != 16 || (a.kslices > 1 && (a.tiles || EPI != kEpiRows)))
        return SWQ_ERR_INVALID_ARGUMENT;
    if (lin.bits == 4) launch_gemm_st<4, SRC, MT, EPI, SUM>(lin.scales_type, a, blocks, s);
    else launch_gemm_st<8, SRC, MT, EPI, SUM>(lin.scales_type, a, blocks, s);
    return launch_status();
}

// Waves per workgroup and ring depths of the DMA GEMMs.  Down and 8-bit
// gate/up (bf16 x): 8 waves (256 down or 128 gate/up columns per workgroup:
// the tile's activation rows are shared by twice the columns), two
// workgroups in a CU's 160 KB of LDS.  4-bit gate/up with bf16 x: 4 waves
// (64 columns, 49 KB), three workgroups per CU: twice the workgroups, which
// spreads the last, partly filled round of tiles over more CUs (gate/up
// 113 -> 108.5 us on the 512-token chunk; down at 4 waves fits only two
// per CU and loses, 80 -> 87 us).  8-bit codes with two activation planes:
// 4 waves.
int dma_waves(int bits, int npl) { return (bits == 8 && npl == 2) || (bits == 4 && npl == 1) ? 4 : 8; }

template <int BITS, int NPL, int EPI>
void launch_dma_st(int stype, const GemmArgs &a, int blocks, hipStream_t s) {
    constexpr int W = (BITS == 8 && NPL == 2) || (BITS == 4 && NPL == 1) ? 4 : 8;
    constexpr int DA = BITS == 4 && NPL == 1 ? 3 : 2;
    constexpr int DB = DA + 1;
    const dim3 th(64 * W);
    if (stype == SWQ_F16)
        hipLaunchKernelGGL((pf_gemm_dma<BITS, SWQ_F16, NPL, EPI, DA, DB, W>), dim3(blocks), th, 0, s, a);
    else if (stype == SWQ_BF16)
        hipLaunchKernelGGL((pf_gemm_dma<BITS, SWQ_BF16, NPL, EPI, DA, DB, W>), dim3(blocks), th, 0, s, a);
    else
        hipLaunchKernelGGL((pf_gemm_dma<BITS, SWQ_F32, NPL, EPI, DA, DB, W>), dim3(blocks), th, 0, s, a);
}

template <int NPL, int EPI>
int launch_dma(const swq_qlinear &lin, const GemmArgs &a, int blocks, hipStream_t s) {
    if (blocks <= 0) return SWQ_OK;
    if (lin.bits == 4) launch_dma_st<4, NPL, EPI>(lin.scales_type, a, blocks, s);
    else launch_dma_st<8, NPL, EPI>(lin.scales_type, a, blocks, s);
    return launch_status();
}

int prefill_impl(const swq_moe_layer *layer, const void *x, int x_dtype, int T, void *out, int out_dtype,
                 int32_t *topk_ids, float *topk_weights, const float *logit_bias, void *ws, size_t ws_bytes,
                 int flags, int stage_mask, void *stream) {
    if (x_dtype != SWQ_F32 && x_dtype != SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if (stage_mask <= 0 || stage_mask > SWQ_PREFILL_ALL) return SWQ_ERR_INVALID_ARGUMENT;
    int st = check_prefill_layer(layer, T);
    if (st != SWQ_OK) return st;
    if (!x || !out) return SWQ_ERR_INVALID_ARGUMENT;
    if (out_dtype != SWQ_F32 && out_dtype != SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if ((flags & ~SWQ_MOE_ACCUMULATE) != 0) return SWQ_ERR_INVALID_ARGUMENT;
    const bool accumulate = (flags & SWQ_MOE_ACCUMULATE) != 0;
    if (accumulate && out_dtype != SWQ_F32) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0)
        return SWQ_ERR_MISALIGNED;
    const PfLayout wl = pf_layout(layer, T);
    if (!ws || ws_bytes < wl.total) return SWQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(ws) % 256 != 0) return SWQ_ERR_MISALIGNED;

    uint8_t *wsb = static_cast<uint8_t *>(ws);
    uint32_t *header = reinterpret_cast<uint32_t *>(wsb + wl.header);
    const int H = layer->hidden, E = layer->num_experts, K = layer->top_k, I = layer->moe_intermediate;
    const int Is = layer->has_shared ? layer->shared_intermediate : 0;
    const int P = T * K;
    const int rows_sorted = P + (layer->has_shared ? T : 0);
    float *logits = reinterpret_cast<float *>(wsb + wl.logits);
    int32_t *tok = reinterpret_cast<int32_t *>(wsb + wl.tok);
    int32_t *pos = reinterpret_cast<int32_t *>(wsb + wl.pos);
    float *wts = reinterpret_cast<float *>(wsb + wl.wts);
    float *sg = reinterpret_cast<float *>(wsb + wl.sg);
    Tile *tiles = reinterpret_cast<Tile *>(wsb + wl.tiles);
    int32_t *n_tiles = reinterpret_cast<int32_t *>(header + 1);
    uint16_t *h_hi = reinterpret_cast<uint16_t *>(wsb + wl.h_hi);
    uint16_t *h_lo = reinterpret_cast<uint16_t *>(wsb + wl.h_lo);
    float *y = reinterpret_cast<float *>(wsb + wl.y);
    float *xs_x = reinterpret_cast<float *>(wsb + wl.xs_x);
    float *xs_h = reinterpret_cast<float *>(wsb + wl.xs_h);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool bf16x = x_dtype == SWQ_BF16;

    // x planes for gate/up (nibble_order for 4-bit codes, hi/lo for fp32 x)
    // and the group sums of x: written by the router GEMM as it stages x
    const bool perm_x = layer->gate.bits == 4;
    const bool planes = perm_x || !bf16x;
    uint16_t *xa0 = reinterpret_cast<uint16_t *>(wsb + wl.xa0);
    uint16_t *xa1 = reinterpret_cast<uint16_t *>(wsb + wl.xa1);
    // 1. router logits
    if (stage_mask & 2) {
        GemmArgs g{};
        g.m[0] = g.m[1] = make_qmat(&layer->router);
        g.a0 = x;
        g.a_ld = H;
        g.o0 = logits;
        g.o_ld = E;
        g.K = g.Ksh = H;
        g.N = g.Nsh = E;
        g.E = -1;
        g.rows_total = T;
        g.a_rows = T;
        g.col_block = 128;
        g.col_wave = 32;
        g.col_op = 16;
        g.nblk = (E + 127) / 128;
        g.kslices = wl.kslices;
        g.kgroups = std::min(kBlockG, H / kGroupK);
        g.o_slice = static_cast<int64_t>(T) * E;
        g.xs_out = xs_x;
        g.xs_ld_out = wl.xs_ld_x;
        g.pl0 = planes ? xa0 : nullptr;
        g.pl1 = planes && !bf16x ? xa1 : nullptr;
        g.pl_perm = perm_x ? 1 : 0;
        const int blocks = gemm_blocks((T + kRouterRows - 1) / kRouterRows, g.nblk);
        st = bf16x ? launch_gemm<kSrcBF16, 1, kEpiRows, kSumStage>(layer->router, g, blocks, s)
                   : launch_gemm<kSrcF32, 1, kEpiRows, kSumStage>(layer->router, g, blocks, s);
        if (st != SWQ_OK) return st;
    }
    // 2. routing and grouping
    if (stage_mask & 4) {
        RouteArgs r{};
        if (layer->has_shared) r.seg = make_qmat(&layer->shared_expert_gate);
        r.x = x;
        r.logits = logits;
        r.lslices = wl.kslices;
        r.lslice = static_cast<int64_t>(T) * E;
        r.bias = logit_bias;
        r.ids = reinterpret_cast<int32_t *>(wsb + wl.ids);
        r.wts = wts;
        r.user_ids = topk_ids;
        r.user_w = topk_weights;
        r.sg = sg;
        r.pos = pos;
        r.tok = tok;
        r.tiles = tiles;
        r.n_tiles = n_tiles;
        r.T = T;
        r.E = E;
        r.K = K;
        r.H = H;
        r.norm = layer->norm_topk_prob ? 1 : 0;
        r.has_shared = layer->has_shared ? 1 : 0;
        const int blocks = (T + kRouteWaves - 1) / kRouteWaves;
        if (bf16x) hipLaunchKernelGGL(pf_route<SWQ_BF16>, dim3(blocks), dim3(kRouteWaves * kWave), 0, s, r);
        else hipLaunchKernelGGL(pf_route<SWQ_F32>, dim3(blocks), dim3(kRouteWaves * kWave), 0, s, r);
        if ((st = launch_status()) != SWQ_OK) return st;
        hipLaunchKernelGGL(pf_group, dim3(1), dim3(kGroupThreads), 0, s, r);
        if ((st = launch_status()) != SWQ_OK) return st;
    }
    // 3. gate/up + SwiGLU over the tiles
    if (stage_mask & 8) {
        GemmArgs g{};
        g.m[0] = make_qmat(&layer->gate);
        g.m[1] = make_qmat(&layer->up);
        if (layer->has_shared) {
            g.sh[0] = make_qmat(&layer->shared_gate);
            g.sh[1] = make_qmat(&layer->shared_up);
        }
        g.a0 = planes ? static_cast<const void *>(xa0) : x;
        g.a1 = xa1;
        g.a_ld = H;
        g.row_src = tok;
        g.tiles = tiles;
        g.n_tiles = n_tiles;
        g.o0 = h_hi;
        g.o1 = h_lo;
        g.o_ld = wl.Ih;
        g.o_perm = layer->down.bits == 4 ? 1 : 0;
        g.rows_total = rows_sorted;
        g.a_rows = T;
        g.xs_in = xs_x;
        g.xs_out = xs_h;
        g.xs_ld = wl.xs_ld_x;
        g.xs_ld_out = wl.xs_ld_h;
        g.K = g.Ksh = H;
        g.N = I;
        g.Nsh = Is;
        g.E = E;
        g.col_wave = 16;
        g.col_block = 16 * dma_waves(layer->gate.bits, bf16x ? 1 : 2);
        g.col_op = 0;
        g.nblk = (wl.Ih + g.col_block - 1) / g.col_block;
        g.max_tiles = wl.max_tiles;
        const int blocks = gemm_blocks(wl.max_tiles, g.nblk);
        st = bf16x ? launch_dma<1, kEpiSwiGLU>(layer->gate, g, blocks, s)
                   : launch_dma<2, kEpiSwiGLU>(layer->gate, g, blocks, s);
        if (st != SWQ_OK) return st;
    }
    // 4. down over the tiles
    if (stage_mask & 16) {
        GemmArgs g{};
        g.m[0] = g.m[1] = make_qmat(&layer->down);
        if (layer->has_shared) g.sh[0] = g.sh[1] = make_qmat(&layer->shared_down);
        g.a0 = h_hi;
        g.a1 = h_lo;
        g.a_ld = wl.Ih;
        g.tiles = tiles;
        g.n_tiles = n_tiles;
        g.o0 = y;
        g.o_ld = H;
        g.rows_total = rows_sorted;
        g.a_rows = rows_sorted;
        g.xs_in = xs_h;
        g.xs_ld = wl.xs_ld_h;
        g.K = I;
        g.Ksh = Is;
        g.N = g.Nsh = H;
        g.E = E;
        g.col_wave = 32;
        g.col_block = 32 * dma_waves(layer->down.bits, 2);
        g.col_op = 16;
        g.nblk = (H + g.col_block - 1) / g.col_block;
        g.max_tiles = wl.max_tiles;
        const int blocks = gemm_blocks(wl.max_tiles, g.nblk);
        if ((st = launch_dma<2, kEpiRows>(layer->down, g, blocks, s)) != SWQ_OK) return st;
    }
    // 5. weighted combine in pick order, then the gated shared expert
    if (stage_mask & 32) {
        CombineArgs c{};
        c.y = y;
        c.pos = pos;
        c.wts = wts;
        c.sg = sg;
        c.out = out;
        c.T = T;
        c.K = K;
        c.H = H;
        c.odt = out_dtype;
        c.accumulate = accumulate ? 1 : 0;
        c.has_shared = layer->has_shared ? 1 : 0;
        hipLaunchKernelGGL(pf_combine, dim3(T), dim3(kPfThreads), 0, s, c);
        if ((st = launch_status()) != SWQ_OK) return st;
    }
    (void)P;
    return SWQ_OK;
}

}  // namespace
}  // namespace swq

using namespace swq;

extern "C" size_t swq_moe_prefill_workspace_bytes(const swq_moe_layer *layer, int tokens) {
    if (check_prefill_layer(layer, tokens) != SWQ_OK) return 0;
    return pf_layout(layer, tokens).total;
}

extern "C" int swq_moe_prefill(const swq_moe_layer *layer, const void *x, int x_dtype, int tokens, void *out,
                               int out_dtype, int32_t *topk_ids, float *topk_weights, void *ws, size_t ws_bytes,
                               int flags, void *stream) {
    return prefill_impl(layer, x, x_dtype, tokens, out, out_dtype, topk_ids, topk_weights, nullptr, ws, ws_bytes,
                        flags, SWQ_PREFILL_ALL, stream);
}

extern "C" int swq_moe_prefill_biased(const swq_moe_layer *layer, const void *x, int x_dtype, int tokens,
                                      void *out, int out_dtype, int32_t *topk_ids, float *topk_weights,
                                      const float *logit_bias, void *ws, size_t ws_bytes, int flags, void *stream) {
    if (!logit_bias) return SWQ_ERR_INVALID_ARGUMENT;
    return prefill_impl(layer, x, x_dtype, tokens, out, out_dtype, topk_ids, topk_weights, logit_bias, ws, ws_bytes,
                        flags, SWQ_PREFILL_ALL, stream);
}

extern "C" int swq_moe_prefill_stages(const swq_moe_layer *layer, const void *x, int x_dtype, int tokens, void *out,
                                      int out_dtype, int32_t *topk_ids, float *topk_weights,
                                      const float *logit_bias, void *ws, size_t ws_bytes, int flags, int stage_mask,
                                      void *stream) {
    return prefill_impl(layer, x, x_dtype, tokens, out, out_dtype, topk_ids, topk_weights, logit_bias, ws, ws_bytes,
                        flags, stage_mask, stream);
}
