// Wave-level row tiles for the vectorised quantized GEMV paths.
//
// A wave computes dot products of RI*RPW weight rows with activation vectors
// held in registers.  Lane layout:  lane = q*LPR + j, where LPR ("lanes per
// row", a power of two <= 64) lanes cover one row and RPW = 64/LPR rows run
// side by side.  Lane j owns the CPL 16-byte chunks c = j + t*LPR (t < CPL)
// of its row and the activations of those chunks, so each load instruction
// reads LPR consecutive chunks per row.  RI = 4/CPL passes, so every lane
// holds four 16-byte code chunks per tile.
//
// Three activation formats:
//   kXF32    fp32 registers; codes go through v_cvt_f32_ubyteN and an fma.
//   kXBF16   (4-bit codes, bf16 activations) packed bf16 pairs; each nibble
//            becomes the bf16 value 128+q with one and-or, and
//            v_dot2c_f32_bf16 accumulates two exact products into fp32.  The
//            128 offset is removed through the bias:
//            s*q + b = s*(128+q) + (b - 128*s).
//   kXBF16X2 (4-bit codes, fp32 activations) each activation split into
//            hi = bf16(x) and lo = bf16(x - hi), both round-to-nearest-even,
//            so hi + lo carries 16 significant bits (relative error at most
//            2^-18); two dot2 per code pair, products still exact.
//
// Loads are branch-free: row and chunk indices are clamped to valid ones (the
// caller drops results of rows past the end; chunks past a row's end get zero
// scale and bias), and scales stay raw bits until every load of the tile is
// in flight.  A conversion or a branch between two loads would make the
// compiler wait for the first before issuing the second.
#pragma once

#include "common.hpp"

namespace swq {

constexpr int kXF32 = 0;
constexpr int kXBF16 = 1;
constexpr int kXBF16X2 = 2;

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

struct LaneMap {
    int lpr;     // lanes per row
    int lpr_log2;
    int rpw;     // rows per pass
    int q;       // row slot of this lane within a pass
    int j;       // lane index within the row
};

__device__ __forceinline__ LaneMap lane_map(int lpr_log2, int lane) {
    LaneMap m;
    m.lpr_log2 = lpr_log2;
    m.lpr = 1 << lpr_log2;
    m.rpw = kWave >> lpr_log2;
    m.q = lane >> lpr_log2;
    m.j = lane & (m.lpr - 1);
    return m;
}

// Rows one wave covers in one tile: 4/CPL passes of 64/LPR rows.
__host__ __device__ __forceinline__ int tile_rows(const QMat &m) { return (4 / m.cpl) * (kWave >> m.lpr_log2); }

// ---------------------------------------------------------------------------
// reductions over the LPR lanes of a row (DPP; the segment's last lane
// always holds the full sum, and for LPR <= 16 every lane does)

template <int CTRL, int ROW_MASK, bool BOUND_CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, BOUND_CTRL));
}

__device__ __forceinline__ float segment_reduce(float v, int lpr_log2) {
    if (lpr_log2 >= 1) v += dpp<0xB1, 0xF, true>(v);    // quad_perm [1,0,3,2]
    if (lpr_log2 >= 2) v += dpp<0x4E, 0xF, true>(v);    // quad_perm [2,3,0,1]
    if (lpr_log2 >= 3) v += dpp<0x141, 0xF, true>(v);   // row_half_mirror
    if (lpr_log2 >= 4) v += dpp<0x140, 0xF, true>(v);   // row_mirror
    if (lpr_log2 >= 5) v += dpp<0x142, 0xA, false>(v);  // row_bcast:15 into rows 1, 3
    if (lpr_log2 >= 6) v += dpp<0x143, 0x8, false>(v);  // row_bcast:31 into row 3
    return v;
}

// ---------------------------------------------------------------------------
// activations

template <int BITS, int CPL, int XF>
struct XSlice;

template <int BITS, int CPL>
struct XSlice<BITS, CPL, kXF32> {
    static constexpr int kCPC = codes_per_chunk<BITS>();
    float v[CPL][kCPC];
    float sum[CPL];
};

template <int CPL>
struct XSlice<4, CPL, kXBF16> {
    uint32_t p[CPL][16];  // pairs {x[8k+m], x[8k+m+4]} for word k, m = 0..3
    float sum[CPL];
};

template <int CPL>
struct XSlice<4, CPL, kXBF16X2> {
    uint32_t hi[CPL][16];  // pairs {hi[8k+m], hi[8k+m+4]} for word k, m = 0..3
    uint32_t lo[CPL][16];  // the same pairs of lo
    float sum[CPL];
};

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
}

typedef __attribute__((ext_vector_type(2))) float f32x2_t;

// hi = bf16(x0) | bf16(x1) << 16 and lo the same of the remainders
// x - float(hi), all round-to-nearest-even (v_cvt_pk_bf16_f32); the
// remainders are exact in fp32.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t &hi, uint32_t &lo) {
    const f32x2_t v = {x0, x1};
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    const f32x2_t r = {x0 - __uint_as_float(hi << 16), x1 - __uint_as_float(hi & 0xFFFF0000u)};
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf16x2_t));
}

// Sum of a 4-bit chunk's activations from its pair words, in a fixed order
// (every path that holds the same pairs gets the same sum).
__device__ __forceinline__ float pair_sum(const uint32_t *hi, const uint32_t *lo) {
    float s[4] = {0.f, 0.f, 0.f, 0.f}, t[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            s[m] = dot2_bf16(hi[4 * k + m], 0x3F803F80u, s[m]);
            t[m] = dot2_bf16(lo[4 * k + m], 0x3F803F80u, t[m]);
        }
    }
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((t[0] + t[1]) + (t[2] + t[3]));
}

// 32 fp32 activations of a 4-bit chunk -> pair words {x[8k+m], x[8k+m+4]}
// (word 4k+m) of hi and lo, and the chunk's sum.
__device__ __forceinline__ void pack_chunk_x2(const float *v, uint32_t *hi, uint32_t *lo, float &sum) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int m = 0; m < 4; ++m) split_pair(v[8 * k + m], v[8 * k + m + 4], hi[4 * k + m], lo[4 * k + m]);
    }
    sum = pair_sum(hi, lo);
}

// (v & mask) | magic in one VOP3 (the compiler otherwise emits two VOP2s
// with literal operands).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(mask), "v"(magic));
    return r;
}

// The raw activation words of a lane's chunks: loads only.  A phase that
// issues all its loads (weights, then these) before converting anything has
// every load in flight at once; a conversion right after its loads would
// make the compiler wait for them before the next load issues.
template <int XDT, int BITS, int CPL>
struct XRaw {
    static constexpr int kCPC = codes_per_chunk<BITS>();
    static constexpr int kN = XDT == 2 ? kCPC / 8 : kCPC / 4;  // 16-byte words per chunk
    uint4 r[CPL][kN];
};

template <int XDT, int BITS, int CPL>
__device__ __forceinline__ void load_xraw(XRaw<XDT, BITS, CPL> &xr, const QMat &m, const LaneMap &lm, const void *x,
                                          int64_t x_base) {
    constexpr int kCPC = codes_per_chunk<BITS>(), kN = XRaw<XDT, BITS, CPL>::kN;
    constexpr int kES = XDT == 2 ? 2 : 4;
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
        const int c = min(lm.j + t * lm.lpr, m.chunks - 1);
        const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(x) +
                                                         (x_base + static_cast<int64_t>(c) * kCPC) * kES);
#pragma unroll
        for (int k = 0; k < kN; ++k) xr.r[t][k] = p[k];
    }
}

// The activation slice from its raw words (the same values and sums as
// reading x directly).
template <int XDT, int BITS, int CPL, int XF>
__device__ __forceinline__ void xslice_convert(XSlice<BITS, CPL, XF> &xs, const XRaw<XDT, BITS, CPL> &xr) {
    constexpr int kCPC = codes_per_chunk<BITS>();
    if constexpr (XF == kXBF16) {
        static_assert(XDT == 2 && BITS == 4, "packed bf16 activations need bf16 x and 4-bit codes");
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            float s[4] = {0.f, 0.f, 0.f, 0.f};  // independent chains
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t d0 = xr.r[t][k].x, d1 = xr.r[t][k].y, d2 = xr.r[t][k].z, d3 = xr.r[t][k].w;
                xs.p[t][4 * k + 0] = (d0 & 0xFFFFu) | (d2 << 16);
                xs.p[t][4 * k + 1] = (d0 >> 16) | (d2 & 0xFFFF0000u);
                xs.p[t][4 * k + 2] = (d1 & 0xFFFFu) | (d3 << 16);
                xs.p[t][4 * k + 3] = (d1 >> 16) | (d3 & 0xFFFF0000u);
#pragma unroll
                for (int mm = 0; mm < 4; ++mm) s[mm] = dot2_bf16(xs.p[t][4 * k + mm], 0x3F803F80u, s[mm]);
            }
            xs.sum[t] = (s[0] + s[1]) + (s[2] + s[3]);
        }
    } else {
        float v[CPL][kCPC];
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
#pragma unroll
            for (int k = 0; k < XRaw<XDT, BITS, CPL>::kN; ++k) {
                const uint32_t u[4] = {xr.r[t][k].x, xr.r[t][k].y, xr.r[t][k].z, xr.r[t][k].w};
                if constexpr (XDT == 2) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        v[t][8 * k + 2 * i] = __uint_as_float(u[i] << 16);
                        v[t][8 * k + 2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[t][4 * k + i] = __uint_as_float(u[i]);
                }
            }
        }
        if constexpr (XF == kXF32) {
#pragma unroll
            for (int t = 0; t < CPL; ++t) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < kCPC; ++i) {
                    xs.v[t][i] = v[t][i];
                    s += v[t][i];
                }
                xs.sum[t] = s;
            }
        } else {
            static_assert(XDT == 0 && BITS == 4, "split bf16 activations need fp32 x and 4-bit codes");
#pragma unroll
            for (int t = 0; t < CPL; ++t) pack_chunk_x2(v[t], xs.hi[t], xs.lo[t], xs.sum[t]);
        }
    }
}

template <int XDT, int BITS, int CPL, int XF>
__device__ __forceinline__ void load_xslice(XSlice<BITS, CPL, XF> &xs, const QMat &m, const LaneMap &lm,
                                            const void *x, int64_t x_base) {
    XRaw<XDT, BITS, CPL> xr;
    load_xraw<XDT>(xr, m, lm, x, x_base);
    xslice_convert(xs, xr);
}

// sum_i (128 + q_i) * x_i over a chunk of 4-bit codes with packed bf16 pairs.
__device__ __forceinline__ float dot_chunk_q4_bf16(const uint4 w, const uint32_t *xp) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float a0 = 0.f, a1 = 0.f;  // two independent chains
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t v = ws[k];
        a0 = dot2_bf16(and_or(v, 0x000F000Fu, 0x43004300u), xp[4 * k + 0], a0);          // {q0, q4}
        a1 = dot2_bf16(and_or(v >> 4, 0x000F000Fu, 0x43004300u), xp[4 * k + 1], a1);   // {q1, q5}
        a0 = dot2_bf16(and_or(v >> 8, 0x000F000Fu, 0x43004300u), xp[4 * k + 2], a0);   // {q2, q6}
        a1 = dot2_bf16(and_or(v >> 12, 0x000F000Fu, 0x43004300u), xp[4 * k + 3], a1);  // {q3, q7}
    }
    return a0 + a1;
}

// sum_i (128 + q_i) * (hi_i + lo_i) over a chunk of 4-bit codes.
__device__ __forceinline__ float dot_chunk_q4_bf16x2(const uint4 w, const uint32_t *hi, const uint32_t *lo) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;  // four independent chains
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t v = ws[k];
        const uint32_t c0 = and_or(v, 0x000F000Fu, 0x43004300u);        // {q0, q4}
        const uint32_t c1 = and_or(v >> 4, 0x000F000Fu, 0x43004300u);   // {q1, q5}
        const uint32_t c2 = and_or(v >> 8, 0x000F000Fu, 0x43004300u);   // {q2, q6}
        const uint32_t c3 = and_or(v >> 12, 0x000F000Fu, 0x43004300u);  // {q3, q7}
        a0 = dot2_bf16(c0, hi[4 * k + 0], a0);
        a1 = dot2_bf16(c1, hi[4 * k + 1], a1);
        b0 = dot2_bf16(c0, lo[4 * k + 0], b0);
        b1 = dot2_bf16(c1, lo[4 * k + 1], b1);
        a0 = dot2_bf16(c2, hi[4 * k + 2], a0);
        a1 = dot2_bf16(c3, hi[4 * k + 3], a1);
        b0 = dot2_bf16(c2, lo[4 * k + 2], b0);
        b1 = dot2_bf16(c3, lo[4 * k + 3], b1);
    }
    return (a0 + a1) + (b0 + b1);
}

// ---------------------------------------------------------------------------
// weights

// Codes plus raw scale/bias bits of RI passes of rows (row0 + i*rpw + q).
// ES is the byte size of a scale element: 2 (f16, bf16) or 4 (f32).  RI
// defaults to 4/CPL passes (four 16-byte code chunks per lane).
template <int BITS, int CPL, int ES, int RI_ = 4 / CPL>
struct RowTile {
    static constexpr int kRI = RI_;
    uint4 w[kRI][CPL];
    uint32_t s[kRI][CPL];
    uint32_t b[kRI][CPL];
};

template <int ES>
__device__ __forceinline__ uint32_t load_scale_raw(const uint8_t *base, int64_t idx) {
    if constexpr (ES == 2) return *reinterpret_cast<const uint16_t *>(base + idx * 2);
    else return *reinterpret_cast<const uint32_t *>(base + idx * 4);
}

template <int ES>
__device__ __forceinline__ float scale_value(uint32_t raw, int stype) {
    if constexpr (ES == 4) {
        return __uint_as_float(raw);
    } else {
        const float h = f16_to_f32(static_cast<uint16_t>(raw));
        const float bf = __uint_as_float(raw << 16);
        return stype == 1 ? h : bf;
    }
}

template <int BITS, int CPL, int ES, int RI_>
__device__ __forceinline__ void load_tile(RowTile<BITS, CPL, ES, RI_> &rt, const QMat &m, int64_t expert,
                                          const LaneMap &lm, int row0, int row_end) {
    constexpr int RI = RI_;
    const uint8_t *wbase = m.w + expert * m.stride_w;
    const uint8_t *sbase = m.s + expert * m.stride_sb;
    const uint8_t *bbase = m.b + expert * m.stride_sb;
    int cc[CPL], gg[CPL];
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
        cc[t] = min(lm.j + t * lm.lpr, m.chunks - 1);
        gg[t] = cc[t] >> m.cpg_log2;  // group of the chunk
    }
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        const int row = min(row0 + i * lm.rpw + lm.q, row_end - 1);
        const uint8_t *wr = wbase + static_cast<int64_t>(row) * m.row_bytes;
        const int64_t g0 = static_cast<int64_t>(row) * m.gpr;
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            rt.w[i][t] = *reinterpret_cast<const uint4 *>(wr + static_cast<int64_t>(cc[t]) * 16);
            rt.s[i][t] = load_scale_raw<ES>(sbase, g0 + gg[t]);
            rt.b[i][t] = load_scale_raw<ES>(bbase, g0 + gg[t]);
        }
    }
}

// res[i] = full dot product of row (row0 + i*rpw + q) with the activations,
// valid in the row segment's last lane (j == LPR-1).
//
// The empty asm statements keep the code unpacking inside the caller's token
// loop: hoisted out of it, the unpacked codes of a tile would stay live
// across the loop and spill.  They all come first, so the passes' arithmetic
// that follows can interleave.
template <int BITS, int CPL, int ES, int XF, int RI_>
__device__ __forceinline__ void dot_tile(float (&res)[RI_], const RowTile<BITS, CPL, ES, RI_> &rt,
                                         const XSlice<BITS, CPL, XF> &xs, const QMat &m, const LaneMap &lm) {
    constexpr int RI = RI_;
    uint4 wt[RI][CPL];
#pragma unroll
    for (int i = 0; i < RI; ++i) {
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            wt[i][t] = rt.w[i][t];
            asm volatile("" : "+v"(wt[i][t].x), "+v"(wt[i][t].y), "+v"(wt[i][t].z), "+v"(wt[i][t].w));
        }
    }
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            const uint4 w = wt[i][t];
            const bool live = lm.j + t * lm.lpr < m.chunks;
            const float sc = live ? scale_value<ES>(rt.s[i][t], m.stype) : 0.f;
            const float bi = live ? scale_value<ES>(rt.b[i][t], m.stype) : 0.f;
            if constexpr (XF == kXF32) {
                const float qd = dot_chunk<BITS>(w, xs.v[t]);
                acc = fmaf(sc, qd, acc);
                acc = fmaf(bi, xs.sum[t], acc);
            } else if constexpr (XF == kXBF16) {
                const float d = dot_chunk_q4_bf16(w, xs.p[t]);
                acc = fmaf(sc, d, acc);
                acc = fmaf(fmaf(-128.f, sc, bi), xs.sum[t], acc);
            } else {
                const float d = dot_chunk_q4_bf16x2(w, xs.hi[t], xs.lo[t]);
                acc = fmaf(sc, d, acc);
                acc = fmaf(fmaf(-128.f, sc, bi), xs.sum[t], acc);
            }
        }
        res[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < RI; ++i) res[i] = segment_reduce(res[i], lm.lpr_log2);
}


// ---------------------------------------------------------------------------
// dot products of NT tiles (one activation slice) with the code words of all
// their chunks interleaved: word k of every chunk before word k + 1 of any,
// so the unpack -> dot chains of different chunks overlap.  A kernel with a
// single wave per SIMD has no other wave to fill the issue slots a chain of
// dependent instructions leaves; with 8-32 independent chains they fill
// themselves.  Each chunk's own summation order is dot_chunk*'s, and the
// per-row combination is dot_tile's, so results equal dot_tile's bit for bit.

template <int BITS, int CPL, int XF, int N>
__device__ __forceinline__ void chunk_dots(float (&d)[N], const uint4 (&w)[N], const XSlice<BITS, CPL, XF> &xs) {
    if constexpr (XF == kXBF16) {
        float a0[N], a1[N];
#pragma unroll
        for (int n = 0; n < N; ++n) a0[n] = a1[n] = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const uint32_t *xp = xs.p[n % CPL];
                const uint32_t v = k == 0 ? w[n].x : k == 1 ? w[n].y : k == 2 ? w[n].z : w[n].w;
                const uint32_t c0 = and_or(v, 0x000F000Fu, 0x43004300u);        // {q0, q4}
                const uint32_t c1 = and_or(v >> 4, 0x000F000Fu, 0x43004300u);   // {q1, q5}
                const uint32_t c2 = and_or(v >> 8, 0x000F000Fu, 0x43004300u);   // {q2, q6}
                const uint32_t c3 = and_or(v >> 12, 0x000F000Fu, 0x43004300u);  // {q3, q7}
                a0[n] = dot2_bf16(c0, xp[4 * k + 0], a0[n]);
                a1[n] = dot2_bf16(c1, xp[4 * k + 1], a1[n]);
                a0[n] = dot2_bf16(c2, xp[4 * k + 2], a0[n]);
                a1[n] = dot2_bf16(c3, xp[4 * k + 3], a1[n]);
            }
        }
#pragma unroll
        for (int n = 0; n < N; ++n) d[n] = a0[n] + a1[n];
    } else if constexpr (XF == kXBF16X2) {
        float a0[N], a1[N], b0[N], b1[N];
#pragma unroll
        for (int n = 0; n < N; ++n) a0[n] = a1[n] = b0[n] = b1[n] = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const uint32_t *hi = xs.hi[n % CPL], *lo = xs.lo[n % CPL];
                const uint32_t v = k == 0 ? w[n].x : k == 1 ? w[n].y : k == 2 ? w[n].z : w[n].w;
                const uint32_t c0 = and_or(v, 0x000F000Fu, 0x43004300u);
                const uint32_t c1 = and_or(v >> 4, 0x000F000Fu, 0x43004300u);
                const uint32_t c2 = and_or(v >> 8, 0x000F000Fu, 0x43004300u);
                const uint32_t c3 = and_or(v >> 12, 0x000F000Fu, 0x43004300u);
                a0[n] = dot2_bf16(c0, hi[4 * k + 0], a0[n]);
                a1[n] = dot2_bf16(c1, hi[4 * k + 1], a1[n]);
                b0[n] = dot2_bf16(c0, lo[4 * k + 0], b0[n]);
                b1[n] = dot2_bf16(c1, lo[4 * k + 1], b1[n]);
                a0[n] = dot2_bf16(c2, hi[4 * k + 2], a0[n]);
                a1[n] = dot2_bf16(c3, hi[4 * k + 3], a1[n]);
                b0[n] = dot2_bf16(c2, lo[4 * k + 2], b0[n]);
                b1[n] = dot2_bf16(c3, lo[4 * k + 3], b1[n]);
            }
        }
#pragma unroll
        for (int n = 0; n < N; ++n) d[n] = (a0[n] + a1[n]) + (b0[n] + b1[n]);
    } else if constexpr (BITS == 8) {
        // dot_chunk_q8: acc[k] over the bytes of word k in order
        float acc[N][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const float *x = xs.v[n % CPL];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t v = k == 0 ? w[n].x : k == 1 ? w[n].y : k == 2 ? w[n].z : w[n].w;
                    acc[n][k] = j == 0 ? ubyte(v, 0) * x[4 * k] : fmaf(ubyte(v, j), x[4 * k + j], acc[n][k]);
                }
            }
        }
#pragma unroll
        for (int n = 0; n < N; ++n) d[n] = (acc[n][0] + acc[n][1]) + (acc[n][2] + acc[n][3]);
    } else {
        // dot_chunk_q4: acc[k] over the nibbles of word k, low byte lane
        // nibbles (0, 2, 4, 6) and high ones (1, 3, 5, 7) alternating
        float acc[N][4];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int n = 0; n < N; ++n) {
                const float *x = xs.v[n % CPL];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t v = k == 0 ? w[n].x : k == 1 ? w[n].y : k == 2 ? w[n].z : w[n].w;
                    const uint32_t nib = (j & 1) ? (v >> 4) & 0x0F0F0F0Fu : v & 0x0F0F0F0Fu;
                    const float q = ubyte(nib, j >> 1);
                    acc[n][k] = j == 0 ? q * x[8 * k] : fmaf(q, x[8 * k + j], acc[n][k]);
                }
            }
        }
#pragma unroll
        for (int n = 0; n < N; ++n) d[n] = (acc[n][0] + acc[n][1]) + (acc[n][2] + acc[n][3]);
    }
}

// res[u][i]: the full dot product of row (row0 + i*rpw + q) of tile u with
// the activations, valid in the row segment's last lane (as dot_tile).
template <int NT, int BITS, int CPL, int ES, int XF, int RI>
__device__ __forceinline__ void dot_tiles(float (&res)[NT][RI], const RowTile<BITS, CPL, ES, RI> *const (&rt)[NT],
                                          const QMat *const (&m)[NT], const XSlice<BITS, CPL, XF> &xs,
                                          const LaneMap &lm) {
    constexpr int N = NT * RI * CPL;  // chunk n = (u*RI + i)*CPL + t
    uint4 w[N];
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
        for (int i = 0; i < RI; ++i)
#pragma unroll
            for (int t = 0; t < CPL; ++t) w[(u * RI + i) * CPL + t] = rt[u]->w[i][t];
    float d[N];
    chunk_dots<BITS, CPL, XF, N>(d, w, xs);
#pragma unroll
    for (int u = 0; u < NT; ++u) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            float acc = 0.f;
#pragma unroll
            for (int t = 0; t < CPL; ++t) {
                const bool live = lm.j + t * lm.lpr < m[u]->chunks;
                const float sc = live ? scale_value<ES>(rt[u]->s[i][t], m[u]->stype) : 0.f;
                const float bi = live ? scale_value<ES>(rt[u]->b[i][t], m[u]->stype) : 0.f;
                const float dd = d[(u * RI + i) * CPL + t];
                if constexpr (XF == kXF32) {
                    acc = fmaf(sc, dd, acc);
                    acc = fmaf(bi, xs.sum[t], acc);
                } else {
                    acc = fmaf(sc, dd, acc);
                    acc = fmaf(fmaf(-128.f, sc, bi), xs.sum[t], acc);
                }
            }
            res[u][i] = segment_reduce(acc, lm.lpr_log2);
        }
    }
}

}  // namespace swq
