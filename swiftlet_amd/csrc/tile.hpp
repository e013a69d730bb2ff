// Wave-level row tiles for the vectorised quantized GEMV paths.
//
// A wave computes dot products of up to RI*RPW weight rows with activation
// vectors held in registers.  Lane layout:  lane = q*LPR + j, where LPR
// ("lanes per row", a power of two <= 64) lanes cover one row and RPW =
// 64/LPR rows run side by side.  Lane j of a row owns the 16-byte chunks
// c = j + t*LPR (t < CPL) of that row, and the activations of those chunks.
//
// Loads are branch-free: row and chunk indices are clamped to valid ones
// (the caller drops results of rows past the end; chunks past a row's end
// get zero scale and bias), and scales are kept as raw bits until every load
// of the tile is in flight.  A conversion or a branch between two loads
// would make the compiler wait for the first before issuing the second.
#pragma once

#include "common.hpp"

namespace swq {

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

// Activations of this lane's chunks (fp32 registers) plus their sums.
template <int BITS, int CPL>
struct XSlice {
    static constexpr int kCPC = codes_per_chunk<BITS>();
    float v[CPL][kCPC];
    float sum[CPL];
};

template <int XDT, int BITS, int CPL>
__device__ __forceinline__ void load_xslice(XSlice<BITS, CPL> &xs, const QMat &m, const LaneMap &lm,
                                            const void *x, int64_t x_base) {
    constexpr int kCPC = codes_per_chunk<BITS>();
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
        const int c = min(lm.j + t * lm.lpr, m.chunks - 1);
        load_x<XDT>(xs.v[t], x, x_base + static_cast<int64_t>(c) * kCPC);
    }
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < kCPC; ++i) s += xs.v[t][i];
        xs.sum[t] = s;
    }
}

// Codes plus raw scale/bias bits of RI passes of rows (row0 + i*rpw + q).
// ES is the byte size of a scale element: 2 (f16, bf16) or 4 (f32).
template <int BITS, int CPL, int RI, int ES>
struct RowTile {
    uint4 w[RI][CPL];
    uint32_t s[RI][CPL];
    uint32_t b[RI][CPL];
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

template <int BITS, int CPL, int RI, int ES>
__device__ __forceinline__ void load_tile(RowTile<BITS, CPL, RI, ES> &rt, const QMat &m, int64_t expert,
                                          const LaneMap &lm, int row0, int row_end) {
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

// res[i] = full dot product of row (row0 + i*rpw + q) with the activations;
// every lane of the row's segment receives it.
//
// The empty asm keeps the code unpacking inside the caller's token loop:
// hoisted out of it, the unpacked codes of a tile (32 floats per chunk)
// would stay live across the loop and spill.
template <int BITS, int CPL, int RI, int ES>
__device__ __forceinline__ void dot_tile(float (&res)[RI], const RowTile<BITS, CPL, RI, ES> &rt,
                                         const XSlice<BITS, CPL> &xs, const QMat &m, const LaneMap &lm) {
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            uint4 w = rt.w[i][t];
            asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w));
            const bool live = lm.j + t * lm.lpr < m.chunks;
            const float sc = live ? scale_value<ES>(rt.s[i][t], m.stype) : 0.f;
            const float bi = live ? scale_value<ES>(rt.b[i][t], m.stype) : 0.f;
            const float qd = dot_chunk<BITS>(w, xs.v[t]);
            acc = fmaf(sc, qd, acc);
            acc = fmaf(bi, xs.sum[t], acc);
        }
        res[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < RI; ++i) res[i] = segment_sum(res[i], lm.lpr);
}

}  // namespace swq
