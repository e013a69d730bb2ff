// Wave-level row tiles for the vectorised quantized GEMV paths.
//
// A wave computes dot products of up to RI*RPW weight rows with activation
// vectors held in registers.  Lane layout:  lane = q*LPR + j, where LPR
// ("lanes per row", a power of two <= 64) lanes cover one row and RPW =
// 64/LPR rows run side by side.  Lane j of a row owns the 16-byte chunks
// c = j + t*LPR (t < CPL) of that row, and the activations of those chunks.
// All weight loads of a tile are issued before any of them is consumed, so
// a wave keeps RI*CPL 16-byte loads in flight.
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
        const int c = lm.j + t * lm.lpr;
        if (c < m.chunks) {
            load_x<XDT>(xs.v[t], x, x_base + static_cast<int64_t>(c) * kCPC);
        } else {
#pragma unroll
            for (int i = 0; i < kCPC; ++i) xs.v[t][i] = 0.f;
        }
    }
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < kCPC; ++i) s += xs.v[t][i];
        xs.sum[t] = s;
    }
}

// Codes, scales and biases of RI passes of rows (rows row0 + i*rpw + q).
template <int BITS, int CPL, int RI>
struct RowTile {
    uint4 w[RI][CPL];
    float s[RI][CPL];
    float b[RI][CPL];
};

template <int BITS, int CPL, int RI>
__device__ __forceinline__ void load_tile(RowTile<BITS, CPL, RI> &rt, const QMat &m, int64_t expert,
                                          const LaneMap &lm, int row0, int row_end) {
    const uint8_t *wbase = m.w + expert * m.stride_w;
    const uint8_t *sbase = m.s + expert * m.stride_sb;
    const uint8_t *bbase = m.b + expert * m.stride_sb;
    constexpr int kCPC = codes_per_chunk<BITS>();
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        const int row = row0 + i * lm.rpw + lm.q;
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            const int c = lm.j + t * lm.lpr;
            if (row < row_end && c < m.chunks) {
                rt.w[i][t] = *reinterpret_cast<const uint4 *>(
                    wbase + static_cast<int64_t>(row) * m.row_bytes + static_cast<int64_t>(c) * 16);
                const int64_t gi = static_cast<int64_t>(row) * m.gpr + (c * kCPC) / m.group;
                rt.s[i][t] = load_scale(sbase, gi, m.stype);
                rt.b[i][t] = load_scale(bbase, gi, m.stype);
            } else {
                rt.w[i][t] = make_uint4(0u, 0u, 0u, 0u);
                rt.s[i][t] = 0.f;
                rt.b[i][t] = 0.f;
            }
        }
    }
}

// res[i] = full dot product of row (row0 + i*rpw + q) with the activations;
// every lane of the row's segment receives it.
//
// The empty asm keeps the code unpacking inside the caller's token loop:
// hoisted out of it, the unpacked codes of a tile (32 floats per chunk)
// would stay live across the loop and spill.
template <int BITS, int CPL, int RI>
__device__ __forceinline__ void dot_tile(float (&res)[RI], const RowTile<BITS, CPL, RI> &rt,
                                         const XSlice<BITS, CPL> &xs, const LaneMap &lm) {
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
            uint4 w = rt.w[i][t];
            asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w));
            const float qd = dot_chunk<BITS>(w, xs.v[t]);
            acc = fmaf(rt.s[i][t], qd, acc);
            acc = fmaf(rt.b[i][t], xs.sum[t], acc);
        }
        res[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < RI; ++i) res[i] = segment_sum(res[i], lm.lpr);
}

}  // namespace swq
