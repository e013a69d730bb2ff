// Host-side helpers shared by the C ABI translation units: descriptor
// validation, QMat construction, workspace layout, HIP error mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/swq.h"
#include "common.hpp"

namespace swq {

inline int hip_status(hipError_t e) { return e == hipSuccess ? SWQ_OK : SWQ_ERR_HIP; }

inline int launch_status() { return hip_status(hipGetLastError()); }

inline int scale_bytes(int stype) { return stype == SWQ_F32 ? 4 : 2; }

inline int ilog2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
}

// Shape and dtype checks common to every path (Checkpoint.swift:170,
// MetalEngine.swift:105-111).
inline int check_linear_shape(const swq_qlinear *l) {
    if (!l || !l->w || !l->scales || !l->biases) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->reserved != 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->out_dim <= 0 || l->in_dim <= 0 || l->group_size <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->w_off < 0 || l->s_off < 0 || l->b_off < 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->expert_stride_w < 0 || l->expert_stride_sb < 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->bits != 2 && l->bits != 4 && l->bits != 8) return SWQ_ERR_UNSUPPORTED_BITS;
    if (l->scales_type < SWQ_F32 || l->scales_type > SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    const int per_word = 32 / l->bits;
    if (l->in_dim % l->group_size != 0) return SWQ_ERR_BAD_SHAPE;
    if (l->group_size % per_word != 0) return SWQ_ERR_BAD_SHAPE;
    return SWQ_OK;
}

// True when the vectorised (16-byte chunk) path can read this linear:
// 4/8-bit codes, groups spanning whole chunks, 16 B aligned rows and
// naturally aligned scales/biases.
inline bool vector_path_ok(const swq_qlinear *l, int64_t w_extra, int64_t s_extra, int64_t b_extra) {
    if (l->bits != 4 && l->bits != 8) return false;
    if ((static_cast<int64_t>(l->in_dim) * l->bits) % 128 != 0) return false;
    if ((static_cast<int64_t>(l->group_size) * l->bits) % 128 != 0) return false;
    const int cpg = static_cast<int>(static_cast<int64_t>(l->group_size) * l->bits / 128);
    if ((cpg & (cpg - 1)) != 0) return false;  // chunks per group: a power of two
    const uintptr_t w = reinterpret_cast<uintptr_t>(l->w) + l->w_off + w_extra;
    if (w % 16 != 0 || l->expert_stride_w % 16 != 0) return false;
    const int sb = scale_bytes(l->scales_type);
    const uintptr_t s = reinterpret_cast<uintptr_t>(l->scales) + l->s_off + s_extra;
    const uintptr_t b = reinterpret_cast<uintptr_t>(l->biases) + l->b_off + b_extra;
    if (s % sb != 0 || b % sb != 0 || l->expert_stride_sb % sb != 0) return false;
    return true;
}

// Lane plan of the vectorised path: each lane walks `cpl` 16-byte chunks of
// a row, and LPR = ceil(chunks / cpl) rounded up to a power of two (at most
// 64) lanes cover the row; lanes past its end idle.
inline int lpr_log2_for(int chunks, int cpl) {
    int lanes = (chunks + cpl - 1) / cpl;
    int l = 0;
    while ((1 << l) < lanes && l < 6) ++l;
    return l;
}

// Activation format and chunks per lane for a matrix read with x of dtype
// x_dtype: 4-bit codes with bf16 x take packed-bf16 dot products over 2
// chunks per lane (rows up to 4096 inputs); everything else fp32 fmas over one chunk per lane (two
// for 8-bit rows wider than 1024).
inline void plan_qmat(QMat *m, int x_dtype) {
    if (m->bits == 4 && x_dtype == SWQ_BF16) {
        m->xf = 1;
        m->cpl = 2;
    } else {
        m->xf = 0;
        m->cpl = m->chunks > 64 ? 2 : 1;
    }
    m->lpr_log2 = lpr_log2_for(m->chunks, m->cpl);
}

// Largest row (in 16-byte chunks) each plan accepts.
inline bool plan_fits(const QMat &m) {
    if (m.xf == 1) return m.chunks <= 2 * kWave;
    return m.chunks <= m.cpl * kWave && (m.bits == 8 || m.cpl == 1);
}

inline QMat make_qmat(const swq_qlinear *l, int64_t w_extra = 0, int64_t s_extra = 0,
                      int64_t b_extra = 0) {
    QMat m{};
    m.w = static_cast<const uint8_t *>(l->w) + l->w_off + w_extra;
    m.s = static_cast<const uint8_t *>(l->scales) + l->s_off + s_extra;
    m.b = static_cast<const uint8_t *>(l->biases) + l->b_off + b_extra;
    m.stride_w = l->expert_stride_w;
    m.stride_sb = l->expert_stride_sb;
    m.rows = l->out_dim;
    m.in = l->in_dim;
    m.group = l->group_size;
    m.bits = l->bits;
    m.stype = l->scales_type;
    m.row_bytes = static_cast<int32_t>(static_cast<int64_t>(l->in_dim) * l->bits / 8);
    m.gpr = l->in_dim / l->group_size;
    m.chunks = static_cast<int32_t>(static_cast<int64_t>(l->in_dim) * l->bits / 128);
    m.chunks_per_group = static_cast<int32_t>(static_cast<int64_t>(l->group_size) * l->bits / 128);
    plan_qmat(&m, SWQ_F32);
    m.cpg_log2 = m.chunks_per_group > 0 ? ilog2_exact(m.chunks_per_group) : 0;
    return m;
}

}  // namespace swq
