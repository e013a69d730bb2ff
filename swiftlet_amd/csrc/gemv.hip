// Quantized GEMV, SwiGLU and dequantisation entry points: the operator
// layer of MetalEngine (MetalEngine.swift:95-232) and Checkpoint's MLX
// affine dequantisation (Checkpoint.swift:168-209), on gfx950.
#include <algorithm>
#include <vector>

#include "internal.hpp"
#include "tile.hpp"

namespace swq {

constexpr int kGemvThreads = 256;

// Vectorised GEMV over fp32 activations: each wave loads its slice of x once
// and walks tiles of rows (4/CPL passes of 64/LPR rows) t, t + W, t + 2W, ...
// (W: the grid's waves), the loads of the next two tiles in flight while the
// current tile's dot products run (a wave-uniform branch skips prefetches
// past the last tile).
constexpr int kGemvMaxBlocks = 1024;  // 4096 waves: 16 per CU

// x (at most kStageMaxIn floats) goes through LDS once per workgroup: each
// thread loads a few 16-byte words of it (and, with NORM, the matching norm
// weights), the RMSNorm's sum of squares is one workgroup reduction, each
// thread normalises its own words (x * (scale * w), the product order of
// QwenCPUModel.rmsNorm), and the waves read their slices from LDS instead
// of each reading all of x (and the weights) from L2: with a wave per 4-row
// tile they would otherwise read them ~4 times as often as the workgroup.
// In LDS, chunk c's 16-byte pieces are rotated by c (piece p at slot
// (p + c) mod P) so the lanes of a wave, which read one chunk each, spread
// over the banks.  `issue` runs between the loads of x and the first wait
// for them: the caller's weight-tile loads go there, since loads complete
// in issue order.  Every thread of the workgroup must call this.
constexpr int kStageMaxIn = 4096;
constexpr int kStageWords = kStageMaxIn / 4 / kGemvThreads;  // 16-byte words of x per thread

struct StagedX {
    uint4 x[kStageMaxIn / 4];
    float red[kGemvThreads / kWave];
};

template <int BITS, bool NORM, typename Issue>
__device__ __forceinline__ void stage_x(StagedX &L, const float *x, int in, const void *norm_w, int norm_dtype,
                                        float eps, Issue issue) {
    constexpr int kP = codes_per_chunk<BITS>() / 4;  // 16-byte words of x per chunk
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int nx = in / 4;
    const uint4 *x4 = reinterpret_cast<const uint4 *>(x);
    uint4 xw[kStageWords], ww[NORM ? kStageWords : 1];
    // every load unconditional (indices clamped; the repeats hit lines
    // already requested): branches around them measured slower
#pragma unroll
    for (int k = 0; k < kStageWords; ++k) xw[k] = x4[min(k * kGemvThreads + tid, nx - 1)];
    if constexpr (NORM) {
        if (norm_dtype == SWQ_F32) {
            const uint4 *w4 = static_cast<const uint4 *>(norm_w);
#pragma unroll
            for (int k = 0; k < kStageWords; ++k) ww[k] = w4[min(k * kGemvThreads + tid, nx - 1)];
        } else {
            const uint2 *w2 = static_cast<const uint2 *>(norm_w);
#pragma unroll
            for (int k = 0; k < kStageWords; ++k) {
                const uint2 r = w2[min(k * kGemvThreads + tid, nx - 1)];
                ww[k] = make_uint4(r.x, r.y, 0u, 0u);
            }
        }
    }
    issue();
    float sc = 1.f;
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < kStageWords; ++k) {
            if (k * kGemvThreads + tid < nx) {
                const float4 v = __builtin_bit_cast(float4, xw[k]);
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) L.red[wave] = ss;
        lds_barrier();
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < kGemvThreads / kWave; ++i) tot += L.red[i];
        sc = 1.0f / __fsqrt_rn(tot / static_cast<float>(in) + eps);
    }
#pragma unroll
    for (int k = 0; k < kStageWords; ++k) {
        const int i = k * kGemvThreads + tid;
        if (i < nx) {
            float4 v = __builtin_bit_cast(float4, xw[k]);
            if constexpr (NORM) {
                float w[4];
                if (norm_dtype == SWQ_F32) {
                    const float4 wf = __builtin_bit_cast(float4, ww[k]);
                    w[0] = wf.x;
                    w[1] = wf.y;
                    w[2] = wf.z;
                    w[3] = wf.w;
                } else {
                    const uint32_t h[4] = {ww[k].x & 0xFFFFu, ww[k].x >> 16, ww[k].y & 0xFFFFu, ww[k].y >> 16};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint16_t raw = static_cast<uint16_t>(h[e]);
                        w[e] = norm_dtype == SWQ_BF16 ? bf16_to_f32(raw) : f16_to_f32(raw);
                    }
                }
                v.x *= sc * w[0];
                v.y *= sc * w[1];
                v.z *= sc * w[2];
                v.w *= sc * w[3];
            }
            const int c = i / kP, p = i - c * kP;
            L.x[c * kP + ((p + c) & (kP - 1))] = __builtin_bit_cast(uint4, v);
        }
    }
    lds_barrier();
}

// The wave's slice of the staged x, with its chunk sums formed as
// load_xslice forms them (so results equal those from x read directly).
template <int BITS, int CPL>
__device__ __forceinline__ void xslice_from_lds(XSlice<BITS, CPL, kXF32> &xs, const StagedX &L, const QMat &m,
                                                const LaneMap &lm) {
    constexpr int kCPC = codes_per_chunk<BITS>(), kP = kCPC / 4;
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
        const int c = min(lm.j + u * lm.lpr, m.chunks - 1);
#pragma unroll
        for (int p = 0; p < kP; ++p) {
            const float4 v = __builtin_bit_cast(float4, L.x[c * kP + ((p + c) & (kP - 1))]);
            xs.v[u][4 * p + 0] = v.x;
            xs.v[u][4 * p + 1] = v.y;
            xs.v[u][4 * p + 2] = v.z;
            xs.v[u][4 * p + 3] = v.w;
        }
    }
#pragma unroll
    for (int u = 0; u < CPL; ++u) {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < kCPC; ++i) sum += xs.v[u][i];
        xs.sum[u] = sum;
    }
}

template <int BITS, int CPL, int ES>
__global__ __launch_bounds__(kGemvThreads) void gemv_vec_kernel(QMat m, int rows, const float *x, float *y) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    const int tile_rows = RI * lm.rpw;
    const int ntiles = (rows + tile_rows - 1) / tile_rows;
    const int nw = gridDim.x * (kGemvThreads / kWave);
    int t = blockIdx.x * (kGemvThreads / kWave) + wave;
    __shared__ StagedX L;
    RowTile<BITS, CPL, ES> cur, next, next2;
    stage_x<BITS, false>(L, x, m.in, nullptr, 0, 0.f, [&] {
        if (t < ntiles) load_tile(cur, m, 0, lm, t * tile_rows, rows);
        if (t + nw < ntiles) load_tile(next, m, 0, lm, (t + nw) * tile_rows, rows);
    });
    if (t >= ntiles) return;  // after the staging, which every wave takes part in
    XSlice<BITS, CPL, kXF32> xs;
    xslice_from_lds(xs, L, m, lm);
    for (;;) {
        const int tn = t + nw;
        if (tn + nw < ntiles) load_tile(next2, m, 0, lm, (tn + nw) * tile_rows, rows);
        float res[RI];
        dot_tile(res, cur, xs, m, lm);
        if (lm.j == lm.lpr - 1) {
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                const int row = t * tile_rows + i * lm.rpw + lm.q;
                if (row < rows) y[row] = res[i];
            }
        }
        if (tn >= ntiles) break;
        cur = next;
        next = next2;
        t = tn;
    }
}

// Several matrices with one input and one lane plan (same in_dim, bits,
// group, scale dtype) in one launch: their row tiles are numbered
// consecutively (matrix i owns tiles [tile_end[i-1], tile_end[i])) and the
// waves walk them as gemv_vec_kernel walks one matrix.  With NORM the input
// is h, and the staging turns it into rmsnorm(h) * w in LDS.
constexpr int kMultiMax = 4;

struct MultiArgs {
    QMat m;  // the shared plan (pointers of matrix 0)
    const uint8_t *w[kMultiMax], *s[kMultiMax], *b[kMultiMax];
    float *y[kMultiMax];
    int32_t rows[kMultiMax];
    int32_t tile_end[kMultiMax];
    int32_t n;
    int32_t norm_dtype;
    const float *x;
    const void *norm_w;
    float eps;
};

template <int BITS, int CPL, int ES, bool NORM>
__global__ __launch_bounds__(kGemvThreads) void gemv_multi_kernel(const MultiArgs a) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    __shared__ StagedX L;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const LaneMap lm = lane_map(a.m.lpr_log2, lane);
    const int tile_rows = RI * lm.rpw;
    const int ntiles = a.tile_end[a.n - 1];
    const int nw = gridDim.x * (kGemvThreads / kWave);
    int t = blockIdx.x * (kGemvThreads / kWave) + wave;
    auto mat_of = [&](int tt) {
        int i = 0;
        while (i + 1 < a.n && tt >= a.tile_end[i]) ++i;
        return i;
    };
    auto qmat = [&](int i) {
        QMat q = a.m;
        q.w = a.w[i];
        q.s = a.s[i];
        q.b = a.b[i];
        return q;
    };
    auto row0_of = [&](int tt, int i) { return (tt - (i ? a.tile_end[i - 1] : 0)) * tile_rows; };
    RowTile<BITS, CPL, ES> cur, next, next2;
    int mc = 0;
    stage_x<BITS, NORM>(L, a.x, a.m.in, a.norm_w, a.norm_dtype, a.eps, [&] {
        if (t < ntiles) {
            mc = mat_of(t);
            load_tile(cur, qmat(mc), 0, lm, row0_of(t, mc), a.rows[mc]);
        }
        if (t + nw < ntiles) {
            const int tn1 = t + nw, mn1 = mat_of(tn1);
            load_tile(next, qmat(mn1), 0, lm, row0_of(tn1, mn1), a.rows[mn1]);
        }
    });
    if (t >= ntiles) return;  // after the staging, which every wave takes part in
    XSlice<BITS, CPL, kXF32> xs;
    xslice_from_lds(xs, L, a.m, lm);
    for (;;) {
        const int tn = t + nw;
        if (tn + nw < ntiles) {
            const int tn2 = tn + nw, mn2 = mat_of(tn2);
            load_tile(next2, qmat(mn2), 0, lm, row0_of(tn2, mn2), a.rows[mn2]);
        }
        float res[RI];
        dot_tile(res, cur, xs, a.m, lm);
        if (lm.j == lm.lpr - 1) {
            const int r0 = row0_of(t, mc);
            float *y = a.y[mc];
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                const int row = r0 + i * lm.rpw + lm.q;
                if (row < a.rows[mc]) y[row] = res[i];
            }
        }
        if (tn >= ntiles) break;
        cur = next;
        next = next2;
        t = tn;
        mc = mat_of(t);
    }
}

// Scalar-form GEMV for any alignment and bits in {2, 4, 8}: one wave per
// row, lanes striding over groups, the factored per-group sum of
// Kernels.metal.txt:56-75 with byte-addressed loads (:27-37).
__global__ __launch_bounds__(kGemvThreads) void gemv_scalar_kernel(const uint8_t *w, const uint8_t *s,
                                                                   const uint8_t *b, int rows, int in,
                                                                   int group, int bits, int stype,
                                                                   const float *x, float *y) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kGemvThreads / kWave) + wave;
    if (row >= rows) return;
    const int per_word = 32 / bits;
    const uint32_t mask = (1u << bits) - 1u;
    const int groups = in / group;
    const int words_per_group = group / per_word;
    const int64_t row_bytes = static_cast<int64_t>(in) * bits / 8;
    const uint8_t *wr = w + static_cast<int64_t>(row) * row_bytes;
    float acc = 0.f;
    for (int g = lane; g < groups; g += kWave) {
        float qdot = 0.f, xsum = 0.f;
        for (int wi = 0; wi < words_per_group; ++wi) {
            uint32_t word = load_u32_bytes(wr + static_cast<int64_t>(g * words_per_group + wi) * 4);
            const float *xx = x + g * group + wi * per_word;
            for (int j = 0; j < per_word; ++j) {
                const float xv = xx[j];
                qdot = fmaf(static_cast<float>(word & mask), xv, qdot);
                xsum += xv;
                word >>= bits;
            }
        }
        const int64_t gi = static_cast<int64_t>(row) * groups + g;
        acc += load_scale_bytes(s, gi, stype) * qdot + load_scale_bytes(b, gi, stype) * xsum;
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

// silu_mul of Kernels.metal.txt:114-124: h = g / (1 + exp(-g)) * u.
__global__ void silu_mul_kernel(float *buf, int count, int64_t g_off, int64_t u_off, int64_t dst_off) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const float g = buf[g_off + i];
    buf[dst_off + i] = (g / (1.0f + __expf(-g))) * buf[u_off + i];
}

// One thread per packed word of rows [row0, row0 + rows) of the flattened
// [experts * out_dim, in] weight; row r of expert e sits at
// e*stride_w + r*row_bytes.  w = scale * q then + bias, rounded separately
// (the two-rounding f32 form of Checkpoint.swift:202).
__global__ void dequant_kernel(const uint8_t *w, const uint8_t *s, const uint8_t *b, int64_t stride_w,
                               int64_t stride_sb, int out_dim, int64_t row0, int64_t rows, int in, int group,
                               int bits, int stype, float *out) {
#pragma clang fp contract(off)
    const int per_word = 32 / bits;
    const int64_t wpr = in / per_word;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= rows * wpr) return;
    const int64_t r = idx / wpr;
    const int wi = static_cast<int>(idx - r * wpr);
    const int64_t flat = row0 + r;
    const int64_t e = flat / out_dim;
    const int64_t rr = flat - e * out_dim;
    const int64_t row_bytes = static_cast<int64_t>(in) * bits / 8;
    const int gpr = in / group;
    uint32_t word = load_u32_bytes(w + e * stride_w + rr * row_bytes + static_cast<int64_t>(wi) * 4);
    const uint8_t *sb = s + e * stride_sb;
    const uint8_t *bb = b + e * stride_sb;
    const uint32_t mask = (1u << bits) - 1u;
    for (int j = 0; j < per_word; ++j) {
        const int col = wi * per_word + j;
        const int64_t gi = rr * gpr + col / group;
        const float sc = load_scale_bytes(sb, gi, stype);
        const float bi = load_scale_bytes(bb, gi, stype);
        const float prod = sc * static_cast<float>(word & mask);  // contract(off): no fused multiply-add
        out[r * in + col] = prod + bi;
        word >>= bits;
    }
}

static int launch_gemv(const swq_qlinear *l, int rows, int64_t w_extra, int64_t s_extra, int64_t b_extra,
                       const float *x, float *y, bool allow_vec, hipStream_t stream) {
    const bool x_aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (allow_vec && x_aligned && vector_path_ok(l, w_extra, s_extra, b_extra)) {
        QMat m = make_qmat(l, w_extra, s_extra, b_extra);
        // 4-bit rows of 65..128 chunks (in_dim up to 4096) with fp32 x: two
        // chunks per lane, a plan only the standalone GEMV compiles
        const bool q4_wide = m.bits == 4 && m.xf == 0 && m.cpl == 2 && m.chunks <= 2 * kWave;
        if ((plan_fits(m) || q4_wide) && m.in <= kStageMaxIn) {
            const int rows_per_block = (kGemvThreads / kWave) * (4 / m.cpl) * (kWave >> m.lpr_log2);
            const dim3 grid(std::min((rows + rows_per_block - 1) / rows_per_block, kGemvMaxBlocks));
#define SWQ_GEMV_LAUNCH(B, C, E) \
    hipLaunchKernelGGL((gemv_vec_kernel<B, C, E>), grid, dim3(kGemvThreads), 0, stream, m, rows, x, y)
            const bool f32s = m.stype == SWQ_F32;
            if (m.bits == 4) {
                if (m.cpl == 1) { if (f32s) SWQ_GEMV_LAUNCH(4, 1, 4); else SWQ_GEMV_LAUNCH(4, 1, 2); }
                else { if (f32s) SWQ_GEMV_LAUNCH(4, 2, 4); else SWQ_GEMV_LAUNCH(4, 2, 2); }
            } else {
                if (m.cpl == 1) { if (f32s) SWQ_GEMV_LAUNCH(8, 1, 4); else SWQ_GEMV_LAUNCH(8, 1, 2); }
                else { if (f32s) SWQ_GEMV_LAUNCH(8, 2, 4); else SWQ_GEMV_LAUNCH(8, 2, 2); }
            }
#undef SWQ_GEMV_LAUNCH
            return launch_status();
        }
    }
    const uint8_t *w = static_cast<const uint8_t *>(l->w) + l->w_off + w_extra;
    const uint8_t *s = static_cast<const uint8_t *>(l->scales) + l->s_off + s_extra;
    const uint8_t *b = static_cast<const uint8_t *>(l->biases) + l->b_off + b_extra;
    const dim3 grid((rows + kGemvThreads / kWave - 1) / (kGemvThreads / kWave));
    hipLaunchKernelGGL(gemv_scalar_kernel, grid, dim3(kGemvThreads), 0, stream, w, s, b, rows, l->in_dim,
                       l->group_size, l->bits, l->scales_type, x, y);
    return launch_status();
}

}  // namespace swq

using namespace swq;

extern "C" int swq_encode_gemv_multi(const swq_qlinear *lins, int n, float *const *ys, const float *x,
                                     const void *norm_weight, int norm_dtype, float norm_eps, void *stream) {
    if (!lins || !ys || !x || n <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (n > kMultiMax) return SWQ_ERR_LIMIT;
    if (norm_weight && norm_dtype != SWQ_F32 && norm_dtype != SWQ_F16 && norm_dtype != SWQ_BF16)
        return SWQ_ERR_UNSUPPORTED_DTYPE;
    if (norm_weight && !(norm_eps >= 0.f)) return SWQ_ERR_INVALID_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(norm_weight) % 16 != 0)
        return SWQ_ERR_MISALIGNED;
    const swq_qlinear &l0 = lins[0];
    MultiArgs a{};
    for (int i = 0; i < n; ++i) {
        const swq_qlinear &l = lins[i];
        int st = check_linear_shape(&l);
        if (st != SWQ_OK) return st;
        if (!ys[i]) return SWQ_ERR_INVALID_ARGUMENT;
        if (l.in_dim != l0.in_dim || l.bits != l0.bits || l.group_size != l0.group_size ||
            l.scales_type != l0.scales_type)
            return SWQ_ERR_BAD_SHAPE;
        if (!vector_path_ok(&l, 0, 0, 0)) return SWQ_ERR_MISALIGNED;
        const QMat mi = make_qmat(&l);
        a.w[i] = mi.w;
        a.s[i] = mi.s;
        a.b[i] = mi.b;
        a.y[i] = ys[i];
        a.rows[i] = l.out_dim;
    }
    a.m = make_qmat(&l0);
    const bool q4_wide = a.m.bits == 4 && a.m.xf == 0 && a.m.cpl == 2 && a.m.chunks <= 2 * kWave;
    if (!(plan_fits(a.m) || q4_wide) || a.m.xf != 0 || a.m.in > kStageMaxIn || a.m.in % 4 != 0)
        return SWQ_ERR_LIMIT;
    const int tile_rows = (4 / a.m.cpl) * (kWave >> a.m.lpr_log2);
    int total = 0;
    for (int i = 0; i < n; ++i) {
        total += (a.rows[i] + tile_rows - 1) / tile_rows;
        a.tile_end[i] = total;
    }
    a.n = n;
    a.x = x;
    a.norm_w = norm_weight;
    a.norm_dtype = norm_dtype;
    a.eps = norm_eps;
    const dim3 grid(std::min((total + kGemvThreads / kWave - 1) / (kGemvThreads / kWave), kGemvMaxBlocks));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool f32s = a.m.stype == SWQ_F32, norm = norm_weight != nullptr;
#define SWQ_MULTI(B, C, E)                                                                          \
    do {                                                                                            \
        if (norm) hipLaunchKernelGGL((gemv_multi_kernel<B, C, E, true>), grid, dim3(kGemvThreads), 0, s, a); \
        else hipLaunchKernelGGL((gemv_multi_kernel<B, C, E, false>), grid, dim3(kGemvThreads), 0, s, a);     \
    } while (0)
    if (a.m.bits == 4) {
        if (a.m.cpl == 1) { if (f32s) SWQ_MULTI(4, 1, 4); else SWQ_MULTI(4, 1, 2); }
        else { if (f32s) SWQ_MULTI(4, 2, 4); else SWQ_MULTI(4, 2, 2); }
    } else {
        if (a.m.cpl == 1) { if (f32s) SWQ_MULTI(8, 1, 4); else SWQ_MULTI(8, 1, 2); }
        else { if (f32s) SWQ_MULTI(8, 2, 4); else SWQ_MULTI(8, 2, 2); }
    }
#undef SWQ_MULTI
    return launch_status();
}

extern "C" int swq_encode_gemv(const swq_qlinear *lin, int rows, int64_t w_extra, int64_t s_extra,
                               int64_t b_extra, const float *x, int64_t x_off, float *y, int64_t y_off,
                               void *stream) {
    int st = check_linear_shape(lin);
    if (st != SWQ_OK) return st;
    if (!x || !y || x_off < 0 || y_off < 0 || w_extra < 0 || s_extra < 0 || b_extra < 0) return SWQ_ERR_INVALID_ARGUMENT;
    const int n = rows > 0 ? rows : lin->out_dim;
    return launch_gemv(lin, n, w_extra, s_extra, b_extra, x + x_off, y + y_off, true,
                       static_cast<hipStream_t>(stream));
}

extern "C" int swq_encode_silu_mul(float *buf, int count, int64_t g_off, int64_t u_off, int64_t dst_off,
                                   void *stream) {
    if (!buf || count <= 0 || g_off < 0 || u_off < 0 || dst_off < 0) return SWQ_ERR_INVALID_ARGUMENT;
    const int tb = 256;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((count + tb - 1) / tb), dim3(tb), 0,
                       static_cast<hipStream_t>(stream), buf, count, g_off, u_off, dst_off);
    return launch_status();
}

extern "C" int swq_dequantize(const swq_qlinear *lin, int64_t row0, int64_t rows, float *out, void *stream) {
    int st = check_linear_shape(lin);
    if (st != SWQ_OK) return st;
    if (!out || row0 < 0 || rows <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    // an unstacked matrix has out_dim rows; a stack's extent is the caller's
    if (lin->expert_stride_w == 0 && row0 + rows > lin->out_dim) return SWQ_ERR_BAD_SHAPE;
    const int per_word = 32 / lin->bits;
    const int64_t words = rows * (lin->in_dim / per_word);
    const int tb = 256;
    const int64_t blocks = (words + tb - 1) / tb;
    if (blocks > 0x7FFFFFFF) return SWQ_ERR_LIMIT;
    hipLaunchKernelGGL(dequant_kernel, dim3(static_cast<unsigned>(blocks)), dim3(tb), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint8_t *>(lin->w) + lin->w_off,
                       static_cast<const uint8_t *>(lin->scales) + lin->s_off,
                       static_cast<const uint8_t *>(lin->biases) + lin->b_off, lin->expert_stride_w,
                       lin->expert_stride_sb, lin->out_dim, row0, rows, lin->in_dim, lin->group_size, lin->bits,
                       lin->scales_type, out);
    return launch_status();
}

extern "C" int swq_gemv_quantized(const float *x, const void *packed, size_t packed_bytes, const void *scales,
                                  size_t scales_bytes, const void *biases, size_t biases_bytes, int out_dim,
                                  int in_dim, int group_size, int bits, int scales_type, int use_fast, float *y) {
    if (!x || !packed || !scales || !biases || !y) return SWQ_ERR_INVALID_ARGUMENT;
    swq_qlinear l{};
    l.out_dim = out_dim;
    l.in_dim = in_dim;
    l.group_size = group_size;
    l.bits = bits;
    l.scales_type = scales_type;
    l.w = packed;
    l.scales = scales;
    l.biases = biases;
    int st = check_linear_shape(&l);
    if (st != SWQ_OK) return st;
    const size_t need_w = static_cast<size_t>(out_dim) * in_dim * bits / 8;
    const size_t need_s = static_cast<size_t>(out_dim) * (in_dim / group_size) * scale_bytes(scales_type);
    if (packed_bytes < need_w || scales_bytes < need_s || biases_bytes < need_s) return SWQ_ERR_BAD_SHAPE;

    void *dx = nullptr, *dw = nullptr, *ds = nullptr, *db = nullptr, *dy = nullptr;
    auto release = [&]() {
        hipFree(dx);
        hipFree(dw);
        hipFree(ds);
        hipFree(db);
        hipFree(dy);
    };
    if (hipMalloc(&dx, static_cast<size_t>(in_dim) * 4) != hipSuccess ||
        hipMalloc(&dw, need_w) != hipSuccess || hipMalloc(&ds, need_s) != hipSuccess ||
        hipMalloc(&db, need_s) != hipSuccess || hipMalloc(&dy, static_cast<size_t>(out_dim) * 4) != hipSuccess) {
        release();
        return SWQ_ERR_HIP;
    }
    st = SWQ_OK;
    if (hipMemcpy(dx, x, static_cast<size_t>(in_dim) * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(dw, packed, need_w, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(ds, scales, need_s, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(db, biases, need_s, hipMemcpyHostToDevice) != hipSuccess)
        st = SWQ_ERR_HIP;
    if (st == SWQ_OK) {
        l.w = dw;
        l.scales = ds;
        l.biases = db;
        st = launch_gemv(&l, out_dim, 0, 0, 0, static_cast<const float *>(dx), static_cast<float *>(dy),
                         use_fast != 0, nullptr);
    }
    if (st == SWQ_OK && hipDeviceSynchronize() != hipSuccess) st = SWQ_ERR_HIP;
    if (st == SWQ_OK && hipMemcpy(y, dy, static_cast<size_t>(out_dim) * 4, hipMemcpyDeviceToHost) != hipSuccess)
        st = SWQ_ERR_HIP;
    release();
    return st;
}
