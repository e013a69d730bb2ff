// MoE-layer decode step on gfx950: three launches per layer.
//
//   stage 1  router GEMV, shared-expert gate GEMV, shared gate/up SwiGLU.
//   stage 2  every workgroup runs softmax, top-k and renormalisation on the
//            router logits itself (and, for batches, the distinct-expert
//            list), then the gate/up SwiGLU rows of its expert: one launch for
//            all selected experts, indexed by device-resident ids.
//   stage 3  down projections of the selected experts and of the shared
//            expert, weighted combine in pick order, then the shared term.
//
// Numerics follow QwenCPUModel.moeForward (QwenCPUModel.swift:500-569):
// router logits -> softmax (:65-71) -> top-k by probability, ties to the
// lower expert id (:508-522) -> w = p / sum_topk p (:546-550) ->
// out = sum_k w_k * down(silu(gate x) * up x) + sigmoid(<w_sg, x>) * shared(x)
// (:549-566).  The reference GPU path issues 4K+6 dispatches plus a host
// round trip for the top-k (QwenMetalModel.swift:798-892); here the ids
// never leave the device.
#include "../../include/swq_bench.h"
#include "internal.hpp"
#include "moe_host.hpp"
#include "route.hpp"
#include "tile.hpp"

#include <atomic>
#include <mutex>

namespace swq {

constexpr int kThreads12 = 256;
constexpr int kMaxPairs = SWQ_MAX_BATCH * SWQ_MAX_TOPK;
constexpr int kRows3 = 16;  // stage-3 rows per workgroup (upper bound)

struct MoEArgs {
    QMat router, gate, up, down, sh_gate, sh_up, sh_down, seg;
    const void *x;
    void *out;
    int32_t *user_ids;
    float *user_w;
    float *logits;         // [B][E]
    float *sg;             // [B] shared gate logit
    float *h_sh;           // [B][Is] shared SwiGLU activations
    int32_t *ids;          // [B][K]
    float *wts;            // [B][K]
    int32_t *n_unique;     // [1]
    int32_t *uniq_e;       // [P] distinct experts, first-appearance order
    int32_t *uniq_np;      // [P] pairs per distinct expert
    int32_t *uniq_pairs;   // [P][B] pair indices b*K + k
    float *h;              // [P][I] routed SwiGLU activations, by pair
    int32_t xdt, odt, accumulate;
    int32_t B, H, E, K, I, Is, norm, has_shared;
    int32_t nr_blocks;     // stage-1 workgroups holding router rows
    int32_t router_tasks;  // waves with router rows
    int32_t shared_tasks;  // waves with shared gate/up rows
    int32_t rows3;         // stage-3 rows per workgroup
};

// Wave-uniform dispatch over a matrix's plan (bits, chunks per lane,
// activation format) and scale bytes.  FN<XDT, BITS, CPL, ES, XF>.
#define SWQ_DISPATCH_ES(XDT, m, FN, ES, ...)                                \
    do {                                                                    \
        if constexpr (XDT == SWQ_BF16) {                                    \
            if ((m).bits == 4) FN<XDT, 4, 2, ES, kXBF16>(__VA_ARGS__);      \
            else if ((m).cpl == 1) FN<XDT, 8, 1, ES, kXF32>(__VA_ARGS__);   \
            else FN<XDT, 8, 2, ES, kXF32>(__VA_ARGS__);                     \
        } else {                                                            \
            if ((m).bits == 4) FN<XDT, 4, 1, ES, kXF32>(__VA_ARGS__);       \
            else if ((m).cpl == 1) FN<XDT, 8, 1, ES, kXF32>(__VA_ARGS__);   \
            else FN<XDT, 8, 2, ES, kXF32>(__VA_ARGS__);                     \
        }                                                                   \
    } while (0)
#define SWQ_DISPATCH(XDT, m, FN, ...)                                       \
    do {                                                                    \
        if ((m).stype == SWQ_F32) SWQ_DISPATCH_ES(XDT, m, FN, 4, __VA_ARGS__); \
        else SWQ_DISPATCH_ES(XDT, m, FN, 2, __VA_ARGS__);                   \
    } while (0)

// Down projections read the fp32 SwiGLU activations: one chunk per lane,
// i.e. up to 2048 inputs at 4 bits and 1024 at 8 bits; 4-bit rows take the
// split-bf16 dot products.
#define SWQ_DISPATCH_DOWN(m, FN, ...)                                       \
    do {                                                                    \
        if ((m).stype == SWQ_F32) {                                         \
            if ((m).bits == 4) FN<SWQ_F32, 4, 1, 4, kXBF16X2>(__VA_ARGS__); \
            else FN<SWQ_F32, 8, 1, 4, kXF32>(__VA_ARGS__);                  \
        } else {                                                            \
            if ((m).bits == 4) FN<SWQ_F32, 4, 1, 2, kXBF16X2>(__VA_ARGS__); \
            else FN<SWQ_F32, 8, 1, 2, kXF32>(__VA_ARGS__);                  \
        }                                                                   \
    } while (0)

// One tile of rows of one matrix against every token's x; the result of
// (token b, row) goes to out[b*ld + row].
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void gemv_rows_tokens(const QMat &m, int row0, int row_end, const void *x,
                                                 int H, int B, float *out, int ld, int lane) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    RowTile<BITS, CPL, ES> rt;
    load_tile(rt, m, 0, lm, row0, row_end);
#pragma unroll 1
    for (int b = 0; b < B; ++b) {
        XSlice<BITS, CPL, XF> xs;
        load_xslice<XDT>(xs, m, lm, x, static_cast<int64_t>(b) * H);
        float res[RI];
        dot_tile(res, rt, xs, m, lm);
        if (lm.j == lm.lpr - 1) {
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                const int row = row0 + i * lm.rpw + lm.q;
                if (row < row_end) out[b * ld + row] = res[i];
            }
        }
    }
}

// SwiGLU rows of one expert: h[p*ld + r] = silu(gate_r . x_b) * (up_r . x_b)
// for each (token b, destination p) pair; pairs == nullptr means p = b.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void gateup_rows(const QMat &g, const QMat &u, int64_t expert, int row0, int row_end,
                                            const void *x, int H, const int32_t *pairs, int npairs, int K,
                                            float *h, int ld, int lane) {
    if (npairs <= 0) return;
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const LaneMap lm = lane_map(g.lpr_log2, lane);
    RowTile<BITS, CPL, ES> tg, tu;
    load_tile(tg, g, expert, lm, row0, row_end);
    load_tile(tu, u, expert, lm, row0, row_end);
#pragma unroll 1
    for (int pi = 0; pi < npairs; ++pi) {
        const int p = pairs ? pairs[pi] : pi;
        const int b = pairs ? p / K : pi;
        XSlice<BITS, CPL, XF> xs;
        load_xslice<XDT>(xs, g, lm, x, static_cast<int64_t>(b) * H);
        float rg[RI], ru[RI];
        dot_tile(rg, tg, xs, g, lm);
        dot_tile(ru, tu, xs, u, lm);
        if (lm.j == lm.lpr - 1) {
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                const int row = row0 + i * lm.rpw + lm.q;
                if (row < row_end) h[static_cast<int64_t>(p) * ld + row] = swiglu(rg[i], ru[i]);
            }
        }
    }
}

// Down rows [row0, row0 + nrows) of one expert for each pair p: the dot of
// the row with h[p] lands in part[part_base + p][row - row0].
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void down_rows(const QMat &m, int64_t expert, int row0, int nrows, int row_end,
                                          const float *h, int ld, const int32_t *pairs, int npairs,
                                          float (*part)[kRows3], int part_base, int lane) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    const int end = min(row0 + nrows, row_end);
#pragma unroll 1
    for (int t0 = row0; t0 < end; t0 += RI * lm.rpw) {
        RowTile<BITS, CPL, ES> rt;
        load_tile(rt, m, expert, lm, t0, end);
#pragma unroll 1
        for (int pi = 0; pi < npairs; ++pi) {
            const int p = pairs ? pairs[pi] : pi;
            XSlice<BITS, CPL, XF> xs;
            load_xslice<XDT>(xs, m, lm, h, static_cast<int64_t>(p) * ld);
            float res[RI];
            dot_tile(res, rt, xs, m, lm);
            if (lm.j == lm.lpr - 1) {
#pragma unroll
                for (int i = 0; i < RI; ++i) {
                    const int row = t0 + i * lm.rpw + lm.q;
                    if (row < end) part[part_base + p][row - row0] = res[i];
                }
            }
        }
    }
}


// Batch-1 SwiGLU rows of expert e, the pick in slot `slot`.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void gateup_rows_b1(const QMat &g, const QMat &u, int e, int slot, int row0,
                                               int row_end, const void *x, float *h, int ld, int lane) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const LaneMap lm = lane_map(g.lpr_log2, lane);
    RowTile<BITS, CPL, ES> tg, tu;
    load_tile(tg, g, e, lm, row0, row_end);
    load_tile(tu, u, e, lm, row0, row_end);
    XSlice<BITS, CPL, XF> xs;
    load_xslice<XDT>(xs, g, lm, x, 0);
    float rg[RI], ru[RI];
    dot_tile(rg, tg, xs, g, lm);
    dot_tile(ru, tu, xs, u, lm);
    if (lm.j == lm.lpr - 1) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int row = row0 + i * lm.rpw + lm.q;
            if (row < row_end) h[static_cast<int64_t>(slot) * ld + row] = swiglu(rg[i], ru[i]);
        }
    }
}

// Batch-1 down rows [row0, row0 + nrows) of the expert in slot `slot` (or of
// the shared expert when ids == nullptr) against activations hv.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void down_rows_b1(const QMat &m, const int32_t *ids, int slot, int row0, int nrows,
                                             int row_end, const float *hv, float (*part)[kRows3], int part_row,
                                             int lane) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    const int end = min(row0 + nrows, row_end);
    XSlice<BITS, CPL, XF> xs;
    load_xslice<XDT>(xs, m, lm, hv, 0);
    const int64_t e = ids ? ids[slot] : 0;
#pragma unroll 1
    for (int t0 = row0; t0 < end; t0 += RI * lm.rpw) {
        RowTile<BITS, CPL, ES> rt;
        load_tile(rt, m, e, lm, t0, end);
        float res[RI];
        dot_tile(res, rt, xs, m, lm);
        if (lm.j == lm.lpr - 1) {
#pragma unroll
            for (int i = 0; i < RI; ++i) {
                const int row = t0 + i * lm.rpw + lm.q;
                if (row < end) part[part_row][row - row0] = res[i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// top-k (one wave per token)

// Top-k of one token's router logits, one wave.  Selection by logit with
// ties to the lower expert id equals the reference's selection by softmax
// probability (QwenCPUModel.swift:508-522; softmax is monotonic) up to fp32
// ties of exp().  Lane l holds experts l*M .. l*M+M-1 as 64-bit keys
// (orderable logit, inverted id), sorted descending; each of the K rounds
// takes the wave-wide maximum head.  Then p_k = exp(l_k - max) / sum_e
// exp(l_e - max) (:65-71) and w_k = p_k / sum_j p_j when norm (:546-550).
// Writes ids[k], w[k] (LDS); sel_l is LDS scratch of K floats.
template <int M>
__device__ __forceinline__ void topk_token(const float *lrow, int E, int K, int norm, int lane, int32_t *ids,
                                           float *w, float *sel_l) {
    float lg[M];
#pragma unroll
    for (int j = 0; j < M; ++j) lg[j] = lrow[min(lane * M + j, E - 1)];  // every load issued first
    uint64_t key[M];
#pragma unroll
    for (int j = 0; j < M; ++j) {
        const int e = lane * M + j;
        const bool valid = e < E;
        key[j] = valid ? (static_cast<uint64_t>(orderable(lg[j])) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(e))
                       : 0;
        if (!valid) lg[j] = -INFINITY;
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
        for (int j = 0; j + 1 < M - i; ++j) {
            if (key[j] < key[j + 1]) {
                const uint64_t t = key[j];
                key[j] = key[j + 1];
                key[j + 1] = t;
            }
        }
    }
    float top = 0.f;
    for (int k = 0; k < K; ++k) {
        const uint32_t hi = static_cast<uint32_t>(key[0] >> 32);
        const uint32_t lo = static_cast<uint32_t>(key[0]);
        const uint32_t mhi = wave_max_u32(hi);
        const uint64_t cand = __ballot(hi == mhi);
        int winner;
        if (__popcll(cand) == 1) {
            winner = __ffsll(static_cast<long long>(cand)) - 1;
        } else {
            const uint32_t mlo = wave_max_u32(hi == mhi ? lo : 0u);
            winner = __ffsll(static_cast<long long>(__ballot(hi == mhi && lo == mlo))) - 1;
        }
        const uint32_t wlo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lo), winner));
        const float l = from_orderable(mhi);
        if (k == 0) top = l;
        if (lane == 0) {
            ids[k] = static_cast<int32_t>(0xFFFFFFFFu - wlo);
            sel_l[k] = l;
        }
        if (lane == winner) {
#pragma unroll
            for (int j = 0; j + 1 < M; ++j) key[j] = key[j + 1];
            key[M - 1] = 0;
        }
    }
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) part += expf(lg[j] - top);  // -inf padding adds 0
    const float denom = wave_sum_all(part);
    const float pk = lane < K ? expf(sel_l[lane] - top) / denom : 0.f;
    const float total = wave_sum_all(pk);
    if (lane < K) w[lane] = norm ? pk / total : pk;
}

// The block's routing, in LDS.
struct Routing {
    int32_t ids[kMaxPairs];    // [B][K] picks, pair p = b*K + k
    float w[kMaxPairs];        // combine weights
    float sel_l[kThreads12 / kWave][SWQ_MAX_TOPK];
    int32_t lead[kMaxPairs];   // pair leads its expert's list
    int32_t slot[kMaxPairs];   // distinct slot of a leading pair
    int32_t uniq_e[kMaxPairs];
    int32_t uniq_np[kMaxPairs];
    int32_t pairs[SWQ_MAX_BATCH];  // pairs of this block's slot
    int32_t n_unique;
};

// Every token's top-k into r (one wave per token), then for batches the
// distinct experts in order of first appearance, each with its pairs in pair
// order (one thread per pair, two O(P) passes).  `my_slot` selects whose pair
// list lands in r.pairs; with `publish` the block also writes the routing to
// the workspace (and the caller's outputs) for stage 3.
__device__ __forceinline__ void route(const MoEArgs &a, Routing &r, int my_slot, bool publish) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int M = (a.E + kWave - 1) / kWave;
    for (int b = wave; b < a.B; b += kThreads12 / kWave) {
        const float *lrow = a.logits + static_cast<int64_t>(b) * a.E;
        int32_t *ids = r.ids + b * a.K;
        float *w = r.w + b * a.K;
        if (M <= 1) topk_token<1>(lrow, a.E, a.K, a.norm, lane, ids, w, r.sel_l[wave]);
        else if (M <= 2) topk_token<2>(lrow, a.E, a.K, a.norm, lane, ids, w, r.sel_l[wave]);
        else if (M <= 4) topk_token<4>(lrow, a.E, a.K, a.norm, lane, ids, w, r.sel_l[wave]);
        else if (M <= 8) topk_token<8>(lrow, a.E, a.K, a.norm, lane, ids, w, r.sel_l[wave]);
        else topk_token<16>(lrow, a.E, a.K, a.norm, lane, ids, w, r.sel_l[wave]);
    }
    __syncthreads();
    const int P = a.B * a.K;
    const int p = threadIdx.x;
    if (publish && p < P) {
        a.ids[p] = r.ids[p];
        a.wts[p] = r.w[p];
        if (a.user_ids) a.user_ids[p] = r.ids[p];
        if (a.user_w) a.user_w[p] = r.w[p];
    }
    if (a.B == 1) {
        if (p == 0) r.n_unique = a.K;  // a token's picks are distinct
        __syncthreads();
        return;
    }
    int first = p, pos = 0, count = 0;
    if (p < P) {
        const int e = r.ids[p];
        for (int q = 0; q < P; ++q) {
            const bool same = r.ids[q] == e;
            if (same && q < p) {
                first = min(first, q);
                ++pos;
            }
            count += same ? 1 : 0;
        }
        r.lead[p] = (first == p) ? 1 : 0;
    }
    __syncthreads();
    if (p < P && first == p) {
        int rank = 0, total = 0;
        for (int q = 0; q < P; ++q) {
            rank += (q < p) ? r.lead[q] : 0;
            total += r.lead[q];
        }
        r.slot[p] = rank;
        r.uniq_e[rank] = r.ids[p];
        r.uniq_np[rank] = count;
        if (p == 0) r.n_unique = total;
        if (publish) {
            a.uniq_e[rank] = r.ids[p];
            a.uniq_np[rank] = count;
            if (p == 0) *a.n_unique = total;
        }
    }
    __syncthreads();
    if (p < P) {
        const int slot = r.slot[first];
        if (slot == my_slot) r.pairs[pos] = p;
        if (publish) a.uniq_pairs[slot * a.B + pos] = p;
    }
    __syncthreads();
}

// Pull this workgroup's share (part `part` of `parts`) of a matrix's codes,
// scales and biases toward the last-level cache: plain loads whose values are
// only kept alive.  Stage 3 then reads the down projections from cache.
__device__ __forceinline__ uint32_t touch_share(const QMat &m, int64_t expert, int part, int parts) {
    const int64_t wbytes = static_cast<int64_t>(m.rows) * m.row_bytes;
    const int64_t sbytes = static_cast<int64_t>(m.rows) * m.gpr * (m.stype == SWQ_F32 ? 4 : 2);
    const uint8_t *w = m.w + expert * m.stride_w;
    const uint8_t *sc = m.s + expert * m.stride_sb;
    const uint8_t *bi = m.b + expert * m.stride_sb;
    const int64_t wshare = (wbytes / parts) & ~static_cast<int64_t>(63);
    const int64_t sshare = (sbytes / parts) & ~static_cast<int64_t>(63);
    uint32_t acc = 0;
    // one 16-byte load per 64 bytes: one per 64-byte segment of each cache line
    for (int64_t o = static_cast<int64_t>(threadIdx.x) * 64; o < wshare; o += blockDim.x * 64)
        acc ^= reinterpret_cast<const uint4 *>(w + part * wshare + o)->x;
    for (int64_t o = static_cast<int64_t>(threadIdx.x) * 64; o < sshare; o += blockDim.x * 64) {
        acc ^= *reinterpret_cast<const uint32_t *>(sc + part * sshare + o);
        acc ^= *reinterpret_cast<const uint32_t *>(bi + part * sshare + o);
    }
    return acc;
}

__device__ __forceinline__ void keep(uint32_t v) { asm volatile("" ::"v"(v)); }

template <int XDT>
__global__ __launch_bounds__(kThreads12) void moe_stage1(MoEArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int task = blockIdx.x * (kThreads12 / kWave) + wave;
    if (static_cast<int>(blockIdx.x) < a.nr_blocks) {
        if (task < a.router_tasks)
            SWQ_DISPATCH(XDT, a.router, gemv_rows_tokens, a.router, task * tile_rows(a.router), a.E, a.x,
                         a.H, a.B, a.logits, a.E, lane);
        return;
    }
    // shared-expert workgroups; the shared down projection is pulled toward
    // the cache for stage 3 meanwhile
    if (!a.has_shared) return;
    const int sb = blockIdx.x - a.nr_blocks;
    const uint32_t t = touch_share(a.sh_down, 0, sb, gridDim.x - a.nr_blocks);
    const int st = task - a.nr_blocks * (kThreads12 / kWave);
    if (st == 0) {
        SWQ_DISPATCH(XDT, a.seg, gemv_rows_tokens, a.seg, 0, 1, a.x, a.H, a.B, a.sg, 1, lane);
    } else if (st - 1 < a.shared_tasks) {
        SWQ_DISPATCH(XDT, a.sh_gate, gateup_rows, a.sh_gate, a.sh_up, 0, (st - 1) * tile_rows(a.sh_gate), a.Is,
                     a.x, a.H, nullptr, a.B, a.K, a.h_sh, a.Is, lane);
    }
    keep(t);
}

template <int XDT>
__global__ __launch_bounds__(kThreads12) void moe_stage2(MoEArgs a) {
    __shared__ Routing r;
    const int slot = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    route(a, r, slot, blockIdx.x == 0 && blockIdx.y == 0);
    if (slot >= r.n_unique) return;
    const int e = a.B == 1 ? r.ids[slot] : r.uniq_e[slot];
    const uint32_t t = touch_share(a.down, e, blockIdx.x, gridDim.x);
    const int row0 = (blockIdx.x * (kThreads12 / kWave) + wave) * tile_rows(a.gate);
    if (row0 < a.I) {
        if (a.B == 1) {
            SWQ_DISPATCH(XDT, a.gate, gateup_rows_b1, a.gate, a.up, e, slot, row0, a.I, a.x, a.h, a.I, lane);
        } else {
            SWQ_DISPATCH(XDT, a.gate, gateup_rows, a.gate, a.up, e, row0, a.I, a.x, a.H, r.pairs,
                         r.uniq_np[slot], a.K, a.h, a.I, lane);
        }
    }
    keep(t);
}

constexpr int kStage3MaxWaves = 12;

__global__ __launch_bounds__(kStage3MaxWaves * 64) void moe_stage3(MoEArgs a) {
    __shared__ float part[kMaxPairs + SWQ_MAX_BATCH][kRows3];
    __shared__ float s_w[kMaxPairs];
    __shared__ float s_gate[SWQ_MAX_BATCH];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nw = blockDim.x >> 6;
    const int r0 = blockIdx.x * a.rows3;
    const int P = a.B * a.K;
    // combine weights and shared-gate logits: loaded into registers now,
    // staged in LDS only after the projections, so their latency overlaps.
    float w_pre[4];  // P <= 4 * blockDim (the host sizes the block 64*min(12, slots))
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned t = threadIdx.x + i * blockDim.x;
        w_pre[i] = t < static_cast<unsigned>(P) ? a.wts[t] : 0.f;
    }
    const float sg_pre = (a.has_shared && threadIdx.x < static_cast<unsigned>(a.B)) ? a.sg[threadIdx.x] : 0.f;
    if (a.B == 1) {
        const int nslots = a.K + (a.has_shared ? 1 : 0);
#pragma unroll 1
        for (int s = wave; s < nslots; s += nw) {
            if (s < a.K) {
                SWQ_DISPATCH_DOWN(a.down, down_rows_b1, a.down, a.ids, s, r0, a.rows3, a.H,
                                  a.h + static_cast<int64_t>(s) * a.I, part, s, lane);
            } else {
                SWQ_DISPATCH_DOWN(a.sh_down, down_rows_b1, a.sh_down, nullptr, 0, r0, a.rows3, a.H, a.h_sh,
                                  part, P, lane);
            }
        }
    } else {
        const int nu = *a.n_unique;
        const int nslots = nu + (a.has_shared ? 1 : 0);
#pragma unroll 1
        for (int s = wave; s < nslots; s += nw) {
            if (s < nu) {
                SWQ_DISPATCH_DOWN(a.down, down_rows, a.down, a.uniq_e[s], r0, a.rows3, a.H, a.h, a.I,
                                  a.uniq_pairs + s * a.B, a.uniq_np[s], part, 0, lane);
            } else {
                SWQ_DISPATCH_DOWN(a.sh_down, down_rows, a.sh_down, 0, r0, a.rows3, a.H, a.h_sh, a.Is,
                                  nullptr, a.B, part, P, lane);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned t = threadIdx.x + i * blockDim.x;
        if (t < static_cast<unsigned>(P)) s_w[t] = w_pre[i];
    }
    if (a.has_shared && threadIdx.x < static_cast<unsigned>(a.B)) s_gate[threadIdx.x] = sigmoidf_ref(sg_pre);
    __syncthreads();
    for (int t = threadIdx.x; t < a.B * a.rows3; t += blockDim.x) {
        const int b = t / a.rows3, rr = t - b * a.rows3;
        const int row = r0 + rr;
        if (row >= a.H) continue;
        // out = sum_k w_k d_k in pick order, then + sigmoid(sg) * shared
        // (QwenCPUModel.swift:549-566)
        float acc = 0.f;
        for (int k = 0; k < a.K; ++k) acc += s_w[b * a.K + k] * part[b * a.K + k][rr];
        if (a.has_shared) acc += s_gate[b] * part[P + b][rr];
        const int64_t o = static_cast<int64_t>(b) * a.H + row;
        if (a.odt == SWQ_BF16) {
            static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_rne(acc);
        } else {
            float *out = static_cast<float *>(a.out);
            out[o] = a.accumulate ? out[o] + acc : acc;
        }
    }
}

// Zero-fills n bytes (a fill kernel rather than hipMemsetAsync, so that a
// caller may also record it into a graph).
__global__ void zero_bytes_kernel(uint8_t *p, size_t n) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if ((reinterpret_cast<uintptr_t>(p) & 15) == 0) {
        const size_t n16 = n / 16;
        for (size_t j = i; j < n16; j += stride) reinterpret_cast<uint4 *>(p)[j] = make_uint4(0, 0, 0, 0);
        for (size_t j = n16 * 16 + i; j < n; j += stride) p[j] = 0;
    } else {
        for (size_t j = i; j < n; j += stride) p[j] = 0;
    }
}

int zero_fill(void *p, size_t n, hipStream_t stream) {
    if (n == 0) return SWQ_OK;
    const size_t blocks = min(static_cast<size_t>(1024), (n / 16 + 255) / 256 + 1);
    hipLaunchKernelGGL(zero_bytes_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       static_cast<uint8_t *>(p), n);
    return launch_status();
}

// ---------------------------------------------------------------------------
// host side

}  // namespace swq

using namespace swq;

extern "C" size_t swq_moe_decode_workspace_bytes(const swq_moe_layer *layer, int batch) {
    if (check_layer(layer, batch, SWQ_BF16) != SWQ_OK) return 0;
    return decode_ws_bytes(layer, batch, false);
}

extern "C" int swq_moe_workspace_init(void *ws, size_t ws_bytes, void *stream) {
    if (!ws || ws_bytes < 256) return SWQ_ERR_WORKSPACE;
    const int st = fused_probe_device(static_cast<hipStream_t>(stream));
    if (st != SWQ_OK) return st;
    return zero_fill(ws, ws_bytes, static_cast<hipStream_t>(stream));
}

extern "C" size_t swq_moe_workspace_error_offset(const swq_moe_layer *layer, int batch) {
    if (check_layer(layer, batch, SWQ_BF16) != SWQ_OK) return 0;
    return kWsErrByte;
}

extern "C" int swq_moe_workspace_status(void *ws, size_t ws_bytes, int clear, void *stream) {
    if (!ws || ws_bytes < 256) return SWQ_ERR_WORKSPACE;
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t *word = reinterpret_cast<uint32_t *>(static_cast<uint8_t *>(ws) + kWsErrByte);
    uint32_t v = 0;
    hipError_t e = hipMemcpyAsync(&v, word, 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return SWQ_ERR_HIP;
    if (v != 0 && clear) {
        const uint32_t zero = 0;
        e = hipMemcpyAsync(word, &zero, 4, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) return SWQ_ERR_HIP;
    }
    return v != 0 ? SWQ_ERR_STALLED : SWQ_OK;
}

// stage_mask: bits 0-2 run the staged kernels' stages; SWQ_STAGES_FUSED
// runs the single-launch path (SWQ_ERR_LIMIT when this layer, batch or device
// cannot); 0 picks the single launch when possible, else the three stages.
static int moe_decode_impl(const swq_moe_layer *layer, const void *x, int x_dtype, int batch, void *out,
                           int out_dtype, int32_t *topk_ids, float *topk_weights, void *ws, size_t ws_bytes,
                           int flags, int stage_mask, void *stream, bool max_layout = false) {
    if (x_dtype != SWQ_F32 && x_dtype != SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    int st = check_layer(layer, batch, x_dtype);
    if (st != SWQ_OK) return st;
    if (!x || !out) return SWQ_ERR_INVALID_ARGUMENT;
    if (out_dtype != SWQ_F32 && out_dtype != SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if ((flags & ~SWQ_MOE_ACCUMULATE) != 0) return SWQ_ERR_INVALID_ARGUMENT;
    const bool accumulate = (flags & SWQ_MOE_ACCUMULATE) != 0;
    if (accumulate && out_dtype != SWQ_F32) return SWQ_ERR_UNSUPPORTED_DTYPE;
    const int H = layer->hidden;
    const int xes = x_dtype == SWQ_F32 ? 4 : 2;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || (static_cast<int64_t>(H) * xes) % 16 != 0) return SWQ_ERR_MISALIGNED;
    const FusedLayout fl = fused_layout(layer, max_layout);
    const WsLayout wl = ws_layout(layer, batch, fl.total);
    if (!ws || ws_bytes < wl.total) return SWQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(ws) % 256 != 0) return SWQ_ERR_MISALIGNED;

    uint8_t *wsb = static_cast<uint8_t *>(ws);
    MoEArgs a{};
    a.router = make_qmat(&layer->router);
    a.gate = make_qmat(&layer->gate);
    a.up = make_qmat(&layer->up);
    a.down = make_qmat(&layer->down);
    if (layer->has_shared) {
        a.sh_gate = make_qmat(&layer->shared_gate);
        a.sh_up = make_qmat(&layer->shared_up);
        a.sh_down = make_qmat(&layer->shared_down);
        a.seg = make_qmat(&layer->shared_expert_gate);
    }
    plan_qmat(&a.router, x_dtype);
    plan_qmat(&a.gate, x_dtype);
    plan_qmat(&a.up, x_dtype);
    plan_qmat(&a.sh_gate, x_dtype);
    plan_qmat(&a.sh_up, x_dtype);
    plan_qmat(&a.seg, x_dtype);
    plan_qmat(&a.down, SWQ_F32);
    plan_qmat(&a.sh_down, SWQ_F32);
    a.x = x;
    a.out = out;
    a.user_ids = topk_ids;
    a.user_w = topk_weights;
    a.logits = reinterpret_cast<float *>(wsb + wl.logits);
    a.sg = reinterpret_cast<float *>(wsb + wl.sg);
    a.h_sh = reinterpret_cast<float *>(wsb + wl.h_sh);
    a.ids = reinterpret_cast<int32_t *>(wsb + wl.ids);
    a.wts = reinterpret_cast<float *>(wsb + wl.wts);
    a.n_unique = reinterpret_cast<int32_t *>(wsb + wl.n_unique);
    a.uniq_e = reinterpret_cast<int32_t *>(wsb + wl.uniq_e);
    a.uniq_np = reinterpret_cast<int32_t *>(wsb + wl.uniq_np);
    a.uniq_pairs = reinterpret_cast<int32_t *>(wsb + wl.uniq_pairs);
    a.h = reinterpret_cast<float *>(wsb + wl.h);
    a.xdt = x_dtype;
    a.odt = out_dtype;
    a.accumulate = accumulate ? 1 : 0;
    a.B = batch;
    a.H = H;
    a.E = layer->num_experts;
    a.K = layer->top_k;
    a.I = layer->moe_intermediate;
    a.Is = layer->has_shared ? layer->shared_intermediate : 0;
    a.norm = layer->norm_topk_prob ? 1 : 0;
    a.has_shared = layer->has_shared ? 1 : 0;

    const int waves12 = kThreads12 / kWave;
    const int router_rows_per_task = tile_rows(a.router);
    a.router_tasks = (a.E + router_rows_per_task - 1) / router_rows_per_task;
    a.nr_blocks = (a.router_tasks + waves12 - 1) / waves12;
    int shared_blocks = 0;
    if (a.has_shared) {
        const int sh_rows_per_task = tile_rows(a.sh_gate);
        a.shared_tasks = (a.Is + sh_rows_per_task - 1) / sh_rows_per_task;
        shared_blocks = (a.shared_tasks + 1 + waves12 - 1) / waves12;  // +1: shared gate row
    }
    a.rows3 = min(kRows3, tile_rows(a.down));

    if (stage_mask != SWQ_STAGES_FUSED && (stage_mask & ~7)) return SWQ_ERR_INVALID_ARGUMENT;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (stage_mask == 0 || stage_mask == SWQ_STAGES_FUSED) {
        bool taken = false;
        st = fused_decode(layer, x, x_dtype, batch, out, out_dtype, topk_ids, topk_weights, ws, fl, accumulate, s,
                          &taken);
        if (st != SWQ_OK || taken) return st;
        if (stage_mask == SWQ_STAGES_FUSED) return SWQ_ERR_LIMIT;
        stage_mask = 7;
    }
    if (stage_mask & 1) {
        if (x_dtype == SWQ_BF16) hipLaunchKernelGGL(moe_stage1<SWQ_BF16>, dim3(a.nr_blocks + shared_blocks), dim3(kThreads12), 0, s, a);
        else hipLaunchKernelGGL(moe_stage1<SWQ_F32>, dim3(a.nr_blocks + shared_blocks), dim3(kThreads12), 0, s, a);
        if ((st = launch_status()) != SWQ_OK) return st;
    }

    const int P = batch * a.K;
    const int max_slots = min(P, a.E);
    const int rows2 = tile_rows(a.gate) * waves12;
    const dim3 grid2((a.I + rows2 - 1) / rows2, max_slots);
    if (stage_mask & 2) {
        if (x_dtype == SWQ_BF16) hipLaunchKernelGGL(moe_stage2<SWQ_BF16>, grid2, dim3(kThreads12), 0, s, a);
        else hipLaunchKernelGGL(moe_stage2<SWQ_F32>, grid2, dim3(kThreads12), 0, s, a);
        if ((st = launch_status()) != SWQ_OK) return st;
    }
    if (stage_mask & 4) {
        const int nw3 = min(kStage3MaxWaves, max_slots + a.has_shared);
        hipLaunchKernelGGL(moe_stage3, dim3((H + a.rows3 - 1) / a.rows3), dim3(nw3 * kWave), 0, s, a);
        if ((st = launch_status()) != SWQ_OK) return st;
    }
    return SWQ_OK;
}

extern "C" int swq_moe_decode_norm(const swq_moe_layer *layer, const float *h, const float *residual,
                                   const void *norm_weight, int norm_dtype, float norm_eps, float *out,
                                   int32_t *topk_ids, float *topk_weights, void *ws, size_t ws_bytes, void *stream) {
    int st = check_layer(layer, 1, SWQ_F32);
    if (st != SWQ_OK) return st;
    if (!h || !out || !norm_weight) return SWQ_ERR_INVALID_ARGUMENT;
    if (norm_dtype != SWQ_F32 && norm_dtype != SWQ_F16 && norm_dtype != SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if (!(norm_eps >= 0.f)) return SWQ_ERR_INVALID_ARGUMENT;
    const int64_t H = layer->hidden;
    auto overlaps = [H](const float *p, const float *q) { return p && q && p < q + H && q < p + H; };
    if (overlaps(out, h) || overlaps(out, residual)) return SWQ_ERR_INVALID_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(h) % 4 != 0 || reinterpret_cast<uintptr_t>(residual) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(out) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(norm_weight) % (norm_dtype == SWQ_F32 ? 4 : 2) != 0)
        return SWQ_ERR_MISALIGNED;
    const FusedLayout fl = fused_layout(layer, false);
    if (!ws || ws_bytes < decode_ws_bytes(layer, 1, false)) return SWQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(ws) % 256 != 0) return SWQ_ERR_MISALIGNED;
    const FusedPrenorm pn{h, residual, norm_weight, norm_dtype, norm_eps};
    bool taken = false;
    st = fused_decode(layer, nullptr, SWQ_F32, 1, out, SWQ_F32, topk_ids, topk_weights, ws, fl, false,
                      static_cast<hipStream_t>(stream), &taken, &pn);
    if (st != SWQ_OK) return st;
    return taken ? SWQ_OK : SWQ_ERR_LIMIT;
}

extern "C" int swq_moe_decode_stages(const swq_moe_layer *layer, const void *x, int x_dtype, int batch,
                                     void *out, int out_dtype, int32_t *topk_ids, float *topk_weights, void *ws,
                                     size_t ws_bytes, int flags, int stage_mask, void *stream) {
    if (stage_mask == 0) return SWQ_ERR_INVALID_ARGUMENT;
    return moe_decode_impl(layer, x, x_dtype, batch, out, out_dtype, topk_ids, topk_weights, ws, ws_bytes, flags,
                           stage_mask, stream);
}

extern "C" int swq_moe_decode(const swq_moe_layer *layer, const void *x, int x_dtype, int batch, void *out,
                              int out_dtype, int32_t *topk_ids, float *topk_weights, void *ws, size_t ws_bytes,
                              int flags, void *stream) {
    return moe_decode_impl(layer, x, x_dtype, batch, out, out_dtype, topk_ids, topk_weights, ws, ws_bytes, flags, 0,
                           stream);
}

// ---------------------------------------------------------------------------
// swq_moe_decode without a caller workspace: the workspace is `scratch`, a
// static device array of kScratchBytes, one per GPU the library runs on,
// held until the process ends.  Its layout places the single launch's
// exchange regions at the compiled maxima, so calls on any layer and batch
// share it: the epoch counters sit at a fixed place and every call's epoch
// is above those of all words earlier calls left.  Calls that overlap in
// time on one GPU race for it.

constexpr size_t kScratchBytes = static_cast<size_t>(4) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
struct ScratchDevice {
    std::once_flag once;
    std::atomic<uint8_t *> ptr{nullptr};
    std::atomic<int> status{SWQ_ERR_HIP};
};
ScratchDevice g_scratch_dev[64];
}  // namespace

// Once per device, with that device current: the array's device address
// (in host code the array's name is only a stand-in, so it appears nowhere
// but in HIP_SYMBOL here), the single launch's XCD probe (writing into the
// array rather than into an allocation), then the whole array zero-filled by
// a kernel.  Blocking (first call on a device only).
static int scratch_for_device(hipStream_t stream, uint8_t **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return SWQ_ERR_HIP;
    ScratchDevice &d = g_scratch_dev[dev];
    std::call_once(d.once, [&]() {
        void *p = nullptr;
        int st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess && p ? SWQ_OK : SWQ_ERR_HIP;
        if (st == SWQ_OK) st = fused_probe_device(stream, p);
        if (st == SWQ_OK) st = zero_fill(p, kScratchBytes, stream);
        if (st == SWQ_OK && hipStreamSynchronize(stream) != hipSuccess) st = SWQ_ERR_HIP;
        d.ptr.store(static_cast<uint8_t *>(p), std::memory_order_release);
        d.status.store(st, std::memory_order_release);
    });
    const int st = d.status.load(std::memory_order_acquire);
    if (st != SWQ_OK) return st;
    *out = d.ptr.load(std::memory_order_acquire);
    return SWQ_OK;
}

extern "C" int swq_moe_decode_noalloc(const swq_moe_layer *layer, const void *x, int x_dtype, int batch, void *out,
                                      int out_dtype, int32_t *topk_ids, float *topk_weights, int flags,
                                      void *stream) {
    const int st0 = check_layer(layer, batch, SWQ_BF16);
    if (st0 != SWQ_OK) return st0;
    if (decode_ws_bytes(layer, batch, true) > kScratchBytes) return SWQ_ERR_LIMIT;
    uint8_t *ws = nullptr;
    const int st = scratch_for_device(static_cast<hipStream_t>(stream), &ws);
    if (st != SWQ_OK) return st;
    return moe_decode_impl(layer, x, x_dtype, batch, out, out_dtype, topk_ids, topk_weights, ws, kScratchBytes, flags,
                           0, stream, true);
}
