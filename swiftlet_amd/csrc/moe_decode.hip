// MoE-layer decode step on gfx950: three launches per layer.
//
//   stage 1  router GEMV, shared-expert gate GEMV, shared gate/up SwiGLU;
//            the last router workgroup to finish runs softmax, top-k and
//            renormalisation for every token and (for batches) the
//            distinct-expert list, and publishes them.
//   stage 2  the gate/up SwiGLU rows of every selected expert: one launch
//            for all of them, indexed by the device-resident tables.
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

// Phase stamps of the staged kernels for timing studies (SWQ_FUSED_TRACE
// builds only): s_memrealtime per (workgroup, wave, point) into LDS, copied
// to a global array at the end of the kernel.
#ifdef SWQ_FUSED_TRACE
constexpr int kTraceWaves = 16;  // waves per workgroup the stamps cover
static __device__ unsigned long long g_swq_stage_trace[1024 * kTraceWaves * 16];
extern "C" int swq_stage_trace(void *host, size_t bytes, int clear) {
    if (clear) {
        static unsigned long long z[1024 * kTraceWaves * 16];
        return hipMemcpyToSymbol(HIP_SYMBOL(g_swq_stage_trace), z, sizeof(z)) == hipSuccess ? 0 : -1;
    }
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_swq_stage_trace), bytes) == hipSuccess ? 0 : -1;
}
__device__ __forceinline__ unsigned long long *stage_trace_lds() {
    __shared__ unsigned long long t[kTraceWaves * 16];
    return t;
}
#define STAGE_TRACE_DECL                                                                                \
    if ((threadIdx.x & 63) < 16) stage_trace_lds()[(threadIdx.x >> 6) * 16 + (threadIdx.x & 63)] = 0
#define STAGE_STAMP(n)                                                                                  \
    do {                                                                                                \
        if ((threadIdx.x & 63) == 0 && (n) < 16)                                                        \
            stage_trace_lds()[(threadIdx.x >> 6) * 16 + (n)] = __builtin_amdgcn_s_memrealtime();       \
    } while (0)
#define STAGE_TRACE_FLUSH(base)                                                                         \
    do {                                                                                                \
        __syncthreads();                                                                                \
        for (int i_ = threadIdx.x; i_ < kTraceWaves * 16; i_ += blockDim.x)                             \
            g_swq_stage_trace[((base) + blockIdx.x) * (kTraceWaves * 16) + i_] =                        \
                i_ < static_cast<int>(blockDim.x >> 6) * 16 ? stage_trace_lds()[i_] : 0ull;             \
    } while (0)
#else
#define STAGE_TRACE_DECL \
    do {                 \
    } while (0)
#define STAGE_STAMP(n) \
    do {               \
    } while (0)
#define STAGE_TRACE_FLUSH(base) \
    do {                        \
    } while (0)
#endif

namespace swq {

constexpr int kThreads12 = 256;
constexpr int kMaxPairs = SWQ_MAX_BATCH * SWQ_MAX_TOPK;
constexpr int kRows3 = 16;  // stage-3 rows per workgroup (upper bound)
constexpr int kStage2Blocks = 256;  // stage-2 workgroups at most: one per CU (one wave per SIMD)

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
    int32_t *arrive;       // stage-1 router workgroups done (the last one routes)
    int32_t xdt, odt, accumulate;
    int32_t B, H, E, K, I, Is, norm, has_shared;
    int32_t nr_blocks;     // stage-1 workgroups holding router rows
    int32_t router_tasks;  // router row tiles (one wave each per token)
    int32_t shared_tasks;  // waves with shared gate/up rows
    int32_t rows3;         // stage-3 rows per workgroup
};

// The routing stage 1 published (for batch 1, the picks; for batches, the
// distinct experts), in LDS: expert, pair count and pair list of each slot.
struct Slots {
    int32_t e[kMaxPairs];
    int32_t np[kMaxPairs];
    int16_t pairs[kMaxPairs * SWQ_MAX_BATCH];  // [slot][B]
    int32_t n;
};

// Loads the published routing into sl in one round trip (entries past the
// slot count unused); the caller synchronises before reading it.
__device__ __forceinline__ void load_slots(const MoEArgs &a, Slots &sl) {
    const int P = a.B * a.K;
    for (int t = threadIdx.x; t < P; t += blockDim.x) {
        sl.e[t] = a.B == 1 ? a.ids[t] : a.uniq_e[t];
        sl.np[t] = a.B == 1 ? 1 : a.uniq_np[t];
    }
    for (int t = threadIdx.x; t < P * a.B; t += blockDim.x)
        sl.pairs[t] = static_cast<int16_t>(a.B == 1 ? t : a.uniq_pairs[t]);
    if (threadIdx.x == 0) sl.n = a.B == 1 ? a.K : *a.n_unique;
}

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
// (token b, row) goes to out[b*ld + row].  Token b + 1's activations load
// while token b's dot products run.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void rows_token(const QMat &m, const LaneMap &lm, const RowTile<BITS, CPL, ES> &rt,
                                           const XRaw<XDT, BITS, CPL> &xr, int row0, int row_end, float *out) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    XSlice<BITS, CPL, XF> xs;
    xslice_convert(xs, xr);
    float res[RI];
    dot_tile(res, rt, xs, m, lm);
    if (lm.j == lm.lpr - 1) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int row = row0 + i * lm.rpw + lm.q;
            if (row < row_end) out[row] = res[i];
        }
    }
}

template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void gemv_rows_tokens(const QMat &m, int row0, int row_end, const void *x,
                                                 int H, int B, float *out, int ld, int lane) {
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    RowTile<BITS, CPL, ES> rt;
    load_tile(rt, m, 0, lm, row0, row_end);
    XRaw<XDT, BITS, CPL> xa, xb;
    load_xraw<XDT>(xa, m, lm, x, 0);
#pragma unroll 1
    for (int b = 0; b < B; b += 2) {
        if (b + 1 < B) load_xraw<XDT>(xb, m, lm, x, static_cast<int64_t>(b + 1) * H);
        rows_token<XDT, BITS, CPL, ES, XF>(m, lm, rt, xa, row0, row_end, out + b * ld);
        if (b + 1 >= B) break;
        if (b + 2 < B) load_xraw<XDT>(xa, m, lm, x, static_cast<int64_t>(b + 2) * H);
        rows_token<XDT, BITS, CPL, ES, XF>(m, lm, rt, xb, row0, row_end, out + (b + 1) * ld);
    }
}

// SwiGLU rows of one tile for one token: h[r] = silu(gate_r . x) * (up_r . x).
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void swiglu_token(const QMat &g, const QMat &u, const LaneMap &lm,
                                             const RowTile<BITS, CPL, ES> &tg, const RowTile<BITS, CPL, ES> &tu,
                                             const XRaw<XDT, BITS, CPL> &xr, int row0, int row_end, float *h) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    XSlice<BITS, CPL, XF> xs;
    xslice_convert(xs, xr);
    float rg[RI], ru[RI];
    dot_tile(rg, tg, xs, g, lm);
    dot_tile(ru, tu, xs, u, lm);
    if (lm.j == lm.lpr - 1) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int row = row0 + i * lm.rpw + lm.q;
            if (row < row_end) h[row] = swiglu(rg[i], ru[i]);
        }
    }
}

// SwiGLU rows of one expert for every token b: h[b*ld + r] = silu(gate_r .
// x_b) * (up_r . x_b); token b + 1's activations load while token b's dot
// products run.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void gateup_rows_tokens(const QMat &g, const QMat &u, int64_t expert, int row0,
                                                   int row_end, const void *x, int H, int B, float *h, int ld,
                                                   int lane) {
    const LaneMap lm = lane_map(g.lpr_log2, lane);
    RowTile<BITS, CPL, ES> tg, tu;
    load_tile(tg, g, expert, lm, row0, row_end);
    load_tile(tu, u, expert, lm, row0, row_end);
    XRaw<XDT, BITS, CPL> xa, xb;
    load_xraw<XDT>(xa, g, lm, x, 0);
#pragma unroll 1
    for (int b = 0; b < B; b += 2) {
        if (b + 1 < B) load_xraw<XDT>(xb, g, lm, x, static_cast<int64_t>(b + 1) * H);
        swiglu_token<XDT, BITS, CPL, ES, XF>(g, u, lm, tg, tu, xa, row0, row_end, h + static_cast<int64_t>(b) * ld);
        if (b + 1 >= B) break;
        if (b + 2 < B) load_xraw<XDT>(xa, g, lm, x, static_cast<int64_t>(b + 2) * H);
        swiglu_token<XDT, BITS, CPL, ES, XF>(g, u, lm, tg, tu, xb, row0, row_end,
                                             h + static_cast<int64_t>(b + 1) * ld);
    }
}

// One down tile against one activation row hv: the dot of each row with hv
// lands in prow[row - r0].
template <int BITS, int ES, int XF>
__device__ __forceinline__ void down_tile_row(const QMat &m, const LaneMap &lm, const RowTile<BITS, 1, ES> &dt,
                                              const XRaw<SWQ_F32, BITS, 1> &xr, int r0, int end, float *prow) {
    constexpr int RI = RowTile<BITS, 1, ES>::kRI;
    XSlice<BITS, 1, XF> xs;
    xslice_convert(xs, xr);
    float res[RI];
    dot_tile(res, dt, xs, m, lm);
    if (lm.j == lm.lpr - 1) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int row = r0 + i * lm.rpw + lm.q;
            if (row < end) prow[row - r0] = res[i];
        }
    }
}


// Stage 3's slots for one wave: slots s = s0, s0 + ds, ... below nu, each
// one down tile (rows [r0, r0 + rows3)) against every pair of the slot,
// results to part[p][row - r0].  HELD slots' tiles and first activation
// rows are in flight at once.  SH (the shared expert's down matrix on the
// routed plan): slots 0 .. B-1 are the shared expert's tile against token
// s's activations (results to part[B*K + s]), then the routed slots.
template <int XDT, int BITS, int CPL, int ES, int XF, int HELD = 2, bool SH = false>
__device__ __forceinline__ void down_slots(const MoEArgs &a, const Slots &sl, int s0, int ds, int nu, int r0,
                                           float (*part)[kRows3], int lane) {
    static_assert(XDT == SWQ_F32 && CPL == 1, "down rows read fp32 activations, one chunk per lane");
    const int nsh = SH && a.has_shared ? a.B : 0;
    nu += nsh;
    if (s0 >= nu) return;
    const LaneMap lm = lane_map(a.down.lpr_log2, lane);
    const int end = min(r0 + a.rows3, a.H);
    using Tile = RowTile<BITS, 1, ES>;
    using Raw = XRaw<SWQ_F32, BITS, 1>;
    auto first_pair = [&](int s) { return static_cast<int>(sl.pairs[s * a.B]); };
    // one code path for both kinds of slot: the matrix, expert, activation
    // row and result row selected (wave-uniform)
    auto issue = [&](Tile &t, Raw &xr, int s) __attribute__((always_inline)) {
        const bool sh = SH && s < nsh;
        const int su = s - nsh;
        const QMat &m = sh ? a.sh_down : a.down;
        load_tile(t, m, sh ? 0 : sl.e[su], lm, r0, end);
        load_xraw<SWQ_F32>(xr, m, lm, sh ? a.h_sh : a.h,
                           sh ? static_cast<int64_t>(s) * a.Is : static_cast<int64_t>(first_pair(su)) * a.I);
    };
    auto run = [&](const Tile &t, const Raw &xr, int s) __attribute__((always_inline)) {
        const bool sh = SH && s < nsh;
        s -= nsh;
        down_tile_row<BITS, ES, XF>(sh ? a.sh_down : a.down, lm, t, xr, r0, end,
                                    part[sh ? a.B * a.K + s + nsh : first_pair(s)]);
        if (sh) return;
        const int np = sl.np[s];
        for (int pi = 1; pi < np; ++pi) {
            const int p = sl.pairs[s * a.B + pi];
            Raw xo;
            load_xraw<SWQ_F32>(xo, a.down, lm, a.h, static_cast<int64_t>(p) * a.I);
            down_tile_row<BITS, ES, XF>(a.down, lm, t, xo, r0, end, part[p]);
        }
    };
    // a ring of HELD slots in flight: slot j of each round reuses the
    // buffers of slot j of the previous round
    Tile t[HELD];
    Raw x[HELD];
#pragma unroll
    for (int j = 0; j < HELD; ++j)
        if (s0 + ds * j < nu) issue(t[j], x[j], s0 + ds * j);
    [[maybe_unused]] int k = 2;
    for (int base = 0; s0 + ds * base < nu; base += HELD) {
#pragma unroll
        for (int j = 0; j < HELD; ++j) {
            const int sj = s0 + ds * (base + j);
            if (sj < nu) {
                run(t[j], x[j], sj);
                STAGE_STAMP(k);
                ++k;
                if (sj + ds * HELD < nu) issue(t[j], x[j], sj + ds * HELD);
            }
        }
    }
}

// The shared expert's down rows [r0, r0 + rows3) for every token b:
// part[P + b][row - r0].  rows3 is the routed down matrix's tile height; the
// shared matrix's plan (a longer row: fewer rows per tile) may need several
// of its tiles for it.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void down_shared(const MoEArgs &a, int r0, float (*part)[kRows3], int lane) {
    static_assert(XDT == SWQ_F32 && CPL == 1, "down rows read fp32 activations, one chunk per lane");
    const LaneMap lm = lane_map(a.sh_down.lpr_log2, lane);
    const int end = min(r0 + a.rows3, a.H);
    const int P = a.B * a.K;
    constexpr int RI = RowTile<BITS, 1, ES>::kRI;
#pragma unroll 1
    for (int rp = r0; rp < end; rp += RI * lm.rpw) {
        RowTile<BITS, 1, ES> t;
        load_tile(t, a.sh_down, 0, lm, rp, end);
        XRaw<SWQ_F32, BITS, 1> xa, xb;
        load_xraw<SWQ_F32>(xa, a.sh_down, lm, a.h_sh, 0);
#pragma unroll 1
        for (int b = 0; b < a.B; b += 2) {
            if (b + 1 < a.B) load_xraw<SWQ_F32>(xb, a.sh_down, lm, a.h_sh, static_cast<int64_t>(b + 1) * a.Is);
            down_tile_row<BITS, ES, XF>(a.sh_down, lm, t, xa, rp, end, part[P + b] + (rp - r0));
            if (b + 1 >= a.B) break;
            if (b + 2 < a.B) load_xraw<SWQ_F32>(xa, a.sh_down, lm, a.h_sh, static_cast<int64_t>(b + 2) * a.Is);
            down_tile_row<BITS, ES, XF>(a.sh_down, lm, t, xb, rp, end, part[P + b + 1] + (rp - r0));
        }
    }
}

// ---------------------------------------------------------------------------
// top-k (one wave per token)

// Top-k of one token's router logits on one wave (the rounds of route.hpp):
// picks to ids[k] in pick order, combine weights to w[k].  The same picks,
// weights and summation order as the single launch's routing wave.
template <int M>
__device__ __forceinline__ void topk_token(const float *lrow, int E, int K, int norm, int lane, int32_t *ids,
                                           float *w) {
    float v[M];
#pragma unroll
    for (int j = 0; j < M; ++j) v[j] = lrow[min(lane * M + j, E - 1)];  // every load issued first
    Rounds<M> rd;
    rounds_init(rd, v, E, lane);
    rounds_run(rd, K, lane, ids);
    const float wk = rounds_weight(rd, K, norm, lane);
    if (lane < K) w[lane] = wk;
}

// The block's routing, in LDS.
struct Routing {
    int32_t ids[kMaxPairs];    // [B][K] picks, pair p = b*K + k
    float w[kMaxPairs];        // combine weights
    int32_t lead[kMaxPairs];   // pair leads its expert's list
    int32_t slot[kMaxPairs];   // distinct slot of a leading pair
    int32_t uniq_e[kMaxPairs];
    int32_t uniq_np[kMaxPairs];
    int16_t upairs[kMaxPairs * SWQ_MAX_BATCH];  // [slot][B]: each distinct slot's pairs, in pair order
    int32_t n_unique;
};

// Every token's top-k into r (one wave per token), then for batches the
// distinct experts in order of first appearance, each with its pairs in pair
// order (one thread per pair, two O(P) passes) in r.upairs; with `publish`
// the block also writes the routing to the workspace (and the caller's
// outputs) for stage 3.
__device__ __forceinline__ void route(const MoEArgs &a, Routing &r, bool publish) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int M = (a.E + kWave - 1) / kWave;
    for (int b = wave; b < a.B; b += kThreads12 / kWave) {
        const float *lrow = a.logits + static_cast<int64_t>(b) * a.E;
        int32_t *ids = r.ids + b * a.K;
        float *w = r.w + b * a.K;
        if (M <= 1) topk_token<1>(lrow, a.E, a.K, a.norm, lane, ids, w);
        else if (M <= 2) topk_token<2>(lrow, a.E, a.K, a.norm, lane, ids, w);
        else if (M <= 4) topk_token<4>(lrow, a.E, a.K, a.norm, lane, ids, w);
        else if (M <= 8) topk_token<8>(lrow, a.E, a.K, a.norm, lane, ids, w);
        else topk_token<16>(lrow, a.E, a.K, a.norm, lane, ids, w);
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
        r.upairs[slot * a.B + pos] = static_cast<int16_t>(p);
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


// Tokens per stage-1 router wave.
constexpr int kRouterTokens = 2;

template <int XDT>
__global__ __launch_bounds__(kThreads12) void moe_stage1(MoEArgs a) {
    __shared__ Routing r;
    __shared__ int32_t s_last;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int task = blockIdx.x * (kThreads12 / kWave) + wave;
    if (static_cast<int>(blockIdx.x) < a.nr_blocks) {
        // one (row tile, kRouterTokens tokens) per wave, the waves of a tile
        // side by side: the router's dot products are VALU work, spread over
        // more waves, while the tile's codes come from memory once and then
        // from cache
        const int groups = (a.B + kRouterTokens - 1) / kRouterTokens;
        if (task < a.router_tasks * groups) {
            const int tile = task / groups, b0 = (task - tile * groups) * kRouterTokens;
            const void *xb =
                static_cast<const uint8_t *>(a.x) + static_cast<int64_t>(b0) * a.H * (XDT == SWQ_BF16 ? 2 : 4);
            SWQ_DISPATCH(XDT, a.router, gemv_rows_tokens, a.router, tile * tile_rows(a.router), a.E, xb, a.H,
                         min(kRouterTokens, a.B - b0), a.logits + static_cast<int64_t>(b0) * a.E, a.E, lane);
        }
        // The last router workgroup to finish routes every token (softmax,
        // top-k, the distinct experts) and publishes the tables stage 2 and 3
        // read, while the shared-expert workgroups still run.  Release: this
        // workgroup's logits reach memory before its arrival counts; acquire:
        // the last one sees every workgroup's logits.  Only the last one
        // acquires: an agent-scope acquire invalidates the XCD's L2 under the
        // other workgroups' loads (a full fence here cost ~1 us of stage 1).
        __syncthreads();
        if (threadIdx.x == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            const int32_t old = __hip_atomic_fetch_add(a.arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = old == a.nr_blocks - 1 ? 1 : 0;
        }
        __syncthreads();
        if (s_last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            route(a, r, true);
            if (threadIdx.x == 0) __hip_atomic_store(a.arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    // shared-expert workgroups; the shared down projection is pulled toward
    // the cache for stage 3 meanwhile
    if (!a.has_shared) return;
    const int sb = blockIdx.x - a.nr_blocks;
    const uint32_t t = touch_share(a.sh_down, 0, sb, gridDim.x - a.nr_blocks);
    const int st = task - a.nr_blocks * (kThreads12 / kWave);
    // the shared gate/up rows as the router's: one (row tile, kRouterTokens
    // tokens) per wave
    const int groups = (a.B + kRouterTokens - 1) / kRouterTokens;
    if (st == 0) {
        SWQ_DISPATCH(XDT, a.seg, gemv_rows_tokens, a.seg, 0, 1, a.x, a.H, a.B, a.sg, 1, lane);
    } else if (st - 1 < a.shared_tasks * groups) {
        const int tile = (st - 1) / groups, b0 = (st - 1 - tile * groups) * kRouterTokens;
        const void *xb =
            static_cast<const uint8_t *>(a.x) + static_cast<int64_t>(b0) * a.H * (XDT == SWQ_BF16 ? 2 : 4);
        SWQ_DISPATCH(XDT, a.sh_gate, gateup_rows_tokens, a.sh_gate, a.sh_up, 0, tile * tile_rows(a.sh_gate), a.Is,
                     xb, a.H, min(kRouterTokens, a.B - b0), a.h_sh + static_cast<int64_t>(b0) * a.Is, a.Is, lane);
    }
    keep(t);
}

// Stage 2's work for one wave: units u0, u0 + W, ... below nu, unit u the
// gate/up row tile u % tps of distinct slot u / tps, for every token pair of
// the slot: h[p][row] = silu(gate_row . x_b) * (up_row . x_b).  The next
// unit's tiles and first activation slice load while the current unit's dot
// products run.
__device__ __forceinline__ int64_t unit_expert(const MoEArgs &, const Slots &r, int s) { return r.e[s]; }
__device__ __forceinline__ int unit_pair(const MoEArgs &a, const Slots &r, int s, int pi) {
    return r.pairs[s * a.B + pi];
}

template <int XDT, int BITS, int CPL, int ES>
__device__ __forceinline__ void gateup_issue(const MoEArgs &a, const Slots &r, const LaneMap &lm, int tps, int u,
                                             RowTile<BITS, CPL, ES> &tg, RowTile<BITS, CPL, ES> &tu,
                                             XRaw<XDT, BITS, CPL> &xr) {
    const int s = u / tps, t = u - s * tps, rows = RowTile<BITS, CPL, ES>::kRI * lm.rpw;
    const int64_t e = unit_expert(a, r, s);
    load_tile(tg, a.gate, e, lm, t * rows, a.I);
    load_tile(tu, a.up, e, lm, t * rows, a.I);
    load_xraw<XDT>(xr, a.gate, lm, a.x, static_cast<int64_t>(unit_pair(a, r, s, 0) / a.K) * a.H);
}

// Stage-2 waves per SIMD by plan: 8-bit tiles fit two waves' registers (the
// other wave's dot products fill the issue slots one wave's loads leave
// idle), except with two chunks of fp32 activations per lane; 4-bit ones
// with packed-bf16 activations do not.
template <int XDT, int BITS, int CPL>
constexpr int kStage2Waves = BITS == 8 && (XDT == SWQ_BF16 || CPL == 1) ? 2 : 1;

template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void gateup_pair(const MoEArgs &a, const LaneMap &lm, int row0, int p,
                                            const RowTile<BITS, CPL, ES> &tg, const RowTile<BITS, CPL, ES> &tu,
                                            const XSlice<BITS, CPL, XF> &xs) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    float r[2][RI];
    if constexpr (kStage2Waves<XDT, BITS, CPL> == 1) {
        // both tiles' chunks interleaved: independent chains for a wave that
        // has its SIMD to itself; the same results as a dot_tile per tile
        const RowTile<BITS, CPL, ES> *tiles[2] = {&tg, &tu};
        const QMat *mats[2] = {&a.gate, &a.up};
        dot_tiles<2>(r, tiles, mats, xs, lm);
    } else {
        dot_tile(r[0], tg, xs, a.gate, lm);
        dot_tile(r[1], tu, xs, a.up, lm);
    }
    if (lm.j == lm.lpr - 1) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int row = row0 + i * lm.rpw + lm.q;
            if (row < a.I) a.h[static_cast<int64_t>(p) * a.I + row] = swiglu(r[0][i], r[1][i]);
        }
    }
}

template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void gateup_run(const MoEArgs &a, const Slots &r, const LaneMap &lm, int tps, int u,
                                           const RowTile<BITS, CPL, ES> &tg, const RowTile<BITS, CPL, ES> &tu,
                                           const XRaw<XDT, BITS, CPL> &xr) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const int s = u / tps, t = u - s * tps, row0 = t * RI * lm.rpw;
    {
        // the first pair from the prefetched activations; the rest (tokens
        // sharing this expert) load theirs here.  Kept apart so the two
        // sources are never one runtime-selected array.
        XSlice<BITS, CPL, XF> xs;
        xslice_convert(xs, xr);
        gateup_pair<XDT>(a, lm, row0, unit_pair(a, r, s, 0), tg, tu, xs);
    }
    const int np = r.np[s];
    for (int pi = 1; pi < np; ++pi) {
        const int p = unit_pair(a, r, s, pi);
        XSlice<BITS, CPL, XF> xs;
        load_xslice<XDT>(xs, a.gate, lm, a.x, static_cast<int64_t>(p / a.K) * a.H);
        gateup_pair<XDT>(a, lm, row0, p, tg, tu, xs);
    }
}

template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void gateup_units(const MoEArgs &a, const Slots &r, int u0, int W, int tps, int nu,
                                             int lane) {
    if (u0 >= nu) return;
    const LaneMap lm = lane_map(a.gate.lpr_log2, lane);
    RowTile<BITS, CPL, ES> tg0, tu0, tg1, tu1;
    XRaw<XDT, BITS, CPL> xr0, xr1;
    gateup_issue<XDT>(a, r, lm, tps, u0, tg0, tu0, xr0);
    [[maybe_unused]] int k = 2;
    for (int u = u0; u < nu; u += 2 * W) {
        if (u + W < nu) gateup_issue<XDT>(a, r, lm, tps, u + W, tg1, tu1, xr1);
        gateup_run<XDT, BITS, CPL, ES, XF>(a, r, lm, tps, u, tg0, tu0, xr0);
        STAGE_STAMP(k);
        ++k;
        if (u + W >= nu) break;
        if (u + 2 * W < nu) gateup_issue<XDT>(a, r, lm, tps, u + 2 * W, tg0, tu0, xr0);
        gateup_run<XDT, BITS, CPL, ES, XF>(a, r, lm, tps, u + W, tg1, tu1, xr1);
        STAGE_STAMP(k);
        ++k;
    }
}

// The routing stage 1 published into LDS, then the waves take the (slot,
// row tile) units of the distinct experts' gate/up rows grid-stride.
// One instance per plan of the gate/up matrices, so that each allocates
// only the registers its own tiles need.
template <int XDT, int BITS, int CPL, int ES, int XF>
__global__ __launch_bounds__(kThreads12) __attribute__((amdgpu_waves_per_eu(kStage2Waves<XDT, BITS, CPL>))) void moe_stage2(
    MoEArgs a) {
    __shared__ Slots sl;
    STAGE_TRACE_DECL;
    STAGE_STAMP(0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    load_slots(a, sl);
    __syncthreads();
    STAGE_STAMP(1);
    const int rows = tile_rows(a.gate);
    const int tps = (a.I + rows - 1) / rows;
    const int nu = sl.n * tps;
    const int W = gridDim.x * (kThreads12 / kWave);
    gateup_units<XDT, BITS, CPL, ES, XF>(a, sl, blockIdx.x * (kThreads12 / kWave) + wave, W, tps, nu, lane);
    STAGE_STAMP(15);
    STAGE_TRACE_FLUSH(0);
}

// Stage 2 over `units` wave units: at most the workgroups the device holds at
// once (occupancy x CUs, looked up once per device and instance), each wave
// walking its units grid-stride.
template <int XDT, int BITS, int CPL, int ES, int XF>
void launch_stage2_plan(const MoEArgs &a, int units, hipStream_t s) {
    static std::atomic<int> resident[64];
    constexpr int waves = kThreads12 / kWave;
    int blocks = min(kStage2Blocks, (units + waves - 1) / waves), dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
        int r = resident[dev].load(std::memory_order_acquire);
        if (r == 0) {
            int cus = 0, occ = 0;
            if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, moe_stage2<XDT, BITS, CPL, ES, XF>, kThreads12,
                                                             0) == hipSuccess)
                r = cus * occ;
            r = r > 0 ? r : -1;
            resident[dev].store(r, std::memory_order_release);
        }
        if (r > 0) blocks = min(r, (units + waves - 1) / waves);
    }
    hipLaunchKernelGGL((moe_stage2<XDT, BITS, CPL, ES, XF>), dim3(blocks), dim3(kThreads12), 0, s, a);
}

template <int XDT, int ES>
void launch_stage2_es(const MoEArgs &a, int units, hipStream_t s) {
    if constexpr (XDT == SWQ_BF16) {
        if (a.gate.bits == 4) launch_stage2_plan<XDT, 4, 2, ES, kXBF16>(a, units, s);
        else if (a.gate.cpl == 1) launch_stage2_plan<XDT, 8, 1, ES, kXF32>(a, units, s);
        else launch_stage2_plan<XDT, 8, 2, ES, kXF32>(a, units, s);
    } else {
        if (a.gate.bits == 4) launch_stage2_plan<XDT, 4, 1, ES, kXF32>(a, units, s);
        else if (a.gate.cpl == 1) launch_stage2_plan<XDT, 8, 1, ES, kXF32>(a, units, s);
        else launch_stage2_plan<XDT, 8, 2, ES, kXF32>(a, units, s);
    }
}

template <int XDT>
void launch_stage2(const MoEArgs &a, int units, hipStream_t s) {
    if (a.gate.stype == SWQ_F32) launch_stage2_es<XDT, 4>(a, units, s);
    else launch_stage2_es<XDT, 2>(a, units, s);
}

// One instance per plan of the routed down matrix, at most WAVES waves of
// HELD slots in flight each.  SAME_SH: the shared expert's down matrix has
// the routed one's plan, and its tile joins the slots once per token (else
// one wave runs it on its own plan for every token, before its routed
// slots).  8-bit rows with the shared expert on their plan fit sixteen
// waves (four per SIMD) of one slot each; the rest take eight waves of two.
template <int BITS, int ES, int XF, int WAVES, int HELD, bool SAME_SH>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(WAVES / 4))) void moe_stage3(
    MoEArgs a) {
    __shared__ float part[kMaxPairs + SWQ_MAX_BATCH][kRows3];
    __shared__ float s_w[kMaxPairs];
    __shared__ float s_gate[SWQ_MAX_BATCH];
    __shared__ Slots sl;
    STAGE_TRACE_DECL;
    STAGE_STAMP(0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nw = blockDim.x >> 6;
    const int r0 = blockIdx.x * a.rows3;
    const int P = a.B * a.K;
    load_slots(a, sl);
    // combine weights and shared-gate logits: loaded into registers now,
    // staged in LDS only after the projections, so their latency overlaps.
    // one weight per lane: the host sizes the block 64 * min(WAVES, min(P, E)
    // + shared) lanes, which is >= 512 >= P = B*K <= 256, or >= 64 * P, or
    // >= 64 * E >= 16 * K >= P (and checks P <= blockDim)
    const float w_pre = threadIdx.x < static_cast<unsigned>(P) ? a.wts[threadIdx.x] : 0.f;
    const float sg_pre = (a.has_shared && threadIdx.x < static_cast<unsigned>(a.B)) ? a.sg[threadIdx.x] : 0.f;
    __syncthreads();  // sl
    STAGE_STAMP(1);
    // without SAME_SH: the shared expert's tile on the wave with the fewest
    // routed slots (first, so its loads start with the others')
    if constexpr (!SAME_SH) {
        if (a.has_shared && wave == sl.n % nw) {
            SWQ_DISPATCH_DOWN(a.sh_down, down_shared, a, r0, part, lane);
            STAGE_STAMP(13);
        }
    }
    down_slots<SWQ_F32, BITS, 1, ES, XF, HELD, SAME_SH>(a, sl, wave, nw, sl.n, r0, part, lane);
    STAGE_STAMP(14);
    if (threadIdx.x < static_cast<unsigned>(P)) s_w[threadIdx.x] = w_pre;
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
    STAGE_STAMP(15);
    STAGE_TRACE_FLUSH(512);
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

static int scratch_if_set(uint8_t **out);

extern "C" int swq_moe_workspace_status(void *ws, size_t ws_bytes, int clear, void *stream) {
    if (!ws && ws_bytes == 0) {
        // the current device's swq_moe_decode_noalloc array (nothing ran on
        // this device if it was never set up)
        uint8_t *p = nullptr;
        const int st = scratch_if_set(&p);
        if (st != SWQ_OK || !p) return st;
        ws = p;
        ws_bytes = 256;
    }
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
    a.arrive = reinterpret_cast<int32_t *>(wsb + kWsArriveByte);
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
    a.nr_blocks = (a.router_tasks * ((batch + kRouterTokens - 1) / kRouterTokens) + waves12 - 1) / waves12;
    int shared_blocks = 0;
    if (a.has_shared) {
        const int sh_rows_per_task = tile_rows(a.sh_gate);
        a.shared_tasks = (a.Is + sh_rows_per_task - 1) / sh_rows_per_task;
        // +1: shared gate row
        shared_blocks = (a.shared_tasks * ((batch + kRouterTokens - 1) / kRouterTokens) + 1 + waves12 - 1) / waves12;
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
    const int tps2 = (a.I + tile_rows(a.gate) - 1) / tile_rows(a.gate);
    if (stage_mask & 2) {
        if (x_dtype == SWQ_BF16) launch_stage2<SWQ_BF16>(a, max_slots * tps2, s);
        else launch_stage2<SWQ_F32>(a, max_slots * tps2, s);
        if ((st = launch_status()) != SWQ_OK) return st;
    }
    if (stage_mask & 4) {
        // the shared expert's down matrix on the routed plan (same lane map and tile rows)
        const bool same_sh = !a.has_shared ||
                             (a.sh_down.bits == a.down.bits && a.sh_down.stype == a.down.stype &&
                              a.sh_down.xf == a.down.xf && a.sh_down.cpl == a.down.cpl &&
                              a.sh_down.lpr_log2 == a.down.lpr_log2);
        const bool wide = a.down.bits == 8 && same_sh;
        const int slots3 = max_slots + (same_sh ? batch : 1) * a.has_shared;
        const int nw3 = min(wide ? 16 : 8, slots3);
        if (P > nw3 * kWave) return SWQ_ERR_LIMIT;  // one combine weight per lane
        const dim3 g3((H + a.rows3 - 1) / a.rows3), b3(nw3 * kWave);
        if (wide) {
            if (a.down.stype == SWQ_F32) hipLaunchKernelGGL((moe_stage3<8, 4, kXF32, 16, 1, true>), g3, b3, 0, s, a);
            else hipLaunchKernelGGL((moe_stage3<8, 2, kXF32, 16, 1, true>), g3, b3, 0, s, a);
        } else if (same_sh && a.down.bits == 4) {
            if (a.down.stype == SWQ_F32) hipLaunchKernelGGL((moe_stage3<4, 4, kXBF16X2, 8, 2, true>), g3, b3, 0, s, a);
            else hipLaunchKernelGGL((moe_stage3<4, 2, kXBF16X2, 8, 2, true>), g3, b3, 0, s, a);
        } else if (a.down.stype == SWQ_F32) {
            if (a.down.bits == 4) hipLaunchKernelGGL((moe_stage3<4, 4, kXBF16X2, 8, 2, false>), g3, b3, 0, s, a);
            else hipLaunchKernelGGL((moe_stage3<8, 4, kXF32, 8, 2, false>), g3, b3, 0, s, a);
        } else {
            if (a.down.bits == 4) hipLaunchKernelGGL((moe_stage3<4, 2, kXBF16X2, 8, 2, false>), g3, b3, 0, s, a);
            else hipLaunchKernelGGL((moe_stage3<8, 2, kXF32, 8, 2, false>), g3, b3, 0, s, a);
        }
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
    std::mutex mu;  // serialises the set-up
    std::atomic<uint8_t *> ptr{nullptr};  // set once the set-up succeeded
};
ScratchDevice g_scratch_dev[64];
}  // namespace

static int current_device(int *dev) {
    if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= 64) return SWQ_ERR_HIP;
    return SWQ_OK;
}

// This device's array if its set-up has run (else null).
static int scratch_if_set(uint8_t **out) {
    int dev = 0;
    const int st = current_device(&dev);
    if (st != SWQ_OK) return st;
    *out = g_scratch_dev[dev].ptr.load(std::memory_order_acquire);
    return SWQ_OK;
}

// Once per device, with that device current: the array's device address
// (in host code the array's name is only a stand-in, so it appears nowhere
// but in HIP_SYMBOL here), the single launch's XCD probe (writing into the
// array rather than into an allocation), then the whole array zero-filled by
// a kernel.  Blocking (first call on a device only).  A stream under capture
// cannot run it: the call returns SWQ_ERR_INVALID_ARGUMENT and the set-up
// stays pending, as it does after any failure, for the next call outside
// capture.
static int scratch_for_device(hipStream_t stream, uint8_t **out) {
    int dev = 0;
    int st = current_device(&dev);
    if (st != SWQ_OK) return st;
    ScratchDevice &d = g_scratch_dev[dev];
    uint8_t *p = d.ptr.load(std::memory_order_acquire);
    if (p) {
        *out = p;
        return SWQ_OK;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return SWQ_ERR_HIP;
    if (cs != hipStreamCaptureStatusNone) return SWQ_ERR_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(d.mu);
    p = d.ptr.load(std::memory_order_acquire);
    if (!p) {
        void *q = nullptr;
        st = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) == hipSuccess && q ? SWQ_OK : SWQ_ERR_HIP;
        if (st == SWQ_OK) st = fused_probe_device(stream, q);
        if (st == SWQ_OK) st = zero_fill(q, kScratchBytes, stream);
        if (st == SWQ_OK && hipStreamSynchronize(stream) != hipSuccess) st = SWQ_ERR_HIP;
        if (st != SWQ_OK) return st;
        p = static_cast<uint8_t *>(q);
        d.ptr.store(p, std::memory_order_release);
    }
    *out = p;
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
