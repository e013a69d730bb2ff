// MoE-layer decode step on gfx950: three launches per layer.
//
//   stage 1  router GEMV (+ shared-expert gate GEMV + shared gate/up SwiGLU);
//            the last router workgroup to finish runs softmax, top-k and
//            renormalisation and builds the distinct-expert list.
//   stage 2  gate/up SwiGLU of every distinct selected expert, indexed by
//            the device-resident top-k ids (one launch for all experts).
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
#include "tile.hpp"

namespace swq {

constexpr int kRI = 4;  // row passes per wave tile
constexpr int kThreads12 = 256;
constexpr int kMaxPairs = SWQ_MAX_BATCH * SWQ_MAX_TOPK;
constexpr int kMaxExperts = 1024;
constexpr int kRows3 = 16;  // stage-3 rows per workgroup (upper bound)

struct MoEArgs {
    QMat router, gate, up, down, sh_gate, sh_up, sh_down, seg;
    const void *x;
    void *out;
    int32_t *user_ids;
    float *user_w;
    unsigned *counter;     // [1] router workgroups finished (self-resetting)
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

// Wave-uniform dispatch over (bits, chunks per lane, scale bytes) of a
// matrix.  Rows of up to 2048 inputs: 4-bit rows take one 16-byte chunk per
// lane, 8-bit rows one or two (the host rejects wider rows with
// SWQ_ERR_LIMIT).
#define SWQ_DISPATCH_ES(XDT, m, FN, ES, ...)                       \
    do {                                                           \
        if ((m).bits == 4) FN<XDT, 4, 1, ES>(__VA_ARGS__);         \
        else if ((m).cpl == 1) FN<XDT, 8, 1, ES>(__VA_ARGS__);     \
        else FN<XDT, 8, 2, ES>(__VA_ARGS__);                       \
    } while (0)
#define SWQ_DISPATCH(XDT, m, FN, ...)                              \
    do {                                                           \
        if ((m).stype == SWQ_F32) SWQ_DISPATCH_ES(XDT, m, FN, 4, __VA_ARGS__); \
        else SWQ_DISPATCH_ES(XDT, m, FN, 2, __VA_ARGS__);          \
    } while (0)

// Down projections (stage 3): one chunk per lane, i.e. up to 2048 inputs at
// 4 bits and 1024 at 8 bits.
#define SWQ_DISPATCH_DOWN(m, FN, ...)                              \
    do {                                                           \
        if ((m).stype == SWQ_F32) {                                \
            if ((m).bits == 4) FN<0, 4, 1, 4>(__VA_ARGS__);        \
            else FN<0, 8, 1, 4>(__VA_ARGS__);                      \
        } else {                                                   \
            if ((m).bits == 4) FN<0, 4, 1, 2>(__VA_ARGS__);        \
            else FN<0, 8, 1, 2>(__VA_ARGS__);                      \
        }                                                          \
    } while (0)

__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_coherent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Rows [row0, row0 + kRI*rpw) of one matrix against every token's x;
// result of (token b, row) goes to out[b*ld + row].
template <int XDT, int BITS, int CPL, int ES>
__device__ __forceinline__ void gemv_rows_tokens(const QMat &m, int row0, int row_end, const void *x,
                                 int H, int B, float *out, int ld, bool coherent, int lane) {
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    RowTile<BITS, CPL, kRI, ES> rt;
    load_tile(rt, m, 0, lm, row0, row_end);
#pragma unroll 1
    for (int b = 0; b < B; ++b) {
        XSlice<BITS, CPL> xs;
        load_xslice<XDT>(xs, m, lm, x, static_cast<int64_t>(b) * H);
        float res[kRI];
        dot_tile(res, rt, xs, m, lm);
        if (lm.j == 0) {
#pragma unroll
            for (int i = 0; i < kRI; ++i) {
                const int row = row0 + i * lm.rpw + lm.q;
                if (row < row_end) {
                    if (coherent) store_coherent(out + b * ld + row, res[i]);
                    else out[b * ld + row] = res[i];
                }
            }
        }
    }
}

// SwiGLU rows of one expert: h[dst_p*ld + r] = silu(gate_r . x_b) * (up_r . x_b)
// for each (token b, destination p) pair.  pairs == nullptr means p = b.
template <int XDT, int BITS, int CPL, int ES>
__device__ __forceinline__ void gateup_rows(const QMat &g, const QMat &u, int64_t expert, int row0, int row_end,
                            const void *x, int H, const int32_t *pairs, int npairs, int K,
                            float *h, int ld, int lane) {
    const LaneMap lm = lane_map(g.lpr_log2, lane);
    RowTile<BITS, CPL, kRI, ES> tg, tu;
    load_tile(tg, g, expert, lm, row0, row_end);
    load_tile(tu, u, expert, lm, row0, row_end);
#pragma unroll 1
    for (int pi = 0; pi < npairs; ++pi) {
        const int p = pairs ? pairs[pi] : pi;
        const int b = pairs ? p / K : pi;
        XSlice<BITS, CPL> xs;
        load_xslice<XDT>(xs, g, lm, x, static_cast<int64_t>(b) * H);
        float rg[kRI], ru[kRI];
        dot_tile(rg, tg, xs, g, lm);
        dot_tile(ru, tu, xs, u, lm);
        if (lm.j == 0) {
#pragma unroll
            for (int i = 0; i < kRI; ++i) {
                const int row = row0 + i * lm.rpw + lm.q;
                if (row < row_end) h[static_cast<int64_t>(p) * ld + row] = swiglu(rg[i], ru[i]);
            }
        }
    }
}

// Down rows [row0, row0 + nrows) of one expert for each pair p: the dot of
// the row with h[p] lands in part[slot_base + pi][row - row0].
template <int XDT, int BITS, int CPL, int ES>
__device__ __forceinline__ void down_rows(const QMat &m, int64_t expert, int row0, int nrows, int row_end,
                          const float *h, int ld, const int32_t *pairs, int npairs,
                          float (*part)[kRows3], int part_base, int lane) {
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    const int tile_rows = kRI * lm.rpw;
    const int end = min(row0 + nrows, row_end);
#pragma unroll 1
    for (int t0 = row0; t0 < end; t0 += tile_rows) {
        RowTile<BITS, CPL, kRI, ES> rt;
        load_tile(rt, m, expert, lm, t0, end);
#pragma unroll 1
        for (int pi = 0; pi < npairs; ++pi) {
            const int p = pairs ? pairs[pi] : pi;
            XSlice<BITS, CPL> xs;
            load_xslice<0>(xs, m, lm, h, static_cast<int64_t>(p) * ld);
            float res[kRI];
            dot_tile(res, rt, xs, m, lm);
            if (lm.j == 0) {
#pragma unroll
                for (int i = 0; i < kRI; ++i) {
                    const int row = t0 + i * lm.rpw + lm.q;
                    if (row < end) part[part_base + p][row - row0] = res[i];
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// top-k (one wave per token)

__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_orderable(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    for (int off = 32; off > 0; off >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, kWave)));
    return v;
}

// Selection by logit with ties to the lower expert id equals the
// reference's selection by softmax probability (softmax is monotonic) up to
// fp32 ties of exp().  Each lane holds experts lane*M .. lane*M+M-1 as
// 64-bit keys (orderable logit, inverted id), sorted descending; K rounds
// take the wave-wide maximum head.
template <int M>
__device__ __forceinline__ void topk_token(const MoEArgs &a, int b, int lane, int32_t *sel_e, float *sel_l) {
    uint64_t key[M];
    float lg[M];
#pragma unroll
    for (int j = 0; j < M; ++j) {
        const int e = lane * M + j;
        if (e < a.E) {
            const float l = load_coherent(a.logits + static_cast<int64_t>(b) * a.E + e);
            lg[j] = l;
            key[j] = (static_cast<uint64_t>(orderable(l)) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(e));
        } else {
            lg[j] = -INFINITY;
            key[j] = 0;
        }
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
    for (int k = 0; k < a.K; ++k) {
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
        const uint32_t wlo = static_cast<uint32_t>(__shfl(static_cast<int>(lo), winner, kWave));
        if (lane == 0) {
            sel_e[k] = static_cast<int32_t>(0xFFFFFFFFu - wlo);
            sel_l[k] = from_orderable(mhi);
        }
        if (lane == winner) {
#pragma unroll
            for (int j = 0; j + 1 < M; ++j) key[j] = key[j + 1];
            key[M - 1] = 0;
        }
    }
    // softmax denominator over all experts (max = the first pick's logit)
    const float m = __shfl(sel_l[0], 0, kWave);
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) part += (lane * M + j < a.E) ? expf(lg[j] - m) : 0.f;
    const float denom = wave_sum(part);
    if (lane == 0) {
        // p_k = exp(l_k - m) / sum; w_k = p_k / sum_j p_j in pick order
        // (QwenCPUModel.swift:546-550)
        float total = 0.f;
        for (int k = 0; k < a.K; ++k) total += expf(sel_l[k] - m) / denom;
        for (int k = 0; k < a.K; ++k) {
            const float pk = expf(sel_l[k] - m) / denom;
            const float w = a.norm ? pk / total : pk;
            const int idx = b * a.K + k;
            a.ids[idx] = sel_e[k];
            a.wts[idx] = w;
            if (a.user_ids) a.user_ids[idx] = sel_e[k];
            if (a.user_w) a.user_w[idx] = w;
        }
    }
}

// Distinct experts over all (token, pick) pairs p = b*K + k, in order of
// first appearance; each pair joins its expert's list in pair order.  One
// thread per pair (P <= blockDim.x), two O(P) passes over the ids in LDS.
__device__ __forceinline__ void build_unique(const MoEArgs &a, const int32_t *s_ids, int32_t *s_lead, int32_t *s_slot) {
    const int P = a.B * a.K;
    const int p = threadIdx.x;
    int first = p, pos = 0, count = 0;
    if (p < P) {
        const int e = s_ids[p];
        for (int q = 0; q < P; ++q) {
            const bool same = s_ids[q] == e;
            if (same && q < p) {
                first = min(first, q);
                ++pos;
            }
            count += same ? 1 : 0;
        }
        s_lead[p] = (first == p) ? 1 : 0;
    }
    __syncthreads();
    if (p < P && first == p) {
        int rank = 0, total = 0;
        for (int q = 0; q < P; ++q) {
            rank += (q < p) ? s_lead[q] : 0;
            total += s_lead[q];
        }
        s_slot[p] = rank;
        a.uniq_e[rank] = s_ids[p];
        a.uniq_np[rank] = count;
        if (p == 0) *a.n_unique = total;
    }
    __syncthreads();
    if (p < P) a.uniq_pairs[s_slot[first] * a.B + pos] = p;
}

template <int M>
__device__ __forceinline__ void topk_all(const MoEArgs &a, int32_t (*sel_e)[SWQ_MAX_TOPK], float (*sel_l)[SWQ_MAX_TOPK],
                         int32_t *s_ids) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int b = wave; b < a.B; b += kThreads12 / kWave) {
        topk_token<M>(a, b, lane, sel_e[wave], sel_l[wave]);
        if (lane < a.K) s_ids[b * a.K + lane] = sel_e[wave][lane];
    }
}

template <int XDT>
__global__ __launch_bounds__(kThreads12) void moe_stage1(MoEArgs a) {
    __shared__ int32_t s_sel_e[kThreads12 / kWave][SWQ_MAX_TOPK];
    __shared__ float s_sel_l[kThreads12 / kWave][SWQ_MAX_TOPK];
    __shared__ int32_t s_ids[kMaxPairs];
    __shared__ int32_t s_lead[kMaxPairs];
    __shared__ int32_t s_slot[kMaxPairs];
    __shared__ int s_is_last;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int task = blockIdx.x * (kThreads12 / kWave) + wave;

    if (static_cast<int>(blockIdx.x) < a.nr_blocks) {
        if (task < a.router_tasks) {
            const int rows_per_task = kRI * (kWave >> a.router.lpr_log2);
            SWQ_DISPATCH(XDT, a.router, gemv_rows_tokens, a.router, task * rows_per_task, a.E, a.x,
                         a.H, a.B, a.logits, a.E, true, lane);
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            __threadfence();
            const unsigned done = atomicAdd(a.counter, 1u);
            s_is_last = (done == static_cast<unsigned>(a.nr_blocks - 1));
        }
        __syncthreads();
        if (!s_is_last) return;
        __threadfence();
        // the last router workgroup: softmax, top-k, renormalisation
        const int M = (a.E + kWave - 1) / kWave;
        if (M <= 1) topk_all<1>(a, s_sel_e, s_sel_l, s_ids);
        else if (M <= 2) topk_all<2>(a, s_sel_e, s_sel_l, s_ids);
        else if (M <= 4) topk_all<4>(a, s_sel_e, s_sel_l, s_ids);
        else if (M <= 8) topk_all<8>(a, s_sel_e, s_sel_l, s_ids);
        else topk_all<16>(a, s_sel_e, s_sel_l, s_ids);
        __syncthreads();
        build_unique(a, s_ids, s_lead, s_slot);
        if (threadIdx.x == 0) __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // shared-expert workgroups
    const int t = task - a.nr_blocks * (kThreads12 / kWave);
    if (!a.has_shared) return;
    if (t == 0) {
        SWQ_DISPATCH(XDT, a.seg, gemv_rows_tokens, a.seg, 0, 1, a.x, a.H, a.B, a.sg, 1, false, lane);
    } else if (t - 1 < a.shared_tasks) {
        const int rows_per_task = kRI * (kWave >> a.sh_gate.lpr_log2);
        SWQ_DISPATCH(XDT, a.sh_gate, gateup_rows, a.sh_gate, a.sh_up, 0, (t - 1) * rows_per_task, a.Is,
                     a.x, a.H, nullptr, a.B, a.K, a.h_sh, a.Is, lane);
    }
}

template <int XDT>
__global__ __launch_bounds__(kThreads12) void moe_stage2(MoEArgs a) {
    const int slot = blockIdx.y;
    if (slot >= *a.n_unique) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = a.uniq_e[slot];
    const int np = a.uniq_np[slot];
    const int rows_per_task = kRI * (kWave >> a.gate.lpr_log2);
    const int row0 = (blockIdx.x * (kThreads12 / kWave) + wave) * rows_per_task;
    if (row0 >= a.I) return;
    SWQ_DISPATCH(XDT, a.gate, gateup_rows, a.gate, a.up, e, row0, a.I, a.x, a.H,
                 a.uniq_pairs + slot * a.B, np, a.K, a.h, a.I, lane);
}

__global__ __launch_bounds__(1024) void moe_stage3(MoEArgs a) {
    __shared__ float part[kMaxPairs + SWQ_MAX_BATCH][kRows3];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nw = blockDim.x >> 6;
    const int r0 = blockIdx.x * a.rows3;
    const int nu = *a.n_unique;
    const int nslots = nu + (a.has_shared ? 1 : 0);
    const int P = a.B * a.K;
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
    __syncthreads();
    for (int t = threadIdx.x; t < a.B * a.rows3; t += blockDim.x) {
        const int b = t / a.rows3, rr = t - b * a.rows3;
        const int row = r0 + rr;
        if (row >= a.H) continue;
        float acc = 0.f;
        for (int k = 0; k < a.K; ++k) acc += a.wts[b * a.K + k] * part[b * a.K + k][rr];
        if (a.has_shared) acc += sigmoidf_ref(a.sg[b]) * part[P + b][rr];
        const int64_t o = static_cast<int64_t>(b) * a.H + row;
        if (a.odt == SWQ_BF16) {
            static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_rne(acc);
        } else {
            float *out = static_cast<float *>(a.out);
            out[o] = a.accumulate ? out[o] + acc : acc;
        }
    }
}

// ---------------------------------------------------------------------------
// host side

struct WsLayout {
    size_t counter, logits, sg, h_sh, ids, wts, n_unique, uniq_e, uniq_np, uniq_pairs, h, total;
};

static size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

static WsLayout ws_layout(const swq_moe_layer *l, int B) {
    WsLayout w{};
    size_t off = 0;
    auto take = [&](size_t n) {
        const size_t o = off;
        off = align256(off + n);
        return o;
    };
    const size_t P = static_cast<size_t>(B) * l->top_k;
    w.counter = take(256);
    w.logits = take(static_cast<size_t>(B) * l->num_experts * 4);
    w.sg = take(static_cast<size_t>(B) * 4);
    w.h_sh = take(static_cast<size_t>(B) * (l->has_shared ? l->shared_intermediate : 1) * 4);
    w.ids = take(P * 4);
    w.wts = take(P * 4);
    w.n_unique = take(4);
    w.uniq_e = take(P * 4);
    w.uniq_np = take(P * 4);
    w.uniq_pairs = take(P * B * 4);
    w.h = take(P * l->moe_intermediate * 4);
    w.total = off;
    return w;
}

static int check_vec(const swq_qlinear *l, int out_dim, int in_dim, bool stacked, int E, int max_cpl) {
    int st = check_linear_shape(l);
    if (st != SWQ_OK) return st;
    if (l->out_dim != out_dim || l->in_dim != in_dim) return SWQ_ERR_BAD_SHAPE;
    if (l->bits != 4 && l->bits != 8) return SWQ_ERR_UNSUPPORTED_BITS;
    if ((static_cast<int64_t>(in_dim) * l->bits) % 128 != 0) return SWQ_ERR_BAD_SHAPE;
    if ((static_cast<int64_t>(l->group_size) * l->bits) % 128 != 0) return SWQ_ERR_BAD_SHAPE;
    if (!vector_path_ok(l, 0, 0, 0)) return SWQ_ERR_MISALIGNED;
    const int chunks = static_cast<int>(static_cast<int64_t>(in_dim) * l->bits / 128);
    int lpr_log2, cpl;
    lane_plan(chunks, &lpr_log2, &cpl);
    if (cpl > max_cpl || (l->bits == 4 && cpl > 1)) return SWQ_ERR_LIMIT;
    if (stacked && E > 1 && (l->expert_stride_w == 0 || l->expert_stride_sb == 0)) return SWQ_ERR_INVALID_ARGUMENT;
    return SWQ_OK;
}

static int check_layer(const swq_moe_layer *l, int B) {
    if (!l) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->reserved != 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (B <= 0 || l->hidden <= 0 || l->num_experts <= 0 || l->moe_intermediate <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->top_k <= 0 || l->top_k > l->num_experts) return SWQ_ERR_EXPERT_RANGE;
    if (l->top_k > SWQ_MAX_TOPK || B > SWQ_MAX_BATCH || l->num_experts > kMaxExperts) return SWQ_ERR_LIMIT;
    const int H = l->hidden, E = l->num_experts, I = l->moe_intermediate;
    int st;
    if ((st = check_vec(&l->router, E, H, false, E, 2)) != SWQ_OK) return st;
    if ((st = check_vec(&l->gate, I, H, true, E, 2)) != SWQ_OK) return st;
    if ((st = check_vec(&l->up, I, H, true, E, 2)) != SWQ_OK) return st;
    if ((st = check_vec(&l->down, H, I, true, E, 1)) != SWQ_OK) return st;
    if (l->gate.bits != l->up.bits || l->gate.in_dim != l->up.in_dim) return SWQ_ERR_BAD_SHAPE;
    if (l->has_shared) {
        const int Is = l->shared_intermediate;
        if (Is <= 0) return SWQ_ERR_INVALID_ARGUMENT;
        if ((st = check_vec(&l->shared_gate, Is, H, false, 1, 2)) != SWQ_OK) return st;
        if ((st = check_vec(&l->shared_up, Is, H, false, 1, 2)) != SWQ_OK) return st;
        if ((st = check_vec(&l->shared_down, H, Is, false, 1, 1)) != SWQ_OK) return st;
        if ((st = check_vec(&l->shared_expert_gate, 1, H, false, 1, 2)) != SWQ_OK) return st;
        if (l->shared_gate.bits != l->shared_up.bits) return SWQ_ERR_BAD_SHAPE;
    }
    return SWQ_OK;
}

}  // namespace swq

using namespace swq;

extern "C" size_t swq_moe_decode_workspace_bytes(const swq_moe_layer *layer, int batch) {
    if (check_layer(layer, batch) != SWQ_OK) return 0;
    return ws_layout(layer, batch).total;
}

extern "C" int swq_moe_workspace_init(void *ws, size_t ws_bytes, void *stream) {
    if (!ws || ws_bytes < 256) return SWQ_ERR_WORKSPACE;
    return hip_status(hipMemsetAsync(ws, 0, 256, static_cast<hipStream_t>(stream)));
}

extern "C" int swq_moe_decode_stages(const swq_moe_layer *layer, const void *x, int x_dtype, int batch,
                                     void *out, int out_dtype, int32_t *topk_ids, float *topk_weights, void *ws,
                                     size_t ws_bytes, int flags, int stage_mask, void *stream) {
    int st = check_layer(layer, batch);
    if (st != SWQ_OK) return st;
    if (!x || !out) return SWQ_ERR_INVALID_ARGUMENT;
    if (x_dtype != SWQ_F32 && x_dtype != SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if (out_dtype != SWQ_F32 && out_dtype != SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if ((flags & ~SWQ_MOE_ACCUMULATE) != 0) return SWQ_ERR_INVALID_ARGUMENT;
    const bool accumulate = (flags & SWQ_MOE_ACCUMULATE) != 0;
    if (accumulate && out_dtype != SWQ_F32) return SWQ_ERR_UNSUPPORTED_DTYPE;
    const int H = layer->hidden;
    const int xes = x_dtype == SWQ_F32 ? 4 : 2;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || (static_cast<int64_t>(H) * xes) % 16 != 0) return SWQ_ERR_MISALIGNED;
    const WsLayout wl = ws_layout(layer, batch);
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
    a.x = x;
    a.out = out;
    a.user_ids = topk_ids;
    a.user_w = topk_weights;
    a.counter = reinterpret_cast<unsigned *>(wsb + wl.counter);
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
    const int router_rows_per_task = kRI * (kWave >> a.router.lpr_log2);
    a.router_tasks = (a.E + router_rows_per_task - 1) / router_rows_per_task;
    a.nr_blocks = (a.router_tasks + waves12 - 1) / waves12;
    int shared_blocks = 0;
    if (a.has_shared) {
        const int sh_rows_per_task = kRI * (kWave >> a.sh_gate.lpr_log2);
        a.shared_tasks = (a.Is + sh_rows_per_task - 1) / sh_rows_per_task;
        shared_blocks = (a.shared_tasks + 1 + waves12 - 1) / waves12;  // +1: shared gate row
    }
    const int down_rpw = kWave >> a.down.lpr_log2;
    a.rows3 = min(kRows3, kRI * down_rpw);
    if (a.rows3 < 1) a.rows3 = 1;

    if (stage_mask & ~7) return SWQ_ERR_INVALID_ARGUMENT;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (stage_mask & 1) {
        if (x_dtype == SWQ_BF16) hipLaunchKernelGGL(moe_stage1<SWQ_BF16>, dim3(a.nr_blocks + shared_blocks), dim3(kThreads12), 0, s, a);
        else hipLaunchKernelGGL(moe_stage1<SWQ_F32>, dim3(a.nr_blocks + shared_blocks), dim3(kThreads12), 0, s, a);
        if ((st = launch_status()) != SWQ_OK) return st;
    }

    const int P = batch * a.K;
    const int max_slots = min(P, a.E);
    const int rows2 = kRI * (kWave >> a.gate.lpr_log2) * waves12;
    const dim3 grid2((a.I + rows2 - 1) / rows2, max_slots);
    if (stage_mask & 2) {
        if (x_dtype == SWQ_BF16) hipLaunchKernelGGL(moe_stage2<SWQ_BF16>, grid2, dim3(kThreads12), 0, s, a);
        else hipLaunchKernelGGL(moe_stage2<SWQ_F32>, grid2, dim3(kThreads12), 0, s, a);
        if ((st = launch_status()) != SWQ_OK) return st;
    }
    if (stage_mask & 4) {
        const int nw3 = min(16, max_slots + a.has_shared);
        hipLaunchKernelGGL(moe_stage3, dim3((H + a.rows3 - 1) / a.rows3), dim3(nw3 * kWave), 0, s, a);
        if ((st = launch_status()) != SWQ_OK) return st;
    }
    return SWQ_OK;
}

extern "C" int swq_moe_decode(const swq_moe_layer *layer, const void *x, int x_dtype, int batch, void *out,
                              int out_dtype, int32_t *topk_ids, float *topk_weights, void *ws, size_t ws_bytes,
                              int flags, void *stream) {
    return swq_moe_decode_stages(layer, x, x_dtype, batch, out, out_dtype, topk_ids, topk_weights, ws, ws_bytes,
                                 flags, 7, stream);
}
