// Host-side validation and workspace layout of the MoE decode step, shared by
// the staged and the single-launch paths.
#pragma once

#include "internal.hpp"

namespace swq {

constexpr int kMaxExperts = 1024;
// Byte offset, in the 256-byte workspace header, of the word the
// single-launch path sets when one of its bounded waits runs out.
constexpr size_t kWsErrByte = 64;
constexpr size_t kWsArriveByte = 128;  // the staged path's stage-1 arrival counter (zero between calls)
int zero_fill(void *p, size_t n, hipStream_t stream);

struct WsLayout {
    size_t header, logits, sg, h_sh, ids, wts, n_unique, uniq_e, uniq_np, uniq_pairs, h, total;
};

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

// The staged path's regions, from `base` (after the header and the single
// launch's regions, so that neither depends on the batch).
inline WsLayout ws_layout(const swq_moe_layer *l, int B, size_t base) {
    WsLayout w{};
    size_t off = align256(base);
    auto take = [&](size_t n) {
        const size_t o = off;
        off = align256(off + n);
        return o;
    };
    const size_t P = static_cast<size_t>(B) * l->top_k;
    w.header = 0;  // zeroed by swq_moe_workspace_init; word kWsErrByte/4: the stall record
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

// A matrix of the layer: shape, format and alignment, and whether its plan
// fits the compiled kernels when read with activations of dtype x_dtype
// (reads_h: the fp32 SwiGLU activations of stage 3).
inline int check_vec(const swq_qlinear *l, int out_dim, int in_dim, bool stacked, int E, int x_dtype,
                     bool reads_h) {
    int st = check_linear_shape(l);
    if (st != SWQ_OK) return st;
    if (l->out_dim != out_dim || l->in_dim != in_dim) return SWQ_ERR_BAD_SHAPE;
    if (l->bits != 4 && l->bits != 8) return SWQ_ERR_UNSUPPORTED_BITS;
    if ((static_cast<int64_t>(in_dim) * l->bits) % 128 != 0) return SWQ_ERR_BAD_SHAPE;
    if ((static_cast<int64_t>(l->group_size) * l->bits) % 128 != 0) return SWQ_ERR_BAD_SHAPE;
    if (!vector_path_ok(l, 0, 0, 0)) return SWQ_ERR_MISALIGNED;
    QMat m = make_qmat(l);
    plan_qmat(&m, reads_h ? SWQ_F32 : x_dtype);
    if (!plan_fits(m) || (reads_h && m.cpl != 1)) return SWQ_ERR_LIMIT;
    if (stacked && E > 1 && (l->expert_stride_w == 0 || l->expert_stride_sb == 0)) return SWQ_ERR_INVALID_ARGUMENT;
    return SWQ_OK;
}

inline int check_layer(const swq_moe_layer *l, int B, int x_dtype) {
    if (!l) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->reserved != 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (B <= 0 || l->hidden <= 0 || l->num_experts <= 0 || l->moe_intermediate <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->top_k <= 0 || l->top_k > l->num_experts) return SWQ_ERR_EXPERT_RANGE;
    if (l->top_k > SWQ_MAX_TOPK || B > SWQ_MAX_BATCH || l->num_experts > kMaxExperts) return SWQ_ERR_LIMIT;
    const int H = l->hidden, E = l->num_experts, I = l->moe_intermediate;
    const int xd = x_dtype;
    int st;
    if ((st = check_vec(&l->router, E, H, false, E, xd, false)) != SWQ_OK) return st;
    if ((st = check_vec(&l->gate, I, H, true, E, xd, false)) != SWQ_OK) return st;
    if ((st = check_vec(&l->up, I, H, true, E, xd, false)) != SWQ_OK) return st;
    if ((st = check_vec(&l->down, H, I, true, E, xd, true)) != SWQ_OK) return st;
    if (l->gate.bits != l->up.bits || l->gate.in_dim != l->up.in_dim) return SWQ_ERR_BAD_SHAPE;
    if (l->has_shared) {
        const int Is = l->shared_intermediate;
        if (Is <= 0) return SWQ_ERR_INVALID_ARGUMENT;
        if ((st = check_vec(&l->shared_gate, Is, H, false, 1, xd, false)) != SWQ_OK) return st;
        if ((st = check_vec(&l->shared_up, Is, H, false, 1, xd, false)) != SWQ_OK) return st;
        if ((st = check_vec(&l->shared_down, H, Is, false, 1, xd, true)) != SWQ_OK) return st;
        if ((st = check_vec(&l->shared_expert_gate, 1, H, false, 1, xd, false)) != SWQ_OK) return st;
        if (l->shared_gate.bits != l->shared_up.bits) return SWQ_ERR_BAD_SHAPE;
    }
    return SWQ_OK;
}

// Workspace of a decode call:
//   [0, 256)          header (kWsErrByte: the stall record; kWsArriveByte:
//                     the staged path's stage-1 arrival counter)
//   [256, 4352)       the single launch's per-workgroup epoch counters
//   [4352, ...)       its exchange words (logit replicas, activations,
//                     partial outputs), sized for the layer, or for the
//                     compiled maxima (kFusedMax*) in the scratch of the
//                     no-allocation entry point, so that calls on any layer
//                     and batch can share it
//   then              the staged path's regions (ws_layout)
// Epoch counters at a fixed place keep every call's epoch above those of the
// words any earlier call left, whatever layer it ran.
constexpr int kFusedMaxBlocks = 1024;   // epoch counters kept in step
constexpr int kFusedReplicas = 8;       // logit replicas (one per XCD group)
constexpr int kFusedMaxHidden = 8192;   // the compiled maxima of the scratch layout
constexpr int kFusedMaxInter = 2048;
constexpr int kFusedMaxBatch = 4;       // tokens of one single-launch step
struct FusedLayout {
    size_t gen, logit_x, hsh_x, h_x, part_x, total;
    int rep_stride;
    int max_batch;  // tokens the exchange regions hold
};

inline FusedLayout fused_layout(const swq_moe_layer *l, bool max_shape) {
    FusedLayout f{};
    size_t off = 256;
    auto take = [&](size_t n) {
        const size_t o = off;
        off = align256(off + n);
        return o;
    };
    const size_t E = max_shape ? kMaxExperts : l->num_experts;
    const size_t K = max_shape ? SWQ_MAX_TOPK : l->top_k;
    const size_t I = max_shape ? kFusedMaxInter : l->moe_intermediate;
    const size_t Is = max_shape ? kFusedMaxInter : (l->has_shared ? l->shared_intermediate : 1);
    const size_t H = max_shape ? kFusedMaxHidden : l->hidden;
    // a layer's own layout holds the largest single-launch batch, so that
    // one workspace serves every batch; the compiled-maxima layout (the
    // no-allocation scratch) holds one token
    const size_t Bc = max_shape ? 1 : kFusedMaxBatch;
    f.max_batch = static_cast<int>(Bc);
    // replicas 4 KiB apart plus a 256-byte skew, so they sit in different
    // memory channels
    const size_t rep_bytes = ((E * 8 + 4095) & ~static_cast<size_t>(4095)) + 256;
    f.rep_stride = static_cast<int>(rep_bytes / 8);
    f.gen = take(kFusedMaxBlocks * 4);
    f.logit_x = take(rep_bytes * kFusedReplicas * Bc);  // a set of replicas per token
    f.hsh_x = take(Bc * Is * 8);
    f.h_x = take(Bc * K * I * 8);
    f.part_x = take(Bc * K * H * 8);
    f.total = off;
    return f;
}

// Bytes of the whole decode workspace for `batch` tokens.
inline size_t decode_ws_bytes(const swq_moe_layer *l, int batch, bool max_shape) {
    return ws_layout(l, batch, fused_layout(l, max_shape).total).total;
}

// The single-launch path (moe_fused.hip), in the regions `fl` places.
// fused_decode launches it when the layer, the batch and the device allow
// (*taken), else leaves the work to the caller.  fused_probe_device probes
// the XCD placement once per device; `buf`, if given, is device memory of
// at least kFusedMaxBlocks words it may use instead of allocating.
int fused_probe_device(hipStream_t stream, void *buf = nullptr);
// The layer's post-attention norm folded into the single launch:
// x = rmsnorm(h + residual) * weight, out = (h + residual) + moe(x).
struct FusedPrenorm {
    const float *h, *residual;  // residual may be null
    const void *weight;
    int dtype;
    float eps;
};
int fused_decode(const swq_moe_layer *layer, const void *x, int x_dtype, int batch, void *out, int out_dtype,
                 int32_t *topk_ids, float *topk_weights, void *ws, const FusedLayout &fl, bool accumulate,
                 hipStream_t stream, bool *taken, const FusedPrenorm *prenorm = nullptr);

}  // namespace swq
