// Gated DeltaNet decode step on the device: one token through the block
// between its input projections and out_proj, as QwenCPUModel.deltaNetForward
// computes it (QwenCPUModel.swift:371-496) and QwenMetalModel.encDeltaLayer
// encodes it (QwenMetalModel.swift:989-1084: deinterleave_qkvz, conv_step,
// delta_pre, rmsnorm_rows for q/k, gated_delta_step, gated_norm_mul —
// Kernels.metal.txt:126-214, :305-422, :497-519), here in one launch.
//
// One workgroup per value head hv (key head hk = hv / rep, rep = nv / nk):
//   1. conv step + silu of the head's channels — q and k of hk, v of hv —
//      read straight from the projection outputs in either layout (no
//      deinterleave pass); the new mixed row goes into the conv ring;
//   2. g = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b);
//      q and k RMS-normalised without weight (eps 1e-6), q scaled by 1/dk
//      and k by 1/sqrt(dk);
//   3. the recurrence on the head's state rows S[hv][d][:] (dk floats, in
//      place):  S *= g;  delta = (v[d] - S.k) * beta;  S += delta * k;
//      o[d] = S.q — four lanes per row, float4 chunks;
//   4. the gated RMSNorm: y = o * (scale * w) * silu(z).
//
// Conv history: a ring of K rows [K][convD]; the row of position p sits in
// slot p % K.  A step at position p reads slots (p+1 .. p+K-1) % K (positions
// p-K+1 .. p-1) and writes slot p % K, so no workgroup overwrites a row
// another still reads; the q/k channels of a key head are written by the
// workgroup with ri = 0 only.  A zeroed ring is the reference's fresh
// session (zeros before the first token).
#include "internal.hpp"

namespace swq {
namespace {

constexpr int kDnThreads = 512;
constexpr int kDnWaves = kDnThreads / kWave;
constexpr int kDnMaxDv = 1024;
constexpr int kDnMaxConv = 8;

struct DnArgs {
    const float *qkvz, *ba;
    const float *conv_w, *a_log, *dt_bias, *norm_w;
    float *ring;   // [K][convD]
    float *state;  // [nv][dv][dk]
    float *out;    // [nv * dv]
    int32_t nk, nv, dk, dv, K, layout, rep, keyD, valD, convD, slot_new;
    float eps;
};

__device__ __forceinline__ float sigmoid_acc(float v) { return 1.0f / (1.0f + expf(-v)); }
__device__ __forceinline__ float silu_acc(float v) { return v * sigmoid_acc(v); }

// Mixed channel c ([q | k | v] order) of the token's projections.
__device__ __forceinline__ float mixed_in(const DnArgs &a, int c) {
    if (a.layout == SWQ_DELTA_SPLIT) return a.qkvz[c];
    const int chunk = 2 * a.dk + 2 * a.rep * a.dv;
    if (c < a.keyD) return a.qkvz[(c / a.dk) * chunk + c % a.dk];
    if (c < 2 * a.keyD) {
        const int t = c - a.keyD;
        return a.qkvz[(t / a.dk) * chunk + a.dk + t % a.dk];
    }
    const int t = c - 2 * a.keyD, hv = t / a.dv, i = t % a.dv;
    return a.qkvz[(hv / a.rep) * chunk + 2 * a.dk + (hv % a.rep) * a.dv + i];
}

__device__ __forceinline__ float z_in(const DnArgs &a, int hv, int i) {
    if (a.layout == SWQ_DELTA_SPLIT) return a.qkvz[a.convD + hv * a.dv + i];
    const int chunk = 2 * a.dk + 2 * a.rep * a.dv;
    return a.qkvz[(hv / a.rep) * chunk + 2 * a.dk + a.rep * a.dv + (hv % a.rep) * a.dv + i];
}

// b (which = 0) or a (which = 1) of value head hv.
__device__ __forceinline__ float ba_in(const DnArgs &a, int hv, int which) {
    if (a.layout == SWQ_DELTA_SPLIT) return a.ba[which * a.nv + hv];
    return a.ba[(hv / a.rep) * 2 * a.rep + which * a.rep + hv % a.rep];
}

__device__ __forceinline__ float block_sum(float v, float *s_part) {
    v = wave_sum(v);
    __syncthreads();  // s_part may still be read by an earlier reduction
    if ((threadIdx.x & (kWave - 1)) == 0) s_part[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kDnWaves; ++i) t += s_part[i];
    return t;
}

template <int DK>
__global__ __launch_bounds__(kDnThreads) void deltanet_step_kernel(const DnArgs a) {
    constexpr int C4 = DK / 4;            // float4 chunks per state row
    constexpr int G = C4 < 4 ? C4 : 4;    // lanes per row
    constexpr int CPL = C4 / G;           // chunks per lane
    constexpr int RPW = kWave / G;        // rows per wave and pass
    __shared__ float s_q[DK], s_k[DK];
    __shared__ float s_v[kDnMaxDv], s_o[kDnMaxDv];
    __shared__ float s_part[kDnWaves];
    __shared__ float s_gb[2];
    const int hv = blockIdx.x, hk = hv / a.rep, ri = hv % a.rep;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;

    // the state rows of the recurrence's first pass, loaded before the conv
    // step: they depend on nothing the step computes, and their round trip
    // then overlaps its loads and the norms
    const int gl = lane % G;
    float *st_head = a.state + static_cast<int64_t>(hv) * a.dv * DK;
    const int row_first = wave * RPW + lane / G;
    float4 s0[CPL];
    if (row_first < a.dv) {
        const float4 *sr = reinterpret_cast<const float4 *>(st_head + static_cast<int64_t>(row_first) * DK);
#pragma unroll
        for (int m = 0; m < CPL; ++m) s0[m] = sr[gl + G * m];
    }
    // and the gated norm's inputs of this thread's first output (z and the
    // norm weight), which would otherwise cost a round trip at the end
    float z0 = 0.f, nw0 = 0.f;
    if (tid < a.dv) {
        z0 = z_in(a, hv, tid);
        nw0 = a.norm_w[tid];
    }
    asm volatile("" ::: "memory");

    // 1. conv step + silu (acc += w[c][j] * row_j, j = 0..K-1, the newest
    // row last; multiply and add rounded separately as the reference does)
    const int nch = 2 * DK + a.dv;
    for (int t = tid; t < nch; t += kDnThreads) {
        int c;
        float *dst;
        bool own;
        if (t < DK) {
            c = hk * DK + t;
            dst = &s_q[t];
            own = ri == 0;
        } else if (t < 2 * DK) {
            c = a.keyD + hk * DK + (t - DK);
            dst = &s_k[t - DK];
            own = ri == 0;
        } else {
            c = 2 * a.keyD + hv * a.dv + (t - 2 * DK);
            dst = &s_v[t - 2 * DK];
            own = true;
        }
        const float xn = mixed_in(a, c);
        const float *w = a.conv_w + static_cast<int64_t>(c) * a.K;
        float acc = 0.f;
        for (int j = 0; j + 1 < a.K; ++j) {
            const int slot = (a.slot_new + 1 + j) % a.K;
            acc = __fadd_rn(acc, __fmul_rn(w[j], a.ring[static_cast<int64_t>(slot) * a.convD + c]));
        }
        acc = __fadd_rn(acc, __fmul_rn(w[a.K - 1], xn));
        *dst = silu_acc(acc);
        if (own) a.ring[static_cast<int64_t>(a.slot_new) * a.convD + c] = xn;
    }
    // 2. gates (delta_pre, softplus as log1p(exp(.)) below 20)
    if (tid == 0) {
        const float av = ba_in(a, hv, 1) + a.dt_bias[hv];
        const float sp = av > 20.f ? av : log1pf(expf(av));
        s_gb[0] = expf(-expf(a.a_log[hv]) * sp);
        s_gb[1] = sigmoid_acc(ba_in(a, hv, 0));
    }
    __syncthreads();
    float ssq = 0.f, ssk = 0.f;
    for (int i = tid; i < DK; i += kDnThreads) {
        ssq += s_q[i] * s_q[i];
        ssk += s_k[i] * s_k[i];
    }
    ssq = block_sum(ssq, s_part);
    ssk = block_sum(ssk, s_part);
    const float inv = 1.0f / __fsqrt_rn(static_cast<float>(DK));
    const float scq = 1.0f / __fsqrt_rn(ssq / static_cast<float>(DK) + 1e-6f);
    const float sck = 1.0f / __fsqrt_rn(ssk / static_cast<float>(DK) + 1e-6f);
    const float g = s_gb[0], beta = s_gb[1];

    // 3. recurrence: lane group of G lanes per row, chunk m of lane j is
    // chunk j + G*m of the row (G consecutive 16-byte chunks per load)
    float4 qv[CPL], kv[CPL];
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
        const int e = 4 * (gl + G * m);
        qv[m] = make_float4(s_q[e] * scq * (inv * inv), s_q[e + 1] * scq * (inv * inv), s_q[e + 2] * scq * (inv * inv),
                            s_q[e + 3] * scq * (inv * inv));
        kv[m] = make_float4(s_k[e] * sck * inv, s_k[e + 1] * sck * inv, s_k[e + 2] * sck * inv, s_k[e + 3] * sck * inv);
    }
    for (int row = row_first; row < a.dv; row += kDnWaves * RPW) {
        float4 *sr = reinterpret_cast<float4 *>(st_head + static_cast<int64_t>(row) * DK);
        float4 s[CPL];
#pragma unroll
        for (int m = 0; m < CPL; ++m) s[m] = row == row_first ? s0[m] : sr[gl + G * m];
        float mem = 0.f;
#pragma unroll
        for (int m = 0; m < CPL; ++m) {
            s[m].x *= g;
            s[m].y *= g;
            s[m].z *= g;
            s[m].w *= g;
            mem += s[m].x * kv[m].x + s[m].y * kv[m].y + s[m].z * kv[m].z + s[m].w * kv[m].w;
        }
        mem = segment_sum(mem, G);
        const float delta = (s_v[row] - mem) * beta;
        float o = 0.f;
#pragma unroll
        for (int m = 0; m < CPL; ++m) {
            s[m].x += kv[m].x * delta;
            s[m].y += kv[m].y * delta;
            s[m].z += kv[m].z * delta;
            s[m].w += kv[m].w * delta;
            o += s[m].x * qv[m].x + s[m].y * qv[m].y + s[m].z * qv[m].z + s[m].w * qv[m].w;
            sr[gl + G * m] = s[m];
        }
        o = segment_sum(o, G);
        if (gl == 0) s_o[row] = o;
    }
    __syncthreads();

    // 4. gated RMSNorm: y = o * (scale * w) * silu(z)
    float sso = 0.f;
    for (int i = tid; i < a.dv; i += kDnThreads) sso += s_o[i] * s_o[i];
    sso = block_sum(sso, s_part);
    const float sc = 1.0f / __fsqrt_rn(sso / static_cast<float>(a.dv) + a.eps);
    for (int i = tid; i < a.dv; i += kDnThreads) {
        const float y = s_o[i] * (sc * (i == tid ? nw0 : a.norm_w[i]));
        a.out[hv * a.dv + i] = y * silu_acc(i == tid ? z0 : z_in(a, hv, i));
    }
}

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

int check_layer(const swq_deltanet_layer *l) {
    if (!l) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->reserved != 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->num_key_heads <= 0 || l->num_value_heads <= 0 || l->num_value_heads % l->num_key_heads != 0)
        return SWQ_ERR_BAD_SHAPE;
    if (l->key_head_dim <= 0 || l->value_head_dim <= 0 || l->conv_kernel <= 0) return SWQ_ERR_BAD_SHAPE;
    const int dk = l->key_head_dim;
    if (dk != 8 && dk != 16 && dk != 32 && dk != 64 && dk != 128 && dk != 256) return SWQ_ERR_LIMIT;
    if (l->value_head_dim > kDnMaxDv || l->conv_kernel > kDnMaxConv) return SWQ_ERR_LIMIT;
    if (l->layout != SWQ_DELTA_INTERLEAVED && l->layout != SWQ_DELTA_SPLIT) return SWQ_ERR_INVALID_ARGUMENT;
    if (!(l->norm_eps >= 0.f)) return SWQ_ERR_INVALID_ARGUMENT;
    if (!l->conv_weight || !l->a_log || !l->dt_bias || !l->norm_weight) return SWQ_ERR_INVALID_ARGUMENT;
    return SWQ_OK;
}

size_t ring_bytes(const swq_deltanet_layer *l) {
    const int64_t convD = 2LL * l->num_key_heads * l->key_head_dim + 1LL * l->num_value_heads * l->value_head_dim;
    return align256(static_cast<size_t>(l->conv_kernel) * convD * 4);
}

}  // namespace
}  // namespace swq

using namespace swq;

extern "C" size_t swq_deltanet_state_bytes(const swq_deltanet_layer *l) {
    if (check_layer(l) != SWQ_OK) return 0;
    return ring_bytes(l) +
           static_cast<size_t>(l->num_value_heads) * l->value_head_dim * l->key_head_dim * sizeof(float);
}

extern "C" int swq_deltanet_step(const swq_deltanet_layer *l, const float *qkvz, const float *ba, void *state,
                                 size_t state_bytes, int64_t position, float *out, void *stream) {
    int st = check_layer(l);
    if (st != SWQ_OK) return st;
    if (!qkvz || !ba || !state || !out || position < 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (state_bytes < swq_deltanet_state_bytes(l)) return SWQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(state) % 256 != 0 || reinterpret_cast<uintptr_t>(qkvz) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(ba) % 4 != 0 || reinterpret_cast<uintptr_t>(out) % 4 != 0)
        return SWQ_ERR_MISALIGNED;
    DnArgs a{};
    a.qkvz = qkvz;
    a.ba = ba;
    a.conv_w = l->conv_weight;
    a.a_log = l->a_log;
    a.dt_bias = l->dt_bias;
    a.norm_w = l->norm_weight;
    a.ring = static_cast<float *>(state);
    a.state = reinterpret_cast<float *>(static_cast<uint8_t *>(state) + ring_bytes(l));
    a.out = out;
    a.nk = l->num_key_heads;
    a.nv = l->num_value_heads;
    a.dk = l->key_head_dim;
    a.dv = l->value_head_dim;
    a.K = l->conv_kernel;
    a.layout = l->layout;
    a.rep = a.nv / a.nk;
    a.keyD = a.nk * a.dk;
    a.valD = a.nv * a.dv;
    a.convD = 2 * a.keyD + a.valD;
    a.slot_new = static_cast<int32_t>(position % a.K);
    a.eps = l->norm_eps;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(a.nv), block(kDnThreads);
    switch (a.dk) {
        case 8: hipLaunchKernelGGL(deltanet_step_kernel<8>, grid, block, 0, s, a); break;
        case 16: hipLaunchKernelGGL(deltanet_step_kernel<16>, grid, block, 0, s, a); break;
        case 32: hipLaunchKernelGGL(deltanet_step_kernel<32>, grid, block, 0, s, a); break;
        case 64: hipLaunchKernelGGL(deltanet_step_kernel<64>, grid, block, 0, s, a); break;
        case 128: hipLaunchKernelGGL(deltanet_step_kernel<128>, grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL(deltanet_step_kernel<256>, grid, block, 0, s, a); break;
    }
    return launch_status();
}
