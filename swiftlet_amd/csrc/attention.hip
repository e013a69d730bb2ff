// Gated GQA attention for one decode token on the device, between q/k/v_proj
// and o_proj: the numerics of QwenCPUModel.attentionForward for one token
// (QwenCPUModel.swift:285-345, applyRope :348-367), which the reference's
// GPU path runs on the host (attnCoreCPU, QwenMetalModel.swift:1086-1134).
//
// Two launches, split over the cached positions:
//   attn_partial  grid (splits, KVH), one wave per query head of the kv
//                 head's group: the head's query RMS-normalised (q_norm) and
//                 rotated (partial NeoX RoPE), the new key likewise (k_norm)
//                 and appended with the new value by the split holding the
//                 current position; then an online softmax over the split's
//                 positions: running max m, sum l and sum of p * v.
//   attn_combine  one wave per query head: the splits merged
//                 (exp(m_s - M) weights), divided by the total, times
//                 sigmoid(gate).
// The cache is f32 [max_positions][KVH][hd] for k and for v, the order in
// which the reference appends rows (state.kv).
#include <cmath>

#include "internal.hpp"

namespace swq {
namespace {

constexpr int kAttnMaxGroup = 16;   // query heads per kv head (waves per workgroup)
constexpr int kAttnMaxSplits = 128;
constexpr int kAttnMinChunk = 64;   // positions per split at least

struct AttnArgs {
    const float *q_proj, *k_proj, *v_proj;
    const float *q_norm_w, *k_norm_w;
    float *cache_k, *cache_v;
    float *part;  // [H][splits][hd + 2]
    float *out;   // [H * hd]
    int32_t H, KVH, hd, rot, group, splits, chunk;
    int32_t position;
    float theta, eps, scale;
};

__device__ __forceinline__ float sigmoid_acc(float v) { return 1.0f / (1.0f + expf(-v)); }

// Element e of a head vector held EPL per lane (lanes >= HD / EPL hold none).
template <int HD>
struct HeadVec {
    static constexpr int EPL = HD >= kWave ? HD / kWave : 1;
    static constexpr int LANES = HD / EPL;
    float v[EPL];
};

// RMS-normalise a head vector (x *= scale * w) and rotate its first `rot`
// elements (pairs j, j + rot/2), with the reference's operation order.  The
// wave's copy goes through `lds` (HD floats) so that a lane can read its
// rotation partner.
template <int HD>
__device__ __forceinline__ void norm_rope(HeadVec<HD> &x, const float *w, float eps, int rot, float theta,
                                          float pos, float *lds) {
    constexpr int EPL = HeadVec<HD>::EPL, LANES = HeadVec<HD>::LANES;
    const int lane = threadIdx.x & (kWave - 1);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) ss += x.v[e] * x.v[e];
    ss = wave_sum(ss);
    const float sc = 1.0f / __fsqrt_rn(ss / static_cast<float>(HD) + eps);
    if (lane < LANES) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            x.v[e] *= sc * w[lane * EPL + e];
            lds[lane * EPL + e] = x.v[e];
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int half = rot / 2;
    if (lane < LANES) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int i = lane * EPL + e;
            if (i < rot) {
                const int j = i < half ? i : i - half;
                // powf / cosf / sinf of the reference's float operands,
                // evaluated in double and rounded once (a correctly rounded
                // float libm gives the same values)
                const float ex = -static_cast<float>(2 * j) / static_cast<float>(rot);
                const float inv_freq = static_cast<float>(pow(static_cast<double>(theta), static_cast<double>(ex)));
                const float ang = pos * inv_freq;
                const float c = static_cast<float>(cos(static_cast<double>(ang)));
                const float s = static_cast<float>(sin(static_cast<double>(ang)));
                const float a = lds[j], b = lds[j + half];
                x.v[e] = i < half ? a * c - b * s : b * c + a * s;
            }
        }
    }
}

template <int HD>
__global__ __launch_bounds__(kAttnMaxGroup *kWave) void attn_partial(const AttnArgs a) {
    constexpr int EPL = HeadVec<HD>::EPL, LANES = HeadVec<HD>::LANES;
    __shared__ float s_vec[kAttnMaxGroup][HD];
    __shared__ float s_knew[HD], s_vnew[HD];
    const int split = blockIdx.x, g = blockIdx.y;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
    const int h = g * a.group + wave;
    const int p0 = split * a.chunk, p1 = min(p0 + a.chunk, a.position + 1);
    const bool has_new = a.position >= p0 && a.position < p1;
    const float pos = static_cast<float>(a.position);

    // the new key (wave 0) and value, only where this split needs them
    if (has_new && wave == 0) {
        HeadVec<HD> k;
#pragma unroll
        for (int e = 0; e < EPL; ++e) k.v[e] = 0.f;
        if (lane < LANES) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) k.v[e] = a.k_proj[g * HD + lane * EPL + e];
        }
        norm_rope<HD>(k, a.k_norm_w, a.eps, a.rot, a.theta, pos, s_vec[0]);
        if (lane < LANES) {
            float *ck = a.cache_k + (static_cast<int64_t>(a.position) * a.KVH + g) * HD;
            float *cv = a.cache_v + (static_cast<int64_t>(a.position) * a.KVH + g) * HD;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int i = lane * EPL + e;
                const float vv = a.v_proj[g * HD + i];
                s_knew[i] = k.v[e];
                s_vnew[i] = vv;
                ck[i] = k.v[e];
                cv[i] = vv;
            }
        }
    }
    __syncthreads();
    // the wave's query
    HeadVec<HD> q;
#pragma unroll
    for (int e = 0; e < EPL; ++e) q.v[e] = 0.f;
    if (lane < LANES) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) q.v[e] = a.q_proj[static_cast<int64_t>(h) * 2 * HD + lane * EPL + e];
    }
    norm_rope<HD>(q, a.q_norm_w, a.eps, a.rot, a.theta, pos, s_vec[wave]);

    float m = -INFINITY, l = 0.f, acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
    for (int p = p0; p < p1; ++p) {
        const float *kp = p == a.position ? s_knew : a.cache_k + (static_cast<int64_t>(p) * a.KVH + g) * HD;
        const float *vp = p == a.position ? s_vnew : a.cache_v + (static_cast<int64_t>(p) * a.KVH + g) * HD;
        float d = 0.f, vv[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) vv[e] = 0.f;
        if (lane < LANES) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int i = lane * EPL + e;
                d += q.v[e] * kp[i];
                vv[e] = vp[i];
            }
        }
        const float s = wave_sum(d) * a.scale;
        const float mn = fmaxf(m, s);
        const float corr = expf(m - mn), w = expf(s - mn);
        l = l * corr + w;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = acc[e] * corr + w * vv[e];
        m = mn;
    }
    float *dst = a.part + (static_cast<int64_t>(h) * a.splits + split) * (HD + 2);
    if (lane < LANES) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) dst[lane * EPL + e] = acc[e];
    }
    if (lane == 0) {
        dst[HD] = m;
        dst[HD + 1] = l;
    }
}

template <int HD>
__global__ __launch_bounds__(kWave) void attn_combine(const AttnArgs a) {
    constexpr int EPL = HeadVec<HD>::EPL, LANES = HeadVec<HD>::LANES;
    const int h = blockIdx.x, lane = threadIdx.x;
    const int used = a.splits;
    const float *src = a.part + static_cast<int64_t>(h) * a.splits * (HD + 2);
    float M = -INFINITY;
    for (int s = 0; s < used; ++s) M = fmaxf(M, src[s * (HD + 2) + HD]);
    float L = 0.f, acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
    for (int s = 0; s < used; ++s) {
        const float *ps = src + s * (HD + 2);
        const float w = expf(ps[HD] - M);
        L += w * ps[HD + 1];
        if (lane < LANES) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[e] += w * ps[lane * EPL + e];
        }
    }
    if (lane < LANES) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int i = lane * EPL + e;
            const float gate = a.q_proj[static_cast<int64_t>(h) * 2 * HD + HD + i];
            a.out[h * HD + i] = (acc[e] / L) * sigmoid_acc(gate);
        }
    }
}

inline size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

int check_layer(const swq_attention_layer *l) {
    if (!l || l->reserved != 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (l->num_heads <= 0 || l->num_kv_heads <= 0 || l->num_heads % l->num_kv_heads != 0) return SWQ_ERR_BAD_SHAPE;
    if (l->num_heads / l->num_kv_heads > kAttnMaxGroup) return SWQ_ERR_LIMIT;
    const int hd = l->head_dim;
    if (hd != 16 && hd != 32 && hd != 64 && hd != 128 && hd != 256) return SWQ_ERR_LIMIT;
    if (l->rotary_dims < 0 || l->rotary_dims > hd || l->rotary_dims % 2 != 0) return SWQ_ERR_BAD_SHAPE;
    if (l->max_positions <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (!(l->rope_theta > 0.f) || !(l->norm_eps >= 0.f)) return SWQ_ERR_INVALID_ARGUMENT;
    if (!l->q_norm_weight || !l->k_norm_weight) return SWQ_ERR_INVALID_ARGUMENT;
    return SWQ_OK;
}

size_t half_cache(const swq_attention_layer *l) {
    return align256(static_cast<size_t>(l->max_positions) * l->num_kv_heads * l->head_dim * sizeof(float));
}

template <int HD>
void launch(const AttnArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(attn_partial<HD>, dim3(a.splits, a.KVH), dim3(a.group * kWave), 0, s, a);
    hipLaunchKernelGGL(attn_combine<HD>, dim3(a.H), dim3(kWave), 0, s, a);
}

}  // namespace
}  // namespace swq

using namespace swq;

extern "C" size_t swq_attention_cache_bytes(const swq_attention_layer *l) {
    return check_layer(l) == SWQ_OK ? 2 * half_cache(l) : 0;
}

extern "C" size_t swq_attention_workspace_bytes(const swq_attention_layer *l) {
    if (check_layer(l) != SWQ_OK) return 0;
    return static_cast<size_t>(l->num_heads) * kAttnMaxSplits * (l->head_dim + 2) * sizeof(float);
}

extern "C" int swq_attention_step(const swq_attention_layer *l, const float *q_proj, const float *k_proj,
                                  const float *v_proj, void *cache, size_t cache_bytes, int64_t position,
                                  float *out, void *ws, size_t ws_bytes, void *stream) {
    int st = check_layer(l);
    if (st != SWQ_OK) return st;
    if (!q_proj || !k_proj || !v_proj || !cache || !out || position < 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (position >= l->max_positions) return SWQ_ERR_LIMIT;
    if (cache_bytes < swq_attention_cache_bytes(l)) return SWQ_ERR_WORKSPACE;
    if (!ws || ws_bytes < swq_attention_workspace_bytes(l)) return SWQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(cache) % 256 != 0 || reinterpret_cast<uintptr_t>(ws) % 256 != 0)
        return SWQ_ERR_MISALIGNED;
    AttnArgs a{};
    a.q_proj = q_proj;
    a.k_proj = k_proj;
    a.v_proj = v_proj;
    a.q_norm_w = l->q_norm_weight;
    a.k_norm_w = l->k_norm_weight;
    a.cache_k = static_cast<float *>(cache);
    a.cache_v = reinterpret_cast<float *>(static_cast<uint8_t *>(cache) + half_cache(l));
    a.part = static_cast<float *>(ws);
    a.out = out;
    a.H = l->num_heads;
    a.KVH = l->num_kv_heads;
    a.hd = l->head_dim;
    a.rot = l->rotary_dims;
    a.group = a.H / a.KVH;
    a.position = static_cast<int32_t>(position);
    const int n = a.position + 1;
    a.chunk = std::max(kAttnMinChunk, (n + kAttnMaxSplits - 1) / kAttnMaxSplits);
    a.splits = (n + a.chunk - 1) / a.chunk;
    a.theta = l->rope_theta;
    a.eps = l->norm_eps;
    a.scale = 1.0f / std::sqrt(static_cast<float>(a.hd));
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (a.hd) {
        case 16: launch<16>(a, s); break;
        case 32: launch<32>(a, s); break;
        case 64: launch<64>(a, s); break;
        case 128: launch<128>(a, s); break;
        default: launch<256>(a, s); break;
    }
    return launch_status();
}
