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

constexpr int kAttnMaxGroup = 16;  // query heads per kv head
constexpr int kAttnThreads = 512;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kAttnChunk = 64;     // positions per workgroup (one per lane)
constexpr int kAttnMaxRot = 256;

struct AttnArgs {
    const float *q_proj, *k_proj, *v_proj;
    const float *q_norm_w, *k_norm_w;
    float *cache_k, *cache_v;
    float *part;  // [H][splits][hd + 2]
    float *out;   // [H * hd]
    int32_t H, KVH, hd, rot, group, splits, chunk;
    int32_t position;
    float theta, eps, scale;
    // the rotation of `position`: cos and sin of position * theta^(-2j/rot),
    // j < rot/2, from the host (kernel arguments)
    float rope_cos[kAttnMaxRot / 2], rope_sin[kAttnMaxRot / 2];
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
// elements (pairs j, j + rot/2) with the rotation table, in the reference's
// operation order.  The wave's copy goes through `lds` (HD floats) so that a
// lane can read its rotation partner.
template <int HD>
__device__ __forceinline__ void norm_rope(HeadVec<HD> &x, const float *w, float eps, int rot, const float *cs,
                                          const float *sn, float *lds) {
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
                const float c = cs[j], s = sn[j];
                const float a = lds[j], b = lds[j + half];
                x.v[e] = i < half ? a * c - b * s : b * c + a * s;
            }
        }
    }
}

// One workgroup per (64-position chunk, kv head): 8 waves.  The chunk's K
// and V rows are loaded at the start, K row by row (coalesced), V a dim per
// thread:
//   keys    K goes to LDS transposed, [dim][position] (a padded row per dim),
//           so a lane can walk one position's dims without bank conflicts;
//   scores  wave w sums dims [w*hd/8, (w+1)*hd/8) of each position (lane)
//           against each query of the group (broadcast from LDS); the 8
//           partial sums meet in LDS;
//   softmax per query head over the chunk (wave-wide max and sum);
//   values  thread t holds dim t % hd of 64 / (512 / hd) positions and adds
//           p * v for every head; the position groups meet in LDS.
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_partial(const AttnArgs a) {
    constexpr int EPL = HeadVec<HD>::EPL;
    constexpr int DS = HD / kAttnWaves;           // key dims per wave (and K floats per thread)
    constexpr int VW = HD >= 32 ? 4 : 1;          // K load width
    constexpr int NK = DS / VW;                   // K loads per thread
    constexpr int UPR = HD / VW;                  // K load units per row
    constexpr int PG = kAttnThreads / HD;         // position groups of the value pass
    constexpr int PPG = kAttnChunk / PG;          // positions per group
    constexpr int KT = HD * (kAttnChunk + 1);     // transposed K, padded
    constexpr int AC = PG * kAttnMaxGroup * HD;   // value partials
    __shared__ float s_q[kAttnMaxGroup][HD];
    __shared__ float s_knew[HD], s_vnew[HD];
    __shared__ float s_part[kAttnWaves][kAttnMaxGroup][kAttnChunk + 1];
    __shared__ float s_e[kAttnMaxGroup][kAttnChunk];
    __shared__ float s_ml[kAttnMaxGroup][2];
    __shared__ float s_big[KT > AC ? KT : AC];    // transposed K, later the value partials
    const int split = blockIdx.x, g = blockIdx.y;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
    const int p0 = split * kAttnChunk;
    const int np = min(kAttnChunk, a.position + 1 - p0);  // positions of this chunk (the last one may be short)
    const bool has_new = a.position < p0 + kAttnChunk;
    const int pnew = a.position - p0;                     // the new position within the chunk (if has_new)
    const int G = a.group;

    // loads first: K unit f = i * 512 + tid is row f / UPR, dims
    // (f % UPR) * VW ..; V: thread = dim, position group.  Rows past the
    // chunk or at the new position read nothing (row 0 stands in).
    float kr[DS], vr[PPG];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const int f = i * kAttnThreads + tid, r = f / UPR, c = (f % UPR) * VW;
        const bool ok = r < np && r != pnew;
        const float *src = a.cache_k + (static_cast<int64_t>(ok ? p0 + r : 0) * a.KVH + g) * HD + c;
        if constexpr (VW == 4) {
            const float4 v = *reinterpret_cast<const float4 *>(src);
            kr[4 * i] = ok ? v.x : 0.f;
            kr[4 * i + 1] = ok ? v.y : 0.f;
            kr[4 * i + 2] = ok ? v.z : 0.f;
            kr[4 * i + 3] = ok ? v.w : 0.f;
        } else {
            const float v = *src;
            kr[i] = ok ? v : 0.f;
        }
    }
    const int vd = tid % HD, vg = tid / HD;
#pragma unroll
    for (int j = 0; j < PPG; ++j) {
        const int pl = vg * PPG + j;
        const bool ok = pl < np && pl != pnew;
        const float v = a.cache_v[(static_cast<int64_t>(ok ? p0 + pl : 0) * a.KVH + g) * HD + vd];
        vr[j] = ok ? v : 0.f;
    }

    // the new key and value (wave 0 of the chunk holding the position)
    if (has_new && wave == 0) {
        HeadVec<HD> k;
#pragma unroll
        for (int e = 0; e < EPL; ++e) k.v[e] = 0.f;
        if (lane < HeadVec<HD>::LANES) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) k.v[e] = a.k_proj[g * HD + lane * EPL + e];
        }
        norm_rope<HD>(k, a.k_norm_w, a.eps, a.rot, a.rope_cos, a.rope_sin, s_q[0]);
        if (lane < HeadVec<HD>::LANES) {
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
    lds_barrier();
    // the group's queries, normalised and rotated, into LDS
    for (int hh = wave; hh < G; hh += kAttnWaves) {
        const int h = g * G + hh;
        HeadVec<HD> q;
#pragma unroll
        for (int e = 0; e < EPL; ++e) q.v[e] = 0.f;
        if (lane < HeadVec<HD>::LANES) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) q.v[e] = a.q_proj[static_cast<int64_t>(h) * 2 * HD + lane * EPL + e];
        }
        norm_rope<HD>(q, a.q_norm_w, a.eps, a.rot, a.rope_cos, a.rope_sin, s_q[hh]);
        __builtin_amdgcn_wave_barrier();
        if (lane < HeadVec<HD>::LANES) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) s_q[hh][lane * EPL + e] = q.v[e];
        }
    }
    // K into LDS, transposed; the new row from its LDS copy
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const int f = i * kAttnThreads + tid, r = f / UPR, c = (f % UPR) * VW;
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            const float v = (has_new && r == pnew) ? s_knew[c + e] : kr[VW * i + e];
            s_big[(c + e) * (kAttnChunk + 1) + r] = v;
        }
    }
    if (has_new) {
#pragma unroll
        for (int j = 0; j < PPG; ++j)
            if (vg * PPG + j == pnew) vr[j] = s_vnew[vd];
    }
    lds_barrier();

    // scores: partial dots over this wave's dims (lane = position)
    for (int hh = 0; hh < G; ++hh) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < DS; ++i) d += s_big[(wave * DS + i) * (kAttnChunk + 1) + lane] * s_q[hh][wave * DS + i];
        s_part[wave][hh][lane] = d;
    }
    lds_barrier();
    // softmax per head over the chunk: wave w takes heads w, w + 8
    for (int hh = wave; hh < G; hh += kAttnWaves) {
        float sc = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) sc += s_part[w][hh][lane];
        sc = lane < np ? sc * a.scale : -INFINITY;
        const float m = wave_max(sc);
        const float e = lane < np ? expf(sc - m) : 0.f;
        const float l = wave_sum(e);
        s_e[hh][lane] = e;
        if (lane == 0) {
            s_ml[hh][0] = m;
            s_ml[hh][1] = l;
        }
    }
    lds_barrier();
    // values: p * v for every head (the value partials reuse the K space)
    float *s_acc = s_big;
    for (int hh = 0; hh < G; ++hh) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < PPG; ++j) acc += s_e[hh][vg * PPG + j] * vr[j];
        s_acc[(vg * kAttnMaxGroup + hh) * HD + vd] = acc;
    }
    lds_barrier();
    for (int t = tid; t < G * HD; t += kAttnThreads) {
        const int hh = t / HD, d = t % HD;
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < PG; ++q) acc += s_acc[(q * kAttnMaxGroup + hh) * HD + d];
        a.part[(static_cast<int64_t>(g * G + hh) * a.splits + split) * (HD + 2) + d] = acc;
    }
    if (tid < G) {
        float *dst = a.part + (static_cast<int64_t>(g * G + tid) * a.splits + split) * (HD + 2);
        dst[HD] = s_ml[tid][0];
        dst[HD + 1] = s_ml[tid][1];
    }
}

// One workgroup of 1024 threads per query head: the splits' maxima and
// weighted sums reduced across the threads (M = max m_s, L = sum
// exp(m_s - M) l_s), then thread (d, q) sums exp(m_s - M) * acc_s[d] over
// every SG-th split (SG = 1024 / hd), four splits per round; the SG partial
// sums meet in LDS; out = acc / L * sigmoid(gate).
constexpr int kCombineThreads = 1024;

__device__ __forceinline__ float block_reduce(float v, float *s_red, bool is_max) {
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) s_red[threadIdx.x / kWave] = v;
    __syncthreads();
    float r = s_red[0];
    for (int i = 1; i < kCombineThreads / kWave; ++i) r = is_max ? fmaxf(r, s_red[i]) : r + s_red[i];
    return r;
}

template <int HD>
__global__ __launch_bounds__(kCombineThreads) void attn_combine(const AttnArgs a) {
    constexpr int SG = kCombineThreads / HD;
    constexpr int U = 8;  // splits per round of a thread's value loop
    __shared__ float s_red[kCombineThreads / kWave];
    __shared__ float s_acc[SG][HD];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int64_t stride = HD + 2;
    const float *src = a.part + static_cast<int64_t>(h) * a.splits * stride;
    // maxima and sums: one load round per 1024 splits
    float m = -INFINITY, mm[4], ll[4];
    int n = 0;
    for (int s = tid; s < a.splits; s += kCombineThreads, ++n) {
        if (n < 4) {
            mm[n] = src[s * stride + HD];
            ll[n] = src[s * stride + HD + 1];
            m = fmaxf(m, mm[n]);
        } else {
            m = fmaxf(m, src[s * stride + HD]);
        }
    }
    const float M = block_reduce(m, s_red, true);
    float l = 0.f;
    n = 0;
    for (int s = tid; s < a.splits; s += kCombineThreads, ++n)
        l += n < 4 ? expf(mm[n] - M) * ll[n] : expf(src[s * stride + HD] - M) * src[s * stride + HD + 1];
    const float L = block_reduce(l, s_red, false);
    // values: thread (d, q) takes splits q, q + SG, ..., U per round
    const int d = tid % HD, q = tid / HD;
    float acc = 0.f;
    int s = q;
    for (; s + (U - 1) * SG < a.splits; s += U * SG) {
        float w[U], v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            w[u] = src[(s + u * SG) * stride + HD];
            v[u] = src[(s + u * SG) * stride + d];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc += expf(w[u] - M) * v[u];
    }
    for (; s < a.splits; s += SG) acc += expf(src[s * stride + HD] - M) * src[s * stride + d];
    s_acc[q][d] = acc;
    __syncthreads();
    if (tid < HD) {
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < SG; ++i) t += s_acc[i][tid];
        const float gate = a.q_proj[static_cast<int64_t>(h) * 2 * HD + HD + tid];
        a.out[h * HD + tid] = (t / L) * sigmoid_acc(gate);
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
    hipLaunchKernelGGL(attn_partial<HD>, dim3(a.splits, a.KVH), dim3(kAttnThreads), 0, s, a);
    hipLaunchKernelGGL(attn_combine<HD>, dim3(a.H), dim3(kCombineThreads), 0, s, a);
}

}  // namespace
}  // namespace swq

using namespace swq;

extern "C" size_t swq_attention_cache_bytes(const swq_attention_layer *l) {
    return check_layer(l) == SWQ_OK ? 2 * half_cache(l) : 0;
}

extern "C" size_t swq_attention_workspace_bytes(const swq_attention_layer *l) {
    if (check_layer(l) != SWQ_OK) return 0;
    const size_t splits = (static_cast<size_t>(l->max_positions) + kAttnChunk - 1) / kAttnChunk;
    return static_cast<size_t>(l->num_heads) * splits * (l->head_dim + 2) * sizeof(float);
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
    a.chunk = kAttnChunk;
    a.splits = (a.position + kAttnChunk) / kAttnChunk;  // chunks holding positions 0..position
    a.theta = l->rope_theta;
    a.eps = l->norm_eps;
    // the rotation table: powf / cosf / sinf of the reference's float
    // operands (applyRope, QwenCPUModel.swift:356-358), evaluated in double and
    // rounded once, as a correctly rounded float libm returns them
    for (int j = 0; j < a.rot / 2; ++j) {
        const float ex = -static_cast<float>(2 * j) / static_cast<float>(a.rot);
        const float inv_freq = static_cast<float>(std::pow(static_cast<double>(a.theta), static_cast<double>(ex)));
        const float ang = static_cast<float>(a.position) * inv_freq;
        a.rope_cos[j] = static_cast<float>(std::cos(static_cast<double>(ang)));
        a.rope_sin[j] = static_cast<float>(std::sin(static_cast<double>(ang)));
    }
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
