// Wave-level helpers for routing: order-preserving float keys and wave-wide
// maximum / sum through DPP.
#pragma once

#include "tile.hpp"

namespace swq {

__device__ __forceinline__ uint32_t orderable(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_orderable(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Wave-wide maximum: DPP within each 16-lane row, then the four row maxima
// through scalar registers.  Every lane receives it.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, true));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
    v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
    v = max(v, dpp_u32<0x141>(v));  // row_half_mirror
    v = max(v, dpp_u32<0x140>(v));  // row_mirror
    const uint32_t r0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0));
    const uint32_t r1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16));
    const uint32_t r2 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
    const uint32_t r3 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 48));
    return max(max(r0, r1), max(r2, r3));
}

// Sum over the wave, returned to every lane (the last lane of the DPP scan
// holds it; readlane broadcasts).
__device__ __forceinline__ float wave_sum_all(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(segment_reduce(v, 6)), 63));
}

// routing: top-k of the logits in LDS, one wave

// Lane l holds experts l*M .. l*M+M-1, sorted by (logit desc, id asc); each
// of the K rounds takes the wave-wide maximum head, the lowest lane holding
// it wins (lower lanes hold lower ids), and the winner pops its head.  Lane k
// ends up with pick k.  Selection by logit with ties to the lower id equals
// the reference's selection by probability (QwenCPUModel.swift:508-522)
// except where two distinct logits give the same fp32 probability.
// p_k = exp(l_k - max) / sum_e exp(l_e - max) (:65-71); w_k = p_k / sum_j p_j
// when norm (:546-550).
template <int M>
__device__ __forceinline__ void topk_lds(const float *lg_lds, int E, int K, int norm, int lane, int32_t &my_id,
                                         float &my_w) {
    float lg[M];
    uint32_t key[M];
    int32_t id[M];
#pragma unroll
    for (int j = 0; j < M; ++j) {
        const int e = lane * M + j;
        const float v = lg_lds[min(e, E - 1)];
        lg[j] = e < E ? v : -INFINITY;
        key[j] = e < E ? orderable(v) : 0u;
        id[j] = e;
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
        for (int j = 0; j + 1 < M - i; ++j) {
            const bool sw = key[j] < key[j + 1];
            const uint32_t k0 = key[j], k1 = key[j + 1];
            const int32_t i0 = id[j], i1 = id[j + 1];
            key[j] = sw ? k1 : k0;
            key[j + 1] = sw ? k0 : k1;
            id[j] = sw ? i1 : i0;
            id[j + 1] = sw ? i0 : i1;
        }
    }
    uint32_t top_key = 0, my_key = 0;
    my_id = 0;
    for (int k = 0; k < K; ++k) {
        const uint32_t gmax = wave_max_u32(key[0]);
        const uint64_t cand = __ballot(key[0] == gmax);
        const int winner = cand ? __builtin_ctzll(cand) : 0;
        const int32_t e = __builtin_amdgcn_readlane(id[0], winner);
        if (k == 0) top_key = gmax;
        if (lane == k) {
            my_id = e;
            my_key = gmax;
        }
        if (lane == winner) {
#pragma unroll
            for (int j = 0; j + 1 < M; ++j) {
                key[j] = key[j + 1];
                id[j] = id[j + 1];
            }
            key[M - 1] = 0;
        }
    }
    const float top = from_orderable(top_key);
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) part += expf(lg[j] - top);  // -inf padding adds 0
    const float denom = wave_sum_all(part);
    const float pk = lane < K ? expf(from_orderable(my_key) - top) / denom : 0.f;
    const float total = wave_sum_all(pk);
    my_w = norm ? pk / total : pk;
}

// topk_lds with the per-lane depth M = ceil(E / 64) (E <= 1024).
__device__ __forceinline__ void topk_wave(const float *lg_lds, int E, int K, int norm, int lane, int32_t &my_id,
                                          float &my_w) {
    const int M = (E + kWave - 1) / kWave;
    if (M <= 1) topk_lds<1>(lg_lds, E, K, norm, lane, my_id, my_w);
    else if (M <= 2) topk_lds<2>(lg_lds, E, K, norm, lane, my_id, my_w);
    else if (M <= 4) topk_lds<4>(lg_lds, E, K, norm, lane, my_id, my_w);
    else if (M <= 8) topk_lds<8>(lg_lds, E, K, norm, lane, my_id, my_w);
    else topk_lds<16>(lg_lds, E, K, norm, lane, my_id, my_w);
}

}  // namespace swq
