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

// ---------------------------------------------------------------------------
// routing: the top-k rounds on one wave with the keys in registers
//
// Lane l holds experts l*M .. l*M+M-1, sorted by (logit desc, id asc) with a
// stable odd-even transposition sort.  Each round takes the wave-wide
// maximum head; the lowest lane holding it wins (lower lanes hold lower
// ids) and pops its head.  Selection by logit with ties to the lower id
// equals the reference's selection by probability (QwenCPUModel.swift:
// 508-522) except where two distinct logits give the same fp32 probability.

template <int M>
struct Rounds {
    uint32_t key[M];
    int32_t jj[M];
    float lg[M];        // the lane's logits in expert order (-inf past E)
    uint32_t my_key;    // lane k: the key of pick k
    uint32_t top_key;   // the largest key
    int done;           // rounds finished
};

template <int CTRL, int RM>
__device__ __forceinline__ uint32_t dpp_max_step(uint32_t v) {
    return max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, RM, 0xF, false)));
}

// The maximum over the wave, read from lane 63.
__device__ __forceinline__ uint32_t wave_max_bcast(uint32_t v) {
    v = dpp_max_step<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_max_step<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_max_step<0x141, 0xF>(v);  // row_half_mirror
    v = dpp_max_step<0x140, 0xF>(v);  // row_mirror
    v = dpp_max_step<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
    v = dpp_max_step<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

template <int M>
__device__ __forceinline__ void rounds_init(Rounds<M> &r, const float (&v)[M], int E, int lane) {
#pragma unroll
    for (int j = 0; j < M; ++j) {
        const bool valid = lane * M + j < E;
        r.lg[j] = valid ? v[j] : -INFINITY;
        r.key[j] = valid ? orderable(v[j]) : 0u;
        r.jj[j] = j;
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
        for (int j = i & 1; j + 1 < M; j += 2) {
            const bool sw = r.key[j] < r.key[j + 1];
            const uint32_t k0 = r.key[j], k1 = r.key[j + 1];
            const int32_t i0 = r.jj[j], i1 = r.jj[j + 1];
            r.key[j] = sw ? k1 : k0;
            r.key[j + 1] = sw ? k0 : k1;
            r.jj[j] = sw ? i1 : i0;
            r.jj[j + 1] = sw ? i0 : i1;
        }
    }
    r.my_key = 0;
    r.top_key = 0;
    r.done = 0;
}

// Rounds up to (not including) `upto`; pick k goes to s_ids[k] the moment
// its round ends, written by the winning lane.
template <int M>
__device__ __forceinline__ void rounds_run(Rounds<M> &r, int upto, int lane, int32_t *s_ids) {
    for (int k = r.done; k < upto; ++k) {
        const uint32_t gmax = wave_max_bcast(r.key[0]);
        const bool hold = r.key[0] == gmax;
        const uint64_t cand = __ballot(hold);
        // the lowest lane holding the maximum wins: no candidate below it
        // (lane arithmetic only, no scalar find-first round trip)
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(cand >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(cand), 0u));
        const bool pop = hold && below == 0;
        if (pop)
            __hip_atomic_store(&s_ids[k], lane * M + r.jj[0], __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (k == 0) r.top_key = gmax;
        r.my_key = lane == k ? gmax : r.my_key;
#pragma unroll
        for (int j = 0; j + 1 < M; ++j) {
            r.key[j] = pop ? r.key[j + 1] : r.key[j];
            r.jj[j] = pop ? r.jj[j + 1] : r.jj[j];
        }
        r.key[M - 1] = pop ? 0u : r.key[M - 1];
    }
    r.done = max(r.done, upto);
}

// Combine weights: p_k = exp(l_k - max) / sum_e exp(l_e - max) (:65-71),
// w_k = p_k / sum_j p_j when norm (:546-550); the staged path's sums in the
// same order.
template <int M>
__device__ __forceinline__ float rounds_weight(const Rounds<M> &r, int K, int norm, int lane) {
    const float top = from_orderable(r.top_key);
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) part += expf(r.lg[j] - top);  // -inf padding adds 0
    const float denom = wave_sum_all(part);
    const float pk = lane < K ? expf(from_orderable(r.my_key) - top) / denom : 0.f;
    const float total = wave_sum_all(pk);
    return norm ? pk / total : pk;
}

}  // namespace swq
