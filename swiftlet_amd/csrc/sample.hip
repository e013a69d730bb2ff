// Next-token sampling on the device: SwiftletSession.sample
// (SwiftletSession.swift:226-273) over the lm_head logits.
//
//   1. each workgroup takes a slice of the vocabulary into LDS, applies the
//      penalties that fall in it (banned tokens -- the suppressed ids, and EOS
//      while it is banned -- become -inf; every seen token t loses
//      presence + frequency * count(t); :227-236) and keeps its top-K,
//      sorted by (logit desc, id asc);
//   2. one workgroup merges the slices' lists into the global top-K, then:
//      temperature <= 0: the first maximum (:238-242); else the top-k
//      candidates (:244-253), p_i = exp((l_i - l_0) / T) (:254), the top-p
//      cut (:256-265) and the draw r = u * sum, first i with r - sum_{<=i} p
//      <= 0 (:266-271), u in [0, 1) from the caller (the reference's
//      Float.random).
// Selection ties go to the lower token id: the reference's greedy loop keeps
// the first maximum and its candidate scan replaces only on a strictly
// larger logit.
#include "internal.hpp"
#include "route.hpp"

namespace swq {
namespace {

constexpr int kSampleThreads = 256;
constexpr int kSampleMaxK = 64;
constexpr int kSampleSlices = 256;  // workgroups of step 2
constexpr int kPerThread = 8;       // logits per thread of step 2 (slice = 2048)

// (logit, id) as one key: larger logit first, then lower id.
__device__ __forceinline__ uint64_t cand_key(float l, int id) {
    return (static_cast<uint64_t>(orderable(l)) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(id));
}
__device__ __forceinline__ int key_id(uint64_t k) { return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(k)); }
__device__ __forceinline__ float key_logit(uint64_t k) { return from_orderable(static_cast<uint32_t>(k >> 32)); }

// The largest key of the wave (every lane receives it): the largest logit
// bits, then the largest id bits among the lanes holding them; DPP and
// scalar maxima only.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
    const uint32_t hi = static_cast<uint32_t>(k >> 32), lo = static_cast<uint32_t>(k);
    const uint32_t mh = wave_max_u32(hi);
    const uint32_t ml = wave_max_u32(hi == mh ? lo : 0u);
    return (static_cast<uint64_t>(mh) << 32) | ml;
}

struct SampleArgs {
    const float *logits;
    uint64_t *cand;            // [kSampleSlices][kSampleMaxK]
    const int32_t *seen_ids, *seen_counts, *banned_ids;
    int32_t *out;
    int32_t vocab, n_seen, n_banned, k, slices, slice;
    float temperature, top_p, presence, frequency, u;
};

// step 1: the slice's penalised logits in LDS, its top-k, sorted, into
// cand[slice][0..k) (missing: 0).  Each wave takes the top-k of its 512
// logits by k rounds of wave maxima (each lane's 8 keys sorted, the winner
// pops its head), then wave 0 merges the four sorted lists the same way.
__global__ __launch_bounds__(kSampleThreads) void sample_slices(const SampleArgs a) {
    __shared__ float s_l[kSampleThreads * kPerThread];
    __shared__ uint64_t s_top[kSampleThreads / kWave][kSampleMaxK];
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int v0 = blockIdx.x * a.slice;
    for (int i = threadIdx.x; i < a.slice; i += kSampleThreads) s_l[i] = a.logits[min(v0 + i, a.vocab - 1)];
    __syncthreads();
    // penalties inside the slice: the seen tokens, then the banned ones
    const float pen = a.presence;
    for (int i = threadIdx.x; i < a.n_seen; i += kSampleThreads) {
        const int t = a.seen_ids[i] - v0;
        if (t >= 0 && t < a.slice) atomicAdd(&s_l[t], -(pen + a.frequency * static_cast<float>(a.seen_counts[i])));
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.n_banned; i += kSampleThreads) {
        const int t = a.banned_ids[i] - v0;
        if (t >= 0 && t < a.slice) s_l[t] = -INFINITY;
    }
    __syncthreads();
    uint64_t key[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int i = wave * (kPerThread * kWave) + j * kWave + lane;
        key[j] = v0 + i < a.vocab ? cand_key(s_l[i], v0 + i) : 0ull;
    }
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
#pragma unroll
        for (int j = 0; j + 1 < kPerThread - i; ++j) {
            const uint64_t x = key[j], y = key[j + 1];
            key[j] = x > y ? x : y;
            key[j + 1] = x > y ? y : x;
        }
    for (int r = 0; r < a.k; ++r) {
        const uint64_t m = wave_max_key(key[0]);
        if (lane == 0) s_top[wave][r] = m;
        if (m != 0ull && key[0] == m) {  // keys are unique (ids differ): one winner pops
#pragma unroll
            for (int j = 0; j + 1 < kPerThread; ++j) key[j] = key[j + 1];
            key[kPerThread - 1] = 0ull;
        }
    }
    __syncthreads();
    if (wave != 0) return;
    // lanes 0..3 walk the four waves' lists
    int pos = 0;
    const bool has = lane < kSampleThreads / kWave;
    uint64_t head = has ? s_top[lane][0] : 0ull;
    for (int r = 0; r < a.k; ++r) {
        const uint64_t m = wave_max_key(head);
        if (lane == 0) a.cand[blockIdx.x * kSampleMaxK + r] = m;
        if (has && m != 0ull && head == m) {
            ++pos;
            head = pos < a.k ? s_top[lane][pos] : 0ull;
        }
    }
}

// step 2 (one workgroup): merge and draw.  The slices' lists come into LDS
// first; wave 0 merges them: lane l walks the lists of slices l, l + 64,
// l + 128, l + 192 (slices <= 256), its best head competes in each round.
constexpr int kMergeK = 24;  // list entries held in LDS per slice (k <= 24)

__global__ __launch_bounds__(kSampleThreads) void sample_final(const SampleArgs a) {
    __shared__ uint64_t s_lists[kSampleSlices * kMergeK];
    __shared__ uint64_t s_top[kSampleMaxK];
    __shared__ float probs[kSampleMaxK];  // the draw's weights (LDS: no private memory)
    constexpr int LPL = kSampleSlices / kWave;  // lists per lane
    const int lane = threadIdx.x & (kWave - 1);
    const bool in_lds = a.k <= kMergeK;
    if (in_lds) {
        for (int i = threadIdx.x; i < a.slices * a.k; i += kSampleThreads) {
            const int sl = i / a.k, r = i - sl * a.k;
            s_lists[sl * kMergeK + r] = a.cand[sl * kSampleMaxK + r];
        }
        __syncthreads();
    }
    auto entry = [&](int sl, int r) {
        return in_lds ? s_lists[sl * kMergeK + r] : a.cand[sl * kSampleMaxK + r];
    };
    if (threadIdx.x < kWave) {
        int pos[LPL];
        uint64_t head[LPL];
#pragma unroll
        for (int q = 0; q < LPL; ++q) {
            const int sl = lane + q * kWave;
            pos[q] = 0;
            head[q] = sl < a.slices ? entry(sl, 0) : 0ull;
        }
        for (int r = 0; r < a.k; ++r) {
            uint64_t best = head[0];
#pragma unroll
            for (int q = 1; q < LPL; ++q) best = head[q] > best ? head[q] : best;
            const uint64_t m = wave_max_key(best);
            if (lane == 0) s_top[r] = m;
#pragma unroll
            for (int q = 0; q < LPL; ++q) {
                if (m != 0ull && head[q] == m) {
                    ++pos[q];
                    head[q] = pos[q] < a.k ? entry(lane + q * kWave, pos[q]) : 0ull;
                }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int pick = key_id(s_top[0]);
        if (a.temperature > 0.f) {
            // candidates with a logit (fewer than k only if the vocabulary is)
            int n = 0;
            while (n < a.k && s_top[n] != 0ull) ++n;
            const float l0 = key_logit(s_top[0]);
            float sum = 0.f;
            for (int i = 0; i < n; ++i) {
                probs[i] = expf((key_logit(s_top[i]) - l0) / a.temperature);
                sum += probs[i];
            }
            if (a.top_p < 1.f) {
                float cum = 0.f;
                int cut = n;
                for (int i = 0; i < n; ++i) {
                    cum += probs[i] / sum;
                    if (cum >= a.top_p) {
                        cut = i + 1;
                        break;
                    }
                }
                n = cut;
                sum = 0.f;
                for (int i = 0; i < n; ++i) sum += probs[i];
            }
            float r = a.u * sum;
            for (int i = 0; i < n; ++i) {
                r -= probs[i];
                if (r <= 0.f) {
                    pick = key_id(s_top[i]);
                    break;
                }
            }
        }
        *a.out = pick;
    }
}

size_t sample_ws_bytes() { return static_cast<size_t>(kSampleSlices) * kSampleMaxK * 8; }

}  // namespace
}  // namespace swq

using namespace swq;

extern "C" size_t swq_sample_workspace_bytes(int vocab) {
    if (vocab <= 0 || vocab > kSampleSlices * kSampleThreads * kPerThread) return 0;
    return sample_ws_bytes();
}

extern "C" int swq_sample(const float *logits, int vocab, const swq_sample_options *opt, const int32_t *seen_ids,
                          const int32_t *seen_counts, int n_seen, const int32_t *banned_ids, int n_banned, float u,
                          int32_t *out_token, void *ws, size_t ws_bytes, void *stream) {
    if (!logits || !opt || !out_token || vocab <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (vocab > kSampleSlices * kSampleThreads * kPerThread) return SWQ_ERR_LIMIT;
    if (n_seen < 0 || n_banned < 0 || (n_seen > 0 && (!seen_ids || !seen_counts)) || (n_banned > 0 && !banned_ids))
        return SWQ_ERR_INVALID_ARGUMENT;
    if (!(u >= 0.f && u < 1.f)) return SWQ_ERR_INVALID_ARGUMENT;
    if (!(opt->presence_penalty >= 0.f) || !(opt->frequency_penalty >= 0.f)) return SWQ_ERR_INVALID_ARGUMENT;
    const bool greedy = !(opt->temperature > 0.f);
    const int k = greedy ? 1 : std::max(1, std::min(opt->top_k, vocab));
    if (k > kSampleMaxK) return SWQ_ERR_LIMIT;
    if (!ws || ws_bytes < sample_ws_bytes()) return SWQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(ws) % 256 != 0 || reinterpret_cast<uintptr_t>(logits) % 4 != 0)
        return SWQ_ERR_MISALIGNED;
    SampleArgs a{};
    uint8_t *w = static_cast<uint8_t *>(ws);
    a.logits = logits;
    a.cand = reinterpret_cast<uint64_t *>(w);
    a.seen_ids = seen_ids;
    a.seen_counts = seen_counts;
    a.banned_ids = banned_ids;
    a.out = out_token;
    a.vocab = vocab;
    a.n_seen = n_seen;
    a.n_banned = n_banned;
    a.k = k;
    a.slice = kSampleThreads * kPerThread;
    a.slices = (vocab + a.slice - 1) / a.slice;
    a.temperature = greedy ? 0.f : opt->temperature;
    a.top_p = opt->top_p;
    a.presence = opt->presence_penalty;
    a.frequency = opt->frequency_penalty;
    a.u = u;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sample_slices, dim3(a.slices), dim3(kSampleThreads), 0, s, a);
    hipLaunchKernelGGL(sample_final, dim3(1), dim3(kSampleThreads), 0, s, a);
    return launch_status();
}
