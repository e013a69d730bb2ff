// Next-token sampling on the device: SwiftletSession.sample
// (SwiftletSession.swift:226-273) over the lm_head logits.
//
//   1. penalties: banned tokens (suppressed ids, and EOS while it is banned)
//      become -inf, every seen token t loses presence + frequency * count(t)
//      (:227-236).  They go into a per-token delta array of the workspace
//      (zero between calls: step 3 puts the touched entries back to zero).
//   2. each workgroup takes a slice of the vocabulary and keeps its top-K of
//      the penalised logits, sorted by (logit desc, id asc).
//   3. one workgroup merges the slices' lists into the global top-K, then:
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

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(v, off);
        v = o > v ? o : v;
    }
    return v;
}

// The largest key over the workgroup (every thread receives it).
__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t *s_red) {
    v = wave_max_u64(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    uint64_t m = s_red[0];
#pragma unroll
    for (int i = 1; i < kSampleThreads / kWave; ++i) m = s_red[i] > m ? s_red[i] : m;
    return m;
}

struct SampleArgs {
    const float *logits;
    float *delta;              // [vocab], zero between calls
    uint64_t *cand;            // [kSampleSlices][kSampleMaxK]
    const int32_t *seen_ids, *seen_counts, *banned_ids;
    int32_t *out;
    int32_t vocab, n_seen, n_banned, k, slices, slice;
    float temperature, top_p, presence, frequency, u;
};

// step 1 (one workgroup): seen tokens first, then the banned ones (-inf
// whatever the penalty).
__global__ __launch_bounds__(kSampleThreads) void sample_penalise(const SampleArgs a) {
    const float pen = a.presence;
    for (int i = threadIdx.x; i < a.n_seen; i += kSampleThreads) {
        const int t = a.seen_ids[i];
        if (t >= 0 && t < a.vocab) atomicAdd(&a.delta[t], -(pen + a.frequency * static_cast<float>(a.seen_counts[i])));
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.n_banned; i += kSampleThreads) {
        const int t = a.banned_ids[i];
        if (t >= 0 && t < a.vocab) a.delta[t] = -INFINITY;
    }
}

// step 2: the slice's top-k, sorted, into cand[slice][0..k) (missing: 0).
__global__ __launch_bounds__(kSampleThreads) void sample_slices(const SampleArgs a) {
    __shared__ uint64_t s_red[kSampleThreads / kWave];
    const int v0 = blockIdx.x * a.slice;
    uint64_t key[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int v = v0 + j * kSampleThreads + threadIdx.x;
        const int vc = min(v, a.vocab - 1);
        const float l = a.logits[vc] + a.delta[vc];
        key[j] = v < a.vocab && v < v0 + a.slice ? cand_key(l, v) : 0ull;
    }
    // each thread's keys in descending order
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
#pragma unroll
        for (int j = 0; j + 1 < kPerThread - i; ++j) {
            const uint64_t x = key[j], y = key[j + 1];
            key[j] = x > y ? x : y;
            key[j + 1] = x > y ? y : x;
        }
    for (int r = 0; r < a.k; ++r) {
        const uint64_t m = block_max_u64(key[0], s_red);
        if (threadIdx.x == 0) a.cand[blockIdx.x * kSampleMaxK + r] = m;
        if (m != 0ull && key[0] == m) {  // keys are unique (ids differ): one winner pops
#pragma unroll
            for (int j = 0; j + 1 < kPerThread; ++j) key[j] = key[j + 1];
            key[kPerThread - 1] = 0ull;
        }
    }
}

// step 3 (one workgroup): merge, draw, and put the penalised entries back.
__global__ __launch_bounds__(kSampleThreads) void sample_final(const SampleArgs a) {
    __shared__ uint64_t s_red[kSampleThreads / kWave];
    __shared__ uint64_t s_top[kSampleMaxK];
    // thread s walks slice s's sorted list (slices <= kSampleThreads)
    int pos = 0;
    const bool has = static_cast<int>(threadIdx.x) < a.slices;
    uint64_t head = has ? a.cand[threadIdx.x * kSampleMaxK] : 0ull;
    for (int r = 0; r < a.k; ++r) {
        const uint64_t m = block_max_u64(head, s_red);
        if (threadIdx.x == 0) s_top[r] = m;
        if (has && m != 0ull && head == m) {
            ++pos;
            head = pos < a.k ? a.cand[threadIdx.x * kSampleMaxK + pos] : 0ull;
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
            float probs[kSampleMaxK];
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
    // the delta array back to zero for the next call
    for (int i = threadIdx.x; i < a.n_seen; i += kSampleThreads) {
        const int t = a.seen_ids[i];
        if (t >= 0 && t < a.vocab) a.delta[t] = 0.f;
    }
    for (int i = threadIdx.x; i < a.n_banned; i += kSampleThreads) {
        const int t = a.banned_ids[i];
        if (t >= 0 && t < a.vocab) a.delta[t] = 0.f;
    }
}

struct SampleLayout {
    size_t delta, cand, total;
};

SampleLayout sample_layout(int vocab) {
    SampleLayout l{};
    l.delta = 0;
    l.cand = (static_cast<size_t>(vocab) * 4 + 255) & ~static_cast<size_t>(255);
    l.total = l.cand + static_cast<size_t>(kSampleSlices) * kSampleMaxK * 8;
    return l;
}

}  // namespace
}  // namespace swq

using namespace swq;

extern "C" size_t swq_sample_workspace_bytes(int vocab) {
    if (vocab <= 0 || vocab > kSampleSlices * kSampleThreads * kPerThread) return 0;
    return sample_layout(vocab).total;
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
    const SampleLayout l = sample_layout(vocab);
    if (!ws || ws_bytes < l.total) return SWQ_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(ws) % 256 != 0 || reinterpret_cast<uintptr_t>(logits) % 4 != 0)
        return SWQ_ERR_MISALIGNED;
    SampleArgs a{};
    uint8_t *w = static_cast<uint8_t *>(ws);
    a.logits = logits;
    a.delta = reinterpret_cast<float *>(w + l.delta);
    a.cand = reinterpret_cast<uint64_t *>(w + l.cand);
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
    if (n_seen > 0 || n_banned > 0) hipLaunchKernelGGL(sample_penalise, dim3(1), dim3(kSampleThreads), 0, s, a);
    hipLaunchKernelGGL(sample_slices, dim3(a.slices), dim3(kSampleThreads), 0, s, a);
    hipLaunchKernelGGL(sample_final, dim3(1), dim3(kSampleThreads), 0, s, a);
    return launch_status();
}
