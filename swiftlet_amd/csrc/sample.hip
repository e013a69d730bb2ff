// Next-token sampling on the device: SwiftletSession.sample
// (SwiftletSession.swift:226-273) over the lm_head logits, one launch.
//
//   1. each workgroup takes a 2048-logit slice of the vocabulary into LDS,
//      applies the penalties that fall in it (banned tokens -- the suppressed
//      ids, and EOS while it is banned -- become -inf; every seen token t
//      loses presence + frequency * count(t); :227-236) and writes its top-K,
//      sorted by (logit desc, id asc), to the workspace;
//   2. the last workgroup to finish step 1 (an arrival counter in the
//      workspace, reset by that workgroup) selects the global top-K from the
//      slices' lists, then: temperature <= 0: the first maximum (:238-242);
//      else the top-k candidates (:244-253), p_i = exp((l_i - l_0) / T)
//      (:254), the top-p cut (:256-265) and the draw r = u * sum, first i
//      with r - sum_{<=i} p <= 0 (:266-271), u in [0, 1) from the caller (the
//      reference's Float.random).
// Selection ties go to the lower token id: the reference's greedy loop keeps
// the first maximum and its candidate scan replaces only on a strictly
// larger logit.
//
// Selection without sequential rounds: a lower bound t of the K-th largest
// value (each wave's K-th largest lane value by rank, the largest of those),
// every value >= t compacted into LDS (at least K of them), each one's rank
// among those counted in parallel, rank < K placed at its position.
#include "internal.hpp"
#include "route.hpp"

namespace swq {
namespace {

constexpr int kSampleThreads = 256;
constexpr int kSampleWaves = kSampleThreads / kWave;
constexpr int kSampleMaxK = 64;
constexpr int kSampleSlices = 256;  // workgroups (vocabulary slices) at most
constexpr int kPerThread = 8;       // logits per thread (slice = 2048)
constexpr int kSlice = kSampleThreads * kPerThread;
// candidates held in LDS: a slice has at most 8 keys from each of a wave's K
// best lanes (4 * 8 * 64 = 2048); the last step at most K entries from each
// of the K lists whose heads are the K largest (64 * 64)
constexpr int kCandCap = kSampleMaxK * kSampleMaxK;

// (logit, id) as one key: larger logit first, then lower id.  Never 0 for a
// token (the id part is nonzero), so 0 marks "none".
__device__ __forceinline__ uint64_t cand_key(float l, int id) {
    return (static_cast<uint64_t>(orderable(l)) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(id));
}
__device__ __forceinline__ int key_id(uint64_t k) { return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(k)); }
__device__ __forceinline__ float key_logit(uint64_t k) { return from_orderable(static_cast<uint32_t>(k >> 32)); }

struct SampleArgs {
    const float *logits;
    uint64_t *cand;            // [kSampleSlices][kSampleMaxK] each slice's sorted top-k (0: none)
    uint32_t *arrived;         // slices done with this call (the last one resets it)
    const int32_t *seen_ids, *seen_counts, *banned_ids;
    int32_t *out;
    int32_t vocab, n_seen, n_banned, k, slices, slice;
    float temperature, top_p, presence, frequency, u;
};

struct SampleLds {
    uint64_t big[kCandCap];      // the slice's logits (as floats), then candidates
    uint64_t vals[kSampleThreads];
    uint64_t tau[kSampleWaves];
    uint64_t top[kSampleMaxK];
    uint64_t kth;
    uint32_t count[3];
    uint32_t last;
};

// A lower bound of the k-th largest of the workgroup's values v (one per
// thread, 0 = none, nonzero values distinct): each wave's k-th largest by
// rank (0 if the wave holds fewer than k nonzero values), the largest of
// those.  At least min(k, nonzero count) values are >= it, and every value
// among the k largest is.
__device__ uint64_t kth_lower_bound(uint64_t v, int k, SampleLds &L) {
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    L.vals[tid] = v;
    if (lane == 0) L.tau[wave] = 0ull;
    __syncthreads();
    const uint64_t *w = L.vals + wave * kWave;
    int rank = 0;
#pragma unroll 16
    for (int j = 0; j < kWave; ++j) rank += w[j] > v;
    if (rank == k - 1 && v != 0ull) L.tau[wave] = v;
    __syncthreads();
    uint64_t t = L.tau[0];
#pragma unroll
    for (int i = 1; i < kSampleWaves; ++i) t = L.tau[i] > t ? L.tau[i] : t;
    return t;
}

// Rank of x among the n distinct candidates in LDS: the number larger.
__device__ __forceinline__ int rank_of(uint64_t x, const uint64_t *c, int n) {
    int r = 0;
#pragma unroll 8
    for (int j = 0; j < n; ++j) r += c[j] > x;
    return r;
}

// The draw on wave 0 (lane i holds candidate i), in the reference's order of
// float32 operations: sums left to right, no fused multiply-adds.
__device__ void sample_draw(const SampleArgs &a, const uint64_t *top) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x;
    const uint64_t key = lane < a.k ? top[lane] : 0ull;
    int pick = key_id(top[0]);
    if (a.temperature > 0.f) {
        // candidates with a logit (fewer than k only if the vocabulary is): a prefix
        int n = __popcll(__ballot(key != 0ull));
        const float l0 = key_logit(top[0]);
        const float p = lane < n ? expf((key_logit(key) - l0) / a.temperature) : 0.f;
        auto at = [](float v, int i) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i)); };
        float sum = 0.f;
        for (int i = 0; i < n; ++i) sum += at(p, i);
        if (a.top_p < 1.f) {
            const float q = p / sum;
            float cum = 0.f;
            int cut = n;
            for (int i = 0; i < n; ++i) {
                cum += at(q, i);
                if (cum >= a.top_p) {
                    cut = i + 1;
                    break;
                }
            }
            n = cut;
            sum = 0.f;
            for (int i = 0; i < n; ++i) sum += at(p, i);
        }
        float r = a.u * sum;
        for (int i = 0; i < n; ++i) {
            r -= at(p, i);
            if (r <= 0.f) {
                pick = key_id(top[i]);
                break;
            }
        }
    }
    if (lane == 0) *a.out = pick;
}

// step 2 (the last slice's workgroup): the global top-k from the slices'
// sorted lists, then the draw.
__device__ void sample_final(const SampleArgs &a, SampleLds &L) {
    const int tid = threadIdx.x;
    // list tid's first 8 entries (its head first) in one round of loads
    const uint64_t *list = a.cand + min(tid, a.slices - 1) * kSampleMaxK;
    uint64_t e[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) e[q] = list[min(q, a.k - 1)];
    const uint64_t h = tid < a.slices ? e[0] : 0ull;
    const uint64_t lb = kth_lower_bound(h, a.k, L);
    // the exact k-th largest head: heads >= lb (the k largest among them) ranked
    const bool near = h != 0ull && h >= lb;
    if (near) L.vals[atomicAdd(&L.count[1], 1u)] = h;  // vals is free again
    __syncthreads();
    if (near && rank_of(h, L.vals, static_cast<int>(L.count[1])) == a.k - 1) L.kth = h;
    __syncthreads();
    const uint64_t kth = L.kth;  // 0 if fewer than k lists hold a token
    // candidates: the entries >= kth of the (at most k) lists whose head is
    // >= kth -- sorted lists, so a prefix, 8 entries at a time
    if (h != 0ull && h >= kth) {
        for (int r0 = 0; r0 < a.k; r0 += 8) {
            if (r0 > 0) {
#pragma unroll
                for (int q = 0; q < 8; ++q) e[q] = list[min(r0 + q, a.k - 1)];
            }
            int c = 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) c += r0 + q < a.k && e[q] != 0ull && e[q] >= kth;
            const uint32_t off = atomicAdd(&L.count[2], static_cast<uint32_t>(c));
#pragma unroll
            for (int q = 0; q < 8; ++q)
                if (q < c && off + q < static_cast<uint32_t>(kCandCap)) L.big[off + q] = e[q];
            if (c < 8) break;
        }
    }
    __syncthreads();
    const int n = min(static_cast<int>(L.count[2]), kCandCap);  // <= k * k by the bound above
    for (int i = tid; i < n; i += kSampleThreads) {
        const uint64_t x = L.big[i];
        const int r = rank_of(x, L.big, n);
        if (r < a.k) L.top[r] = x;
    }
    for (int i = n + tid; i < a.k; i += kSampleThreads) L.top[i] = 0ull;
    __syncthreads();
    if (tid < kWave) sample_draw(a, L.top);
}

// step 1: the slice's penalised logits in LDS, its top-k, sorted, into
// cand[slice][0..k) (missing: 0); the last slice to finish runs step 2.
__global__ __launch_bounds__(kSampleThreads) void sample_slices(const SampleArgs a) {
#pragma clang fp contract(off)
    __shared__ SampleLds L;
    static_assert(kCandCap * 8 >= kSlice * 4, "the slice's logits fit the candidate buffer");
    float *s_l = reinterpret_cast<float *>(L.big);
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int v0 = blockIdx.x * kSlice;
    if (tid == 0) {
        L.count[0] = L.count[1] = L.count[2] = 0u;
        L.kth = 0ull;
    }
    // the slice's logits and the first entries of the penalty lists, all
    // loads in flight together (clamped indices, no guarded loads)
    float lv[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) lv[j] = a.logits[min(v0 + j * kSampleThreads + tid, a.vocab - 1)];
    int seen0 = 0, count0 = 0, banned0 = 0;
    if (a.n_seen > 0) {
        seen0 = a.seen_ids[min(tid, a.n_seen - 1)];
        count0 = a.seen_counts[min(tid, a.n_seen - 1)];
    }
    if (a.n_banned > 0) banned0 = a.banned_ids[min(tid, a.n_banned - 1)];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) s_l[j * kSampleThreads + tid] = lv[j];
    __syncthreads();
    // penalties inside the slice: the seen tokens, then the banned ones
    for (int i = tid; i < a.n_seen; i += kSampleThreads) {
        const int t = (i == tid ? seen0 : a.seen_ids[i]) - v0;
        const int c = i == tid ? count0 : a.seen_counts[i];
        if (t >= 0 && t < kSlice) atomicAdd(&s_l[t], -(a.presence + a.frequency * static_cast<float>(c)));
    }
    __syncthreads();
    for (int i = tid; i < a.n_banned; i += kSampleThreads) {
        const int t = (i == tid ? banned0 : a.banned_ids[i]) - v0;
        if (t >= 0 && t < kSlice) s_l[t] = -INFINITY;
    }
    __syncthreads();
    // each thread's 8 keys and their maximum
    uint64_t key[kPerThread];
    uint64_t head = 0ull;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int i = wave * (kPerThread * kWave) + j * kWave + lane;
        key[j] = v0 + i < a.vocab ? cand_key(s_l[i], v0 + i) : 0ull;
        head = key[j] > head ? key[j] : head;
    }
    // the slice's top-k: every key >= a lower bound of the k-th largest
    // head, ranked (logits in LDS are dead: the bound's barriers follow
    // their last read)
    const uint64_t lb = kth_lower_bound(head, a.k, L);
    int c = 0;
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) c += key[j] != 0ull && key[j] >= lb;
    if (c > 0) {
        uint32_t off = atomicAdd(&L.count[0], static_cast<uint32_t>(c));
#pragma unroll
        for (int j = 0; j < kPerThread; ++j)
            if (key[j] != 0ull && key[j] >= lb) L.big[off++] = key[j];
    }
    __syncthreads();
    const int n = static_cast<int>(L.count[0]);
    for (int i = tid; i < n; i += kSampleThreads) {
        const uint64_t x = L.big[i];
        const int r = rank_of(x, L.big, n);
        if (r < a.k) L.top[r] = x;
    }
    for (int i = n + tid; i < a.k; i += kSampleThreads) L.top[i] = 0ull;
    __syncthreads();
    // The list goes out from wave 0, the wave whose thread 0 then counts the
    // arrival: that agent-scope release waits for the wave's stores and
    // writes them back past this XCD's L2; the acquire fence every thread of
    // the last workgroup passes makes every slice's list visible on whichever
    // XCD that slice ran.  The count itself only releases: an acquire
    // invalidates the XCD's L2, which only the last workgroup needs.
    if (tid < a.k) a.cand[blockIdx.x * kSampleMaxK + tid] = L.top[tid];
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(a.arrived, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        L.last = prev == static_cast<uint32_t>(a.slices - 1);
        if (L.last) __hip_atomic_store(a.arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!L.last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    sample_final(a, L);
}

size_t sample_ws_bytes() { return static_cast<size_t>(kSampleSlices) * kSampleMaxK * 8 + 256; }

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
    a.arrived = reinterpret_cast<uint32_t *>(w + static_cast<size_t>(kSampleSlices) * kSampleMaxK * 8);
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
    return launch_status();
}
