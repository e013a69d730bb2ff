// MoE-layer decode step for one token in a single launch on gfx950.
//
// One workgroup of eight waves (two per SIMD) per CU, launched as an
// ordinary kernel: on a device with no other work the whole grid is resident
// at once.  Eight waves halve each wave's rows of every dot product (at one
// wave per SIMD a dependency chain leaves most issue slots empty); against
// four-wave workgroups, measured: the 80B, 8-bit and folded-norm steps
// 0.6-0.8 us faster, the 4-bit 35B step unchanged, the single-expert step
// 0.2 us slower.  The stages hand data to each other through
// the workspace instead of kernel boundaries: every value crossing
// workgroups is one 8-byte word (fp32 value, call epoch), written and polled
// with relaxed device-scope atomics, so a consumer polls the data itself and
// needs no separate flag, fence or cache write-back.
//
// Workgroup b belongs to XCD group grp = b mod 8 (the hardware hands
// workgroups to the eight XCDs round robin; checked once per device) with
// rank b / 8 inside it.  Group grp owns routed slots grp, grp + 8, ...: their
// gate/up rows, the SwiGLU activations between them (exchanged inside the
// XCD's L2) and their down rows.
//
//   phase A  (routing-independent, from the first instruction) router rows,
//            one pass of rows per wave, -> logits, written to one replica
//            per XCD group; shared-expert gate/up rows -> SwiGLU
//            activations; the shared-expert gate logit (every workgroup, for
//            its own combine); then the shared expert's down rows of the
//            workgroup's own output rows.
//   routing  wave 0 polls its replica of the logits and runs the top-k
//            rounds; each pick goes to LDS the moment its round ends, so a
//            group starts loading its expert's rows after round grp + 1
//            while the other groups' rounds continue: the routed weight
//            stream is spread over the rounds instead of waiting for all of
//            them.  The rounds of picks the workgroup does not own, and the
//            combine weights, finish after its routed work.
//   routed   per owned slot: gate/up rows (+ SwiGLU) -> activations in the
//            XCD's L2; the slot's activations -> LDS (each wave polls an
//            eighth); down rows (their loads issued with the gate/up
//            loads) -> partial outputs, one word per (slot, output row).
//   combine  the workgroup's output rows: routed partials in pick order,
//            then the gated shared expert (+ the residual stream).
//
// Numerics are those of the staged kernels (QwenCPUModel.moeForward,
// QwenCPUModel.swift:500-569): the same lane plans, per-row reductions and
// summation orders, so both paths agree bit for bit.
//
// Epochs: workgroup b keeps gen[b] (written only by itself); every call
// increments all of them, so every workgroup derives the same epoch
// g = gen[b] + 1 without communicating, and stale words of earlier calls
// never match.  Every wait is bounded (about a second); one that runs out
// records itself in the workspace header (swq_moe_workspace_status) and the
// workgroup carries on.
#pragma once

#include "../../include/swq_bench.h"
#include "moe_host.hpp"
#include "route.hpp"
#include "tile.hpp"

#include <utility>

// Phase stamps for timing studies: SWQ_FUSED_TRACE builds record
// s_memrealtime per (workgroup, wave, point); product builds compile them out.
#ifdef SWQ_FUSED_TRACE
// 16 stamps per (workgroup, wave), 8 waves per workgroup
static __device__ unsigned long long g_swq_fused_trace[1024 * 8 * 16];
// host access to one translation unit's stamps (the array is per code object)
#define SWQ_TRACE_ACCESSOR(name)                                                                        \
    extern "C" int name(void *host, size_t bytes, int clear) {                                          \
        if (clear) {                                                                                    \
            static unsigned long long z[1024 * 8 * 16];                                                 \
            return hipMemcpyToSymbol(HIP_SYMBOL(g_swq_fused_trace), z, sizeof(z)) == hipSuccess ? 0 : -1; \
        }                                                                                               \
        return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_swq_fused_trace), bytes) == hipSuccess ? 0 : -1;  \
    }
// Stamps go to LDS as they are taken (a global store per stamp would join
// the wave's vector-memory count, which every later load wait also drains)
// and to the global array once, at the end of the kernel.
#define SWQ_TRACE_DECL                                                                      \
    __shared__ unsigned long long s_trace[8 * 16];                                          \
    if ((threadIdx.x & 63) < 16) s_trace[(threadIdx.x >> 6) * 16 + (threadIdx.x & 63)] = 0
#define SWQ_STAMP(n)                                                                        \
    do {                                                                                    \
        if ((threadIdx.x & 63) == 0) s_trace[(threadIdx.x >> 6) * 16 + (n)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define SWQ_TRACE_FLUSH                                                                     \
    do {                                                                                    \
        __syncthreads();                                                                    \
        if (threadIdx.x < 128) g_swq_fused_trace[blockIdx.x * 128 + threadIdx.x] = s_trace[threadIdx.x]; \
    } while (0)
#else
#define SWQ_TRACE_DECL \
    do {               \
    } while (0)
#define SWQ_STAMP(n) \
    do {             \
    } while (0)
#define SWQ_TRACE_FLUSH \
    do {                \
    } while (0)
#endif

namespace swq {

constexpr int kFusedWaves = 8;  // two per SIMD: one workgroup per CU
constexpr int kFusedThreads = kFusedWaves * kWave;
constexpr int kGroups = 8;
constexpr int kReplicas = kFusedReplicas;  // logit replicas (one per XCD group)
constexpr int kMaxInterFused = kFusedMaxInter;  // activations of one slot
constexpr int kMaxCombineRows = 16;        // output rows per workgroup
constexpr int kPrenormMaxHidden = 4096;    // hidden size the folded-in norm holds in LDS
constexpr uint32_t kSpinLimit = 1u << 20;  // polls of ~0.1-1 us each: about a second

struct FusedArgs {
    QMat router, gate, up, down, sh_gate, sh_up, sh_down, seg;
    const void *x;
    void *out;
    int32_t *user_ids;
    float *user_w;
    uint32_t *gen;      // [kFusedMaxBlocks]
    uint32_t *err;      // the workspace's stall record
    uint64_t *logit_x;  // [B][kReplicas][rep_stride] (logit, epoch): token-major replica sets
    uint64_t *hsh_x;    // [B][Is] shared SwiGLU activations
    uint64_t *h_x;      // [B K][I] routed SwiGLU activations, slot s = token s / K, pick s % K
    uint64_t *part_x;   // [B K][H] routed down outputs
    int32_t rep_stride;
    int32_t odt, accumulate;
    int32_t H, E, K, I, Is, norm, has_shared;
    int32_t nb;
    int32_t sh_tiles;   // shared gate/up tiles (one pass of rows each)
    int32_t gu_tpe;     // routed gate/up tiles per slot
    int32_t dn_tpe;     // routed down tiles per slot
    int32_t local;      // a group's workgroups share an XCD (verified on the host)
    int32_t rows_cmb;   // output rows combined per workgroup
    // the layer's post-attention norm folded in (the PN kernels):
    // x = rmsnorm(h_in + res_in) * norm_w, out = (h_in + res_in) + moe(x)
    const float *h_in, *res_in;
    const void *norm_w;
    int32_t norm_dtype;
    float norm_eps;
    // tokens of the batched kernel (moe_fused_batch.hpp); last, so that the
    // fields the single-token kernel reads first keep their places
    int32_t B;
};

// ---------------------------------------------------------------------------
// kernel arguments: the compiler loads them lazily, each scalar load followed
// by a wait, so a phase that first touches a matrix descriptor pays a round
// trip per line.  One scalar load per 64-byte line of the argument block,
// all issued before a single wait, brings it into the scalar cache up front.
// The loads and the wait are one asm statement with a distinct output per
// load: scalar loads complete out of order, and a destination register the
// compiler considered free before the wait could be overwritten by a load
// still in flight (outputs are early-clobber, so none shares the base).
__device__ __forceinline__ void prefetch_kernargs() {
    static_assert(sizeof(FusedArgs) > 896 && sizeof(FusedArgs) <= 960, "fifteen 64-byte lines");
    const auto *kp = __builtin_amdgcn_kernarg_segment_ptr();
    uint32_t d0, d1, d2, d3, d4, d5, d6, d7, d8, d9, d10, d11, d12, d13, d14;
    asm volatile(
        "s_load_dword %0, %15, 0x0\n\ts_load_dword %1, %15, 0x40\n\t"
        "s_load_dword %2, %15, 0x80\n\ts_load_dword %3, %15, 0xc0\n\t"
        "s_load_dword %4, %15, 0x100\n\ts_load_dword %5, %15, 0x140\n\t"
        "s_load_dword %6, %15, 0x180\n\ts_load_dword %7, %15, 0x1c0\n\t"
        "s_load_dword %8, %15, 0x200\n\ts_load_dword %9, %15, 0x240\n\t"
        "s_load_dword %10, %15, 0x280\n\ts_load_dword %11, %15, 0x2c0\n\t"
        "s_load_dword %12, %15, 0x300\n\ts_load_dword %13, %15, 0x340\n\t"
        "s_load_dword %14, %15, 0x380\n\ts_waitcnt lgkmcnt(0)"
        : "=&s"(d0), "=&s"(d1), "=&s"(d2), "=&s"(d3), "=&s"(d4), "=&s"(d5), "=&s"(d6), "=&s"(d7), "=&s"(d8),
          "=&s"(d9), "=&s"(d10), "=&s"(d11), "=&s"(d12), "=&s"(d13), "=&s"(d14)
        : "s"(kp)
        : "memory");
}

// ---------------------------------------------------------------------------
// (value, epoch) words

__device__ __forceinline__ uint64_t pack_pair(float v, uint32_t g) {
    return (static_cast<uint64_t>(g) << 32) | __float_as_uint(v);
}

__device__ __forceinline__ void put_pair(uint64_t *p, float v, uint32_t g) {
    __hip_atomic_store(p, pack_pair(v, g), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A word for readers on this XCD only: a plain store, which stays in the
// XCD's L2, where their device-scope loads find it.  Used only when the host
// has verified that a group's workgroups share an XCD.
__device__ __forceinline__ void put_pair_group(uint64_t *p, float v, uint32_t g, int local) {
    if (local) __hip_atomic_store(p, pack_pair(v, g), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else __hip_atomic_store(p, pack_pair(v, g), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t get_pair(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void record_stall(uint32_t *err, uint32_t bit) {
    __hip_atomic_fetch_or(err, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Each lane waits for its N words p[c] (where live[c]) to carry epoch g and
// returns their values.  All loads of a round are in flight together; a lane
// stops loading a word once it is valid.
template <int N>
__device__ __forceinline__ void poll_words(const uint64_t *const (&p)[N], const bool (&live)[N], uint32_t g,
                                           float (&v)[N], uint32_t *err, uint32_t bit) {
    bool pend[N];
#pragma unroll
    for (int c = 0; c < N; ++c) {
        pend[c] = live[c];
        v[c] = 0.f;
    }
    for (uint32_t it = 0;; ++it) {
        uint64_t w[N];
#pragma unroll
        for (int c = 0; c < N; ++c) w[c] = pend[c] ? get_pair(p[c]) : 0;
        bool any = false;
#pragma unroll
        for (int c = 0; c < N; ++c) {
            if (pend[c] && static_cast<uint32_t>(w[c] >> 32) == g) {
                v[c] = __uint_as_float(static_cast<uint32_t>(w[c]));
                pend[c] = false;
            }
            any = any || pend[c];
        }
        if (__ballot(any) == 0) return;
        if (it > kSpinLimit) {
            if ((threadIdx.x & 63) == 0) record_stall(err, bit);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// poll_words whose first round runs mid() between issuing its loads and
// checking them: loads mid() issues then travel with the poll's instead of
// ahead of it (loads complete in issue order, so a poll issued behind them
// would wait for them too).  The compiler barriers keep mid()'s loads
// between the two.
template <int N, typename F>
__device__ __forceinline__ void poll_words_mid(const uint64_t *const (&p)[N], const bool (&live)[N], uint32_t g,
                                               float (&v)[N], uint32_t *err, uint32_t bit, F &&mid) {
    bool pend[N];
    {
        uint64_t w[N];
#pragma unroll
        for (int c = 0; c < N; ++c) {
            pend[c] = live[c];
            v[c] = 0.f;
            w[c] = pend[c] ? get_pair(p[c]) : 0;
        }
        asm volatile("" ::: "memory");
        mid();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int c = 0; c < N; ++c)
            if (pend[c] && static_cast<uint32_t>(w[c] >> 32) == g) {
                v[c] = __uint_as_float(static_cast<uint32_t>(w[c]));
                pend[c] = false;
            }
    }
    // later rounds as poll_words (the words of a round die with it)
    for (uint32_t it = 0;; ++it) {
        bool any = false;
#pragma unroll
        for (int c = 0; c < N; ++c) any = any || pend[c];
        if (__ballot(any) == 0) return;
        if (it > kSpinLimit) {
            if ((threadIdx.x & 63) == 0) record_stall(err, bit);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
        uint64_t w[N];
#pragma unroll
        for (int c = 0; c < N; ++c) w[c] = pend[c] ? get_pair(p[c]) : 0;
#pragma unroll
        for (int c = 0; c < N; ++c)
            if (pend[c] && static_cast<uint32_t>(w[c] >> 32) == g) {
                v[c] = __uint_as_float(static_cast<uint32_t>(w[c]));
                pend[c] = false;
            }
    }
}

// Bounded wait until the LDS word becomes non-negative; returns it (0 if the
// wait ran out).
__device__ __forceinline__ int32_t wait_lds_nonneg(int32_t *p, uint32_t *err) {
    for (uint32_t it = 0;; ++it) {
        const int32_t v = __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (v >= 0) return v;
        if (it > kSpinLimit) {
            if ((threadIdx.x & 63) == 0) record_stall(err, 4u);
            return 0;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One tile's row dot products through dot_tiles (chunks interleaved).
template <int BITS, int CPL, int ES, int XF, int RI>
__device__ __forceinline__ void dot_rows(float (&res)[RI], const RowTile<BITS, CPL, ES, RI> &rt, const QMat &m,
                                         const XSlice<BITS, CPL, XF> &xs, const LaneMap &lm) {
    const RowTile<BITS, CPL, ES, RI> *tiles[1] = {&rt};
    const QMat *mats[1] = {&m};
    float r[1][RI];
    dot_tiles<1>(r, tiles, mats, xs, lm);
#pragma unroll
    for (int i = 0; i < RI; ++i) res[i] = r[0][i];
}

// The gate and up tiles' row dot products, their chunks interleaved.
template <int BITS, int CPL, int ES, int XF, int RI>
__device__ __forceinline__ void dot_rows2(float (&rg)[RI], float (&ru)[RI], const RowTile<BITS, CPL, ES, RI> &tg,
                                          const RowTile<BITS, CPL, ES, RI> &tu, const QMat &mg, const QMat &mu,
                                          const XSlice<BITS, CPL, XF> &xs, const LaneMap &lm) {
    const RowTile<BITS, CPL, ES, RI> *tiles[2] = {&tg, &tu};
    const QMat *mats[2] = {&mg, &mu};
    float r[2][RI];
    dot_tiles<2>(r, tiles, mats, xs, lm);
#pragma unroll
    for (int i = 0; i < RI; ++i) {
        rg[i] = r[0][i];
        ru[i] = r[1][i];
    }
}

// ---------------------------------------------------------------------------
// activations in LDS for the down rows
//
// 4-bit down rows take each fp32 activation as hi = bf16(x), lo = bf16(x -
// hi) in pair words (the kXBF16X2 format): chunk c (32 activations) is words
// [32c, 32c + 32), its eight 16-byte groups (hi words 0-3, 4-7, 8-11, 12-15,
// then lo) with group i stored at (i + c) mod 8, so the lanes of a down tile,
// which read chunk j each, spread over the LDS banks.  Pair p of the
// activations (p < n/2) is {x[e], x[e + 4]}, e = 32(p/16) + 8((p%16)/4) +
// p%4.  8-bit down rows take the fp32 activations as they are (pair p =
// {x[2p], x[2p + 1]}).
__device__ __forceinline__ int x2_word(int c, int grp16, int d) { return 32 * c + 4 * ((grp16 + c) & 7) + d; }

template <int DB>
__device__ __forceinline__ int pair_first(int p) {
    if constexpr (DB == 4) return 32 * (p >> 4) + 8 * ((p & 15) >> 2) + (p & 3);
    else return 2 * p;
}

template <int DB>
__device__ __forceinline__ int pair_second(int p) {
    if constexpr (DB == 4) return pair_first<4>(p) + 4;
    else return 2 * p + 1;
}

template <int DB>
__device__ __forceinline__ void store_pair_lds(uint32_t *buf, int p, float x0, float x1) {
    if constexpr (DB == 4) {
        uint32_t hi, lo;
        split_pair(x0, x1, hi, lo);
        const int c = p >> 4, w = p & 15;
        buf[x2_word(c, w >> 2, w & 3)] = hi;
        buf[x2_word(c, 4 + (w >> 2), w & 3)] = lo;
    } else {
        buf[2 * p] = __float_as_uint(x0);
        buf[2 * p + 1] = __float_as_uint(x1);
    }
}

// Pairs [p0, p1) of the activation words at src into LDS, polled by one
// wave, two pairs per lane and round.
template <int DB>
__device__ __forceinline__ void fetch_acts(const uint64_t *src, int p0, int p1, uint32_t g, uint32_t *buf, int lane,
                                           uint32_t *err) {
    for (int q = p0; q < p1; q += 2 * kWave) {
        const uint64_t *pp[4];
        bool live[4];
        int pr[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            pr[c] = q + c * kWave + lane;
            live[2 * c] = live[2 * c + 1] = pr[c] < p1;
            const int pc = min(pr[c], p1 - 1);
            pp[2 * c] = src + pair_first<DB>(pc);
            pp[2 * c + 1] = src + pair_second<DB>(pc);
        }
        float v[4];
        poll_words<4>(pp, live, g, v, err, 1u);
#pragma unroll
        for (int c = 0; c < 2; ++c)
            if (live[2 * c]) store_pair_lds<DB>(buf, pr[c], v[2 * c], v[2 * c + 1]);
    }
}

// poll_words split in two: issue() sends the first round of loads, finish()
// checks them and polls on for the words still stale, so that other work
// can run while the first round is in flight.
template <int N>
struct EarlyPoll {
    const uint64_t *p[N];
    bool pend[N];
    uint64_t w[N];
    __device__ __forceinline__ void issue() {
#pragma unroll
        for (int c = 0; c < N; ++c) w[c] = pend[c] ? get_pair(p[c]) : 0;
    }
    __device__ __forceinline__ void finish(uint32_t g, float (&v)[N], uint32_t *err, uint32_t bit) {
#pragma unroll
        for (int c = 0; c < N; ++c) v[c] = 0.f;
        for (uint32_t it = 0;; ++it) {
            bool any = false;
#pragma unroll
            for (int c = 0; c < N; ++c) {
                if (pend[c] && static_cast<uint32_t>(w[c] >> 32) == g) {
                    v[c] = __uint_as_float(static_cast<uint32_t>(w[c]));
                    pend[c] = false;
                }
                any = any || pend[c];
            }
            if (__ballot(any) == 0) return;
            if (it > kSpinLimit) {
                if ((threadIdx.x & 63) == 0) record_stall(err, bit);
                return;
            }
            __builtin_amdgcn_s_sleep(1);
            issue();
        }
    }
};

// Pairs [p0, p1) of NS slots' words (at src[i], none where live_slot[i] is
// false) into buf[i], and pairs [s0, s1) of the words at ssrc into sbuf, all
// in each polling round: one pair of each per lane and round.
template <int DB, int NS>
__device__ __forceinline__ void fetch_acts_multi(const uint64_t *const (&src)[NS], uint32_t *const (&buf)[NS],
                                                 const bool (&live_slot)[NS], int p0, int p1, const uint64_t *ssrc,
                                                 int s0, int s1, uint32_t *sbuf, uint32_t g, int lane,
                                                 uint32_t *err) {
    for (int r = 0; p0 + r < p1 || s0 + r < s1; r += kWave) {
        constexpr int N = 2 * NS + 2;
        const uint64_t *pp[N];
        bool live[N];
        const int pr = p0 + r + lane, sr = s0 + r + lane;
        const int pc = min(pr, max(p1 - 1, p0)), sc = min(sr, max(s1 - 1, s0));
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            live[2 * i] = live[2 * i + 1] = live_slot[i] && pr < p1;
            pp[2 * i] = src[i] + pair_first<DB>(pc);
            pp[2 * i + 1] = src[i] + pair_second<DB>(pc);
        }
        live[2 * NS] = live[2 * NS + 1] = sr < s1;
        pp[2 * NS] = ssrc + pair_first<DB>(sc);
        pp[2 * NS + 1] = ssrc + pair_second<DB>(sc);
        float v[N];
        poll_words<N>(pp, live, g, v, err, 1u);
#pragma unroll
        for (int i = 0; i < NS; ++i)
            if (live[2 * i]) store_pair_lds<DB>(buf[i], pr, v[2 * i], v[2 * i + 1]);
        if (live[2 * NS]) store_pair_lds<DB>(sbuf, sr, v[2 * NS], v[2 * NS + 1]);
    }
}

// Pairs [p0, p1) of the words at src into buf and [s0, s1) of those at ssrc
// into sbuf, each at most a wave's 64, polled together in one round per
// lane (the second set is ready earlier: it rides the first's wait).
template <int DB>
__device__ __forceinline__ void fetch_acts_with(const uint64_t *src, int p0, int p1, uint32_t *buf,
                                                const uint64_t *ssrc, int s0, int s1, uint32_t *sbuf, uint32_t g,
                                                int lane, uint32_t *err) {
    const uint64_t *pp[4];
    bool live[4];
    const int pr = p0 + lane, sr = s0 + lane;
    live[0] = live[1] = pr < p1;
    live[2] = live[3] = sr < s1;
    const int pc = min(pr, max(p1 - 1, p0)), sc = min(sr, max(s1 - 1, s0));
    pp[0] = src + pair_first<DB>(pc);
    pp[1] = src + pair_second<DB>(pc);
    pp[2] = ssrc + pair_first<DB>(sc);
    pp[3] = ssrc + pair_second<DB>(sc);
    float v[4];
    poll_words<4>(pp, live, g, v, err, 1u);
    if (live[0]) store_pair_lds<DB>(buf, pr, v[0], v[1]);
    if (live[2]) store_pair_lds<DB>(sbuf, sr, v[2], v[3]);
}

// Dot products of a down tile with the activations in LDS.
template <int DB, int DRI>
__device__ __forceinline__ void down_dot(float (&res)[DRI], const RowTile<DB, 1, 2, DRI> &dt, const QMat &m,
                                         const LaneMap &lm, const uint32_t *buf) {
    const int c = min(lm.j, m.chunks - 1);
    if constexpr (DB == 4) {
        XSlice<4, 1, kXBF16X2> xs;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 h = *reinterpret_cast<const uint4 *>(buf + x2_word(c, i, 0));
            const uint4 l = *reinterpret_cast<const uint4 *>(buf + x2_word(c, 4 + i, 0));
            xs.hi[0][4 * i] = h.x;
            xs.hi[0][4 * i + 1] = h.y;
            xs.hi[0][4 * i + 2] = h.z;
            xs.hi[0][4 * i + 3] = h.w;
            xs.lo[0][4 * i] = l.x;
            xs.lo[0][4 * i + 1] = l.y;
            xs.lo[0][4 * i + 2] = l.z;
            xs.lo[0][4 * i + 3] = l.w;
        }
        xs.sum[0] = pair_sum(xs.hi[0], xs.lo[0]);
        dot_rows(res, dt, m, xs, lm);
    } else {
        XSlice<8, 1, kXF32> xs;
        const float4 *p = reinterpret_cast<const float4 *>(buf + c * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = p[i];
            xs.v[0][4 * i] = v.x;
            xs.v[0][4 * i + 1] = v.y;
            xs.v[0][4 * i + 2] = v.z;
            xs.v[0][4 * i + 3] = v.w;
        }
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) s += xs.v[0][i];
        xs.sum[0] = s;
        dot_rows(res, dt, m, xs, lm);
    }
}


// ---------------------------------------------------------------------------
// the kernel.  XDT activation dtype; GB/GC/GX/GRI the gate/up format (bits,
// chunks per lane, activation format) and passes per tile; DB/DRI the down
// rows' bits (routed and shared alike) and passes per tile; RC chunks per
// lane of the 8-bit router and shared-expert gate rows; M logits per lane
// of the routing wave.

template <int XDT, int GB, int GC, int GX, int GRI, int DB, int DRI, int RC, int M, bool PN>
__global__ __launch_bounds__(kFusedThreads) __attribute__((amdgpu_waves_per_eu(kFusedWaves / 4, kFusedWaves / 4))) void moe_fused(FusedArgs a) {
    __shared__ int32_t s_ids[SWQ_MAX_TOPK];
    __shared__ float s_w[SWQ_MAX_TOPK];
    __shared__ __attribute__((aligned(16))) uint32_t s_hb[kMaxInterFused];   // a routed slot's activations
    __shared__ __attribute__((aligned(16))) uint32_t s_hsh[kMaxInterFused];  // the shared expert's
    // two split slots' activations (512 experts and more)
    __shared__ __attribute__((aligned(16))) uint32_t s_hb2[M >= 8 ? kMaxInterFused : 4];
    __shared__ __attribute__((aligned(16))) uint32_t s_hb3[M >= 8 ? kMaxInterFused : 4];
    __shared__ float s_cmb[SWQ_MAX_TOPK * kMaxCombineRows];
    __shared__ float s_shd[kMaxCombineRows];  // shared-expert down rows of the combine rows
    __shared__ float s_sg;                    // shared-expert gate logit
    __shared__ int32_t s_arrive;              // waves with their share of the shared activations in
    __shared__ __attribute__((aligned(16))) float s_x[PN ? kPrenormMaxHidden : 4];  // the normalised input
    __shared__ float s_red[kFusedWaves];

    static_assert(sizeof(FusedArgs) <= 1024, "kernel arguments");
    SWQ_TRACE_DECL;
    prefetch_kernargs();
    SWQ_STAMP(0);
    const int wave = threadIdx.x >> 6;
    // Each phase takes the lane index through an empty asm: its per-lane
    // address arithmetic then cannot be hoisted to the top of the kernel,
    // where it would stay live across the earlier phases.
    int lane = threadIdx.x & 63;
    const int b = blockIdx.x, NB = a.nb;
    const int grp = b % kGroups, rank = b / kGroups, NPG = NB / kGroups;
    if (threadIdx.x < SWQ_MAX_TOPK) s_ids[threadIdx.x] = -1;
    if (threadIdx.x == 0) s_arrive = 0;
    const void *x = a.x;
    if constexpr (PN) {
        // the post-attention RMSNorm of the layer, per workgroup into LDS:
        // s_x = (h_in + res_in) * (scale * w) (QwenCPUModel.rmsNorm and the
        // residual add before it, QwenCPUModel.swift:47-59, :276-277); one
        // round trip, indices clamped, values past H masked
        constexpr int kPer = kPrenormMaxHidden / kFusedThreads;
        const bool has_r = a.res_in != nullptr, wf32 = a.norm_dtype == SWQ_F32;
        const float *rp = has_r ? a.res_in : a.h_in;
        float hr[kPer], rr[kPer];
        uint32_t wr[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int ic = min(static_cast<int>(threadIdx.x) + k * kFusedThreads, a.H - 1);
            hr[k] = a.h_in[ic];
            rr[k] = rp[ic];
            wr[k] = wf32 ? static_cast<const uint32_t *>(a.norm_w)[ic] : static_cast<const uint16_t *>(a.norm_w)[ic];
        }
        float v[kPer], wv[kPer];
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const bool valid = static_cast<int>(threadIdx.x) + k * kFusedThreads < a.H;
            v[k] = valid ? (has_r ? hr[k] + rr[k] : hr[k]) : 0.f;
            wv[k] = wf32 ? __uint_as_float(wr[k])
                         : (a.norm_dtype == SWQ_BF16 ? bf16_to_f32(static_cast<uint16_t>(wr[k]))
                                                     : f16_to_f32(static_cast<uint16_t>(wr[k])));
            ss += v[k] * v[k];
        }
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int i = 0; i < kFusedWaves; ++i) tot += s_red[i];
        const float sc = 1.0f / __fsqrt_rn(tot / static_cast<float>(a.H) + a.norm_eps);
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int i = threadIdx.x + k * kFusedThreads;
            if (i < a.H) s_x[i] = v[k] * (sc * wv[k]);
        }
        x = s_x;
    }
    __syncthreads();
    const int r0 = b * a.rows_cmb;                      // this workgroup's output rows
    const int nr = max(0, min(a.rows_cmb, a.H - r0));

    // ---- phase A ------------------------------------------------------------
    // Every load first (weights, then activations), conversions after: the
    // router row is on the critical path, and a conversion between two loads
    // would make the second wait for the first.
    asm volatile("" : "+v"(lane));
    const LaneMap lmg = lane_map(a.gate.lpr_log2, lane);
    const LaneMap lmr = lane_map(a.router.lpr_log2, lane);
    // router and shared gate/up tiles: tile b + NB * w on wave w of workgroup b
    const int t_r = b + NB * wave;  // first router tile of this wave
    const bool has_r = t_r * lmr.rpw < a.E;
    const bool do_seg = a.has_shared && wave == 1;
    const int t_s = b + NB * (kFusedWaves - 1 - wave);  // first shared gate/up tile
    const bool has_s = a.has_shared && t_s < a.sh_tiles;
    RowTile<8, RC, 2, 1> rt;
    if (has_r) load_tile(rt, a.router, 0, lmr, t_r * lmr.rpw, a.E);
    else if (do_seg) load_tile(rt, a.seg, 0, lmr, 0, 1);
    RowTile<GB, GC, 2, 1> stg, stu;
    if (has_s) {
        load_tile(stg, a.sh_gate, 0, lmg, t_s * lmg.rpw, a.Is);
        load_tile(stu, a.sh_up, 0, lmg, t_s * lmg.rpw, a.Is);
    }
    // the shared expert's down rows of this workgroup's output rows: one
    // pass of rows each for waves 1.., loaded now, used once the shared
    // activations are in
    const LaneMap lms = lane_map(a.sh_down.lpr_log2, lane);
    const bool sh_rows = a.has_shared && nr > 0;
    const int sh_passes = sh_rows ? (nr + lms.rpw - 1) / lms.rpw : 0;
    const int sp0 = wave - 1;
    RowTile<DB, 1, 2, 1> sdt;
    if (wave >= 1 && sp0 < sh_passes) load_tile(sdt, a.sh_down, 0, lms, r0 + sp0 * lms.rpw, r0 + nr);
    XRaw<XDT, 8, RC> xrr;
    if (has_r || do_seg) load_xraw<XDT>(xrr, a.router, lmr, x, 0);
    // (the PN kernels read their gate/up slice from LDS after the router
    // rows: LDS reads ahead of the loads here delay them)
    XRaw<XDT, GB, GC> xgr;
    if constexpr (!PN) load_xraw<XDT>(xgr, a.gate, lmg, x, 0);
    // The call's epoch, loaded after every other load of phase A: vector
    // loads complete in issue order, so the first wait for it waits for them
    // too, which the router row needs anyway; issued first, any wait for it
    // after the roles' branches would drain every load.
    asm volatile("" ::: "memory");
    const uint32_t g = __hip_atomic_load(a.gen + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    if (has_r || do_seg) {
        XSlice<8, RC, kXF32> xr;
        xslice_convert(xr, xrr);
        for (int t = t_r; t * lmr.rpw < a.E; t += NB * kFusedWaves) {
            // router tiles t_r, t_r + 8 NB, ...: one pass of rows each -> logits
            if (t != t_r) load_tile(rt, a.router, 0, lmr, t * lmr.rpw, a.E);
            float res[1];
            dot_rows(res, rt, a.router, xr, lmr);
            const int row = t * lmr.rpw + lmr.q;
            if (lmr.j == lmr.lpr - 1 && row < a.E) {
#pragma unroll
                for (int r = 0; r < kReplicas; ++r) put_pair(a.logit_x + r * a.rep_stride + row, res[0], g);
            }
            SWQ_STAMP(10);
        }
        if (do_seg) {
            // the shared-expert gate logit <w_sg, x> (this workgroup's combine)
            if (has_r) load_tile(rt, a.seg, 0, lmr, 0, 1);
            float res[1];
            dot_rows(res, rt, a.seg, xr, lmr);
            if (lane == lmr.lpr - 1) s_sg = res[0];
        }
    }
    // activations in the gate/up format (shared and routed rows), held for
    // the whole call
    if constexpr (PN) load_xraw<XDT>(xgr, a.gate, lmg, x, 0);
    XSlice<GB, GC, GX> xg;
    xslice_convert(xg, xgr);
    asm volatile("" : "+v"(lane));
    for (int t = t_s; has_s && t < a.sh_tiles; t += NB * kFusedWaves) {
        // shared-expert gate/up tiles t_s, t_s + 8 NB, ...: SwiGLU activations
        const int row0 = t * lmg.rpw;
        if (t != t_s) {
            load_tile(stg, a.sh_gate, 0, lmg, row0, a.Is);
            load_tile(stu, a.sh_up, 0, lmg, row0, a.Is);
        }
        float rg[1], ru[1];
        dot_rows2(rg, ru, stg, stu, a.sh_gate, a.sh_up, xg, lmg);
        const int row = row0 + lmg.q;
        if (lmg.j == lmg.lpr - 1 && row < a.Is) put_pair(a.hsh_x + row, swiglu(rg[0], ru[0]), g);
        SWQ_STAMP(11);
    }
    SWQ_STAMP(1);

    // ---- routing (wave 0) ---------------------------------------------------
    Rounds<M> rd;
    asm volatile("" : "+v"(lane));
    if (wave == 0) {
        const uint64_t *rep = a.logit_x + (b % kReplicas) * a.rep_stride;
        const uint64_t *pp[M];
        bool live[M];
#pragma unroll
        for (int j = 0; j < M; ++j) {
            const int e = lane * M + j;
            live[j] = e < a.E;
            pp[j] = rep + min(e, a.E - 1);
        }
        float v[M];
        poll_words<M>(pp, live, g, v, a.err, 2u);
        SWQ_STAMP(2);
        rounds_init(rd, v, a.E, lane);
        // the rounds up to this group's last owned slot; the rest after the
        // routed work
        int own_last = a.K > grp ? grp + kGroups * ((a.K - 1 - grp) / kGroups) : -1;
        // (512 experts and more: picks past the eighth are every group's)
        if constexpr (M >= 8) own_last = a.K > kGroups ? a.K - 1 : own_last;
        rounds_run(rd, own_last + 1, lane, s_ids);
        SWQ_STAMP(3);
    }

    // ---- routed slots of the group -------------------------------------------
    // When a wave's shares of a slot's and of the shared expert's activation
    // pairs each fit one polling round, the group's first slot fetches the
    // shared expert's along with its own (they were written in phase A), so
    // the tail's shared down rows need no fetch of their own.
    const int np_r = a.I / 2, q_r = (np_r + kFusedWaves - 1) / kFusedWaves;
    const int np_s = a.Is / 2, q_s = (np_s + kFusedWaves - 1) / kFusedWaves;
    const bool sh_early = sh_rows && grp < a.K && q_r <= kWave && q_s <= kWave;
    asm volatile("" : "+v"(lane));
    {
        const LaneMap lmd = lane_map(a.down.lpr_log2, lane);
        const int t0 = rank + NPG * wave;  // this wave's first tile of a slot
        if constexpr (M < 8) {
            for (int s = grp; s < a.K; s += kGroups) {
                const int64_t e = min(wait_lds_nonneg(&s_ids[s], a.err), a.E - 1);
                // loads in the order they are needed: the first gate/up tile,
                // then the first down tile (used only after the activations'
                // round trip)
                RowTile<GB, GC, 2, GRI> tg, tu;
                RowTile<DB, 1, 2, DRI> dt0;
                for (int t = t0; t < a.gu_tpe; t += NPG * kFusedWaves) {
                    const int row0 = t * GRI * lmg.rpw;
                    load_tile(tg, a.gate, e, lmg, row0, a.I);
                    load_tile(tu, a.up, e, lmg, row0, a.I);
                    float rg[GRI], ru[GRI];
                    dot_rows2(rg, ru, tg, tu, a.gate, a.up, xg, lmg);
                    if (lmg.j == lmg.lpr - 1) {
    #pragma unroll
                        for (int i = 0; i < GRI; ++i) {
                            const int row = row0 + i * lmg.rpw + lmg.q;
                            if (row < a.I)
                                put_pair_group(a.h_x + static_cast<int64_t>(s) * a.I + row, swiglu(rg[i], ru[i]), g,
                                               a.local);
                        }
                    }
                }
                SWQ_STAMP(4);
                // the first down tile: its loads issued once the gate/up bytes,
                // which the step waits for first, are in; used after the
                // activations' round trip
                if (t0 < a.dn_tpe) load_tile(dt0, a.down, e, lmd, t0 * DRI * lmd.rpw, a.H);
                // Without this the compiler may sink the loads below the polls
                // and the barrier that follow (allowed across an acquire), so they
                // would start only once the activations are in.
                asm volatile("" ::: "memory");
                // the slot's activations: each wave polls an eighth into LDS
                if (sh_early && s == grp)
                    fetch_acts_with<DB>(a.h_x + static_cast<int64_t>(s) * a.I, min(np_r, wave * q_r),
                                        min(np_r, (wave + 1) * q_r), s_hb, a.hsh_x, min(np_s, wave * q_s),
                                        min(np_s, (wave + 1) * q_s), s_hsh, g, lane, a.err);
                else
                    fetch_acts<DB>(a.h_x + static_cast<int64_t>(s) * a.I, min(np_r, wave * q_r),
                                   min(np_r, (wave + 1) * q_r), g, s_hb, lane, a.err);
                __syncthreads();
                SWQ_STAMP(5);
                for (int t = t0; t < a.dn_tpe; t += NPG * kFusedWaves) {
                    const int row0 = t * DRI * lmd.rpw;
                    if (t != t0) load_tile(dt0, a.down, e, lmd, row0, a.H);
                    float res[DRI];
                    down_dot<DB, DRI>(res, dt0, a.down, lmd, s_hb);
                    if (lmd.j == lmd.lpr - 1) {
    #pragma unroll
                        for (int i = 0; i < DRI; ++i) {
                            const int row = row0 + i * lmd.rpw + lmd.q;
                            if (row < a.H) put_pair(a.part_x + static_cast<int64_t>(s) * a.H + row, res[i], g);
                        }
                    }
                }
                SWQ_STAMP(6);
                // s_hb is rewritten by the next slot; after the group's last one
                // each wave goes on to the tail as soon as its own rows are done
                if (s + kGroups < a.K) __syncthreads();
            }
        } else {
            // 512 experts and more: picks past the eighth (the 80B layer's
            // top-10) are split over every workgroup instead of falling to
            // groups 0 and 1 as a second slot.  Split slot j's gate/up and
            // down tiles go one per workgroup to wave 1 + j (its tiles
            // issued with the wave's own slot's, so that they are in when the
            // own slot's dot products end); its activations cross XCDs, two
            // split slots' in one polling round once the own slot's down rows
            // are done.
            const int nsplit = max(a.K - kGroups, 0);
            const int js = (wave + kFusedWaves - 1) % kFusedWaves;  // this wave's split slot
            const bool own = grp < a.K;
            const bool spl = js < nsplit;
            // that slot's tiles on this wave: b, b + NB, ... (one wave of
            // every workgroup takes each split slot)
            const int t_sp = b, sp_step = NB;
            auto gate_up_rows = [&](int s, int64_t e, int row0, int local, const RowTile<GB, GC, 2, GRI> &tg,
                                    const RowTile<GB, GC, 2, GRI> &tu) {
                float rg[GRI], ru[GRI];
                dot_rows2(rg, ru, tg, tu, a.gate, a.up, xg, lmg);
                if (lmg.j == lmg.lpr - 1) {
#pragma unroll
                    for (int i = 0; i < GRI; ++i) {
                        const int row = row0 + i * lmg.rpw + lmg.q;
                        if (row < a.I)
                            put_pair_group(a.h_x + static_cast<int64_t>(s) * a.I + row, swiglu(rg[i], ru[i]), g,
                                           local);
                    }
                }
            };
            auto down_rows = [&](int s, int64_t e, RowTile<DB, 1, 2, DRI> &dt0, int t_first, int t_step,
                                 const uint32_t *hb) {
                for (int t = t_first; t < a.dn_tpe; t += t_step) {
                    const int row0 = t * DRI * lmd.rpw;
                    if (t != t_first) load_tile(dt0, a.down, e, lmd, row0, a.H);
                    float res[DRI];
                    down_dot<DB, DRI>(res, dt0, a.down, lmd, hb);
                    if (lmd.j == lmd.lpr - 1) {
#pragma unroll
                        for (int i = 0; i < DRI; ++i) {
                            const int row = row0 + i * lmd.rpw + lmd.q;
                            if (row < a.H) put_pair(a.part_x + static_cast<int64_t>(s) * a.H + row, res[i], g);
                        }
                    }
                }
            };
            int64_t e_own = 0, e_sp = 0;
            {
                RowTile<GB, GC, 2, GRI> tg, tu, tgs, tus;
                if (own) {
                    e_own = min(wait_lds_nonneg(&s_ids[grp], a.err), a.E - 1);
                    if (t0 < a.gu_tpe) {
                        load_tile(tg, a.gate, e_own, lmg, t0 * GRI * lmg.rpw, a.I);
                        load_tile(tu, a.up, e_own, lmg, t0 * GRI * lmg.rpw, a.I);
                    }
                }
                if (spl) {
                    e_sp = min(wait_lds_nonneg(&s_ids[kGroups + js], a.err), a.E - 1);
                    if (t_sp < a.gu_tpe) {
                        load_tile(tgs, a.gate, e_sp, lmg, t_sp * GRI * lmg.rpw, a.I);
                        load_tile(tus, a.up, e_sp, lmg, t_sp * GRI * lmg.rpw, a.I);
                    }
                }
                asm volatile("" ::: "memory");
                if (own) {
                    for (int t = t0; t < a.gu_tpe; t += NPG * kFusedWaves) {
                        const int row0 = t * GRI * lmg.rpw;
                        if (t != t0) {
                            load_tile(tg, a.gate, e_own, lmg, row0, a.I);
                            load_tile(tu, a.up, e_own, lmg, row0, a.I);
                        }
                        gate_up_rows(grp, e_own, row0, a.local, tg, tu);
                    }
                    SWQ_STAMP(4);
                }
                if (spl) {
                    for (int t = t_sp; t < a.gu_tpe; t += sp_step) {
                        const int row0 = t * GRI * lmg.rpw;
                        if (t != t_sp) {
                            load_tile(tgs, a.gate, e_sp, lmg, row0, a.I);
                            load_tile(tus, a.up, e_sp, lmg, row0, a.I);
                        }
                        gate_up_rows(kGroups + js, e_sp, row0, 0, tgs, tus);
                    }
                }
                SWQ_STAMP(22);
            }
            // split slots 0 and 1: when a wave's share of their activations
            // fits one polling round, its loads go out before the own slot's
            // down rows and are checked after them
            const int pr0 = min(np_r, wave * q_r), pr1 = min(np_r, (wave + 1) * q_r);
            const bool early = nsplit > 0 && q_r <= kWave;
            EarlyPoll<4> ep;
            {
                const int pr = pr0 + lane;
                const int pc = min(pr, max(pr1 - 1, pr0));
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const uint64_t *src = a.h_x + static_cast<int64_t>(kGroups + u) * a.I;
                    ep.pend[2 * u] = ep.pend[2 * u + 1] = early && u < nsplit && pr < pr1;
                    ep.p[2 * u] = src + pair_first<DB>(pc);
                    ep.p[2 * u + 1] = src + pair_second<DB>(pc);
                }
            }
            if (own) {
                RowTile<DB, 1, 2, DRI> dt0;
                // the first down tile, issued before the activation polls
                if (t0 < a.dn_tpe) load_tile(dt0, a.down, e_own, lmd, t0 * DRI * lmd.rpw, a.H);
                // Without this the compiler may sink the loads below the polls
                // and the barrier that follow (allowed across an acquire), so they
                // would start only once the activations are in.
                asm volatile("" ::: "memory");
                // the slot's activations: each wave polls an eighth into LDS
                if (sh_early)
                    fetch_acts_with<DB>(a.h_x + static_cast<int64_t>(grp) * a.I, min(np_r, wave * q_r),
                                        min(np_r, (wave + 1) * q_r), s_hb, a.hsh_x, min(np_s, wave * q_s),
                                        min(np_s, (wave + 1) * q_s), s_hsh, g, lane, a.err);
                else
                    fetch_acts<DB>(a.h_x + static_cast<int64_t>(grp) * a.I, min(np_r, wave * q_r),
                                   min(np_r, (wave + 1) * q_r), g, s_hb, lane, a.err);
                __syncthreads();
                SWQ_STAMP(5);
                if (early) ep.issue();
                asm volatile("" ::: "memory");
                down_rows(grp, e_own, dt0, t0, NPG * kFusedWaves, s_hb);
                SWQ_STAMP(6);
            } else if (early) {
                ep.issue();
            }
            // split slots two at a time: their activations in one polling
            // round into s_hb2 and s_hb3 (the first round needs no barrier
            // before it: the own slot's down rows read s_hb), then each down
            // row of a split slot on the wave that owns the slot
            for (int j0 = 0; j0 < nsplit; j0 += 2) {
                const bool two = j0 + 1 < nsplit;
                const bool mine = spl && (js == j0 || js == j0 + 1);
                RowTile<DB, 1, 2, DRI> dts;
                if (mine && t_sp < a.dn_tpe) load_tile(dts, a.down, e_sp, lmd, t_sp * DRI * lmd.rpw, a.H);
                asm volatile("" ::: "memory");
                if (j0 > 0) __syncthreads();  // s_hb2 and s_hb3 held the previous split slots' activations
                if (j0 == 0 && early) {
                    float v[4];
                    ep.finish(g, v, a.err, 1u);
                    const int pr = pr0 + lane;
                    if (pr < pr1) {
                        store_pair_lds<DB>(s_hb2, pr, v[0], v[1]);
                        if (two) store_pair_lds<DB>(s_hb3, pr, v[2], v[3]);
                    }
                } else {
                    const uint64_t *h0 = a.h_x + static_cast<int64_t>(kGroups + j0) * a.I;
                    const uint64_t *src[2] = {h0, h0 + a.I};
                    uint32_t *const buf[2] = {s_hb2, s_hb3};
                    const bool lv[2] = {true, two};
                    fetch_acts_multi<DB, 2>(src, buf, lv, pr0, pr1, a.hsh_x, 0, 0, s_hsh, g, lane, a.err);
                }
                __syncthreads();
                SWQ_STAMP(23);
                if (mine) down_rows(kGroups + js, e_sp, dts, t_sp, sp_step, js == j0 ? s_hb2 : s_hb3);
                SWQ_STAMP(24);
            }
        }
    }
    // ---- wave 0: the remaining picks, the weights, this workgroup's rows of
    // every slot's down output; waves 1..: the shared expert's down rows ---
    asm volatile("" : "+v"(lane));
    if (wave == 0) {
        rounds_run(rd, a.K, lane, s_ids);
        const float w = rounds_weight(rd, a.K, a.norm, lane);
        if (lane < a.K) {
            s_w[lane] = w;
            if (b == 0) {
                if (a.user_ids) a.user_ids[lane] = s_ids[lane];
                if (a.user_w) a.user_w[lane] = w;
            }
        }
        const int n = a.K * nr;
        for (int j0 = 0; j0 < n; j0 += 2 * kWave) {
            const uint64_t *pp[2];
            bool live[2];
            int jj[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                jj[c] = j0 + c * kWave + lane;
                live[c] = jj[c] < n;
                const int jc = min(jj[c], n - 1), k = jc / nr;
                pp[c] = a.part_x + static_cast<int64_t>(k) * a.H + r0 + (jc - k * nr);
            }
            float v[2];
            poll_words<2>(pp, live, g, v, a.err, 8u);
#pragma unroll
            for (int c = 0; c < 2; ++c)
                if (live[c]) s_cmb[jj[c]] = v[c];
        }
        SWQ_STAMP(8);
    } else if (sh_rows) {
        // (unless the first slot brought them) a share of the shared
        // activations -> LDS, then, once every wave's share is in, this
        // wave's passes of the shared down rows
        if (!sh_early) {
            const int q3 = (np_s + kFusedWaves - 2) / (kFusedWaves - 1);
            fetch_acts<DB>(a.hsh_x, min(np_s, sp0 * q3), min(np_s, (sp0 + 1) * q3), g, s_hsh, lane, a.err);
            SWQ_STAMP(12);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_fetch_add(&s_arrive, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            for (uint32_t it = 0; __hip_atomic_load(&s_arrive, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) <
                                  kFusedWaves - 1;
                 ++it) {
                if (it > kSpinLimit) {
                    if (lane == 0) record_stall(a.err, 16u);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        for (int sp = sp0; sp < sh_passes; sp += kFusedWaves - 1) {
            const int row0 = r0 + sp * lms.rpw;
            if (sp != sp0) load_tile(sdt, a.sh_down, 0, lms, row0, r0 + nr);
            float res[1];
            down_dot<DB, 1>(res, sdt, a.sh_down, lms, s_hsh);
            const int row = row0 + lms.q;
            if (lms.j == lms.lpr - 1 && row < r0 + nr) s_shd[row - r0] = res[0];
        }
        SWQ_STAMP(7);
    }
    __syncthreads();  // s_w, s_cmb, s_shd, s_sg

    // ---- combine ------------------------------------------------------------
    if (wave == 0) {
        const float gate = a.has_shared ? sigmoidf_ref(s_sg) : 0.f;
        if (lane < nr) {
            // out = sum_k w_k d_k in pick order, then + sigmoid(sg) * shared
            // (QwenCPUModel.swift:549-566)
            float acc = 0.f;
            for (int k = 0; k < a.K; ++k) acc += s_w[k] * s_cmb[k * nr + lane];
            if (a.has_shared) acc += gate * s_shd[lane];
            const int row = r0 + lane;
            if (a.odt == SWQ_BF16) {
                static_cast<uint16_t *>(a.out)[row] = f32_to_bf16_rne(acc);
            } else {
                float *out = static_cast<float *>(a.out);
                if constexpr (PN) {
                    // the layer's residual stream: (h + r) + moe (QwenCPUModel.swift:276-279)
                    float hv = a.h_in[row];
                    if (a.res_in) hv += a.res_in[row];
                    out[row] = hv + acc;
                } else {
                    out[row] = a.accumulate ? out[row] + acc : acc;
                }
            }
        }
        // the next call's epoch: every entry, whatever grid the next call uses
        for (int i = b + NB * lane; i < kFusedMaxBlocks; i += NB * kWave)
            __hip_atomic_store(a.gen + i, g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        SWQ_STAMP(9);
    }
    SWQ_TRACE_FLUSH;
}

using FusedKernel = void (*)(FusedArgs);

// Passes per tile, chosen so that a slot's gate/up and down rows at the
// benchmark shapes are one tile per wave (I = 512 rows over the 256 waves of
// a group: 2 rows per wave and matrix; H = 2048 down rows: 8 per wave).
constexpr int gate_passes(int gb, int gc) { return gb == 4 && gc == 2 ? 1 : 2; }
constexpr int down_passes(int db) { return db == 4 ? 2 : 4; }

template <int XDT, int GB, int GC, int GX, int DB, int RC, bool PN>
static FusedKernel fused_by_m(int M) {
    constexpr int GRI = gate_passes(GB, GC), DRI = down_passes(DB);
    switch (M) {
        case 1: return moe_fused<XDT, GB, GC, GX, GRI, DB, DRI, RC, 1, PN>;
        case 2: return moe_fused<XDT, GB, GC, GX, GRI, DB, DRI, RC, 2, PN>;
        case 4: return moe_fused<XDT, GB, GC, GX, GRI, DB, DRI, RC, 4, PN>;
        case 8: return moe_fused<XDT, GB, GC, GX, GRI, DB, DRI, RC, 8, PN>;
        default: return moe_fused<XDT, GB, GC, GX, GRI, DB, DRI, RC, 16, PN>;
    }
}

// Gate/up formats of the single launch: 4-bit codes, 8-bit codes with two
// chunks per lane, 8-bit codes with one.
enum FusedGateFormat { kFusedQ4 = 0, kFusedQ8C2 = 1, kFusedQ8C1 = 2 };

// The instantiation for (gate/up format, router chunks per lane 2 or 1,
// logits per routing lane M), one per activation format; nullptr for none.
FusedKernel fused_select_bf16(int gfmt, bool rc2, int M);
FusedKernel fused_select_f32(int gfmt, bool rc2, int M);
FusedKernel fused_select_pn(int gfmt, bool rc2, int M);
// the same for 2 or 4 tokens (kernels holding kFusedMaxBatch)
FusedKernel fused_select_bf16_batch(int gfmt, bool rc2, int M);
FusedKernel fused_select_f32_batch(int gfmt, bool rc2, int M);
// the one-expert launch (moe_fused_one.hpp; batch 1, one routed expert, no
// shared expert) for bf16 or f32 activations
FusedKernel fused_select_one(int x_dtype, int gfmt, bool rc2);

}  // namespace swq
