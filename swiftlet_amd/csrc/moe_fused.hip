// MoE-layer decode step for one token in a single launch on gfx950.
//
// One workgroup per CU, launched as an ordinary kernel: on a device with no other work every
// workgroup is resident at once.  (A cooperative launch would guarantee
// that, but costs ~18 us more per launch on this device, in graphs too.)
// If other work delays some workgroups, the waits below only last longer;
// no workgroup waits on a later one's launch.  The stages hand data to each
// other through the workspace instead of through kernel boundaries: every value crossing workgroups is stored together with
// the call's epoch as one 8-byte word, written and read with agent-coherent
// (relaxed, device-scope) atomics, so a consumer polls the data itself and
// needs no separate flag, no cache write-back and no fence.  Each XCD has its
// own L2; device-scope accesses are coherent across them.
//
//   phase 1  router rows -> logits (written to one replica per XCD, so the
//            pollers spread over separate lines); shared-expert gate/up rows
//            -> SwiGLU activations; shared-expert gate logit (every workgroup,
//            for its own combine); waves whose down tile belongs to the shared
//            expert load that tile now.
//   routing  wave 0 of every workgroup polls its replica of the logits and
//            runs softmax / top-k / renormalisation itself.
//   phase 2  routed gate/up rows -> SwiGLU activations; waves with a routed
//            down tile load it now, before their gate/up rows are done.
//   phase 3  down tiles: poll the slot's activations, dot, publish partial
//            sums per (slot, output row).
//   combine  the last wave of each workgroup polls its rows' partial sums of
//            every slot, combines them in pick order, adds the gated shared
//            expert and writes the output.
//
// Numerics are those of the staged kernels (QwenCPUModel.moeForward,
// QwenCPUModel.swift:500-569): the same tiles, the same reduction orders.
//
// Epochs: workgroup b keeps gen[b] (written only by itself); every call of a
// workspace increments all of them, so every workgroup derives the same epoch
// g = gen[b] + 1 without communicating.  Polls are bounded; a poll that runs
// out sets the workspace's error word and the workgroup carries on.
#include "../../include/swq_bench.h"
#include "moe_host.hpp"
#include "route.hpp"
#include "tile.hpp"

namespace swq {

constexpr int kFusedWaves = 8;
constexpr int kFusedThreads = kFusedWaves * kWave;
constexpr int kWorkWaves = kFusedWaves - 1;  // waves 0..6 carry tiles, wave 7 combines
constexpr int kFusedMaxBlocks = 1024;        // gen[] entries kept in step
constexpr int kReplicas = 8;                 // logit replicas (one per XCD)
constexpr int kMaxInterFused = 2048;         // activations a down tile reads
constexpr int kMaxCombineRows = 64;
constexpr int kPrenormMaxHidden = 4096;  // hidden size the folded-in norm holds in LDS
constexpr uint32_t kSpinLimit = 1u << 20;  // polls of ~1 us: about a second

struct FusedArgs {
    QMat router, gate, up, down, sh_gate, sh_up, sh_down, seg;
    const void *x;
    void *out;
    int32_t *user_ids;
    float *user_w;
    uint32_t *gen;       // [kFusedMaxBlocks]
    uint32_t *err;       // nonzero after a poll ran out
    uint64_t *logit_x;   // [kReplicas][rep_stride] (logit, epoch)
    uint64_t *hsh_x;     // [Is] shared SwiGLU activations
    uint64_t *h_x;       // [K][I] routed SwiGLU activations
    uint64_t *part_x;    // [K+1][H] down partial sums (slot K: shared expert)
    int32_t rep_stride;
    int32_t odt, accumulate;
    int32_t H, E, K, I, Is, norm, has_shared;
    int32_t nb;
    int32_t router_tiles, p1_tiles;  // phase-1 tiles: router rows, then shared gate/up rows
    int32_t gu_tpe, gu_tiles;        // routed gate/up tiles per expert, in all
    int32_t dn_tpe, dn_tpe_sh;       // down tiles per routed slot, of the shared expert
    int32_t local;                   // a group's workgroups share an XCD (verified on the host)
    int32_t rows_cmb;                // output rows combined per workgroup
    // the layer's post-attention norm folded in (the PRENORM kernels):
    // x = rmsnorm(h_in + res_in) * norm_w, out = (h_in + res_in) + moe(x)
    const float *h_in, *res_in;
    const void *norm_w;
    int32_t norm_dtype;
    float norm_eps;
};

// ---------------------------------------------------------------------------
// kernel arguments

// The compiler loads kernel arguments lazily, each scalar load followed by a
// wait, so a phase that first touches a matrix descriptor pays a cache-miss
// round trip per line.  One scalar load per 64-byte line of the argument
// block, all issued before a single wait, brings the block into the scalar
// cache up front (reads only).
// Fifteen lines: the argument block is 897..960 bytes (checked below).
__device__ __forceinline__ void prefetch_kernargs() {
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
        : "=s"(d0), "=s"(d1), "=s"(d2), "=s"(d3), "=s"(d4), "=s"(d5), "=s"(d6), "=s"(d7), "=s"(d8), "=s"(d9),
          "=s"(d10), "=s"(d11), "=s"(d12), "=s"(d13), "=s"(d14)
        : "s"(kp)
        : "memory");
}

// ---------------------------------------------------------------------------
// (value, epoch) words

__device__ __forceinline__ void put_pair(uint64_t *p, float v, uint32_t g) {
    __hip_atomic_store(p, (static_cast<uint64_t>(g) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t get_pair(uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t get_u32(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave waits until the n words src[(j / seg) * stride + j % seg], j < n,
// carry epoch g, and leaves their values in dst[(j / seg) * dpitch + j % seg]
// (LDS; dpitch 0 means seg).  Up to eight loads
// per lane are in flight per round (512 words); a lane stops loading a word
// once it is valid.
constexpr int kPollPerLane = 8;

__device__ __forceinline__ void poll_pairs(uint64_t *src, int n, int seg, int stride, uint32_t g, float *dst,
                                           int lane, uint32_t *err, int dpitch = 0) {
    if (dpitch == 0) dpitch = seg;
    for (int j0 = 0; j0 < n; j0 += kPollPerLane * kWave) {
        uint64_t *pp[kPollPerLane];
        float *dd[kPollPerLane];
        bool pend[kPollPerLane];
#pragma unroll
        for (int c = 0; c < kPollPerLane; ++c) {
            const int j = j0 + c * kWave + lane;
            pend[c] = j < n;
            const int jc = min(j, n - 1);
            const int q = jc / seg;
            pp[c] = src + static_cast<int64_t>(q) * stride + (jc - q * seg);
            dd[c] = dst + q * dpitch + (jc - q * seg);
        }
        uint32_t it = 0;
        for (;;) {
            uint64_t v[kPollPerLane];
#pragma unroll
            for (int c = 0; c < kPollPerLane; ++c) v[c] = pend[c] ? get_pair(pp[c]) : 0;
            bool any = false;
#pragma unroll
            for (int c = 0; c < kPollPerLane; ++c) {
                if (pend[c] && static_cast<uint32_t>(v[c] >> 32) == g) {
                    *dd[c] = __uint_as_float(static_cast<uint32_t>(v[c]));
                    pend[c] = false;
                }
                any = any || pend[c];
            }
            if (__ballot(any) == 0) break;
            if (++it > kSpinLimit) {
                if (lane == 0) atomicOr(err, 1u);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    // the wave reads dst right after: order its LDS writes before those reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// phase-1 jobs (runtime format dispatch; nothing is held across phases)

// Router rows of tile `tile` -> logits, one copy per replica.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void router_job(const FusedArgs &a, const void *x, int tile, uint32_t g, int lane) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const QMat &m = a.router;
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    const int row0 = tile * RI * lm.rpw;
    RowTile<BITS, CPL, ES> rt;
    load_tile(rt, m, 0, lm, row0, a.E);
    XSlice<BITS, CPL, XF> xs;
    load_xslice<XDT>(xs, m, lm, x, 0);
    float res[RI];
    dot_tile(res, rt, xs, m, lm);
    if (lm.j == lm.lpr - 1) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int row = row0 + i * lm.rpw + lm.q;
            if (row < a.E) {
#pragma unroll
                for (int r = 0; r < kReplicas; ++r) put_pair(a.logit_x + r * a.rep_stride + row, res[i], g);
            }
        }
    }
}

// Shared-expert gate/up rows of tile `tile` -> silu(g) * u.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void shared_gateup_job(const FusedArgs &a, const void *x, int tile, uint32_t g, int lane) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const LaneMap lm = lane_map(a.sh_gate.lpr_log2, lane);
    const int row0 = tile * RI * lm.rpw;
    RowTile<BITS, CPL, ES> tg, tu;
    load_tile(tg, a.sh_gate, 0, lm, row0, a.Is);
    load_tile(tu, a.sh_up, 0, lm, row0, a.Is);
    XSlice<BITS, CPL, XF> xs;
    load_xslice<XDT>(xs, a.sh_gate, lm, x, 0);
    float rg[RI], ru[RI];
    dot_tile(rg, tg, xs, a.sh_gate, lm);
    dot_tile(ru, tu, xs, a.sh_up, lm);
    if (lm.j == lm.lpr - 1) {
#pragma unroll
        for (int i = 0; i < RI; ++i) {
            const int row = row0 + i * lm.rpw + lm.q;
            if (row < a.Is) put_pair(a.hsh_x + row, swiglu(rg[i], ru[i]), g);
        }
    }
}

// The shared-expert gate logit <w_sg, x>, returned to every lane.
template <int XDT, int BITS, int CPL, int ES, int XF>
__device__ __forceinline__ void seg_job(const FusedArgs &a, const void *x, int lane, float &sg) {
    constexpr int RI = RowTile<BITS, CPL, ES>::kRI;
    const LaneMap lm = lane_map(a.seg.lpr_log2, lane);
    RowTile<BITS, CPL, ES> rt;
    load_tile(rt, a.seg, 0, lm, 0, 1);
    XSlice<BITS, CPL, XF> xs;
    load_xslice<XDT>(xs, a.seg, lm, x, 0);
    float res[RI];
    dot_tile(res, rt, xs, a.seg, lm);
    // row 0 is pass 0, row slot 0: the last lane of the first segment
    sg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(res[0]), lm.lpr - 1));
}

// Formats with 2-byte scales only (the fused path's precondition).
#define SWQ_DISPATCH2(XDT, m, FN, ...)                                      \
    do {                                                                    \
        if constexpr (XDT == SWQ_BF16) {                                    \
            if ((m).bits == 4) FN<XDT, 4, 2, 2, kXBF16>(__VA_ARGS__);       \
            else if ((m).cpl == 1) FN<XDT, 8, 1, 2, kXF32>(__VA_ARGS__);    \
            else FN<XDT, 8, 2, 2, kXF32>(__VA_ARGS__);                      \
        } else {                                                            \
            if ((m).bits == 4) FN<XDT, 4, 1, 2, kXF32>(__VA_ARGS__);        \
            else if ((m).cpl == 1) FN<XDT, 8, 1, 2, kXF32>(__VA_ARGS__);    \
            else FN<XDT, 8, 2, 2, kXF32>(__VA_ARGS__);                      \
        }                                                                   \
    } while (0)

// fp32 activations of a down tile from LDS (one chunk per lane).
template <int BITS>
__device__ __forceinline__ void load_xslice_lds(XSlice<BITS, 1, kXF32> &xs, const QMat &m, const LaneMap &lm,
                                                const float *h) {
    constexpr int kCPC = codes_per_chunk<BITS>();
    const int c = min(lm.j, m.chunks - 1);
    const float4 *p = reinterpret_cast<const float4 *>(h + c * kCPC);
#pragma unroll
    for (int i = 0; i < kCPC / 4; ++i) {
        const float4 v = p[i];
        xs.v[0][4 * i] = v.x;
        xs.v[0][4 * i + 1] = v.y;
        xs.v[0][4 * i + 2] = v.z;
        xs.v[0][4 * i + 3] = v.w;
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kCPC; ++i) s += xs.v[0][i];
    xs.sum[0] = s;
}

// Waits (bounded) until the LDS counter reaches `target`.
__device__ __forceinline__ void wait_count(int32_t *c, int target, uint32_t *err, int lane) {
    uint32_t it = 0;
    while (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
        if (++it > kSpinLimit) {
            if (lane == 0) atomicOr(err, 4u);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

__device__ __forceinline__ void count_done(int32_t *c, int lane) {
    if (lane == 0) __hip_atomic_fetch_add(c, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// LDS activations of one slot.  The fetching wave polls them in as fp32;
// for 4-bit down rows it then rewrites them as hi/lo bf16 pair words (the
// kXBF16X2 format), chunk c (32 activations) in words [32c, 32c + 32): its
// eight 16-byte groups (hi words 0-3, 4-7, 8-11, 12-15, then lo) with group
// i stored at (i + c) mod 8, so the lanes of a down tile, which read chunk j
// each, spread over the LDS banks.  One pair per lane and round: the reads
// of a round all complete before its writes (in-order LDS within a wave).
__device__ __forceinline__ int x2_word(int c, int grp16, int d) { return 32 * c + 4 * ((grp16 + c) & 7) + d; }

__device__ __forceinline__ void convert_x2_lds(float *buf, int n, int lane) {
    uint32_t *wbuf = reinterpret_cast<uint32_t *>(buf);
    const int npairs = n / 2;
    for (int p0 = 0; p0 < npairs; p0 += 4 * kWave) {
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = min(p0 + r * kWave + lane, npairs - 1);
            const int c = p >> 4, w = p & 15;
            const int e0 = 32 * c + 8 * (w >> 2) + (w & 3);
            split_pair(buf[e0], buf[e0 + 4], hi[r], lo[r]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int p = p0 + r * kWave + lane;
            if (p < npairs) {
                const int c = p >> 4, w = p & 15;
                wbuf[x2_word(c, w >> 2, w & 3)] = hi[r];
                wbuf[x2_word(c, 4 + (w >> 2), w & 3)] = lo[r];
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// One down tile of matrix m, rows from row0: dot with the activations in LDS
// (split bf16 pairs and chunk sums for 4-bit rows, fp32 for 8-bit rows),
// publish (partial sum, epoch) to part_x[slot][row].
template <int DB>
__device__ __forceinline__ void down_dot(const FusedArgs &a, const QMat &m, const RowTile<DB, 1, 2> &dt, int row0,
                                         int slot, const float *h_lds, uint32_t g, int lane) {
    constexpr int DRI = RowTile<DB, 1, 2>::kRI;
    const LaneMap lm = lane_map(m.lpr_log2, lane);
    float res[DRI];
    if constexpr (DB == 4) {
        XSlice<4, 1, kXBF16X2> xs;
        const int c = min(lm.j, m.chunks - 1);
        const uint32_t *wb = reinterpret_cast<const uint32_t *>(h_lds);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 h = *reinterpret_cast<const uint4 *>(wb + x2_word(c, i, 0));
            const uint4 l = *reinterpret_cast<const uint4 *>(wb + x2_word(c, 4 + i, 0));
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
        dot_tile(res, dt, xs, m, lm);
    } else {
        XSlice<DB, 1, kXF32> xs;
        load_xslice_lds<DB>(xs, m, lm, h_lds);
        dot_tile(res, dt, xs, m, lm);
    }
    if (lm.j == lm.lpr - 1) {
#pragma unroll
        for (int i = 0; i < DRI; ++i) {
            const int row = row0 + i * lm.rpw + lm.q;
            if (row < a.H) put_pair(a.part_x + static_cast<int64_t>(slot) * a.H + row, res[i], g);
        }
    }
}

// Bounded wait for an LDS flag set by the workgroup's fetching wave.
__device__ __forceinline__ void wait_ready(int32_t *flag, uint32_t *err, int lane) {
    uint32_t it = 0;
    while (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0) {
        if (++it > kSpinLimit) {
            if (lane == 0) atomicOr(err, 2u);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// (value, epoch) word written for readers on this XCD only: a plain store,
// which stays in the XCD's L2, where their agent-coherent loads find it.
// Used only when the host has verified that a group's workgroups share an
// XCD; otherwise the agent-coherent store.
__device__ __forceinline__ void put_pair_group(uint64_t *p, float v, uint32_t g, int local) {
    const uint64_t w = (static_cast<uint64_t>(g) << 32) | __float_as_uint(v);
    if (local) __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// the kernel: XDT activation dtype; GB/GC/GX the routed gate/up format; DB
// the down projections' bits (routed and shared alike).  Scales are 2 bytes.
//
// Workgroups form kGroups groups, g = b % kGroups (the hardware hands
// workgroups to XCDs round robin, so a group sits on one XCD); rank r =
// b / kGroups.  Group g owns routed slots g, g + kGroups, ...: their gate/up
// rows, their down tiles and the SwiGLU activations between them.  A down
// tile is ~360 VALU instructions of one wave at batch 1, so the down tiles
// are spread over four waves per workgroup.  Waves:
//   0-3  routed gate/up tiles of the group (wave 0 first routes); then wave 3
//        takes a share of the group's routed down tiles and wave 1 the shared
//        expert's down tiles
//   4-6  phase-1 jobs; then routed down tiles of the group, the first one
//        loaded right after routing and held until the activations arrive
//   7    shared-expert gate logit; fetches the activations the workgroup's
//        down tiles read into LDS; combines its output rows

constexpr int kGroups = 8;
constexpr int kGuWaves = 4;
constexpr int kDnShares = 4;           // routed down tiles: waves 4, 5, 6 and 3
constexpr int kDnLateWave = 3;         // the share taken after gate/up
constexpr int kShWave = 1, kAuxWave = 7;
constexpr int kGroupSlots = (SWQ_MAX_TOPK + kGroups - 1) / kGroups;  // routed slots per group
constexpr int kShBuf = kGroupSlots;                                    // LDS buffer of the shared slot

template <int XDT, int GB, int GC, int GX, int DB, bool PN>
__global__ __launch_bounds__(kFusedThreads) void moe_fused(FusedArgs a) {
    __shared__ float s_logits[kMaxExperts];
    __shared__ int32_t s_ids[SWQ_MAX_TOPK];
    __shared__ float s_w[SWQ_MAX_TOPK];
    __shared__ __attribute__((aligned(16))) float s_hb[kGroupSlots + 1][kMaxInterFused];
    __shared__ int32_t s_ready[kGroupSlots + 1];
    // waves of this workgroup done with: [0] phase 1 (with PN: its router
    // tiles), [1] gate/up, [2] down.
    // A wave that waits on other workgroups' results starts polling global
    // memory only once its own workgroup's share of that step is done: polls
    // issued earlier would only compete with the weight stream.
    __shared__ int32_t s_cnt[3];
    __shared__ float s_cmb[(SWQ_MAX_TOPK + 1) * kMaxCombineRows];
    __shared__ __attribute__((aligned(16))) float s_x[PN ? kPrenormMaxHidden : 4];  // the normalised input
    __shared__ float s_red[kFusedWaves];

    static_assert(sizeof(FusedArgs) > 896 && sizeof(FusedArgs) <= 960, "prefetch_kernargs covers 15 lines");
    prefetch_kernargs();
    const int wave = threadIdx.x >> 6;
    const int b = blockIdx.x, NB = a.nb;
    const int grp = b % kGroups, rank = b / kGroups, NPG = NB / kGroups;
    // Each phase takes the lane index through an empty asm: its per-lane
    // address arithmetic then cannot be hoisted to the top of the kernel,
    // where it would stay live (and spill) across the earlier phases.
    int lane = threadIdx.x & 63;
    // the call's epoch; its first use waits for the load
    const uint32_t g = get_u32(a.gen + b) + 1u;
    const int nsg = a.K > grp ? (a.K - grp + kGroups - 1) / kGroups : 0;  // routed slots of the group
    const bool has_sh_tiles = a.has_shared && b < a.dn_tpe_sh;
    if (threadIdx.x <= kGroupSlots) s_ready[threadIdx.x] = 0;
    if (threadIdx.x < 3) s_cnt[threadIdx.x] = 0;
    const void *x = a.x;
    if constexpr (PN) {
        // the post-attention RMSNorm of the layer, per workgroup into LDS:
        // s_x = h_in + res_in, then x = s_x * (scale * w) (QwenCPUModel.rmsNorm
        // and the residual add before it, QwenCPUModel.swift:47-59, :276-277)
        // one round trip: h, r and the weights of this thread's elements,
        // loaded unconditionally (indices clamped, values past H masked)
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
    constexpr int DRI = RowTile<DB, 1, 2>::kRI;
    RowTile<DB, 1, 2> dt0;
    float sg = 0.f;

    // ---- phase 1 ----------------------------------------------------------
    asm volatile("" : "+v"(lane));
    if (wave < kAuxWave) {
#pragma unroll 1
        for (int p = (kAuxWave - 1 - wave) * NB + b; p < a.p1_tiles; p += kAuxWave * NB) {
            if (p < a.router_tiles) SWQ_DISPATCH2(XDT, a.router, router_job, a, x, p, g, lane);
            else SWQ_DISPATCH2(XDT, a.sh_gate, shared_gateup_job, a, x, p - a.router_tiles, g, lane);
        }
        if (!PN || (kAuxWave - 1 - wave) * NB + b < a.router_tiles) count_done(&s_cnt[0], lane);
    } else if (a.has_shared) {
        SWQ_DISPATCH2(XDT, a.seg, seg_job, a, x, lane, sg);
    }

    // ---- routing ------------------------------------------------------------
    asm volatile("" : "+v"(lane));
    if (wave == 0) {
        // The polls wait for this workgroup's phase-1 waves.  Behind the
        // norm prologue (PN) only for its router tiles, so a wave still busy
        // with shared-expert rows does not hold up the routing (measured:
        // the folded step 22.3 -> 21.6 us); without the prologue the early
        // polls slow the step (18.6 -> 19.0 us), so there it waits for all.
        int waves = kAuxWave;
        if constexpr (PN) {
            waves = 0;
            for (int w = 0; w < kAuxWave; ++w) waves += (kAuxWave - 1 - w) * NB + b < a.router_tiles;
        }
        wait_count(&s_cnt[0], waves, a.err, lane);
        poll_pairs(a.logit_x + (b % kReplicas) * a.rep_stride, a.E, a.E, 0, g, s_logits, lane, a.err);
        int32_t my_id;
        float my_w;
        topk_wave(s_logits, a.E, a.K, a.norm, lane, my_id, my_w);
        if (lane < a.K) {
            s_ids[lane] = my_id;
            s_w[lane] = my_w;
            if (b == 0) {
                if (a.user_ids) a.user_ids[lane] = my_id;
                if (a.user_w) a.user_w[lane] = my_w;
            }
        }
    }
    __syncthreads();
    asm volatile("" : "+v"(lane));

    if (wave < kAuxWave) {
        const int dshare = wave >= kGuWaves ? wave - kGuWaves : (wave == kDnLateWave ? kDnShares - 1 : -1);
        const LaneMap lmd = lane_map(a.down.lpr_log2, lane);
        const int nqd = nsg * a.dn_tpe;
        const int qd0 = rank + NPG * dshare;
        const bool early = wave >= kGuWaves && dshare >= 0 && qd0 < nqd;
        if (early) {
            // ---- the first routed down tile, held until the activations
            // arrive.  Loaded once this workgroup's gate/up rows are in: the
            // gate/up loads are on the critical path, the down tiles are
            // needed only after the activations' round trip.
            wait_count(&s_cnt[1], kGuWaves, a.err, lane);
            const int j = qd0 / a.dn_tpe;
            load_tile(dt0, a.down, s_ids[grp + kGroups * j], lmd, (qd0 - j * a.dn_tpe) * DRI * lmd.rpw, a.H);
            // Without this the compiler may sink the loads below the waits
            // that follow (allowed across an acquire), so they would start
            // only once the activations are in.
            asm volatile("" ::: "memory");
        }
        if (wave < kGuWaves) {
            // ---- routed gate/up tiles of the group --------------------------
            constexpr int GRI = RowTile<GB, GC, 2>::kRI;
            const LaneMap lm = lane_map(a.gate.lpr_log2, lane);
            const int nq = nsg * a.gu_tpe;
#pragma unroll 1
            for (int q = rank + NPG * wave; q < nq; q += NPG * kGuWaves) {
                const int j = q / a.gu_tpe;
                const int slot = grp + kGroups * j;
                const int row0 = (q - j * a.gu_tpe) * GRI * lm.rpw;
                const int64_t e = s_ids[slot];
                RowTile<GB, GC, 2> tg, tu;
                load_tile(tg, a.gate, e, lm, row0, a.I);
                load_tile(tu, a.up, e, lm, row0, a.I);
                XSlice<GB, GC, GX> xs;
                load_xslice<XDT>(xs, a.gate, lm, x, 0);
                float rg[GRI], ru[GRI];
                dot_tile(rg, tg, xs, a.gate, lm);
                dot_tile(ru, tu, xs, a.up, lm);
                if (lm.j == lm.lpr - 1) {
#pragma unroll
                    for (int i = 0; i < GRI; ++i) {
                        const int row = row0 + i * lm.rpw + lm.q;
                        if (row < a.I)
                            put_pair_group(a.h_x + static_cast<int64_t>(slot) * a.I + row, swiglu(rg[i], ru[i]), g,
                                           a.local);
                    }
                }
            }
            count_done(&s_cnt[1], lane);
        }
        asm volatile("" : "+v"(lane));
        if (dshare >= 0) {
            // ---- routed down tiles of the group ---------------------------------
#pragma unroll 1
            for (int q = qd0; q < nqd; q += NPG * kDnShares) {
                const int j = q / a.dn_tpe;
                const int row0 = (q - j * a.dn_tpe) * DRI * lmd.rpw;
                if (!(early && q == qd0)) load_tile(dt0, a.down, s_ids[grp + kGroups * j], lmd, row0, a.H);
                wait_ready(&s_ready[j], a.err, lane);
                down_dot<DB>(a, a.down, dt0, row0, grp + kGroups * j, s_hb[j], g, lane);
            }
        }
        if (wave == kShWave && has_sh_tiles) {
            // ---- the shared expert's down tiles ---------------------------------
            const LaneMap lm = lane_map(a.sh_down.lpr_log2, lane);
#pragma unroll 1
            for (int q = b; q < a.dn_tpe_sh; q += NB) {
                load_tile(dt0, a.sh_down, 0, lm, q * DRI * lm.rpw, a.H);
                wait_ready(&s_ready[kShBuf], a.err, lane);
                down_dot<DB>(a, a.sh_down, dt0, q * DRI * lm.rpw, a.K, s_hb[kShBuf], g, lane);
            }
        }
        count_done(&s_cnt[2], lane);
    } else {
        // ---- fetch the activations this workgroup's down tiles read ------------
        if (has_sh_tiles) {
            poll_pairs(a.hsh_x, a.Is, a.Is, 0, g, s_hb[kShBuf], lane, a.err);
            if constexpr (DB == 4) convert_x2_lds(s_hb[kShBuf], a.Is, lane);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_store(&s_ready[kShBuf], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        // routed: once this workgroup's own gate/up rows are out, the group's
        // slots (rows grp, grp + kGroups, ... of h_x), one poll for all
        wait_count(&s_cnt[1], kGuWaves, a.err, lane);
        if (nsg > 0) {
            poll_pairs(a.h_x + static_cast<int64_t>(grp) * a.I, nsg * a.I, a.I, kGroups * a.I, g, &s_hb[0][0], lane,
                       a.err, kMaxInterFused);
            if constexpr (DB == 4) {
                for (int j = 0; j < nsg; ++j) convert_x2_lds(s_hb[j], a.I, lane);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane < nsg) __hip_atomic_store(&s_ready[lane], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        // ---- combine ------------------------------------------------------------
        const int r0 = b * a.rows_cmb;
        const int nr = min(a.rows_cmb, a.H - r0);
        if (nr > 0) {
            const int slots = a.K + (a.has_shared ? 1 : 0);
            wait_count(&s_cnt[2], kAuxWave, a.err, lane);
            poll_pairs(a.part_x + r0, slots * nr, nr, a.H, g, s_cmb, lane, a.err);
            const float gate = a.has_shared ? sigmoidf_ref(sg) : 0.f;
            for (int rr = lane; rr < nr; rr += kWave) {
                // out = sum_k w_k d_k in pick order, then + sigmoid(sg) * shared
                // (QwenCPUModel.swift:549-566)
                float acc = 0.f;
                for (int k = 0; k < a.K; ++k) acc += s_w[k] * s_cmb[k * nr + rr];
                if (a.has_shared) acc += gate * s_cmb[a.K * nr + rr];
                const int row = r0 + rr;
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
        }
        // the next call's epoch: every entry, whatever grid the next call uses
        if (lane == 0) {
            for (int i = b; i < kFusedMaxBlocks; i += NB)
                __hip_atomic_store(a.gen + i, g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ---------------------------------------------------------------------------
// host side

struct FusedLayout {
    size_t gen, err, logit_x, hsh_x, h_x, part_x, total;
    int rep_stride;
};

// Placed after the staged path's regions of the same workspace.
inline FusedLayout fused_layout(const swq_moe_layer *l, size_t base) {
    FusedLayout f{};
    size_t off = align256(base);
    auto take = [&](size_t n) {
        const size_t o = off;
        off = align256(off + n);
        return o;
    };
    // replicas 4 KiB apart plus a 256-byte skew, so they sit in different
    // memory channels
    const size_t rep_bytes = ((static_cast<size_t>(l->num_experts) * 8 + 4095) & ~static_cast<size_t>(4095)) + 256;
    f.rep_stride = static_cast<int>(rep_bytes / 8);
    f.gen = take(kFusedMaxBlocks * 4);
    f.err = take(4);
    f.logit_x = take(rep_bytes * kReplicas);
    f.hsh_x = take(static_cast<size_t>(l->has_shared ? l->shared_intermediate : 1) * 8);
    f.h_x = take(static_cast<size_t>(l->top_k) * l->moe_intermediate * 8);
    f.part_x = take(static_cast<size_t>(l->top_k + 1) * l->hidden * 8);
    f.total = off;
    return f;
}

using FusedKernel = void (*)(FusedArgs);

// The instantiation for this layer's formats, or nullptr.
static FusedKernel fused_kernel_for(const QMat &gate, const QMat &down, int x_dtype, bool prenorm) {
    if (prenorm) {  // x is the f32 normalised input in LDS
        if (x_dtype != SWQ_F32) return nullptr;
        if (gate.bits == 4 && gate.xf == 0 && gate.cpl == 1 && down.bits == 4) return moe_fused<SWQ_F32, 4, 1, kXF32, 4, true>;
        if (gate.bits == 8 && gate.cpl == 2 && down.bits == 8) return moe_fused<SWQ_F32, 8, 2, kXF32, 8, true>;
        if (gate.bits == 8 && gate.cpl == 1 && down.bits == 8) return moe_fused<SWQ_F32, 8, 1, kXF32, 8, true>;
        return nullptr;
    }
    if (x_dtype == SWQ_BF16) {
        if (gate.bits == 4 && gate.xf == 1 && gate.cpl == 2 && down.bits == 4) return moe_fused<SWQ_BF16, 4, 2, kXBF16, 4, false>;
        if (gate.bits == 8 && gate.cpl == 2 && down.bits == 8) return moe_fused<SWQ_BF16, 8, 2, kXF32, 8, false>;
        if (gate.bits == 8 && gate.cpl == 1 && down.bits == 8) return moe_fused<SWQ_BF16, 8, 1, kXF32, 8, false>;
    } else {
        if (gate.bits == 4 && gate.xf == 0 && gate.cpl == 1 && down.bits == 4) return moe_fused<SWQ_F32, 4, 1, kXF32, 4, false>;
        if (gate.bits == 8 && gate.cpl == 2 && down.bits == 8) return moe_fused<SWQ_F32, 8, 2, kXF32, 8, false>;
        if (gate.bits == 8 && gate.cpl == 1 && down.bits == 8) return moe_fused<SWQ_F32, 8, 1, kXF32, 8, false>;
    }
    return nullptr;
}

// Per device: whether the workgroups of each group (b % kGroups) of a grid
// of one workgroup per CU run on one XCD (1), do not (0), or unknown (-1,
// before the first swq_moe_workspace_init on the device).
static int g_groups_local[64] = {-1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1,
                                 -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1,
                                 -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1,
                                 -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1};

__global__ __launch_bounds__(kFusedThreads) void xcd_probe_kernel(int32_t *out) {
    if (threadIdx.x == 0) {
        uint32_t v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        out[blockIdx.x] = static_cast<int32_t>(v & 0xFu);
    }
}

// Workgroups of the fused launch on the current device: one per CU (rounded
// down to whole groups), provided a workgroup fits a CU, so the grid is
// resident at once on an idle device; 0 if not.  Cached per device and kernel.
static int fused_blocks(FusedKernel k) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    static FusedKernel cached_k[64];
    static int cached_n[64];
    if (cached_k[dev] == k) return cached_n[dev];
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(k), kFusedThreads, 0) !=
        hipSuccess)
        return 0;
    const int n = per_cu >= 1 ? min(cus, kFusedMaxBlocks) / kGroups * kGroups : 0;
    cached_n[dev] = n;
    cached_k[dev] = k;
    return n;
}

// The fused launch's arguments for this layer, or no kernel when the layer,
// the batch or the device does not take the fused path.
static FusedKernel fused_plan(const swq_moe_layer *layer, int x_dtype, int batch, bool prenorm, FusedArgs *fa,
                              int *nb) {
    if (batch != 1) return nullptr;
    const swq_qlinear *mats[8] = {&layer->router, &layer->gate, &layer->up, &layer->down,
                                  &layer->shared_gate, &layer->shared_up, &layer->shared_down,
                                  &layer->shared_expert_gate};
    const int nmats = layer->has_shared ? 8 : 4;
    for (int i = 0; i < nmats; ++i)
        if (mats[i]->scales_type == SWQ_F32) return nullptr;
    FusedArgs a{};
    a.router = make_qmat(&layer->router);
    a.gate = make_qmat(&layer->gate);
    a.up = make_qmat(&layer->up);
    a.down = make_qmat(&layer->down);
    plan_qmat(&a.router, x_dtype);
    plan_qmat(&a.gate, x_dtype);
    plan_qmat(&a.up, x_dtype);
    plan_qmat(&a.down, SWQ_F32);
    if (layer->has_shared) {
        a.sh_gate = make_qmat(&layer->shared_gate);
        a.sh_up = make_qmat(&layer->shared_up);
        a.sh_down = make_qmat(&layer->shared_down);
        a.seg = make_qmat(&layer->shared_expert_gate);
        plan_qmat(&a.sh_gate, x_dtype);
        plan_qmat(&a.sh_up, x_dtype);
        plan_qmat(&a.seg, x_dtype);
        plan_qmat(&a.sh_down, SWQ_F32);
        if (a.sh_down.bits != a.down.bits) return nullptr;
    }
    if (layer->moe_intermediate > kMaxInterFused) return nullptr;
    if (layer->has_shared && layer->shared_intermediate > kMaxInterFused) return nullptr;
    if (prenorm && layer->hidden > kPrenormMaxHidden) return nullptr;
    FusedKernel kern = fused_kernel_for(a.gate, a.down, x_dtype, prenorm);
    if (!kern) return nullptr;
    const int blocks = fused_blocks(kern);
    if (blocks <= 0) return nullptr;
    const int H = layer->hidden;
    a.nb = blocks;
    a.rows_cmb = (H + blocks - 1) / blocks;
    if (a.rows_cmb > kMaxCombineRows) return nullptr;
    a.H = H;
    a.E = layer->num_experts;
    a.K = layer->top_k;
    a.I = layer->moe_intermediate;
    a.Is = layer->has_shared ? layer->shared_intermediate : 0;
    a.norm = layer->norm_topk_prob ? 1 : 0;
    a.has_shared = layer->has_shared ? 1 : 0;
    a.router_tiles = (a.E + tile_rows(a.router) - 1) / tile_rows(a.router);
    a.p1_tiles = a.router_tiles + (a.has_shared ? (a.Is + tile_rows(a.sh_gate) - 1) / tile_rows(a.sh_gate) : 0);
    a.gu_tpe = (a.I + tile_rows(a.gate) - 1) / tile_rows(a.gate);
    a.gu_tiles = a.K * a.gu_tpe;
    a.dn_tpe = (H + tile_rows(a.down) - 1) / tile_rows(a.down);
    a.dn_tpe_sh = a.has_shared ? (H + tile_rows(a.sh_down) - 1) / tile_rows(a.sh_down) : 0;
    int dev = 0;
    a.local = (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64 && g_groups_local[dev] == 1) ? 1 : 0;
    *fa = a;
    *nb = blocks;
    return kern;
}

size_t fused_ws_bytes(const swq_moe_layer *l, size_t base) { return fused_layout(l, base).total; }

int fused_decode(const swq_moe_layer *layer, const void *x, int x_dtype, int batch, void *out, int out_dtype,
                 int32_t *topk_ids, float *topk_weights, void *ws, size_t ws_bytes, size_t staged_bytes,
                 bool accumulate, hipStream_t stream, bool *taken, const FusedPrenorm *pn) {
    *taken = false;
    FusedArgs a;
    int nb = 0;
    FusedKernel k = fused_plan(layer, x_dtype, batch, pn != nullptr, &a, &nb);
    if (!k) return SWQ_OK;
    const FusedLayout fl = fused_layout(layer, staged_bytes);
    if (ws_bytes < fl.total) return SWQ_OK;
    uint8_t *wsb = static_cast<uint8_t *>(ws);
    a.x = x;
    a.out = out;
    a.user_ids = topk_ids;
    a.user_w = topk_weights;
    a.gen = reinterpret_cast<uint32_t *>(wsb + fl.gen);
    a.err = reinterpret_cast<uint32_t *>(wsb + kWsErrByte);
    a.logit_x = reinterpret_cast<uint64_t *>(wsb + fl.logit_x);
    a.hsh_x = reinterpret_cast<uint64_t *>(wsb + fl.hsh_x);
    a.h_x = reinterpret_cast<uint64_t *>(wsb + fl.h_x);
    a.part_x = reinterpret_cast<uint64_t *>(wsb + fl.part_x);
    a.rep_stride = fl.rep_stride;
    a.odt = out_dtype;
    a.accumulate = accumulate ? 1 : 0;
    if (pn) {
        a.h_in = pn->h;
        a.res_in = pn->residual;
        a.norm_w = pn->weight;
        a.norm_dtype = pn->dtype;
        a.norm_eps = pn->eps;
    }
    hipLaunchKernelGGL(k, dim3(nb), dim3(kFusedThreads), 0, stream, a);
    const int st = launch_status();
    if (st != SWQ_OK) return st;
    *taken = true;
    return SWQ_OK;
}

size_t fused_err_offset(const swq_moe_layer *l, size_t base) { return fused_layout(l, base).err; }

// Records, once per device, whether a grid of one workgroup per CU places
// every group's workgroups on one XCD: a launch of that grid reports each
// workgroup's XCC_ID.  Blocking; runs on `stream`.
int fused_probe_device(hipStream_t stream) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return SWQ_ERR_HIP;
    if (g_groups_local[dev] >= 0) return SWQ_OK;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return SWQ_ERR_HIP;
    const int n = min(cus, kFusedMaxBlocks) / kGroups * kGroups;
    if (n < kGroups) {
        g_groups_local[dev] = 0;
        return SWQ_OK;
    }
    int32_t *d = nullptr;
    if (hipMalloc(&d, n * sizeof(int32_t)) != hipSuccess) return SWQ_ERR_HIP;
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(n), dim3(kFusedThreads), 0, stream, d);
    int32_t h[kFusedMaxBlocks];
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpyAsync(h, d, n * sizeof(int32_t), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    hipFree(d);
    if (e != hipSuccess) return SWQ_ERR_HIP;
    int ok = 1;
    for (int i = kGroups; i < n; ++i) ok &= h[i] == h[i % kGroups];
    g_groups_local[dev] = ok;
    return SWQ_OK;
}

}  // namespace swq
