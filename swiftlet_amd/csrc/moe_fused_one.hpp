// The single launch for a layer of one routed expert and no shared expert at
// batch 1: the expert's SwiGLU MLP behind a one-row router (the single-expert
// workload of QwenCPUModel.moeForward, QwenCPUModel.swift:500-569, with E = 1).
//
// With one expert there is nothing to route between workgroups: the pick is
// expert 0 and its weight is the softmax of one logit (normalised or not).
// Against moe_fused, whose slot 0 would sit on one XCD group and whose output
// rows come back through a second exchange hop, this kernel
// - computes the router's one logit in every workgroup (on its last wave) and
//   the weight from it by the same rounds, so no logit crosses workgroups;
// - spreads the gate/up tiles over wave pairs of the grid (tile t on pair
//   t / NB of workgroup t mod NB: its gate rows on the even wave, its up rows
//   on the odd one, handed over in LDS for the SwiGLU), each activation
//   published as one (value, epoch) word for every XCD;
// - has every workgroup poll all the activations into LDS and compute its own
//   output rows whole, so no partial output crosses workgroups.
// Tiles, lane maps and reduction orders are moe_fused's, so the results equal
// the other decode paths' bit for bit.
#pragma once

#include "moe_fused.hpp"

namespace swq {

template <int XDT, int GB, int GC, int GX, int GRI, int DB, int RC>
__global__ __launch_bounds__(kFusedThreads) __attribute__((amdgpu_waves_per_eu(kFusedWaves / 4, kFusedWaves / 4))) void moe_fused_one(FusedArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t s_hb[kMaxInterFused];  // the expert's activations
    __shared__ int32_t s_ids[1];
    __shared__ float s_w;
    __shared__ float s_up[kFusedWaves / 2][2 * kWave];  // up rows of each wave pair's tile (at most 2 x 64)

    static_assert(sizeof(FusedArgs) <= 1024, "kernel arguments");
    SWQ_TRACE_DECL;
    prefetch_kernargs();
    SWQ_STAMP(0);
    const int wave = threadIdx.x >> 6;
    int lane = threadIdx.x & 63;
    const int b = blockIdx.x, NB = a.nb;
    const int r0 = b * a.rows_cmb;  // this workgroup's output rows
    const int nr = max(0, min(a.rows_cmb, a.H - r0));
    asm volatile("" : "+v"(lane));
    const LaneMap lmg = lane_map(a.gate.lpr_log2, lane);
    const LaneMap lmd = lane_map(a.down.lpr_log2, lane);
    const LaneMap lmr = lane_map(a.router.lpr_log2, lane);

    // gate/up tile t on the wave pair t / NB of workgroup t mod NB: its gate
    // rows on the even wave, its up rows on the odd one
    const int pair = wave >> 1, is_up = wave & 1;
    const int t0 = b + NB * pair;
    const int gu_iters = (a.gu_tpe + NB * (kFusedWaves / 2) - 1) / (NB * (kFusedWaves / 2));  // uniform
    const bool has_g = t0 < a.gu_tpe;
    const bool rwave = wave == kFusedWaves - 1;
    const int passes = (nr + lmd.rpw - 1) / lmd.rpw;  // passes of this workgroup's down rows, pass p on wave p
    const bool has_d = wave < passes;
    // Loads in the order they are needed: the wave's gate or up rows and their
    // x slice, the epoch, this wave's first pass of the workgroup's down rows,
    // then (last wave) the router row and its x slice, whose logit is needed
    // only for the output.
    RowTile<GB, GC, 2, GRI> tg;
    if (has_g) load_tile(tg, is_up ? a.up : a.gate, 0, lmg, t0 * GRI * lmg.rpw, a.I);
    XRaw<XDT, GB, GC> xgr;
    if (has_g) load_xraw<XDT>(xgr, a.gate, lmg, a.x, 0);
    asm volatile("" ::: "memory");
    const uint32_t g = __hip_atomic_load(a.gen + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    asm volatile("" ::: "memory");
    RowTile<DB, 1, 2, 1> dt;
    if (has_d) load_tile(dt, a.down, 0, lmd, r0 + wave * lmd.rpw, r0 + nr);
    RowTile<8, RC, 2, 1> rt;
    XRaw<XDT, 8, RC> xrr;
    if (rwave) {
        load_tile(rt, a.router, 0, lmr, 0, a.E);
        load_xraw<XDT>(xrr, a.router, lmr, a.x, 0);
    }
    asm volatile("" ::: "memory");

    // ---- gate/up + SwiGLU: wave pairs over the grid ------------------------
    {
        XSlice<GB, GC, GX> xg;
        if (has_g) xslice_convert(xg, xgr);
        for (int it = 0; it < gu_iters; ++it) {
            const int t = t0 + it * NB * (kFusedWaves / 2);
            const bool live = t < a.gu_tpe;
            const int row0 = t * GRI * lmg.rpw;
            float r[GRI];
            if (live) {
                if (it > 0) load_tile(tg, is_up ? a.up : a.gate, 0, lmg, row0, a.I);
                dot_rows(r, tg, is_up ? a.up : a.gate, xg, lmg);
                if (is_up && lmg.j == lmg.lpr - 1) {
#pragma unroll
                    for (int i = 0; i < GRI; ++i) s_up[pair][i * lmg.rpw + lmg.q] = r[i];
                }
            }
            __syncthreads();  // s_up
            if (live && !is_up && lmg.j == lmg.lpr - 1) {
#pragma unroll
                for (int i = 0; i < GRI; ++i) {
                    const int row = row0 + i * lmg.rpw + lmg.q;
                    if (row < a.I) put_pair(a.h_x + row, swiglu(r[i], s_up[pair][i * lmg.rpw + lmg.q]), g);
                }
            }
            if (it + 1 < gu_iters) __syncthreads();  // s_up is rewritten
        }
        SWQ_STAMP(4);
    }

    // ---- the router's logit and the weight (last wave) -----------------------
    asm volatile("" : "+v"(lane));
    if (rwave) {
        XSlice<8, RC, kXF32> xr;
        xslice_convert(xr, xrr);
        float res[1];
        dot_rows(res, rt, a.router, xr, lmr);
        // row 0's sum sits on its last lane
        float v[1] = {__shfl(res[0], lmr.lpr - 1, kWave)};
        Rounds<1> rd;
        rounds_init(rd, v, a.E, lane);
        rounds_run(rd, 1, lane, s_ids);
        const float w = rounds_weight(rd, 1, a.norm, lane);
        if (lane == 0) {
            s_w = w;
            if (b == 0) {
                if (a.user_ids) a.user_ids[0] = s_ids[0];
                if (a.user_w) a.user_w[0] = w;
            }
        }
        SWQ_STAMP(2);
    }

    // ---- every activation into LDS, an eighth per wave -----------------------
    const int np = a.I / 2, q = (np + kFusedWaves - 1) / kFusedWaves;
    fetch_acts<DB>(a.h_x, min(np, wave * q), min(np, (wave + 1) * q), g, s_hb, lane, a.err);
    __syncthreads();  // s_hb, s_w
    SWQ_STAMP(5);

    // ---- this workgroup's output rows ----------------------------------------
    asm volatile("" : "+v"(lane));
    for (int p = wave; p < passes; p += kFusedWaves) {
        const int row0 = r0 + p * lmd.rpw;
        if (p != wave) load_tile(dt, a.down, 0, lmd, row0, r0 + nr);
        float res[1];
        down_dot<DB, 1>(res, dt, a.down, lmd, s_hb);
        const int row = row0 + lmd.q;
        if (lmd.j == lmd.lpr - 1 && row < r0 + nr) {
            // out = w_0 d_0 (QwenCPUModel.swift:549-556), summed as the
            // other paths' combine
            float acc = 0.f;
            acc += s_w * res[0];
            if (a.odt == SWQ_BF16) {
                static_cast<uint16_t *>(a.out)[row] = f32_to_bf16_rne(acc);
            } else {
                float *out = static_cast<float *>(a.out);
                out[row] = a.accumulate ? out[row] + acc : acc;
            }
        }
    }
    SWQ_STAMP(6);
    if (wave == 0) {
        // the next call's epoch: every entry, whatever grid the next call uses
        for (int i = b + NB * lane; i < kFusedMaxBlocks; i += NB * kWave)
            __hip_atomic_store(a.gen + i, g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        SWQ_STAMP(9);
    }
    SWQ_TRACE_FLUSH;
}

}  // namespace swq
