// The MoE-layer decode step for 2 or 4 tokens in one launch (gfx950).
//
// The single-token kernel of moe_fused.hpp with token-major slots: slot s is
// pick s % K of token s / K, and XCD group grp owns slots grp, grp + 8, ...
// (kFusedMaxSlots at most).  Each (token, pick) is computed as the
// single-token kernel computes a pick (the same tiles, lane plans and
// summation orders), so the outputs equal the three-launch path's bit for
// bit; an expert picked by two tokens is read once per token (the three
// launches read it once).  Phase A splits the router and the shared expert
// into (tile, token) units over the waves (B divides 8, so a wave's units are
// of one token); wave t routes token t; the routed work is phase-major: the
// gate/up rows of every owned slot stream with one slot in flight ahead,
// then one exchange wait brings the activations of every owned slot but the
// last, whose wait comes after the other slots' down rows; the combine
// writes token t's rows on wave t.
#pragma once

#include "moe_fused.hpp"

namespace swq {

constexpr int kFusedMaxSlots = 4;  // slots per XCD group: B K <= 32

// One wave's activation pairs [p0, p1) of the slots grp + 8 j, j0 <= j < j1
// (token-major rows of I words at hx), into hbb[j], and with NS > 0 its
// pairs [f0, f1) of the shared expert's activations of all tokens laid end to
// end (rows of Is words at hs, nps pairs each) into hsh: each polling round
// takes 2 routed and NS shared pairs per lane, so the usual shapes need one
// round trip for everything.  mid() runs once, between the first round's
// loads and their check (with no pairs at all, before returning).
template <int DB, int NS, typename F>
__device__ __forceinline__ void fetch_slots(const uint64_t *hx, int I, int grp, int j0, int j1, int p0, int p1,
                                            uint32_t (*hbb)[kMaxInterFused], const uint64_t *hs, int Is, int nps,
                                            int f0, int f1, uint32_t (*hsh)[kMaxInterFused], uint32_t g, int lane,
                                            uint32_t *err, F &&mid) {
    constexpr int N = 4 + 2 * NS;
    const int c = p1 - p0, nr = c > 0 && j1 > j0 ? (j1 - j0) * c : 0;
    const int ns = NS > 0 ? max(f1 - f0, 0) : 0;
    if (nr <= 0 && ns <= 0) mid();
    for (int q = 0, qs = 0; q < nr || qs < ns; q += 2 * kWave, qs += NS * kWave) {
        const uint64_t *pp[N];
        bool live[N];
        int rj[2], rp[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int f = q + u * kWave + lane;
            live[2 * u] = live[2 * u + 1] = f < nr;
            const int fc = f < nr ? f : 0;
            const int jj = c > 0 ? fc / c : 0;
            rj[u] = j0 + jj;
            rp[u] = p0 + fc - jj * c;
            const uint64_t *row = hx + static_cast<int64_t>(grp + kGroups * rj[u]) * I;
            pp[2 * u] = row + pair_first<DB>(rp[u]);
            pp[2 * u + 1] = row + pair_second<DB>(rp[u]);
        }
        int st[NS > 0 ? NS : 1], sq[NS > 0 ? NS : 1];
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int f = f0 + qs + u * kWave + lane;
            const bool l = qs + u * kWave + lane < ns;
            live[4 + 2 * u] = live[5 + 2 * u] = l;
            const int fc = l ? f : f0;
            st[u] = fc / nps;
            sq[u] = fc - st[u] * nps;
            const uint64_t *row = hs + static_cast<int64_t>(st[u]) * Is;
            pp[4 + 2 * u] = row + pair_first<DB>(sq[u]);
            pp[5 + 2 * u] = row + pair_second<DB>(sq[u]);
        }
        float v[N];
        if (q == 0) poll_words_mid<N>(pp, live, g, v, err, 1u, mid);
        else poll_words<N>(pp, live, g, v, err, 1u);
#pragma unroll
        for (int u = 0; u < 2; ++u)
            if (live[2 * u]) store_pair_lds<DB>(hbb[rj[u]], rp[u], v[2 * u], v[2 * u + 1]);
#pragma unroll
        for (int u = 0; u < NS; ++u)
            if (live[4 + 2 * u]) store_pair_lds<DB>(hsh[st[u]], sq[u], v[4 + 2 * u], v[5 + 2 * u]);
    }
}

template <int XDT, int GB, int GC, int GX, int GRI, int DB, int DRI, int RC, int M>
__global__ __launch_bounds__(kFusedThreads) __attribute__((amdgpu_waves_per_eu(kFusedWaves / 4, kFusedWaves / 4))) void moe_fused_batch(FusedArgs a) {
    constexpr int MB = kFusedMaxBatch;
    static_assert(kFusedWaves % MB == 0, "tokens: a divisor of the waves");
    __shared__ int32_t s_ids[MB * SWQ_MAX_TOPK];  // picks, token-major
    __shared__ float s_w[MB * SWQ_MAX_TOPK];
    __shared__ __attribute__((aligned(16))) uint32_t s_hbb[kFusedMaxSlots][kMaxInterFused];  // owned slots' activations
    __shared__ __attribute__((aligned(16))) uint32_t s_hsh[MB][kMaxInterFused];  // the shared expert's
    __shared__ float s_cmb[MB * SWQ_MAX_TOPK * kMaxCombineRows];
    __shared__ float s_shd[MB][kMaxCombineRows];  // shared-expert down rows of the combine rows
    __shared__ float s_sg[MB];    // shared-expert gate logits

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
    const int B = a.B;  // 2 or 4
    const int bl = B == 4 ? 2 : 1;  // log2 B
    const int grp = b % kGroups, rank = b / kGroups, NPG = NB / kGroups;
    if (threadIdx.x < MB * SWQ_MAX_TOPK) s_ids[threadIdx.x] = -1;
    const void *x = a.x;
    __syncthreads();
    const int r0 = b * a.rows_cmb;                      // this workgroup's output rows
    const int nr = max(0, min(a.rows_cmb, a.H - r0));
    const int64_t x_stride = static_cast<int64_t>(a.H) * (XDT == 2 ? 2 : 4);
    auto xtok = [&](int t) -> const void * { return static_cast<const uint8_t *>(x) + t * x_stride; };

    // ---- phase A ------------------------------------------------------------
    // Every load first (weights, then activations), conversions after: the
    // router row is on the critical path, and a conversion between two loads
    // would make the second wait for the first.
    asm volatile("" : "+v"(lane));
    const LaneMap lmg = lane_map(a.gate.lpr_log2, lane);
    const LaneMap lmr = lane_map(a.router.lpr_log2, lane);
    // Router units (tile, token): this workgroup's router tiles are
    // b, b + NB, ...; unit u = (tile u / B, token u % B) runs on wave u mod 8.
    // Shared gate/up units likewise, unit u on wave 7 - (u mod 8).  With one
    // token, wave w takes router tile b + NB w and shared tile b + NB (7 - w);
    // B divides 8, so each wave's units are of one token.
    const int r_tiles = (a.E + lmr.rpw - 1) / lmr.rpw;
    const bool has_r = b + NB * (wave >> bl) < r_tiles;
    // token t's shared-expert gate logit on wave 7 - t, the wave of its
    // shared gate/up unit (with one shared tile per workgroup)
    const int seg_tok = kFusedWaves - 1 - wave;
    const bool do_seg = a.has_shared && seg_tok < B;
    const int us0 = kFusedWaves - 1 - wave;  // this wave's first shared unit
    const bool has_s = a.has_shared && b + NB * (us0 >> bl) < a.sh_tiles;
    RowTile<8, RC, 2, 1> rt;
    if (has_r) load_tile(rt, a.router, 0, lmr, (b + NB * (wave >> bl)) * lmr.rpw, a.E);
    else if (do_seg) load_tile(rt, a.seg, 0, lmr, 0, 1);
    RowTile<GB, GC, 2, 1> stg, stu;
    if (has_s) {
        load_tile(stg, a.sh_gate, 0, lmg, (b + NB * (us0 >> bl)) * lmg.rpw, a.Is);
        load_tile(stu, a.sh_up, 0, lmg, (b + NB * (us0 >> bl)) * lmg.rpw, a.Is);
    }
    // the shared expert's down rows of this workgroup's output rows: one
    // pass of rows each for waves 1.., loaded now, used once the shared
    // activations are in
    const LaneMap lms = lane_map(a.sh_down.lpr_log2, lane);
    const bool sh_rows = a.has_shared && nr > 0;
    const int sh_passes = sh_rows ? (nr + lms.rpw - 1) / lms.rpw : 0;
    // (the waves from B on, which have no token to route and combine)
    const int sp0 = wave - B, nsw = kFusedWaves - B;
    XRaw<XDT, 8, RC> xrr;
    if (has_r) load_xraw<XDT>(xrr, a.router, lmr, xtok(wave & (B - 1)), 0);
    else if (do_seg) load_xraw<XDT>(xrr, a.router, lmr, xtok(seg_tok), 0);
    // the gate/up slice of this wave's shared units' token
    XRaw<XDT, GB, GC> xgr;
    if (has_s) load_xraw<XDT>(xgr, a.gate, lmg, xtok(us0 & (B - 1)), 0);
    // The call's epoch, loaded after every other load of phase A: vector
    // loads complete in issue order, so the first wait for it waits for them
    // too, which the router row needs anyway; issued first, any wait for it
    // after the roles' branches would drain every load.
    asm volatile("" ::: "memory");
    const uint32_t g = __hip_atomic_load(a.gen + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    if (has_r || do_seg) {
        XSlice<8, RC, kXF32> xr;
        xslice_convert(xr, xrr);
        int xr_tok = has_r ? wave & (B - 1) : seg_tok;  // the token of xr
        for (int u = wave; b + NB * (u >> bl) < r_tiles; u += kFusedWaves) {
            // router units: one pass of rows of tile b + NB (u / B) for token
            // u % B -> logits
            const int t = b + NB * (u >> bl), tok = u & (B - 1);
            if (u != wave) load_tile(rt, a.router, 0, lmr, t * lmr.rpw, a.E);
            float res[1];
            dot_rows(res, rt, a.router, xr, lmr);
            const int row = t * lmr.rpw + lmr.q;
            if (lmr.j == lmr.lpr - 1 && row < a.E) {
#pragma unroll
                for (int r = 0; r < kReplicas; ++r)
                    put_pair(a.logit_x + (tok * kReplicas + r) * a.rep_stride + row, res[0], g);
            }
            SWQ_STAMP(10);
        }
        if (do_seg) {
            // token seg_tok's shared-expert gate logit <w_sg, x_t> (this
            // workgroup's combine)
            if (has_r) load_tile(rt, a.seg, 0, lmr, 0, 1);
            if (seg_tok != xr_tok) {
                load_xraw<XDT>(xrr, a.router, lmr, xtok(seg_tok), 0);
                xslice_convert(xr, xrr);
            }
            float res[1];
            dot_rows(res, rt, a.seg, xr, lmr);
            if (lane == lmr.lpr - 1) s_sg[seg_tok] = res[0];
        }
    }
    asm volatile("" : "+v"(lane));
    if (has_s) {
        XSlice<GB, GC, GX> xg;
        xslice_convert(xg, xgr);
        for (int u = us0; a.has_shared && b + NB * (u >> bl) < a.sh_tiles; u += kFusedWaves) {
            // shared-expert gate/up units: one pass of rows of tile b + NB (u / B)
            // for token u % B -> SwiGLU activations
            const int row0 = (b + NB * (u >> bl)) * lmg.rpw, tok = u & (B - 1);
            if (u != us0) {
                load_tile(stg, a.sh_gate, 0, lmg, row0, a.Is);
                load_tile(stu, a.sh_up, 0, lmg, row0, a.Is);
            }
            float rg[1], ru[1];
            dot_rows2(rg, ru, stg, stu, a.sh_gate, a.sh_up, xg, lmg);
            const int row = row0 + lmg.q;
            if (lmg.j == lmg.lpr - 1 && row < a.Is) put_pair(a.hsh_x + tok * a.Is + row, swiglu(rg[0], ru[0]), g);
            SWQ_STAMP(11);
        }
    }
    SWQ_STAMP(1);

    // ---- routing (wave t routes token t) -------------------------------------
    // Slot s (0 <= s < B K) is pick s mod K of token s / K; group grp owns
    // slots grp, grp + 8, ...  Each pick goes to LDS as its round ends.
    Rounds<M> rd;
    asm volatile("" : "+v"(lane));
    if (wave < B) {
        const uint64_t *rep = a.logit_x + (wave * kReplicas + b % kReplicas) * a.rep_stride;
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
        // the rounds up to this group's last pick of this token; the rest
        // after the routed work
        const int k0 = ((grp - wave * a.K) % kGroups + kGroups) % kGroups;
        const int own_last = k0 < a.K ? k0 + kGroups * ((a.K - 1 - k0) / kGroups) : -1;
        rounds_run(rd, own_last + 1, lane, s_ids + wave * a.K);
        SWQ_STAMP(3);
    }

    // ---- routed slots of the group: gate/up of every owned slot, then down --
    // Slot s (0 <= s < B K) is pick s % K of token s / K; group grp owns the
    // slots grp + 8 j, j < nsl <= kFusedMaxSlots.  Phase G streams their
    // gate/up rows with the next slot's tiles (and its token's x slice) in
    // flight during the current slot's dot products; phase D streams the
    // down rows the same way, polling the last slot's activations only after
    // the other slots' down rows.
    const int S = B * a.K;
    const int nsl = S > grp ? (S - 1 - grp) / kGroups + 1 : 0;
    const int np_r = a.I / 2, q_r = (np_r + kFusedWaves - 1) / kFusedWaves;
    const int np_s = a.Is / 2;
    asm volatile("" : "+v"(lane));
    const LaneMap lmd = lane_map(a.down.lpr_log2, lane);
    const int t0 = rank + NPG * wave;  // this wave's first tile of a slot
    const bool gu1 = t0 < a.gu_tpe, dn1 = t0 < a.dn_tpe;
    int64_t ex[kFusedMaxSlots];  // the owned slots' experts
    // Down tiles of slots j (mod 2): the first two go out before the
    // activation polls, slot j + 2's as soon as slot j's down rows are done.
    // (Issued during the last slot's gate/up rows instead, they overlap
    // more, but the tiles then live across the gate/up code and the 8-bit
    // kernels spill: 68.7 against 39.0 us at batch 4.)
    using DTile = RowTile<DB, 1, 2, DRI>;
    DTile dt0, dt1;
    RowTile<DB, 1, 2, 1> sdt;
    {
        using GTile = RowTile<GB, GC, 2, GRI>;
        using GX_ = XRaw<XDT, GB, GC>;
        GTile tga, tua, tgb, tub;
        GX_ xra, xrb;
        // slot j's pick, its token's slice and its first gate/up tiles
        auto issue = [&](int j, GTile &tg, GTile &tu, GX_ &xr) {
            const int s = grp + kGroups * j;
            ex[j] = min(wait_lds_nonneg(&s_ids[s], a.err), a.E - 1);
            load_xraw<XDT>(xr, a.gate, lmg, xtok(s / a.K), 0);
            if (gu1) {
                load_tile(tg, a.gate, ex[j], lmg, t0 * GRI * lmg.rpw, a.I);
                load_tile(tu, a.up, ex[j], lmg, t0 * GRI * lmg.rpw, a.I);
            }
        };
        // slot j's gate/up rows + SwiGLU -> activations (XCD-local words)
        auto compute = [&](int j, GTile &tg, GTile &tu, const GX_ &xr) {
            const int s = grp + kGroups * j;
            XSlice<GB, GC, GX> xs;
            xslice_convert(xs, xr);
            for (int t = t0; t < a.gu_tpe; t += NPG * kFusedWaves) {
                const int row0 = t * GRI * lmg.rpw;
                if (t != t0) {
                    load_tile(tg, a.gate, ex[j], lmg, row0, a.I);
                    load_tile(tu, a.up, ex[j], lmg, row0, a.I);
                }
                float rg[GRI], ru[GRI];
                dot_rows2(rg, ru, tg, tu, a.gate, a.up, xs, lmg);
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
        };
        if (nsl > 0) issue(0, tga, tua, xra);
#pragma unroll
        for (int j = 0; j < kFusedMaxSlots; ++j) {
            if (j < nsl) {
                if (j + 1 < nsl) {
                    if (j & 1) issue(j + 1, tga, tua, xra);
                    else issue(j + 1, tgb, tub, xrb);
                }
                if (j & 1) compute(j, tgb, tub, xrb);
                else compute(j, tga, tua, xra);
                SWQ_STAMP(4);
            }
        }
    }
    {
        // The first two slots' down tiles (and on the waves from B on the
        // shared down tile).  4-bit down rows: issued between the activation
        // poll's loads and their check (issued first, they would hold the
        // poll's round trip behind their own: 35B q4 at batch 4 38.8 ->
        // 35.8 us, the 80B layer at batch 2 37.5 -> 31.3).  8-bit rows go out
        // before the poll (between its loads and check they measured 41.6 us
        // at batch 4 against 36.9 this way).
        auto tiles = [&]() __attribute__((always_inline)) {
            if (nsl > 0 && dn1) {
                load_tile(dt0, a.down, ex[0], lmd, t0 * DRI * lmd.rpw, a.H);
                if (nsl > 1) load_tile(dt1, a.down, ex[1], lmd, t0 * DRI * lmd.rpw, a.H);
            }
            if (wave >= B && sp0 < sh_passes) load_tile(sdt, a.sh_down, 0, lms, r0 + sp0 * lms.rpw, r0 + nr);
        };
        constexpr bool kTilesMid = DB == 4;
        if constexpr (!kTilesMid) {
            tiles();
            // Without this the compiler may sink the down tiles' loads below
            // the polls and the barrier that follow (allowed across an
            // acquire), so they would start only once the activations are in.
            asm volatile("" ::: "memory");
        }
        auto mid = [&]() __attribute__((always_inline)) {
            if constexpr (kTilesMid) tiles();
        };
        // The activations of every owned slot but the last (an eighth polled
        // by each wave) and, on the waves from B on, a share of the shared
        // expert's activations of every token (written in phase A), in one
        // round trip; the last slot's come after the other slots' down rows,
        // so that the group's last gate/up rows are not waited for first.
        const int pr0 = min(np_r, wave * q_r), pr1 = min(np_r, (wave + 1) * q_r);
        const int jl = max(nsl - 1, 0);
        if (wave >= B && sh_rows) {
            const int nf = B * np_s, q3 = (nf + nsw - 1) / nsw;
            fetch_slots<DB, 4>(a.h_x, a.I, grp, 0, jl, pr0, pr1, s_hbb, a.hsh_x, a.Is, np_s, min(nf, sp0 * q3),
                               min(nf, (sp0 + 1) * q3), s_hsh, g, lane, a.err, mid);
        } else {
            fetch_slots<DB, 0>(a.h_x, a.I, grp, 0, jl, pr0, pr1, s_hbb, a.hsh_x, a.Is, np_s, 0, 0, s_hsh, g, lane,
                               a.err, mid);
        }
        __syncthreads();
        SWQ_STAMP(5);
#pragma unroll
        for (int j = 0; j < kFusedMaxSlots; ++j) {
            if (j < nsl) {
                const int s = grp + kGroups * j;
                if (j == jl) {  // nsl is the same on every wave
                    fetch_slots<DB, 0>(a.h_x, a.I, grp, jl, jl + 1, pr0, pr1, s_hbb, a.hsh_x, a.Is, np_s, 0, 0,
                                       s_hsh, g, lane, a.err, [] {});
                    __syncthreads();
                }
                DTile &dt = (j & 1) ? dt1 : dt0;
                for (int t = t0; t < a.dn_tpe; t += NPG * kFusedWaves) {
                    const int row0 = t * DRI * lmd.rpw;
                    if (t != t0) load_tile(dt, a.down, ex[j], lmd, row0, a.H);
                    float res[DRI];
                    down_dot<DB, DRI>(res, dt, a.down, lmd, s_hbb[j]);
                    if (lmd.j == lmd.lpr - 1) {
#pragma unroll
                        for (int i = 0; i < DRI; ++i) {
                            const int row = row0 + i * lmd.rpw + lmd.q;
                            if (row < a.H) put_pair(a.part_x + static_cast<int64_t>(s) * a.H + row, res[i], g);
                        }
                    }
                }
                if (j + 2 < nsl && dn1) load_tile(dt, a.down, ex[j + 2], lmd, t0 * DRI * lmd.rpw, a.H);
            }
        }
        SWQ_STAMP(6);
    }
    // ---- tail: waves B..: the shared expert's down rows for every token;
    // wave t < B: token t's remaining picks, its weights and this
    // workgroup's rows of each of its slots' down outputs --------------------
    asm volatile("" : "+v"(lane));
    if (wave >= B && sh_rows) {
        // this wave's passes of the shared down rows for each token (the
        // shared activations came in with the routed ones)
        for (int sp = sp0; sp < sh_passes; sp += nsw) {
            const int row0 = r0 + sp * lms.rpw;
            if (sp != sp0) load_tile(sdt, a.sh_down, 0, lms, row0, r0 + nr);
            const int row = row0 + lms.q;
            for (int tok = 0; tok < B; ++tok) {
                float res[1];
                down_dot<DB, 1>(res, sdt, a.sh_down, lms, s_hsh[tok]);
                if (lms.j == lms.lpr - 1 && row < r0 + nr) s_shd[tok][row - r0] = res[0];
            }
        }
        SWQ_STAMP(7);
    }
    if (wave < B) {
        const int t = wave;
        rounds_run(rd, a.K, lane, s_ids + t * a.K);
        const float w = rounds_weight(rd, a.K, a.norm, lane);
        if (lane < a.K) {
            s_w[t * a.K + lane] = w;
            if (b == 0) {
                if (a.user_ids) a.user_ids[t * a.K + lane] = s_ids[t * a.K + lane];
                if (a.user_w) a.user_w[t * a.K + lane] = w;
            }
        }
        const int n = a.K * nr;
        const uint64_t *pt = a.part_x + static_cast<int64_t>(t) * a.K * a.H;
        float *ct = s_cmb + t * a.K * nr;
        for (int j0 = 0; j0 < n; j0 += 2 * kWave) {
            const uint64_t *pp[2];
            bool live[2];
            int jj[2];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                jj[c] = j0 + c * kWave + lane;
                live[c] = jj[c] < n;
                const int jc = min(jj[c], n - 1), k = jc / nr;
                pp[c] = pt + static_cast<int64_t>(k) * a.H + r0 + (jc - k * nr);
            }
            float v[2];
            poll_words<2>(pp, live, g, v, a.err, 8u);
#pragma unroll
            for (int c = 0; c < 2; ++c)
                if (live[c]) ct[jj[c]] = v[c];
        }
        SWQ_STAMP(8);
    }
    __syncthreads();  // s_w, s_cmb, s_shd, s_sg

    // ---- combine (wave t: token t) -------------------------------------------
    if (wave < B) {
        const int t = wave;
        const float gate = a.has_shared ? sigmoidf_ref(s_sg[t]) : 0.f;
        if (lane < nr) {
            // out = sum_k w_k d_k in pick order, then + sigmoid(sg) * shared
            // (QwenCPUModel.swift:549-566)
            float acc = 0.f;
            for (int k = 0; k < a.K; ++k) acc += s_w[t * a.K + k] * s_cmb[(t * a.K + k) * nr + lane];
            if (a.has_shared) acc += gate * s_shd[t][lane];
            const int64_t row = static_cast<int64_t>(t) * a.H + r0 + lane;
            if (a.odt == SWQ_BF16) {
                static_cast<uint16_t *>(a.out)[row] = f32_to_bf16_rne(acc);
            } else {
                float *out = static_cast<float *>(a.out);
                out[row] = a.accumulate ? out[row] + acc : acc;
            }
        }
    }
    if (wave == 0) {
        // the next call's epoch: every entry, whatever grid the next call uses
        for (int i = b + NB * lane; i < kFusedMaxBlocks; i += NB * kWave)
            __hip_atomic_store(a.gen + i, g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        SWQ_STAMP(9);
    }
    SWQ_TRACE_FLUSH;
}

template <int XDT, int GB, int GC, int GX, int DB, int RC>
static FusedKernel fused_batch_by_m(int M) {
    constexpr int GRI = gate_passes(GB, GC), DRI = down_passes(DB);
    switch (M) {
        case 1: return moe_fused_batch<XDT, GB, GC, GX, GRI, DB, DRI, RC, 1>;
        case 2: return moe_fused_batch<XDT, GB, GC, GX, GRI, DB, DRI, RC, 2>;
        case 4: return moe_fused_batch<XDT, GB, GC, GX, GRI, DB, DRI, RC, 4>;
        case 8: return moe_fused_batch<XDT, GB, GC, GX, GRI, DB, DRI, RC, 8>;
        default: return moe_fused_batch<XDT, GB, GC, GX, GRI, DB, DRI, RC, 16>;
    }
}

}  // namespace swq
