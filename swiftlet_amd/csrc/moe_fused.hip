// Host side of the single-launch MoE decode step: plan, workspace layout,
// launch and the per-device probe.  The kernel is in moe_fused.hpp.
#include "moe_fused_batch.hpp"

#include <atomic>
#include <mutex>
#include <utility>
#include <vector>

namespace swq {

// ---------------------------------------------------------------------------
// host side

// The instantiation for this layer's formats, or nullptr: routed and shared
// gate/up rows in one format, 4- or 8-bit down rows, an 8-bit router and
// shared-expert gate.  M = ceil(E / 64), as the staged path's routing wave.
// `one`: the one-expert launch (moe_fused_one.hpp) in the same formats.
static FusedKernel fused_kernel_for(const QMat &router, const QMat &gate, const QMat &down, int x_dtype, int E,
                                    bool prenorm, bool batched, bool one) {
    if (router.bits != 8) return nullptr;
    const int m = (E + kWave - 1) / kWave;
    const int M = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : m <= 8 ? 8 : 16;
    const bool rc2 = router.cpl == 2;
    int gfmt = -1;
    if (gate.bits == 4 && down.bits == 4) {
        // 4-bit rows: packed bf16 activations (two chunks per lane) for bf16
        // x, fp32 (one chunk per lane) for f32 x
        if (x_dtype == SWQ_BF16 && !prenorm && gate.xf == 1 && gate.cpl == 2) gfmt = kFusedQ4;
        if ((x_dtype == SWQ_F32 || prenorm) && gate.xf == 0 && gate.cpl == 1) gfmt = kFusedQ4;
    } else if (gate.bits == 8 && down.bits == 8) {
        gfmt = gate.cpl == 2 ? kFusedQ8C2 : kFusedQ8C1;
    }
    if (gfmt < 0) return nullptr;
    if (one) return fused_select_one(x_dtype, gfmt, rc2);
    if (prenorm) return x_dtype == SWQ_F32 && !batched ? fused_select_pn(gfmt, rc2, M) : nullptr;
    if (batched) return x_dtype == SWQ_BF16 ? fused_select_bf16_batch(gfmt, rc2, M) : fused_select_f32_batch(gfmt, rc2, M);
    return x_dtype == SWQ_BF16 ? fused_select_bf16(gfmt, rc2, M) : fused_select_f32(gfmt, rc2, M);
}

// Per device, set once by fused_probe_device (under probe_mu, then read
// with acquire loads; cus > 0 once set): the CU count and whether the
// workgroups of each group (b mod kGroups) of a grid of one workgroup per CU
// run on one XCD.  The kernels whose occupancy has been checked sit in a
// small list under a mutex.
struct FusedDevice {
    std::mutex probe_mu;
    std::atomic<int> cus{0};
    std::atomic<int> local{0};
    std::mutex mu;
    std::vector<std::pair<FusedKernel, int>> fits;
};
static FusedDevice g_fused_dev[64];

__global__ __launch_bounds__(kFusedThreads) void xcd_probe_kernel(int32_t *out) {
    if (threadIdx.x == 0) {
        uint32_t v;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
        out[blockIdx.x] = static_cast<int32_t>(v & 0xFu);
    }
}

// Workgroups of the fused launch on device `dev`: one per CU, rounded down
// to whole groups, provided the kernel fits one workgroup per CU (so the
// grid is resident at once on an idle device); 0 if not, or before the
// device's probe.
static int fused_blocks(FusedKernel k, int dev) {
    FusedDevice &d = g_fused_dev[dev];
    const int cus = d.cus.load(std::memory_order_acquire);
    if (cus <= 0) return 0;
    int fits = -1;
    {
        std::lock_guard<std::mutex> lock(d.mu);
        for (const auto &f : d.fits)
            if (f.first == k) fits = f.second;
        if (fits < 0) {
            int per_cu = 0;
            fits = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(k),
                                                                kFusedThreads, 0) == hipSuccess &&
                           per_cu >= 1
                       ? 1
                       : 0;
            d.fits.emplace_back(k, fits);
        }
    }
    return fits ? min(cus, kFusedMaxBlocks) / kGroups * kGroups : 0;
}

// The fused launch's arguments for this layer, or no kernel when the layer,
// the batch or the device does not take the fused path.
static FusedKernel fused_plan(const swq_moe_layer *layer, int x_dtype, int batch, int max_batch, bool prenorm,
                              FusedArgs *fa, int *nb) {
    // one token, or 2 or 4 (a divisor of the eight waves, so that each wave's
    // phase-A units are of one token); others take the three stages
    if (batch != 1 && batch != 2 && batch != 4) return nullptr;
    if (batch > min(max_batch, kFusedMaxBatch) || (prenorm && batch != 1)) return nullptr;
    if (batch * layer->top_k > kFusedMaxSlots * kGroups) return nullptr;  // slots per XCD group
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
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
        // the shared rows take the routed ones' activation slices and tiles
        if (a.sh_gate.bits != a.gate.bits || a.sh_gate.lpr_log2 != a.gate.lpr_log2 || a.sh_gate.cpl != a.gate.cpl ||
            a.sh_gate.xf != a.gate.xf)
            return nullptr;
        if (a.sh_down.bits != a.down.bits || a.sh_down.cpl != 1) return nullptr;
        if (a.seg.bits != a.router.bits || a.seg.lpr_log2 != a.router.lpr_log2 || a.seg.cpl != a.router.cpl)
            return nullptr;
        if (layer->shared_intermediate > kMaxInterFused || layer->shared_intermediate % 2 != 0) return nullptr;
    }
    if (a.down.cpl != 1 || a.router.xf != 0) return nullptr;
    if (layer->moe_intermediate > kMaxInterFused || layer->moe_intermediate % 2 != 0) return nullptr;
    if (prenorm && layer->hidden > kPrenormMaxHidden) return nullptr;
    if (layer->hidden > kFusedMaxHidden || layer->num_experts > kMaxExperts) return nullptr;
    // one routed expert and no shared expert at batch 1: the one-expert launch
    const bool one = batch == 1 && !prenorm && layer->num_experts == 1 && !layer->has_shared;
    FusedKernel kern =
        fused_kernel_for(a.router, a.gate, a.down, x_dtype, layer->num_experts, prenorm, batch > 1, one);
    if (!kern) return nullptr;
    const int blocks = fused_blocks(kern, dev);
    if (blocks <= 0) return nullptr;
    const int H = layer->hidden;
    a.nb = blocks;
    a.B = batch;
    a.rows_cmb = (H + blocks - 1) / blocks;
    if (a.rows_cmb > kMaxCombineRows) return nullptr;
    a.H = H;
    a.E = layer->num_experts;
    a.K = layer->top_k;
    a.I = layer->moe_intermediate;
    a.Is = layer->has_shared ? layer->shared_intermediate : 0;
    a.norm = layer->norm_topk_prob ? 1 : 0;
    a.has_shared = layer->has_shared ? 1 : 0;
    const int gate_rpw = kWave >> a.gate.lpr_log2;
    a.sh_tiles = a.has_shared ? (a.Is + gate_rpw - 1) / gate_rpw : 0;
    const int gate_rows = gate_passes(a.gate.bits, a.gate.cpl) * gate_rpw;
    a.gu_tpe = (a.I + gate_rows - 1) / gate_rows;
    const int down_rows = down_passes(a.down.bits) * (kWave >> a.down.lpr_log2);
    a.dn_tpe = (H + down_rows - 1) / down_rows;
    a.local = g_fused_dev[dev].local.load(std::memory_order_acquire);
    *fa = a;
    *nb = blocks;
    return kern;
}

int fused_decode(const swq_moe_layer *layer, const void *x, int x_dtype, int batch, void *out, int out_dtype,
                 int32_t *topk_ids, float *topk_weights, void *ws, const FusedLayout &fl, bool accumulate,
                 hipStream_t stream, bool *taken, const FusedPrenorm *pn) {
    *taken = false;
    FusedArgs a;
    int nb = 0;
    FusedKernel k = fused_plan(layer, x_dtype, batch, fl.max_batch, pn != nullptr, &a, &nb);
    if (!k) return SWQ_OK;
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

// Once per device: the CU count and whether a grid of one workgroup per CU
// places every group's workgroups on one XCD (a launch of that grid reports
// each workgroup's XCC_ID).  Blocking; runs on `stream`.  Thread-safe: the
// first caller for a device runs the probe under a mutex, later ones wait
// for it.  Until a probe has succeeded the device keeps the three-launch
// path, and a failed probe (or a call on a stream under capture, which
// cannot block: SWQ_ERR_INVALID_ARGUMENT) leaves it to the next call.  The
// probe writes one word per workgroup into `given` when the caller passes
// device memory of kFusedMaxBlocks words, else into a buffer it allocates.
int fused_probe_device(hipStream_t stream, void *given) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return SWQ_ERR_HIP;
    FusedDevice &d = g_fused_dev[dev];
    if (d.cus.load(std::memory_order_acquire) > 0) return SWQ_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return SWQ_ERR_HIP;
    if (cs != hipStreamCaptureStatusNone) return SWQ_ERR_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(d.probe_mu);
    if (d.cus.load(std::memory_order_acquire) > 0) return SWQ_OK;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return SWQ_ERR_HIP;
    const int n = min(cus, kFusedMaxBlocks) / kGroups * kGroups;  // the fused grid
    int ok = 0;
    if (n >= kGroups) {
        int32_t *buf = static_cast<int32_t *>(given);
        if (!buf && hipMalloc(&buf, n * sizeof(int32_t)) != hipSuccess) return SWQ_ERR_HIP;
        hipLaunchKernelGGL(xcd_probe_kernel, dim3(n), dim3(kFusedThreads), 0, stream, buf);
        int32_t h[kFusedMaxBlocks];
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(h, buf, n * sizeof(int32_t), hipMemcpyDeviceToHost, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (!given) hipFree(buf);
        if (e != hipSuccess) return SWQ_ERR_HIP;
        ok = 1;
        for (int i = kGroups; i < n; ++i) ok &= h[i] == h[i % kGroups];
    }
    d.local.store(ok, std::memory_order_release);
    d.cus.store(cus, std::memory_order_release);
    return SWQ_OK;
}

}  // namespace swq
