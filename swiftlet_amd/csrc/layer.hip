// The layer tail around the MoE block: the attention branch's residual add
// and the post-attention RMSNorm that makes the MoE input.  The MoE step's
// own residual add is SWQ_MOE_ACCUMULATE of swq_moe_decode / swq_moe_prefill.
//
// Reference: QwenCPUModel.layerForward (QwenCPUModel.swift:259-281) with
// rmsNorm (:47-59); on the GPU path add_inplace + norm_copy
// (Kernels.metal.txt:425-452) as QwenMetalModel.swift:938-951 encodes them.
#include "internal.hpp"
#include "tile.hpp"

namespace swq {
namespace {

constexpr int kNormThreads = 256;

// Row r: h += residual (when given, stored back), then
// out = h * (scale * w) with scale = 1 / sqrt(mean(h^2) + eps): the product
// order of QwenCPUModel.rmsNorm (x[i] *= scale * w[i]).
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(float *h, const float *residual, const void *w,
                                                               int wdt, float eps, int dim, void *out, int odt) {
    __shared__ float s_part[kNormThreads / kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * dim;
    float *hr = h + base;
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += kNormThreads) {
        float v = hr[i];
        if (residual) {
            v += residual[base + i];
            hr[i] = v;
        }
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & (kWave - 1)) == 0) s_part[threadIdx.x / kWave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kNormThreads / kWave; ++i) tot += s_part[i];
    const float scale = 1.f / __builtin_sqrtf(tot / static_cast<float>(dim) + eps);
    for (int i = threadIdx.x; i < dim; i += kNormThreads) {
        float sw = scale;
        if (w) sw = scale * (wdt == SWQ_F32 ? static_cast<const float *>(w)[i]
                                            : load_scale(static_cast<const uint8_t *>(w), i, wdt));
        const float x = hr[i] * sw;
        if (odt == SWQ_BF16) static_cast<uint16_t *>(out)[base + i] = f32_to_bf16_rne(x);
        else static_cast<float *>(out)[base + i] = x;
    }
}

}  // namespace
}  // namespace swq

using namespace swq;

extern "C" int swq_rmsnorm(float *h, const float *residual, const void *weight, int weight_dtype, float eps,
                           int rows, int dim, void *out, int out_dtype, void *stream) {
    if (!h || !out || rows <= 0 || dim <= 0) return SWQ_ERR_INVALID_ARGUMENT;
    if (!(eps >= 0.f)) return SWQ_ERR_INVALID_ARGUMENT;
    if (weight && weight_dtype != SWQ_F32 && weight_dtype != SWQ_F16 && weight_dtype != SWQ_BF16)
        return SWQ_ERR_UNSUPPORTED_DTYPE;
    if (out_dtype != SWQ_F32 && out_dtype != SWQ_BF16) return SWQ_ERR_UNSUPPORTED_DTYPE;
    if (reinterpret_cast<uintptr_t>(h) % 4 != 0 || reinterpret_cast<uintptr_t>(residual) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(out) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(weight) % (weight_dtype == SWQ_F32 ? 4 : 2) != 0)
        return SWQ_ERR_MISALIGNED;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, static_cast<hipStream_t>(stream), h,
                       residual, weight, weight_dtype, eps, dim, out, out_dtype);
    return launch_status();
}
