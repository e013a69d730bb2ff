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
constexpr int kNormChunks = 4;  // float4 chunks per thread held in registers: rows up to 4096

__device__ __forceinline__ float block_sum(float v, float *s_part) {
    v = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) s_part[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kNormThreads / kWave; ++i) t += s_part[i];
    return t;
}

__device__ __forceinline__ float norm_weight(const void *w, int wdt, int i) {
    return wdt == SWQ_F32 ? static_cast<const float *>(w)[i] : load_scale(static_cast<const uint8_t *>(w), i, wdt);
}

__device__ __forceinline__ void norm_store(void *out, int odt, int64_t i, float x) {
    if (odt == SWQ_BF16) static_cast<uint16_t *>(out)[i] = f32_to_bf16_rne(x);
    else static_cast<float *>(out)[i] = x;
}

// Row r: h += residual (when given, stored back), then
// out = h * (scale * w) with scale = 1 / sqrt(mean(h^2) + eps): the product
// order of QwenCPUModel.rmsNorm (x[i] *= scale * w[i]).  Every load of the
// row is issued before the first store (the row lives in registers), so the
// row costs one memory round trip.  dim % 4 == 0, dim <= 4096, 16 B aligned.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_vec_kernel(float *__restrict__ h,
                                                                   const float *__restrict__ residual,
                                                                   const void *__restrict__ w, int wdt, float eps,
                                                                   int dim, void *__restrict__ out, int odt) {
    __shared__ float s_part[kNormThreads / kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * dim;
    const int nc = dim / 4;
    float4 v[kNormChunks];
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k) {
        const int c = min(static_cast<int>(threadIdx.x) + k * kNormThreads, nc - 1);
        v[k] = reinterpret_cast<const float4 *>(h + base)[c];
        if (residual) {
            const float4 r = reinterpret_cast<const float4 *>(residual + base)[c];
            v[k].x += r.x;
            v[k].y += r.y;
            v[k].z += r.z;
            v[k].w += r.w;
        }
    }
    float wv[kNormChunks][4];  // the weights too, before the reduction's barrier
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k) {
        const int c = min(static_cast<int>(threadIdx.x) + k * kNormThreads, nc - 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) wv[k][q] = w ? norm_weight(w, wdt, 4 * c + q) : 1.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k) {
        if (static_cast<int>(threadIdx.x) + k * kNormThreads < nc) {
            ss += v[k].x * v[k].x;
            ss += v[k].y * v[k].y;
            ss += v[k].z * v[k].z;
            ss += v[k].w * v[k].w;
        }
    }
    const float scale = 1.f / __builtin_sqrtf(block_sum(ss, s_part) / static_cast<float>(dim) + eps);
#pragma unroll
    for (int k = 0; k < kNormChunks; ++k) {
        const int c = static_cast<int>(threadIdx.x) + k * kNormThreads;
        if (c >= nc) break;
        if (residual) reinterpret_cast<float4 *>(h + base)[c] = v[k];
        const float e[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            norm_store(out, odt, base + 4 * c + q, e[q] * (w ? scale * wv[k][q] : scale));
        }
    }
}

// Any dim: the same arithmetic in two passes over the row.
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
        ss += v * v;
    }
    const float scale = 1.f / __builtin_sqrtf(block_sum(ss, s_part) / static_cast<float>(dim) + eps);
    for (int i = threadIdx.x; i < dim; i += kNormThreads) {
        const float sw = w ? scale * norm_weight(w, wdt, i) : scale;
        norm_store(out, odt, base + i, hr[i] * sw);
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
    const bool vec = dim % 4 == 0 && dim <= 4 * kNormThreads * kNormChunks &&
                     reinterpret_cast<uintptr_t>(h) % 16 == 0 && reinterpret_cast<uintptr_t>(residual) % 16 == 0;
    if (vec)
        hipLaunchKernelGGL(rmsnorm_vec_kernel, dim3(rows), dim3(kNormThreads), 0, static_cast<hipStream_t>(stream), h,
                           residual, weight, weight_dtype, eps, dim, out, out_dtype);
    else
        hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, static_cast<hipStream_t>(stream), h,
                           residual, weight, weight_dtype, eps, dim, out, out_dtype);
    return launch_status();
}
