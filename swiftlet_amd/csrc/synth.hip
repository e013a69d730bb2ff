// Benchmark support: device generator of the seeded synthetic weights and a
// bounded stream stall.
#include "../../include/swq_bench.h"
#include "internal.hpp"

namespace swq {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__host__ __device__ __forceinline__ uint64_t sm_fin(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return sm_fin(seed * kGamma + stream * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull);
}

__global__ void synth_u32_kernel(uint32_t *dst, int64_t count, uint64_t key, int64_t start) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint64_t z = key + static_cast<uint64_t>(start + i + 1) * kGamma;
    dst[i] = static_cast<uint32_t>(sm_fin(z) >> 32);
}

__global__ void synth_scales_kernel(uint16_t *s, uint16_t *b, int64_t count, uint64_t key, int64_t start,
                                    uint32_t lo, uint32_t cnt, float step, uint32_t bias_exp) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint64_t z = key + static_cast<uint64_t>(start + i + 1) * kGamma;
    const uint32_t r = static_cast<uint32_t>(sm_fin(z) >> 32);
    const float v = static_cast<float>(lo + r % cnt) * step;  // exact: < 2^12 times a power of two
    const _Float16 h = static_cast<_Float16>(v);              // round to nearest even
    uint16_t hb;
    __builtin_memcpy(&hb, &h, 2);
    s[i] = hb;
    b[i] = static_cast<uint16_t>((hb + (bias_exp << 10)) | 0x8000u);
}

__global__ void stall_kernel(int iterations) {
    for (int i = 0; i < iterations; ++i) __builtin_amdgcn_s_sleep(127);
}

}  // namespace swq

using namespace swq;

extern "C" int swq_bench_stall(int iterations, void *stream) {
    if (iterations < 0 || iterations > 1000000) return SWQ_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(stall_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), iterations);
    return launch_status();
}

extern "C" int swq_synth_u32(uint32_t *dst, int64_t count, uint64_t seed, uint64_t stream, int64_t start,
                             void *hip_stream) {
    if (!dst || count <= 0 || start < 0) return SWQ_ERR_INVALID_ARGUMENT;
    const int tb = 256;
    const int64_t blocks = (count + tb - 1) / tb;
    if (blocks > 0x7FFFFFFF) return SWQ_ERR_LIMIT;
    hipLaunchKernelGGL(synth_u32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(tb), 0,
                       static_cast<hipStream_t>(hip_stream), dst, count, stream_key(seed, stream), start);
    return launch_status();
}

extern "C" int swq_synth_scales(uint16_t *scales, uint16_t *biases, int64_t count, int bits, uint64_t seed,
                                uint64_t stream, int64_t start, void *hip_stream) {
    if (!scales || !biases || count <= 0 || start < 0) return SWQ_ERR_INVALID_ARGUMENT;
    uint32_t lo, cnt, ex, bias_exp;
    if (bits == 4) {
        lo = 655; cnt = 1966; ex = 17; bias_exp = 3;
    } else if (bits == 8) {
        lo = 629; cnt = 1888; ex = 21; bias_exp = 7;
    } else {
        return SWQ_ERR_UNSUPPORTED_BITS;
    }
    const float step = __builtin_ldexpf(1.0f, -static_cast<int>(ex));
    const int tb = 256;
    const int64_t blocks = (count + tb - 1) / tb;
    if (blocks > 0x7FFFFFFF) return SWQ_ERR_LIMIT;
    hipLaunchKernelGGL(synth_scales_kernel, dim3(static_cast<unsigned>(blocks)), dim3(tb), 0,
                       static_cast<hipStream_t>(hip_stream), scales, biases, count, stream_key(seed, stream),
                       start, lo, cnt, step, bias_exp);
    return launch_status();
}
