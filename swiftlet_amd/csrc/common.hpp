// Device-side building blocks shared by the gfx950 kernels: MLX affine
// weight views, scale decoding, 16-byte code-chunk dot products and
// wave64 reductions.
//
// Format (Checkpoint.swift:168-209, Kernels.metal.txt:4-7): a weight row of
// `in` inputs is in*bits/32 uint32 words, codes LSB-first; one scale and one
// bias per `group` consecutive inputs; w = scale*q + bias.
//
// The vectorised kernels read a row as 16-byte "chunks": 32 codes at 4 bits,
// 16 codes at 8 bits.  A chunk never straddles a group when the group spans
// a whole number of chunks (group*bits % 128 == 0), which the host checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace swq {

constexpr int kWave = 64;

// Device view of one quantized matrix (one expert's slice is selected by
// adding e*stride_w / e*stride_sb).
struct QMat {
    const uint8_t *w;      // first row of the matrix (expert 0 if stacked)
    const uint8_t *s;      // scales of row 0
    const uint8_t *b;      // biases of row 0
    int64_t stride_w;      // bytes between experts' codes
    int64_t stride_sb;     // bytes between experts' scales/biases
    int32_t rows;          // rows of one matrix
    int32_t in;            // logical input dim
    int32_t group;         // group size
    int32_t bits;          // 4 or 8 on the vectorised path
    int32_t stype;         // 0 f32, 1 f16, 2 bf16
    int32_t row_bytes;     // in*bits/8
    int32_t gpr;           // groups per row
    int32_t chunks;        // 16-byte chunks per row
    int32_t chunks_per_group;
    int32_t lpr_log2;      // log2(lanes per row) of the vectorised path
    int32_t cpl;           // 16-byte chunks per lane
    int32_t cpg_log2;      // log2(chunks per group)
    int32_t xf;            // activation format: 0 fp32 fma, 1 packed bf16 dot2
    int32_t pad_;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t u) {
    return __uint_as_float(static_cast<uint32_t>(u) << 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t u) {
    _Float16 h;
    __builtin_memcpy(&h, &u, 2);
    return static_cast<float>(h);
}

// One scale or bias (element `idx` of a per-group tensor).  The fused paths
// require natural alignment (4 B for f32, 2 B for 16-bit types).
__device__ __forceinline__ float load_scale(const uint8_t *base, int64_t idx, int stype) {
    if (stype == 1) return f16_to_f32(*reinterpret_cast<const uint16_t *>(base + idx * 2));
    if (stype == 2) return bf16_to_f32(*reinterpret_cast<const uint16_t *>(base + idx * 2));
    return *reinterpret_cast<const float *>(base + idx * 4);
}

// Byte-addressed variants for arbitrary (2-byte aligned) offsets, the
// situation Kernels.metal.txt:9-12 describes for whole-shard mmaps.
__device__ __forceinline__ uint32_t load_u32_bytes(const uint8_t *p) {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) |
           (static_cast<uint32_t>(p[2]) << 16) | (static_cast<uint32_t>(p[3]) << 24);
}

__device__ __forceinline__ float load_scale_bytes(const uint8_t *base, int64_t idx, int stype) {
    if (stype == 0) return __uint_as_float(load_u32_bytes(base + idx * 4));
    const uint8_t *p = base + idx * 2;
    uint16_t u = static_cast<uint16_t>(p[0] | (p[1] << 8));
    return stype == 1 ? f16_to_f32(u) : bf16_to_f32(u);
}

__device__ __forceinline__ float ubyte(uint32_t v, int n) {
    return static_cast<float>((v >> (8 * n)) & 0xFFu);  // v_cvt_f32_ubyteN
}

// sum_i q_i * x_i over one 16-byte chunk of 4-bit codes; x holds the 32
// matching inputs.  Nibble j of word k is input 8k + j.  Four independent
// accumulator chains (one per word), summed pairwise at the end.
__device__ __forceinline__ float dot_chunk_q4(const uint4 w, const float *x) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float acc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t lo = ws[k] & 0x0F0F0F0Fu;         // nibbles 0,2,4,6
        const uint32_t hi = (ws[k] >> 4) & 0x0F0F0F0Fu;  // nibbles 1,3,5,7
        const float *xx = x + 8 * k;
        float a = ubyte(lo, 0) * xx[0];
        a = fmaf(ubyte(hi, 0), xx[1], a);
        a = fmaf(ubyte(lo, 1), xx[2], a);
        a = fmaf(ubyte(hi, 1), xx[3], a);
        a = fmaf(ubyte(lo, 2), xx[4], a);
        a = fmaf(ubyte(hi, 2), xx[5], a);
        a = fmaf(ubyte(lo, 3), xx[6], a);
        a = fmaf(ubyte(hi, 3), xx[7], a);
        acc[k] = a;
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// Same for 8-bit codes: 16 inputs per chunk, byte j of word k is input 4k+j.
__device__ __forceinline__ float dot_chunk_q8(const uint4 w, const float *x) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float acc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float *xx = x + 4 * k;
        float a = ubyte(ws[k], 0) * xx[0];
        a = fmaf(ubyte(ws[k], 1), xx[1], a);
        a = fmaf(ubyte(ws[k], 2), xx[2], a);
        a = fmaf(ubyte(ws[k], 3), xx[3], a);
        acc[k] = a;
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

template <int BITS>
__device__ __forceinline__ float dot_chunk(const uint4 w, const float *x) {
    if constexpr (BITS == 4) return dot_chunk_q4(w, x);
    else return dot_chunk_q8(w, x);
}

template <int BITS>
constexpr int codes_per_chunk() { return 128 / BITS; }

// Sum over `width` consecutive lanes (width a power of two <= 64); every
// lane of the segment receives the segment's sum.
__device__ __forceinline__ float segment_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return segment_sum(v, kWave); }

// Workgroup barrier for LDS traffic only: each wave's LDS operations
// complete, then s_barrier.  Global loads stay in flight across it (a full
// __syncthreads would wait for them too).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// Load N activations starting at element `e0` into fp32 registers.  x is
// fp32 (XDT 0) or bf16 (XDT 2); N is a multiple of 8.
template <int XDT, int N>
__device__ __forceinline__ void load_x(float (&dst)[N], const void *x, int64_t e0) {
    if constexpr (XDT == 2) {
        const uint16_t *p = static_cast<const uint16_t *>(x) + e0;
#pragma unroll
        for (int i = 0; i < N; i += 8) {
            const uint4 v = *reinterpret_cast<const uint4 *>(p + i);
            const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                dst[i + 2 * k] = __uint_as_float(u[k] << 16);
                dst[i + 2 * k + 1] = __uint_as_float(u[k] & 0xFFFF0000u);
            }
        }
    } else {
        const float *p = static_cast<const float *>(x) + e0;
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(p + i);
            dst[i] = v.x;
            dst[i + 1] = v.y;
            dst[i + 2] = v.z;
            dst[i + 3] = v.w;
        }
    }
}

__device__ __forceinline__ float sigmoidf_ref(float v) { return 1.0f / (1.0f + __expf(-v)); }

// silu(g) * u with the reference's form g * (1 / (1 + exp(-g)))
// (QwenCPUModel.swift:61-62).
__device__ __forceinline__ float swiglu(float g, float u) { return g * sigmoidf_ref(g) * u; }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

}  // namespace swq
