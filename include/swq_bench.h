/*
 * swq_bench.h — benchmark and test support for libswq.so.
 *
 * Not part of the drop-in boundary (include/swq.h); the reference has no
 * counterpart.  These entry points generate the seeded synthetic weights on
 * the device, run chosen stages of the decode step for per-kernel timing,
 * and stall a stream for a bounded time so that a timed region's launches
 * queue up behind it.
 *
 * Synthetic streams: element i of stream `stream` is the high 32 bits of
 * splitmix64 output i+1 for the key
 *     key = mix(seed * 0x9E3779B97F4A7C15 + stream * 0xD1B54A32D192ED03
 *               + 0x632BE59BD9B4E019),
 * with mix the splitmix64 output function; swiftlet_amd/synth.py computes
 * the same values on the host, bit for bit.
 */
#ifndef SWQ_BENCH_H
#define SWQ_BENCH_H

#include <stddef.h>
#include <stdint.h>

#include "swq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* dst[i] = element (start + i) of the stream, i < count (device memory). */
int swq_synth_u32(uint32_t *dst, int64_t count, uint64_t seed, uint64_t stream, int64_t start,
                  void *hip_stream);

/* fp16 scales and biases from elements (start + i) of the stream:
 *   bits 4: scale = fp16(m * 2^-17), m = 655 + r % 1966, bias = -8 * scale
 *   bits 8: scale = fp16(m * 2^-21), m = 629 + r % 1888, bias = -128 * scale */
int swq_synth_scales(uint16_t *scales, uint16_t *biases, int64_t count, int bits, uint64_t seed,
                     uint64_t stream, int64_t start, void *hip_stream);

/* swq_moe_decode on a chosen path.  stage_mask bits 0-2 run stages of the
 * three-launch path (bit 0: router + shared gate/up + shared-expert gate,
 * bit 1: top-k + routed gate/up, bit 2: down + combine); a stage reads what
 * the earlier stages left in the workspace.  SWQ_STAGES_FUSED runs the
 * single-launch path, or returns SWQ_ERR_LIMIT when the layer, the batch or
 * the device cannot take it. */
enum { SWQ_STAGES_FUSED = 8 };

int swq_moe_decode_stages(const swq_moe_layer *layer, const void *x, int x_dtype, int batch, void *out,
                          int out_dtype, int32_t *topk_ids, float *topk_weights, void *ws, size_t ws_bytes,
                          int flags, int stage_mask, void *stream);

/* Byte offset in the workspace of a 32-bit word that the single-launch path
 * sets nonzero if one of its bounded waits ran out (0 on bad input). */
size_t swq_moe_workspace_error_offset(const swq_moe_layer *layer, int batch);

/* swq_moe_prefill with logit_bias[e] (device, [num_experts] f32) added to
 * every token's router logit of expert e before the softmax: the synthetic
 * skewed-load workload, whose per-expert token counts follow a chosen
 * distribution.  The reference has no such bias; with all entries 0 the
 * result equals swq_moe_prefill's. */
int swq_moe_prefill_biased(const swq_moe_layer *layer, const void *x, int x_dtype, int tokens, void *out,
                           int out_dtype, int32_t *topk_ids, float *topk_weights, const float *logit_bias,
                           void *ws, size_t ws_bytes, int flags, void *stream);

/* swq_moe_prefill_biased (logit_bias may be NULL: none) running only the
 * launches whose bits are set in stage_mask: 2 router GEMM (with the
 * activation planes and group sums of x gate/up reads), 4 routing and
 * grouping, 8 gate/up + SwiGLU, 16 down, 32 combine (bit 1, which named a
 * separate activation prep, launches nothing).  A
 * launch reads what the earlier ones left in the workspace (a full call on
 * the same inputs leaves everything each one needs). */
enum { SWQ_PREFILL_ALL = 63 };

int swq_moe_prefill_stages(const swq_moe_layer *layer, const void *x, int x_dtype, int tokens, void *out,
                           int out_dtype, int32_t *topk_ids, float *topk_weights, const float *logit_bias,
                           void *ws, size_t ws_bytes, int flags, int stage_mask, void *stream);

/* One single-wave kernel that sleeps `iterations` times (s_sleep 127, about
 * 8k cycles each) and exits; iterations <= 1000000. */
int swq_bench_stall(int iterations, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SWQ_BENCH_H */
