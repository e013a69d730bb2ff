/*
 * swq.h — C ABI of the MI355X (gfx950) MoE decode hot path.
 *
 * This is the drop-in boundary for SwiftletCore's quantized-matmul and MoE
 * layer operator API.  Swift (or any FFI) binds these symbols through a
 * module.modulemap; Python binds them with ctypes.  Every signature uses
 * plain pointers and sizes only.
 *
 * Conventions
 *   - Every entry point returns SWQ_OK (0) or a negative SWQ_ERR_* code;
 *     no C++ exception and no HIP error escapes.  swq_strerror() names it.
 *   - "device pointer" = memory from hipMalloc (or any HBM allocation) on the
 *     current HIP device.  Weights are never copied: a swq_qlinear is a
 *     non-owning view, like GPULinear (MetalShardStore.swift:48-62).
 *   - `stream` is a hipStream_t passed as void*; NULL means the null stream.
 *     Stream-ordered entry points return after enqueueing.
 *   - The hot entry points (swq_encode_gemv, swq_moe_decode,
 *     swq_moe_prefill) allocate nothing; scratch comes from a caller-owned
 *     workspace sized by the matching *_workspace_bytes query.
 *   - A workspace belongs to one stream at a time: two calls that overlap in
 *     time must use different workspaces.
 *   - MLX affine format (Checkpoint.swift:168-209): a weight row is
 *     in_dim*bits/32 uint32 words, codes packed LSB-first; one scale and one
 *     bias per group_size consecutive inputs; w = scale*q + bias.
 */
#ifndef SWQ_H
#define SWQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
enum {
    SWQ_OK = 0,
    SWQ_ERR_INVALID_ARGUMENT = -1,  /* null pointer, non-positive size        */
    SWQ_ERR_BAD_SHAPE = -2,         /* in_dim % group_size, group % per-word  */
    SWQ_ERR_UNSUPPORTED_BITS = -3,  /* Checkpoint.Error.unsupportedBits       */
    SWQ_ERR_UNSUPPORTED_DTYPE = -4, /* scale / activation dtype not 0,1,2     */
    SWQ_ERR_MISALIGNED = -5,        /* fused path needs 16 B rows, 2/4 B s/b  */
    SWQ_ERR_WORKSPACE = -6,         /* workspace null or smaller than query   */
    SWQ_ERR_EXPERT_RANGE = -7,      /* top_k outside [1, num_experts]         */
    SWQ_ERR_HIP = -8,               /* a HIP runtime call failed              */
    SWQ_ERR_NO_DEVICE = -9,         /* MetalEngine.Error.noDevice             */
    SWQ_ERR_LIMIT = -10,            /* batch / top_k above compiled maximum   */
    SWQ_ERR_MISSING_TENSOR = -11,   /* Checkpoint.Error.missingTensor         */
    SWQ_ERR_IO = -12,               /* a file could not be opened or read     */
    SWQ_ERR_FORMAT = -13,           /* malformed safetensors / JSON / qpack   */
    SWQ_ERR_STALLED = -14           /* a single-launch MoE call ran out of a
                                       bounded wait (see swq_moe_workspace_status) */
};

/* Scale, bias and activation dtypes.  The values equal
 * MetalEngine.ScalesType (MetalEngine.swift:69-80): 0 f32, 1 f16, 2 bf16. */
enum { SWQ_F32 = 0, SWQ_F16 = 1, SWQ_BF16 = 2 };

/* Compiled limits of the fused MoE kernels. */
enum { SWQ_MAX_BATCH = 16, SWQ_MAX_TOPK = 16 };

/* swq_moe_decode / swq_moe_prefill flags. */
enum {
    /* out += moe(x) instead of out = moe(x): the residual add that
     * weighted_accum fuses (Kernels.metal.txt:463-478).  Needs out_dtype f32. */
    SWQ_MOE_ACCUMULATE = 1
};

/* One quantized linear module, optionally a stack of experts.
 * Replaces GPULinear (MetalShardStore.swift:48-62) plus ExpertStack's
 * per-expert strides (QwenMetalModel.swift:16-21). */
typedef struct swq_qlinear {
    const void *w;           /* packed uint32 codes (device)                  */
    const void *scales;      /* one per group (device)                        */
    const void *biases;      /* one per group (device)                        */
    int64_t w_off;           /* byte offsets added to w / scales / biases     */
    int64_t s_off;
    int64_t b_off;
    int32_t out_dim;         /* rows of one matrix (of one expert if stacked) */
    int32_t in_dim;          /* logical input dimension                       */
    int32_t group_size;
    int32_t bits;            /* 2, 4 or 8                                     */
    int32_t scales_type;     /* SWQ_F32 / SWQ_F16 / SWQ_BF16                  */
    int32_t reserved;        /* must be 0                                     */
    int64_t expert_stride_w;  /* bytes between experts' codes (0: unstacked)  */
    int64_t expert_stride_sb; /* bytes between experts' scales and biases     */
} swq_qlinear;

/* One routed-expert SwiGLU MoE layer with a sigmoid-gated shared expert.
 * Replaces MoEGPU (QwenMetalModel.swift:34-39) + the config fields that
 * moeForward reads (QwenCPUModel.swift:500-504). */
typedef struct swq_moe_layer {
    swq_qlinear router;            /* mlp.gate            [E, H]              */
    swq_qlinear gate;              /* switch_mlp.gate_proj [E][I, H] stacked  */
    swq_qlinear up;                /* switch_mlp.up_proj   [E][I, H] stacked  */
    swq_qlinear down;              /* switch_mlp.down_proj [E][H, I] stacked  */
    swq_qlinear shared_gate;       /* shared_expert.gate_proj [Is, H]         */
    swq_qlinear shared_up;         /* shared_expert.up_proj   [Is, H]         */
    swq_qlinear shared_down;       /* shared_expert.down_proj [H, Is]         */
    swq_qlinear shared_expert_gate;/* mlp.shared_expert_gate [1, H]           */
    int32_t hidden;                /* H                                        */
    int32_t num_experts;           /* E                                        */
    int32_t top_k;                 /* K                                        */
    int32_t moe_intermediate;      /* I                                        */
    int32_t shared_intermediate;   /* Is                                       */
    int32_t norm_topk_prob;        /* 1: w_k = p_k / sum_topk p (:546-550)     */
    int32_t has_shared;            /* 0: no shared expert / shared gate        */
    int32_t reserved;              /* must be 0                                */
} swq_moe_layer;

/* ---- library ----------------------------------------------------------- */

/* Human-readable name of a status code (never NULL). */
const char *swq_strerror(int status);

/* ABI version: major*10000 + minor*100 + patch. */
int swq_version(void);

/* Number of visible HIP devices; SWQ_ERR_NO_DEVICE if none.
 * Mirrors the MetalEngine() constructor's device check (MetalEngine.swift:22-27). */
int swq_device_count(int *count);

/* ---- quantized GEMV ---------------------------------------------------- */

/* Blocking, host-memory GEMV: y = W x.  Copies every input to the device and
 * y back, as MetalEngine.gemvQuantized does (MetalEngine.swift:190-232).
 * use_fast selects the vectorised kernel (bits 4/8) instead of the scalar
 * one; both compute the same sum.  Allocates; not for the hot loop. */
int swq_gemv_quantized(const float *x,
                       const void *packed, size_t packed_bytes,
                       const void *scales, size_t scales_bytes,
                       const void *biases, size_t biases_bytes,
                       int out_dim, int in_dim, int group_size, int bits,
                       int scales_type, int use_fast, float *y);

/* Stream-ordered GEMV over a device-resident linear: y[y_off + r] =
 * sum_i W[r, i] x[x_off + i] for r < rows (rows <= 0: lin->out_dim).
 * w_extra / s_extra / b_extra advance into a stacked tensor in bytes.
 * Replaces MetalEngine.encodeGemv (MetalEngine.swift:95-170): picks the
 * vectorised kernel when rows are 16 B aligned, else the scalar one. */
int swq_encode_gemv(const swq_qlinear *lin, int rows,
                    int64_t w_extra, int64_t s_extra, int64_t b_extra,
                    const float *x, int64_t x_off, float *y, int64_t y_off,
                    void *stream);

/* y_i = W_i x for n <= 4 linears that share x and one format (in_dim, bits,
 * group_size, scales_type), in one launch; ys: host array of n device
 * pointers.  With norm_weight != NULL the input is first replaced by
 * rmsnorm(x) * norm_weight (norm_dtype SWQ_F32 / SWQ_F16 / SWQ_BF16, eps)
 * inside the kernel — the input RMSNorm of a decoder layer fused into its
 * projections.  x and norm_weight 16 B aligned.  Formats the vectorised
 * GEMV does not take, or in_dim above 4096: SWQ_ERR_LIMIT (call
 * swq_encode_gemv per matrix instead).
 * Replaces encNormCopy + the projections' encodeGemv calls of one layer
 * (QwenMetalModel.swift:997-1006, :924-931). */
int swq_encode_gemv_multi(const swq_qlinear *lins, int n, float *const *ys, const float *x,
                          const void *norm_weight, int norm_dtype, float norm_eps, void *stream);

/* buf[dst_off + i] = silu(buf[g_off + i]) * buf[u_off + i], i < count.
 * Replaces MetalEngine.encodeSiluMul (MetalEngine.swift:172-187). */
int swq_encode_silu_mul(float *buf, int count, int64_t g_off, int64_t u_off,
                        int64_t dst_off, void *stream);

/* Materialise rows [row0, row0+rows) of the flattened [.., out, in] weight
 * as fp32: out[r*in + i] = scale*q + bias (multiply, then add; no FMA).
 * Replaces Checkpoint.moduleWeightSlice / dequantized (Checkpoint.swift:148-209).
 * Stacked linears: row r of expert e is flattened row e*out_dim + r. */
int swq_dequantize(const swq_qlinear *lin, int64_t row0, int64_t rows,
                   float *out, void *stream);

/* ---- layer tail --------------------------------------------------------- */

/* For each of `rows` rows of `dim` floats: h += residual (when residual is
 * not NULL; h is updated in place), then
 *     out = h * (scale * weight),  scale = 1 / sqrt(mean(h^2) + eps)
 * (weight NULL: h * scale).  weight: [dim] of weight_dtype (SWQ_F32 / SWQ_F16
 * / SWQ_BF16); out: [rows, dim] of out_dtype (SWQ_F32 / SWQ_BF16; bf16 is
 * rounded to nearest even).  This is the MoE input of a decoder layer; the MoE
 * step's own residual add is SWQ_MOE_ACCUMULATE into h.
 * Replaces add_inplace + norm_copy (Kernels.metal.txt:425-452) as
 * QwenMetalModel.swift:938-951 encodes them around the MoE block, with the
 * numerics of QwenCPUModel.rmsNorm (QwenCPUModel.swift:47-59, :276-277). */
int swq_rmsnorm(float *h, const float *residual, const void *weight, int weight_dtype, float eps,
                int rows, int dim, void *out, int out_dtype, void *stream);

/* ---- next-token sampling ------------------------------------------------ */

/* GenerationOptions (SwiftletSession.swift:19-41). */
typedef struct {
    float temperature;        /* <= 0: greedy (the first maximum) */
    int32_t top_k;            /* candidates when sampling, 1..64 */
    float top_p;              /* nucleus cut; >= 1: none */
    float presence_penalty;   /* >= 0, subtracted once from every seen token */
    float frequency_penalty;  /* >= 0, times the token's count */
} swq_sample_options;

/* Workspace bytes of swq_sample for `vocab` logits (0: vocab above 524288).
 * The workspace must be zero-filled before its first call (it holds the
 * arrival counter of the call's workgroups); every call leaves it so.  Calls
 * that run at the same time need workspaces of their own. */
size_t swq_sample_workspace_bytes(int vocab);

/* One next token from `vocab` f32 logits (device), entirely on the device:
 * banned_ids (the suppressed ids, plus EOS while it is banned) become -inf,
 * each seen_ids[i] loses presence + frequency * seen_counts[i]; then the
 * first maximum (temperature <= 0), or the top_k candidates by logit (ties
 * to the lower id), p_i = exp((l_i - l_0) / temperature), the top-p cut and
 * the draw r = u * sum p, the first i with r - (p_0 + .. + p_i) <= 0.
 * u in [0, 1) is the caller's uniform number (the reference draws
 * Float.random).  out_token: one int32 on the device.  Id lists and counts
 * are device arrays.  Replaces SwiftletSession.sample
 * (SwiftletSession.swift:226-273). */
int swq_sample(const float *logits, int vocab, const swq_sample_options *options,
               const int32_t *seen_ids, const int32_t *seen_counts, int n_seen,
               const int32_t *banned_ids, int n_banned, float u, int32_t *out_token,
               void *ws, size_t ws_bytes, void *stream);

/* ---- gated DeltaNet decode step ---------------------------------------- */

/* Layouts of the DeltaNet input projections (QwenConfig.DeltaProjectionLayout). */
enum {
    /* qwen3_next: in_proj_qkvz per key head [q(dk) k(dk) v(rep*dv) z(rep*dv)],
     * in_proj_ba per key head [b(rep) a(rep)] (QwenCPUModel.swift:386-410). */
    SWQ_DELTA_INTERLEAVED = 0,
    /* qwen3_5: in_proj_qkv [q | k | v] followed by in_proj_z [z] in one
     * buffer; in_proj_b [b] followed by in_proj_a [a] (:411-415). */
    SWQ_DELTA_SPLIT = 1
};

/* One gated DeltaNet block (linear_attn) between its input projections and
 * out_proj.  The small parameters are f32 device arrays, as the reference
 * holds them (QwenMetalModel FastLayer convW/aLog/dtBias/deltaNormW). */
typedef struct swq_deltanet_layer {
    int32_t num_key_heads;       /* nk                                        */
    int32_t num_value_heads;     /* nv, a multiple of nk                      */
    int32_t key_head_dim;        /* dk: 8, 16, 32, 64, 128 or 256             */
    int32_t value_head_dim;      /* dv <= 1024                                */
    int32_t conv_kernel;         /* K <= 8 (linear_conv_kernel_dim)           */
    int32_t layout;              /* SWQ_DELTA_INTERLEAVED / SWQ_DELTA_SPLIT   */
    float norm_eps;              /* rms_norm_eps of the gated norm            */
    int32_t reserved;            /* must be 0                                 */
    const float *conv_weight;    /* conv1d.weight [2*nk*dk + nv*dv][K]        */
    const float *a_log;          /* A_log [nv]                                */
    const float *dt_bias;        /* dt_bias [nv]                              */
    const float *norm_weight;    /* norm.weight [dv]                          */
} swq_deltanet_layer;

/* Bytes of one sequence's DeltaNet state for this layer (0 on bad input): the
 * conv history as a ring of K rows [K][convD] f32, then (at the next 256-byte
 * boundary) the recurrent state [nv][dv][dk] f32.  All zeros is a fresh
 * session (the reference's resetGPUState / empty DecodeState). */
size_t swq_deltanet_state_bytes(const swq_deltanet_layer *layer);

/* One token: qkvz / ba are the input projections' outputs (f32, device) in
 * the layer's layout; position is the number of tokens already in `state`
 * (the row of position p lives in ring slot p % K).  out: [nv*dv] f32, the
 * gated-normed output, the input of out_proj.  Updates `state` in place.
 * Replaces encDeltaLayer's deinterleave_qkvz, conv_step, delta_pre,
 * rmsnorm_rows (q, k), gated_delta_step and gated_norm_mul
 * (QwenMetalModel.swift:989-1084; Kernels.metal.txt:126-214, :305-422,
 * :497-519) with the numerics of QwenCPUModel.deltaNetForward for one token
 * (QwenCPUModel.swift:417-493). */
int swq_deltanet_step(const swq_deltanet_layer *layer, const float *qkvz, const float *ba, void *state,
                      size_t state_bytes, int64_t position, float *out, void *stream);

/* ---- gated GQA attention decode step ------------------------------------ */

/* One full-attention block (self_attn) between q/k/v_proj and o_proj. */
typedef struct swq_attention_layer {
    int32_t num_heads;           /* H                                         */
    int32_t num_kv_heads;        /* KVH; H / KVH <= 16                        */
    int32_t head_dim;            /* hd: 16, 32, 64, 128 or 256                */
    int32_t rotary_dims;         /* even, <= hd (QwenConfig.rotaryDims)       */
    float rope_theta;
    float norm_eps;              /* rms_norm_eps of q_norm / k_norm           */
    int32_t max_positions;       /* rows of the KV cache                      */
    int32_t reserved;            /* must be 0                                 */
    const float *q_norm_weight;  /* q_norm.weight [hd] f32 (device)           */
    const float *k_norm_weight;  /* k_norm.weight [hd] f32 (device)           */
} swq_attention_layer;

/* Bytes of one sequence's KV cache: k then v (at a 256-byte boundary), each
 * f32 [max_positions][KVH][hd], rows in position order as the reference
 * appends them (DecodeState.kv).  0 on bad input. */
size_t swq_attention_cache_bytes(const swq_attention_layer *layer);

/* Workspace bytes of swq_attention_step (per-split partial results). */
size_t swq_attention_workspace_bytes(const swq_attention_layer *layer);

/* One token at `position` (= the cached positions): q_proj [H][2*hd] (per
 * head the query, then the output gate), k_proj / v_proj [KVH*hd], f32
 * device vectors.  q and k are RMS-normalised with their weights and rotated
 * (partial NeoX RoPE on the first rotary_dims, angle = position *
 * theta^(-2j/rotary_dims)); k and v are appended to the cache at `position`;
 * each head attends over positions 0..position of its kv head (head / (H/KVH))
 * with scale 1/sqrt(hd); out [H*hd] = attention * sigmoid(gate), the input of
 * o_proj.  position >= max_positions: SWQ_ERR_LIMIT.  Two launches; the
 * launch shape depends on `position` (a captured graph holds one position).
 * Replaces attnCoreCPU (QwenMetalModel.swift:1086-1134) with the numerics of
 * QwenCPUModel.attentionForward for one token (QwenCPUModel.swift:285-367). */
int swq_attention_step(const swq_attention_layer *layer, const float *q_proj, const float *k_proj,
                       const float *v_proj, void *cache, size_t cache_bytes, int64_t position, float *out,
                       void *ws, size_t ws_bytes, void *stream);

/* ---- checkpoint and .qpack loading ----------------------------------- */

enum { SWQ_MAX_DIMS = 8 };

/* A stored tensor: safetensors dtype name ("U32", "F16", "BF16", "F32", ...),
 * shape and byte size (SafetensorsFile.TensorInfo). */
typedef struct {
    char dtype[8];
    int32_t ndim;
    int64_t shape[SWQ_MAX_DIMS];
    int64_t nbytes;
} swq_tensor_info;

/* An mlx-lm checkpoint directory: model.safetensors, or the shards that
 * model.safetensors.index.json maps, and config.json's "quantization" block.
 * Replaces Checkpoint (Checkpoint.swift:28-72).  Not thread-safe. */
typedef struct swq_checkpoint swq_checkpoint;

int swq_checkpoint_open(const char *dir, swq_checkpoint **out);
void swq_checkpoint_close(swq_checkpoint *ckpt);

/* Checkpoint.tensorNames: count, and name i (valid until close). */
int swq_checkpoint_tensor_count(const swq_checkpoint *ckpt);
const char *swq_checkpoint_tensor_name(const swq_checkpoint *ckpt, int i);

/* Tensor info; "language_model."-prefixed names resolve as
 * Checkpoint.resolve (Checkpoint.swift:76-80).  SWQ_ERR_MISSING_TENSOR if absent. */
int swq_checkpoint_tensor(const swq_checkpoint *ckpt, const char *name, swq_tensor_info *info);

/* Checkpoint.quantSpec(for:) (Checkpoint.swift:111-120) of module `path`
 * (e.g. "model.layers.0.mlp.gate"): SWQ_ERR_MISSING_TENSOR when the module
 * is not stored quantized or no spec applies.  Of several matching
 * per-module overrides the longest key wins. */
int swq_checkpoint_quant(const swq_checkpoint *ckpt, const char *path, int *group_size, int *bits);

/* Raw stored bytes into host memory (Checkpoint.rawTensor, :86-90). */
int swq_checkpoint_read(const swq_checkpoint *ckpt, const char *name, void *dst, int64_t dst_bytes);

/* Raw stored bytes into device memory through pinned staging; returns when
 * the copy has completed.  For norms, embeddings and other plain tensors. */
int swq_checkpoint_load(swq_checkpoint *ckpt, const char *name, void *dst, int64_t dst_bytes, void *stream);

/* Device bytes swq_checkpoint_linear needs for module `path` (>= 0), or a
 * negative status. */
int64_t swq_checkpoint_linear_bytes(const swq_checkpoint *ckpt, const char *path);

/* A quantized module (path.weight/.scales/.biases) resident in one device
 * buffer (codes at 0, scales and biases at the next 256-byte boundaries;
 * dst 256-byte aligned) and its descriptor.  rows_per_expert > 0 describes a
 * stacked switch_mlp tensor as an expert stack with out_dim rows per expert
 * (ExpertStack strides, QwenMetalModel.swift:167-188).  Unquantized modules:
 * SWQ_ERR_UNSUPPORTED_BITS.  Replaces MetalShardStore.residentLinear
 * (MetalShardStore.swift:67-118); the file-backed gpuLinear (:120-158) has no
 * counterpart: weights always live in HBM. */
int swq_checkpoint_linear(swq_checkpoint *ckpt, const char *path, int rows_per_expert, void *dst,
                          int64_t dst_bytes, swq_qlinear *out, void *stream);

/* A .qpack container (Qpack.swift:3-17): packed_experts/layout.json,
 * manifest.json and packed_experts/layer_NN.bin, one fixed-stride blob per
 * expert.  Replaces QpackExpertReader (Qpack.swift:168-203).  Not thread-safe. */
typedef struct swq_qpack swq_qpack;

typedef struct {
    int32_t expert_count, layer_count;  /* Qpack.Layout (Qpack.swift:30-36)  */
    int64_t expert_stride;              /* bytes per blob, 16 KiB multiple    */
    int32_t quant_bits, quant_group_size; /* Qpack.Manifest; 0 if absent     */
    int32_t section_count;
} swq_qpack_layout_info;

int swq_qpack_open(const char *container_dir, swq_qpack **out);
void swq_qpack_close(swq_qpack *qp);
int swq_qpack_layout(const swq_qpack *qp, swq_qpack_layout_info *info);

/* Layout.linearLayers[layer]: 1 / 0, or a negative status. */
int swq_qpack_is_linear_layer(const swq_qpack *qp, int layer);

/* Section i (Qpack.Section, Qpack.swift:22-28): name (valid until close),
 * byte offset inside a blob, dtype and per-expert shape. */
int swq_qpack_section(const swq_qpack *qp, int index, const char **name, int64_t *offset,
                      swq_tensor_info *info);
/* QpackExpertReader.section(_:) (Qpack.swift:199-201): the section's index. */
int swq_qpack_find_section(const swq_qpack *qp, const char *name);

/* One blob into host memory, one pread of expert_stride bytes
 * (QpackExpertReader.readExpert, Qpack.swift:185-197). */
int swq_qpack_read_expert(swq_qpack *qp, int layer, int expert, void *dst, int64_t dst_bytes);

/* Blobs [first_expert, first_expert + count) of a layer into device memory,
 * byte for byte (count * expert_stride bytes); the whole layer is
 * first_expert 0, count expert_count.  Returns when the copy has completed.
 * Replaces ExpertCache's slot fill (ExpertCache.swift:66-69). */
int swq_qpack_load_experts(swq_qpack *qp, int layer, int first_expert, int count, void *dst,
                           int64_t dst_bytes, void *stream);

/* The expert stack of projection `proj` ("gate_proj", "up_proj", "down_proj")
 * inside blobs resident at `base` (blob 0 of the loaded range): offsets are
 * the sections', expert_stride_w = expert_stride_sb = expert_stride, bits and
 * group from the manifest.  Replaces ExpertProj (QwenMetalModel.swift:137-165). */
int swq_qpack_expert_linear(const swq_qpack *qp, const void *base, const char *proj, swq_qlinear *out);

/* ---- MoE layer decode ------------------------------------------------- */

/* Workspace bytes swq_moe_decode needs for `batch` tokens (0 on bad input). */
size_t swq_moe_decode_workspace_bytes(const swq_moe_layer *layer, int batch);

/* Prepare a fresh workspace: zeroes it, and on the first call for the
 * current device checks (one small blocking launch) whether the batch-1
 * kernel's workgroup groups share an XCD.  Call once after allocating the
 * workspace, outside stream capture; swq_moe_decode leaves it ready for the
 * next call. */
int swq_moe_workspace_init(void *ws, size_t ws_bytes, void *stream);

/* Whether every swq_moe_decode / swq_moe_decode_norm call on this workspace
 * since the last cleared check completed normally: SWQ_OK, or
 * SWQ_ERR_STALLED when one ran out of a bounded wait.  The single-launch
 * (batch 1) kernel has one workgroup per CU and hands data between them
 * through the workspace; it assumes the whole grid is resident at once,
 * which holds on a device running nothing else.  If other work occupies
 * CUs, a wait can last about a second and then give up, and that call's
 * outputs are invalid (the reference throws, MetalEngine.swift:8-11;
 * a stream-ordered call cannot, so the failure is recorded here).
 * Blocking: waits for the stream's earlier work, then reads the record
 * (one 4-byte copy) and, when clear != 0, resets it.  Not capturable.
 * ws = NULL with ws_bytes = 0 names the current device's
 * swq_moe_decode_noalloc array (SWQ_OK if it was never set up). */
int swq_moe_workspace_status(void *ws, size_t ws_bytes, int clear, void *stream);

/* One MoE-layer decode step for `batch` independent tokens, entirely on the
 * device.  Batch 1 runs as one launch (router, softmax, top-k with ties to the
 * lower expert id, renormalisation, routed SwiGLU experts, down projections,
 * sigmoid-gated shared expert and the weighted combine; its stages hand data
 * to each other through the workspace).  Batches run as three launches:
 *   1. router GEMV + shared-gate GEMV + shared gate/up SwiGLU;
 *   2. top-k per token, the distinct experts, their gate/up SwiGLU rows for
 *      all their tokens, indexed by the device-resident ids;
 *   3. down projections + weighted combine + sigmoid-gated shared expert.
 * x: [batch, hidden] of x_dtype (SWQ_F32 / SWQ_BF16).  out: [batch, hidden]
 * of out_dtype (SWQ_F32 / SWQ_BF16).  topk_ids [batch, top_k] int32 and
 * topk_weights [batch, top_k] f32 receive the routing (either may be NULL).
 * The workspace must come from swq_moe_workspace_init and serve one stream
 * at a time.
 * Replaces QwenMetalModel.moeForward / routerPicks / encodePendingMoE
 * (QwenMetalModel.swift:609-716, 798-892) with the numerics of
 * QwenCPUModel.moeForward (QwenCPUModel.swift:500-569). */
int swq_moe_decode(const swq_moe_layer *layer,
                   const void *x, int x_dtype, int batch,
                   void *out, int out_dtype,
                   int32_t *topk_ids, float *topk_weights,
                   void *ws, size_t ws_bytes, int flags, void *stream);

/* swq_moe_decode with no workspace argument and no allocation: for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * The workspace is a static 4 MiB device array inside the library, one per
 * GPU it runs on, held until the process ends; every call on a GPU shares
 * that GPU's array, so calls that overlap in time on one GPU race (run them
 * on one stream).  Layers whose workspace at `batch` does not fit it return
 * SWQ_ERR_LIMIT (the limit covers the benchmark shapes at any batch up to
 * SWQ_MAX_BATCH; use swq_moe_decode for larger ones).  The first call on a
 * device sets the array up (its address, the single launch's XCD probe, a
 * zero fill) and blocks until done: make it outside stream capture (under
 * capture it returns SWQ_ERR_INVALID_ARGUMENT and the set-up waits for the
 * next call; after it, calls may be captured).  Calls on any layer and
 * batch may follow one another.  A stall of the single launch is recorded
 * in the array: swq_moe_workspace_status(NULL, 0, clear, stream) reads it.
 * Arguments and results are swq_moe_decode's. */
int swq_moe_decode_noalloc(const swq_moe_layer *layer,
                           const void *x, int x_dtype, int batch,
                           void *out, int out_dtype,
                           int32_t *topk_ids, float *topk_weights,
                           int flags, void *stream);

/* The MoE step of one token with the layer's residual add and post-attention
 * RMSNorm folded into the same launch:
 *     h1  = h + residual                      (residual may be NULL)
 *     out = h1 + moe(rmsnorm(h1) * norm_weight)
 * h, residual, out: [hidden] f32 device vectors; out must not overlap h or
 * residual (the hidden state alternates between two buffers).  norm_weight:
 * [hidden] of norm_dtype (SWQ_F32 / SWQ_F16 / SWQ_BF16).  The workspace is
 * swq_moe_decode's for batch 1.  SWQ_ERR_LIMIT when the layer does not take
 * the single-launch path (or hidden > 4096): call swq_rmsnorm and
 * swq_moe_decode instead.  Replaces add_inplace + norm_copy + the MoE
 * dispatches of one layer (QwenMetalModel.swift:938-951, :798-873), numerics
 * of QwenCPUModel.layerForward's second half (QwenCPUModel.swift:276-279). */
int swq_moe_decode_norm(const swq_moe_layer *layer, const float *h, const float *residual,
                        const void *norm_weight, int norm_dtype, float norm_eps, float *out,
                        int32_t *topk_ids, float *topk_weights, void *ws, size_t ws_bytes, void *stream);

/* ---- MoE layer prefill ------------------------------------------------ */

/* Workspace bytes swq_moe_prefill needs for `tokens` tokens; 0 on bad input
 * or a layer outside the prefill formats (below). */
size_t swq_moe_prefill_workspace_bytes(const swq_moe_layer *layer, int tokens);

/* The MoE layer over a chunk of `tokens` tokens (a prompt), each token routed
 * on its own exactly as in swq_moe_decode, with the (token, expert) pairs
 * grouped by expert so each expert's weights are contracted against all of
 * its tokens at once on the bf16 matrix cores (codes exact in bf16, fp32
 * accumulation, per-group scales applied in fp32).  Five launches: router
 * GEMM; top-k + grouping; gate/up + SwiGLU; down; weighted combine in pick
 * order, then the sigmoid-gated shared expert.
 * Formats: 4/8-bit codes with group 64 for the router, routed and shared
 * matrices; in_dim a multiple of 128 and at most 4096; the shared gate/up and
 * down matrices with the routed ones' bit widths.  Others: SWQ_ERR_LIMIT.
 * x: [tokens, hidden] of x_dtype (SWQ_F32 / SWQ_BF16); out: [tokens, hidden]
 * of out_dtype; topk_ids / topk_weights: [tokens, top_k] (either may be NULL).
 * The workspace comes from swq_moe_workspace_init, sized by
 * swq_moe_prefill_workspace_bytes, and is left ready for the next call; it is
 * not shared with swq_moe_decode.
 * Replaces the per-token loop of QwenMetalModel.step (QwenMetalModel.swift:359-366)
 * with the grouped form of mlx's SwitchGLU (switch_layers.py:12-24, 75-90,
 * 176-199) and the numerics of QwenCPUModel.moeForward for S tokens
 * (QwenCPUModel.swift:500-569). */
int swq_moe_prefill(const swq_moe_layer *layer,
                    const void *x, int x_dtype, int tokens,
                    void *out, int out_dtype,
                    int32_t *topk_ids, float *topk_weights,
                    void *ws, size_t ws_bytes, int flags, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SWQ_H */
