/*
 * atlas_hip_ops.h -- C ABI of libatlas_hip_ops.so, the MI355X (gfx950)
 * implementation of Atlas's fused per-layer elementwise / normalisation ops.
 *
 * This library replaces, for these ops only, the Metal dispatch of
 * bisegni/atlas (crates/atlas-metal).  Citations are `path:line` into that
 * tree and name the reference interface each entry point stands in for.
 *
 * Conventions
 *  - Every function returns an atlas_status (0 = OK, negative = error); the
 *    message of the last error on a context is atlas_hip_last_error(ctx).
 *  - `atlas_hip_*` device-pointer ops enqueue work on the context's stream
 *    and return immediately (the ResidentCommand model: work completes at
 *    atlas_hip_sync, crates/atlas-metal/src/lib.rs:743-755).  They never
 *    allocate.  Pointers are device pointers owned by the caller; vector
 *    paths are taken when they are 16-byte aligned (hipMalloc gives 256).
 *    Aliasing follows the reference call sites: in-place norms, input ==
 *    normalized, out == lhs and in-place scaling are allowed because every
 *    row is fully read before it is written.
 *  - `atlas_ops_*` host-slice ops mirror atlas_ops::NeuralOps /
 *    MetalRuntime (crates/atlas-ops/src/lib.rs:20-147): validate with the
 *    reference's predicates, copy in, run, copy out, synchronise, and fill an
 *    atlas_dispatch_timing.  Invalid input returns ATLAS_ERR_INVALID_INPUT
 *    before any device work, like MetalError::InvalidInput.
 *  - Reduction order of the row sums of squares (atlas_hip_set_reduction):
 *    ATLAS_REDUCTION_SEQUENTIAL folds left to right in f32, bit-identical to
 *    the reference's CPU operators (crates/atlas-ops/tests/
 *    phase_02_operators.rs:223-242).  ATLAS_REDUCTION_WIDE uses lane-parallel
 *    partial sums + a cross-lane tree everywhere, the strategy of the
 *    reference's rms_norm_decode_batch_f32 and *_wide kernels
 *    (crates/atlas-metal/src/kernels.metal:119-133,1053-1195).
 *    ATLAS_REDUCTION_AUTO (the default) takes the tree where the output is a
 *    plain scaled row (rms_norm f32/f16, the add-norm's y: within 2e-6
 *    relative of the CPU operator on the configs' rows) and the sequential
 *    fold where an epilogue can cancel (the residual and add-scale
 *    epilogues, QK-norm + RoPE, the stable group norm), so those stay
 *    bit-identical to the CPU operators.
 *  - One context per host thread; calls on one context are not re-entrant.
 */
#ifndef ATLAS_HIP_OPS_H
#define ATLAS_HIP_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ATLAS_HIP_OPS_ABI_VERSION 1

/* Error codes: MetalError (crates/atlas-metal/src/lib.rs:37-53). */
typedef enum atlas_status {
    ATLAS_OK = 0,
    ATLAS_ERR_NO_DEVICE = -1,      /* MetalError::NoDevice */
    ATLAS_ERR_INVALID_INPUT = -2,  /* MetalError::InvalidInput */
    ATLAS_ERR_COMMAND_FAILED = -3, /* MetalError::CommandFailed / CommandCreation */
    ATLAS_ERR_OUT_OF_MEMORY = -4
} atlas_status;

typedef enum atlas_reduction {
    ATLAS_REDUCTION_SEQUENTIAL = 0,
    ATLAS_REDUCTION_WIDE = 1,
    ATLAS_REDUCTION_AUTO = 2
} atlas_reduction;

/* DispatchTiming (crates/atlas-metal/src/lib.rs:81-88). */
typedef struct atlas_dispatch_timing {
    double wall_ms; /* host wall time of the whole call */
    double gpu_ms;  /* hipEvent time around the kernel launch(es) */
} atlas_dispatch_timing;

/* RuntimeTelemetry (crates/atlas-metal/src/lib.rs:91-193), the subset that
 * applies to this library. */
typedef struct atlas_hip_telemetry {
    uint64_t dispatches;
    uint64_t syncs;
    uint64_t upload_bytes;
    uint64_t readback_bytes;
    uint64_t allocations;
    uint64_t resident_bytes;
    uint64_t peak_resident_bytes;
} atlas_hip_telemetry;

typedef struct atlas_hip_ctx atlas_hip_ctx;

/* ---- context (MetalRuntime::new / ResidentCommand::finish) -------------- */

/* Number of visible HIP devices (0 when none). */
int atlas_hip_device_count(int *count);
/* MetalRuntime::new (crates/atlas-metal/src/lib.rs:909-1061): select
 * `device`, create a stream.  ATLAS_ERR_NO_DEVICE when no GPU is present. */
int atlas_hip_init(int device, atlas_hip_ctx **out);
void atlas_hip_destroy(atlas_hip_ctx *ctx);
/* ResidentCommand::finish (lib.rs:743-755): wait for all enqueued work and
 * surface device-side failures as ATLAS_ERR_COMMAND_FAILED. */
int atlas_hip_sync(atlas_hip_ctx *ctx);
/* Enqueue on a caller-owned hipStream_t (NULL restores the context stream). */
int atlas_hip_set_stream(atlas_hip_ctx *ctx, void *hip_stream);
void *atlas_hip_get_stream(atlas_hip_ctx *ctx);
int atlas_hip_set_reduction(atlas_hip_ctx *ctx, int reduction);
const char *atlas_hip_last_error(const atlas_hip_ctx *ctx);
int atlas_hip_get_telemetry(const atlas_hip_ctx *ctx, atlas_hip_telemetry *out);

/* ---- device memory and timing plumbing (GpuBuffer, lib.rs:225-238) ------ */
int atlas_hip_malloc(atlas_hip_ctx *ctx, size_t bytes, void **device_ptr);
int atlas_hip_free(atlas_hip_ctx *ctx, void *device_ptr);
int atlas_hip_upload(atlas_hip_ctx *ctx, void *device_dst, const void *host_src, size_t bytes);
int atlas_hip_download(atlas_hip_ctx *ctx, void *host_dst, const void *device_src, size_t bytes);
int atlas_hip_memset(atlas_hip_ctx *ctx, void *device_dst, int value, size_t bytes);
int atlas_hip_copy_d2d(atlas_hip_ctx *ctx, void *device_dst, const void *device_src, size_t bytes);
/* Events recorded on the context stream (exact per-dispatch timing,
 * lib.rs:605-671). */
int atlas_hip_event_create(atlas_hip_ctx *ctx, void **event);
int atlas_hip_event_record(atlas_hip_ctx *ctx, void *event);
int atlas_hip_event_elapsed_ms(atlas_hip_ctx *ctx, void *start, void *stop, float *ms);
int atlas_hip_event_destroy(atlas_hip_ctx *ctx, void *event);

/* ---- graph capture (replaces re-encoding a ResidentCommand per token) ---- */

/* The reference encodes every dispatch of a decode token into a fresh Metal
 * command buffer each token (begin_resident_command, lib.rs:1232-1253;
 * gemma4_executor.rs:4123-4690).  On MI355X the executor instead records the
 * chain once and replays it: atlas_hip_graph_begin starts capturing the
 * context stream, every atlas_hip_* op enqueued until atlas_hip_graph_end is
 * recorded (not run), and atlas_hip_graph_launch replays the whole chain with
 * one submission.  Kernel arguments are frozen at capture time, so per-token
 * values must live in device buffers (as the reference's scalar buffers do,
 * gemma4_executor.rs:1852-1895).  While capturing, call only device-pointer
 * ops: no atlas_ops_*, sync, upload, download, memset or copy. */
int atlas_hip_graph_begin(atlas_hip_ctx *ctx);
int atlas_hip_graph_end(atlas_hip_ctx *ctx, void **graph);
int atlas_hip_graph_launch(atlas_hip_ctx *ctx, void *graph);
int atlas_hip_graph_destroy(atlas_hip_ctx *ctx, void *graph);

/* ---- RMSNorm family (device pointers, async) ---------------------------- */

/* rms_norm_f32 / rms_norm_decode_batch_f32 (kernels.metal:106-133); caller
 * MetalRuntime::rms_norm (lib.rs:1485-1520), Gemma prefill
 * (gemma4_executor.rs:3732).  y = (x * inv) * w per row. */
int atlas_hip_rms_norm_f32(atlas_hip_ctx *ctx, const float *input, const float *weight,
                           float *output, uint32_t rows, uint32_t hidden, float epsilon);

/* gemma4_rms_residual_f32 (kernels.metal:183-214; caller
 * gemma4_executor.rs:4492-4506): n = (x*inv)*w; normalized = n (optional,
 * may be NULL or alias input); output = residual + n (may alias residual). */
int atlas_hip_rms_norm_residual_f32(atlas_hip_ctx *ctx, const float *input, const float *weight,
                                    const float *residual, float *normalized, float *output,
                                    uint32_t rows, uint32_t hidden, float epsilon);

/* Llama pre-norm vector_add_f32 + rms_norm (executor.rs:1258-1286):
 * residual_out = input + residual; output = rms_norm(residual_out). */
int atlas_hip_add_rms_norm_f32(atlas_hip_ctx *ctx, const float *input, const float *residual,
                               const float *weight, float *residual_out, float *output,
                               uint32_t rows, uint32_t hidden, float epsilon);

/* gemma4_ple_rms_add_scale_f32 (kernels.metal:228-258; caller
 * gemma4_executor.rs:4627-4641): state = (state + (x*inv)*w) * (*scale),
 * `scale` is a device scalar. */
int atlas_hip_rms_norm_add_scale_f32(atlas_hip_ctx *ctx, const float *input, const float *weight,
                                     float *state, const float *scale, uint32_t rows,
                                     uint32_t hidden, float epsilon);

/* rms_norm_groups_in_place_stable_f32 (kernels.metal:897-917; callers
 * gemma4_executor.rs:3600-3611, 4206-4217): max-scaled RMSNorm of `groups`
 * groups of `width` values, in place. */
int atlas_hip_rms_norm_groups_stable_f32(atlas_hip_ctx *ctx, float *values, const float *weight,
                                         uint32_t width, uint32_t groups, float epsilon);

/* FP16-storage RMSNorm with FP32 math (config C2; no FP16 path exists in the
 * reference, which is FP32-only).  Outputs rounded IEEE RNE. */
int atlas_hip_rms_norm_f16(atlas_hip_ctx *ctx, const uint16_t *input, const uint16_t *weight,
                           uint16_t *output, uint32_t rows, uint32_t hidden, float epsilon);
/* FP16-storage pre-norm add + RMSNorm: residual_out = rne16(input + residual),
 * output = rms_norm(residual_out). */
int atlas_hip_add_rms_norm_f16(atlas_hip_ctx *ctx, const uint16_t *input, const uint16_t *residual,
                               const uint16_t *weight, uint16_t *residual_out, uint16_t *output,
                               uint32_t rows, uint32_t hidden, float epsilon);

/* ---- RoPE --------------------------------------------------------------- */

/* gemma4_qk_norm_rope_fused[_batch]_f32[_wide] (kernels.metal:1004-1195;
 * callers gemma4_executor.rs:2614-2668, 3799-3825).  q [tokens, q_heads,
 * head_dim], k [tokens, head_dim] (read only when has_key), cos/sin
 * [tokens, rope_stride].  Per (token, head): weighted RMSNorm over head_dim
 * then half-split RoPE.  q_out may alias q, k_out may alias k. */
int atlas_hip_qk_norm_rope_f32(atlas_hip_ctx *ctx, const float *q, const float *k,
                               const float *q_weight, const float *k_weight, const float *cosine,
                               const float *sine, float *q_out, float *k_out, uint32_t tokens,
                               uint32_t q_heads, uint32_t has_key, uint32_t head_dim,
                               uint32_t rope_stride, float epsilon);

/* Llama half-split RoPE: net effect of rope_half_to_interleaved_f32 +
 * rope_f32 + rope_interleaved_to_half_f32 (kernels.metal:940-994; caller
 * executor.rs:1120-1166).  x [tokens, heads, head_dim], cos/sin
 * [tokens, rope_stride]. */
int atlas_hip_rope_half_f32(atlas_hip_ctx *ctx, const float *input, const float *cosine,
                            const float *sine, float *output, uint32_t tokens, uint32_t heads,
                            uint32_t head_dim, uint32_t rope_stride);
int atlas_hip_rope_half_f16(atlas_hip_ctx *ctx, const uint16_t *input, const float *cosine,
                            const float *sine, uint16_t *output, uint32_t tokens, uint32_t heads,
                            uint32_t head_dim, uint32_t rope_stride);
/* The Llama decode rotates Q and then K of the same tokens with the same
 * cos/sin rows, each through the three-dispatch chain above (executor.rs:
 * 1120-1166).  This is both tensors in one launch: q [tokens, q_heads,
 * head_dim], k [tokens, k_heads, head_dim]; results as two rope_half calls. */
int atlas_hip_rope_half_qk_f32(atlas_hip_ctx *ctx, const float *q, const float *k, const float *cosine,
                               const float *sine, float *q_out, float *k_out, uint32_t tokens, uint32_t q_heads,
                               uint32_t k_heads, uint32_t head_dim, uint32_t rope_stride);
int atlas_hip_rope_half_qk_f16(atlas_hip_ctx *ctx, const uint16_t *q, const uint16_t *k, const float *cosine,
                               const float *sine, uint16_t *q_out, uint16_t *k_out, uint32_t tokens,
                               uint32_t q_heads, uint32_t k_heads, uint32_t head_dim, uint32_t rope_stride);
/* rope_f32 (kernels.metal:940-949) = NeuralOps::rope: interleaved pairs, one
 * cos/sin row of hidden/2 shared by all rows. */
int atlas_hip_rope_interleaved_f32(atlas_hip_ctx *ctx, const float *input, const float *cosine,
                                   const float *sine, float *output, uint32_t rows,
                                   uint32_t hidden);

/* Host RoPE tables (the reference computes them on the host in f32 with the
 * platform libm): gemma4_rope_angle (gemma4_executor.rs:622-633; prefill
 * layout :3494-3519) and write_rope_tables (executor.rs:632-647).
 * frequency_factors may be NULL (all 1). */
int atlas_rope_tables_gemma4(const uint32_t *positions, size_t tokens, size_t rope_pairs,
                             size_t rotary, float theta, const float *frequency_factors,
                             float *cos_out, float *sin_out);
int atlas_rope_tables_llama(const uint32_t *positions, size_t tokens, size_t head_dim, float theta,
                            float *cos_out, float *sin_out);

/* ---- gated activations and elementwise ops ------------------------------ */

/* silu_f32 + vector_multiply_f32 (kernels.metal:27-36, 64-69; caller
 * executor.rs:1318-1327): out = silu(gate) * up. */
int atlas_hip_swiglu_f32(atlas_hip_ctx *ctx, const float *gate, const float *up, float *output,
                         uint64_t count);
int atlas_hip_swiglu_f16(atlas_hip_ctx *ctx, const uint16_t *gate, const uint16_t *up,
                         uint16_t *output, uint64_t count);
/* gelu_multiply_f32 (kernels.metal:773-784; callers gemma4_executor.rs:4007,
 * 4527): out = gelu_tanh(gate) * up. */
int atlas_hip_geglu_f32(atlas_hip_ctx *ctx, const float *gate, const float *up, float *output,
                        uint64_t count);
/* ple_gelu_multiply_offset_f32 / gelu_f32 + vector_multiply_offset_batch_f32
 * (kernels.metal:790-801, 83-92; callers gemma4_executor.rs:4063-4081,
 * 4596-4607): out[r, i] = gelu(gate[r, i]) * ple[r*ple_row_stride + ple_offset + i]. */
int atlas_hip_geglu_offset_f32(atlas_hip_ctx *ctx, const float *gate, const float *ple,
                               float *output, uint32_t ple_offset, uint32_t ple_row_stride,
                               uint32_t width, uint32_t rows);
/* silu_f32, gelu_f32, vector_add_f32, vector_multiply_f32, scalar_multiply_f32
 * (kernels.metal:5-36, 64-69, 752-767). */
int atlas_hip_silu_f32(atlas_hip_ctx *ctx, const float *input, float *output, uint64_t count);
int atlas_hip_gelu_f32(atlas_hip_ctx *ctx, const float *input, float *output, uint64_t count);
int atlas_hip_add_f32(atlas_hip_ctx *ctx, const float *lhs, const float *rhs, float *output,
                      uint64_t count);
int atlas_hip_multiply_f32(atlas_hip_ctx *ctx, const float *lhs, const float *rhs, float *output,
                           uint64_t count);
int atlas_hip_scale_f32(atlas_hip_ctx *ctx, const float *input, float scalar, float *output,
                        uint64_t count);

/* ---- gathers ------------------------------------------------------------ */

/* embedding_lookup_f32 (kernels.metal:94-104; caller executor.rs:1063-1074):
 * out[t] = table[ids[t]] * scale (scale 1.0 = pure copy); ids >= vocab give
 * zeros. */
int atlas_hip_embed_f32(atlas_hip_ctx *ctx, const float *table, const uint32_t *ids, float *output,
                        uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale);
/* embedding_lookup_q4_0 / _q6_k + scalar_multiply_f32 (kernels.metal:653-692,
 * 16-25; callers gemma4_executor.rs:3533-3554, 4145-4161): dequantised row
 * times `scale` (Gemma: sqrt(hidden)).  hidden % 32 (Q4_0) / % 256 (Q6_K)
 * == 0; rows whose id >= vocab are left untouched, as in the reference.
 * output must be 16-byte aligned. */
int atlas_hip_embed_q4_0(atlas_hip_ctx *ctx, const uint8_t *table, const uint32_t *ids,
                         float *output, uint32_t vocab, uint32_t hidden, uint32_t tokens,
                         float scale);
int atlas_hip_embed_q6_k(atlas_hip_ctx *ctx, const uint8_t *table, const uint32_t *ids,
                         float *output, uint32_t vocab, uint32_t hidden, uint32_t tokens,
                         float scale);
/* embedding_lookup_q8_0 (kernels.metal:658-661): the Llama resident
 * embedding of Q8_0 tables (resident_embedding_kernel, crates/atlas-model/
 * src/executor.rs:1541-1549, dispatched at :1063-1074, scale 1.0).  34-byte
 * blocks of 32 (f16 d, 32 int8); out = f32(int8) * d * scale.  hidden % 32
 * == 0; rows whose id >= vocab are left untouched; output 16-byte aligned. */
int atlas_hip_embed_q8_0(atlas_hip_ctx *ctx, const uint8_t *table, const uint32_t *ids,
                         float *output, uint32_t vocab, uint32_t hidden, uint32_t tokens,
                         float scale);
/* Gemma PLE chain gather + x sqrt(256) + add + x 1/sqrt(2)
 * (gemma4_executor.rs:3555-3631, 4162-4237; gemma4_combine_ple
 * crates/atlas-model/src/lib.rs:206-219):
 * out[t, l, i] = (deq(table[ids[t]])[l*width + i] * embedding_scale
 *                 + projection[t, l, i]) * output_scale.
 * table rows hold layers*width values; projection/output are
 * [tokens, layers, width] f32, 16-byte aligned. */
int atlas_hip_ple_q4_0(atlas_hip_ctx *ctx, const uint8_t *table, const uint32_t *ids,
                       const float *projection, float *output, uint32_t vocab, uint32_t layers,
                       uint32_t width, uint32_t tokens, float embedding_scale, float output_scale);
int atlas_hip_ple_q6_k(atlas_hip_ctx *ctx, const uint8_t *table, const uint32_t *ids,
                       const float *projection, float *output, uint32_t vocab, uint32_t layers,
                       uint32_t width, uint32_t tokens, float embedding_scale, float output_scale);

/* ---- RMS-folded Q4_0 decode projections (one token) --------------------- */

/* output[o] = inv_rms(input) * sum_k (input[k] * rms_weight[k]) * deq(W[o, k])
 * with inv_rms = 1 / sqrt(sum_k input[k]^2 / input_width + epsilon): the
 * RMS-normalised input of a decode step folded into its projection.  With
 * rms_weight == NULL it is the plain Q4_0 matvec (output = W . input).
 * W is [output_width, input_width] in Q4_0 blocks (18 bytes per 32 values,
 * rows contiguous); input_width is a multiple of 32 and at most 4096;
 * input and rms_weight are 16-byte aligned f32 vectors, W is 2-byte aligned
 * (16-byte aligned takes the wide staging path).  Floating-point parity is
 * the reference's own contract (normalise-then-matvec CPU oracle, max-abs
 * < 1e-3, crates/atlas-metal/tests/matvec_rms_fused_parity.rs).
 * matvec_q4_0_16row_mv_rms (kernels.metal:3786-3864); caller
 * Gemma4Executor::matvec_rms_labeled (gemma4_executor.rs:2082-2119). */
int atlas_hip_matvec_q4_0_rms_f32(atlas_hip_ctx *ctx, const float *input, const uint8_t *weights,
                                  float *output, uint32_t input_width, uint32_t output_width,
                                  const float *rms_weight, float epsilon);
/* matmul_q4_0_qkv_16row_mv_rms (kernels.metal:3368-3467; caller
 * Gemma4Executor::matmul_q4_0_qkv, gemma4_executor.rs:2502-2558): the Q, K and
 * V projections of one input in one launch; K and V share kv_width. */
int atlas_hip_matmul_q4_0_qkv_rms_f32(atlas_hip_ctx *ctx, const float *input, const uint8_t *q_weights,
                                      const uint8_t *k_weights, const uint8_t *v_weights, float *q_output,
                                      float *k_output, float *v_output, uint32_t input_width,
                                      uint32_t q_width, uint32_t kv_width, const float *rms_weight,
                                      float epsilon);
/* matmul_q4_0_gate_up_16row_mv_rms (kernels.metal:3468-3564; caller
 * Gemma4Executor::matmul_q4_0_gate_up, gemma4_executor.rs:2560-2612). */
int atlas_hip_matmul_q4_0_gate_up_rms_f32(atlas_hip_ctx *ctx, const float *input,
                                          const uint8_t *gate_weights, const uint8_t *up_weights,
                                          float *gate_output, float *up_output, uint32_t input_width,
                                          uint32_t output_width, const float *rms_weight, float epsilon);

/* gemma4_ple_gate_gelu_f32 (kernels.metal:803-881; the fused form of
 * matvec_q4_0_16row_mv + ple_gelu_multiply_offset_f32, caller
 * gemma4_executor.rs:4063-4081): the PLE input gate of one decode token,
 * output[o] = gelu_tanh(sum_k input[k] * deq(W[o, k])) * ple[ple_offset + o],
 * with the reference's GELU (kernels.metal:752-767).  W as above
 * ([output_width, input_width] Q4_0, input_width % 32 == 0, <= 4096); the
 * projection is floating point (tolerance parity), the GELU and the product
 * are the reference's roundings. */
int atlas_hip_ple_gate_gelu_f32(atlas_hip_ctx *ctx, const float *input, const uint8_t *weights,
                                const float *ple, uint32_t ple_offset, float *output, uint32_t input_width,
                                uint32_t output_width);

/* The PLE projection of one decode token with its norm, in one call:
 * matvec_f16 (kernels.metal:731-740), scalar_multiply_f32 by `scale`, then
 * rms_norm_groups_in_place_stable_f32 (kernels.metal:897-917) over `groups`
 * groups of `width` values; callers gemma4_executor.rs:4184-4214 (the
 * decode PLE chain: ple_projection, its scale, ple_norm).
 *   p[o]   = (sum_k input[k] * W[o, k]) * scale,  o < groups * width
 *   out[g] = stable_rms_norm(p[g * width .. (g + 1) * width), norm_weight)
 * W is F16 [groups * width, hidden] (row o contiguous, the GGUF layout of
 * per_layer_model_proj); hidden % 8 == 0 and <= 4096, width % 16 == 0 and
 * <= 1024, groups <= 1024; input and W 16-byte aligned.  Like the
 * reference's matvec_f16 the dot is floating point (tolerance parity); the
 * norm follows the reference's steps on the dots (its sum of squares in a
 * fixed tree order).  Two launches on the context's stream: the scaled
 * dots into `output`, then the norm in place. */
int atlas_hip_ple_projection_f16(atlas_hip_ctx *ctx, const float *input, const uint16_t *weights,
                                 const float *norm_weight, float *output, uint32_t hidden, uint32_t width,
                                 uint32_t groups, float scale, float epsilon);

/* ---- KV-cache append with the fused V RMSNorm and Q8_0/Q4_0 encoders ----- */

/* kv_append_decode_{f32,q8_0,q4_0}[_batch|_vnorm] (kernels.metal:1197-1436;
 * callers gemma4_executor.rs:3826-3850 prefill, :4326-4368 decode).
 * key/value: [tokens, kv_width] f32; positions: [tokens] device u32 (decode:
 * tokens = 1 and the position buffer); tokens whose position is >= capacity
 * are skipped.  cache layout [K | V][capacity][row]: a row is kv_width f32
 * (f32) or kv_width/32 blocks of 34 (Q8_0) / 18 (Q4_0) bytes.  vnorm != 0
 * scales each V row by 1 / sqrt(sum v^2 / kv_width + epsilon) (sum in index
 * order: rms_norm_groups_in_place_unweighted_f32, kernels.metal:919-929)
 * before it is stored; the value buffer is not modified.  kv_width <= 4096,
 * a multiple of 4 (f32) or 32 (Q8_0, Q4_0).  Bit-exact against the CPU
 * restatement of the Metal encoders (IEEE division and sqrt). */
int atlas_hip_kv_append_f32(atlas_hip_ctx *ctx, const float *key, const float *value, float *cache,
                            uint32_t kv_width, uint32_t capacity, const uint32_t *positions,
                            uint32_t tokens, int vnorm, float epsilon);
int atlas_hip_kv_append_q8_0(atlas_hip_ctx *ctx, const float *key, const float *value, uint8_t *cache,
                             uint32_t kv_width, uint32_t capacity, const uint32_t *positions,
                             uint32_t tokens, int vnorm, float epsilon);
int atlas_hip_kv_append_q4_0(atlas_hip_ctx *ctx, const float *key, const float *value, uint8_t *cache,
                             uint32_t kv_width, uint32_t capacity, const uint32_t *positions,
                             uint32_t tokens, int vnorm, float epsilon);

/* ---- logits: soft cap and greedy argmax (decode tail) -------------------- */

/* softcap_f32 (kernels.metal:931-934; callers gemma4_executor.rs:3673-3676,
 * 4678-4682; CPU form gemma4_softcap_logits,
 * crates/atlas-model/src/lib.rs:223-232): output = cap * tanh(input / cap)
 * over `count` values; output may alias input (the reference caps in
 * place).  cap must be finite and positive, as gemma4_softcap_logits
 * ensures.  The tanh is this library's (within 1.4 ulp of float64); the
 * reference's Metal/libm tanh bits are not reproducible off Apple, so parity
 * with the reference is the operator tolerance, bit-exact with the oracle. */
int atlas_hip_softcap_f32(atlas_hip_ctx *ctx, const float *input, float *output, uint64_t count, float cap);
/* argmax_f32 (kernels.metal:2033-2066; callers gemma4_executor.rs:3678-3683,
 * 4683-4688, executor.rs:1381 via dispatch_decode_argmax :1515): for each of
 * `rows` rows of `count` values, selected[r] = the largest index holding the
 * row's maximum (the reference's tie rule: the later token id wins); NaN is
 * never selected and +0 equals -0, as under the kernel's comparisons; a row
 * of NaN selects 0.  count >= 1 (argmax_for_test, lib.rs:1623-1628). */
int atlas_hip_argmax_f32(atlas_hip_ctx *ctx, const float *values, uint32_t *selected, uint32_t rows,
                         uint32_t count);
/* The argmax entry points keep per-workgroup partial results in a 512 KiB
 * workspace that atlas_hip_init allocates for the context; every call
 * overwrites it.  Calls on one context are ordered by its stream; a caller
 * that moves the context to another stream (atlas_hip_set_stream) between
 * two argmax calls must synchronise in between, or the two race. */
/* softcap_f32 followed by argmax_f32, the decode tail of
 * encode_current_token (gemma4_executor.rs:4678-4688), in one pass:
 * capped = cap * tanh(logits / cap) (may alias logits; NULL skips the
 * store), selected[r] = argmax of capped row r.  Same results as the two
 * entry points above in sequence. */
int atlas_hip_softcap_argmax_f32(atlas_hip_ctx *ctx, const float *logits, float *capped, uint32_t *selected,
                                 uint32_t rows, uint32_t count, float cap);
/* No counterpart in the reference: atlas_hip_softcap_argmax_f32 for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, validation and results;
 * the per-workgroup partial keys go to a 128 KiB static device array of the
 * library (16384 slots, one copy per GPU, resolved by atlas_hip_init)
 * instead of the context's workspace, and the call allocates nothing.  A
 * row longer than one workgroup's share (1024 values; 4096 in batches of
 * 2^22 values or more) is split over several workgroups whose partial keys
 * must all fit the 16384 slots in one launch pair: sizes whose rows x
 * workgroups per row exceed them are rejected with ATLAS_ERR_INVALID_INPUT
 * (256 rows of 262144 values fit, as do 64 rows of 1048576).  Rows of one
 * workgroup use no slots, at any row count (launches of up to 65535 rows).
 * Every call on one GPU shares the array: calls that overlap on one GPU (two
 * streams or contexts) race. */
int atlas_hip_softcap_argmax_f32_noalloc(atlas_hip_ctx *ctx, const float *logits, float *capped,
                                         uint32_t *selected, uint32_t rows, uint32_t count, float cap);

/* ---- host-slice operator API (atlas_ops::NeuralOps) --------------------- */

/* NeuralOps::embedding -> MetalRuntime::embedding_lookup (lib.rs:1393-1433). */
int atlas_ops_embedding(atlas_hip_ctx *ctx, const float *table, size_t table_len, size_t vocabulary,
                        size_t hidden, const uint32_t *token_ids, size_t token_count, float *output,
                        size_t output_len, atlas_dispatch_timing *timing);
/* MetalRuntime::embedding_lookup_q6_k (lib.rs:1437-1483). */
int atlas_ops_embedding_q6_k(atlas_hip_ctx *ctx, const uint8_t *weights, size_t weights_len,
                             size_t vocabulary, size_t hidden, const uint32_t *token_ids,
                             size_t token_count, float *output, size_t output_len,
                             atlas_dispatch_timing *timing);
/* NeuralOps::add -> MetalRuntime::vector_add (lib.rs:1323-1346). */
int atlas_ops_add(atlas_hip_ctx *ctx, const float *lhs, size_t lhs_len, const float *rhs,
                  size_t rhs_len, float *output, size_t output_len, atlas_dispatch_timing *timing);
/* NeuralOps::multiply -> MetalRuntime::vector_multiply (lib.rs:1368-1391). */
int atlas_ops_multiply(atlas_hip_ctx *ctx, const float *lhs, size_t lhs_len, const float *rhs,
                       size_t rhs_len, float *output, size_t output_len,
                       atlas_dispatch_timing *timing);
/* MetalRuntime::scalar_multiply (lib.rs:1348-1366). */
int atlas_ops_scalar_multiply(atlas_hip_ctx *ctx, const float *input, size_t input_len, float scalar,
                              float *output, size_t output_len, atlas_dispatch_timing *timing);
/* NeuralOps::silu -> MetalRuntime::silu (lib.rs:1897-1910). */
int atlas_ops_silu(atlas_hip_ctx *ctx, const float *input, size_t input_len, float *output,
                   size_t output_len, atlas_dispatch_timing *timing);
/* MetalRuntime::gelu (lib.rs:1913-1926). */
int atlas_ops_gelu(atlas_hip_ctx *ctx, const float *input, size_t input_len, float *output,
                   size_t output_len, atlas_dispatch_timing *timing);
/* NeuralOps::rms_norm -> MetalRuntime::rms_norm (lib.rs:1485-1520). */
int atlas_ops_rms_norm(atlas_hip_ctx *ctx, const float *input, size_t input_len, size_t rows,
                       size_t hidden, const float *weight, size_t weight_len, float epsilon,
                       float *output, size_t output_len, atlas_dispatch_timing *timing);
/* NeuralOps::rope -> MetalRuntime::rope (lib.rs:1697-1733). */
int atlas_ops_rope(atlas_hip_ctx *ctx, const float *input, size_t input_len, size_t rows,
                   size_t hidden, const float *cosine, size_t cosine_len, const float *sine,
                   size_t sine_len, float *output, size_t output_len,
                   atlas_dispatch_timing *timing);

#ifdef __cplusplus
}
#endif

#endif /* ATLAS_HIP_OPS_H */
