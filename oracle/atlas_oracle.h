/*
 * atlas_oracle.h -- CPU restatement of Atlas's fused per-layer
 * elementwise / normalisation operators.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * HIP kernels in atlas_amd/csrc and the CPU baseline timed by bench.py.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product library (libatlas_hip_ops.so) never links or calls it.
 *
 * Arithmetic contract: IEEE-754 binary32, round-to-nearest-even, no FMA
 * contraction (built with -ffp-contract=off; the only fused multiply-adds
 * are the explicit fmaf calls of oracle_expf), fixed evaluation order that
 * restates the reference's Rust CPU oracles and Metal kernels, cited per
 * function as `path:line` into the bisegni/atlas tree.
 *
 * Parity pins (what checks each function, see tests/test_oracle_*.py):
 *   - f16 decode:      exhaustive over all 65536 codes vs numpy float16.
 *   - rms_norm:        reference KAT input (phase_02_operators.rs:94-104) vs a
 *                      float64 restatement; scale invariance; row RMS of y/w.
 *   - rope:            reference KAT (phase_02_operators.rs:127-135); angle
 *                      KATs (gemma4_executor.rs:4906-4914); position-0
 *                      identity; pair-norm preservation.
 *   - exp/silu/gelu:   float64 math within stated ULP bounds; reference GELU
 *                      extreme-input KAT (phase_00_bootstrap.rs:126-145).
 *   - dequant/gathers: reference Q4_0 / Q6_K KATs (phase_11a_gguf.rs:57-97),
 *                      the independent llama.cpp-order Q6_K decoder
 *                      (phase_11a_gguf.rs:11-31), brute force over every code.
 *   - PLE combine:     reference KAT (gemma4_primitives.rs:3-10).
 *   - fused epilogues: equal to the composition of the unfused oracle steps
 *                      (the reference's dispatch_fusion_parity.rs contract).
 *   - tanh_precise:    float64 tanh (< 1.4 ulp over a dense binary32 sweep)
 *                      and glibc tanhf (<= 2 ulp); soft-cap KAT
 *                      (gemma4_primitives.rs:13-19).
 *   - argmax:          the reference's large-vocabulary tie KAT
 *                      (crates/atlas-metal/src/lib.rs:2217-2230), numpy argmax
 *                      of the reversed row, brute-force tie/NaN/-0 cases.
 */
#ifndef ATLAS_ORACLE_H
#define ATLAS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 codec ---------------------------------------------------------- */
float oracle_f16_to_f32(uint16_t bits);
uint16_t oracle_f32_to_f16_rne(float value);
void oracle_f16_to_f32_n(const uint16_t *src, float *dst, size_t n);
void oracle_f32_to_f16_rne_n(const float *src, uint16_t *dst, size_t n);

/* ---- transcendental kernel shared by the activation oracles ------------- */
float oracle_expf(float x);
float oracle_tanhf(float x);
float oracle_silu(float x);
float oracle_gelu_tanh(float x);

/* ---- RMSNorm family ----------------------------------------------------- */
float oracle_inverse_rms(const float *row, size_t hidden, float epsilon);
void oracle_rms_norm_f32(const float *input, const float *weight, float *output,
                         size_t rows, size_t hidden, float epsilon);
void oracle_rms_norm_residual_f32(const float *input, const float *weight,
                                  const float *residual, float *normalized,
                                  float *output, size_t rows, size_t hidden,
                                  float epsilon);
void oracle_add_rms_norm_f32(const float *input, const float *residual,
                             const float *weight, float *residual_out,
                             float *output, size_t rows, size_t hidden,
                             float epsilon);
void oracle_rms_norm_add_scale_f32(const float *input, const float *weight,
                                   float *state, float scale, size_t rows,
                                   size_t hidden, float epsilon);
void oracle_rms_norm_groups_stable_f32(float *values, const float *weight,
                                       size_t width, size_t groups,
                                       float epsilon);
/* matvec_f16 (kernels.metal:731-740) * scale, then the stable group norm:
 * the decode PLE projection (gemma4_executor.rs:4184-4214). */
void oracle_ple_projection_f16(const float *input, const uint16_t *weights, const float *norm_weight,
                               float *output, size_t hidden, size_t width, size_t groups, float scale,
                               float epsilon);
void oracle_rms_norm_f16(const uint16_t *input, const uint16_t *weight,
                         uint16_t *output, size_t rows, size_t hidden,
                         float epsilon);
void oracle_add_rms_norm_f16(const uint16_t *input, const uint16_t *residual,
                             const uint16_t *weight, uint16_t *residual_out,
                             uint16_t *output, size_t rows, size_t hidden,
                             float epsilon);

/* ---- RoPE --------------------------------------------------------------- */
float oracle_gemma4_rope_angle(size_t position, size_t pair, size_t rotary,
                               float theta, float frequency_factor);
void oracle_rope_tables_gemma4(const uint32_t *positions, size_t tokens,
                               size_t rope_pairs, size_t rotary, float theta,
                               const float *frequency_factors, float *cos_out,
                               float *sin_out);
void oracle_rope_tables_llama(const uint32_t *positions, size_t tokens,
                              size_t head_dim, float theta, float *cos_out,
                              float *sin_out);
void oracle_rope_interleaved_f32(const float *input, size_t rows, size_t hidden,
                                 const float *cosine, const float *sine,
                                 float *output);
void oracle_rope_half_f32(const float *input, const float *cosine,
                          const float *sine, float *output, size_t tokens,
                          size_t heads, size_t head_dim, size_t rope_stride);
void oracle_rope_half_f16(const uint16_t *input, const float *cosine,
                          const float *sine, uint16_t *output, size_t tokens,
                          size_t heads, size_t head_dim, size_t rope_stride);
void oracle_qk_norm_rope_f32(const float *q, const float *k,
                             const float *q_weight, const float *k_weight,
                             const float *cosine, const float *sine,
                             float *q_out, float *k_out, size_t tokens,
                             size_t q_heads, int has_key, size_t head_dim,
                             size_t rope_stride, float epsilon);

/* ---- gated activations -------------------------------------------------- */
void oracle_silu_f32(const float *input, float *output, size_t n);
void oracle_gelu_f32(const float *input, float *output, size_t n);
void oracle_swiglu_f32(const float *gate, const float *up, float *output,
                       size_t n);
void oracle_swiglu_f16(const uint16_t *gate, const uint16_t *up,
                       uint16_t *output, size_t n);
void oracle_geglu_f32(const float *gate, const float *up, float *output,
                      size_t n);
void oracle_geglu_offset_f32(const float *gate, const float *ple,
                             float *output, size_t ple_offset,
                             size_t ple_row_stride, size_t width, size_t rows);

/* ---- gathers and block dequant ------------------------------------------ */
void oracle_dequant_q4_0_block(const uint8_t *block, float *out32);
void oracle_dequant_q8_0_block(const uint8_t *block, float *out32);
void oracle_dequant_q6_k_block(const uint8_t *block, float *out256);
void oracle_dequant_q6_k_block_llama_order(const uint8_t *block, float *out256);
void oracle_embed_f32(const float *table, const uint32_t *ids, float *output,
                      size_t vocab, size_t hidden, size_t tokens);
void oracle_embed_q4_0(const uint8_t *table, const uint32_t *ids, float *output,
                       size_t vocab, size_t hidden, size_t tokens, float scale);
void oracle_embed_q8_0(const uint8_t *table, const uint32_t *ids, float *output,
                       size_t vocab, size_t hidden, size_t tokens, float scale);
void oracle_embed_q6_k(const uint8_t *table, const uint32_t *ids, float *output,
                       size_t vocab, size_t hidden, size_t tokens, float scale);
void oracle_ple_q4_0(const uint8_t *table, const uint32_t *ids,
                     const float *projection, float *output, size_t vocab,
                     size_t layers, size_t width, size_t tokens,
                     float embedding_scale, float output_scale);
void oracle_ple_q6_k(const uint8_t *table, const uint32_t *ids,
                     const float *projection, float *output, size_t vocab,
                     size_t layers, size_t width, size_t tokens,
                     float embedding_scale, float output_scale);
void oracle_combine_ple(const float *identity, const float *context,
                        float *output, size_t n);

/* ---- elementwise helpers from the operator API -------------------------- */
void oracle_add_f32(const float *lhs, const float *rhs, float *output, size_t n);
void oracle_multiply_f32(const float *lhs, const float *rhs, float *output,
                         size_t n);
void oracle_scale_f32(const float *input, float scalar, float *output, size_t n);

/* RMS-folded Q4_0 decode projections (matvec_rms_fused_parity.rs:51-80
 * oracle in f32, and a float64 restatement with the error magnitude). */
void oracle_matvec_q4_0_rms_ref(const float *input, const uint8_t *weights, const float *rms_weight,
                                size_t input_width, size_t output_width, float epsilon, float *output);
void oracle_matvec_q4_0_rms_f64(const float *input, const uint8_t *weights, const float *rms_weight,
                                size_t input_width, size_t output_width, float epsilon, double *output,
                                double *magnitude);

/* KV-cache append with the fused V RMSNorm and the Q8_0 / Q4_0 encoders
 * (kernels.metal:919-929, 1197-1436).  format: 0 f32, 1 Q8_0, 2 Q4_0. */
void oracle_encode_q8_0_block(const float *v, uint8_t *out34);
void oracle_encode_q4_0_block(const float *v, uint8_t *out18);
void oracle_kv_append(int format, const float *key, const float *value, uint8_t *cache, size_t kv_width,
                      size_t capacity, const uint32_t *positions, size_t tokens, int vnorm, float epsilon);

/* Logits: soft cap (softcap_f32, kernels.metal:931-934; CPU
 * gemma4_softcap_logits, crates/atlas-model/src/lib.rs:223-232) and argmax
 * (argmax_f32, kernels.metal:2033-2066). */
float oracle_tanh_precise(float x);
void oracle_softcap_f32(const float *input, float *output, size_t n, float cap);
uint32_t oracle_argmax_f32(const float *values, size_t count);
void oracle_softcap_argmax_rows(float *logits, uint32_t *selected, size_t rows, size_t count, float cap);

#ifdef __cplusplus
}
#endif

#endif
