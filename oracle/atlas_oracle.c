/*
 * atlas_oracle.c -- CPU restatement of Atlas's fused per-layer operators.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline); see the header
 * atlas_oracle.h for the arithmetic contract and the checks that pin each
 * function.  Build: oracle/Makefile (-O3 -ffp-contract=off, no fast-math).
 *
 * Reference citations are `path:line` into bisegni/atlas.
 */
#include "atlas_oracle.h"

#include <math.h>
#include <string.h>

/* ======================================================================== */
/* f16 codec                                                                */
/* ======================================================================== */

/* Restates f16_bits_to_f32 (crates/atlas-core/src/tensor.rs:286-305):
 * exact widening of normals, subnormals (normalise loop), signed zero,
 * infinities and NaN payloads. */
float oracle_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exponent = (bits >> 10) & 0x1fu;
    uint32_t mantissa = bits & 0x03ffu;
    uint32_t out;
    if (exponent == 0) {
        if (mantissa == 0) {
            out = sign;
        } else {
            int32_t e = -14;
            while ((mantissa & 0x400u) == 0) {
                mantissa <<= 1;
                e -= 1;
            }
            out = sign | ((uint32_t)(e + 127) << 23) | ((mantissa & 0x3ffu) << 13);
        }
    } else if (exponent == 31) {
        out = sign | 0x7f800000u | (mantissa << 13);
    } else {
        out = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float value;
    memcpy(&value, &out, sizeof value);
    return value;
}

/* IEEE-754 round-to-nearest-even binary32 -> binary16.  This is deliberately
 * NOT Atlas's f32_to_f16_bits (crates/atlas-core/src/tensor.rs:265-283),
 * which rounds ties up and can carry into the exponent incorrectly; FP16
 * storage outputs are defined as IEEE RNE. */
uint16_t oracle_f32_to_f16_rne(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t abs = x & 0x7fffffffu;
    if (abs >= 0x7f800000u) { /* inf or nan */
        if (abs > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((abs >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (abs >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 */
    if (abs < 0x38800000u) {                                    /* f16 subnormal / zero */
        if (abs < 0x33000000u) return sign;                     /* < 2^-25: rounds to 0 */
        uint32_t e = abs >> 23;
        uint32_t m = (abs & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* value = m * 2^(e-150); unit 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (abs >> 23) - 112u;
    uint32_t m = abs & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

void oracle_f16_to_f32_n(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = oracle_f16_to_f32(src[i]);
}

void oracle_f32_to_f16_rne_n(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_f16_rne(src[i]);
}

/* ======================================================================== */
/* exp / tanh / activations                                                 */
/* ======================================================================== */

static float pow2i(int k) { /* 2^k for k in [-126, 127] */
    uint32_t bits = (uint32_t)(k + 127) << 23;
    float v;
    memcpy(&v, &bits, sizeof v);
    return v;
}

/* binary32 exp by Cody & Waite argument reduction (Cody and Waite, "Software
 * Manual for the Elementary Functions", 1980: x = n ln2 + r with ln2 split
 * into a 9-bit head and a tail so n*head is exact) and the degree-7 Taylor
 * polynomial of e^r on |r| <= ln2/2 (truncation < 2^-27 relative) in Horner
 * form with fused multiply-adds.  Only IEEE fma, floor and exact powers of
 * two are used (C99 fmaf is a correctly rounded fused multiply-add), so the
 * same steps give the same bits on the GPU.  The reference evaluates
 * Metal's exp (crates/atlas-metal/src/kernels.metal:27-36, 742-750); its
 * bits are not pinned, so this function is pinned against float64 exp
 * (tests/test_oracle_pins.py: faithful, < 1 ulp). */
float oracle_expf(float x) {
    if (x != x) return x;
    if (x > 89.0f) return INFINITY;
    if (x < -104.0f) return 0.0f;
    const float log2e = 1.44269502162933349609375f; /* nearest f32 to log2(e) */
    const float ln2_hi = 0.693359375f;              /* 355/512 */
    const float ln2_lo = -2.12194440e-4f;           /* ln2 - ln2_hi */
    float fn = floorf(fmaf(x, log2e, 0.5f));
    int n = (int)fn;
    float r = fmaf(-fn, ln2_lo, fmaf(-fn, ln2_hi, x));
    float p = 1.0f / 5040.0f;
    p = fmaf(p, r, 1.0f / 720.0f);
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    if (n > 127) return (p * pow2i(127)) * pow2i(n - 127);
    if (n < -126) return (p * pow2i(n + 100)) * pow2i(-100);
    return p * pow2i(n);
}

/* atlas_tanh_f32 (crates/atlas-metal/src/kernels.metal:742-750): saturate at
 * |x| >= 10, otherwise (e^{2x} - 1) / (e^{2x} + 1). */
float oracle_tanhf(float value) {
    if (value >= 10.0f) return 1.0f;
    if (value <= -10.0f) return -1.0f;
    float e = oracle_expf(2.0f * value);
    return (e - 1.0f) / (e + 1.0f);
}

/* silu_f32 (kernels.metal:27-36) and the CPU oracle
 * `value / (1.0 + (-value).exp())` (crates/atlas-ops/tests/phase_02_operators.rs:88-92). */
float oracle_silu(float x) { return x / (1.0f + oracle_expf(-x)); }

/* gelu_f32 (kernels.metal:752-767): tanh-GELU with the inf guard.  Order:
 * a = c0 * (x + ((c1 * x) * x) * x); g = (0.5 * x) * (1 + tanh(a)). */
float oracle_gelu_tanh(float x) {
    float argument = 0.7978845608f * (x + 0.044715f * x * x * x);
    if (isinf(argument)) return argument > 0.0f ? x : 0.0f;
    return 0.5f * x * (1.0f + oracle_tanhf(argument));
}

void oracle_silu_f32(const float *input, float *output, size_t n) {
    for (size_t i = 0; i < n; ++i) output[i] = oracle_silu(input[i]);
}

void oracle_gelu_f32(const float *input, float *output, size_t n) {
    for (size_t i = 0; i < n; ++i) output[i] = oracle_gelu_tanh(input[i]);
}

/* SwiGLU: silu_f32 then vector_multiply_f32 (kernels.metal:27-36, 64-69;
 * Llama decode crates/atlas-model/src/executor.rs:1318-1327).  The activated
 * value is an f32 intermediate, so fusing changes nothing. */
void oracle_swiglu_f32(const float *gate, const float *up, float *output, size_t n) {
    for (size_t i = 0; i < n; ++i) output[i] = oracle_silu(gate[i]) * up[i];
}

/* FP16 storage, FP32 math: exact widening, f32 result rounded RNE. */
void oracle_swiglu_f16(const uint16_t *gate, const uint16_t *up, uint16_t *output,
                       size_t n) {
    for (size_t i = 0; i < n; ++i) {
        float g = oracle_silu(oracle_f16_to_f32(gate[i]));
        output[i] = oracle_f32_to_f16_rne(g * oracle_f16_to_f32(up[i]));
    }
}

/* gelu_multiply_f32 (kernels.metal:773-784): gelu(gate) * up. */
void oracle_geglu_f32(const float *gate, const float *up, float *output, size_t n) {
    for (size_t i = 0; i < n; ++i) output[i] = oracle_gelu_tanh(gate[i]) * up[i];
}

/* PLE gating: gelu(gate) * ple[token * ple_row_stride + ple_offset + lane]
 * (ple_gelu_multiply_offset_f32 kernels.metal:790-801 for one token and
 * vector_multiply_offset_batch_f32 kernels.metal:83-92 for a batch). */
void oracle_geglu_offset_f32(const float *gate, const float *ple, float *output,
                             size_t ple_offset, size_t ple_row_stride, size_t width,
                             size_t rows) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t i = 0; i < width; ++i)
            output[r * width + i] =
                oracle_gelu_tanh(gate[r * width + i]) * ple[r * ple_row_stride + ple_offset + i];
}

/* ======================================================================== */
/* RMSNorm family                                                           */
/* ======================================================================== */

/* cpu_rms_norm (crates/atlas-ops/tests/phase_02_operators.rs:223-242):
 *   inverse = (sum_i x_i*x_i  /  hidden + epsilon).sqrt().recip()
 * with the sum a sequential left-to-right f32 fold (Rust's f32 Sum). */
float oracle_inverse_rms(const float *row, size_t hidden, float epsilon) {
    float sum = 0.0f;
    for (size_t i = 0; i < hidden; ++i) {
        float sq = row[i] * row[i];
        sum = sum + sq;
    }
    float mean = sum / (float)hidden;
    float root = sqrtf(mean + epsilon);
    return 1.0f / root;
}

/* y_i = (x_i * inverse) * w_i  (phase_02_operators.rs:238-240). */
void oracle_rms_norm_f32(const float *input, const float *weight, float *output,
                         size_t rows, size_t hidden, float epsilon) {
    for (size_t r = 0; r < rows; ++r) {
        const float *x = input + r * hidden;
        float inv = oracle_inverse_rms(x, hidden, epsilon);
        for (size_t i = 0; i < hidden; ++i) output[r * hidden + i] = x[i] * inv * weight[i];
    }
}

/* Post-norm residual epilogue gemma4_rms_residual_f32 (kernels.metal:183-214),
 * parity contract = rms_norm then vector_add (crates/atlas-metal/tests/
 * dispatch_fusion_parity.rs:185-258): n = (x*inv)*w is an f32 value (the
 * "volatile normalized" boundary), out = residual + n.  `normalized` may be
 * NULL; input/normalized/out may alias as in the reference call sites
 * (crates/atlas-model/src/gemma4_executor.rs:4492-4506). */
void oracle_rms_norm_residual_f32(const float *input, const float *weight,
                                  const float *residual, float *normalized, float *output,
                                  size_t rows, size_t hidden, float epsilon) {
    for (size_t r = 0; r < rows; ++r) {
        const float *x = input + r * hidden;
        float inv = oracle_inverse_rms(x, hidden, epsilon);
        for (size_t i = 0; i < hidden; ++i) {
            float n = x[i] * inv * weight[i];
            float res = residual[r * hidden + i];
            if (normalized) normalized[r * hidden + i] = n;
            output[r * hidden + i] = res + n;
        }
    }
}

/* Pre-norm add + RMSNorm (Llama: vector_add_f32 then rms_norm,
 * crates/atlas-model/src/executor.rs:1258-1286; AtlasModel::layer
 * crates/atlas-model/src/lib.rs:1076-1081): r = x + residual (stored),
 * y = rms_norm(r). */
void oracle_add_rms_norm_f32(const float *input, const float *residual, const float *weight,
                             float *residual_out, float *output, size_t rows, size_t hidden,
                             float epsilon) {
    for (size_t r = 0; r < rows; ++r) {
        float *rs = residual_out + r * hidden;
        for (size_t i = 0; i < hidden; ++i) rs[i] = input[r * hidden + i] + residual[r * hidden + i];
        float inv = oracle_inverse_rms(rs, hidden, epsilon);
        for (size_t i = 0; i < hidden; ++i) output[r * hidden + i] = rs[i] * inv * weight[i];
    }
}

/* gemma4_ple_rms_add_scale_f32 (kernels.metal:228-258):
 *   n = (x*inv)*w; state = (state + n) * scale. */
void oracle_rms_norm_add_scale_f32(const float *input, const float *weight, float *state,
                                   float scale, size_t rows, size_t hidden, float epsilon) {
    for (size_t r = 0; r < rows; ++r) {
        const float *x = input + r * hidden;
        float inv = oracle_inverse_rms(x, hidden, epsilon);
        for (size_t i = 0; i < hidden; ++i) {
            float n = x[i] * inv * weight[i];
            state[r * hidden + i] = (state[r * hidden + i] + n) * scale;
        }
    }
}

/* rms_norm_groups_in_place_stable_f32 (kernels.metal:897-917): per group,
 * m = max|v|; m == 0 -> zeros; s = sum (v/m)^2 sequential;
 * inv = (1/sqrt(s/width + eps/(m*m))) / m; v = (v*inv)*w.
 * The Metal kernel uses rsqrt; the oracle keeps the CPU operators'
 * sqrt-then-reciprocal (phase_02_operators.rs:233-235). */
void oracle_rms_norm_groups_stable_f32(float *values, const float *weight, size_t width,
                                       size_t groups, float epsilon) {
    for (size_t g = 0; g < groups; ++g) {
        float *v = values + g * width;
        float maximum = 0.0f;
        for (size_t i = 0; i < width; ++i) maximum = fmaxf(maximum, fabsf(v[i]));
        if (maximum == 0.0f) {
            for (size_t i = 0; i < width; ++i) v[i] = 0.0f;
            continue;
        }
        float sum = 0.0f;
        for (size_t i = 0; i < width; ++i) {
            float scaled = v[i] / maximum;
            float sq = scaled * scaled;
            sum = sum + sq;
        }
        float root = sqrtf(sum / (float)width + epsilon / (maximum * maximum));
        float inv = (1.0f / root) / maximum;
        for (size_t i = 0; i < width; ++i) v[i] = v[i] * inv * weight[i];
    }
}

/* The decode PLE chain's projection (gemma4_executor.rs:4184-4214):
 * matvec_f16 (kernels.metal:731-740: one row at a time, sum += input[k] *
 * float(W[o, k]) in column order), scalar_multiply_f32 by `scale`, then
 * rms_norm_groups_in_place_stable_f32 over `groups` groups of `width`. */
void oracle_ple_projection_f16(const float *input, const uint16_t *weights, const float *norm_weight,
                               float *output, size_t hidden, size_t width, size_t groups, float scale,
                               float epsilon) {
    for (size_t o = 0; o < groups * width; ++o) {
        float sum = 0.0f;
        for (size_t k = 0; k < hidden; ++k) {
            const float product = input[k] * oracle_f16_to_f32(weights[o * hidden + k]);
            sum = sum + product;
        }
        output[o] = sum * scale;
    }
    oracle_rms_norm_groups_stable_f32(output, norm_weight, width, groups, epsilon);
}

/* FP16-storage RMSNorm (config C2): exact widening, FP32 math as
 * oracle_rms_norm_f32, output rounded RNE to f16. */
void oracle_rms_norm_f16(const uint16_t *input, const uint16_t *weight, uint16_t *output,
                         size_t rows, size_t hidden, float epsilon) {
    for (size_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (size_t i = 0; i < hidden; ++i) {
            float x = oracle_f16_to_f32(input[r * hidden + i]);
            float sq = x * x;
            sum = sum + sq;
        }
        float inv = 1.0f / sqrtf(sum / (float)hidden + epsilon);
        for (size_t i = 0; i < hidden; ++i) {
            float x = oracle_f16_to_f32(input[r * hidden + i]);
            float y = x * inv * oracle_f16_to_f32(weight[i]);
            output[r * hidden + i] = oracle_f32_to_f16_rne(y);
        }
    }
}

/* FP16-storage pre-norm add + RMSNorm: r = rne16(x + residual) is the stored
 * residual stream; the norm reads that stored value back (the two-kernel
 * chain of executor.rs:1258-1286 with f16 buffers). */
void oracle_add_rms_norm_f16(const uint16_t *input, const uint16_t *residual,
                             const uint16_t *weight, uint16_t *residual_out, uint16_t *output,
                             size_t rows, size_t hidden, float epsilon) {
    for (size_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (size_t i = 0; i < hidden; ++i) {
            float a = oracle_f16_to_f32(input[r * hidden + i]);
            float b = oracle_f16_to_f32(residual[r * hidden + i]);
            uint16_t stored = oracle_f32_to_f16_rne(a + b);
            residual_out[r * hidden + i] = stored;
            float x = oracle_f16_to_f32(stored);
            float sq = x * x;
            sum = sum + sq;
        }
        float inv = 1.0f / sqrtf(sum / (float)hidden + epsilon);
        for (size_t i = 0; i < hidden; ++i) {
            float x = oracle_f16_to_f32(residual_out[r * hidden + i]);
            float y = x * inv * oracle_f16_to_f32(weight[i]);
            output[r * hidden + i] = oracle_f32_to_f16_rne(y);
        }
    }
}

/* ======================================================================== */
/* RoPE                                                                     */
/* ======================================================================== */

/* gemma4_rope_angle (crates/atlas-model/src/gemma4_executor.rs:622-633):
 * pair >= rotary/2 -> 0; else pos / theta^((2*pair)/rotary) / factor,
 * all in f32 with the host libm powf. */
float oracle_gemma4_rope_angle(size_t position, size_t pair, size_t rotary, float theta,
                               float frequency_factor) {
    if (pair >= rotary / 2) return 0.0f;
    return (float)position / powf(theta, (float)(pair * 2) / (float)rotary) / frequency_factor;
}

/* Prefill table layout [token][rope_pairs] (gemma4_executor.rs:3494-3519). */
void oracle_rope_tables_gemma4(const uint32_t *positions, size_t tokens, size_t rope_pairs,
                               size_t rotary, float theta, const float *frequency_factors,
                               float *cos_out, float *sin_out) {
    for (size_t t = 0; t < tokens; ++t)
        for (size_t p = 0; p < rope_pairs; ++p) {
            float factor = frequency_factors ? frequency_factors[p] : 1.0f;
            float angle = oracle_gemma4_rope_angle(positions[t], p, rotary, theta, factor);
            cos_out[t * rope_pairs + p] = cosf(angle);
            sin_out[t * rope_pairs + p] = sinf(angle);
        }
}

/* write_rope_tables / AtlasModel::rope (crates/atlas-model/src/executor.rs:
 * 632-647, crates/atlas-model/src/lib.rs:1168-1180):
 * angle = pos / theta^((2*pair)/head_dim), layout [token][head_dim/2]. */
void oracle_rope_tables_llama(const uint32_t *positions, size_t tokens, size_t head_dim,
                              float theta, float *cos_out, float *sin_out) {
    size_t pairs = head_dim / 2;
    for (size_t t = 0; t < tokens; ++t)
        for (size_t p = 0; p < pairs; ++p) {
            float angle = (float)positions[t] / powf(theta, (float)(p * 2) / (float)head_dim);
            cos_out[t * pairs + p] = cosf(angle);
            sin_out[t * pairs + p] = sinf(angle);
        }
}

/* cpu_rope (crates/atlas-ops/tests/phase_02_operators.rs:262-272) = the
 * NeuralOps::rope contract: interleaved pairs, one cos/sin row shared by
 * every input row. */
void oracle_rope_interleaved_f32(const float *input, size_t rows, size_t hidden,
                                 const float *cosine, const float *sine, float *output) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t p = 0; p < hidden / 2; ++p) {
            size_t b = r * hidden + p * 2;
            float x0 = input[b], x1 = input[b + 1];
            float c = cosine[p], s = sine[p];
            output[b] = x0 * c - x1 * s;
            output[b + 1] = x0 * s + x1 * c;
        }
}

/* Llama half-split RoPE: the net effect of rope_half_to_interleaved_f32,
 * rope_f32, rope_interleaved_to_half_f32 (kernels.metal:940-949, 972-994;
 * executor.rs:1120-1166; AtlasModel::rope lib.rs:1168-1217):
 *   out[p] = x[p]*c - x[p+d/2]*s;  out[p+d/2] = x[p]*s + x[p+d/2]*c,
 * with per-token tables cos/sin[token*rope_stride + p]. */
void oracle_rope_half_f32(const float *input, const float *cosine, const float *sine,
                          float *output, size_t tokens, size_t heads, size_t head_dim,
                          size_t rope_stride) {
    size_t half = head_dim / 2;
    for (size_t t = 0; t < tokens; ++t)
        for (size_t h = 0; h < heads; ++h) {
            size_t b = (t * heads + h) * head_dim;
            for (size_t p = 0; p < half; ++p) {
                float x0 = input[b + p], x1 = input[b + p + half];
                float c = cosine[t * rope_stride + p], s = sine[t * rope_stride + p];
                output[b + p] = x0 * c - x1 * s;
                output[b + p + half] = x0 * s + x1 * c;
            }
        }
}

void oracle_rope_half_f16(const uint16_t *input, const float *cosine, const float *sine,
                          uint16_t *output, size_t tokens, size_t heads, size_t head_dim,
                          size_t rope_stride) {
    size_t half = head_dim / 2;
    for (size_t t = 0; t < tokens; ++t)
        for (size_t h = 0; h < heads; ++h) {
            size_t b = (t * heads + h) * head_dim;
            for (size_t p = 0; p < half; ++p) {
                float x0 = oracle_f16_to_f32(input[b + p]);
                float x1 = oracle_f16_to_f32(input[b + p + half]);
                float c = cosine[t * rope_stride + p], s = sine[t * rope_stride + p];
                output[b + p] = oracle_f32_to_f16_rne(x0 * c - x1 * s);
                output[b + p + half] = oracle_f32_to_f16_rne(x0 * s + x1 * c);
            }
        }
}

/* gemma4_qk_norm_rope_fused_batch_f32 (kernels.metal:1098-1142), the exact
 * oracle kernel: per (token, head) unit over Q heads then the optional single
 * K head, s = sum x^2 sequential, inv = 1/sqrt(s/d + eps) (CPU operator
 * semantics, phase_02_operators.rs:233-235), x0 = (x[p]*inv)*w[p],
 * x1 = (x[p+d/2]*inv)*w[p+d/2], out[p] = x0*c - x1*s, out[p+d/2] = x0*s + x1*c,
 * cos/sin[token*rope_stride + p]. */
void oracle_qk_norm_rope_f32(const float *q, const float *k, const float *q_weight,
                             const float *k_weight, const float *cosine, const float *sine,
                             float *q_out, float *k_out, size_t tokens, size_t q_heads,
                             int has_key, size_t head_dim, size_t rope_stride, float epsilon) {
    size_t half = head_dim / 2;
    size_t total = q_heads + (has_key ? 1 : 0);
    for (size_t t = 0; t < tokens; ++t)
        for (size_t local = 0; local < total; ++local) {
            int key = local >= q_heads;
            const float *in = key ? k + t * head_dim : q + (t * q_heads + local) * head_dim;
            float *out = key ? k_out + t * head_dim : q_out + (t * q_heads + local) * head_dim;
            const float *w = key ? k_weight : q_weight;
            float inv = oracle_inverse_rms(in, head_dim, epsilon);
            for (size_t p = 0; p < half; ++p) {
                float x0 = in[p] * inv * w[p];
                float x1 = in[p + half] * inv * w[p + half];
                float c = cosine[t * rope_stride + p], s = sine[t * rope_stride + p];
                /* both outputs are computed before either store: in == out is allowed */
                float o0 = x0 * c - x1 * s;
                float o1 = x0 * s + x1 * c;
                out[p] = o0;
                out[p + half] = o1;
            }
        }
}

/* ======================================================================== */
/* Gathers and block dequantisation                                         */
/* ======================================================================== */

/* Q4_0 (crates/atlas-core/src/gguf.rs:418-429): 18-byte block = f16 d (LE)
 * + 16 bytes; value i < 16 uses the low nibble of byte i, value i >= 16 the
 * high nibble of byte i-16; v = f32(nibble - 8) * f32(d)  (exact in f32). */
void oracle_dequant_q4_0_block(const uint8_t *block, float *out32) {
    float d = oracle_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
    for (int i = 0; i < 32; ++i) {
        uint8_t nibble = i < 16 ? (block[2 + i] & 15) : (block[2 + i - 16] >> 4);
        out32[i] = (float)((int)nibble - 8) * d;
    }
}

/* Q8_0 (crates/atlas-core/src/gguf.rs:431-435): 34-byte block = f16 d (LE)
 * then 32 signed bytes; v = f32((int8)q) * d (exact in f32: 8 x 11 bits). */
void oracle_dequant_q8_0_block(const uint8_t *block, float *out32) {
    float d = oracle_f16_to_f32((uint16_t)(block[0] | (block[1] << 8)));
    for (int i = 0; i < 32; ++i) out32[i] = (float)(int8_t)block[2 + i] * d;
}

/* Q6_K (crates/atlas-core/src/gguf.rs:384-413): 210-byte super-block =
 * ql[128] | qh[64] | scales[16] (i8) | d (f16 at byte 208).  For i < 256:
 * half = i/128, w = i%128, stream = w/32, lane = w%32;
 * low = nibble of ql[half*64 + lane + (stream odd ? 32 : 0)] (high nibble
 * when stream >= 2); high = (qh[half*32 + lane] >> 2*stream) & 3;
 * v = (f32(((high<<4)|low) - 32) * f32(scales[half*8 + lane/16 + 2*stream])) * d. */
void oracle_dequant_q6_k_block(const uint8_t *block, float *out256) {
    float d = oracle_f16_to_f32((uint16_t)(block[208] | (block[209] << 8)));
    const uint8_t *ql = block, *qh = block + 128;
    const int8_t *scales = (const int8_t *)(block + 192);
    for (int i = 0; i < 256; ++i) {
        int half = i / 128, within = i % 128, stream = within / 32, lane = within % 32;
        uint8_t packed = ql[half * 64 + lane + ((stream & 1) ? 32 : 0)];
        uint8_t low = stream >= 2 ? (packed >> 4) : (packed & 15);
        uint8_t high = (qh[half * 32 + lane] >> (stream * 2)) & 3;
        float scale = (float)scales[half * 8 + lane / 16 + stream * 2];
        out256[i] = (float)((int)((high << 4) | low) - 32) * scale * d;
    }
}

/* Independent decoder in llama.cpp's loop order (half, lane, stream), kept
 * apart from the production-order decoder exactly as the reference does
 * (crates/atlas-core/tests/phase_11a_gguf.rs:11-31). */
void oracle_dequant_q6_k_block_llama_order(const uint8_t *block, float *out256) {
    float d = oracle_f16_to_f32((uint16_t)(block[208] | (block[209] << 8)));
    for (int half = 0; half < 2; ++half)
        for (int lane = 0; lane < 32; ++lane) {
            uint8_t qh = block[128 + half * 32 + lane];
            for (int stream = 0; stream < 4; ++stream) {
                uint8_t ql = block[half * 64 + lane + ((stream % 2 == 1) ? 32 : 0)];
                uint8_t low = stream < 2 ? (ql & 0x0f) : (ql >> 4);
                uint8_t high = (qh >> (stream * 2)) & 0x03;
                float scale = (float)(int8_t)block[192 + half * 8 + stream * 2 + lane / 16];
                out256[half * 128 + stream * 32 + lane] =
                    (float)((int)((high << 4) | low) - 32) * scale * d;
            }
        }
}

/* embedding_lookup_f32 (kernels.metal:94-104): out[t, j] = table[id*h + j],
 * 0.0 when id >= vocab. */
void oracle_embed_f32(const float *table, const uint32_t *ids, float *output, size_t vocab,
                      size_t hidden, size_t tokens) {
    for (size_t t = 0; t < tokens; ++t) {
        uint32_t id = ids[t];
        for (size_t j = 0; j < hidden; ++j)
            output[t * hidden + j] = id < vocab ? table[(size_t)id * hidden + j] : 0.0f;
    }
}

/* embedding_lookup_q4_0 + scalar_multiply_f32 (kernels.metal:653-656, 16-25;
 * gemma4_executor.rs:4145-4161): out = deq * scale (one rounding).  As in
 * the reference kernel, rows whose id >= vocab are left untouched. */
void oracle_embed_q4_0(const uint8_t *table, const uint32_t *ids, float *output, size_t vocab,
                       size_t hidden, size_t tokens, float scale) {
    size_t blocks = hidden / 32;
    float tmp[32];
    for (size_t t = 0; t < tokens; ++t) {
        uint32_t id = ids[t];
        if (id >= vocab) continue;
        for (size_t b = 0; b < blocks; ++b) {
            oracle_dequant_q4_0_block(table + ((size_t)id * blocks + b) * 18, tmp);
            for (int i = 0; i < 32; ++i) output[t * hidden + b * 32 + i] = tmp[i] * scale;
        }
    }
}

/* embedding_lookup_q8_0 (kernels.metal:658-661; the Llama resident embedding
 * for Q8_0 tables, crates/atlas-model/src/executor.rs:1541-1549), then the
 * optional scalar_multiply_f32 by `scale` (1 for the Llama path). */
void oracle_embed_q8_0(const uint8_t *table, const uint32_t *ids, float *output, size_t vocab,
                       size_t hidden, size_t tokens, float scale) {
    size_t blocks = hidden / 32;
    float tmp[32];
    for (size_t t = 0; t < tokens; ++t) {
        uint32_t id = ids[t];
        if (id >= vocab) continue;
        for (size_t b = 0; b < blocks; ++b) {
            oracle_dequant_q8_0_block(table + ((size_t)id * blocks + b) * 34, tmp);
            for (int i = 0; i < 32; ++i) output[t * hidden + b * 32 + i] = tmp[i] * scale;
        }
    }
}

/* embedding_lookup_q6_k + scalar_multiply_f32 (kernels.metal:663-692). */
void oracle_embed_q6_k(const uint8_t *table, const uint32_t *ids, float *output, size_t vocab,
                       size_t hidden, size_t tokens, float scale) {
    size_t blocks = hidden / 256;
    float tmp[256];
    for (size_t t = 0; t < tokens; ++t) {
        uint32_t id = ids[t];
        if (id >= vocab) continue;
        for (size_t b = 0; b < blocks; ++b) {
            oracle_dequant_q6_k_block(table + ((size_t)id * blocks + b) * 210, tmp);
            for (int i = 0; i < 256; ++i) output[t * hidden + b * 256 + i] = tmp[i] * scale;
        }
    }
}

/* Gemma PLE composition (gemma4_executor.rs:4162-4237 decode, 3555-3631
 * prefill; gemma4_combine_ple crates/atlas-model/src/lib.rs:206-219):
 *   lookup = deq(PLE[id])[l*width + i] * embedding_scale   (x sqrt(256))
 *   out    = (lookup + projection[t, l, i]) * output_scale  (x 1/sqrt(2))
 * Each step rounds once, in that order.  id >= vocab leaves the row untouched. */
static void ple_common(const uint8_t *table, const uint32_t *ids, const float *projection,
                       float *output, size_t vocab, size_t layers, size_t width, size_t tokens,
                       float embedding_scale, float output_scale, int q6) {
    size_t row = layers * width;
    size_t qk = q6 ? 256 : 32, bytes = q6 ? 210 : 18;
    size_t blocks = row / qk;
    float tmp[256];
    for (size_t t = 0; t < tokens; ++t) {
        uint32_t id = ids[t];
        if (id >= vocab) continue;
        for (size_t b = 0; b < blocks; ++b) {
            const uint8_t *blk = table + ((size_t)id * blocks + b) * bytes;
            if (q6)
                oracle_dequant_q6_k_block(blk, tmp);
            else
                oracle_dequant_q4_0_block(blk, tmp);
            for (size_t i = 0; i < qk; ++i) {
                size_t j = t * row + b * qk + i;
                float lookup = tmp[i] * embedding_scale;
                float sum = lookup + projection[j];
                output[j] = sum * output_scale;
            }
        }
    }
}

void oracle_ple_q4_0(const uint8_t *table, const uint32_t *ids, const float *projection,
                     float *output, size_t vocab, size_t layers, size_t width, size_t tokens,
                     float embedding_scale, float output_scale) {
    ple_common(table, ids, projection, output, vocab, layers, width, tokens, embedding_scale,
               output_scale, 0);
}

void oracle_ple_q6_k(const uint8_t *table, const uint32_t *ids, const float *projection,
                     float *output, size_t vocab, size_t layers, size_t width, size_t tokens,
                     float embedding_scale, float output_scale) {
    ple_common(table, ids, projection, output, vocab, layers, width, tokens, embedding_scale,
               output_scale, 1);
}

/* gemma4_combine_ple (crates/atlas-model/src/lib.rs:206-219):
 * (identity + context) * 0.707_106_77. */
void oracle_combine_ple(const float *identity, const float *context, float *output, size_t n) {
    const float inv_sqrt2 = 0.70710677f;
    for (size_t i = 0; i < n; ++i) output[i] = (identity[i] + context[i]) * inv_sqrt2;
}

/* ======================================================================== */
/* elementwise helpers (vector_add_f32 / vector_multiply_f32 /              */
/* scalar_multiply_f32, kernels.metal:5-25, 64-69)                          */
/* ======================================================================== */

void oracle_add_f32(const float *lhs, const float *rhs, float *output, size_t n) {
    for (size_t i = 0; i < n; ++i) output[i] = lhs[i] + rhs[i];
}

void oracle_multiply_f32(const float *lhs, const float *rhs, float *output, size_t n) {
    for (size_t i = 0; i < n; ++i) output[i] = lhs[i] * rhs[i];
}

void oracle_scale_f32(const float *input, float scalar, float *output, size_t n) {
    for (size_t i = 0; i < n; ++i) output[i] = input[i] * scalar;
}

/* ======================================================================== */
/* RMS-folded Q4_0 decode projections                                       */
/* ======================================================================== */

/* The reference's own CPU oracle for the _rms matvec kernels
 * (crates/atlas-metal/tests/matvec_rms_fused_parity.rs:51-80), in f32:
 * cpu_rms_normalize -- mean_sq = (sequential sum of x*x) / n,
 * inv = 1 / sqrt(mean_sq + eps), normalized = (x * w) * inv -- then
 * cpu_q4_matvec -- acc += normalized[k] * dequantize_block(...)[lane],
 * blocks and lanes in order.  rms_weight == NULL: the plain matvec of x. */
void oracle_matvec_q4_0_rms_ref(const float *input, const uint8_t *weights, const float *rms_weight,
                                size_t input_width, size_t output_width, float epsilon, float *output) {
    const size_t blocks = input_width / 32;
    float normalized[8192];
    if (input_width > 8192) return;
    if (rms_weight) {
        float sum = 0.0f;
        for (size_t k = 0; k < input_width; ++k) sum = sum + input[k] * input[k];
        const float mean_sq = sum / (float)input_width;
        const float inv = 1.0f / sqrtf(mean_sq + epsilon);
        for (size_t k = 0; k < input_width; ++k) normalized[k] = input[k] * rms_weight[k] * inv;
    } else {
        for (size_t k = 0; k < input_width; ++k) normalized[k] = input[k];
    }
    float block[32];
    for (size_t row = 0; row < output_width; ++row) {
        float acc = 0.0f;
        for (size_t b = 0; b < blocks; ++b) {
            oracle_dequant_q4_0_block(weights + (row * blocks + b) * 18, block);
            for (size_t lane = 0; lane < 32; ++lane) acc = acc + normalized[b * 32 + lane] * block[lane];
        }
        output[row] = acc;
    }
}

/* The same projection in float64 from the same f32 inputs: the exact value
 * of inv_rms(x) * sum_k (x_k * w_k) * deq_k up to float64 rounding, and
 * magnitude[o] = inv * sum_k 16 * |x_k * w_k * d_block(k)|, a bound on every
 * partial sum an f32 evaluation forms (codes q in [0, 15], offset 8), i.e.
 * the scale of its rounding error in any summation order. */
void oracle_matvec_q4_0_rms_f64(const float *input, const uint8_t *weights, const float *rms_weight,
                                size_t input_width, size_t output_width, float epsilon, double *output,
                                double *magnitude) {
    const size_t blocks = input_width / 32;
    double inv = 1.0;
    if (rms_weight) {
        double sum = 0.0;
        for (size_t k = 0; k < input_width; ++k) sum += (double)input[k] * (double)input[k];
        inv = 1.0 / sqrt(sum / (double)input_width + (double)epsilon);
    }
    float block[32];
    for (size_t row = 0; row < output_width; ++row) {
        double acc = 0.0, mag = 0.0;
        for (size_t b = 0; b < blocks; ++b) {
            const uint8_t *blk = weights + (row * blocks + b) * 18;
            oracle_dequant_q4_0_block(blk, block);
            const double d = fabs((double)oracle_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8))));
            for (size_t lane = 0; lane < 32; ++lane) {
                const size_t k = b * 32 + lane;
                const double y = (double)input[k] * (rms_weight ? (double)rms_weight[k] : 1.0);
                acc += y * (double)block[lane];
                mag += 16.0 * fabs(y) * d;
            }
        }
        output[row] = acc * inv;
        magnitude[row] = mag * inv;
    }
}

/* ======================================================================== */
/* KV-cache append, fused V RMSNorm, Q8_0 / Q4_0 encoders                   */
/* ======================================================================== */

/* Restates kv_append_decode_{f32,q8_0,q4_0}[_batch] (crates/atlas-metal/src/
 * kernels.metal:1197-1344) and the unfused V norm
 * rms_norm_groups_in_place_unweighted_f32 (:919-929) that the _vnorm
 * kernels fold in (:1346-1436): inv = 1 / sqrt(sum v^2 / width + eps) with
 * the sum in index order (IEEE sqrt and division; Metal's rsqrt cannot be
 * reproduced off Apple hardware), v' = v * inv. */
static float kv_inv_rms(const float *v, size_t width, float epsilon) {
    float s = 0.0f;
    for (size_t i = 0; i < width; ++i) s = s + v[i] * v[i];
    return 1.0f / sqrtf(s / (float)width + epsilon);
}

/* Q8_0 block (kv_append_decode_q8_0, kernels.metal:1222-1231): m = max|v|,
 * scale = m == 0 ? 0 : m / 127, code = round-half-away(clamp(v / scale,
 * -127, 127)), f16 scale with IEEE RNE. */
void oracle_encode_q8_0_block(const float *v, uint8_t *out34) {
    float maximum = 0.0f;
    for (int i = 0; i < 32; ++i) maximum = fmaxf(maximum, fabsf(v[i]));
    const float scale = maximum == 0.0f ? 0.0f : maximum / 127.0f;
    const uint16_t bits = oracle_f32_to_f16_rne(scale);
    out34[0] = (uint8_t)bits;
    out34[1] = (uint8_t)(bits >> 8);
    for (int i = 0; i < 32; ++i) {
        int code = 0;
        if (scale != 0.0f) code = (int)roundf(fminf(fmaxf(v[i] / scale, -127.0f), 127.0f));
        out34[2 + i] = (uint8_t)(int8_t)code;
    }
}

/* Q4_0 block (kv_append_decode_q4_0, kernels.metal:1247-1256): the first
 * value with the largest |v| (strictly greater replaces) is the signed
 * maximum s, scale = s / -8, code = clamp(trunc(v / scale + 8.5), 0, 15)
 * (NaN -> 0), byte j = code_j | code_{j+16} << 4, f16 scale with IEEE RNE. */
static int q4_code(float v, float scale) {
    if (scale == 0.0f) return 0;
    const float t = v / scale + 8.5f;
    if (t >= 15.0f) return 15;
    if (t > 0.0f) return (int)t;
    return 0;
}

void oracle_encode_q4_0_block(const float *v, uint8_t *out18) {
    float maximum = 0.0f, signed_maximum = 0.0f;
    for (int i = 0; i < 32; ++i) {
        if (fabsf(v[i]) > maximum) {
            maximum = fabsf(v[i]);
            signed_maximum = v[i];
        }
    }
    const float scale = maximum == 0.0f ? 0.0f : signed_maximum / -8.0f;
    const uint16_t bits = oracle_f32_to_f16_rne(scale);
    out18[0] = (uint8_t)bits;
    out18[1] = (uint8_t)(bits >> 8);
    for (int i = 0; i < 16; ++i)
        out18[2 + i] = (uint8_t)(q4_code(v[i], scale) | (q4_code(v[i + 16], scale) << 4));
}

/* format: 0 f32, 1 Q8_0, 2 Q4_0.  Tokens with positions[t] >= capacity are
 * skipped; the value input is not modified. */
void oracle_kv_append(int format, const float *key, const float *value, uint8_t *cache, size_t kv_width,
                      size_t capacity, const uint32_t *positions, size_t tokens, int vnorm, float epsilon) {
    float v[4096];
    if (kv_width > 4096) return;
    const size_t row = format == 0 ? kv_width * 4 : (kv_width / 32) * (format == 1 ? 34 : 18);
    for (size_t t = 0; t < tokens; ++t) {
        const size_t position = positions[t];
        if (position >= capacity) continue;
        const float *k = key + t * kv_width;
        memcpy(v, value + t * kv_width, kv_width * sizeof(float));
        if (vnorm) {
            const float inv = kv_inv_rms(v, kv_width, epsilon);
            for (size_t i = 0; i < kv_width; ++i) v[i] = v[i] * inv;
        }
        uint8_t *kc = cache + position * row;
        uint8_t *vc = cache + (capacity + position) * row;
        if (format == 0) {
            memcpy(kc, k, kv_width * sizeof(float));
            memcpy(vc, v, kv_width * sizeof(float));
        } else {
            const size_t bytes = format == 1 ? 34 : 18;
            for (size_t b = 0; b < kv_width / 32; ++b) {
                if (format == 1) {
                    oracle_encode_q8_0_block(k + 32 * b, kc + bytes * b);
                    oracle_encode_q8_0_block(v + 32 * b, vc + bytes * b);
                } else {
                    oracle_encode_q4_0_block(k + 32 * b, kc + bytes * b);
                    oracle_encode_q4_0_block(v + 32 * b, vc + bytes * b);
                }
            }
        }
    }
}


/* ======================================================================== */
/* logits: soft cap and argmax                                              */
/* ======================================================================== */

/* Coefficients of the Maclaurin series of tanh,
 * tanh(a) = sum_n 2^{2n} (2^{2n} - 1) B_{2n} a^{2n-1} / (2n)!  (B = Bernoulli
 * numbers): -1/3, 2/15, -17/315, 62/2835, -1382/155925, 21844/6081075,
 * -929569/638512875, 6404582/10854718875, -443861162/1856156927625, each
 * rounded to binary32. */
static const float kTanhSeries[9] = {
    -0x1.555556p-2f, 0x1.111112p-3f, -0x1.ba1ba2p-5f, 0x1.664f48p-6f, -0x1.226e36p-7f,
    0x1.d6d3d0p-9f,  -0x1.7da364p-10f, 0x1.355824p-11f, -0x1.f57d78p-13f,
};

/* tanh for the logit soft cap.  The reference evaluates Metal's built-in
 * tanh on the GPU (softcap_f32, crates/atlas-metal/src/kernels.metal:931-934)
 * and Rust's f32::tanh on the CPU (gemma4_softcap_logits,
 * crates/atlas-model/src/lib.rs:223-232); neither is reproducible here, so
 * this is a restated method pinned against float64: for |x| < 0.625 the
 * series above through a^19 (truncation < 2^-28 relative), evaluated as
 * a + (a*z)*P(z), z = a*a, in Horner form with fmaf; above, the identity
 * 1 - 2/(e^{2a} + 1) with oracle_expf, saturating to 1 once e^{2a}
 * overflows.  The sign is copied from x; NaN propagates.  Within 1.4 ulp of
 * float64 tanh over every binary32 input (tests/test_oracle_pins.py). */
float oracle_tanh_precise(float x) {
    const float a = fabsf(x);
    if (a < 0.625f) {
        const float z = a * a;
        float p = kTanhSeries[8];
        for (int i = 7; i >= 0; --i) p = fmaf(p, z, kTanhSeries[i]);
        return copysignf(fmaf(a * z, p, a), x);
    }
    const float e = oracle_expf(2.0f * a);
    return copysignf(1.0f - 2.0f / (e + 1.0f), x);
}

/* softcap_f32 (kernels.metal:931-934) = gemma4_softcap_logits
 * (crates/atlas-model/src/lib.rs:223-232): v = cap * tanh(v / cap), applied
 * to `n` values. */
void oracle_softcap_f32(const float *input, float *output, size_t n, float cap) {
    for (size_t i = 0; i < n; ++i) output[i] = cap * oracle_tanh_precise(input[i] / cap);
}

/* argmax_f32 (kernels.metal:2033-2066): every lane scans its stride with
 * `value >= best` from (-inf, 0) and the tree keeps the larger value, or the
 * larger index on equal values.  The result is therefore the largest index
 * holding the maximum of the non-NaN values (NaN compares false and is never
 * taken; +0 and -0 compare equal), and 0 when every value is NaN.  A single
 * left-to-right scan with the same `>=` gives the same index. */
uint32_t oracle_argmax_f32(const float *values, size_t count) {
    float best = -INFINITY;
    uint32_t id = 0;
    for (size_t i = 0; i < count; ++i) {
        if (values[i] >= best) {
            best = values[i];
            id = (uint32_t)i;
        }
    }
    return id;
}

/* The decode tail of the Gemma executor for `rows` sequences
 * (gemma4_executor.rs:4678-4688): softcap_f32 over each row of `count`
 * logits in place, then argmax_f32 of the capped row.  cap <= 0 skips the
 * soft cap (argmax only). */
void oracle_softcap_argmax_rows(float *logits, uint32_t *selected, size_t rows, size_t count, float cap) {
    for (size_t r = 0; r < rows; ++r) {
        float *row = logits + r * count;
        if (cap > 0.0f) oracle_softcap_f32(row, row, count, cap);
        selected[r] = oracle_argmax_f32(row, count);
    }
}
