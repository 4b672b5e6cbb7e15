// device_common.hpp -- shared device helpers for the gfx950 fused-op kernels.
//
// Every kernel translation unit is compiled with -ffp-contract=off and without
// fast-math, so each `a * b + c` below is two IEEE-rounded operations, exactly
// as the reference's Rust CPU operators evaluate them.  Division and square
// root must be correctly rounded as well (Rust's f32 `/` and `sqrt`): see
// fdiv_rn / sqrt_rn.  (HIP's __fsqrt_rn maps to the native ~1 ulp v_sqrt_f32
// unless OCML rounded operations are enabled, so it is not used.)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace atlas {

constexpr int kWave = 64;  // CDNA wavefront width

// IEEE binary32 division, correctly rounded: HIP's default lowering of '/'
// (v_div_scale / v_rcp / Newton steps / v_div_fmas / v_div_fixup).
__device__ __forceinline__ float fdiv_rn(float a, float b) { return a / b; }

// IEEE binary32 square root, correctly rounded.  llvm.sqrt.f32 under HIP's
// default -fhip-fp32-correctly-rounded-divide-sqrt.
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float pow2i(int k) {  // 2^k, k in [-126, 127]
    return __uint_as_float(static_cast<uint32_t>(k + 127) << 23);
}

// binary32 exp: Cody & Waite reduction x = n*ln2 + r (ln2 split into the
// 9-bit head 355/512 and its tail so n*head is exact), then the degree-7
// Taylor polynomial of e^r on |r| <= ln2/2 in Horner form with fused
// multiply-adds (each step one IEEE fma, correctly rounded), and the 2^n
// scale assembled in the exponent field.  Every step is an IEEE operation
// (fma, floor, exact power-of-two multiply), so the CPU oracle's restatement
// with C99 fmaf gives the same bits; the result is faithfully rounded
// (< 1 ulp against float64 exp over the finite range).
__device__ __forceinline__ float exp_f32(float x) {
    if (x != x) return x;
    if (x > 89.0f) return __builtin_inff();
    if (x < -104.0f) return 0.0f;
    const float log2e = 1.44269502162933349609375f;
    const float ln2_hi = 0.693359375f;
    const float ln2_lo = -2.12194440e-4f;
    const float fn = floorf(__builtin_fmaf(x, log2e, 0.5f));
    const int n = static_cast<int>(fn);
    const float r = __builtin_fmaf(-fn, ln2_lo, __builtin_fmaf(-fn, ln2_hi, x));
    float p = 1.0f / 5040.0f;
    p = __builtin_fmaf(p, r, 1.0f / 720.0f);
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    if (n > 127) return (p * pow2i(127)) * pow2i(n - 127);
    if (n < -126) return (p * pow2i(n + 100)) * pow2i(-100);
    return p * pow2i(n);
}

// tanh through its exponential identity with saturation at |x| >= 10
// (Atlas atlas_tanh_f32, crates/atlas-metal/src/kernels.metal:742-750).
__device__ __forceinline__ float tanh_f32(float v) {
    if (v >= 10.0f) return 1.0f;
    if (v <= -10.0f) return -1.0f;
    float e = exp_f32(2.0f * v);
    return fdiv_rn(e - 1.0f, e + 1.0f);
}

// x / (1 + e^-x)   (kernels.metal:27-36)
__device__ __forceinline__ float silu_f32(float x) { return fdiv_rn(x, 1.0f + exp_f32(-x)); }

// tanh-GELU with the overflow guard (kernels.metal:752-767):
// a = c0*(x + ((c1*x)*x)*x); inf(a) -> (a > 0 ? x : 0); else (0.5*x)*(1 + tanh(a)).
__device__ __forceinline__ float gelu_tanh_f32(float x) {
    float argument = 0.7978845608f * (x + 0.044715f * x * x * x);
    if (__builtin_isinf(argument)) return argument > 0.0f ? x : 0.0f;
    return 0.5f * x * (1.0f + tanh_f32(argument));
}

// 1 / sqrt(mean + eps) with the CPU operators' two roundings
// (phase_02_operators.rs:233-235: `.sqrt().recip()`).
__device__ __forceinline__ float inverse_rms(float sum, float hidden, float epsilon) {
    return fdiv_rn(1.0f, sqrt_rn(fdiv_rn(sum, hidden) + epsilon));
}

__device__ __forceinline__ float h2f(uint16_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, bits));
}

// Materialise an f32 value in a VGPR.  The empty asm (register constraint
// only, no instruction) stops instruction selection from folding the
// producing multiply into the f32 -> f16 conversion (v_fma_mix*_f16 rounds
// the exact product once, where the reference rounds to f32 first).
__device__ __forceinline__ float materialize(float v) {
    __asm__ volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ uint16_t f2h(float v) {  // IEEE RNE of the f32 value
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(materialize(v)));
}

// Sequential f32 fold of n4 (<= 64) float4 of squares from LDS into s, in
// index order.  A full chunk is straight-line code in groups of 8 float4:
// the next group's reads are issued before the current group's 32 adds, so
// LDS latency hides under the dependent add chain (~8 cycles per add).
__device__ __forceinline__ float fold_lds_chunk(const f32x4* p, uint32_t n4, float s) {
    if (n4 == 64) {
        f32x4 cur[8], nxt[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) cur[i] = p[i];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            if (g < 7) {
#pragma unroll
                for (int i = 0; i < 8; ++i) nxt[i] = p[8 * (g + 1) + i];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                s = s + cur[i].x;
                s = s + cur[i].y;
                s = s + cur[i].z;
                s = s + cur[i].w;
            }
            if (g < 7) {
#pragma unroll
                for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
            }
        }
        return s;
    }
#pragma unroll 8
    for (uint32_t k = 0; k < n4; ++k) {
        const f32x4 v = p[k];
        s = s + v.x;
        s = s + v.y;
        s = s + v.z;
        s = s + v.w;
    }
    return s;
}

}  // namespace atlas
