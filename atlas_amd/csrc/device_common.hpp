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
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Store cache policies (gfx950 buffer-instruction bits: sc0 = 1, nt = 2,
// sc1 = 16).  kPolicyWriteThrough = sc0 | sc1 | nt: system-scope,
// nontemporal -- the line is written through to memory at once instead of
// staying dirty in L2, so the kernel's end has no write-back left to drain.
// It pays where a kernel's bytes are mostly written (the token gathers write
// 7 bytes per byte read: Q4_0 at T = 4096 5.25 against 5.74 us with
// nontemporal stores); where reads dominate it costs (QK-norm + RoPE 15.4
// against 14.2 us, RMSNorm 9.4 against 8.8, GeGLU 49.5 against 47.8).
// sc0 | sc1 without nt timed faster per gather launch (4.99 against 5.25 us)
// but made the seven-op T = 4096 step 10.6 us slower (155.8 against 145.2):
// its writes are still draining while the next op runs.
constexpr int kPolicyNt = 2;
constexpr int kPolicyWriteThrough = 19;

// Buffer resource over `bytes` from a wavefront-uniform `base` (raw
// buffer, no swizzle): stores through it at a per-lane byte offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
template <int POL>
__device__ __forceinline__ void st_span4(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), rs, byte_off, 0, POL);
}
template <int POL>
__device__ __forceinline__ void st_span2(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off, float a, float b) {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{__float_as_uint(a), __float_as_uint(b)}, rs, byte_off, 0, POL);
}
template <int POL>
__device__ __forceinline__ void st_span1(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off, float a) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(a), rs, byte_off, 0, POL);
}

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
//
// The kernels stream HBM, so control flow is kept out of the math: the
// special ranges are selected after the fact instead of branched on (a
// branch per element costs an exec-mask round trip per wave and measured
// ~10 % of GeGLU's time).  exp_small_f32 is the form for arguments known to
// lie in (-87, 87), where no special range applies.
__device__ __forceinline__ float exp_reduced(float x, int& n) {
    const float log2e = 1.44269502162933349609375f;
    const float ln2_hi = 0.693359375f;
    const float ln2_lo = -2.12194440e-4f;
    // floor(x*log2e + 1/2), clamped so the integer conversion is defined for
    // every input.  One v_med3 (instead of a min and a max): the two clamps
    // differ only for NaN, whose result stays NaN through r either way, and
    // the clamp only acts for |x| > 138, whose results every caller selects
    // away.
    const float fn = __builtin_amdgcn_fmed3f(floorf(__builtin_fmaf(x, log2e, 0.5f)), -200.0f, 200.0f);
    n = static_cast<int>(fn);
    const float r = __builtin_fmaf(-fn, ln2_lo, __builtin_fmaf(-fn, ln2_hi, x));
    float p = 1.0f / 5040.0f;
    p = __builtin_fmaf(p, r, 1.0f / 720.0f);
    p = __builtin_fmaf(p, r, 1.0f / 120.0f);
    p = __builtin_fmaf(p, r, 1.0f / 24.0f);
    p = __builtin_fmaf(p, r, 1.0f / 6.0f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return p;
}

// e^x for |x| < 87 (n in [-125, 126], so p * 2^n is a normal number and the
// scale is exact: ldexp gives the product p * 2^n bit for bit, in one
// instruction instead of building 2^n and multiplying).  Outside that domain
// the value is meaningless and must be selected away by the caller.
__device__ __forceinline__ float exp_small_f32(float x) {
    int n;
    const float p = exp_reduced(x, n);
    return __builtin_ldexpf(p, n);
}

// e^x over the whole binary32 range.  Outside n in [-126, 127] the scale is
// split in two steps, (p * 2^127) * 2^(n-127) or (p * 2^(n+100)) * 2^-100,
// so the only rounding is the final (possibly subnormal) product; in range
// the second factor is 1.0.  NaN returns x, x > 89 returns +inf and
// x < -104 returns +0.
__device__ __forceinline__ float exp_f32(float x) {
    int n;
    const float p = exp_reduced(x, n);  // n in [-200, 200]
    const int s1 = n > 127 ? 127 : (n < -126 ? n + 100 : n);
    const int s2 = n > 127 ? n - 127 : (n < -126 ? -100 : 0);
    const float y = (p * pow2i(s1)) * pow2i(s2);
    const float big = x > 89.0f ? __builtin_inff() : y;
    const float out = x < -104.0f ? 0.0f : big;
    return x != x ? x : out;
}

// a / b in four operations instead of the IEEE sequence's ten, for the
// activations' in-range forms below: q0 = a * rcp(b), the exact residual
// fma(-q0, b, a), q = fma(residual, rcp(b), q0), and the sign of a (b > 0
// for every caller, so the quotient's sign is a's; this also keeps -0).
// Not correctly rounded in general -- v_rcp_f32 is within 1 ulp of 1/b,
// where Markstein's theorem needs the rounded reciprocal -- but equal to
// fdiv_rn bit for bit on every operand pair its callers pass: a GPU test
// (tests/test_gpu_division.py) runs tanh_with, gelu_finite_with and
// silu_small_with on every binary32 input of their domains with both
// divisions and finds no difference, and finds differences for the
// uncorrected product and for the form without the sign step.
__device__ __forceinline__ float div_inrange(float a, float b) {
    const float r = __builtin_amdgcn_rcpf(b);
    const float q0 = a * r;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, b, a), r, q0);
    return __builtin_copysignf(q, a);
}
struct DivIeee {
    __device__ static float div(float a, float b) { return fdiv_rn(a, b); }
};
struct DivInRange {
    __device__ static float div(float a, float b) { return div_inrange(a, b); }
};

// tanh through its exponential identity with saturation at |x| >= 10
// (Atlas atlas_tanh_f32, crates/atlas-metal/src/kernels.metal:742-750).
// Inside (-10, 10), 2v is inside (-20, 20), where exp_small_f32 is exact
// to exp_f32; outside, the quotient is computed and discarded.  NaN
// propagates through the quotient (with DivIeee; DivInRange takes finite v).
template <class D>
__device__ __forceinline__ float tanh_with(float v) {
    const float e = exp_small_f32(2.0f * v);
    const float q = D::div(e - 1.0f, e + 1.0f);
    // v >= 10 -> 1, v <= -10 -> -1, else q (NaN: the compare fails, q is NaN)
    return __builtin_fabsf(v) >= 10.0f ? __builtin_copysignf(1.0f, v) : q;
}
__device__ __forceinline__ float tanh_f32(float v) { return tanh_with<DivIeee>(v); }

// tanh for the logit soft cap, where small arguments must keep their
// relative accuracy (the (e-1)/(e+1) identity above cancels near 0).  Two
// ranges, the same IEEE steps as the CPU oracle's restatement:
//  - |x| < 0.625: the Maclaurin series of tanh through a^19,
//    a + (a*z)*P(z) with z = a*a and P in Horner form (fma);
//  - otherwise 1 - 2/(e^{2a} + 1), which saturates to 1 once e^{2a}
//    overflows; NaN propagates.
// Within 1.4 ulp of float64 tanh over every binary32 input.
__device__ __forceinline__ float tanh_series_abs(float a) {
    const float z = a * a;
    float p = -0x1.f57d78p-13f;  // -443861162/1856156927625
    p = __builtin_fmaf(p, z, 0x1.355824p-11f);   // 6404582/10854718875
    p = __builtin_fmaf(p, z, -0x1.7da364p-10f);  // -929569/638512875
    p = __builtin_fmaf(p, z, 0x1.d6d3d0p-9f);    // 21844/6081075
    p = __builtin_fmaf(p, z, -0x1.226e36p-7f);   // -1382/155925
    p = __builtin_fmaf(p, z, 0x1.664f48p-6f);    // 62/2835
    p = __builtin_fmaf(p, z, -0x1.ba1ba2p-5f);   // -17/315
    p = __builtin_fmaf(p, z, 0x1.111112p-3f);    // 2/15
    p = __builtin_fmaf(p, z, -0x1.555556p-2f);   // -1/3
    return __builtin_fmaf(a * z, p, a);
}
__device__ __forceinline__ float tanh_exp_abs(float a) {
    const float e = exp_f32(2.0f * a);
    return 1.0f - fdiv_rn(2.0f, e + 1.0f);
}
__device__ __forceinline__ bool tanh_series_range(float a) { return a < 0.625f; }

// x / (1 + e^-x)   (kernels.metal:27-36)
__device__ __forceinline__ float silu_f32(float x) { return fdiv_rn(x, 1.0f + exp_f32(-x)); }

// silu_f32 for |x| < 87, where exp_small_f32(-x) == exp_f32(-x) and the
// in-range division gives fdiv_rn's bits.
template <class D>
__device__ __forceinline__ float silu_small_with(float x) { return D::div(x, 1.0f + exp_small_f32(-x)); }
__device__ __forceinline__ float silu_small_f32(float x) { return silu_small_with<DivInRange>(x); }

// SiLU of N values held by each lane.  When every value of the wavefront
// lies in (-87, 87) -- all ordinary activations -- the straight-line
// in-range form runs; otherwise (huge inputs, inf, NaN) the full-range form
// runs for the whole wavefront.  One wave-uniform branch, same bits.
template <int N>
__device__ __forceinline__ void silu_lanes(float (&v)[N]) {
    bool small = true;
#pragma unroll
    for (int i = 0; i < N; ++i) small = small && __builtin_fabsf(v[i]) < 87.0f;
    if (__builtin_amdgcn_ballot_w64(!small) == 0) {
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = silu_small_f32(v[i]);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = silu_f32(v[i]);
    }
}

// tanh-GELU with the overflow guard (kernels.metal:752-767):
// a = c0*(x + ((c1*x)*x)*x); inf(a) -> (a > 0 ? x : 0); else (0.5*x)*(1 + tanh(a)).
__device__ __forceinline__ float gelu_argument(float x) { return 0.7978845608f * (x + 0.044715f * x * x * x); }
template <class D>
__device__ __forceinline__ float gelu_finite_with(float x, float argument) {
    return 0.5f * x * (1.0f + tanh_with<D>(argument));
}
__device__ __forceinline__ float gelu_finite_f32(float x, float argument) {
    return gelu_finite_with<DivIeee>(x, argument);
}
__device__ __forceinline__ float gelu_tanh_f32(float x) {
    const float argument = gelu_argument(x);
    const float g = gelu_finite_f32(x, argument);
    return __builtin_isinf(argument) ? (argument > 0.0f ? x : 0.0f) : g;
}

// tanh-GELU of N values held by each lane, with the bits of gelu_tanh_f32.
// The compiler lowers gelu_tanh_f32's overflow guard to a branch per value,
// which serialises the N exp/divide chains; here one wave-uniform test
// replaces it: when every argument of the wavefront is finite (every
// |x| < ~1.9e12, no NaN), the guard selects g for every value, so the
// straight-line form with the in-range division runs; otherwise the guarded
// IEEE form runs for the whole wavefront.
template <int N>
__device__ __forceinline__ void gelu_lanes(float (&v)[N]) {
    float argument[N];
    bool special = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        argument[i] = gelu_argument(v[i]);
        special = special || !(__builtin_fabsf(argument[i]) < __builtin_inff());
    }
    if (__builtin_amdgcn_ballot_w64(special) == 0) {
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = gelu_finite_with<DivInRange>(v[i], argument[i]);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] = gelu_tanh_f32(v[i]);
    }
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

// a * h with one rounding, where h is the low (HI = 0) or high (HI = 1)
// binary16 half of `pair`: v_fma_mix_f32 widens the half exactly inside the
// multiply and adds -0.0f (held in a register), which changes no product (a
// zero product keeps its sign) -- the bits of a * h2f(half), one VALU
// instruction instead of a conversion and a multiply.  (Written out because
// the compiler folds fma(a, b, -0) back into a multiply of the converted
// operand.)
template <int HI>
__device__ __forceinline__ float mul_f16_half(float a, uint32_t pair) {
    float r;
    const float neg_zero = -0.0f;
    if constexpr (HI)
        __asm__("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
                : "=v"(r) : "v"(a), "v"(pair), "s"(neg_zero));
    else
        __asm__("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[0,1,0]"
                : "=v"(r) : "v"(a), "v"(pair), "s"(neg_zero));
    return r;
}

// Sequential f32 fold of n4 (<= 64) float4 of squares from LDS into s, in
// index order.  A full chunk is straight-line code in groups of 8 float4:
// the next group's reads are issued before the current group's 32 adds, so
// LDS latency hides under the dependent add chain.  The scheduling barriers
// keep it that way: left alone, the scheduler interleaves each read just
// one float4 ahead of its adds, and the chain then waits on LDS latency
// (one wavefront on gfx950: 8.7 cycles per add, 6.6 with the barriers; a
// register-fed chain is 5.6).  The schedule holds with the groups written
// out here: the same loop moved into a template helper compiled to all reads
// hoisted ahead of the adds, spilled to AGPRs (QK-norm + RoPE at 4096 tokens
// 21.6 us against 14.2, the residual epilogue 20.1 against 13.7); check the
// ISA after any change to this function.
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
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                s = s + cur[i].x;
                s = s + cur[i].y;
                s = s + cur[i].z;
                s = s + cur[i].w;
            }
            __builtin_amdgcn_sched_barrier(0);
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

// ---------------------------------------------------------------------------
// Exact wave-parallel continuation of a sequential f32 fold.
//
// The CPU operators fold x_i*x_i left to right in f32, and the cancelling
// epilogues make that order observable, so the sum must come out bit-exact.
// A dependent add chain costs ~8 cycles per add; this computes the same
// bits with the chunk spread across the wavefront:
//
//  * The running sum s is a non-negative float in a binade [2^E, 2^(E+1)),
//    so it is an integer k of ulps u = 2^(E-23).  While the sum stays in the
//    binade, s + a rounds to s + round(a/u)*u: every addend contributes an
//    integer number of ulps that does not depend on s -- except at an exact
//    tie (a/u = m + 1/2), where round-half-even looks at the parity of k.
//  * So each lane converts its S addends to ulps (exact: a scale by a power
//    of two, rint, and an exact sum of at most S integers below 2^21) and
//    the wavefront takes an inclusive prefix sum of the per-lane counts
//    (DPP row shifts and row broadcasts, u32).
//  * In integer form, adding P ulps to s within the binade is adding P to
//    its bit pattern.  The first lane whose prefix reaches the next power of
//    two (K = 2^24 - k ulps away), or that holds a tie or an out-of-range
//    addend, is an event: the lanes before it are applied as one integer add,
//    the event lane's S values are folded one by one in f32, and the scan is
//    reused (same binade) or recomputed (new binade).  Every lane folds its
//    own S values from the start it would have as the event lane (the sum
//    plus its exclusive prefix), which is exact for the real event lane, and
//    one readlane takes that lane's result: the add chain does not wait for
//    the event lane to be known, and no values move between lanes.
//  * Sums outside [2^-100, 2^125), inf and NaN fold lane by lane in f32.
//
// Every step either is the sequential fold's own f32 add or provably equals
// it, so the result is the sequential fold's bit pattern.  The wave must be
// fully active (64 lanes) and all addends >= +0 or NaN (squares).
//
// v: lane l's S consecutive addends [S*l, S*l + S) of the chunk;
// sb: bit pattern of the running sum before the chunk (wave-uniform).
// Returns the bit pattern after the chunk (wave-uniform).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, uint32_t lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), static_cast<int>(lane)));
}
__device__ __forceinline__ float readlane_f32(float v, uint32_t lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), static_cast<int>(lane)));
}

// Inclusive prefix sum over the 64 lanes (u32, wrapping).  Row shifts by 1,
// 2, 4, 8 scan each row of 16 lanes (zero fill); row_bcast:15 adds row 0's
// total to row 1 and row 2's to row 3; row_bcast:31 adds rows 0-1's total
// to rows 2 and 3.
__device__ __forceinline__ uint32_t wave_inclusive_scan_u32(uint32_t v) {
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, true));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, true));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, true));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, true));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false));
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false));
    return v;
}

// One binade's scan of a chunk: each lane's ulps (0 for a lane that must
// fold in f32: a tie, an out-of-range count, NaN or inf), their inclusive
// wave prefix sum, and the mask of the f32 lanes.
struct ChunkScan {
    uint32_t inc, incl;
    uint64_t bad;
};

template <int S>
__device__ __forceinline__ ChunkScan chunk_scan(const float (&v)[S], uint32_t ex) {
    const float inv_ulp = __uint_as_float((277u - ex) << 23);  // 2^(23-E)
    float ulps = 0.0f, dev = 0.0f;
#pragma unroll
    for (int i = 0; i < S; ++i) {
        const float q = v[i] * inv_ulp;
        const float m = __builtin_rintf(q);
        dev = fmaxf(dev, __builtin_fabsf(q - m));
        ulps = ulps + m;
    }
    const bool bad = !(ulps < 2097152.0f) || dev == 0.5f;  // out of range, NaN/inf, or a tie
    ChunkScan c;
    c.inc = bad ? 0u : static_cast<uint32_t>(ulps);
    c.incl = wave_inclusive_scan_u32(c.inc);
    c.bad = __builtin_amdgcn_ballot_w64(bad);
    return c;
}

// The event loop in binade ex (sb's, within [27, 251]) from lane l0 with that
// binade's scan: returns the lane to continue from (64 when the chunk is
// done; otherwise the sum has left the binade and needs the next one's scan).
template <int S>
__device__ __forceinline__ uint32_t chunk_walk(const ChunkScan& c, const float (&v)[S], uint32_t& sb, uint32_t l0,
                                               uint32_t ex) {
    uint32_t base = l0 ? readlane_u32(c.incl, l0 - 1) : 0u;
    for (;;) {
        // every lane from its start as the event lane (lanes [l0, lc)
        // stay in the binade, so lane lc's start is exact); issued ahead
        // of the event search, which it does not depend on
        float s = __uint_as_float(sb + (c.incl - c.inc) - base);
#pragma unroll
        for (int i = 0; i < S; ++i) s = s + v[i];
        const uint32_t room = 0x800000u - (sb & 0x7fffffu);  // ulps to the next power of two
        const uint64_t ev = (__builtin_amdgcn_ballot_w64(c.incl - base >= room) | c.bad) & (~0ull << l0);
        __asm__ volatile("" ::"v"(s));  // keep the chain ahead of the branch
        if (ev == 0) {
            sb += readlane_u32(c.incl, 63) - base;
            return 64;
        }
        const uint32_t lc = static_cast<uint32_t>(__builtin_ctzll(ev));
        sb = readlane_u32(__float_as_uint(s), lc);
        base = readlane_u32(c.incl, lc);
        l0 = lc + 1;
        if (l0 >= 64 || (sb >> 23) != ex) return l0;
    }
}

// The same from lane `start` on (lanes before it are already folded).
template <int S>
__device__ __forceinline__ uint32_t fold_chunk_exact_from(const float (&v)[S], uint32_t sb, uint32_t start) {
    uint32_t l0 = start;
    while (l0 < 64) {
        const uint32_t ex = sb >> 23;  // biased exponent (NaN/inf: >= 255)
        if (ex < 27 || ex > 251) {
            float s = __uint_as_float(sb);
#pragma unroll
            for (int i = 0; i < S; ++i) s = s + readlane_f32(v[i], l0);
            sb = __float_as_uint(s);
            ++l0;
            continue;
        }
        l0 = chunk_walk<S>(chunk_scan<S>(v, ex), v, sb, l0, ex);
    }
    return sb;
}

template <int S>
__device__ __forceinline__ uint32_t fold_chunk_exact(const float (&v)[S], uint32_t sb) {
    return fold_chunk_exact_from<S>(v, sb, 0u);
}

// Two independent rows' chunks: both first scans are computed before either
// event loop, so their VALU chains overlap; each row then takes the same
// steps as fold_chunk_exact.
template <int S>
__device__ __forceinline__ void fold_chunk_exact_pair(const float (&v0)[S], uint32_t& sb0, const float (&v1)[S],
                                                      uint32_t& sb1) {
    const uint32_t ex0 = sb0 >> 23, ex1 = sb1 >> 23;
    if (ex0 < 27 || ex0 > 251 || ex1 < 27 || ex1 > 251) {
        sb0 = fold_chunk_exact_from<S>(v0, sb0, 0u);
        sb1 = fold_chunk_exact_from<S>(v1, sb1, 0u);
        return;
    }
    const ChunkScan c0 = chunk_scan<S>(v0, ex0);
    const ChunkScan c1 = chunk_scan<S>(v1, ex1);
    const uint32_t l0 = chunk_walk<S>(c0, v0, sb0, 0u, ex0);
    const uint32_t l1 = chunk_walk<S>(c1, v1, sb1, 0u, ex1);
    if (l0 < 64) sb0 = fold_chunk_exact_from<S>(v0, sb0, l0);
    if (l1 < 64) sb1 = fold_chunk_exact_from<S>(v1, sb1, l1);
}

// ---------------------------------------------------------------------------
// The in-order fold of a row's first 256 squares, with its chain cut by four.
//
// The head is four segments of 64.  Segment 0 starts at exactly 0; segment
// k's start is the fold of the segments before it, known only once they are
// folded -- but approximately known at once: a wave prefix sum of the lanes'
// partial sums estimates it within a few ulps (the in-order fold and the
// estimate differ by their rounding errors, a few ulps over <= 192 adds).  So
// 21 lanes per segment fold it in parallel from 21 consecutive floats around
// the estimate, and the segments are chained by selection: segment k's exact
// start (the selected fold of segment k - 1) picks the lane that started
// there, whose result is bit for bit the in-order fold from that start.  A
// start outside the window (a miss) folds that segment in order from it.
// Every step is either the in-order fold's own f32 adds or a selection of
// them, so the result is the in-order fold's bit pattern in every case.
// Misses measured on MI355X: 12 in 107,776 Gaussian rows of 1536.
//
// h: the 64 float4 of squares in LDS, float4 i at h[i + i / 16] (a pad per
// segment keeps the four segments' reads on distinct banks).  The whole
// wavefront takes part; the result is wave-uniform.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_inclusive_scan_f32(float v) {  // any order: an estimate
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false));
    return v;
}

// 16 float4 folded in order from s (both groups of 8 read ahead of the adds)
__device__ __forceinline__ float fold_lds_16(const f32x4* p, float s) {
    f32x4 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = p[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = p[8 + i];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s = s + a[i].x;
        s = s + a[i].y;
        s = s + a[i].z;
        s = s + a[i].w;
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s = s + b[i].x;
        s = s + b[i].y;
        s = s + b[i].z;
        s = s + b[i].w;
    }
    return s;
}

__device__ __forceinline__ float head_fold_candidates(const f32x4* h, uint32_t lane) {
    const f32x4 mine = h[lane + lane / 16];
    const float pre = wave_inclusive_scan_f32((mine.x + mine.y) + (mine.z + mine.w));
    // lane 0: segment 0 from 0; lanes 1-21, 22-42, 43-63: segments 1-3
    const uint32_t seg = lane == 0 ? 0u : (lane - 1) / 21 + 1;
    const uint32_t j = lane == 0 ? 0u : (lane - 1) % 21;
    const float e1 = readlane_f32(pre, 15), e2 = readlane_f32(pre, 31), e3 = readlane_f32(pre, 47);
    const float est = seg == 1 ? e1 : (seg == 2 ? e2 : e3);
    const uint32_t start = seg == 0 ? 0u : __float_as_uint(est) + j - 10u;  // est - 10 .. est + 10 ulps
    const float res = fold_lds_16(h + 17 * seg, __uint_as_float(start));
    float s = readlane_f32(res, 0);
#pragma unroll
    for (uint32_t k = 1; k < 4; ++k) {
        const uint64_t m = __builtin_amdgcn_ballot_w64(seg == k && start == __float_as_uint(s));
        s = m ? readlane_f32(res, static_cast<uint32_t>(__builtin_ctzll(m))) : fold_lds_16(h + 17 * k, s);
    }
    return s;
}

// ---------------------------------------------------------------------------
// The continuation with its scans computed ahead.
//
// A sum of squares only grows, so its binade only moves up.  fold_scan_ahead
// computes, before the running sum is known, what fold_chunk_exact_from
// recomputes after every binade crossing: the per-lane ulp counts, their
// wave prefix sums and the event lanes, for the NB binades with biased
// exponents e0 .. e0 + NB - 1 (e0 a lower bound of the running sum's
// exponent, e.g. from an approximate sum).  Being independent of the running
// sum, it can overlap the in-order fold that produces it.  fold_walk then
// runs the same event loop, switching to the next binade's scan at a
// crossing instead of recomputing it.  A sum outside those binades (or
// outside the exponent range [27, 251]) finishes in fold_chunk_exact_from
// from the current lane, so the result is the sequential fold's bit pattern
// in every case.
// ---------------------------------------------------------------------------
template <int NB>
struct FoldScans {
    uint32_t inc[NB];   // lane's ulps in binade e0 + b (0 for an event lane)
    uint32_t incl[NB];  // inclusive wave prefix sum of inc
    uint64_t bad[NB];   // lanes that must fold in f32 (tie, out of range)
    uint32_t e0;
};

template <int S, int NB>
__device__ __forceinline__ FoldScans<NB> fold_scan_ahead(const float (&v)[S], uint32_t e0) {
    FoldScans<NB> f;
    f.e0 = e0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        // 2^(23-E) for the binade's ulp (clamped: a binade outside [27, 251]
        // is never walked with its scan)
        const uint32_t ex = min(max(e0 + b, 27u), 251u);
        const float inv_ulp = __uint_as_float((277u - ex) << 23);
        float ulps = 0.0f, dev = 0.0f;
#pragma unroll
        for (int i = 0; i < S; ++i) {
            const float q = v[i] * inv_ulp;
            const float m = __builtin_rintf(q);
            dev = fmaxf(dev, __builtin_fabsf(q - m));
            ulps = ulps + m;
        }
        const bool bad = !(ulps < 2097152.0f) || dev == 0.5f;
        f.inc[b] = bad ? 0u : static_cast<uint32_t>(ulps);
        f.incl[b] = wave_inclusive_scan_u32(f.inc[b]);
        f.bad[b] = __builtin_amdgcn_ballot_w64(bad);
    }
    return f;
}

// v: lane l's S consecutive addends; sb: bit pattern of the running sum
// before them (wave-uniform).  Returns the bit pattern after all 64 * S.
// An event folds every lane's S values from its start as the event lane
// and takes the event lane's result (as in fold_chunk_exact_from).
template <int S, int NB>
__device__ __forceinline__ uint32_t fold_walk(const FoldScans<NB>& f, const float (&v)[S], uint32_t sb) {
    uint32_t l0 = 0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint32_t ex = f.e0 + b;
        if (l0 >= 64 || (sb >> 23) != ex || ex < 27 || ex > 251) continue;
        uint32_t base = l0 ? readlane_u32(f.incl[b], l0 - 1) : 0u;
        for (;;) {
            float s = __uint_as_float(sb + (f.incl[b] - f.inc[b]) - base);
#pragma unroll
            for (int i = 0; i < S; ++i) s = s + v[i];
            const uint32_t room = 0x800000u - (sb & 0x7fffffu);  // ulps to the next power of two
            const uint64_t ev = (__builtin_amdgcn_ballot_w64(f.incl[b] - base >= room) | f.bad[b]) & (~0ull << l0);
            // keep the chain ahead of the branch, where it overlaps the event
            // search (the compiler otherwise sinks it into the event path:
            // C5 epilogues at 256 rows 4.70 against 4.75 us)
            __asm__ volatile("" ::"v"(s));
            if (ev == 0) {
                sb += readlane_u32(f.incl[b], 63) - base;
                l0 = 64;
                break;
            }
            const uint32_t lc = static_cast<uint32_t>(__builtin_ctzll(ev));
            sb = readlane_u32(__float_as_uint(s), lc);
            base = readlane_u32(f.incl[b], lc);
            l0 = lc + 1;
            if (l0 >= 64 || (sb >> 23) != ex) break;
        }
    }
    return l0 < 64 ? fold_chunk_exact_from<S>(v, sb, l0) : sb;
}

// Sum over the 64 lanes in no particular order (an estimate: DPP row
// shifts then row broadcasts, the total in lane 63), broadcast to all lanes.
template <int CTRL, int ROW_MASK, bool BOUND>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, BOUND));
}
// Sum over the wavefront in a fixed tree order, the result in every lane:
// quad_perm xor 1, xor 2, row_half_mirror, row_mirror (16-lane rows), an
// xor-16 ds_swizzle inside each 32-lane half, then half 0 + half 1.  The
// tolerance-level reductions (tree engines) use it; their order is fixed, so
// repeated calls give the same bits.
__device__ __forceinline__ float wave_sum_tree_f32(float v) {
    v = v + dpp_f32<0xb1, 0xf, false>(v);
    v = v + dpp_f32<0x4e, 0xf, false>(v);
    v = v + dpp_f32<0x141, 0xf, false>(v);
    v = v + dpp_f32<0x140, 0xf, false>(v);
    v = v + __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f));
    return readlane_f32(v, 0) + readlane_f32(v, 32);
}

// Maximum over the wavefront by the same DPP / swizzle steps (fmaxf: exact in
// any order; NaN lanes never win over a number), the result in every lane.
__device__ __forceinline__ float wave_max_tree_f32(float v) {
    v = fmaxf(v, dpp_f32<0xb1, 0xf, false>(v));
    v = fmaxf(v, dpp_f32<0x4e, 0xf, false>(v));
    v = fmaxf(v, dpp_f32<0x141, 0xf, false>(v));
    v = fmaxf(v, dpp_f32<0x140, 0xf, false>(v));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401f)));
    return fmaxf(readlane_f32(v, 0), readlane_f32(v, 32));
}

__device__ __forceinline__ float wave_sum_any_order_f32(float v) {
    v += dpp_f32<0x111, 0xf, true>(v);
    v += dpp_f32<0x112, 0xf, true>(v);
    v += dpp_f32<0x114, 0xf, true>(v);
    v += dpp_f32<0x118, 0xf, true>(v);
    v += dpp_f32<0x142, 0xa, false>(v);
    v += dpp_f32<0x143, 0xc, false>(v);
    return readlane_f32(v, 63);
}

}  // namespace atlas
