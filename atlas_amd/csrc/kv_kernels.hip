// kv_kernels.hip -- KV-cache append with the fused V RMSNorm and the
// Q8_0 / Q4_0 encoders, for gfx950.
//
// Reference semantics (bisegni/atlas, crates/atlas-metal/src/kernels.metal):
//   kv_append_decode_{f32,q8_0,q4_0}          :1197-1267  one token at `position`
//   kv_append_decode_{f32,q8_0,q4_0}_batch    :1269-1344  tokens with a positions table
//   kv_append_decode_{f32,q8_0,q4_0}_vnorm    :1346-1436  V RMS-normalised in the same dispatch
//   rms_norm_groups_in_place_unweighted_f32   :919-929    the unfused V norm
//   callers crates/atlas-model/src/gemma4_executor.rs:3826-3850 (prefill),
//           :4326-4368 (decode)
//
// Cache layout (the reference's): [K | V][position][row], a row being
// kv_width f32 values or kv_width/32 blocks of 34 (Q8_0) / 18 (Q4_0) bytes.
// Tokens whose position is >= capacity are skipped.  With vnorm the V row is
// scaled by inv = 1 / sqrt(sum_i v_i^2 / kv_width + eps) (sum in index
// order, as the unfused in-place norm computes it) before it is stored or
// encoded; the V input buffer itself is left untouched.
//
// Encoders (per 32-value block, restating the Metal kernels):
//   Q8_0: m = max|v|; scale = m == 0 ? 0 : m / 127; code = round-half-away(
//         clamp(v / scale, -127, 127)); stored: f16(scale) RNE, 32 int8.
//   Q4_0: the first value with the largest |v| (strictly greater wins) gives
//         the signed maximum s; scale = s / -8; code = clamp(trunc(v / scale
//         + 8.5), 0, 15); stored: f16(scale) RNE, 16 bytes (value j in the
//         low nibble of byte j, value j + 16 in its high nibble).
// The f32 arithmetic is IEEE (correctly rounded division and sqrt).
//
// Layout on CDNA: for kv_width 256, 512 or 1024 with 16-byte aligned rows,
// one wavefront per token (kv_append_row_kernel, below); with the V norm at
// width 256 and at least 256 tokens, worker wavefronts beside one that folds
// every V row of the workgroup (kv_append_rows_kernel).  Otherwise one
// 256-thread workgroup per token: thread t owns values t + 256p of the K and
// V rows; a 32-value block is exactly half a wavefront, so block maxima are
// half-wave reductions (DPP steps and one ds_swizzle) and the Q4_0 nibble
// pairing is an xor-16 swizzle.  The V sum of squares folds in order from
// LDS on one lane in both.
#include "device_common.hpp"
#include "launch.hpp"


namespace atlas {
namespace {

constexpr uint32_t kThreads = 256;

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Exchange with lane ^ 16 inside each 32-lane half (ds_swizzle bit mode:
// and_mask 0x1f, xor_mask 0x10).
__device__ __forceinline__ int swap16(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401f); }

// Maximum over each 32-lane half: four DPP steps inside 16-lane rows
// (quad_perm xor 1, xor 2, row_half_mirror, row_mirror), then one swizzle.
// fmaxf ignores NaN lanes; a half of NaN lanes only gives NaN, so the
// encoders seed the result with 0 as the reference's fold does.
__device__ __forceinline__ float half_wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xb1>(v));
    v = fmaxf(v, dpp_f32<0x4e>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(v, __int_as_float(swap16(__float_as_int(v))));
}

__device__ __forceinline__ uint32_t f16_bits(float v) { return f2h(v); }

// Store one encoded block.  Lanes of a half wave hold the block's 32 values
// (lane % 32 = index in the block); dst points at the block's first byte.
template <int FMT>
__device__ __forceinline__ void encode_block(float v, uint8_t* dst, uint32_t j) {
    // maximum = max(0, |v_0|, ..., |v_31|): an all-NaN block gives 0, so its
    // scale and codes are 0 (kernels.metal:1220-1221, 1244-1245)
    const float amax = fmaxf(0.0f, half_wave_max(__builtin_fabsf(v)));
    if (FMT == kKvQ8_0) {
        const float scale = amax == 0.0f ? 0.0f : fdiv_rn(amax, 127.0f);
        if (j == 0) {
            dst[0] = static_cast<uint8_t>(f16_bits(scale));
            dst[1] = static_cast<uint8_t>(f16_bits(scale) >> 8);
        }
        int code = 0;
        if (scale != 0.0f) code = static_cast<int>(roundf(fminf(fmaxf(fdiv_rn(v, scale), -127.0f), 127.0f)));
        dst[2 + j] = static_cast<uint8_t>(static_cast<int8_t>(code));
    } else {
        // signed maximum: the first lane (lowest index) of each half whose |v|
        // equals that half's maximum; both halves are read with scalar readlanes
        const uint64_t hit = __builtin_amdgcn_ballot_w64(amax > 0.0f && __builtin_fabsf(v) == amax);
        const uint32_t lo = static_cast<uint32_t>(hit), hi = static_cast<uint32_t>(hit >> 32);
        const float s_lo = readlane_f32(v, lo ? static_cast<uint32_t>(__builtin_ctz(lo)) : 0u);
        const float s_hi = readlane_f32(v, hi ? 32u + static_cast<uint32_t>(__builtin_ctz(hi)) : 32u);
        const float smax = (__lane_id() & 32u) ? s_hi : s_lo;
        const float scale = amax == 0.0f ? 0.0f : fdiv_rn(smax, -8.0f);
        int code = 0;
        if (scale != 0.0f) {
            const float t = fdiv_rn(v, scale) + 8.5f;
            code = t >= 15.0f ? 15 : (t > 0.0f ? static_cast<int>(t) : 0);
        }
        const int high = swap16(code);  // lane j < 16 receives the code of value j + 16
        if (j == 0) {
            dst[0] = static_cast<uint8_t>(f16_bits(scale));
            dst[1] = static_cast<uint8_t>(f16_bits(scale) >> 8);
        }
        if (j < 16) dst[2 + j] = static_cast<uint8_t>(code | (high << 4));
    }
}

// Kernel parameters of the KV-append kernels: KvAppendArgs field by field
// (a by-value struct is not preloaded into SGPRs), the counts and positions
// first; all 48 bytes arrive in user SGPRs at wave launch (kernarg preload),
// so the position and row loads wait on no scalar load.
#define ATLAS_KV_KPARAMS                                                                                  \
    uint32_t p_kv_width, uint32_t p_capacity, uint32_t p_tokens, float p_epsilon, const uint32_t* p_positions, \
        const float* p_key, const float* p_value, uint8_t* p_cache
#define ATLAS_KV_UNPACK \
    const KvAppendArgs a { p_key, p_value, p_cache, p_positions, p_kv_width, p_capacity, p_tokens, p_epsilon }
#define ATLAS_KV_KARGS(a) \
    (a).kv_width, (a).capacity, (a).tokens, (a).epsilon, (a).positions, (a).key, (a).value, (a).cache

// P: values per thread and row (kv_width <= 256 * P).
template <int FMT, bool VNORM, int P>
__global__ __launch_bounds__(256) void kv_append_kernel(ATLAS_KV_KPARAMS) {
    ATLAS_KV_UNPACK;
    extern __shared__ __align__(16) float sq[];  // kv_width squares of V (VNORM)
    __shared__ float inv_shared;
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint32_t w = a.kv_width;
    const float* key = a.key + static_cast<size_t>(t) * w;
    const float* value = a.value + static_cast<size_t>(t) * w;
    const uint32_t passes = (w + kThreads - 1) / kThreads;

    // the position's load goes out first and the row's right behind it
    // (loads return in issue order, so the position is waited for alone)
    const uint32_t position = a.positions[t];
    __asm__ volatile("" ::: "memory");
    float k[P], v[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t i = tid + kThreads * p;
        const bool in = p < static_cast<int>(passes) && i < w;
        k[p] = in ? key[i] : 0.0f;
        v[p] = in ? value[i] : 0.0f;
    }
    __asm__ volatile("" ::: "memory");  // keeps the loads above the position test
    if (position >= a.capacity) return;  // workgroup-uniform
    if (VNORM) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t i = tid + kThreads * p;
            if (p < static_cast<int>(passes) && i < w) sq[i] = v[p] * v[p];
        }
        __syncthreads();
        if (tid == 0) {
            float s = 0.0f;
            const f32x4* row = reinterpret_cast<const f32x4*>(sq);
            for (uint32_t c = 0; c < w / 4; c += 64) s = fold_lds_chunk(row + c, min(64u, w / 4 - c), s);
            inv_shared = inverse_rms(s, static_cast<float>(w), a.epsilon);
        }
        __syncthreads();
        const float inv = inv_shared;
#pragma unroll
        for (int p = 0; p < P; ++p) v[p] = v[p] * inv;
    }

    const size_t half = static_cast<size_t>(a.capacity);  // rows per cache half
    if (FMT == kKvF32) {
        float* kc = reinterpret_cast<float*>(a.cache) + static_cast<size_t>(position) * w;
        float* vc = reinterpret_cast<float*>(a.cache) + (half + position) * w;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t i = tid + kThreads * p;
            if (p < static_cast<int>(passes) && i < w) {
                kc[i] = k[p];
                vc[i] = v[p];
            }
        }
    } else {
        constexpr uint32_t kBlock = FMT == kKvQ8_0 ? 34 : 18;
        const uint32_t blocks = w / 32;
        uint8_t* kc = a.cache + static_cast<size_t>(position) * blocks * kBlock;
        uint8_t* vc = a.cache + (half + position) * blocks * kBlock;
        const uint32_t j = tid & 31u;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (p >= static_cast<int>(passes)) break;  // workgroup-uniform
            // kv_width % 32 == 0, so a half wave is all in or all out; every
            // cross-lane step of the encoder stays inside its half (DPP rows,
            // xor-16 swizzle, the half's own readlane), so an inactive half
            // does not affect an active one
            const uint32_t b = (tid + kThreads * p) / 32;
            if (b < blocks) {
                encode_block<FMT>(k[p], kc + b * kBlock, j);
                encode_block<FMT>(v[p], vc + b * kBlock, j);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Row engine: two wavefronts per token (the K row and the V row, side by
// side), two tokens per workgroup, no workgroup barrier.  For kv_width =
// 256 * V4 (V4 = 1, 2, 4) with 16-byte aligned rows: lane l holds values
// [4(l + 64i), +4) of its row (16-byte nontemporal loads), so a 32-value
// block is 8 lanes.  The V sum of squares folds in index order on lane 0 from
// LDS while the K wavefront encodes and stores; each encoded row is
// assembled in LDS and written with 16-byte stores (a Q8_0 / Q4_0 row of 256
// values is 272 / 144 bytes, 16-byte aligned for every position).  The
// encoder (encode_items) gives the bits of the per-value engine above; it
// takes each quotient as a product with the scale's reciprocal where that
// provably yields the same code.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void lds_wave_handoff() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ float group8_max(float v) {
    v = fmaxf(v, dpp_f32<0xb1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4e>(v));   // quad_perm [2,3,0,1]
    return fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
}

// Quotient band.  A code depends on the quotient fl(v / scale) only through
// which pair of consecutive half-integers it lies between (Q8_0 rounds half
// away from zero, Q4_0 truncates fl(q + 8.5) with q + 8.5 < 17, whose
// rounding error is below 2^-20).  For a normal scale (|scale| in
// [2^-126, 2^126]) and |v| <= max|v| of the block, |q| <= 128 and
// v * rcp(scale) (v_rcp_f32 is within 1 ulp) is within 2^-15 of fl(v /
// scale); a product more than 2^-12 from every half-integer therefore gives
// the code of the correctly rounded quotient.  A lane with any product in
// that band, a scale outside the normal range or a NaN value recomputes its
// codes with fdiv_rn and the reference's own steps.
constexpr float kHalfBand = 0x1p-12f;

__device__ __forceinline__ bool scale_normal(float scale) {
    const float a = __builtin_fabsf(scale);
    return a >= 0x1p-126f && a <= 0x1p126f;  // false for 0, inf, NaN
}

__device__ __forceinline__ bool off_half(float q) {  // NaN: false
    return __builtin_fabsf(__builtin_amdgcn_fractf(q) - 0.5f) > kHalfBand;
}

// The reference's code steps on the correctly rounded quotient.
template <int FMT>
__device__ __forceinline__ uint32_t code_exact(float v, float scale) {
    if (FMT == kKvQ8_0) {
        if (scale == 0.0f) return 0u;
        return static_cast<uint32_t>(static_cast<int>(roundf(fminf(fmaxf(fdiv_rn(v, scale), -127.0f), 127.0f)))) &
               0xffu;
    }
    if (scale == 0.0f) return 0u;
    const float t = fdiv_rn(v, scale) + 8.5f;
    return t >= 15.0f ? 15u : (t > 0.0f ? static_cast<uint32_t>(static_cast<int>(t)) : 0u);
}

// The same code from a product q outside the band (round to nearest even
// and round half away agree off the half-integers; trunc of the clamped
// q + 8.5 is the reference's three-way select).
template <int FMT>
__device__ __forceinline__ uint32_t code_fast(float q) {
    if (FMT == kKvQ8_0)
        return static_cast<uint32_t>(static_cast<int>(__builtin_rintf(__builtin_amdgcn_fmed3f(q, -127.0f, 127.0f)))) &
               0xffu;
    return static_cast<uint32_t>(static_cast<int>(__builtin_amdgcn_fmed3f(q + 8.5f, 0.0f, 15.0f)));
}

// fl(a / 127) for the Q8_0 scale (a = a block maximum, >= 0).  For a in
// [2^-100, 2^100], Markstein's correction of the product with c = RN(1/127):
// q0 = a c, r = a - 127 q0 (exact in an fma), q = RN(q0 + r c) -- equal to
// RN(a / 127) for every float of one binade, checked exhaustively, and so
// over the whole range, where every step scales exactly by powers of two.
// a = 0 gives +0 through the same steps; other values take the IEEE
// division, on a branch that is not taken for ordinary data (the empty asm
// keeps the compiler from computing both and selecting).
__device__ __forceinline__ float div127(float a) {
    constexpr float c = 1.0f / 127.0f;
    const float q0 = a * c;
    float q = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, a), c, q0);
    if (!(a == 0.0f || (a >= 0x1p-100f && a <= 0x1p100f))) {
        __asm__ volatile("");
        q = fdiv_rn(a, 127.0f);
    }
    return q;
}

// Maximum of |v| over a 32-value block held by 8 lanes (4 values each),
// seeded with 0 as the reference's fold is (kernels.metal:1220-1221,
// 1244-1245): NaN never raises it and an all-NaN block gives 0.  The lane's
// fmaxf of its 4 |v|, then quad_perm xor 1, xor 2 and row_half_mirror.
__device__ __forceinline__ float block_max(const f32x4 x) {
    float m = 0.0f;
    m = fmaxf(m, __builtin_fabsf(x.x));
    m = fmaxf(m, __builtin_fabsf(x.y));
    m = fmaxf(m, __builtin_fabsf(x.z));
    m = fmaxf(m, __builtin_fabsf(x.w));
    return group8_max(m);
}

// Encode N groups of four values held by the lane: item n is x[n] (times
// inv[n] when NORM: the V norm's scaling, which the encoder applies itself),
// values 4g..4g+3 (g = lane % 8) of block blk[n] in the LDS row buffer
// row[n] (2-byte stores: blocks are 34 / 18 bytes).  bmax[n] is
// block_max(x[n]); the items' chains are independent and overlap.
//  * With NORM the block maximum of y = fl(x inv) is fl(bmax inv): rounding
//    is monotonic, so the largest |x| gives the largest |y|.  Where that
//    product is not finite (a NaN or inf in the row) the maximum is taken
//    over y itself.
//  * Q4_0 signed maximum: the first value of the block with |y| == max
//    (lane order, then position in the lane) is +max or -max, so only its
//    sign travels: two ballots, the first hit lane of the group, its bit.
//  * Quotients: q = x * fl(inv rcp(scale)) (x * rcp(scale) without NORM) is
//    within 2.75 * 2^-16 of fl(y / scale) for a normal scale and a normal
//    fl(inv rcp(scale)), so outside the 2^-12 band it gives the reference's
//    code; each value in the band (or any value when those factors are not
//    normal) is recomputed with fdiv_rn and the reference's steps.
//  * Q4_0 nibble pairing: values j and j + 16 sit in lanes g and g + 4 of
//    the block, exchanged with an xor-4 swizzle.
typedef __attribute__((address_space(3))) volatile uint16_t lds_u16;

template <int FMT, int N, bool NORM>
__device__ __forceinline__ void encode_items(const f32x4 (&x)[N], const float (&inv)[N], const float (&bmax)[N],
                                             uint8_t* const (&row)[N], const uint32_t (&blk)[N], uint32_t g) {
    float scale[N];
    uint32_t code[N][4];
    bool need[N][4];
    bool any = false;
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const float v[4] = {x[n].x, x[n].y, x[n].z, x[n].w};
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = NORM ? v[i] * inv[n] : v[i];
        float amax = NORM ? bmax[n] * inv[n] : bmax[n];
        if (NORM && !__builtin_isfinite(amax)) {  // uniform over the block's 8 lanes
            float m = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) m = fmaxf(m, __builtin_fabsf(y[i]));
            amax = group8_max(m);
        }
        if (FMT == kKvQ8_0) {
            scale[n] = div127(amax);  // amax == 0 gives 0, as the reference's select does
        } else {
            // sign of this lane's first value with |y| == amax (amax > 0)
            bool has = false, neg = false;
#pragma unroll
            for (int i = 3; i >= 0; --i) {
                const bool hit = amax > 0.0f && __builtin_fabsf(y[i]) == amax;
                neg = hit ? __builtin_signbit(y[i]) != 0 : neg;
                has = has || hit;
            }
            const uint64_t hits = __builtin_amdgcn_ballot_w64(has);
            const uint64_t negs = __builtin_amdgcn_ballot_w64(has && neg);
            const uint32_t base = __lane_id() & ~7u;
            const uint32_t mine = static_cast<uint32_t>(hits >> base) & 0xffu;
            const uint32_t first = base + (mine ? static_cast<uint32_t>(__builtin_ctz(mine)) : 0u);
            const float smax = ((negs >> first) & 1u) ? -amax : amax;
            // smax / -8 is exact up to the final rounding, as the product is
            scale[n] = amax == 0.0f ? 0.0f : smax * -0.125f;
        }
        const float r = __builtin_amdgcn_rcpf(scale[n]);
        const float ir = NORM ? inv[n] * r : r;
        const bool ok = scale_normal(scale[n]) && (!NORM || scale_normal(ir));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float q = v[i] * ir;
            need[n][i] = !(ok && off_half(q));
            code[n][i] = code_fast<FMT>(q);
            any = any || need[n][i];
        }
    }
    if (any) {
#pragma unroll
        for (int n = 0; n < N; ++n) {
            const float v[4] = {x[n].x, x[n].y, x[n].z, x[n].w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (need[n][i]) code[n][i] = code_exact<FMT>(NORM ? v[i] * inv[n] : v[i], scale[n]);
        }
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
        const uint32_t packed = code[n][0] | (code[n][1] << 8) | (code[n][2] << 16) | (code[n][3] << 24);
        // volatile keeps the 2-byte writes apart: merged, every other block's
        // pair would be an unaligned 4-byte LDS write, which stalls
        lds_u16* dst = (lds_u16*)(row[n] + blk[n] * (FMT == kKvQ8_0 ? 34u : 18u));  // generic -> LDS
        if (FMT == kKvQ8_0) {
            if (g == 0) dst[0] = f16_bits(scale[n]);
            dst[1 + 2 * g] = static_cast<uint16_t>(packed);
            dst[2 + 2 * g] = static_cast<uint16_t>(packed >> 16);
        } else {
            // lane g < 4 of the block holds values 4g..4g+3 (low nibbles),
            // lane g + 4 the values 16 + 4g.. (high nibbles)
            const uint32_t partner = static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(packed), 0x101f));
            if (g == 0) dst[0] = f16_bits(scale[n]);
            if (g < 4) {
                const uint32_t bytes = packed | (partner << 4);
                dst[1 + 2 * g] = static_cast<uint16_t>(bytes);
                dst[2 + 2 * g] = static_cast<uint16_t>(bytes >> 16);
            }
        }
    }
}

// Write one row: f32 straight from registers, encoded rows through LDS.
template <int FMT, int V4>
__device__ __forceinline__ void store_row(const f32x4 (&x)[V4], uint8_t* dst, uint8_t* lds_row, uint32_t lane,
                                          uint32_t row_bytes) {
    if (FMT == kKvF32) {
#pragma unroll
        for (int i = 0; i < V4; ++i)
            __builtin_nontemporal_store(x[i], reinterpret_cast<f32x4*>(dst) + lane + 64u * i);
    } else {
        uint8_t* rows[V4];
        uint32_t blk[V4];
        float one[V4], bmax[V4];
#pragma unroll
        for (int i = 0; i < V4; ++i) {
            rows[i] = lds_row;
            blk[i] = lane / 8u + 8u * i;
            one[i] = 1.0f;
            bmax[i] = block_max(x[i]);
        }
        encode_items<FMT, V4, false>(x, one, bmax, rows, blk, lane & 7u);
        lds_wave_handoff();
        const uint32_t n16 = row_bytes / 16;  // <= 68 for V4 <= 4
        for (uint32_t u = lane; u < n16; u += kWave)
            __builtin_nontemporal_store(reinterpret_cast<const f32x4*>(lds_row)[u], reinterpret_cast<f32x4*>(dst) + u);
        lds_wave_handoff();  // the buffer is rewritten by the next row
    }
}

// Rows of kv_width 256 for the many-token kernel (one f32x4 per lane per
// row).  Explicit global casts keep the stores global, not flat: LDS waits
// do not count global stores, and they do count flat ones.
typedef __attribute__((address_space(1))) f32x4 global_f32x4;

// Store N f32 rows, scaled by inv[i] when NORM; a row whose `ok` is false
// stores nothing.
template <int N, bool NORM>
__device__ __forceinline__ void store_f32_rows(const f32x4 (&x)[N], const float (&inv)[N], uint8_t* const (&dst)[N],
                                               const bool (&ok)[N], uint32_t lane) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const f32x4 y = NORM ? f32x4{x[i].x * inv[i], x[i].y * inv[i], x[i].z * inv[i], x[i].w * inv[i]} : x[i];
        if (ok[i]) __builtin_nontemporal_store(y, (global_f32x4*)dst[i] + lane);
    }
}

// Encode N rows (scaled by inv[i] when NORM; bmax: their block_max before
// scaling) side by side into the LDS row buffers at `lds`.
template <int FMT, int N, bool NORM>
__device__ __forceinline__ void encode_rows(const f32x4 (&x)[N], const float (&inv)[N], const float (&bmax)[N],
                                            uint8_t* lds, uint32_t lane) {
    constexpr uint32_t kRowBytes = 8u * (FMT == kKvQ8_0 ? 34u : 18u);
    uint8_t* rows[N];
    uint32_t blk[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        rows[i] = lds + i * kRowBytes;
        blk[i] = lane / 8u;
    }
    encode_items<FMT, N, NORM>(x, inv, bmax, rows, blk, lane & 7u);
}

// N encoded rows side by side in LDS at `lds` (N x 17 / N x 9 16-byte
// chunks, one per lane): store them (a row whose `ok` is false stores
// nothing) and return the store's address and data.  The hardware reads a
// vector store's registers after issue, so the compiler makes the first
// instruction that overwrites them wait for every outstanding vector memory
// operation; a caller that keeps them alive (keep_alive) until its end
// leaves that wait out.  The caller hands the LDS over first.
struct PendingStore {
    global_f32x4* addr;
    f32x4 data;
};

template <int FMT, int N>
__device__ __forceinline__ PendingStore flush_rows(const uint8_t* lds, uint8_t* const (&dst)[N], const bool (&ok)[N],
                                                   uint32_t lane) {
    constexpr uint32_t n16 = 8u * (FMT == kKvQ8_0 ? 34u : 18u) / 16u;
    static_assert(N * n16 <= 64, "one 16-byte chunk per lane");
    const uint32_t r = N == 1 ? 0u : min(lane / n16, static_cast<uint32_t>(N - 1)), c = lane - r * n16;
    uint8_t* d = dst[0];
    bool o = ok[0];
#pragma unroll
    for (int i = 1; i < N; ++i) {
        d = r == static_cast<uint32_t>(i) ? dst[i] : d;
        o = r == static_cast<uint32_t>(i) ? ok[i] : o;
    }
    PendingStore st;
    st.addr = (global_f32x4*)d + c;
    st.data = reinterpret_cast<const f32x4*>(lds)[min(lane, N * n16 - 1)];
    if (lane < N * n16 && o) __builtin_nontemporal_store(st.data, st.addr);
    return st;
}

__device__ __forceinline__ void keep_alive(const PendingStore& st) {
    __asm__ volatile("" ::"v"(st.addr), "v"(st.data));
}

template <int FMT, bool VNORM, int V4>
__global__ __launch_bounds__(256) void kv_append_row_kernel(ATLAS_KV_KPARAMS) {
    ATLAS_KV_UNPACK;
    constexpr uint32_t kW = 256u * V4;
    constexpr uint32_t kRowBytes = FMT == kKvF32 ? kW * 4 : (kW / 32) * (FMT == kKvQ8_0 ? 34u : 18u);
    __shared__ __align__(16) f32x4 sq[2][VNORM ? 64 * V4 : 1];
    __shared__ __align__(16) uint8_t rowbuf[4][FMT == kKvF32 ? 16 : kRowBytes];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    // two wavefronts per token: the even one writes the K row, the odd one
    // the V row (with its norm), side by side
    const bool is_v = (wave & 1u) != 0;
    const uint32_t t = blockIdx.x * 2 + (wave >> 1);
    if (t >= a.tokens) return;
    // the position's load goes out first and the row's right behind it (a
    // skipped position only discards them): loads return in issue order,
    // so the position is waited for alone
    const uint32_t position = a.positions[t];
    __asm__ volatile("" ::: "memory");
    const f32x4* src = reinterpret_cast<const f32x4*>((is_v ? a.value : a.key) + static_cast<size_t>(t) * kW);
    f32x4 x[V4];
#pragma unroll
    for (int i = 0; i < V4; ++i) x[i] = __builtin_nontemporal_load(src + lane + 64u * i);
    __asm__ volatile("" ::: "memory");  // keeps the loads above the position test
    if (position >= a.capacity) return;
    uint8_t* dst = a.cache + (static_cast<size_t>(is_v ? a.capacity : 0u) + position) * kRowBytes;
    if (VNORM && is_v) {
        f32x4* sqw = sq[wave >> 1];
#pragma unroll
        for (int i = 0; i < V4; ++i)
            sqw[lane + 64u * i] = f32x4{x[i].x * x[i].x, x[i].y * x[i].y, x[i].z * x[i].z, x[i].w * x[i].w};
        lds_wave_handoff();
        float s = 0.0f;
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < V4; ++i) s = fold_lds_chunk(sqw + 64 * i, 64u, s);
        }
        const float inv = inverse_rms(readlane_f32(s, 0), static_cast<float>(kW), a.epsilon);
#pragma unroll
        for (int i = 0; i < V4; ++i) x[i] = f32x4{x[i].x * inv, x[i].y * inv, x[i].z * inv, x[i].w * inv};
    }
    store_row<FMT, V4>(x, dst, rowbuf[wave], lane, kRowBytes);
}

// V-norm appends of many tokens at kv_width 256: NW worker wavefronts of TW
// tokens each per workgroup, and one more wavefront whose lanes 0 .. NW*TW-1
// fold the V rows' squares in index order in one instruction stream (each
// lane's fold is the per-token kernel's, so the bits are the same) while
// the workers encode and store their K rows and take their V rows' block
// maxima; the V rows are scaled and encoded once their inverse RMS is
// published.  A token at a position past the capacity (or past the last
// token) stores nothing.
template <int TW, int NW>
struct RowsShape {
    static constexpr uint32_t kTokens = TW * NW;
    static constexpr uint32_t kThreads = (NW + 1) * kWave;
};

template <int FMT, int TW, int NW>
__global__ __launch_bounds__((NW + 1) * 64) void kv_append_rows_kernel(ATLAS_KV_KPARAMS) {
    ATLAS_KV_UNPACK;
    constexpr uint32_t kW = 256;
    constexpr uint32_t kTok = RowsShape<TW, NW>::kTokens;
    constexpr uint32_t kRowBytes = FMT == kKvF32 ? kW * 4 : (kW / 32) * (FMT == kKvQ8_0 ? 34u : 18u);
    // V squares, one row per token; a 65-float4 stride puts the rows that
    // the folding lanes read together on distinct LDS banks
    __shared__ __align__(16) f32x4 sq[kTok][65];
    __shared__ float inv_lds[kTok];
    __shared__ __align__(16) uint8_t rowbuf[NW][FMT == kKvF32 ? 16 : 2 * TW * kRowBytes];  // K rows, then V rows
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    const bool folder = wave == NW;
    const uint32_t tb = blockIdx.x * kTok + TW * (folder ? 0u : wave);  // this wavefront's tokens tb .. tb + TW - 1
    f32x4 k[TW], v[TW];
    bool ok[TW];
    uint8_t* kdst[TW];
    uint8_t* vdst[TW];
    if (!folder) {
        // Vector loads return in issue order, so a wait for one load waits
        // for every load issued before it.  Issue order: the positions
        // (needed first, for the store addresses), the V rows (the fold
        // waits only for them), then the K rows, which arrive while the
        // fold runs.
        uint32_t position[TW];
#pragma unroll
        for (int i = 0; i < TW; ++i) position[i] = a.positions[min(tb + i, a.tokens - 1)];
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < TW; ++i) {
            const size_t t = min(tb + i, a.tokens - 1);  // loads of a token past the end are clamped, never stored
            v[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a.value + t * kW) + lane);
        }
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < TW; ++i) {
            const size_t t = min(tb + i, a.tokens - 1);
            k[i] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a.key + t * kW) + lane);
        }
        __asm__ volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < TW; ++i) {
            ok[i] = tb + i < a.tokens && position[i] < a.capacity;
            const uint32_t p = ok[i] ? position[i] : 0u;  // no address is formed past the cache
            kdst[i] = a.cache + static_cast<size_t>(p) * kRowBytes;
            vdst[i] = a.cache + (static_cast<size_t>(a.capacity) + p) * kRowBytes;
        }
#pragma unroll
        for (int i = 0; i < TW; ++i)
            sq[TW * wave + i][lane] = f32x4{v[i].x * v[i].x, v[i].y * v[i].y, v[i].z * v[i].z, v[i].w * v[i].w};
    }
    __syncthreads();
    float vmax[TW];
    PendingStore kstore;
    if (folder) {
        if (lane < kTok)
            inv_lds[lane] = inverse_rms(fold_lds_chunk(sq[lane], 64u, 0.0f), static_cast<float>(kW), a.epsilon);
    } else if (FMT == kKvF32) {
        float one[TW];
#pragma unroll
        for (int i = 0; i < TW; ++i) one[i] = 1.0f;
        store_f32_rows<TW, false>(k, one, kdst, ok, lane);
    } else {
        // while the fold runs: the K rows are encoded and stored (their
        // writes overlap the fold), and the V rows' block maxima are taken
        float one[TW], kmax[TW];
#pragma unroll
        for (int i = 0; i < TW; ++i) {
            one[i] = 1.0f;
            kmax[i] = block_max(k[i]);
        }
        encode_rows<FMT, TW, false>(k, one, kmax, rowbuf[wave], lane);
        lds_wave_handoff();
        kstore = flush_rows<FMT, TW>(rowbuf[wave], kdst, ok, lane);
#pragma unroll
        for (int i = 0; i < TW; ++i) vmax[i] = block_max(v[i]);
    }
    __syncthreads();
    if (folder) return;
    float inv[TW];
#pragma unroll
    for (int i = 0; i < TW; ++i) inv[i] = inv_lds[TW * wave + i];
    if (FMT == kKvF32) {
        store_f32_rows<TW, true>(v, inv, vdst, ok, lane);
    } else {
        encode_rows<FMT, TW, true>(v, inv, vmax, rowbuf[wave] + TW * kRowBytes, lane);
        lds_wave_handoff();
        flush_rows<FMT, TW>(rowbuf[wave] + TW * kRowBytes, vdst, ok, lane);
        keep_alive(kstore);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int FMT>
bool launch_row(hipStream_t stream, const KvAppendArgs& a, bool vnorm) {
    const uint32_t w = a.kv_width;
    if ((w != 256 && w != 512 && w != 1024) || !aligned16(a.key) || !aligned16(a.value) || !aligned16(a.cache))
        return false;
    if (vnorm && w == 256 && a.tokens >= 256) {
        // Tokens per worker wavefront (TW) and workers per workgroup (NW),
        // measured on MI355X at 4096 tokens into a 4096-position cache
        // (TW x NW: f32 / Q8_0 / Q4_0 us): 2x4 4.28 / 5.05 / 5.45, 1x4
        // 4.39 / 4.78 / 4.89, 1x8 4.41 / 4.84 / 4.95, 2x2 4.37 / 5.11 / 5.49,
        // 1x2 4.71 / 5.28 / 5.38, 2x8 4.43 / 5.16 / 5.47.  The encoders'
        // V rows wait for the fold, so one row per worker shortens the chain
        // after it; the f32 rows only scale and store.
        constexpr int kTw = FMT == kKvF32 ? 2 : 1;
        using Shape = RowsShape<kTw, 4>;
        hipLaunchKernelGGL((kv_append_rows_kernel<FMT, kTw, 4>), dim3((a.tokens + Shape::kTokens - 1) / Shape::kTokens),
                           dim3(Shape::kThreads), 0, stream, ATLAS_KV_KARGS(a));
        return true;
    }
    const dim3 grid((a.tokens + 1) / 2);
#define ATLAS_KV_ROW(V)                                                                          \
    if (vnorm)                                                                                   \
        hipLaunchKernelGGL((kv_append_row_kernel<FMT, true, V>), grid, dim3(256), 0, stream, ATLAS_KV_KARGS(a)); \
    else                                                                                         \
        hipLaunchKernelGGL((kv_append_row_kernel<FMT, false, V>), grid, dim3(256), 0, stream, ATLAS_KV_KARGS(a));
    if (w == 256) {
        ATLAS_KV_ROW(1)
    } else if (w == 512) {
        ATLAS_KV_ROW(2)
    } else {
        ATLAS_KV_ROW(4)
    }
#undef ATLAS_KV_ROW
    return true;
}

template <int FMT, int P>
hipError_t launch_p(hipStream_t stream, const KvAppendArgs& a, bool vnorm) {
    if (vnorm)
        hipLaunchKernelGGL((kv_append_kernel<FMT, true, P>), dim3(a.tokens), dim3(kThreads),
                           a.kv_width * sizeof(float), stream, ATLAS_KV_KARGS(a));
    else
        hipLaunchKernelGGL((kv_append_kernel<FMT, false, P>), dim3(a.tokens), dim3(kThreads), 0, stream,
                           ATLAS_KV_KARGS(a));
    return hipGetLastError();
}

// Registers scale with the values per thread, so the row width picks the
// instantiation (256 -> 1 value per thread and row, 4096 -> 16).
template <int FMT>
hipError_t launch_fmt(hipStream_t stream, const KvAppendArgs& a, bool vnorm) {
    if (launch_row<FMT>(stream, a, vnorm)) return hipGetLastError();
    const uint32_t p = (a.kv_width + kThreads - 1) / kThreads;
    if (p <= 1) return launch_p<FMT, 1>(stream, a, vnorm);
    if (p <= 2) return launch_p<FMT, 2>(stream, a, vnorm);
    if (p <= 4) return launch_p<FMT, 4>(stream, a, vnorm);
    if (p <= 8) return launch_p<FMT, 8>(stream, a, vnorm);
    return launch_p<FMT, 16>(stream, a, vnorm);
}

}  // namespace

hipError_t launch_kv_append(hipStream_t stream, int format, bool vnorm, const KvAppendArgs& a) {
    switch (format) {
        case kKvF32: return launch_fmt<kKvF32>(stream, a, vnorm);
        case kKvQ8_0: return launch_fmt<kKvQ8_0>(stream, a, vnorm);
        case kKvQ4_0: return launch_fmt<kKvQ4_0>(stream, a, vnorm);
    }
    return hipErrorInvalidValue;
}

}  // namespace atlas
