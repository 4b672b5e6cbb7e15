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
// one wavefront per token (kv_append_row_kernel, below).  Otherwise one
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

// P: values per thread and row (kv_width <= 256 * P).
template <int FMT, bool VNORM, int P>
__global__ __launch_bounds__(256) void kv_append_kernel(KvAppendArgs a) {
    extern __shared__ __align__(16) float sq[];  // kv_width squares of V (VNORM)
    __shared__ float inv_shared;
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    const uint32_t w = a.kv_width;
    const float* key = a.key + static_cast<size_t>(t) * w;
    const float* value = a.value + static_cast<size_t>(t) * w;
    const uint32_t passes = (w + kThreads - 1) / kThreads;

    // the row's loads go out before the position's round trip returns
    float k[P], v[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t i = tid + kThreads * p;
        const bool in = p < static_cast<int>(passes) && i < w;
        k[p] = in ? key[i] : 0.0f;
        v[p] = in ? value[i] : 0.0f;
    }
    __asm__ volatile("" ::: "memory");  // keeps the loads above the position test
    const uint32_t position = a.positions[t];
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
// values is 272 / 144 bytes, 16-byte aligned for every position).  Same encoders as above:
//  * block maximum over 8 lanes: the lane's fmaxf of its 4 |v|, then
//    quad_perm xor 1, xor 2 and row_half_mirror (fmaxf ignores NaN);
//  * Q4_0 signed maximum: the first value of the block with |v| == max
//    (lane order, then position in the lane), or the block's value 0;
//  * Q4_0 nibble pairing: values j and j + 16 sit in lanes g and g + 4 of
//    the block, exchanged with an xor-4 swizzle.
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

// Encode the lane's 4 values (block b = lane/8 + 8i, index 4(lane%8)) into
// the row buffer `row` (LDS, 2-byte stores: blocks are 34 / 18 bytes).
template <int FMT>
__device__ __forceinline__ void encode4(const f32x4 x, uint8_t* row, uint32_t block, uint32_t g) {
    const float v[4] = {x.x, x.y, x.z, x.w};
    // seeded with 0, as the reference's fold is (kernels.metal:1220-1221,
    // 1244-1245): NaN values never raise it, and an all-NaN block gives 0
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, __builtin_fabsf(v[i]));
    const float amax = group8_max(m);
    uint16_t* dst = reinterpret_cast<uint16_t*>(row + block * (FMT == kKvQ8_0 ? 34u : 18u));
    if (FMT == kKvQ8_0) {
        const float scale = amax == 0.0f ? 0.0f : fdiv_rn(amax, 127.0f);
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int code = 0;
            if (scale != 0.0f) code = static_cast<int>(roundf(fminf(fmaxf(fdiv_rn(v[i], scale), -127.0f), 127.0f)));
            packed |= (static_cast<uint32_t>(code) & 0xffu) << (8 * i);
        }
        if (g == 0) dst[0] = static_cast<uint16_t>(f16_bits(scale));
        dst[1 + 2 * g] = static_cast<uint16_t>(packed);
        dst[2 + 2 * g] = static_cast<uint16_t>(packed >> 16);
    } else {
        // first value of this lane with |v| == amax (amax > 0), else value 0
        float cand = v[0];
        bool has = false;
#pragma unroll
        for (int i = 3; i >= 0; --i) {
            const bool hit = amax > 0.0f && __builtin_fabsf(v[i]) == amax;
            cand = hit ? v[i] : cand;
            has = has || hit;
        }
        const uint64_t hits = __builtin_amdgcn_ballot_w64(has);
        const uint32_t base = __lane_id() & ~7u;
        const uint32_t mine = static_cast<uint32_t>(hits >> base) & 0xffu;
        const uint32_t src = base + (mine ? static_cast<uint32_t>(__builtin_ctz(mine)) : 0u);
        const float smax = __int_as_float(__shfl(__float_as_int(cand), static_cast<int>(src), kWave));
        const float scale = amax == 0.0f ? 0.0f : fdiv_rn(smax, -8.0f);
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int code = 0;
            if (scale != 0.0f) {
                const float t = fdiv_rn(v[i], scale) + 8.5f;
                code = t >= 15.0f ? 15 : (t > 0.0f ? static_cast<int>(t) : 0);
            }
            packed |= static_cast<uint32_t>(code) << (8 * i);
        }
        // lane g < 4 of the block holds values 4g..4g+3 (low nibbles), lane
        // g + 4 the values 16 + 4g.. (high nibbles): xor-4 swizzle
        const uint32_t partner = static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(packed), 0x101f));
        if (g == 0) dst[0] = static_cast<uint16_t>(f16_bits(scale));
        if (g < 4) {
            const uint32_t bytes = packed | (partner << 4);
            dst[1 + 2 * g] = static_cast<uint16_t>(bytes);
            dst[2 + 2 * g] = static_cast<uint16_t>(bytes >> 16);
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
#pragma unroll
        for (int i = 0; i < V4; ++i) encode4<FMT>(x[i], lds_row, lane / 8u + 8u * i, lane & 7u);
        lds_wave_handoff();
        const uint32_t n16 = row_bytes / 16;  // <= 68 for V4 <= 4
        for (uint32_t u = lane; u < n16; u += kWave)
            __builtin_nontemporal_store(reinterpret_cast<const f32x4*>(lds_row)[u], reinterpret_cast<f32x4*>(dst) + u);
        lds_wave_handoff();  // the buffer is rewritten by the next row
    }
}

template <int FMT, bool VNORM, int V4>
__global__ __launch_bounds__(256) void kv_append_row_kernel(KvAppendArgs a) {
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
    // the row's loads go out before the position's round trip returns (a
    // skipped position only discards them)
    const f32x4* src = reinterpret_cast<const f32x4*>((is_v ? a.value : a.key) + static_cast<size_t>(t) * kW);
    f32x4 x[V4];
#pragma unroll
    for (int i = 0; i < V4; ++i) x[i] = __builtin_nontemporal_load(src + lane + 64u * i);
    __asm__ volatile("" ::: "memory");  // keeps the loads above the position test
    const uint32_t position = a.positions[t];
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

// V-norm appends of many tokens at kv_width 256: eight tokens per
// workgroup, two per wavefront.  Lanes 0..7 of wavefront 0 fold the eight V
// rows' squares in index order in one instruction stream (each lane's fold
// is the per-token kernel's, so the bits are the same) while every
// wavefront encodes and stores its K rows; the V rows are scaled and encoded
// once their inverse RMS is published.  A token at a position past the
// capacity (or past the last token) stores nothing.
template <int FMT>
__global__ __launch_bounds__(256) void kv_append_rows8_kernel(KvAppendArgs a) {
    constexpr uint32_t kW = 256;
    constexpr uint32_t kRowBytes = FMT == kKvF32 ? kW * 4 : (kW / 32) * (FMT == kKvQ8_0 ? 34u : 18u);
    // V squares, one row per token; a 65-float4 stride puts the eight rows
    // that lanes 0..7 read together on distinct LDS banks
    __shared__ __align__(16) f32x4 sq[8][65];
    __shared__ float inv_lds[8];
    __shared__ __align__(16) uint8_t rowbuf[4][FMT == kKvF32 ? 16 : kRowBytes];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    const uint32_t tb = blockIdx.x * 8u + 2u * wave;  // this wavefront's tokens tb, tb + 1
    f32x4 k[2][1], v[2][1];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const size_t t = min(tb + i, a.tokens - 1);  // loads of a token past the end are clamped, never stored
        k[i][0] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a.key + t * kW) + lane);
        v[i][0] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a.value + t * kW) + lane);
    }
    __asm__ volatile("" ::: "memory");  // keeps the loads above the position reads
    uint32_t position[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) position[i] = tb + i < a.tokens ? a.positions[tb + i] : a.capacity;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const f32x4 x = v[i][0];
        sq[2 * wave + i][lane] = f32x4{x.x * x.x, x.y * x.y, x.z * x.z, x.w * x.w};
    }
    __syncthreads();
    if (wave == 0 && lane < 8) inv_lds[lane] = inverse_rms(fold_lds_chunk(sq[lane], 64u, 0.0f), static_cast<float>(kW),
                                                           a.epsilon);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (position[i] < a.capacity)
            store_row<FMT, 1>(k[i], a.cache + static_cast<size_t>(position[i]) * kRowBytes, rowbuf[wave], lane,
                              kRowBytes);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if (position[i] >= a.capacity) continue;
        const float inv = inv_lds[2 * wave + i];
        const f32x4 x = v[i][0];
        const f32x4 y[1] = {f32x4{x.x * inv, x.y * inv, x.z * inv, x.w * inv}};
        store_row<FMT, 1>(y, a.cache + (static_cast<size_t>(a.capacity) + position[i]) * kRowBytes, rowbuf[wave],
                          lane, kRowBytes);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int FMT>
bool launch_row(hipStream_t stream, const KvAppendArgs& a, bool vnorm) {
    const uint32_t w = a.kv_width;
    if ((w != 256 && w != 512 && w != 1024) || !aligned16(a.key) || !aligned16(a.value) || !aligned16(a.cache))
        return false;
    if (vnorm && w == 256 && a.tokens >= 256) {
        hipLaunchKernelGGL((kv_append_rows8_kernel<FMT>), dim3((a.tokens + 7) / 8), dim3(256), 0, stream, a);
        return true;
    }
    const dim3 grid((a.tokens + 1) / 2);
#define ATLAS_KV_ROW(V)                                                                          \
    if (vnorm)                                                                                   \
        hipLaunchKernelGGL((kv_append_row_kernel<FMT, true, V>), grid, dim3(256), 0, stream, a);  \
    else                                                                                         \
        hipLaunchKernelGGL((kv_append_row_kernel<FMT, false, V>), grid, dim3(256), 0, stream, a);
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
                           a.kv_width * sizeof(float), stream, a);
    else
        hipLaunchKernelGGL((kv_append_kernel<FMT, false, P>), dim3(a.tokens), dim3(kThreads), 0, stream, a);
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
