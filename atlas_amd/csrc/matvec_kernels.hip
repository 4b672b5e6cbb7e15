// matvec_kernels.hip -- RMS-folded Q4_0 decode projections for gfx950.
//
// Reference semantics (bisegni/atlas, crates/atlas-metal/src/kernels.metal):
//   matvec_q4_0_16row_mv_rms           :3786-3864  one projection
//   matmul_q4_0_qkv_16row_mv_rms       :3368-3467  Q, K and V in one dispatch
//   matmul_q4_0_gate_up_16row_mv_rms   :3468-3564  gate and up in one dispatch
//   gemma4_ple_gate_gelu_f32           :803-881    the PLE input gate: plain
//       matvec, then gelu(gate) * ple[ple_offset + row] (kernels.metal:773-801)
//   callers crates/atlas-model/src/gemma4_executor.rs:2082-2119, 2502-2612
//
// One decode token: output[o] = inv_rms(x) * sum_k (x_k * w_k) * deq(W[o, k]),
// with inv_rms(x) = 1 / sqrt(sum_k x_k^2 / n + eps) -- the RMS normalisation
// of the input folded into the dispatch (its scalar applied once per output,
// as the reference does).  Without an RMS weight it is the plain Q4_0 matvec.
// Q4_0 rows are 18-byte blocks of 32 values (f16 scale d, 16 bytes; value
// j < 16 is the low nibble of byte j, value j + 16 its high nibble, minus 8).
// The reference pins these kernels with a tolerance contract against a
// normalise-then-matvec CPU oracle (crates/atlas-metal/tests/
// matvec_rms_fused_parity.rs: max-abs < 1e-3); the summation order here is
// this kernel's own, deterministic run to run.
//
// Layout on CDNA: the op streams the weight matrix once (it is HBM-bound;
// MFMA does not apply to one token).  One wavefront owns a tile of 16
// consecutive output rows -- a contiguous byte range of the weight matrix --
// and stages it into LDS with 128-bit loads, all issued before the first
// wait.  Meanwhile the lanes form y = x * w (the normalised input before its
// scalar) in LDS with the per-block sums of y and the row sum of squares.
// Lane (g, s), g < 64/LPR, s < LPR, then keeps the y values of blocks
// s, s + LPR, ... in registers and applies them to rows g, g + 64/LPR, ...
// of the tile: 16 nibbles per byte pair decoded with masks and
// v_cvt_f32_ubyte, sum_j q_j * y_j accumulated in f32, and the Q4_0 offset
// folded as d * (acc - 8 * sum(y)).  The LPR partial sums of a row are
// reduced with cross-lane shuffles inside the row's lane group.
#include "device_common.hpp"
#include "launch.hpp"

namespace atlas {
namespace {

constexpr uint32_t kQ4Block = 18;  // bytes per 32 values

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Stage `bytes` (even) starting at `src` into LDS: 16-byte loads when the
// source is 16-byte aligned (the tail in 2-byte units), else 2-byte loads.
// A pass issues K loads per lane before the first LDS write (K = 4 covers a
// wavefront's 4 rows of 864 bytes, the Gemma hidden width, in one pass).  Load and store
// indices are both clamped to the last unit (lanes past the end copy that
// unit again, writing the value it already holds), so no access is
// conditional and the compiler cannot sink a load into a guarded store and
// serialise the pass.
template <int K, typename U>
__device__ __forceinline__ void stage_units(uint8_t* dst, const uint8_t* src, uint32_t units, uint32_t lane) {
    for (uint32_t base = 0; base < units; base += K * kWave) {
        U v[K];
#pragma unroll
        for (int k = 0; k < K; ++k) v[k] = reinterpret_cast<const U*>(src)[min(base + lane + k * kWave, units - 1)];
#pragma unroll
        for (int k = 0; k < K; ++k) reinterpret_cast<U*>(dst)[min(base + lane + k * kWave, units - 1)] = v[k];
    }
}

__device__ __forceinline__ void stage_tile(uint8_t* dst, const uint8_t* src, uint32_t bytes, uint32_t lane) {
    uint32_t done = 0;
    if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
        const uint32_t n16 = bytes / 16;
        if (n16) stage_units<4, uint4>(dst, src, n16, lane);
        done = n16 * 16;
    }
    if (bytes > done) stage_units<8, uint16_t>(dst + done, src + done, (bytes - done) / 2, lane);
}

// Sum over aligned groups of LPR lanes; every lane of a group gets the total.
// Inside a 16-lane DPP row the butterfly is quad_perm (xor 1, xor 2),
// row_half_mirror and row_mirror (VALU ops, no LDS); wider groups add
// cross-row shuffles.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f32<0xb1>(v);                 // quad_perm [1,0,3,2]
    v += dpp_f32<0x4e>(v);                 // quad_perm [2,3,0,1]
    if (LPR >= 8) v += dpp_f32<0x141>(v);   // row_half_mirror
    if (LPR >= 16) v += dpp_f32<0x140>(v);  // row_mirror
    if (LPR >= 32) v += __shfl_xor(v, 16, kWave);
    if (LPR >= 64) v += __shfl_xor(v, 32, kWave);
    return v;
}

// The Q4_0 block at LDS byte offset `off` (even): its f16 scale d and its
// 16 quant bytes as four dwords, read with 4-byte LDS loads.  An offset that
// is 0 mod 4 holds the scale in the low half of the first dword (the five
// dwords end 2 bytes past the block, still inside the LDS allocation); an
// offset that is 2 mod 4 holds it in the high half of the dword before the
// quant bytes, which are then dword aligned.
__device__ __forceinline__ void load_q4_block(const uint8_t* lds, uint32_t off, float& d, uint32_t (&q)[4]) {
    if ((off & 3) == 0) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(lds + off);
        const uint32_t w0 = p[0], w1 = p[1], w2 = p[2], w3 = p[3], w4 = p[4];
        d = h2f(static_cast<uint16_t>(w0));
        q[0] = __builtin_amdgcn_alignbit(w1, w0, 16);
        q[1] = __builtin_amdgcn_alignbit(w2, w1, 16);
        q[2] = __builtin_amdgcn_alignbit(w3, w2, 16);
        q[3] = __builtin_amdgcn_alignbit(w4, w3, 16);
    } else {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(lds + off - 2);
        d = h2f(static_cast<uint16_t>(p[0] >> 16));
        q[0] = p[1];
        q[1] = p[2];
        q[2] = p[3];
        q[3] = p[4];
    }
}

// sum_j q_j * y_j over one Q4_0 block's 32 values (nibble codes 0..15):
// byte j of q holds codes j (low nibble) and j + 16 (high nibble).
__device__ __forceinline__ float q4_block_dot(const uint32_t (&q)[4], const float (&y)[32]) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t lo = q[w] & 0x0f0f0f0fu, hi = (q[w] >> 4) & 0x0f0f0f0fu;
        // hide the masks' known-zero bits: knowing them, the compiler extracts
        // each nibble with a bitfield extract before a byte-0 conversion
        // (two instructions) instead of converting byte k directly (one)
        __asm__("" : "+v"(lo), "+v"(hi));
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // byte-wise conversions (v_cvt_f32_ubyte0..3)
            acc = __builtin_fmaf(static_cast<float>((lo >> (8 * k)) & 0xffu), y[4 * w + k], acc);
            acc = __builtin_fmaf(static_cast<float>((hi >> (8 * k)) & 0xffu), y[4 * w + k + 16], acc);
        }
    }
    return acc;
}

constexpr uint32_t kWaves = 4;  // wavefronts per workgroup
// y is stored block by block with a 36-float stride: the 16 or 32 lanes of
// a row group read 16-byte pieces of consecutive blocks, and a 144-byte
// stride puts those pieces on distinct LDS banks (a 128-byte stride would
// put them all on the same four).
constexpr uint32_t kYStride = 36;

// LPR lanes per output row (one row per lane group), NBT blocks per lane
// (blocks per row <= LPR * NBT).  A workgroup owns kWaves * 64 / LPR rows.
template <int LPR, int NBT, bool ONEPASS>
__global__ __launch_bounds__(256) void q4_0_matvec_kernel(MatvecArgs a) {
    constexpr uint32_t kGroups = kWave / LPR;           // rows per wavefront
    constexpr uint32_t kRows = kWaves * kGroups;        // rows per workgroup
    constexpr int kJ = (LPR * NBT * 32 / 4 + 255) / 256;  // float4 of x per thread
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const uint32_t g = lane / LPR, s = lane % LPR;
    const uint32_t n = a.input_width, n4 = n / 4, nb = n / 32, row_bytes = nb * kQ4Block;

    // The projection this workgroup's rows belong to (segments are tile ranges).
    const uint32_t t = blockIdx.x;
    const uint32_t si = (a.segments > 2 && t >= a.tile_begin[2]) ? 2 : ((a.segments > 1 && t >= a.tile_begin[1]) ? 1 : 0);
    const uint8_t* weights = si == 0 ? a.weights[0] : (si == 1 ? a.weights[1] : a.weights[2]);
    float* out = si == 0 ? a.output[0] : (si == 1 ? a.output[1] : a.output[2]);
    const uint32_t width = si == 0 ? a.width[0] : (si == 1 ? a.width[1] : a.width[2]);
    const uint32_t begin = si == 0 ? a.tile_begin[0] : (si == 1 ? a.tile_begin[1] : a.tile_begin[2]);
    const uint32_t row0 = (t - begin) * kRows;
    const uint32_t nrows = min(kRows, width - row0);
    // this wavefront's rows: [wrow0, wrow0 + wrows) of the tile
    const uint32_t wrow0 = min(wave * kGroups, nrows);
    const uint32_t wrows = min(kGroups, nrows - wrow0);

    uint8_t* tile = smem;                                                         // kRows * row_bytes
    float* ys = reinterpret_cast<float*>(smem + ((kRows * row_bytes + 15) & ~15u));  // nb * kYStride floats
    float* block_sums = ys + nb * kYStride;                                       // nb floats
    float* partial = block_sums + nb;                                             // kWaves floats

    // 1. input and RMS weight: every load of the workgroup issued up front
    //    (indices clamped, duplicates not stored)
    const bool rms = a.rms_weight != nullptr;
    f32x4 xv[kJ], wv[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const uint32_t c = min(tid + 256u * j, n4 - 1);
        xv[j] = reinterpret_cast<const f32x4*>(a.input)[c];
        wv[j] = rms ? reinterpret_cast<const f32x4*>(a.rms_weight)[c] : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
    }

    // 2. this wavefront's weight rows (the dominant stream), staged into LDS.
    //    ONEPASS (16-byte aligned rows of a 16-byte multiple, at most 4 KiB
    //    per wavefront -- four 864-byte rows): the loads land in registers
    //    and are written to LDS only after step 3, so y = x * w and the sums
    //    overlap the HBM round trip.  Loads and stores are unconditional, with
    //    clamped indices: a branch around either lets the compiler merge the
    //    registers or sink the loads to the stores, which waits for the data
    //    before step 3.  A wavefront without rows (the tail of the last tile)
    //    copies its tile's first row into the unused slot at row nrows.
    const uint8_t* wsrc = weights + static_cast<size_t>(row0 + (wrows ? wrow0 : 0u)) * row_bytes;
    const uint32_t n16 = (wrows ? wrows : 1u) * row_bytes / 16;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 w0, w1, w2, w3;
    if constexpr (ONEPASS) {
        const u32x4* src = reinterpret_cast<const u32x4*>(wsrc);  // read once: nontemporal
        w0 = __builtin_nontemporal_load(src + min(lane, n16 - 1));
        w1 = __builtin_nontemporal_load(src + min(lane + kWave, n16 - 1));
        w2 = __builtin_nontemporal_load(src + min(lane + 2 * kWave, n16 - 1));
        w3 = __builtin_nontemporal_load(src + min(lane + 3 * kWave, n16 - 1));
    } else {
        if (wrows) stage_tile(tile + wrow0 * row_bytes, wsrc, wrows * row_bytes, lane);
    }

    // 3. y = x * w (or x), the per-block sums of y (a block is 8 float4, held
    //    by 8 consecutive threads) and the sum of squares
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const uint32_t c = min(tid + 256u * j, n4 - 1);  // duplicates recompute the last float4
        const f32x4 x = xv[j], w = wv[j];
        f32x4 y = x;
        if (rms) y = f32x4{x.x * w.x, x.y * w.y, x.z * w.z, x.w * w.w};
        const float bsum = group_sum<8>((y.x + y.y) + (y.z + y.w));
        if (tid + 256u * j < n4) {
            if (rms) ss = ss + x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
            *reinterpret_cast<f32x4*>(ys + (c / 8) * kYStride + 4 * (c % 8)) = y;
            if (c % 8 == 0) block_sums[c / 8] = bsum;
        }
    }
    ss = group_sum<kWave>(ss);
    if (lane == 0) partial[wave] = ss;
    // y, the block sums and the partial sums are shared; the weight rows are
    // the wavefront's own, so it waits for its rows alone and starts its dot
    // while the workgroup's other rows may still be in flight (gate/up at
    // one token: 5.30 against 5.39 us with the rows written before the
    // barrier)
    __syncthreads();
    if constexpr (ONEPASS) {
        u32x4* dst = reinterpret_cast<u32x4*>(tile + wrow0 * row_bytes);
        dst[min(lane, n16 - 1)] = w0;
        dst[min(lane + kWave, n16 - 1)] = w1;
        dst[min(lane + 2 * kWave, n16 - 1)] = w2;
        dst[min(lane + 3 * kWave, n16 - 1)] = w3;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // The projection is held to a tolerance (this kernel's own summation
    // order), so the inverse RMS takes the hardware reciprocal and reciprocal
    // square root (each within 1 ulp): rsq(sum * rcp(n) + eps), a few ulp,
    // where the IEEE form (two divisions and a square root) costs ~45
    // instructions per wavefront.
    float inv = 1.0f;
    if (rms)
        inv = __builtin_amdgcn_rsqf(((partial[0] + partial[1]) + (partial[2] + partial[3])) *
                                        __builtin_amdgcn_rcpf(static_cast<float>(n)) + a.epsilon);

    // 4. lane (g, s): row wrow0 + g, blocks s + LPR * i
    const uint32_t row = wrow0 + g;
    float acc = 0.0f;
    if (g < wrows) {
        const uint32_t row_off = row * row_bytes;
#pragma unroll
        for (int i = 0; i < NBT; ++i) {
            const uint32_t b = s + LPR * i;
            if (b < nb) {
                float y[32];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(ys + kYStride * b + 4 * k);
                    y[4 * k] = v.x;
                    y[4 * k + 1] = v.y;
                    y[4 * k + 2] = v.z;
                    y[4 * k + 3] = v.w;
                }
                float d;
                uint32_t q[4];
                load_q4_block(tile, row_off + b * kQ4Block, d, q);
                acc = __builtin_fmaf(d, q4_block_dot(q, y) - 8.0f * block_sums[b], acc);
            }
        }
    }
    const float total = group_sum<LPR>(acc);
    if (s == 0 && g < wrows) {
        if (a.ple)  // PLE input gate: GELU of the projection times the layer's PLE slice
            out[row0 + row] = gelu_tanh_f32(total) * a.ple[a.ple_offset + row0 + row];
        else
            out[row0 + row] = rms ? total * inv : total;
    }
}

template <int LPR, int NBT>
hipError_t launch_lpr(hipStream_t stream, MatvecArgs a) {
    constexpr uint32_t kGroupsL = kWave / LPR;
    constexpr uint32_t kRows = kWaves * (kWave / LPR);
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < a.segments; ++i) {
        a.tile_begin[i] = tiles;
        tiles += (a.width[i] + kRows - 1) / kRows;
    }
    const uint32_t nb = a.input_width / 32;
    const size_t lds = ((kRows * nb * kQ4Block + 15) & ~15u) + (nb * kYStride + nb + kWaves) * sizeof(float);
    const uint32_t row_bytes = nb * kQ4Block;
    bool one_pass = row_bytes % 16 == 0 && kGroupsL * row_bytes <= 4 * kWave * 16;
    for (uint32_t i = 0; i < a.segments; ++i) one_pass = one_pass && (reinterpret_cast<uintptr_t>(a.weights[i]) & 15) == 0;
    if (one_pass)
        hipLaunchKernelGGL((q4_0_matvec_kernel<LPR, NBT, true>), dim3(tiles), dim3(kWaves * kWave), lds, stream, a);
    else
        hipLaunchKernelGGL((q4_0_matvec_kernel<LPR, NBT, false>), dim3(tiles), dim3(kWaves * kWave), lds, stream, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The PLE projection of one decode token, p[o] = fl(fl(sum_k input[k] *
// W[o, k]) * scale): matvec_f16 (kernels.metal:731-740) then
// scalar_multiply_f32; the launcher follows it with the stable group norm
// (kernels.metal:897-917) in place.  Caller gemma4_executor.rs:4184-4214
// (decode: ple_projection, its scale, ple_norm).  W is F16 [rows, hidden].
// Like the reference's F16 matvec (one thread per row, its compiler's own
// contraction) the dot is held to a tolerance.
// Layout: RPW rows per wavefront, four wavefronts per workgroup; lane l
// holds input columns 8l + 512c (c < HC) in registers and streams the same
// columns of its rows with 16-byte nontemporal loads, all issued before the
// first FMA; a tree reduction per row.  (The norm as this kernel's epilogue -- the
// last workgroup of each group normalising it -- needs a device-scope
// release per workgroup, an L2 write-back on each XCD: 25 us against 8 for
// two launches.)
// ---------------------------------------------------------------------------
constexpr uint32_t kPleMaxGroups = 1024;

// Kernel parameters of the PLE projection: PleProjArgs field by field (a
// by-value struct is not preloaded into SGPRs), counts first; all 56 bytes
// arrive in user SGPRs at wave launch (kernarg preload).
#define ATLAS_PP_KPARAMS                                                                                 \
    uint32_t p_hidden, uint32_t p_width, uint32_t p_groups, float p_scale, float p_epsilon,                \
        const float* p_input, const uint16_t* p_weights, const float* p_norm_weight, float* p_output
#define ATLAS_PP_UNPACK \
    const PleProjArgs a { p_input, p_weights, p_norm_weight, p_output, p_hidden, p_width, p_groups, p_scale, p_epsilon }
#define ATLAS_PP_KARGS(a) \
    (a).hidden, (a).width, (a).groups, (a).scale, (a).epsilon, (a).input, (a).weights, (a).norm_weight, (a).output

template <int HC, int RPW>
__global__ __launch_bounds__(256) void ple_proj_f16_kernel(ATLAS_PP_KPARAMS) {
    ATLAS_PP_UNPACK;
    const uint32_t tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const uint32_t hidden = a.hidden;
    const uint32_t row0 = blockIdx.x * (4 * RPW) + wave * RPW;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

    // the rows (the dominant stream) first; a column chunk past `hidden`
    // re-reads the row's last 8 columns and meets zero inputs
    u32x4 w[RPW][HC];
#pragma unroll
    for (int i = 0; i < RPW; ++i)
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            const uint32_t col = min(8 * lane + 512 * c, hidden - 8);
            w[i][c] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(a.weights + static_cast<size_t>(row0 + i) * hidden + col));
        }
    float x[HC][8];
#pragma unroll
    for (int c = 0; c < HC; ++c) {
        const uint32_t col = 8 * lane + 512 * c;
        const bool in = col < hidden;
        const f32x4* src = reinterpret_cast<const f32x4*>(a.input + min(col, hidden - 8));
        const f32x4 lo = src[0], hi = src[1];
        const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) x[c][j] = in ? v[j] : 0.0f;
    }
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int c = 0; c < HC; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                const uint32_t word = w[i][c][j / 2];
                acc[i] = __builtin_fmaf(h2f(static_cast<uint16_t>(j & 1 ? word >> 16 : word)), x[c][j], acc[i]);
            }
    float dot[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) dot[i] = wave_sum_tree_f32(acc[i]);
    if (lane < RPW) {
        float d = dot[0];
#pragma unroll
        for (int i = 1; i < RPW; ++i) d = lane == static_cast<uint32_t>(i) ? dot[i] : d;
        a.output[row0 + lane] = d * a.scale;
    }
}

}  // namespace

uint32_t q4_0_matvec_max_input() { return 32 * 4 * 32; }

hipError_t launch_q4_0_matvec(hipStream_t stream, MatvecArgs a) {
    const uint32_t nb = a.input_width / 32;
    uint32_t rows = 0;
    for (uint32_t i = 0; i < a.segments; ++i) rows += a.width[i];
    // Lanes per row: 16 (16 rows per workgroup) when that leaves at least
    // two workgroups per CU and each lane at <= 4 blocks; otherwise 32
    // (8 rows per workgroup, twice the workgroups for small projections).
    if (rows >= 16 * 512 && nb <= 64) {
        if (nb <= 16) return launch_lpr<16, 1>(stream, a);
        if (nb <= 32) return launch_lpr<16, 2>(stream, a);
        if (nb <= 48) return launch_lpr<16, 3>(stream, a);
        return launch_lpr<16, 4>(stream, a);
    }
    if (nb <= 32) return launch_lpr<32, 1>(stream, a);
    if (nb <= 64) return launch_lpr<32, 2>(stream, a);
    if (nb <= 96) return launch_lpr<32, 3>(stream, a);
    return launch_lpr<32, 4>(stream, a);
}

uint32_t ple_projection_max_hidden() { return 512 * 8; }
uint32_t ple_projection_max_groups() { return kPleMaxGroups; }

hipError_t launch_ple_projection_f16(hipStream_t stream, const PleProjArgs& a) {
    // two rows per wavefront (eight per workgroup): 10.45 us for the op at
    // Gemma's shape, against 10.6 with one row and 11.0 with four
    constexpr int kRpw = 2;
    const dim3 grid(a.groups * a.width / (4 * kRpw));
    const uint32_t hc = (a.hidden + 511) / 512;
#define ATLAS_PLE_PROJ(H) hipLaunchKernelGGL((ple_proj_f16_kernel<H, kRpw>), grid, dim3(kWaves * kWave), 0, stream, \
                                            ATLAS_PP_KARGS(a))
    if (hc <= 1)
        ATLAS_PLE_PROJ(1);
    else if (hc <= 2)
        ATLAS_PLE_PROJ(2);
    else if (hc <= 3)
        ATLAS_PLE_PROJ(3);
    else if (hc <= 4)
        ATLAS_PLE_PROJ(4);
    else if (hc <= 6)
        ATLAS_PLE_PROJ(6);
    else
        ATLAS_PLE_PROJ(8);
#undef ATLAS_PLE_PROJ
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // the projection is held to a tolerance, so the norm's sum takes the tree
    return launch_rms_norm_groups_stable_f32(stream, kWide, a.output, a.norm_weight, a.width, a.groups, a.epsilon);
}

}  // namespace atlas
