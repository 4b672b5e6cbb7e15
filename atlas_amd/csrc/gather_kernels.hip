// gather_kernels.hip -- token-embedding gathers (FP32, Q4_0, Q6_K) with the
// sqrt(hidden) scale fused in, and the Gemma per-layer-embedding (PLE)
// gather + dequant + combine.
//
// Reference semantics (bisegni/atlas):
//   embedding_lookup_f32            crates/atlas-metal/src/kernels.metal:94-104
//   embedding_lookup_q4_0           kernels.metal:653-656 (+ scalar_multiply_f32 :16-25)
//   embedding_lookup_q6_k/q6_k_value kernels.metal:663-692
//   block layouts / CPU dequant      crates/atlas-core/src/gguf.rs:379-438
//   PLE chain                        crates/atlas-model/src/gemma4_executor.rs:4162-4237
//                                    (gemma4_combine_ple crates/atlas-model/src/lib.rs:206-219)
//
// Layout on CDNA: one wavefront per gathered row (PLE: one 256-thread block
// per token).  The packed row (Q4_0: 18-byte blocks, Q6_K: 210-byte blocks,
// so rows are only 2/4/16-byte aligned depending on the width) is pulled into
// LDS with the widest coalesced load its alignment allows, then every lane
// unpacks four consecutive outputs from LDS with 16-bit reads and writes them
// with one 128-bit store.  Every dequantised value is exact in f32
// ((code - 8) * d for Q4_0; (code - 32) * scale * d for Q6_K), and the
// scale/combine steps keep the reference's rounding order, so outputs are
// bit-identical to the CPU dequant + scalar ops.
#include "device_common.hpp"
#include "launch.hpp"

namespace atlas {
namespace {

__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) {  // p is 2-byte aligned
    return *reinterpret_cast<const uint16_t*>(p);
}

// Packed table formats of the token gather (GgufTensorType, gguf.rs:16-77).
constexpr int kQuantQ4_0 = 0;
constexpr int kQuantQ6K = 1;
constexpr int kQuantQ8_0 = 2;

__host__ __device__ __forceinline__ uint32_t quant_row_bytes(int fmt, uint32_t hidden) {
    return fmt == kQuantQ6K ? (hidden / 256) * 210 : (hidden / 32) * (fmt == kQuantQ8_0 ? 34u : 18u);
}

// LDS bytes per staged row (16-byte slots).
__host__ __device__ __forceinline__ uint32_t quant_slot_bytes(int fmt, uint32_t hidden) {
    return (quant_row_bytes(fmt, hidden) + 15) & ~15u;
}

// Four consecutive Q4_0 values starting at column `col` (col % 4 == 0).
__device__ __forceinline__ void q4_0_decode4(const uint8_t* row, uint32_t col, float v[4]) {
    const uint32_t blk = (col >> 5) * 18;
    const uint32_t k = col & 31;
    const float d = h2f(static_cast<uint16_t>(lds_u16(row + blk)));
    const uint32_t off = blk + 2 + (k & 15);  // even
    const uint32_t lo = lds_u16(row + off), hi = lds_u16(row + off + 2);
    const uint32_t bytes = lo | (hi << 16);
    // the four nibbles as the bytes of one word; float(nib - 8) ==
    // float(nib) - 8 exactly
    const uint32_t nibs = (bytes >> (k < 16 ? 0 : 4)) & 0x0f0f0f0fu;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (static_cast<float>((nibs >> (8 * j)) & 0xffu) - 8.0f) * d;
}

// Four consecutive Q8_0 values starting at column `col` (col % 4 == 0):
// 34-byte blocks, f16 d then 32 signed bytes (gguf.rs:431-435); every
// product (int8 x f16) is exact in f32.
__device__ __forceinline__ void q8_0_decode4(const uint8_t* row, uint32_t col, float v[4]) {
    const uint32_t blk = (col >> 5) * 34;
    const uint32_t k = col & 31;
    const float d = h2f(static_cast<uint16_t>(lds_u16(row + blk)));
    const uint32_t off = blk + 2 + k;  // even
    const uint32_t bytes = lds_u16(row + off) | (lds_u16(row + off + 2) << 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = static_cast<float>(static_cast<int8_t>(bytes >> (8 * j))) * d;
}

// Four consecutive Q6_K values starting at column `col` (col % 4 == 0).
__device__ __forceinline__ void q6_k_decode4(const uint8_t* row, uint32_t col, float v[4]) {
    const uint32_t blk = (col >> 8) * 210;
    const uint32_t i = col & 255;
    const uint32_t half = i >> 7, w = i & 127, st = w >> 5, l = w & 31;
    const uint32_t ql_off = blk + half * 64 + l + ((st & 1) ? 32 : 0);
    const uint32_t qh_off = blk + 128 + half * 32 + l;
    const uint32_t ql = lds_u16(row + ql_off) | (lds_u16(row + ql_off + 2) << 16);
    const uint32_t qh = lds_u16(row + qh_off) | (lds_u16(row + qh_off + 2) << 16);
    const float sc = static_cast<float>(static_cast<int8_t>(row[blk + 192 + half * 8 + (l >> 4) + 2 * st]));
    const float d = h2f(static_cast<uint16_t>(lds_u16(row + blk + 208)));
    const uint32_t lshift = st >= 2 ? 4 : 0;
    // the four 6-bit codes as the bytes of one word: low nibbles and high
    // bit pairs extracted four at a time (q_j = byte j, 0..63)
    const uint32_t codes = ((ql >> lshift) & 0x0f0f0f0fu) | (((qh >> (2 * st)) & 0x03030303u) << 4);
    // The reference's (q * sc) * d as q * (sc * d): q * sc is exact (|q| <= 32,
    // |sc| <= 128) and so is sc * d (a 7-bit integer times an 11-bit f16
    // significand), so both are the one rounding of q * sc * d; a zero's sign
    // is the XOR of the three factors' signs in either grouping, and a NaN or
    // infinite d propagates alike.  One product per pass instead of one per
    // value.
    const float sd = sc * d;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // byte j to float in one conversion (v_cvt_f32_ubyte<j>); the empty
        // asm keeps the compiler from turning float(q) - 32 back into an
        // integer subtraction and a conversion.  float(q) - 32 ==
        // float(q - 32) exactly (small integers; q = 32 gives +0 either way).
        float q = static_cast<float>((codes >> (8 * j)) & 0xffu);
        __asm__("" : "+v"(q));
        v[j] = (q - 32.0f) * sd;
    }
}

// Copy `units` elements of type U from global `src` to LDS `dst` with
// threads [0, nthreads).  Each pass issues K loads per thread before the
// first LDS write, so a row costs one HBM round trip per pass instead of one
// per load (a plain copy loop waits on every load).  K is sized per call
// site to the row: extra guarded slots cost registers and branches.
template <int K, typename U>
__device__ __forceinline__ void stage_units(uint8_t* dst, const uint8_t* src, uint32_t units, uint32_t tid,
                                            uint32_t nthreads) {
    for (uint32_t base = 0; base < units; base += K * nthreads) {
        U v[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const uint32_t i = base + tid + k * nthreads;
            if (i < units) v[k] = reinterpret_cast<const U*>(src)[i];
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const uint32_t i = base + tid + k * nthreads;
            if (i < units) reinterpret_cast<U*>(dst)[i] = v[k];
        }
    }
}

// Copy `bytes` (even) from global `src` to LDS `dst` with the widest
// access the source alignment permits; threads [0, nthreads).  K16 / K4 /
// K2: loads in flight per thread for 16-, 4- and 2-byte accesses.
template <int K16, int K4, int K2>
__device__ __forceinline__ void stage_row(uint8_t* dst, const uint8_t* src, uint32_t bytes,
                                          uint32_t tid, uint32_t nthreads) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(src);
    if ((a & 15) == 0 && (bytes & 15) == 0)
        stage_units<K16, uint4>(dst, src, bytes / 16, tid, nthreads);
    else if ((a & 3) == 0 && (bytes & 3) == 0)
        stage_units<K4, uint32_t>(dst, src, bytes / 4, tid, nthreads);
    else
        stage_units<K2, uint16_t>(dst, src, bytes / 2, tid, nthreads);
}

// Stage `units` UNIT-byte units of the row behind `rs` into LDS `dst` with
// the lanes of one wavefront.  Every load is unconditional -- lanes past the row
// re-read its last unit -- so a pass's K loads carry no exec-mask branches
// and are all in flight before the first LDS write; units past the row are
// not written.
template <int K, int UNIT>
__device__ __forceinline__ void stage_units_wave(uint8_t* dst, __amdgpu_buffer_rsrc_t rs, uint32_t units,
                                                 uint32_t lane) {
    // units >= 1: the first pass needs no entry test, so nothing between the
    // id and the first row load waits on a branch
    uint32_t base = 0;
    do {
        u32x4_t v[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const uint32_t off = UNIT * min(base + lane + k * kWave, units - 1u);
            if constexpr (UNIT == 16)
                v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
            else if constexpr (UNIT == 4)
                v[k].x = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
            else
                v[k].x = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const uint32_t i = base + lane + k * kWave;
            if (i >= units) continue;
            if constexpr (UNIT == 16)
                reinterpret_cast<u32x4_t*>(dst)[i] = v[k];
            else if constexpr (UNIT == 4)
                reinterpret_cast<uint32_t*>(dst)[i] = v[k].x;
            else
                reinterpret_cast<uint16_t*>(dst)[i] = static_cast<uint16_t>(v[k].x);
        }
        base += K * kWave;
    } while (base < units);
}
typedef float f32x4 __attribute__((ext_vector_type(4)));

// FP32 gather: one wavefront per token; the id is wave-uniform (scalar load).
__global__ __launch_bounds__(64) void embed_f32_kernel(const float* __restrict__ table,
                                                       const uint32_t* __restrict__ ids,
                                                       float* __restrict__ out, uint32_t vocab,
                                                       uint32_t hidden, float scale, int vec) {
    const uint32_t lane = threadIdx.x;
    const uint32_t t = blockIdx.x;
    const uint32_t id = ids[t];
    float* dst = out + static_cast<size_t>(t) * hidden;
    const bool valid = id < vocab;
    const float* src = table + static_cast<size_t>(valid ? id : 0) * hidden;
    const bool scaled = scale != 1.0f;
    if (vec) {
        const auto ro = span_rsrc(dst, hidden * 4u);
        for (uint32_t c = lane * 4; c < hidden; c += 4 * kWave) {
            f32x4 v = valid ? *reinterpret_cast<const f32x4*>(src + c) : f32x4{0.f, 0.f, 0.f, 0.f};
            if (scaled) v = f32x4{v.x * scale, v.y * scale, v.z * scale, v.w * scale};
            st_span4<kPolicyWriteThrough>(ro, 4u * c, v);
        }
    } else {
        for (uint32_t c = lane; c < hidden; c += kWave) {
            float v = valid ? src[c] : 0.0f;
            dst[c] = scaled ? v * scale : v;
        }
    }
}

// Q4_0 / Q6_K / Q8_0 gather: one token per wavefront, WPG wavefronts per
// workgroup.  The id arrives through a scalar load; the packed row is staged
// in the wavefront's own LDS slot (stage_row_wave), then each lane decodes
// four consecutive values
// per step and writes them with one 128-bit write-through store.  The
// handoff from the staging lanes to the decoding lanes is a wavefront-scope
// fence (no workgroup barrier).
template <int FMT, int WPG, int UNIT>
__global__ __launch_bounds__(64 * WPG) void embed_quant_kernel(const uint8_t* __restrict__ table,
                                                               const uint32_t* __restrict__ ids,
                                                               float* __restrict__ out, uint32_t vocab,
                                                               uint32_t hidden, uint32_t tokens, float scale) {
    extern __shared__ __align__(16) uint8_t lds_rows[];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    const uint32_t t = blockIdx.x * WPG + wave;
    const uint32_t row_bytes = quant_row_bytes(FMT, hidden);
    // No early exit before the row is staged, so every kernel argument is
    // loaded at once and the row loads follow the id directly.  A wavefront
    // past the last token (tokens >= 1) re-reads the last id; an id >= vocab
    // stages row 0 -- or nothing, through an empty range, when the table has
    // no rows -- and both skip their stores (the reference kernels leave
    // rows with such ids untouched).
    const uint32_t id = ids[min(t, tokens - 1u)];
    const bool valid = t < tokens && id < vocab;
    const auto rs = span_rsrc(table + static_cast<size_t>(valid ? id : 0u) * row_bytes, vocab ? row_bytes : 0u);
    uint8_t* slot = lds_rows + static_cast<size_t>(wave) * quant_slot_bytes(FMT, hidden);
    // UNIT: the widest access the table's alignment and row stride allow
    // (chosen on the host).  Loads per lane per pass: a C4 Q4_0 row is 54
    // units of 16 bytes, a Q8_0 row 102 units of 16 bytes, a Q6_K row 315
    // units of 4 bytes.
    constexpr int kLoads = UNIT == 16 ? (FMT == kQuantQ8_0 ? 2 : 1) : (UNIT == 4 ? 5 : 8);
    stage_units_wave<kLoads, UNIT>(slot, rs, row_bytes / UNIT, lane);
    if (!valid) return;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // A pass of the wavefront covers 256 columns: 8 Q4_0 / Q8_0 blocks or
    // one Q6_K super-block, so a lane's column within its pass (lane * 4)
    // and every offset derived from it are the same on every pass; only the
    // pass's byte position in the row advances (Q6_K at C4: 6.17-6.24 us
    // against 6.24-6.33 with every offset derived from the column).
    constexpr uint32_t kPassBytes = FMT == kQuantQ6K ? 210u : (FMT == kQuantQ8_0 ? 8u * 34u : 8u * 18u);
    const auto ro = span_rsrc(out + static_cast<size_t>(t) * hidden, hidden * 4u);
    const uint8_t* pass = slot;
    for (uint32_t c = lane * 4; c < hidden; c += 4 * kWave) {
        float v[4];
        if (FMT == kQuantQ6K)
            q6_k_decode4(pass, lane * 4, v);
        else if (FMT == kQuantQ8_0)
            q8_0_decode4(pass, lane * 4, v);
        else
            q4_0_decode4(pass, lane * 4, v);
        st_span4<kPolicyWriteThrough>(ro, 4u * c, f32x4{v[0] * scale, v[1] * scale, v[2] * scale, v[3] * scale});
        pass += kPassBytes;
    }
}

// PLE gather-combine, one float4 per thread:
//   out[t, j] = ((deq(table[id])[j] * embedding_scale) + projection[t, j]) * output_scale
// Workgroup t * segments + s covers float4 [256 F s, 256 F (s + 1)) of token
// t's row, thread i the float4 256 F s + 256 f + i (f < F), and stages only
// that segment's table bytes (1024 F values: 32 F Q4_0 blocks of 18 bytes,
// or 4 F Q6_K super-blocks of 210; the segment starts on a block boundary).
template <bool Q6, int F>
__global__ __launch_bounds__(256) void ple_seg_kernel(const uint8_t* __restrict__ table,
                                                      const uint32_t* __restrict__ ids,
                                                      const float* __restrict__ projection,
                                                      float* __restrict__ out, uint32_t vocab,
                                                      uint32_t row_elems, uint32_t segments,
                                                      float embedding_scale, float output_scale) {
    __shared__ __align__(16) uint8_t seg[Q6 ? 4 * F * 210 : 32 * F * 18];
    const uint32_t t = blockIdx.x / segments;
    const uint32_t sg = blockIdx.x - t * segments;
    const uint32_t n4 = row_elems / 4;
    const size_t base = static_cast<size_t>(t) * row_elems;
    // no early exit on the id: the projection loads stay ahead of the id's
    // round trip and the table's (an invalid id stages nothing and skips the
    // store, so its output stays untouched; the id is workgroup-uniform)
    f32x4 q[F];
#pragma unroll
    for (int f = 0; f < F; ++f) {
        const uint32_t c4 = 256u * (F * sg + f) + threadIdx.x;
        q[f] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(projection + base) + min(c4, n4 - 1));
    }
    const uint32_t id_raw = ids[t];
    const bool valid = id_raw < vocab;
    const uint32_t id = valid ? id_raw : 0u;
    const uint32_t v0 = 1024u * F * sg;
    const uint32_t seg_vals = min(1024u * F, row_elems - v0);
    const uint32_t row_bytes = Q6 ? (row_elems / 256) * 210 : (row_elems / 32) * 18;
    const uint32_t seg_off = Q6 ? (v0 / 256) * 210 : (v0 / 32) * 18;
    const uint32_t seg_bytes = Q6 ? (seg_vals / 256) * 210 : (seg_vals / 32) * 18;
    if (valid)
        stage_row<1, 4, 8>(seg, table + static_cast<size_t>(id) * row_bytes + seg_off, seg_bytes, threadIdx.x,
                           256u);  // the launch's workgroup size (no implicit-argument load)
    __syncthreads();
    const auto ro = span_rsrc(out + base, row_elems * 4u);
#pragma unroll
    for (int f = 0; f < F; ++f) {
        const uint32_t c4 = 256u * (F * sg + f) + threadIdx.x;
        if (valid && c4 < n4) {
            float v[4];
            if (Q6)
                q6_k_decode4(seg, 4 * c4 - v0, v);
            else
                q4_0_decode4(seg, 4 * c4 - v0, v);
            st_span4<kPolicyWriteThrough>(ro, 16u * c4, f32x4{(v[0] * embedding_scale + q[f].x) * output_scale,
                                              (v[1] * embedding_scale + q[f].y) * output_scale,
                                              (v[2] * embedding_scale + q[f].z) * output_scale,
                                              (v[3] * embedding_scale + q[f].w) * output_scale});
        }
    }
}

// One launch covers at most 2^31 - 1 workgroups; longer token ranges are
// split into several launches over consecutive tokens.
template <bool Q6>
hipError_t launch_ple_it(hipStream_t stream, const uint8_t* table, const uint32_t* ids, const float* projection,
                         float* out, uint32_t vocab, uint32_t row_elems, uint32_t tokens, float es, float os) {
    // two float4 per thread (2048 values per workgroup): the projection
    // loads of both go out before the id's and the table's round trips.
    // C4: 48.5 us against 49.8 with one float4 and 49.6 / 49.9 with three /
    // four (a 8960-value row splits into 4 x 2048 + 768)
    constexpr int kF = 2;
    const uint32_t segments = (row_elems / 4 + 256 * kF - 1) / (256 * kF);
    const uint32_t per_launch = 0x7fffffffu / segments;
    for (uint32_t t0 = 0; t0 < tokens; t0 += per_launch) {
        const uint32_t n = min(per_launch, tokens - t0);
        const size_t off = static_cast<size_t>(t0) * row_elems;
        hipLaunchKernelGGL((ple_seg_kernel<Q6, kF>), dim3(n * segments), dim3(256), 0, stream, table, ids + t0,
                           projection + off, out + off, vocab, row_elems, segments, es, os);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_embed_f32(hipStream_t stream, const float* table, const uint32_t* ids, float* out,
                            uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale) {
    const int vec = (hidden % 4) == 0 && (reinterpret_cast<uintptr_t>(table) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    hipLaunchKernelGGL(embed_f32_kernel, dim3(tokens), dim3(kWave), 0, stream, table, ids, out, vocab, hidden,
                       scale, vec);
    return hipGetLastError();
}

template <int FMT, int WPG>
hipError_t launch_embed_quant_cfg(hipStream_t stream, const uint8_t* table, const uint32_t* ids, float* out,
                                  uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale) {
    const size_t lds = static_cast<size_t>(WPG) * quant_slot_bytes(FMT, hidden);
    const dim3 grid((tokens + WPG - 1) / WPG), block(64 * WPG);
    const uint32_t al = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(table)) | quant_row_bytes(FMT, hidden);
    if ((al & 15u) == 0)
        hipLaunchKernelGGL((embed_quant_kernel<FMT, WPG, 16>), grid, block, lds, stream, table, ids, out, vocab,
                           hidden, tokens, scale);
    else if ((al & 3u) == 0)
        hipLaunchKernelGGL((embed_quant_kernel<FMT, WPG, 4>), grid, block, lds, stream, table, ids, out, vocab,
                           hidden, tokens, scale);
    else
        hipLaunchKernelGGL((embed_quant_kernel<FMT, WPG, 2>), grid, block, lds, stream, table, ids, out, vocab,
                           hidden, tokens, scale);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_embed_fmt(hipStream_t stream, const uint8_t* table, const uint32_t* ids, float* out,
                            uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale) {
    // Wavefronts per workgroup, measured on MI355X at C4 (4096 tokens, hidden
    // 1536; sc0|sc1|nt stores, host-selected staging unit): Q4_0 5.09 us
    // with one, 5.12 with two, 5.19 with four, 5.20-5.25 with eight or
    // sixteen; Q6_K 5.42 us with two, 5.51-5.58 with one, 5.46 with four.
    // Decode batches take one (256 tokens spread over 256 CUs), and so do
    // rows whose two slots would not fit 64 KiB of LDS.
    const bool two = FMT != kQuantQ4_0 && tokens >= 2048 && 2u * quant_slot_bytes(FMT, hidden) <= 65536u;
    return two ? launch_embed_quant_cfg<FMT, 2>(stream, table, ids, out, vocab, hidden, tokens, scale)
               : launch_embed_quant_cfg<FMT, 1>(stream, table, ids, out, vocab, hidden, tokens, scale);
}

// One token per wavefront.  Measured and not kept at C4: two or four tokens
// per wavefront (Q4_0 5.7-7.0 us, Q6_K 7.0-9.1 us: a wavefront's second row
// waits behind its first), staging a Q6_K row as 16-byte loads of the aligned
// span around it (6.7 against 5.6 us).
hipError_t launch_embed_quant(hipStream_t stream, int format, const uint8_t* table, const uint32_t* ids,
                              float* out, uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale) {
    switch (format) {
        case kQuantQ4_0: return launch_embed_fmt<kQuantQ4_0>(stream, table, ids, out, vocab, hidden, tokens, scale);
        case kQuantQ6K: return launch_embed_fmt<kQuantQ6K>(stream, table, ids, out, vocab, hidden, tokens, scale);
        case kQuantQ8_0: return launch_embed_fmt<kQuantQ8_0>(stream, table, ids, out, vocab, hidden, tokens, scale);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_ple_quant(hipStream_t stream, int q6k, const uint8_t* table, const uint32_t* ids,
                            const float* projection, float* out, uint32_t vocab, uint32_t layers,
                            uint32_t width, uint32_t tokens, float embedding_scale, float output_scale) {
    const uint32_t row_elems = layers * width;
    if (q6k)
        return launch_ple_it<true>(stream, table, ids, projection, out, vocab, row_elems, tokens, embedding_scale,
                                   output_scale);
    return launch_ple_it<false>(stream, table, ids, projection, out, vocab, row_elems, tokens, embedding_scale,
                                output_scale);
}

}  // namespace atlas
