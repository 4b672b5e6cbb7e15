// norm_kernels.hip -- RMSNorm family for gfx950.
//
// Reference semantics (bisegni/atlas):
//   rms_norm_f32                 crates/atlas-metal/src/kernels.metal:106-114
//   gemma4_rms_residual_f32      kernels.metal:183-214
//   gemma4_ple_rms_add_scale_f32 kernels.metal:228-258
//   vector_add + rms_norm        crates/atlas-model/src/executor.rs:1258-1286
//   rms_norm_groups_in_place_stable_f32  kernels.metal:897-917
//   CPU operator (parity target) crates/atlas-ops/tests/phase_02_operators.rs:223-242
//
// Two reduction orders for the per-row sum of squares:
//
//  * Sequential (default).  The CPU operator folds x_i*x_i left to right in
//    f32.  Fused epilogues (residual add, RoPE rotation) cancel, so any other
//    order shows up as >1e-5 relative error on some elements; this engine
//    reproduces the fold bit-for-bit.  One wavefront owns ROWS rows: all 64
//    lanes stream the rows with 128-bit coalesced loads and write the squares
//    to LDS (row stride hidden+4 floats, so the ROWS chain lanes hit distinct
//    bank groups), then lane r folds row r's squares from LDS with
//    ds_read_b128 in index order, and all lanes apply the epilogue.  Rows are
//    fully read before any output is written, so in-place and aliased calls
//    (x == out, normalized == x, residual_out == x) are safe.
//
//  * Wide.  One wavefront per row, per-lane partial sums and a cross-lane
//    butterfly: the reference's rms_norm_decode_batch_f32 strategy
//    (kernels.metal:119-133).  Tolerance-level against the CPU operator.
#include "device_common.hpp"
#include "launch.hpp"


namespace atlas {
namespace {

struct f4 {
    float x, y, z, w;
};

__device__ __forceinline__ f4 ld4(const float* p) {
    float4 v = *reinterpret_cast<const float4*>(p);
    return {v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ void st4(float* p, f4 v) {
    *reinterpret_cast<float4*>(p) = make_float4(v.x, v.y, v.z, v.w);
}

// Row epilogue shared by both engines.  `inv` is the row's inverse RMS.
template <int MODE>
__device__ __forceinline__ float epilogue(const NormArgs& a, size_t idx, float xv, float inv,
                                          float w, float scale) {
    float n = xv * inv * w;
    if (MODE == kNormPlain || MODE == kNormAddNorm) return n;
    if (MODE == kNormResidual) {
        if (a.normalized) a.normalized[idx] = n;
        return a.residual[idx] + n;
    }
    // kNormAddScale: out aliases state
    return (a.out[idx] + n) * scale;
}

// Kernel parameters of the NormArgs engines.  A by-value struct is not
// preloaded into SGPRs, so the fields are passed one by one, in this order:
// the counts and the pointers the first loads need (and epsilon) fill the
// first 56 bytes, which arrive in user SGPRs at wave launch (kernarg
// preload), so a wavefront's first row load waits on no scalar load; the
// outputs written only at the end follow.  wpb (wavefronts per workgroup)
// and pair_stride (the row distance of a wavefront's second row) come from
// the host instead of blockDim / gridDim, which are kernarg loads too.
#define ATLAS_NORM_KPARAMS                                                                               \
    uint32_t p_rows, uint32_t p_hidden, uint32_t wpb, uint32_t pair_stride, const float* p_x,              \
        const float* p_residual, const float* p_weight, float* p_out, float p_epsilon, float* p_normalized, \
        float* p_residual_out, const float* p_scale
#define ATLAS_NORM_UNPACK                                                                                  \
    const NormArgs a {                                                                                     \
        p_x, p_weight, p_residual, p_normalized, p_residual_out, p_out, p_scale, p_rows, p_hidden, p_epsilon \
    }
#define ATLAS_NORM_KARGS(a, wpb, pair_stride)                                                                   \
    (a).rows, (a).hidden, (wpb), (pair_stride), (a).x, (a).residual, (a).weight, (a).out, (a).epsilon,          \
        (a).normalized, (a).residual_out, (a).scale

template <int ROWS, int MODE, bool VEC>
__global__ __launch_bounds__(64) void rms_seq_kernel(ATLAS_NORM_KPARAMS) {
    ATLAS_NORM_UNPACK;
    extern __shared__ float lds[];
    const uint32_t lane = threadIdx.x;
    const uint32_t h = a.hidden;
    const uint32_t stride = VEC ? h + 4 : h + 1;
    const uint32_t row0 = blockIdx.x * ROWS;
    const uint32_t nrows = min(static_cast<uint32_t>(ROWS), a.rows - row0);
    float* inv_lds = lds + ROWS * stride;

    // Phase A: coalesced loads, squares to LDS.
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        if (r >= static_cast<int>(nrows)) break;
        const size_t base = static_cast<size_t>(row0 + r) * h;
        float* sq = lds + r * stride;
        if (VEC) {
            for (uint32_t c = lane * 4; c < h; c += 4 * kWave) {
                f4 x = ld4(a.x + base + c);
                if (MODE == kNormAddNorm) {
                    f4 res = ld4(a.residual + base + c);
                    x = {x.x + res.x, x.y + res.y, x.z + res.z, x.w + res.w};
                    st4(a.residual_out + base + c, x);
                }
                st4(sq + c, {x.x * x.x, x.y * x.y, x.z * x.z, x.w * x.w});
            }
        } else {
            for (uint32_t c = lane; c < h; c += kWave) {
                float x = a.x[base + c];
                if (MODE == kNormAddNorm) {
                    x = x + a.residual[base + c];
                    a.residual_out[base + c] = x;
                }
                sq[c] = x * x;
            }
        }
    }
    __syncthreads();

    // Phase B: lane r folds row r in index order.
    if (lane < nrows) {
        const float* sq = lds + lane * stride;
        float s = 0.0f;
        if (VEC) {
#pragma unroll 8
            for (uint32_t c = 0; c < h; c += 4) {
                float4 v = *reinterpret_cast<const float4*>(sq + c);
                s = s + v.x;
                s = s + v.y;
                s = s + v.z;
                s = s + v.w;
            }
        } else {
            for (uint32_t c = 0; c < h; ++c) s = s + sq[c];
        }
        inv_lds[lane] = inverse_rms(s, static_cast<float>(h), a.epsilon);
    }
    __syncthreads();

    // Phase C: epilogue.
    const float scale = MODE == kNormAddScale ? *a.scale : 1.0f;
    const float* src = MODE == kNormAddNorm ? a.residual_out : a.x;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        if (r >= static_cast<int>(nrows)) break;
        const float inv = inv_lds[r];
        const size_t base = static_cast<size_t>(row0 + r) * h;
        if (VEC) {
            for (uint32_t c = lane * 4; c < h; c += 4 * kWave) {
                f4 x = ld4(src + base + c);
                f4 w = ld4(a.weight + c);
                f4 y;
                y.x = epilogue<MODE>(a, base + c + 0, x.x, inv, w.x, scale);
                y.y = epilogue<MODE>(a, base + c + 1, x.y, inv, w.y, scale);
                y.z = epilogue<MODE>(a, base + c + 2, x.z, inv, w.z, scale);
                y.w = epilogue<MODE>(a, base + c + 3, x.w, inv, w.w, scale);
                st4(a.out + base + c, y);
            }
        } else {
            for (uint32_t c = lane; c < h; c += kWave)
                a.out[base + c] = epilogue<MODE>(a, base + c, src[base + c], inv, a.weight[c], scale);
        }
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// Wide engine: one wave per row, 4 rows per 256-thread block.
template <int MODE, bool VEC>
__global__ __launch_bounds__(256) void rms_wide_kernel(ATLAS_NORM_KPARAMS) {
    ATLAS_NORM_UNPACK;
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t row = blockIdx.x * 4 + threadIdx.x / kWave;
    if (row >= a.rows) return;
    const uint32_t h = a.hidden;
    const size_t base = static_cast<size_t>(row) * h;
    float partial = 0.0f;
    if (VEC) {
        for (uint32_t c = lane * 4; c < h; c += 4 * kWave) {
            f4 x = ld4(a.x + base + c);
            if (MODE == kNormAddNorm) {
                f4 res = ld4(a.residual + base + c);
                x = {x.x + res.x, x.y + res.y, x.z + res.z, x.w + res.w};
                st4(a.residual_out + base + c, x);
            }
            partial = partial + x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
        }
    } else {
        for (uint32_t c = lane; c < h; c += kWave) {
            float x = a.x[base + c];
            if (MODE == kNormAddNorm) {
                x = x + a.residual[base + c];
                a.residual_out[base + c] = x;
            }
            partial = partial + x * x;
        }
    }
    const float inv = inverse_rms(wave_sum(partial), static_cast<float>(h), a.epsilon);
    const float scale = MODE == kNormAddScale ? *a.scale : 1.0f;
    const float* src = MODE == kNormAddNorm ? a.residual_out : a.x;
    if (VEC) {
        for (uint32_t c = lane * 4; c < h; c += 4 * kWave) {
            f4 x = ld4(src + base + c);
            f4 w = ld4(a.weight + c);
            f4 y;
            y.x = epilogue<MODE>(a, base + c + 0, x.x, inv, w.x, scale);
            y.y = epilogue<MODE>(a, base + c + 1, x.y, inv, w.y, scale);
            y.z = epilogue<MODE>(a, base + c + 2, x.z, inv, w.z, scale);
            y.w = epilogue<MODE>(a, base + c + 3, x.w, inv, w.w, scale);
            st4(a.out + base + c, y);
        }
    } else {
        for (uint32_t c = lane; c < h; c += kWave)
            a.out[base + c] = epilogue<MODE>(a, base + c, src[base + c], inv, a.weight[c], scale);
    }
}

// ---------------------------------------------------------------------------
// Tree engine: the tolerance-level reduction (ATLAS_REDUCTION_AUTO for the
// outputs that are a plain scaled row -- RMSNorm and the add-norm's y --
// and ATLAS_REDUCTION_WIDE for every mode).  Per lane, the squares of its
// float4 columns summed as ((a.x^2 + a.y^2) + (a.z^2 + a.w^2)) in column
// order, then wave_sum_tree_f32; the sum differs from the sequential fold by
// a few units in its last place, so outputs are within ~2e-6 relative of the
// CPU operator (1e-5 is the contract).
//
// Structure (16-byte aligned rows, hidden <= 2048): lane l keeps float4
// columns l + 64j (j < J) in VGPRs.  With PAIR, wavefront w owns rows w and
// w + G (G = the grid's wavefront count, rows/2 rounded up): it issues every
// load of both rows, then finishes row w (sum, stores) while row w + G is
// still landing, then row w + G.  Measured on MI355X at [4096, 1536]:
// 8.95-9.0 us, against 9.9 us with one row per wavefront and 9.3 us for a
// plain streaming copy of the same bytes; G must be exactly rows/2 (1536 or
// 2560 wavefronts of the same loop measured 10.3-10.9 us).  Without PAIR
// (fewer rows), one row per wavefront.  Every row is read completely before
// any of its outputs is written, so in-place and aliased calls are safe.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 ldg_nt(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
}
__device__ __forceinline__ f32x4 ldg(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ void stg_nt(float* p, f32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
}

// 128-bit store of float4 column `c` of a row whose base address is
// wavefront-uniform: POL < 0 a nontemporal global store, otherwise a buffer
// store with that cache policy (gfx950 bits: sc0 = 1, nt = 2, sc1 = 16)
// through a resource covering the row's `bytes`.
template <int POL>
__device__ __forceinline__ void st_row(float* row, uint32_t bytes, uint32_t c, f32x4 v) {
    if constexpr (POL < 0) {
        stg_nt(row + 4 * c, v);
    } else {
        typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(row, 0, bytes, 0x00020000);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), rs, 16u * c, 0, POL);
    }
}

template <int J, int MODE, int POL = -1>
struct TreeRow {
    static constexpr bool kOperand = MODE != kNormPlain;
    f32x4 x[J];
    f32x4 e[kOperand ? J : 1];

    __device__ __forceinline__ void load(const NormArgs& a, const float* operand, uint32_t row, uint32_t lane,
                                         uint32_t nv) {
        const size_t base = static_cast<size_t>(row) * a.hidden;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t c = min(lane + 64u * j, nv - 1);
            x[j] = ldg_nt(a.x + base + 4 * c);
            if (kOperand) e[j] = ldg_nt(operand + base + 4 * c);
        }
    }

    __device__ __forceinline__ void load_x(const NormArgs& a, uint32_t row, uint32_t lane, uint32_t nv) {
        const size_t base = static_cast<size_t>(row) * a.hidden;
#pragma unroll
        for (int j = 0; j < J; ++j) x[j] = ldg_nt(a.x + base + 4 * min(lane + 64u * j, nv - 1));
    }
    __device__ __forceinline__ void load_e(const NormArgs& a, const float* operand, uint32_t row, uint32_t lane,
                                           uint32_t nv) {
        const size_t base = static_cast<size_t>(row) * a.hidden;
        if (kOperand) {
#pragma unroll
            for (int j = 0; j < J; ++j) e[j] = ldg_nt(operand + base + 4 * min(lane + 64u * j, nv - 1));
        }
    }

    __device__ __forceinline__ void finish(const NormArgs& a, const f32x4 (&w)[J], uint32_t row, uint32_t lane,
                                           uint32_t nv, float scale) {
        const size_t base = static_cast<size_t>(row) * a.hidden;
        if (MODE == kNormAddNorm) {  // the stored residual stream r = x + residual
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const f32x4 v = x[j], b = e[j];
                x[j] = f32x4{v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w};
            }
        }
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const f32x4 v = x[j];
            const float q = (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
            p = p + (lane + 64u * j < nv ? q : 0.0f);
        }
        const float inv = inverse_rms(wave_sum_tree_f32(p), static_cast<float>(a.hidden), a.epsilon);
        const uint32_t rb = a.hidden * 4u;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t c = lane + 64u * j;
            if (c >= nv) continue;
            const f32x4 v = x[j], ww = w[j];
            const f32x4 n{v.x * inv * ww.x, v.y * inv * ww.y, v.z * inv * ww.z, v.w * inv * ww.w};
            if (MODE == kNormPlain) {
                st_row<POL>(a.out + base, rb, c, n);
            } else if (MODE == kNormAddNorm) {
                st_row<POL>(a.residual_out + base, rb, c, v);
                st_row<POL>(a.out + base, rb, c, n);
            } else if (MODE == kNormResidual) {
                if (a.normalized) st_row<POL>(a.normalized + base, rb, c, n);
                const f32x4 b = e[j];
                st_row<POL>(a.out + base, rb, c, f32x4{b.x + n.x, b.y + n.y, b.z + n.z, b.w + n.w});
            } else {
                const f32x4 b = e[j];
                st_row<POL>(a.out + base, rb, c,
                            f32x4{(b.x + n.x) * scale, (b.y + n.y) * scale, (b.z + n.z) * scale, (b.w + n.w) * scale});
            }
        }
    }
};

template <int J, int MODE, bool PAIR, bool DEFER = false, int POL = -1>
__global__ __launch_bounds__(256) void rms_tree_kernel(ATLAS_NORM_KPARAMS) {
    ATLAS_NORM_UNPACK;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    const uint32_t r0 = blockIdx.x * wpb + wave;
    if (r0 >= a.rows) return;  // wavefront-uniform
    const uint32_t r1 = r0 + pair_stride;
    const bool second = PAIR && r1 < a.rows;
    const uint32_t nv = a.hidden >> 2;
    const float* operand = MODE == kNormAddScale ? a.out : a.residual;
    TreeRow<J, MODE, POL> row0, row1;
    if constexpr (DEFER) {
        row0.load_x(a, r0, lane, nv);
        if (second) row1.load_x(a, r1, lane, nv);
        row0.load_e(a, operand, r0, lane, nv);
        if (second) row1.load_e(a, operand, r1, lane, nv);
    } else {
        row0.load(a, operand, r0, lane, nv);
        if (second) row1.load(a, operand, r1, lane, nv);
    }
    f32x4 w[J];
#pragma unroll
    for (int j = 0; j < J; ++j) w[j] = ldg(a.weight + 4 * min(lane + 64u * j, nv - 1));
    const float scale = MODE == kNormAddScale ? *a.scale : 1.0f;
    row0.finish(a, w, r0, lane, nv, scale);
    if (second) row1.finish(a, w, r1, lane, nv, scale);
}

// ---------------------------------------------------------------------------
// Register engine: sequential order, the default for 16-byte-aligned rows of
// at most 2048 floats.  One wavefront owns R rows.  Lane l keeps float4
// column c = l + 64*j (j < J) of each of its rows in registers, so HBM sees
// every input once and every output once:
//   1. every load of the wave is issued up front (the rows, the epilogue
//      operand -- residual or state -- and the weights), streamed with
//      nontemporal loads;
//   2. as chunk j lands, it is folded while later chunks are still in
//      flight.  The f32 fold is a dependent add chain (~8 cycles per add on
//      gfx950, ~12K cycles for 1536 values), so it must overlap the loads
//      rather than sit between the load and store phases.  Chunk 0 (256
//      values) always goes to LDS and lane r folds row r in index order.
//      Later chunks either do the same (PAR = false) or go through
//      fold_chunk_exact, the exact wave-parallel continuation of the fold
//      (PAR = true): same bits, a fraction of the latency, more VALU work;
//   3. lane r's inverse RMS is broadcast with readlane and every lane
//      finishes its columns with nontemporal stores.
// Each row is fully read before any of its outputs is written, so the
// aliased bindings of the reference call sites stay valid.
// ---------------------------------------------------------------------------
// The continuation's scans (fold_scan_ahead) as the helper wavefront leaves
// them in LDS for the folding wavefront.
template <int NB>
struct FoldScansLds {
    uint32_t inc[NB][64];
    uint32_t incl[NB][64];
    uint64_t bad[NB];
    uint32_t e0;
};

// RUN: helper wavefronts, one binade's scans each.  Measured on MI355X (C5
// epilogues, with the head folded by candidate segments): four helpers
// 4.54-4.56 us at 256 rows and 3.28-3.39 at one row, against 4.61-4.65 and
// 3.37-3.50 with two helpers of two binades each.
constexpr int kRunHelpers = 4;

template <int R, int J, int MODE, bool PAR, bool STAGE, bool RUN>
__global__ __launch_bounds__(RUN ? 64 * (kRunHelpers + 1) : 64) void rms_reg_kernel(ATLAS_NORM_KPARAMS) {
    ATLAS_NORM_UNPACK;
    // Squares of R rows, (hidden/4 + 1) float4 per row.  The load phase is
    // straight-line code (rows past the end and columns past the row width
    // are clamped to valid duplicate addresses and never stored), so the
    // compiler can wait for chunk j's loads alone before folding it.
    extern __shared__ f32x4 sq4[];
    constexpr bool kOperand = MODE != kNormPlain;
    // RUN: one row; kRunHelpers more wavefronts compute the continuation's
    // scans (fold_scan_ahead, one binade each) while the first folds the
    // head (head_fold_candidates)
    constexpr bool kRun = RUN && PAR && J > 1 && R == 1;
    constexpr int kRunS = 4 * (J > 1 ? J - 1 : 1);
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t h = a.hidden;
    const uint32_t nv = h >> 2;
    // RUN: a row's squares at their columns, zero-padded to 64 * J float4
    const uint32_t stride4 = kRun ? 64u * J + 1 : nv + 1;
    // the wavefront's R consecutive rows; the valid ones are r < nrows
    const uint32_t row0 = blockIdx.x * R;
    const uint32_t nrows = min(static_cast<uint32_t>(R), a.rows - row0);
    // second operand: residual (kNormResidual, kNormAddNorm) or state (kNormAddScale)
    const float* operand = MODE == kNormAddScale ? a.out : a.residual;
    FoldScansLds<4>* scans_lds = reinterpret_cast<FoldScansLds<4>*>(sq4 + stride4);
    // RUN: chunk 0's squares again, laid out for head_fold_candidates
    f32x4* head_pad = sq4 + stride4 + (sizeof(FoldScansLds<4>) + 15) / 16;
    // lane l's run: the 4 * (J - 1) consecutive squares from float4 64 + (J - 1) * l
    auto read_run = [&](float (&run)[kRunS]) {
#pragma unroll
        for (int i = 0; i < J - 1; ++i) {
            const f32x4 q = sq4[64u + (J - 1) * lane + i];
            run[4 * i] = q.x;
            run[4 * i + 1] = q.y;
            run[4 * i + 2] = q.z;
            run[4 * i + 3] = q.w;
        }
    };
    if constexpr (kRun) {
        if (threadIdx.x >= 64) {  // the helper wavefronts
            constexpr int kBph = 4 / kRunHelpers;
            const uint32_t b0 = kBph * (static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) - 1u);
            __syncthreads();  // every square staged
            const f32x4 h0 = sq4[lane];
            const float approx = wave_sum_any_order_f32((h0.x + h0.y) + (h0.z + h0.w));
            // any-order and in-order sums of 256 squares differ by < 3e-5
            // relative, so this is a lower bound of the head's exponent
            const uint32_t e0 = __float_as_uint(approx * 0.999f) >> 23;
            float run[kRunS];
            read_run(run);
            const FoldScans<kBph> f = fold_scan_ahead<kRunS, kBph>(run, e0 + b0);
#pragma unroll
            for (int b = 0; b < kBph; ++b) {
                scans_lds->inc[b0 + b][lane] = f.inc[b];
                scans_lds->incl[b0 + b][lane] = f.incl[b];
            }
            if (lane == 0) {
#pragma unroll
                for (int b = 0; b < kBph; ++b) scans_lds->bad[b0 + b] = f.bad[b];
                if (b0 == 0) scans_lds->e0 = e0;
            }
            __syncthreads();  // scans published
            return;
        }
    }

    f32x4 x[R][J];
    f32x4 e[kOperand ? R : 1][kOperand ? J : 1];
    f32x4 w[J];
    auto load_chunk = [&](int j, uint32_t zero) {
        const uint32_t c = min(lane + 64u * j, nv - 1) + zero;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t idx = static_cast<size_t>(row0 + min(static_cast<uint32_t>(r), nrows - 1)) * h + 4 * c;
            x[r][j] = ldg_nt(a.x + idx);
            if (kOperand) e[r][j] = ldg_nt(operand + idx);
        }
    };
    // STAGE: chunk 0 of every row in the grid is requested first; a wavefront
    // requests its later chunks only once its chunk 0 has landed (the zero
    // offset is produced by an instruction that waits on it), so chunk 0's
    // in-order fold runs while the later chunks are in flight instead of
    // after every chunk of the row has arrived together.
#pragma unroll
    for (int j = 0; j < (STAGE ? 1 : J); ++j) load_chunk(j, 0u);
#pragma unroll
    for (int j = 0; j < J; ++j) w[j] = ldg(a.weight + 4 * min(lane + 64u * j, nv - 1));
    if constexpr (STAGE) {
        uint32_t zero;
        __asm__ volatile("v_mov_b32 %0, 0" : "=v"(zero) : "v"(x[0][0].x));
#pragma unroll
        for (int j = 1; j < J; ++j) load_chunk(j, zero);
    }

    float s = 0.0f;  // lane r < nrows: running sum of squares of row r
    uint32_t sb[R];  // PAR: running sums of squares (bit patterns, wave-uniform)
    // In-order engine (!PAR): the row's last three chunks take the exact
    // wave-parallel fold instead (after the in-order chunks): the later
    // chunks of a row land together, and their in-order adds would run
    // after the read window closes.  Measured on MI355X at [4096, 1536],
    // residual, with both rows' scans side by side (means over three runs
    // per box, two boxes): the last three chunks 13.41 and 13.48 us, the
    // last two 13.46 and 13.50, the last one 13.49, every chunk after the
    // first 14.03; with the rows one after the other and the event lanes'
    // values broadcast from LDS, the last chunk 13.68 against 13.98 in
    // order, the last two 13.90, the last three 13.98.
    // (chunk 0 always folds in order: it sets the sum the tail continues)
    constexpr int kTailN = J > 3 ? 3 : J - 1;
    constexpr bool kTail = !PAR && J > 1;
    static_assert(!kTail || kTailN < J, "the in-order head must precede the parallel tail");
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t creal = lane + 64u * j;
        const uint32_t c = min(creal, nv - 1);
        const bool par_chunk = PAR ? j > 0 : (kTail && j >= J - kTailN);
        float sqr[R][4];  // a wave-parallel chunk's squares, row by row
#pragma unroll
        for (int r = 0; r < R; ++r) {
            f32x4 v = x[r][j];
            if (MODE == kNormAddNorm) {
                const f32x4 b = e[r][j];
                v = f32x4{v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w};
                x[r][j] = v;
            }
            if (!par_chunk) {
                sq4[r * stride4 + c] = f32x4{v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w};
                if (kRun && j == 0) head_pad[lane + lane / 16] = f32x4{v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w};
            } else if (kRun) {
                // staged for the one-step continuation below (+0 past the row
                // width: adding +0 leaves a sum of squares unchanged)
                sq4[r * stride4 + creal] = creal < nv ? f32x4{v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w}
                                                      : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            } else {
                // chunks after the first: exact wave-parallel fold (columns past
                // the row width hold clamped duplicates and contribute +0)
                const bool in_row = creal < nv;
                sqr[r][0] = in_row ? v.x * v.x : 0.0f;
                sqr[r][1] = in_row ? v.y * v.y : 0.0f;
                sqr[r][2] = in_row ? v.z * v.z : 0.0f;
                sqr[r][3] = in_row ? v.w * v.w : 0.0f;
            }
        }
        if (par_chunk && !kRun) {
            // two rows' scans side by side, else row by row (measured on
            // MI355X, residual at [4096, 1536]: 13.50-13.52 against
            // 13.63-13.65 us row by row; the inverse RMS likewise one chain
            // for both rows, below)
            if (R == 2 && nrows == 2) {
                fold_chunk_exact_pair<4>(sqr[0], sb[0], sqr[R - 1], sb[R - 1]);
            } else {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (static_cast<uint32_t>(r) < nrows) sb[r] = fold_chunk_exact<4>(sqr[r], sb[r]);
            }
        }
        if (!par_chunk && !kRun) {
            __syncthreads();
            if (lane < nrows)
                s = fold_lds_chunk(sq4 + lane * stride4 + 64u * j, min(nv, 64u * (j + 1)) - 64u * j, s);
        }
        if ((PAR && !kRun && j == 0) || (kTail && j == J - kTailN - 1)) {
            // the first chunk, where the sum crosses many binades and ties are
            // frequent, folds in order; broadcast each row's partial sum
#pragma unroll
            for (int r = 0; r < R; ++r) sb[r] = readlane_u32(__float_as_uint(s), static_cast<uint32_t>(r));
        }
    }
    if constexpr (kRun) {
        // The continuation (columns 256 .. 256 * J) as one run.  The helper
        // wavefronts compute its scans for four binades from a lower bound
        // of the head's exponent while this one folds the head (four
        // segments folded from candidate starts and chained by selection,
        // 5.13 -> 4.61 us per C5 epilogue at 256 rows with two helpers);
        // the walk then has only the fold's real events (binade crossings,
        // ties) left.
        __syncthreads();  // every square staged
        const float head = head_fold_candidates(head_pad, lane);
        __syncthreads();  // the helper's scans published
        FoldScans<4> f;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            f.inc[b] = scans_lds->inc[b][lane];
            f.incl[b] = scans_lds->incl[b][lane];
            // readfirstlane returns int: widen through uint32_t (no sign extension)
            const uint64_t m = scans_lds->bad[b];
            const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(m)));
            const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(m >> 32)));
            f.bad[b] = static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
        }
        f.e0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(scans_lds->e0));
        float run[kRunS];
        read_run(run);
        sb[0] = fold_walk<kRunS, 4>(f, run, __float_as_uint(head));
    }
    if (MODE == kNormAddNorm) {  // stored residual stream r = x + residual
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (static_cast<uint32_t>(r) >= nrows) break;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const uint32_t c = lane + 64u * j;
                if (c < nv) stg_nt(a.residual_out + static_cast<size_t>(row0 + r) * h + 4 * c, x[r][j]);
            }
        }
    }

    // lane r < nrows: row r's inverse RMS, one chain for every row (the
    // wave-parallel fold leaves row r's sum in sb[r], the in-order one in
    // lane r's s).  A single row with the wave-parallel fold computes it
    // uniformly instead, without the readlane.  Measured on MI355X: the
    // residual epilogue at [4096, 1536] (two rows) 13.61-13.62 against
    // 13.67-13.79 us with a chain per row; C5 at 256 rows (one) 4.74-4.79
    // against 4.70-4.73 with the readlane.
    constexpr bool kUniform = (PAR || kTail) && R == 1;
    float sum_r = s;
    if constexpr (PAR || kTail) {
        uint32_t mine = sb[0];
#pragma unroll
        for (int r = 1; r < R; ++r) mine = lane == static_cast<uint32_t>(r) ? sb[r] : mine;
        sum_r = __uint_as_float(mine);
    }
    const float inv = lane < nrows ? inverse_rms(sum_r, static_cast<float>(h), a.epsilon) : 0.0f;
    const float scale = MODE == kNormAddScale ? *a.scale : 1.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (static_cast<uint32_t>(r) >= nrows) break;
        const float ir = kUniform ? inverse_rms(__uint_as_float(sb[0]), static_cast<float>(h), a.epsilon)
                                  : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), r));
        const size_t base = static_cast<size_t>(row0 + r) * h;
        f32x4 n[J];
        auto emit = [&](int j) {
            const uint32_t c = lane + 64u * j;
            const f32x4 v = x[r][j], ww = w[j];
            n[j] = f32x4{v.x * ir * ww.x, v.y * ir * ww.y, v.z * ir * ww.z, v.w * ir * ww.w};
            if (MODE == kNormPlain || MODE == kNormAddNorm) {
                stg_nt(a.out + base + 4 * c, n[j]);
            } else if (MODE == kNormResidual) {
                const f32x4 b = e[r][j], q = n[j];
                stg_nt(a.out + base + 4 * c, f32x4{b.x + q.x, b.y + q.y, b.z + q.z, b.w + q.w});
            } else {
                const f32x4 b = e[r][j], q = n[j];
                stg_nt(a.out + base + 4 * c,
                       f32x4{(b.x + q.x) * scale, (b.y + q.y) * scale, (b.z + q.z) * scale, (b.w + q.w) * scale});
            }
        };
        // a row that fills every lane's J float4 stores straight-line code;
        // one that does not guards each float4
        const bool full = nv == 64u * J;
        if (full) {
#pragma unroll
            for (int j = 0; j < J; ++j) emit(j);
        } else {
#pragma unroll
            for (int j = 0; j < J; ++j)
                if (lane + 64u * j < nv) emit(j);
        }
        if (MODE == kNormResidual && a.normalized) {
#pragma unroll
            for (int j = 0; j < J; ++j)
                if (full || lane + 64u * j < nv) stg_nt(a.normalized + base + 4 * (lane + 64u * j), n[j]);
        }
    }
}

// Register-engine configuration: rows per wavefront and the fold of the
// chunks after the first (exact wave-parallel, or in order from LDS).  Same
// bits either way.  Measured on MI355X:
//  * rows < 2048 (decode batches): one row per wavefront and the parallel
//    fold -- the in-order chain is fully exposed there (C5 decode step at
//    256 rows: 35.9 -> 30.3 us per layer);
//  * rows >= 2048, plain RMSNorm: one row per wavefront, parallel fold
//    ([4096, 1536]: 11.7 -> 10.6 us);
//  * rows >= 2048 with an epilogue operand (residual, add-norm, add-scale):
//    two rows per wavefront (two wavefronts per SIMD) and the in-order fold
//    up to the last chunk ([4096, 1536] residual: 16.0 us; one row and the
//    parallel fold: 16.7; two rows with the parallel fold after the first
//    chunk, on the later engine: 14.9 against 13.7).
struct RegConfig {
    int rows;
    bool par;
};

RegConfig pick_reg(uint32_t rows, int mode) {
    if (rows >= 2048 && mode != kNormPlain) return RegConfig{2, false};
    return RegConfig{1, true};
}

// The continuation as one run with its scans computed ahead by helper
// wavefronts (RUN).  Measured on MI355X: decode batches gain (C5 step at 256
// rows: 29.5 -> 28.5 us per layer with one helper computing four binades,
// 27.8 -> 26.8 with two helpers of two binades each, whose scans then land
// before the head's in-order fold ends; kRunHelpers has the current count);
// from 2048 rows up the extra wavefronts per row cost more than they hide
// ([4096, 1536]: 10.3 -> 13.9 us with one helper).
bool norm_run(uint32_t rows) { return rows < 2048; }

template <int R, int J, int MODE>
hipError_t launch_reg_rj(hipStream_t s, const NormArgs& a, bool par) {
    // staged loads from 2048 rows up: plain RMSNorm 10.6 -> 10.2 us and the
    // residual epilogue 16.1 -> 15.5 us at [4096, 1536]; at decode batches
    // (256 rows) the extra round trip before the later chunks costs more
    // (30.2 -> 30.8 us per C5 layer).
    const bool stage = a.rows >= 2048;
    const bool run = par && J > 1 && R == 1 && norm_run(a.rows);
    const size_t lds = run ? (64u * J + 1 + (sizeof(FoldScansLds<4>) + 15) / 16 + 68) * sizeof(f32x4)
                           : static_cast<size_t>(R) * (a.hidden / 4 + 1) * sizeof(f32x4);
    const dim3 grid((a.rows + R - 1) / R);
    if constexpr (R == 1 && J > 1) {
        if (run) {
            hipLaunchKernelGGL((rms_reg_kernel<R, J, MODE, true, false, true>), grid, dim3((kRunHelpers + 1) * kWave),
                               lds, s, ATLAS_NORM_KARGS(a, 1u, 0u));
            return hipGetLastError();
        }
    }
    if (par && stage)
        hipLaunchKernelGGL((rms_reg_kernel<R, J, MODE, true, true, false>), grid, dim3(kWave), lds, s,
                           ATLAS_NORM_KARGS(a, 1u, 0u));
    else if (par)
        hipLaunchKernelGGL((rms_reg_kernel<R, J, MODE, true, false, false>), grid, dim3(kWave), lds, s,
                           ATLAS_NORM_KARGS(a, 1u, 0u));
    else if (stage)
        hipLaunchKernelGGL((rms_reg_kernel<R, J, MODE, false, true, false>), grid, dim3(kWave), lds, s,
                           ATLAS_NORM_KARGS(a, 1u, 0u));
    else
        hipLaunchKernelGGL((rms_reg_kernel<R, J, MODE, false, false, false>), grid, dim3(kWave), lds, s,
                           ATLAS_NORM_KARGS(a, 1u, 0u));
    return hipGetLastError();
}

template <int R, int MODE>
hipError_t launch_reg_r(hipStream_t s, const NormArgs& a, int J, bool par) {
    switch (J) {
        case 1: return launch_reg_rj<R, 1, MODE>(s, a, par);
        case 2: return launch_reg_rj<R, 2, MODE>(s, a, par);
        case 3: return launch_reg_rj<R, 3, MODE>(s, a, par);
        case 4: return launch_reg_rj<R, 4, MODE>(s, a, par);
        case 5: return launch_reg_rj<R, 5, MODE>(s, a, par);
        case 6: return launch_reg_rj<R, 6, MODE>(s, a, par);
        case 7: return launch_reg_rj<R, 7, MODE>(s, a, par);
        default: return launch_reg_rj<R, 8, MODE>(s, a, par);
    }
}

template <int MODE>
hipError_t launch_reg(hipStream_t s, const NormArgs& a) {
    const int J = static_cast<int>((a.hidden / 4 + 63) / 64);
    const RegConfig c = pick_reg(a.rows, MODE);
    if (c.rows == 2) return launch_reg_r<2, MODE>(s, a, J, c.par);
    return launch_reg_r<1, MODE>(s, a, J, c.par);
}

// Tree engine: two rows per wavefront (rows w and w + G) from 4096 rows up,
// one row per wavefront below that (fewer rows leave too few wavefronts to
// fill the chip when each takes two).
bool tree_pairs(uint32_t rows) { return rows >= 4096; }

// Wavefronts (rows) per workgroup: one below 2048 rows, so a decode batch
// spreads over every CU instead of a quarter of them (C5 epilogues at 256
// rows under ATLAS_REDUCTION_WIDE: 3.37 against 3.60 us), four above.
uint32_t tree_waves_per_group(uint32_t rows) { return rows < 2048 ? 1u : 4u; }

// The residual and add-scale epilogues need their operand only after the
// sum: it is requested after both rows' x (DEFER).  Measured on MI355X at
// [4096, 1536] (residual, ATLAS_REDUCTION_WIDE): 12.98-13.03 us against
// 13.63-13.64 with x and the operand requested row by row.  Stores are
// nontemporal buffer stores through a per-row resource (policy 2): at
// [4096, 1536] plain 8.57-8.58 us against 8.61-8.66 with global nontemporal
// stores; the sc1 and sc1 + nt store policies were slower (9.46, 9.19).
template <int J, int MODE>
hipError_t launch_tree_j(hipStream_t s, const NormArgs& a) {
    constexpr bool kDefer = MODE == kNormResidual || MODE == kNormAddScale;
    constexpr int kStorePolicy = 2;
    const bool pair = tree_pairs(a.rows);
    const uint32_t waves = pair ? (a.rows + 1) / 2 : a.rows;
    const uint32_t wpb = tree_waves_per_group(a.rows);
    const dim3 grid((waves + wpb - 1) / wpb);
    // a wavefront's second row is G = grid * wpb rows after its first
    const uint32_t pair_stride = grid.x * wpb;
    if (pair)
        hipLaunchKernelGGL((rms_tree_kernel<J, MODE, true, kDefer, kStorePolicy>), grid, dim3(64 * wpb), 0, s,
                           ATLAS_NORM_KARGS(a, wpb, pair_stride));
    else
        hipLaunchKernelGGL((rms_tree_kernel<J, MODE, false, kDefer, kStorePolicy>), grid, dim3(64 * wpb), 0, s,
                           ATLAS_NORM_KARGS(a, wpb, pair_stride));
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_tree(hipStream_t s, const NormArgs& a) {
    switch ((a.hidden / 4 + 63) / 64) {
        case 1: return launch_tree_j<1, MODE>(s, a);
        case 2: return launch_tree_j<2, MODE>(s, a);
        case 3: return launch_tree_j<3, MODE>(s, a);
        case 4: return launch_tree_j<4, MODE>(s, a);
        case 5: return launch_tree_j<5, MODE>(s, a);
        case 6: return launch_tree_j<6, MODE>(s, a);
        case 7: return launch_tree_j<7, MODE>(s, a);
        default: return launch_tree_j<8, MODE>(s, a);
    }
}

// Rows per wavefront for the sequential LDS engine: enough wavefronts to
// keep every SIMD streaming (>= 2048 for large row counts), bounded by 64 KB
// of LDS.
int pick_rows(uint32_t rows, uint32_t hidden) {
    int best = 1;
    for (int r : {2, 4, 8, 16}) {
        size_t lds = (static_cast<size_t>(r) * (hidden + 4) + r) * 4;
        if (lds > 65536) break;
        if ((rows + r - 1) / r >= 2048) best = r;
    }
    return best;
}

template <int ROWS, int MODE>
hipError_t launch_seq_rows(hipStream_t s, const NormArgs& a, bool vec) {
    const uint32_t stride = vec ? a.hidden + 4 : a.hidden + 1;
    const size_t lds = (static_cast<size_t>(ROWS) * stride + ROWS) * sizeof(float);
    const dim3 grid((a.rows + ROWS - 1) / ROWS);
    if (vec)
        hipLaunchKernelGGL((rms_seq_kernel<ROWS, MODE, true>), grid, dim3(kWave), lds, s,
                           ATLAS_NORM_KARGS(a, 1u, 0u));
    else
        hipLaunchKernelGGL((rms_seq_kernel<ROWS, MODE, false>), grid, dim3(kWave), lds, s,
                           ATLAS_NORM_KARGS(a, 1u, 0u));
    return hipGetLastError();
}

template <int MODE>
hipError_t launch_seq(hipStream_t s, const NormArgs& a, bool vec) {
    switch (pick_rows(a.rows, a.hidden)) {
        case 16: return launch_seq_rows<16, MODE>(s, a, vec);
        case 8: return launch_seq_rows<8, MODE>(s, a, vec);
        case 4: return launch_seq_rows<4, MODE>(s, a, vec);
        case 2: return launch_seq_rows<2, MODE>(s, a, vec);
        default: return launch_seq_rows<1, MODE>(s, a, vec);
    }
}

template <int MODE>
hipError_t launch_wide(hipStream_t s, const NormArgs& a, bool vec) {
    const dim3 grid((a.rows + 3) / 4);
    if (vec)
        hipLaunchKernelGGL((rms_wide_kernel<MODE, true>), grid, dim3(256), 0, s, ATLAS_NORM_KARGS(a, 4u, 0u));
    else
        hipLaunchKernelGGL((rms_wide_kernel<MODE, false>), grid, dim3(256), 0, s, ATLAS_NORM_KARGS(a, 4u, 0u));
    return hipGetLastError();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---------------------------------------------------------------------------
// Stable per-group RMSNorm (max-scaled), in place.  One wave per group:
// m = max|v| is order-free (wave max), the (v/m)^2 fold is sequential in
// index order on lane 0 from LDS, then all lanes rewrite the group.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void groups_stable_kernel(float* values, const float* weight,
                                                           uint32_t width, uint32_t groups,
                                                           float epsilon, int sequential) {
    extern __shared__ float sq[];
    const uint32_t g = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    if (g >= groups) return;
    float* v = values + static_cast<size_t>(g) * width;
    float m = 0.0f;
    for (uint32_t i = lane; i < width; i += kWave) m = fmaxf(m, fabsf(v[i]));
    m = wave_max(m);
    if (m == 0.0f) {
        for (uint32_t i = lane; i < width; i += kWave) v[i] = 0.0f;
        return;
    }
    float partial = 0.0f;
    for (uint32_t i = lane; i < width; i += kWave) {
        float scaled = fdiv_rn(v[i], m);
        float s2 = scaled * scaled;
        if (sequential)
            sq[i] = s2;
        else
            partial = partial + s2;
    }
    float sum;
    if (sequential) {
        __syncthreads();
        __shared__ float total;
        if (lane == 0) {
            float s = 0.0f;
            for (uint32_t i = 0; i < width; ++i) s = s + sq[i];
            total = s;
        }
        __syncthreads();
        sum = total;
    } else {
        sum = wave_sum(partial);
    }
    const float root = sqrt_rn(fdiv_rn(sum, static_cast<float>(width)) + fdiv_rn(epsilon, m * m));
    const float inv = fdiv_rn(fdiv_rn(1.0f, root), m);
    for (uint32_t i = lane; i < width; i += kWave) v[i] = v[i] * inv * weight[i];
}

// Groups of width <= 64 * PER: the same steps with the group and its norm
// weights held in registers (lane l: values l + 64k), one read and one write
// of global memory; the sequential fold stages the squares in LDS as above.
// The maximum and the tree sum take DPP steps (no LDS round trips): the
// PLE projection's norm launch, 35 groups of 256, is latency alone.
template <int PER>
__global__ __launch_bounds__(64) void groups_stable_reg_kernel(float* values, const float* weight, uint32_t width,
                                                               float epsilon, int sequential) {
    __shared__ __align__(16) float sq[64 * PER];
    const uint32_t lane = threadIdx.x;
    float* v = values + static_cast<size_t>(blockIdx.x) * width;
    float x[PER], w[PER];
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t i = lane + kWave * k;
        x[k] = i < width ? v[i] : 0.0f;
        w[k] = i < width ? weight[i] : 0.0f;
        m = fmaxf(m, fabsf(x[k]));
    }
    m = wave_max_tree_f32(m);
    if (m == 0.0f) {
#pragma unroll
        for (int k = 0; k < PER; ++k)
            if (lane + kWave * k < width) v[lane + kWave * k] = 0.0f;
        return;
    }
    float partial = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const uint32_t i = lane + kWave * k;
        const float scaled = fdiv_rn(x[k], m);
        const float s2 = scaled * scaled;
        if (sequential) {
            if (i < width) sq[i] = s2;
        } else if (i < width) {
            partial = partial + s2;
        }
    }
    float sum;
    if (sequential) {
        __syncthreads();
        __shared__ float total;
        if (lane == 0) {
            float s = 0.0f;
            if (width % 4 == 0)
                s = fold_lds_chunk(reinterpret_cast<const f32x4*>(sq), width / 4, 0.0f);
            else
                for (uint32_t i = 0; i < width; ++i) s = s + sq[i];
            total = s;
        }
        __syncthreads();
        sum = total;
    } else {
        sum = wave_sum_tree_f32(partial);
    }
    const float root = sqrt_rn(fdiv_rn(sum, static_cast<float>(width)) + fdiv_rn(epsilon, m * m));
    const float inv = fdiv_rn(fdiv_rn(1.0f, root), m);
#pragma unroll
    for (int k = 0; k < PER; ++k)
        if (lane + kWave * k < width) v[lane + kWave * k] = x[k] * inv * w[k];
}

// ---------------------------------------------------------------------------
// FP16-storage RMSNorm (optionally fused with the pre-norm residual add).
// Storage f16, math f32: widening is exact, outputs are rounded RNE.  With a
// residual, r = rne16(x + residual) is stored and the norm reads the stored
// value, matching the two-kernel chain with f16 buffers.
// ---------------------------------------------------------------------------
struct h8 {
    uint16_t v[8];
};

template <bool ADD>
__global__ __launch_bounds__(64) void rms_f16_seq_kernel(const uint16_t* x, const uint16_t* residual,
                                                         const uint16_t* weight,
                                                         uint16_t* residual_out, uint16_t* out,
                                                         uint32_t rows, uint32_t hidden,
                                                         float epsilon, int sequential) {
    extern __shared__ float sq[];
    __shared__ float inv_shared;
    const uint32_t row = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    if (row >= rows) return;
    const size_t base = static_cast<size_t>(row) * hidden;
    const bool vec = (hidden % 8) == 0;
    float partial = 0.0f;
    if (vec) {
        for (uint32_t c = lane * 8; c < hidden; c += 8 * kWave) {
            h8 a = *reinterpret_cast<const h8*>(x + base + c);
            if (ADD) {
                h8 b = *reinterpret_cast<const h8*>(residual + base + c);
#pragma unroll
                for (int j = 0; j < 8; ++j) a.v[j] = f2h(h2f(a.v[j]) + h2f(b.v[j]));
                *reinterpret_cast<h8*>(residual_out + base + c) = a;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float f = h2f(a.v[j]);
                if (sequential)
                    sq[c + j] = f * f;
                else
                    partial = partial + f * f;
            }
        }
    } else {
        for (uint32_t c = lane; c < hidden; c += kWave) {
            uint16_t a = x[base + c];
            if (ADD) {
                a = f2h(h2f(a) + h2f(residual[base + c]));
                residual_out[base + c] = a;
            }
            float f = h2f(a);
            if (sequential)
                sq[c] = f * f;
            else
                partial = partial + f * f;
        }
    }
    float inv;
    if (sequential) {
        __syncthreads();
        if (lane == 0) {
            float s = 0.0f;
            for (uint32_t c = 0; c < hidden; ++c) s = s + sq[c];
            inv_shared = inverse_rms(s, static_cast<float>(hidden), epsilon);
        }
        __syncthreads();
        inv = inv_shared;
    } else {
        inv = inverse_rms(wave_sum(partial), static_cast<float>(hidden), epsilon);
    }
    const uint16_t* src = ADD ? residual_out : x;
    if (vec) {
        for (uint32_t c = lane * 8; c < hidden; c += 8 * kWave) {
            h8 a = *reinterpret_cast<const h8*>(src + base + c);
            h8 w = *reinterpret_cast<const h8*>(weight + c);
            h8 y;
#pragma unroll
            for (int j = 0; j < 8; ++j) y.v[j] = f2h(h2f(a.v[j]) * inv * h2f(w.v[j]));
            *reinterpret_cast<h8*>(out + base + c) = y;
        }
    } else {
        for (uint32_t c = lane; c < hidden; c += kWave)
            out[base + c] = f2h(h2f(src[base + c]) * inv * h2f(weight[c]));
    }
}

// ---------------------------------------------------------------------------
// FP16-storage register engine (sequential order, 16-byte aligned rows with
// hidden % 8 == 0 and hidden <= 4096).  Same structure as rms_reg_kernel:
// lane l keeps 8 halves (one 128-bit load) of column l + 64*j of each row;
// math is f32 on exactly widened values; outputs are rounded RNE once.  With
// ADD the stored residual stream rne16(x + residual) is what is squared and
// normalised, matching the two-kernel chain with f16 buffers.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lo16(uint32_t w) { return h2f(static_cast<uint16_t>(w)); }
__device__ __forceinline__ float hi16(uint32_t w) { return h2f(static_cast<uint16_t>(w >> 16)); }
__device__ __forceinline__ uint32_t pack16(float lo, float hi) {
    return static_cast<uint32_t>(f2h(lo)) | (static_cast<uint32_t>(f2h(hi)) << 16);
}

// FP16 tree engine (ATLAS_REDUCTION_AUTO and _WIDE): rms_tree_kernel's
// structure over binary16 rows, one 16-byte access carrying 8 halves.  The
// math is f32: exact widening, the tree sum of squares, one RNE rounding per
// output; with a residual, residual_out = rne16(x + r) is stored and the
// norm reads that rounded value (as the reference's two-kernel chain over
// f16 buffers does).  y is within one f16 ulp of the sequential fold's.
template <int J, bool ADD>
struct TreeRowF16 {
    u32x4 x[J];
    u32x4 e[ADD ? J : 1];

    __device__ __forceinline__ void load(const uint16_t* xs, const uint16_t* residual, uint32_t row, uint32_t hidden,
                                         uint32_t lane, uint32_t n8) {
        const size_t base = static_cast<size_t>(row) * hidden;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t c = min(lane + 64u * j, n8 - 1);
            x[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xs + base + 8 * c));
            if (ADD) e[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(residual + base + 8 * c));
        }
    }

    __device__ __forceinline__ void finish(const u32x4 (&w)[J], uint16_t* residual_out, uint16_t* out, uint32_t row,
                                           uint32_t hidden, uint32_t lane, uint32_t n8, float epsilon) {
        const size_t base = static_cast<size_t>(row) * hidden;
        if (ADD) {
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const u32x4 v = x[j], b = e[j];
                x[j] = u32x4{pack16(lo16(v.x) + lo16(b.x), hi16(v.x) + hi16(b.x)),
                             pack16(lo16(v.y) + lo16(b.y), hi16(v.y) + hi16(b.y)),
                             pack16(lo16(v.z) + lo16(b.z), hi16(v.z) + hi16(b.z)),
                             pack16(lo16(v.w) + lo16(b.w), hi16(v.w) + hi16(b.w))};
            }
        }
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const u32x4 v = x[j];
            const float a0 = lo16(v.x), a1 = hi16(v.x), a2 = lo16(v.y), a3 = hi16(v.y);
            const float a4 = lo16(v.z), a5 = hi16(v.z), a6 = lo16(v.w), a7 = hi16(v.w);
            const float q = ((a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3)) + ((a4 * a4 + a5 * a5) + (a6 * a6 + a7 * a7));
            p = p + (lane + 64u * j < n8 ? q : 0.0f);
        }
        const float ir = inverse_rms(wave_sum_tree_f32(p), static_cast<float>(hidden), epsilon);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t c = lane + 64u * j;
            if (c >= n8) continue;
            const u32x4 v = x[j], ww = w[j];
            if (ADD) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(residual_out + base + 8 * c));
            const u32x4 y{pack16(lo16(v.x) * ir * lo16(ww.x), hi16(v.x) * ir * hi16(ww.x)),
                          pack16(lo16(v.y) * ir * lo16(ww.y), hi16(v.y) * ir * hi16(ww.y)),
                          pack16(lo16(v.z) * ir * lo16(ww.z), hi16(v.z) * ir * hi16(ww.z)),
                          pack16(lo16(v.w) * ir * lo16(ww.w), hi16(v.w) * ir * hi16(ww.w))};
            __builtin_nontemporal_store(y, reinterpret_cast<u32x4*>(out + base + 8 * c));
        }
    }
};

// Parameters in kernarg-preload order (the counts and the pointers the
// first loads need in the first 56 bytes, as ATLAS_NORM_KPARAMS); wpb and
// pair_stride as there.
template <int J, bool ADD, bool PAIR>
__global__ __launch_bounds__(256) void rms_tree_f16_kernel(uint32_t rows, uint32_t hidden, uint32_t wpb,
                                                           uint32_t pair_stride, const uint16_t* x,
                                                           const uint16_t* residual, const uint16_t* weight,
                                                           float epsilon, uint16_t* residual_out, uint16_t* out) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    const uint32_t r0 = blockIdx.x * wpb + wave;
    if (r0 >= rows) return;  // wavefront-uniform
    const uint32_t r1 = r0 + pair_stride;
    const bool second = PAIR && r1 < rows;
    const uint32_t n8 = hidden >> 3;
    TreeRowF16<J, ADD> row0, row1;
    row0.load(x, residual, r0, hidden, lane, n8);
    if (second) row1.load(x, residual, r1, hidden, lane, n8);
    u32x4 w[J];
#pragma unroll
    for (int j = 0; j < J; ++j) w[j] = *reinterpret_cast<const u32x4*>(weight + 8 * min(lane + 64u * j, n8 - 1));
    row0.finish(w, residual_out, out, r0, hidden, lane, n8, epsilon);
    if (second) row1.finish(w, residual_out, out, r1, hidden, lane, n8, epsilon);
}

template <int R, int J, bool ADD, bool STAGE>
__global__ __launch_bounds__(64) void rms_reg_f16_kernel(const uint16_t* x, const uint16_t* residual,
                                                         const uint16_t* weight, uint16_t* residual_out,
                                                         uint16_t* out, uint32_t rows, uint32_t hidden,
                                                         float epsilon) {
    extern __shared__ f32x4 sq4[];  // R rows x (hidden/4 + 1) float4 of squares
    const uint32_t lane = threadIdx.x;
    const uint32_t n8 = hidden >> 3;          // 8-half groups per row
    const uint32_t stride4 = (hidden >> 2) + 1;
    const uint32_t row0 = blockIdx.x * R;
    const uint32_t nrows = min(static_cast<uint32_t>(R), rows - row0);

    u32x4 xv[R][J];
    u32x4 ev[ADD ? R : 1][ADD ? J : 1];
    u32x4 wv[J];
    auto load_chunk = [&](int j, uint32_t zero) {
        const uint32_t c = min(lane + 64u * j, n8 - 1) + zero;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t idx = static_cast<size_t>(row0 + min(static_cast<uint32_t>(r), nrows - 1)) * hidden + 8 * c;
            xv[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + idx));
            if (ADD) ev[r][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(residual + idx));
        }
    };
    // STAGE: chunk 0 first, the later chunks once it has landed (as in
    // rms_reg_kernel), so the in-order fold starts with the first data
#pragma unroll
    for (int j = 0; j < (STAGE ? 1 : J); ++j) load_chunk(j, 0u);
#pragma unroll
    for (int j = 0; j < J; ++j)
        wv[j] = *reinterpret_cast<const u32x4*>(weight + 8 * min(lane + 64u * j, n8 - 1));
    if constexpr (STAGE) {
        uint32_t zero;
        __asm__ volatile("v_mov_b32 %0, 0" : "=v"(zero) : "v"(xv[0][0].x));
#pragma unroll
        for (int j = 1; j < J; ++j) load_chunk(j, zero);
    }

    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t creal = lane + 64u * j;
        const uint32_t c = min(creal, n8 - 1);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            u32x4 v = xv[r][j];
            if (ADD) {
                const u32x4 b = ev[r][j];
                v = u32x4{pack16(lo16(v.x) + lo16(b.x), hi16(v.x) + hi16(b.x)),
                          pack16(lo16(v.y) + lo16(b.y), hi16(v.y) + hi16(b.y)),
                          pack16(lo16(v.z) + lo16(b.z), hi16(v.z) + hi16(b.z)),
                          pack16(lo16(v.w) + lo16(b.w), hi16(v.w) + hi16(b.w))};
                xv[r][j] = v;
            }
            const float a0 = lo16(v.x), a1 = hi16(v.x), a2 = lo16(v.y), a3 = hi16(v.y);
            const float a4 = lo16(v.z), a5 = hi16(v.z), a6 = lo16(v.w), a7 = hi16(v.w);
            sq4[r * stride4 + 2 * c] = f32x4{a0 * a0, a1 * a1, a2 * a2, a3 * a3};
            sq4[r * stride4 + 2 * c + 1] = f32x4{a4 * a4, a5 * a5, a6 * a6, a7 * a7};
        }
        __syncthreads();
        if (lane < nrows) {
            const uint32_t begin = 128u * j, end = min(2 * n8, 128u * (j + 1));
            const f32x4* row = sq4 + lane * stride4;
            for (uint32_t k = begin; k < end; k += 64) s = fold_lds_chunk(row + k, min(64u, end - k), s);
        }
    }
    if (ADD) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (static_cast<uint32_t>(r) >= nrows) break;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const uint32_t c = lane + 64u * j;
                if (c < n8)
                    __builtin_nontemporal_store(
                        xv[r][j], reinterpret_cast<u32x4*>(residual_out + static_cast<size_t>(row0 + r) * hidden + 8 * c));
            }
        }
    }
    const float inv = lane < nrows ? inverse_rms(s, static_cast<float>(hidden), epsilon) : 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (static_cast<uint32_t>(r) >= nrows) break;
        const float ir = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), r));
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint32_t c = lane + 64u * j;
            if (c >= n8) continue;
            const u32x4 v = xv[r][j], w = wv[j];
            const u32x4 y{pack16(lo16(v.x) * ir * lo16(w.x), hi16(v.x) * ir * hi16(w.x)),
                          pack16(lo16(v.y) * ir * lo16(w.y), hi16(v.y) * ir * hi16(w.y)),
                          pack16(lo16(v.z) * ir * lo16(w.z), hi16(v.z) * ir * hi16(w.z)),
                          pack16(lo16(v.w) * ir * lo16(w.w), hi16(v.w) * ir * hi16(w.w))};
            __builtin_nontemporal_store(y, reinterpret_cast<u32x4*>(out + static_cast<size_t>(row0 + r) * hidden + 8 * c));
        }
    }
}

template <int J, bool ADD>
hipError_t launch_f16_reg_j(hipStream_t s, const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                            uint16_t* residual_out, uint16_t* out, uint32_t rows, uint32_t hidden, float eps) {
    // one row per wavefront (C2 [2048, 2048]: 13.2 us, against 13.6 with two
    // rows per wavefront), staged loads from 2048 rows up; the exact
    // wave-parallel fold measured slower here (13.8 -> 16.7 us), so every
    // chunk folds in order
    const size_t lds = (hidden / 4 + 1) * sizeof(f32x4);
    const dim3 grid(rows);
    if (rows >= 2048)
        hipLaunchKernelGGL((rms_reg_f16_kernel<1, J, ADD, true>), grid, dim3(kWave), lds, s, x, residual, weight,
                           residual_out, out, rows, hidden, eps);
    else
        hipLaunchKernelGGL((rms_reg_f16_kernel<1, J, ADD, false>), grid, dim3(kWave), lds, s, x, residual, weight,
                           residual_out, out, rows, hidden, eps);
    return hipGetLastError();
}

template <int J, bool ADD>
hipError_t launch_f16_tree_j(hipStream_t s, const uint16_t* x, const uint16_t* residual, const uint16_t* weight,
                             uint16_t* residual_out, uint16_t* out, uint32_t rows, uint32_t hidden, float eps) {
    const bool pair = tree_pairs(rows);
    const uint32_t waves = pair ? (rows + 1) / 2 : rows;
    const uint32_t wpb = tree_waves_per_group(rows);
    const dim3 grid((waves + wpb - 1) / wpb);
    const uint32_t pair_stride = grid.x * wpb;
    if (pair)
        hipLaunchKernelGGL((rms_tree_f16_kernel<J, ADD, true>), grid, dim3(64 * wpb), 0, s, rows, hidden, wpb,
                           pair_stride, x, residual, weight, eps, residual_out, out);
    else
        hipLaunchKernelGGL((rms_tree_f16_kernel<J, ADD, false>), grid, dim3(64 * wpb), 0, s, rows, hidden, wpb,
                           pair_stride, x, residual, weight, eps, residual_out, out);
    return hipGetLastError();
}

// hidden % 8 == 0, hidden <= 4096 (J <= 8 chunks of 512 halves)
template <bool ADD>
hipError_t launch_f16_vec(hipStream_t s, bool tree, const uint16_t* x, const uint16_t* residual,
                          const uint16_t* weight, uint16_t* residual_out, uint16_t* out, uint32_t rows,
                          uint32_t hidden, float eps) {
#define ATLAS_F16_J(JJ)                                                                                        \
    case JJ:                                                                                                    \
        return tree ? launch_f16_tree_j<JJ, ADD>(s, x, residual, weight, residual_out, out, rows, hidden, eps) \
                    : launch_f16_reg_j<JJ, ADD>(s, x, residual, weight, residual_out, out, rows, hidden, eps);
    switch ((hidden / 8 + 63) / 64) {
        ATLAS_F16_J(1)
        ATLAS_F16_J(2)
        ATLAS_F16_J(3)
        ATLAS_F16_J(4)
        ATLAS_F16_J(5)
        ATLAS_F16_J(6)
        ATLAS_F16_J(7)
        default:
            return tree ? launch_f16_tree_j<8, ADD>(s, x, residual, weight, residual_out, out, rows, hidden, eps)
                        : launch_f16_reg_j<8, ADD>(s, x, residual, weight, residual_out, out, rows, hidden, eps);
    }
#undef ATLAS_F16_J
}

}  // namespace

// Engine choice.  kSequential: the sequential fold everywhere (register
// engine, or the LDS engine for hidden > 2048 or unaligned rows).  kAuto
// (the default): the tree engine where the output is a plain scaled row
// (RMSNorm, the add-norm's y), the sequential fold where an epilogue
// cancels (residual add, PLE add-scale), whose elementwise error would
// otherwise be unbounded relative to the output.  kWide: the tree engine
// everywhere.
hipError_t launch_rms_norm_f32(hipStream_t stream, NormMode mode, Reduction red, const NormArgs& a) {
    const bool vec = (a.hidden % 4) == 0 && aligned16(a.x) && aligned16(a.weight) && aligned16(a.out) &&
                     (!a.residual || aligned16(a.residual)) && (!a.normalized || aligned16(a.normalized)) &&
                     (!a.residual_out || aligned16(a.residual_out));
    const bool cancels = mode == kNormResidual || mode == kNormAddScale;
    const bool tree = red == kWide || (red == kAuto && !cancels);
    if (tree && vec && a.hidden <= 2048) {
        switch (mode) {
            case kNormPlain: return launch_tree<kNormPlain>(stream, a);
            case kNormResidual: return launch_tree<kNormResidual>(stream, a);
            case kNormAddNorm: return launch_tree<kNormAddNorm>(stream, a);
            case kNormAddScale: return launch_tree<kNormAddScale>(stream, a);
        }
    } else if (tree) {
        switch (mode) {
            case kNormPlain: return launch_wide<kNormPlain>(stream, a, vec);
            case kNormResidual: return launch_wide<kNormResidual>(stream, a, vec);
            case kNormAddNorm: return launch_wide<kNormAddNorm>(stream, a, vec);
            case kNormAddScale: return launch_wide<kNormAddScale>(stream, a, vec);
        }
    } else if (vec && a.hidden <= 2048) {
        switch (mode) {
            case kNormPlain: return launch_reg<kNormPlain>(stream, a);
            case kNormResidual: return launch_reg<kNormResidual>(stream, a);
            case kNormAddNorm: return launch_reg<kNormAddNorm>(stream, a);
            case kNormAddScale: return launch_reg<kNormAddScale>(stream, a);
        }
    } else {
        switch (mode) {
            case kNormPlain: return launch_seq<kNormPlain>(stream, a, vec);
            case kNormResidual: return launch_seq<kNormResidual>(stream, a, vec);
            case kNormAddNorm: return launch_seq<kNormAddNorm>(stream, a, vec);
            case kNormAddScale: return launch_seq<kNormAddScale>(stream, a, vec);
        }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_rms_norm_groups_stable_f32(hipStream_t stream, Reduction red, float* values,
                                             const float* weight, uint32_t width, uint32_t groups,
                                             float epsilon) {
    // kAuto keeps the sequential fold: one wavefront per 256-wide group folds
    // its squares in order from LDS at no measurable cost
    const bool seq = red != kWide;
    if (width <= 64 * 16) {
        const int q = seq ? 1 : 0;
        if (width <= 64 * 4)
            hipLaunchKernelGGL((groups_stable_reg_kernel<4>), dim3(groups), dim3(kWave), 0, stream, values, weight,
                               width, epsilon, q);
        else if (width <= 64 * 8)
            hipLaunchKernelGGL((groups_stable_reg_kernel<8>), dim3(groups), dim3(kWave), 0, stream, values, weight,
                               width, epsilon, q);
        else
            hipLaunchKernelGGL((groups_stable_reg_kernel<16>), dim3(groups), dim3(kWave), 0, stream, values, weight,
                               width, epsilon, q);
        return hipGetLastError();
    }
    const size_t lds = seq ? static_cast<size_t>(width) * sizeof(float) : 0;
    hipLaunchKernelGGL(groups_stable_kernel, dim3(groups), dim3(kWave), lds, stream, values, weight,
                       width, groups, epsilon, seq ? 1 : 0);
    return hipGetLastError();
}

// FP16 rows: the outputs are plain scaled rows (residual_out does not
// depend on the reduction), so kAuto and kWide take the tree engine.
hipError_t launch_rms_norm_f16(hipStream_t stream, Reduction red, const uint16_t* x,
                               const uint16_t* residual, const uint16_t* weight,
                               uint16_t* residual_out, uint16_t* out, uint32_t rows,
                               uint32_t hidden, float epsilon) {
    const bool tree = red != kSequential;
    const bool vec = hidden % 8 == 0 && hidden <= 4096 && aligned16(x) && aligned16(weight) && aligned16(out) &&
                     (!residual || (aligned16(residual) && aligned16(residual_out)));
    if (vec) {
        if (residual)
            return launch_f16_vec<true>(stream, tree, x, residual, weight, residual_out, out, rows, hidden, epsilon);
        return launch_f16_vec<false>(stream, tree, x, residual, weight, residual_out, out, rows, hidden, epsilon);
    }
    const int seq = tree ? 0 : 1;
    const size_t lds = seq ? static_cast<size_t>(hidden) * sizeof(float) : 0;
    if (residual)
        hipLaunchKernelGGL((rms_f16_seq_kernel<true>), dim3(rows), dim3(kWave), lds, stream, x,
                           residual, weight, residual_out, out, rows, hidden, epsilon, seq);
    else
        hipLaunchKernelGGL((rms_f16_seq_kernel<false>), dim3(rows), dim3(kWave), lds, stream, x,
                           residual, weight, residual_out, out, rows, hidden, epsilon, seq);
    return hipGetLastError();
}

}  // namespace atlas
