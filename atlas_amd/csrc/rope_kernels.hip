// rope_kernels.hip -- per-head QK-RMSNorm fused with half-split RoPE, plain
// half-split RoPE (f32 / f16 storage) and the interleaved operator-API RoPE.
//
// Reference semantics (bisegni/atlas):
//   gemma4_qk_norm_rope_fused_batch_f32   crates/atlas-metal/src/kernels.metal:1098-1142
//   (exact oracle kernel; the _wide variants at :1053-1090, :1151-1195 reorder
//   the sum of squares)
//   Llama half-split RoPE = rope_half_to_interleaved_f32 + rope_f32 +
//   rope_interleaved_to_half_f32   kernels.metal:940-949, 972-994
//   NeuralOps::rope (interleaved) = rope_f32; CPU oracle cpu_rope
//   crates/atlas-ops/tests/phase_02_operators.rs:262-272
//
// QK-norm+RoPE mapping on CDNA: a "unit" is one (token, head) row of
// head_dim floats; Q heads come first, then the optional single K head.  One
// wavefront owns UNITS consecutive units.  With head_dim = 64*V every lane
// holds V consecutive floats of each unit in registers (one 128-bit load for
// V = 4), and the RoPE partner x[p + d/2] of the value x[p] held by lane l
// sits in lane l^32, so the pair is exchanged with one cross-lane swap and
// never round-trips through memory.  The squares go to LDS for the
// sequential fold (lane u folds unit u in index order), which makes the
// result bit-identical to the CPU composition rms_norm -> rope.
#include "device_common.hpp"
#include "launch.hpp"


namespace atlas {
namespace {

template <int V>
struct vecf {
    float v[V];
};

template <int V>
__device__ __forceinline__ vecf<V> ldv(const float* p) {
    vecf<V> r;
    if constexpr (V == 2) {
        float2 a = *reinterpret_cast<const float2*>(p);
        r.v[0] = a.x;
        r.v[1] = a.y;
    } else if constexpr (V == 4) {
        float4 a = *reinterpret_cast<const float4*>(p);
        r.v[0] = a.x;
        r.v[1] = a.y;
        r.v[2] = a.z;
        r.v[3] = a.w;
    } else {
#pragma unroll
        for (int j = 0; j < V; j += 4) {
            float4 a = *reinterpret_cast<const float4*>(p + j);
            r.v[j] = a.x;
            r.v[j + 1] = a.y;
            r.v[j + 2] = a.z;
            r.v[j + 3] = a.w;
        }
    }
    return r;
}

template <int V>
__device__ __forceinline__ void stv(float* p, const vecf<V>& r) {
    if constexpr (V == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(r.v[0], r.v[1]);
    } else {
#pragma unroll
        for (int j = 0; j < V; j += 4)
            *reinterpret_cast<float4*>(p + j) = make_float4(r.v[j], r.v[j + 1], r.v[j + 2], r.v[j + 3]);
    }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <int V, int UNITS, bool SEQ>
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(
    const float* q, const float* k, const float* q_weight, const float* k_weight,
    const float* cosine, const float* sine, float* q_out, float* k_out, uint32_t tokens,
    uint32_t q_heads, uint32_t has_key, uint32_t rope_stride, float epsilon) {
    constexpr uint32_t D = 64 * V;
    constexpr uint32_t HALF = D / 2;
    constexpr uint32_t STRIDE = D + 4;
    __shared__ float sq[SEQ ? UNITS * STRIDE : 1];
    __shared__ float inv_lds[UNITS];

    const uint32_t lane = threadIdx.x;
    const uint32_t total = q_heads + has_key;
    const uint32_t units = tokens * total;
    const uint32_t u0 = blockIdx.x * UNITS;
    const bool low = lane < 32;
    const uint32_t col = lane * V;                        // this lane's first column
    const uint32_t pair = low ? col : col - HALF;         // first RoPE pair index
    const uint32_t partner_col = low ? col + HALF : col - HALF;

    vecf<V> x[UNITS];
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
        const uint32_t unit = u0 + u;
        if (unit < units) {
            const uint32_t t = unit / total, local = unit % total;
            const float* src = local >= q_heads ? k + static_cast<size_t>(t) * D
                                                : q + (static_cast<size_t>(t) * q_heads + local) * D;
            x[u] = ldv<V>(src + col);
        } else {
#pragma unroll
            for (int j = 0; j < V; ++j) x[u].v[j] = 0.0f;
        }
    }

    if constexpr (SEQ) {
#pragma unroll
        for (int u = 0; u < UNITS; ++u) {
            vecf<V> s2;
#pragma unroll
            for (int j = 0; j < V; ++j) s2.v[j] = x[u].v[j] * x[u].v[j];
            stv<V>(sq + u * STRIDE + col, s2);
        }
        __syncthreads();
        if (lane < UNITS) {
            const float* row = sq + lane * STRIDE;
            float s = 0.0f;
#pragma unroll 8
            for (uint32_t c = 0; c < D; c += 4) {
                float4 v = *reinterpret_cast<const float4*>(row + c);
                s = s + v.x;
                s = s + v.y;
                s = s + v.z;
                s = s + v.w;
            }
            inv_lds[lane] = inverse_rms(s, static_cast<float>(D), epsilon);
        }
        __syncthreads();
    } else {
#pragma unroll
        for (int u = 0; u < UNITS; ++u) {
            float partial = 0.0f;
#pragma unroll
            for (int j = 0; j < V; ++j) partial = partial + x[u].v[j] * x[u].v[j];
            float s = wave_sum(partial);
            if (lane == 0) inv_lds[u] = inverse_rms(s, static_cast<float>(D), epsilon);
        }
        __syncthreads();
    }

    const vecf<V> qw_own = ldv<V>(q_weight + col), qw_par = ldv<V>(q_weight + partner_col);
    vecf<V> kw_own = qw_own, kw_par = qw_par;
    if (has_key) {
        kw_own = ldv<V>(k_weight + col);
        kw_par = ldv<V>(k_weight + partner_col);
    }

#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
        const uint32_t unit = u0 + u;
        // exchange halves: lane l <-> lane l^32 (executed by the whole wave)
        vecf<V> other;
#pragma unroll
        for (int j = 0; j < V; ++j) other.v[j] = __shfl_xor(x[u].v[j], 32, kWave);
        if (unit >= units) continue;
        const uint32_t t = unit / total, local = unit % total;
        const bool key = local >= q_heads;
        const float inv = inv_lds[u];
        const vecf<V>& w_own = key ? kw_own : qw_own;
        const vecf<V>& w_par = key ? kw_par : qw_par;
        const vecf<V> c = ldv<V>(cosine + static_cast<size_t>(t) * rope_stride + pair);
        const vecf<V> s = ldv<V>(sine + static_cast<size_t>(t) * rope_stride + pair);
        vecf<V> y;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const float own = x[u].v[j] * inv * w_own.v[j];
            const float par = other.v[j] * inv * w_par.v[j];
            // low lanes hold x0 (own) and receive x1; high lanes the reverse
            const float x0 = low ? own : par;
            const float x1 = low ? par : own;
            y.v[j] = low ? x0 * c.v[j] - x1 * s.v[j] : x0 * s.v[j] + x1 * c.v[j];
        }
        float* dst = key ? k_out + static_cast<size_t>(t) * D
                         : q_out + (static_cast<size_t>(t) * q_heads + local) * D;
        stv<V>(dst + col, y);
    }
}

// Token engine (sequential order, the default for head_dim = 128*P): one
// wavefront per token covers its q_heads Q rows and the optional K row
// (U = q_heads + has_key <= MAXU units).  Lane l owns RoPE pairs
// [l*P, l*P + P) of every unit and keeps both halves x[p] and x[p + d/2] in
// registers, so the rotation needs no cross-lane exchange; the token's
// cos/sin row and the four weight slices are loaded once per wavefront.
// Loads are straight-line (units past U are clamped to a valid duplicate
// address, never stored) and nontemporal; squares go to LDS and lane u folds
// unit u in index order (bit-identical to the CPU composition
// rms_norm -> rope).  Every unit is fully read before it is written, so
// q_out == q and k_out == k are allowed.
template <int P>
struct pvec {
    float v[P];
};

template <int P, bool NT>
__device__ __forceinline__ pvec<P> ld_p(const float* p) {
    constexpr bool nt = NT;
    pvec<P> r;
    if constexpr (P == 1) {
        r.v[0] = nt ? __builtin_nontemporal_load(p) : *p;
    } else if constexpr (P == 2) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        const f2 a = nt ? __builtin_nontemporal_load(reinterpret_cast<const f2*>(p)) : *reinterpret_cast<const f2*>(p);
        r.v[0] = a.x;
        r.v[1] = a.y;
    } else {
        typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int j = 0; j < P; j += 4) {
            const f4 a = nt ? __builtin_nontemporal_load(reinterpret_cast<const f4*>(p + j))
                            : *reinterpret_cast<const f4*>(p + j);
            r.v[j] = a.x;
            r.v[j + 1] = a.y;
            r.v[j + 2] = a.z;
            r.v[j + 3] = a.w;
        }
    }
    return r;
}

template <int P>
__device__ __forceinline__ void st_p(float* p, const pvec<P>& r) {
    if constexpr (P == 1) {
        __builtin_nontemporal_store(r.v[0], p);
    } else if constexpr (P == 2) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        __builtin_nontemporal_store(f2{r.v[0], r.v[1]}, reinterpret_cast<f2*>(p));
    } else {
        typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int j = 0; j < P; j += 4)
            __builtin_nontemporal_store(f4{r.v[j], r.v[j + 1], r.v[j + 2], r.v[j + 3]},
                                        reinterpret_cast<f4*>(p + j));
    }
}

template <int P>
__device__ __forceinline__ void sq_p(float* dst, const pvec<P>& x) {
#pragma unroll
    for (int j = 0; j < P; ++j) dst[j] = x.v[j] * x.v[j];
}

// TPW tokens per wavefront (tokens w and w + G, G = the grid's wavefront
// count) and WPG wavefronts per workgroup; each wavefront uses its own LDS
// region, so the handoff between the lanes that square and the lanes that
// fold is a wavefront-scope fence, not a workgroup barrier.  SPLIT: a
// token's units are spread over ceil(units / MAXU) consecutive wavefronts,
// MAXU each (TPW = 1).  SEQ = false (ATLAS_REDUCTION_WIDE): each unit's sum
// of squares is a wavefront tree sum of the lanes' partial sums instead of
// the in-order fold (no LDS), tolerance-level against the CPU operator.
// Parameter order: what the first loads' addresses need (the counts, the
// rows, cos/sin) and epsilon fill the first 56 bytes, which arrive in SGPRs
// at wave launch (kernarg preload); the weights and outputs, needed only
// after the fold, follow.
template <int P, int MAXU, int TPW, int WPG, bool SPLIT = false, bool SEQ = true>
__global__ __launch_bounds__(64 * WPG) void qk_norm_rope_token_kernel(
    uint32_t tokens, uint32_t q_heads, uint32_t has_key, uint32_t rope_stride, const float* q, const float* k,
    const float* cosine, const float* sine, float epsilon, const float* q_weight, const float* k_weight,
    float* q_out, float* k_out) {
    constexpr uint32_t HALF = 64 * P;
    constexpr uint32_t D = 2 * HALF;
    constexpr uint32_t STRIDE = D + 4;
    // head_dim 256 with one unit per wavefront: the unit's sum by candidate
    // segments (head_fold_candidates), from a padded copy of its squares
    // (float f at f + 4 (f / 64), 68 float4)
    constexpr bool kCand = SEQ && D == 256 && TPW == 1 && MAXU == 1;
    constexpr uint32_t kLds = kCand ? 272 : (SEQ ? TPW * MAXU * STRIDE : 4);
    __shared__ __align__(16) float sq_all[WPG][kLds];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    float* sq = sq_all[wave];
    static_assert(!SPLIT || TPW == 1, "a split token is one wavefront's only token");
    const uint32_t total = q_heads + has_key;
    const uint32_t wv = blockIdx.x * WPG + wave;
    const uint32_t parts = SPLIT ? (total + MAXU - 1) / MAXU : 1u;
    const uint32_t w0 = SPLIT ? wv / parts : wv;
    const uint32_t ubase = SPLIT ? (wv - w0 * parts) * MAXU : 0u;  // the wavefront's first unit
    const uint32_t G = gridDim.x * WPG;
    if (w0 >= tokens) return;  // wavefront-uniform
    const uint32_t p0 = lane * P;
    uint32_t tok[TPW];
    uint32_t ntok = 0;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        tok[i] = w0 + i * G;
        ntok += tok[i] < tokens ? 1u : 0u;
    }

    pvec<P> lo[TPW][MAXU], hi[TPW][MAXU];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const uint32_t t = min(tok[i], tokens - 1);
#pragma unroll
        for (int u = 0; u < MAXU; ++u) {
            const uint32_t uu = min(ubase + u, total - 1);
            const float* src = uu >= q_heads ? k + static_cast<size_t>(t) * D
                                             : q + (static_cast<size_t>(t) * q_heads + uu) * D;
            lo[i][u] = ld_p<P, true>(src + p0);
            hi[i][u] = ld_p<P, true>(src + HALF + p0);
        }
    }
    pvec<P> cs[TPW], sn[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const size_t tb = static_cast<size_t>(min(tok[i], tokens - 1)) * rope_stride + p0;
        cs[i] = ld_p<P, false>(cosine + tb);
        sn[i] = ld_p<P, false>(sine + tb);
    }
    const pvec<P> qwl = ld_p<P, false>(q_weight + p0), qwh = ld_p<P, false>(q_weight + HALF + p0);
    const float* kw = has_key ? k_weight : q_weight;
    const pvec<P> kwl = ld_p<P, false>(kw + p0), kwh = ld_p<P, false>(kw + HALF + p0);

    // lane i * MAXU + u holds the sum of squares of unit u of the
    // wavefront's token i
    float sum = 0.0f;
    const uint32_t li = lane / MAXU, lu = lane - li * MAXU;
    const bool folds = li < ntok && ubase + lu < total;
    if constexpr (kCand) {
        // lane l's values p0, p0 + 1 (P = 2) and HALF + p0, ...: each pair
        // inside one 64-float segment
        sq_p<P>(sq + p0 + 4 * (p0 / 64), lo[0][0]);
        sq_p<P>(sq + HALF + p0 + 4 * ((HALF + p0) / 64), hi[0][0]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float t = head_fold_candidates(reinterpret_cast<const f32x4*>(sq), lane);
        sum = lane == 0 ? t : sum;
    } else if constexpr (SEQ) {
#pragma unroll
        for (int i = 0; i < TPW; ++i)
#pragma unroll
            for (int u = 0; u < MAXU; ++u) {
                sq_p<P>(sq + (i * MAXU + u) * STRIDE + p0, lo[i][u]);
                sq_p<P>(sq + (i * MAXU + u) * STRIDE + HALF + p0, hi[i][u]);
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // in index order
        if (folds) {
            const f32x4* row = reinterpret_cast<const f32x4*>(sq + lane * STRIDE);
#pragma unroll
            for (uint32_t c = 0; c < D / 4; c += 64)
                sum = fold_lds_chunk(row + c, D / 4 - c < 64 ? D / 4 - c : 64, sum);
        }
    } else {
        (void)sq;
#pragma unroll
        for (int i = 0; i < TPW; ++i)
#pragma unroll
            for (int u = 0; u < MAXU; ++u) {
                float part = 0.0f;
#pragma unroll
                for (int j = 0; j < P; ++j) part = part + lo[i][u].v[j] * lo[i][u].v[j];
#pragma unroll
                for (int j = 0; j < P; ++j) part = part + hi[i][u].v[j] * hi[i][u].v[j];
                const float t = wave_sum_tree_f32(part);
                sum = lane == static_cast<uint32_t>(i * MAXU + u) ? t : sum;
            }
    }
    const float inv = folds ? inverse_rms(sum, static_cast<float>(D), epsilon) : 0.0f;

#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        if (static_cast<uint32_t>(i) >= ntok) break;
        const uint32_t t = tok[i];
        const pvec<P>& c = cs[i];
        const pvec<P>& s = sn[i];
#pragma unroll
        for (int u = 0; u < MAXU; ++u) {
            if (ubase + u < total) {
                const float iu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), i * MAXU + u));
                const bool key = ubase + u >= q_heads;
                pvec<P> ol, oh;
#pragma unroll
                for (int j = 0; j < P; ++j) {
                    const float wl = key ? kwl.v[j] : qwl.v[j];
                    const float wh = key ? kwh.v[j] : qwh.v[j];
                    const float x0 = lo[i][u].v[j] * iu * wl;
                    const float x1 = hi[i][u].v[j] * iu * wh;
                    ol.v[j] = x0 * c.v[j] - x1 * s.v[j];
                    oh.v[j] = x0 * s.v[j] + x1 * c.v[j];
                }
                float* dst = key ? k_out + static_cast<size_t>(t) * D
                                 : q_out + (static_cast<size_t>(t) * q_heads + ubase + u) * D;
                st_p<P>(dst + p0, ol);
                st_p<P>(dst + HALF + p0, oh);
            }
        }
    }
}

template <int P, int TPW, int WPG, bool SEQ>
hipError_t launch_qk_token_cfg(hipStream_t s, const float* q, const float* k, const float* qw, const float* kw,
                               const float* c, const float* sn, float* qo, float* ko, uint32_t tokens,
                               uint32_t q_heads, uint32_t has_key, uint32_t rope_stride, float eps) {
    const uint32_t total = q_heads + has_key;
    const uint32_t waves = (tokens + TPW - 1) / TPW;
    const dim3 grid((waves + WPG - 1) / WPG);
#define ATLAS_QK_CASE(U)                                                                                          \
    if (total <= U) {                                                                                             \
        hipLaunchKernelGGL((qk_norm_rope_token_kernel<P, U, TPW, WPG, false, SEQ>), grid, dim3(64 * WPG), 0, s,      \
                           tokens, q_heads, has_key, rope_stride, q, k, c, sn, eps, qw, kw, qo, ko);            \
        return hipGetLastError();                                                                                 \
    }
    ATLAS_QK_CASE(1)
    ATLAS_QK_CASE(2)
    ATLAS_QK_CASE(4)
    ATLAS_QK_CASE(8)
    ATLAS_QK_CASE(9)
    ATLAS_QK_CASE(12)
    ATLAS_QK_CASE(16)
#undef ATLAS_QK_CASE
    return hipErrorInvalidValue;
}

// A token's units over ceil(units / U) wavefronts, one wavefront per workgroup.
template <int P, int U, bool SEQ>
hipError_t launch_qk_split(hipStream_t s, const float* q, const float* k, const float* qw, const float* kw,
                           const float* c, const float* sn, float* qo, float* ko, uint32_t tokens, uint32_t q_heads,
                           uint32_t has_key, uint32_t rope_stride, float eps) {
    const uint32_t total = q_heads + has_key;
    const uint64_t waves = static_cast<uint64_t>(tokens) * ((total + U - 1) / U);
    if (waves > 0x7fffffffu) return hipErrorInvalidValue;
    hipLaunchKernelGGL((qk_norm_rope_token_kernel<P, U, 1, 1, true, SEQ>), dim3(static_cast<uint32_t>(waves)), dim3(64), 0,
                       s, tokens, q_heads, has_key, rope_stride, q, k, c, sn, eps, qw, kw, qo, ko);
    return hipGetLastError();
}

// Wavefronts per token by token count.  A wavefront folds its units' rows
// in order (lane u, unit u), a chain of 2 * P * 64 adds whatever the unit
// count, while its loads, squares and rotations grow with the units it
// holds; few tokens leave most CUs idle, so below 768 tokens a token's
// units are spread over several wavefronts.  Measured on MI355X (8 Q heads
// + K, head_dim 256, per launch over rotating buffer sets):
//   tokens     1 unit/wave  2 units  1 token/wave  4 tokens/workgroup
//   256          4.80        4.81      5.46          6.10 us
//   512          5.78        5.32      6.06          6.27
//   1024         8.32        7.45      6.62          6.51
//   1536        10.63        9.70      7.16          7.45
//   2047        13.00       11.07      7.88          8.00
// and at 4096 tokens 14.17 us with four wavefronts per workgroup against
// 14.25-14.33 with one and 18.3 with two units per wavefront.  With one unit
// per wavefront the unit's fold runs by candidate segments (head_dim 256),
// which moves the first crossover: 256 tokens 3.87 against 4.08 us with two
// units per wavefront, 384 4.31 against 4.39, 512 4.85 against 4.76, 767
// 6.47 against 5.93.  In the C5 decode step (a graph of 35 launches): 256
// tokens 3.59-3.60 us (3.86 with two units per wavefront, 4.72 with one
// wavefront per token); one token 2.20-2.22 (2.55 with the in-order fold).
template <int P, bool SEQ>
hipError_t launch_qk_token_p(hipStream_t s, const float* q, const float* k, const float* qw, const float* kw,
                             const float* c, const float* sn, float* qo, float* ko, uint32_t tokens,
                             uint32_t q_heads, uint32_t has_key, uint32_t rope_stride, float eps) {
    if (tokens >= 2048)
        return launch_qk_token_cfg<P, 1, 4, SEQ>(s, q, k, qw, kw, c, sn, qo, ko, tokens, q_heads, has_key, rope_stride,
                                            eps);
    if (tokens >= 768)
        return launch_qk_token_cfg<P, 1, 1, SEQ>(s, q, k, qw, kw, c, sn, qo, ko, tokens, q_heads, has_key, rope_stride,
                                            eps);
    if (tokens >= 512)
        return launch_qk_split<P, 2, SEQ>(s, q, k, qw, kw, c, sn, qo, ko, tokens, q_heads, has_key, rope_stride, eps);
    return launch_qk_split<P, 1, SEQ>(s, q, k, qw, kw, c, sn, qo, ko, tokens, q_heads, has_key, rope_stride, eps);
}

// Generic head_dim fallback (even head_dim not of the form 64*V): one wave
// per unit, row staged in LDS.
__global__ __launch_bounds__(64) void qk_norm_rope_generic_kernel(
    const float* q, const float* k, const float* q_weight, const float* k_weight,
    const float* cosine, const float* sine, float* q_out, float* k_out, uint32_t tokens,
    uint32_t q_heads, uint32_t has_key, uint32_t head_dim, uint32_t rope_stride, float epsilon,
    int sequential) {
    extern __shared__ float row[];
    __shared__ float inv_shared;
    const uint32_t lane = threadIdx.x;
    const uint32_t total = q_heads + has_key;
    const uint32_t unit = blockIdx.x;
    if (unit >= tokens * total) return;
    const uint32_t t = unit / total, local = unit % total;
    const bool key = local >= q_heads;
    const float* src = key ? k + static_cast<size_t>(t) * head_dim
                           : q + (static_cast<size_t>(t) * q_heads + local) * head_dim;
    float* dst = key ? k_out + static_cast<size_t>(t) * head_dim
                     : q_out + (static_cast<size_t>(t) * q_heads + local) * head_dim;
    const float* w = key ? k_weight : q_weight;
    float partial = 0.0f;
    for (uint32_t i = lane; i < head_dim; i += kWave) {
        float v = src[i];
        row[i] = v;
        partial = partial + v * v;
    }
    __syncthreads();
    float inv;
    if (sequential) {
        if (lane == 0) {
            float s = 0.0f;
            for (uint32_t i = 0; i < head_dim; ++i) s = s + row[i] * row[i];
            inv_shared = inverse_rms(s, static_cast<float>(head_dim), epsilon);
        }
        __syncthreads();
        inv = inv_shared;
    } else {
        inv = inverse_rms(wave_sum(partial), static_cast<float>(head_dim), epsilon);
    }
    const uint32_t half = head_dim / 2;
    for (uint32_t p = lane; p < half; p += kWave) {
        const float x0 = row[p] * inv * w[p];
        const float x1 = row[p + half] * inv * w[p + half];
        const float c = cosine[static_cast<size_t>(t) * rope_stride + p];
        const float s = sine[static_cast<size_t>(t) * rope_stride + p];
        dst[p] = x0 * c - x1 * s;
        dst[p + half] = x0 * s + x1 * c;
    }
}

// Half-split RoPE.  Each thread rotates P consecutive pairs of one
// (token, head): x[p..p+P) and x[p+d/2..p+d/2+P) with cos/sin[t*stride + p..]
// -- 128-bit accesses for the vector forms (P = 4 f32, P = 8 f16),
// nontemporal for the streamed rows, cached for the per-token tables that
// every head of the token reuses.
template <int P>
__device__ __forceinline__ void ld_tab(const float* p, float* dst) {
    if constexpr (P % 4 == 0) {
#pragma unroll
        for (int j = 0; j < P; j += 4) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(p + j);
            dst[j] = v.x;
            dst[j + 1] = v.y;
            dst[j + 2] = v.z;
            dst[j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < P; ++j) dst[j] = p[j];
    }
}

// One thread's P pairs (starting at pair p) of one (token t, head) unit of a
// [tokens, heads, head_dim] tensor; `unit` = t * heads + head.
template <int P>
__device__ __forceinline__ void rope_half_f32_unit(const float* x, const float* cosine, const float* sine,
                                                   float* out, uint64_t unit, uint32_t p, uint32_t t,
                                                   uint32_t head_dim, uint32_t rope_stride) {
    const uint32_t half = head_dim / 2;
    const size_t base = unit * head_dim;
    float a[P], b[P], c[P], s[P];
    if constexpr (P == 4) {
        const f32x4 va = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + base + p));
        const f32x4 vb = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + base + p + half));
        a[0] = va.x; a[1] = va.y; a[2] = va.z; a[3] = va.w;
        b[0] = vb.x; b[1] = vb.y; b[2] = vb.z; b[3] = vb.w;
    } else {
        a[0] = x[base + p];
        b[0] = x[base + p + half];
    }
    const size_t tb = static_cast<size_t>(t) * rope_stride + p;
    ld_tab<P>(cosine + tb, c);
    ld_tab<P>(sine + tb, s);
    float o0[P], o1[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        o0[j] = a[j] * c[j] - b[j] * s[j];
        o1[j] = a[j] * s[j] + b[j] * c[j];
    }
    if constexpr (P == 4) {
        __builtin_nontemporal_store(f32x4{o0[0], o0[1], o0[2], o0[3]}, reinterpret_cast<f32x4*>(out + base + p));
        __builtin_nontemporal_store(f32x4{o1[0], o1[1], o1[2], o1[3]},
                                    reinterpret_cast<f32x4*>(out + base + p + half));
    } else {
        out[base + p] = o0[0];
        out[base + p + half] = o1[0];
    }
}

typedef uint32_t u32x4r __attribute__((ext_vector_type(4)));

template <int P>
__device__ __forceinline__ void rope_half_f16_unit(const uint16_t* x, const float* cosine, const float* sine,
                                                   uint16_t* out, uint64_t unit, uint32_t p, uint32_t t,
                                                   uint32_t head_dim, uint32_t rope_stride) {
    const uint32_t half = head_dim / 2;
    const size_t base = unit * head_dim;
    uint16_t a[P], b[P];
    if constexpr (P == 8) {
        const u32x4r va = __builtin_nontemporal_load(reinterpret_cast<const u32x4r*>(x + base + p));
        const u32x4r vb = __builtin_nontemporal_load(reinterpret_cast<const u32x4r*>(x + base + p + half));
        const uint32_t wa[4] = {va.x, va.y, va.z, va.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[2 * j] = static_cast<uint16_t>(wa[j]);
            a[2 * j + 1] = static_cast<uint16_t>(wa[j] >> 16);
            b[2 * j] = static_cast<uint16_t>(wb[j]);
            b[2 * j + 1] = static_cast<uint16_t>(wb[j] >> 16);
        }
    } else {
        a[0] = x[base + p];
        b[0] = x[base + p + half];
    }
    const size_t tb = static_cast<size_t>(t) * rope_stride + p;
    float c[P], s[P];
    ld_tab<P>(cosine + tb, c);
    ld_tab<P>(sine + tb, s);
    uint16_t o0[P], o1[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        const float x0 = h2f(a[j]), x1 = h2f(b[j]);
        o0[j] = f2h(x0 * c[j] - x1 * s[j]);
        o1[j] = f2h(x0 * s[j] + x1 * c[j]);
    }
    if constexpr (P == 8) {
        u32x4r r0, r1;
        r0.x = o0[0] | (static_cast<uint32_t>(o0[1]) << 16);
        r0.y = o0[2] | (static_cast<uint32_t>(o0[3]) << 16);
        r0.z = o0[4] | (static_cast<uint32_t>(o0[5]) << 16);
        r0.w = o0[6] | (static_cast<uint32_t>(o0[7]) << 16);
        r1.x = o1[0] | (static_cast<uint32_t>(o1[1]) << 16);
        r1.y = o1[2] | (static_cast<uint32_t>(o1[3]) << 16);
        r1.z = o1[4] | (static_cast<uint32_t>(o1[5]) << 16);
        r1.w = o1[6] | (static_cast<uint32_t>(o1[7]) << 16);
        __builtin_nontemporal_store(r0, reinterpret_cast<u32x4r*>(out + base + p));
        __builtin_nontemporal_store(r1, reinterpret_cast<u32x4r*>(out + base + p + half));
    } else {
        out[base + p] = o0[0];
        out[base + p + half] = o1[0];
    }
}

// Interleaved pairs (NeuralOps::rope): out[2p] = x0*c - x1*s, out[2p+1] = x0*s + x1*c,
// one cos/sin row shared by every input row.
__global__ __launch_bounds__(256) void rope_interleaved_kernel(const float* x, const float* cosine,
                                                               const float* sine, float* out,
                                                               uint32_t rows, uint32_t hidden) {
    const uint32_t pairs = hidden / 2;
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<uint64_t>(rows) * pairs) return;
    const uint32_t p = static_cast<uint32_t>(i % pairs);
    const size_t b = (i / pairs) * hidden + 2 * p;
    const float x0 = x[b], x1 = x[b + 1];
    const float c = cosine[p], s = sine[p];
    const float o0 = x0 * c - x1 * s;
    const float o1 = x0 * s + x1 * c;
    out[b] = o0;
    out[b + 1] = o1;
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

template <int V, int UNITS>
hipError_t launch_qk(hipStream_t s, bool seq, const float* q, const float* k, const float* qw,
                     const float* kw, const float* c, const float* sn, float* qo, float* ko,
                     uint32_t tokens, uint32_t q_heads, uint32_t has_key, uint32_t rope_stride,
                     float eps) {
    const uint32_t units = tokens * (q_heads + has_key);
    const dim3 grid((units + UNITS - 1) / UNITS);
    if (seq)
        hipLaunchKernelGGL((qk_norm_rope_kernel<V, UNITS, true>), grid, dim3(kWave), 0, s, q, k, qw,
                           kw, c, sn, qo, ko, tokens, q_heads, has_key, rope_stride, eps);
    else
        hipLaunchKernelGGL((qk_norm_rope_kernel<V, UNITS, false>), grid, dim3(kWave), 0, s, q, k, qw,
                           kw, c, sn, qo, ko, tokens, q_heads, has_key, rope_stride, eps);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_qk_norm_rope_f32(hipStream_t stream, Reduction red, const float* q, const float* k,
                                   const float* q_weight, const float* k_weight,
                                   const float* cosine, const float* sine, float* q_out,
                                   float* k_out, uint32_t tokens, uint32_t q_heads,
                                   uint32_t has_key, uint32_t head_dim, uint32_t rope_stride,
                                   float epsilon) {
    // the rotation after the norm can cancel, so only ATLAS_REDUCTION_WIDE
    // reorders the sum of squares here; kAuto keeps the sequential fold
    const bool seq = red != kWide;
    // Token engine: head_dim = 128*P, at most 16 units per token, operands
    // and per-token cos/sin rows aligned to P floats; the in-order fold, or
    // under WIDE the wavefront tree sum.  Measured on MI355X (C5 decode, 8 Q
    // heads + K, head_dim 256): WIDE took 12.7 us at 256 tokens and 9.5 at
    // one token on the unit engine below, which puts 16 units on one
    // wavefront one after another.
    {
        const uint32_t P = head_dim / 128;
        const uintptr_t pa = 4u * (P == 0 ? 1 : P) > 16 ? 16 : 4u * (P == 0 ? 1 : P);
        const bool ok = head_dim % 128 == 0 && (P == 1 || P == 2 || P == 4) && q_heads + has_key <= 16 &&
                        q_heads + has_key > 0 && aligned(q, pa) && aligned(q_out, pa) && aligned(q_weight, pa) &&
                        aligned(cosine, pa) && aligned(sine, pa) && rope_stride % P == 0 &&
                        (!has_key || (aligned(k, pa) && aligned(k_out, pa) && aligned(k_weight, pa)));
        if (ok) {
#define ATLAS_QK_TOKEN(PP)                                                                                        \
    return seq ? launch_qk_token_p<PP, true>(stream, q, k, q_weight, k_weight, cosine, sine, q_out, k_out, tokens, \
                                             q_heads, has_key, rope_stride, epsilon)                                 \
               : launch_qk_token_p<PP, false>(stream, q, k, q_weight, k_weight, cosine, sine, q_out, k_out,         \
                                              tokens, q_heads, has_key, rope_stride, epsilon);
            if (P == 1) ATLAS_QK_TOKEN(1)
            if (P == 2) ATLAS_QK_TOKEN(2)
            ATLAS_QK_TOKEN(4)
#undef ATLAS_QK_TOKEN
        }
    }
    // Unit engine: head_dim = 64*V, 16-byte aligned operands (8-byte for V=2),
    // and per-token cos/sin rows aligned to the vector width.
    const uintptr_t va = head_dim == 128 ? 8 : 16;
    const bool vec_ok = (head_dim == 128 || head_dim == 256 || head_dim == 512) && aligned(q, va) &&
                        aligned(q_out, va) && aligned(q_weight, va) && aligned(cosine, va) &&
                        aligned(sine, va) && (rope_stride % (head_dim / 64)) == 0 &&
                        (!has_key || (aligned(k, va) && aligned(k_out, va) && aligned(k_weight, va)));
    if (vec_ok) {
        if (head_dim == 256)
            return launch_qk<4, 16>(stream, seq, q, k, q_weight, k_weight, cosine, sine, q_out, k_out,
                                    tokens, q_heads, has_key, rope_stride, epsilon);
        if (head_dim == 512)
            return launch_qk<8, 8>(stream, seq, q, k, q_weight, k_weight, cosine, sine, q_out, k_out,
                                   tokens, q_heads, has_key, rope_stride, epsilon);
        return launch_qk<2, 16>(stream, seq, q, k, q_weight, k_weight, cosine, sine, q_out, k_out,
                                tokens, q_heads, has_key, rope_stride, epsilon);
    }
    const uint32_t units = tokens * (q_heads + has_key);
    hipLaunchKernelGGL(qk_norm_rope_generic_kernel, dim3(units), dim3(kWave),
                       static_cast<size_t>(head_dim) * sizeof(float), stream, q, k, q_weight,
                       k_weight, cosine, sine, q_out, k_out, tokens, q_heads, has_key, head_dim,
                       rope_stride, epsilon, seq ? 1 : 0);
    return hipGetLastError();
}

// Two tensors sharing the cos/sin rows (Q and K of the same tokens): threads
// [0, tokens*heads0*groups) rotate x0, the following ones x1; heads1 = 0
// rotates one tensor.  Parameters in kernarg-preload order: the counts, the inputs and
// cos/sin fill the first 56 bytes (user SGPRs at wave launch), the outputs
// follow.
template <int P>
__global__ __launch_bounds__(256) void rope_half_f32_kernel(uint32_t tokens, uint32_t head_dim,
                                                            uint32_t rope_stride, uint32_t heads0, uint32_t heads1,
                                                            const float* x0, const float* x1, const float* cosine,
                                                            const float* sine, float* out0, float* out1) {
    const uint32_t groups = (head_dim / 2) / P;
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;  // 256-thread workgroups
    const uint64_t total0 = static_cast<uint64_t>(tokens) * heads0 * groups;
    const uint64_t total1 = static_cast<uint64_t>(tokens) * heads1 * groups;
    const bool second = i >= total0;
    if (second && i - total0 >= total1) return;
    const uint64_t j = second ? i - total0 : i;
    const uint64_t unit = j / groups;
    const uint32_t t = static_cast<uint32_t>(unit / (second ? heads1 : heads0));
    const uint32_t p = static_cast<uint32_t>(j - unit * groups) * P;
    if (second)
        rope_half_f32_unit<P>(x1, cosine, sine, out1, unit, p, t, head_dim, rope_stride);
    else
        rope_half_f32_unit<P>(x0, cosine, sine, out0, unit, p, t, head_dim, rope_stride);
}

template <int P>
__global__ __launch_bounds__(256) void rope_half_f16_kernel(uint32_t tokens, uint32_t head_dim,
                                                            uint32_t rope_stride, uint32_t heads0, uint32_t heads1,
                                                            const uint16_t* x0, const uint16_t* x1, const float* cosine,
                                                            const float* sine, uint16_t* out0, uint16_t* out1) {
    const uint32_t groups = (head_dim / 2) / P;
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 256u + threadIdx.x;  // 256-thread workgroups
    const uint64_t total0 = static_cast<uint64_t>(tokens) * heads0 * groups;
    const uint64_t total1 = static_cast<uint64_t>(tokens) * heads1 * groups;
    const bool second = i >= total0;
    if (second && i - total0 >= total1) return;
    const uint64_t j = second ? i - total0 : i;
    const uint64_t unit = j / groups;
    const uint32_t t = static_cast<uint32_t>(unit / (second ? heads1 : heads0));
    const uint32_t p = static_cast<uint32_t>(j - unit * groups) * P;
    if (second)
        rope_half_f16_unit<P>(x1, cosine, sine, out1, unit, p, t, head_dim, rope_stride);
    else
        rope_half_f16_unit<P>(x0, cosine, sine, out0, unit, p, t, head_dim, rope_stride);
}

// Token engine for the half-split rotation: one wavefront per token covers
// every head of both tensors.  A head row of d elements is 2G 16-byte
// vectors (G = (d/2)/V, V = 8 halves or 4 floats); lane l holds vector
// c = l mod 2G of heads l/2G, l/2G + 64/2G, ..., so each load and store
// instruction covers whole consecutive rows.  Lanes c < G hold x[p] (first
// half), lanes c >= G hold x[p + d/2]; the partner vector sits in lane l ^ G
// and is exchanged with one cross-lane shuffle per dword.  The token's
// cos/sin group (pairs [(c mod G)V, +V)) is loaded once per lane and reused by
// all its heads.  Every head's loads are issued before the first rotation
// (NI head steps per lane, clamped to a valid head and never stored past the
// end).  Same roundings as rope_half_f*_unit: (x0*c) - (x1*s) for the first
// half, (x0*s) + (x1*c) for the second.
//
// GSH = log2(G) when it is 2 or 3 (G = 4: f16 head_dim 64; G = 8: f32
// head_dim 64, f16 head_dim 128): the lanes of the second half hold their
// vectors in reverse order (lane G + j holds vector 2G - 1 - j), so a lane's
// partner is its mirror within the 2G-lane group and the exchange is one
// DPP move per dword (row_half_mirror / row_mirror) instead of a cross-lane
// shuffle through the LDS crossbar.  GSH = -1: G from g_shift at run time,
// natural order, shuffle exchange.
template <int GSH>
__device__ __forceinline__ uint32_t rope_partner(uint32_t own, uint32_t G) {
    if constexpr (GSH == 2)
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(own), 0x141, 0xf, 0xf, false));
    else if constexpr (GSH == 3)
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(own), 0x140, 0xf, 0xf, false));
    else
        return static_cast<uint32_t>(__shfl_xor(static_cast<int>(own), static_cast<int>(G), kWave));
}

// Parameter order: the counts, the input rows and cos/sin fill the first 56
// bytes, which arrive in SGPRs at wave launch (kernarg preload); the
// outputs, needed only at the stores, follow.
template <bool F16, int NI, int GSH>
__global__ __launch_bounds__(256) void rope_half_token_kernel(uint32_t tokens, uint32_t head_dim, uint32_t heads0,
                                                              uint32_t heads1, uint32_t rope_stride,
                                                              uint32_t g_shift_rt, const uint8_t* x0,
                                                              const uint8_t* x1, const float* cosine,
                                                              const float* sine, uint8_t* out0, uint8_t* out1) {
    constexpr uint32_t V = F16 ? 8 : 4;
    constexpr uint32_t kEsz = F16 ? 2 : 4;
    constexpr bool kMirror = GSH >= 0;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= tokens) return;
    const uint32_t g_shift = kMirror ? static_cast<uint32_t>(GSH) : g_shift_rt;
    const uint32_t G = 1u << g_shift;
    const uint32_t c = lane & (2 * G - 1), hl = lane >> (g_shift + 1);
    const bool first = c < G;
    // the vector of the head row this lane holds, and its pair group
    const uint32_t vec = first || !kMirror ? c : 3 * G - 1 - c;
    const uint32_t g = vec & (G - 1);
    const uint32_t hps = 32u >> g_shift;  // heads per step
    const uint32_t heads = heads0 + heads1;
    const size_t row_bytes = static_cast<size_t>(head_dim) * kEsz;
    float cs[V], sn[V];
    ld_tab<V>(cosine + static_cast<size_t>(t) * rope_stride + g * V, cs);
    ld_tab<V>(sine + static_cast<size_t>(t) * rope_stride + g * V, sn);
    // Both halves as one form, y = own*c + par*s' with s' = -s on the first
    // half's lanes: x0*c - x1*s is x0*c + x1*(-s) (IEEE subtraction adds the
    // negation, and round-to-nearest is symmetric in sign, so fl(x1*(-s)) =
    // -fl(x1*s), zeros included), and x0*s + x1*c is x1*c + x0*s (addition
    // commutes).  No per-value select between the halves' formulas.
#pragma unroll
    for (int j = 0; j < static_cast<int>(V); ++j) sn[j] = first ? -sn[j] : sn[j];
    // row offset of head step i (clamped to a valid head for the load; a step
    // past the last head is never stored, so the store reuses the offset)
    size_t off[NI];
    bool sec[NI];
    u32x4r v[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const uint32_t h = min(hl + static_cast<uint32_t>(i) * hps, heads - 1);
        sec[i] = h >= heads0;
        off[i] = (sec[i] ? static_cast<size_t>(t) * heads1 + (h - heads0) : static_cast<size_t>(t) * heads0 + h) *
                     row_bytes + vec * 16u;
        v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4r*>((sec[i] ? x1 : x0) + off[i]));
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        // partner vector: the same pairs of the other half (lane ^ G, same head)
        const uint32_t own[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        uint32_t par[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) par[w] = rope_partner<GSH>(own[w], G);
        if (hl + static_cast<uint32_t>(i) * hps < heads) {
            u32x4r r;
            uint32_t* o = reinterpret_cast<uint32_t*>(&r);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                if constexpr (F16) {
                    // each product rounded once (the f16 operand widens inside
                    // the multiply), then the sum
                    const float y0 = mul_f16_half<0>(cs[2 * w], own[w]) + mul_f16_half<0>(sn[2 * w], par[w]);
                    const float y1 = mul_f16_half<1>(cs[2 * w + 1], own[w]) + mul_f16_half<1>(sn[2 * w + 1], par[w]);
                    o[w] = static_cast<uint32_t>(f2h(y0)) | (static_cast<uint32_t>(f2h(y1)) << 16);
                } else {
                    o[w] = __float_as_uint(__uint_as_float(own[w]) * cs[w] + __uint_as_float(par[w]) * sn[w]);
                }
            }
            __builtin_nontemporal_store(r, reinterpret_cast<u32x4r*>((sec[i] ? out1 : out0) + off[i]));
        }
    }
}

// Launches the token engine when its layout applies: 16-byte aligned
// operands, (d/2) a multiple of the vector width with a power-of-two number
// of vectors per head (2G <= 64), cos/sin rows on 16-byte boundaries, at
// most 8 head steps per lane, and at least 8192 (token, head) rows.  Returns
// false to fall back to the per-pair kernels.
template <bool F16>
bool launch_rope_half_token(hipStream_t stream, const void* x0, void* out0, uint32_t heads0, const void* x1,
                            void* out1, uint32_t heads1, const float* cosine, const float* sine, uint32_t tokens,
                            uint32_t head_dim, uint32_t rope_stride) {
    constexpr uint32_t V = F16 ? 8 : 4;
    const uint32_t half = head_dim / 2;
    if (half == 0 || half % V != 0 || rope_stride % 4 != 0 || tokens == 0) return false;
    const uint32_t G = half / V;
    if (G > 32 || (G & (G - 1)) != 0) return false;
    if (!aligned(x0, 16) || !aligned(out0, 16) || !aligned(cosine, 16) || !aligned(sine, 16) ||
        (heads1 != 0 && (!aligned(x1, 16) || !aligned(out1, 16))))
        return false;
    const uint32_t g_shift = static_cast<uint32_t>(__builtin_ctz(G));
    const uint32_t hps = 32u >> g_shift;
    const uint32_t heads = heads0 + heads1;
    if (heads == 0) return false;
    // small batches are latency-bound and measured faster on the per-pair
    // kernels (SmolLM2 shape, 128 tokens x 12 heads: 4.2 against 4.4 us)
    if (static_cast<uint64_t>(tokens) * heads < 8192) return false;
    const uint32_t ni = (heads + hps - 1) / hps;
    const dim3 grid((tokens + 3) / 4);
    const uint8_t* a0 = static_cast<const uint8_t*>(x0);
    const uint8_t* a1 = static_cast<const uint8_t*>(x1);
    uint8_t* b0 = static_cast<uint8_t*>(out0);
    uint8_t* b1 = static_cast<uint8_t*>(out1);
#define ATLAS_ROPE_TOKEN_CASE(N)                                                                                 \
    case N:                                                                                                      \
        if (g_shift == 2)                                                                                        \
            hipLaunchKernelGGL((rope_half_token_kernel<F16, N, 2>), grid, dim3(256), 0, stream, tokens, head_dim,   \
                               heads0, heads1, rope_stride, g_shift, a0, a1, cosine, sine, b0, b1);              \
        else if (g_shift == 3)                                                                                   \
            hipLaunchKernelGGL((rope_half_token_kernel<F16, N, 3>), grid, dim3(256), 0, stream, tokens, head_dim,   \
                               heads0, heads1, rope_stride, g_shift, a0, a1, cosine, sine, b0, b1);              \
        else                                                                                                     \
            hipLaunchKernelGGL((rope_half_token_kernel<F16, N, -1>), grid, dim3(256), 0, stream, tokens, head_dim, \
                               heads0, heads1, rope_stride, g_shift, a0, a1, cosine, sine, b0, b1);              \
        return true;
    switch (ni) {
        ATLAS_ROPE_TOKEN_CASE(1) ATLAS_ROPE_TOKEN_CASE(2) ATLAS_ROPE_TOKEN_CASE(3) ATLAS_ROPE_TOKEN_CASE(4)
        ATLAS_ROPE_TOKEN_CASE(5) ATLAS_ROPE_TOKEN_CASE(6) ATLAS_ROPE_TOKEN_CASE(7) ATLAS_ROPE_TOKEN_CASE(8)
        default: return false;
    }
#undef ATLAS_ROPE_TOKEN_CASE
}

hipError_t launch_rope_half_pair_f32(hipStream_t stream, const float* x0, float* out0, uint32_t heads0,
                                     const float* x1, float* out1, uint32_t heads1, const float* cosine,
                                     const float* sine, uint32_t tokens, uint32_t head_dim, uint32_t rope_stride) {
    if (launch_rope_half_token<false>(stream, x0, out0, heads0, x1, out1, heads1, cosine, sine, tokens, head_dim,
                                      rope_stride))
        return hipGetLastError();
    const uint32_t half = head_dim / 2;
    const bool vec = (half % 4) == 0 && (rope_stride % 4) == 0 && aligned(x0, 16) && aligned(out0, 16) &&
                     (heads1 == 0 || (aligned(x1, 16) && aligned(out1, 16))) && aligned(cosine, 16) &&
                     aligned(sine, 16);
    const uint32_t P = vec ? 4 : 1;
    const uint64_t threads = static_cast<uint64_t>(tokens) * (static_cast<uint64_t>(heads0) + heads1) * (half / P);
    const dim3 grid(static_cast<uint32_t>((threads + 255) / 256));
    if (vec)
        hipLaunchKernelGGL((rope_half_f32_kernel<4>), grid, dim3(256), 0, stream, tokens, head_dim, rope_stride,
                           heads0, heads1, x0, x1, cosine, sine, out0, out1);
    else
        hipLaunchKernelGGL((rope_half_f32_kernel<1>), grid, dim3(256), 0, stream, tokens, head_dim, rope_stride,
                           heads0, heads1, x0, x1, cosine, sine, out0, out1);
    return hipGetLastError();
}

hipError_t launch_rope_half_pair_f16(hipStream_t stream, const uint16_t* x0, uint16_t* out0, uint32_t heads0,
                                     const uint16_t* x1, uint16_t* out1, uint32_t heads1, const float* cosine,
                                     const float* sine, uint32_t tokens, uint32_t head_dim, uint32_t rope_stride) {
    if (launch_rope_half_token<true>(stream, x0, out0, heads0, x1, out1, heads1, cosine, sine, tokens, head_dim,
                                     rope_stride))
        return hipGetLastError();
    const uint32_t half = head_dim / 2;
    const bool vec = (half % 8) == 0 && (rope_stride % 4) == 0 && aligned(x0, 16) && aligned(out0, 16) &&
                     (heads1 == 0 || (aligned(x1, 16) && aligned(out1, 16))) && aligned(cosine, 16) &&
                     aligned(sine, 16);
    const uint32_t P = vec ? 8 : 1;
    const uint64_t threads = static_cast<uint64_t>(tokens) * (static_cast<uint64_t>(heads0) + heads1) * (half / P);
    const dim3 grid(static_cast<uint32_t>((threads + 255) / 256));
    if (vec)
        hipLaunchKernelGGL((rope_half_f16_kernel<8>), grid, dim3(256), 0, stream, tokens, head_dim, rope_stride,
                           heads0, heads1, x0, x1, cosine, sine, out0, out1);
    else
        hipLaunchKernelGGL((rope_half_f16_kernel<1>), grid, dim3(256), 0, stream, tokens, head_dim, rope_stride,
                           heads0, heads1, x0, x1, cosine, sine, out0, out1);
    return hipGetLastError();
}

hipError_t launch_rope_half_f32(hipStream_t stream, const float* x, const float* cosine, const float* sine,
                                float* out, uint32_t tokens, uint32_t heads, uint32_t head_dim,
                                uint32_t rope_stride) {
    return launch_rope_half_pair_f32(stream, x, out, heads, nullptr, nullptr, 0, cosine, sine, tokens, head_dim,
                                     rope_stride);
}

hipError_t launch_rope_half_f16(hipStream_t stream, const uint16_t* x, const float* cosine, const float* sine,
                                uint16_t* out, uint32_t tokens, uint32_t heads, uint32_t head_dim,
                                uint32_t rope_stride) {
    return launch_rope_half_pair_f16(stream, x, out, heads, nullptr, nullptr, 0, cosine, sine, tokens, head_dim,
                                     rope_stride);
}

hipError_t launch_rope_interleaved_f32(hipStream_t stream, const float* x, const float* cosine,
                                       const float* sine, float* out, uint32_t rows,
                                       uint32_t hidden) {
    const uint64_t threads = static_cast<uint64_t>(rows) * (hidden / 2);
    const dim3 grid(static_cast<uint32_t>((threads + 255) / 256));
    hipLaunchKernelGGL(rope_interleaved_kernel, grid, dim3(256), 0, stream, x, cosine, sine, out, rows,
                       hidden);
    return hipGetLastError();
}

}  // namespace atlas
