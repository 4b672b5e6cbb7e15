// glu_kernels.hip -- gated activations (SwiGLU / GeGLU), their PLE variant
// and the operator-API elementwise ops.
//
// Reference semantics (bisegni/atlas, crates/atlas-metal/src/kernels.metal):
//   vector_add_f32 :5-14, scalar_multiply_f32 :16-25, silu_f32 :27-36,
//   vector_multiply_f32 :64-69, gelu_f32 :752-767, gelu_multiply_f32 :773-784,
//   ple_gelu_multiply_offset_f32 :790-801, vector_multiply_offset_batch_f32 :83-92.
// The fused SwiGLU is silu_f32 then vector_multiply_f32 with the activated
// value kept in a register instead of an HBM round trip (same f32 rounding).
//
// Streaming layout: each thread moves 4 consecutive elements per operand with
// one 128-bit load / store; the grid is sized so every CU holds several
// waves and each thread walks a short grid-stride loop.
#include "device_common.hpp"
#include "launch.hpp"

namespace atlas {
namespace {

template <int OP>
__device__ __forceinline__ float elt(float a, float b, float scalar) {
    if (OP == kEltSilu) return silu_f32(a);
    if (OP == kEltGelu) return gelu_tanh_f32(a);
    if (OP == kEltSwiglu) return silu_f32(a) * b;
    if (OP == kEltGeglu) return gelu_tanh_f32(a) * b;
    if (OP == kEltAdd) return a + b;
    if (OP == kEltMul) return a * b;
    return a * scalar;  // kEltScale
}

constexpr bool binary(int op) { return op == kEltSwiglu || op == kEltGeglu || op == kEltAdd || op == kEltMul; }

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One float4 per operand per thread per iteration, nontemporal loads and
// stores (each byte is touched once, so caching it only evicts other data).
template <int OP>
__global__ __launch_bounds__(256) void elementwise_vec_kernel(const float* a, const float* b,
                                                              float scalar, float* out, uint64_t n4) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const f32x4 va = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a) + i);
        f32x4 vb = f32x4{0.f, 0.f, 0.f, 0.f};
        if (binary(OP)) vb = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(b) + i);
        f32x4 r;
        if (OP == kEltSilu || OP == kEltSwiglu || OP == kEltGelu || OP == kEltGeglu) {
            float g[4] = {va.x, va.y, va.z, va.w};
            if (OP == kEltSilu || OP == kEltSwiglu)
                silu_lanes(g);
            else
                gelu_lanes(g);
            r = binary(OP) ? f32x4{g[0] * vb.x, g[1] * vb.y, g[2] * vb.z, g[3] * vb.w}
                           : f32x4{g[0], g[1], g[2], g[3]};
        } else {
            r.x = elt<OP>(va.x, vb.x, scalar);
            r.y = elt<OP>(va.y, vb.y, scalar);
            r.z = elt<OP>(va.z, vb.z, scalar);
            r.w = elt<OP>(va.w, vb.w, scalar);
        }
        __builtin_nontemporal_store(r, reinterpret_cast<f32x4*>(out) + i);
    }
}

template <int OP>
__global__ __launch_bounds__(256) void elementwise_scalar_kernel(const float* a, const float* b,
                                                                 float scalar, float* out,
                                                                 uint64_t begin, uint64_t n) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = begin + static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = elt<OP>(a[i], binary(OP) ? b[i] : 0.0f, scalar);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Eight f16 values per operand per thread (one 128-bit nontemporal access).
// Gates are widened exactly to f32; a wavefront holding a gate of magnitude
// >= 87 (or inf/NaN) takes silu_lanes' full-range form.
__device__ __forceinline__ uint32_t mul_pack_f16(float g_lo, float g_hi, uint32_t u) {
    const uint32_t lo = f2h(mul_f16_half<0>(g_lo, u));
    const uint32_t hi = f2h(mul_f16_half<1>(g_hi, u));
    return lo | (hi << 16);
}

__global__ __launch_bounds__(256) void swiglu_f16_kernel(const uint16_t* gate, const uint16_t* up,
                                                         uint16_t* out, uint64_t n8) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const u32x4 g = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gate) + i);
        const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(up) + i);
        float a[8] = {h2f(static_cast<uint16_t>(g.x)), h2f(static_cast<uint16_t>(g.x >> 16)),
                      h2f(static_cast<uint16_t>(g.y)), h2f(static_cast<uint16_t>(g.y >> 16)),
                      h2f(static_cast<uint16_t>(g.z)), h2f(static_cast<uint16_t>(g.z >> 16)),
                      h2f(static_cast<uint16_t>(g.w)), h2f(static_cast<uint16_t>(g.w >> 16))};
        silu_lanes(a);
        const u32x4 r{mul_pack_f16(a[0], a[1], u.x), mul_pack_f16(a[2], a[3], u.y), mul_pack_f16(a[4], a[5], u.z),
                      mul_pack_f16(a[6], a[7], u.w)};
        __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(out) + i);
    }
}

__global__ __launch_bounds__(256) void swiglu_f16_tail_kernel(const uint16_t* gate, const uint16_t* up,
                                                              uint16_t* out, uint64_t begin, uint64_t n) {
    const uint64_t i = begin + static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f2h(silu_f32(h2f(gate[i])) * h2f(up[i]));
}

// out[r, i] = gelu(gate[r, i]) * ple[r * ple_row_stride + ple_offset + i]
__global__ __launch_bounds__(256) void geglu_offset_kernel(const float* gate, const float* ple,
                                                           float* out, uint32_t ple_offset,
                                                           uint32_t ple_row_stride, uint32_t width,
                                                           uint32_t rows) {
    const uint64_t n = static_cast<uint64_t>(rows) * width;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t r = i / width, c = i % width;
        out[i] = gelu_tanh_f32(gate[i]) * ple[r * ple_row_stride + ple_offset + c];
    }
}

// The same product, four columns per thread with 128-bit accesses: needs
// width, ple_offset and ple_row_stride divisible by 4, 16-byte aligned
// buffers and rows * width / 4 < 2^32 (all in float4 units below).
template <int V>
struct VecOf;
template <>
struct VecOf<1> {
    typedef float type;
};
template <>
struct VecOf<4> {
    typedef f32x4 type;
};

template <int V>
__global__ __launch_bounds__(256) void geglu_offset_vec_kernel(const float* gate, const float* ple, float* out,
                                                               uint32_t ple_offset_v, uint32_t ple_row_stride_v,
                                                               uint32_t width_v, uint32_t nv) {
    typedef typename VecOf<V>::type vt;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nv) return;
    const uint32_t r = i / width_v, c = i - r * width_v;
    const vt g = __builtin_nontemporal_load(reinterpret_cast<const vt*>(gate) + i);
    const vt p = reinterpret_cast<const vt*>(ple)[static_cast<uint64_t>(r) * ple_row_stride_v + ple_offset_v + c];
    float v[V], pv[V];
    if constexpr (V == 1) {
        v[0] = g;
        pv[0] = p;
    } else {
#pragma unroll
        for (int k = 0; k < V; ++k) {
            v[k] = g[k];
            pv[k] = p[k];
        }
    }
    gelu_lanes(v);
    vt o;
    if constexpr (V == 1) {
        o = v[0] * pv[0];
    } else {
#pragma unroll
        for (int k = 0; k < V; ++k) o[k] = v[k] * pv[k];
    }
    __builtin_nontemporal_store(o, reinterpret_cast<vt*>(out) + i);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// 256-thread blocks, one work item per thread up to 2^20 blocks (one pass
// over the data measured fastest on MI355X); larger ranges use the
// grid-stride loop.
uint32_t grid_for(uint64_t work_items) {
    uint64_t blocks = (work_items + 255) / 256;
    const uint64_t cap = 1ull << 20;
    if (blocks > cap) blocks = cap;
    if (blocks == 0) blocks = 1;
    return static_cast<uint32_t>(blocks);
}

template <int OP>
hipError_t launch_op(hipStream_t s, const float* a, const float* b, float scalar, float* out, uint64_t n) {
    const bool vec = aligned16(a) && aligned16(out) && (!binary(OP) || aligned16(b));
    uint64_t done = 0;
    if (vec && n >= 4) {
        const uint64_t n4 = n / 4;
        hipLaunchKernelGGL((elementwise_vec_kernel<OP>), dim3(grid_for(n4)), dim3(256), 0, s, a, b, scalar,
                           out, n4);
        done = n4 * 4;
    }
    if (done < n)
        hipLaunchKernelGGL((elementwise_scalar_kernel<OP>), dim3(grid_for(n - done)), dim3(256), 0, s, a, b,
                           scalar, out, done, n);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_elementwise_f32(hipStream_t stream, EltOp op, const float* a, const float* b,
                                  float scalar, float* out, uint64_t n) {
    switch (op) {
        case kEltSilu: return launch_op<kEltSilu>(stream, a, b, scalar, out, n);
        case kEltGelu: return launch_op<kEltGelu>(stream, a, b, scalar, out, n);
        case kEltSwiglu: return launch_op<kEltSwiglu>(stream, a, b, scalar, out, n);
        case kEltGeglu: return launch_op<kEltGeglu>(stream, a, b, scalar, out, n);
        case kEltAdd: return launch_op<kEltAdd>(stream, a, b, scalar, out, n);
        case kEltMul: return launch_op<kEltMul>(stream, a, b, scalar, out, n);
        case kEltScale: return launch_op<kEltScale>(stream, a, b, scalar, out, n);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_swiglu_f16(hipStream_t stream, const uint16_t* gate, const uint16_t* up, uint16_t* out,
                             uint64_t n) {
    const bool vec = aligned16(gate) && aligned16(up) && aligned16(out);
    uint64_t done = 0;
    if (vec && n >= 8) {
        const uint64_t n8 = n / 8;
        // one item per thread (a grid of 2048 resident workgroups, each
        // thread requesting its next item before computing the current one,
        // measured slower at C2: 18.5-19.1 against 18.1-18.3 us)
        hipLaunchKernelGGL(swiglu_f16_kernel, dim3(grid_for(n8)), dim3(256), 0, stream, gate, up, out, n8);
        done = n8 * 8;
    }
    if (done < n) {
        const uint64_t rest = n - done;
        hipLaunchKernelGGL(swiglu_f16_tail_kernel, dim3(static_cast<uint32_t>((rest + 255) / 256)), dim3(256), 0,
                           stream, gate, up, out, done, n);
    }
    return hipGetLastError();
}

hipError_t launch_geglu_offset_f32(hipStream_t stream, const float* gate, const float* ple, float* out,
                                   uint32_t ple_offset, uint32_t ple_row_stride, uint32_t width,
                                   uint32_t rows) {
    const uint64_t n = static_cast<uint64_t>(rows) * width;
    if (n == 0) return hipSuccess;
    if (width % 4 == 0 && ple_offset % 4 == 0 && ple_row_stride % 4 == 0 && n / 4 < (1ull << 32) &&
        aligned16(gate) && aligned16(ple) && aligned16(out)) {
        // 64-thread blocks while the whole range is under 2048 full blocks, so
        // a decode-sized range (256 rows x 256) still spreads over every CU.
        // From 16384 values (256 wavefronts at one value per lane) up to that
        // size, one value per lane: the GELU's dependent chain, not the bytes,
        // bounds a decode-sized launch, and four values per lane leave three of
        // each CU's SIMDs idle.  Measured on MI355X (C5 decode, 256 x 256):
        // 2.24-2.25 us against 2.39 with four values per lane and 2.26 with two;
        // one row (256 values) 1.78 with four against 1.86-1.87.
        const uint32_t n4 = static_cast<uint32_t>(n / 4);
        if (n >= 16384u && n4 < 256u * 2048u) {
            // 256-thread workgroups: 2.20 us against 2.22-2.23 with 128 and
            // 2.25 with 64 at 256 x 256
            const uint32_t n1 = static_cast<uint32_t>(n);
            constexpr uint32_t kTpb = 256;
            hipLaunchKernelGGL((geglu_offset_vec_kernel<1>), dim3((n1 + kTpb - 1) / kTpb), dim3(kTpb), 0, stream, gate,
                               ple, out, ple_offset, ple_row_stride, width, n1);
            return hipGetLastError();
        }
        const uint32_t threads = n4 >= 256u * 2048u ? 256u : 64u;
        hipLaunchKernelGGL((geglu_offset_vec_kernel<4>), dim3((n4 + threads - 1) / threads), dim3(threads), 0, stream,
                           gate, ple, out, ple_offset / 4, ple_row_stride / 4, width / 4, n4);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(geglu_offset_kernel, dim3(grid_for(n)), dim3(256), 0, stream, gate, ple, out, ple_offset,
                       ple_row_stride, width, rows);
    return hipGetLastError();
}

}  // namespace atlas
