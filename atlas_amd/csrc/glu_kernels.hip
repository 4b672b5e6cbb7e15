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

template <int OP>
__global__ __launch_bounds__(256) void elementwise_vec_kernel(const float* a, const float* b,
                                                              float scalar, float* out, uint64_t n4) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        float4 va = reinterpret_cast<const float4*>(a)[i];
        float4 vb = make_float4(0.f, 0.f, 0.f, 0.f);
        if (binary(OP)) vb = reinterpret_cast<const float4*>(b)[i];
        float4 r;
        r.x = elt<OP>(va.x, vb.x, scalar);
        r.y = elt<OP>(va.y, vb.y, scalar);
        r.z = elt<OP>(va.z, vb.z, scalar);
        r.w = elt<OP>(va.w, vb.w, scalar);
        reinterpret_cast<float4*>(out)[i] = r;
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

struct h4 {
    uint16_t v[4];
};

__global__ __launch_bounds__(256) void swiglu_f16_kernel(const uint16_t* gate, const uint16_t* up,
                                                         uint16_t* out, uint64_t n4) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        h4 g = reinterpret_cast<const h4*>(gate)[i];
        h4 u = reinterpret_cast<const h4*>(up)[i];
        h4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r.v[j] = f2h(silu_f32(h2f(g.v[j])) * h2f(u.v[j]));
        reinterpret_cast<h4*>(out)[i] = r;
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// 256-thread blocks; at most 8 blocks per CU worth of grid (256 CUs), the
// rest is covered by the grid-stride loop.
uint32_t grid_for(uint64_t work_items) {
    uint64_t blocks = (work_items + 255) / 256;
    const uint64_t cap = 256ull * 16;
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
    const bool vec = (reinterpret_cast<uintptr_t>(gate) & 7) == 0 &&
                     (reinterpret_cast<uintptr_t>(up) & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0;
    uint64_t done = 0;
    if (vec && n >= 4) {
        const uint64_t n4 = n / 4;
        hipLaunchKernelGGL(swiglu_f16_kernel, dim3(grid_for(n4)), dim3(256), 0, stream, gate, up, out, n4);
        done = n4 * 4;
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
    hipLaunchKernelGGL(geglu_offset_kernel, dim3(grid_for(n)), dim3(256), 0, stream, gate, ple, out, ple_offset,
                       ple_row_stride, width, rows);
    return hipGetLastError();
}

}  // namespace atlas
