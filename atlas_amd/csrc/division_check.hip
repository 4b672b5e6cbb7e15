// division_check.hip -- test-only enumeration of the activations' in-range
// division (device_common.hpp, div_inrange).
//
// Not part of the operator library (built into libatlas_division_check.so,
// loaded only by the GPU tests).  div_inrange replaces fdiv_rn in the
// straight-line forms of GELU and SiLU; it is not correctly rounded for every
// operand pair, so its use rests on this check: each kernel below evaluates a
// product helper with the IEEE division and with div_inrange on EVERY binary32
// input of the domain that the product sends to the in-range form, and counts
// the inputs whose bits differ.  v_rcp_f32 is a deterministic function of its
// operand, so a zero count over the whole domain is a proof for that domain.
// Two planted mistakes run beside it and must be seen: the uncorrected
// product a * rcp(b), and the corrected form without its sign step.
//
// Domains (the in-range branch conditions of device_common.hpp):
//   0  tanh_with:        every finite v (gelu_lanes' branch passes only finite
//                        arguments; |v| >= 10 selects +-1 after the quotient)
//   1  gelu_finite_with: every x whose GELU argument is finite
//   2  silu_small_with:  every x with |x| < 87 (silu_lanes' branch)
#include "device_common.hpp"

#include <stdint.h>

namespace atlas {
namespace {

struct DivProduct {  // planted mistake 1: no correction step
    __device__ static float div(float a, float b) { return a * __builtin_amdgcn_rcpf(b); }
};
struct DivNoSign {  // planted mistake 2: no sign step
    __device__ static float div(float a, float b) {
        const float r = __builtin_amdgcn_rcpf(b);
        const float q0 = a * r;
        return __builtin_fmaf(__builtin_fmaf(-q0, b, a), r, q0);
    }
};

template <int DOMAIN, class D>
__device__ __forceinline__ float eval(float x) {
    if (DOMAIN == 0) return tanh_with<D>(x);
    if (DOMAIN == 1) return gelu_finite_with<D>(x, gelu_argument(x));
    return silu_small_with<D>(x);
}

template <int DOMAIN>
__device__ __forceinline__ bool in_domain(float x) {
    if (DOMAIN == 0) return __builtin_fabsf(x) < __builtin_inff();
    if (DOMAIN == 1) return __builtin_fabsf(gelu_argument(x)) < __builtin_inff();
    return __builtin_fabsf(x) < 87.0f;
}

// counts[0] inputs in the domain, [1] in-range mismatches, [2] and [3] the
// planted mistakes' mismatches.  Every thread walks bit patterns
// i, i + stride, ... below 2^32 and adds its four counts once at the end.
template <int DOMAIN>
__global__ __launch_bounds__(256) void enumerate_kernel(unsigned long long* counts) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    uint32_t n = 0, bad = 0, bad_product = 0, bad_sign = 0;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < (1ull << 32); i += stride) {
        const float x = __uint_as_float(static_cast<uint32_t>(i));
        if (!in_domain<DOMAIN>(x)) continue;
        const uint32_t ref = __float_as_uint(eval<DOMAIN, DivIeee>(x));
        ++n;
        bad += __float_as_uint(eval<DOMAIN, DivInRange>(x)) != ref;
        bad_product += __float_as_uint(eval<DOMAIN, DivProduct>(x)) != ref;
        bad_sign += __float_as_uint(eval<DOMAIN, DivNoSign>(x)) != ref;
    }
    atomicAdd(counts + 0, static_cast<unsigned long long>(n));
    atomicAdd(counts + 1, static_cast<unsigned long long>(bad));
    atomicAdd(counts + 2, static_cast<unsigned long long>(bad_product));
    atomicAdd(counts + 3, static_cast<unsigned long long>(bad_sign));
}

}  // namespace
}  // namespace atlas

// Runs the enumeration of `domain` (0 tanh, 1 GELU, 2 SiLU) on the current
// device and writes the four counts to host memory.  Returns 0, -1 for an
// unknown domain, or the HIP error code.
extern "C" int atlas_division_check(int domain, uint64_t* counts) {
    if (domain < 0 || domain > 2 || counts == nullptr) return -1;
    unsigned long long* d = nullptr;
    hipError_t e = hipMalloc(&d, 4 * sizeof(unsigned long long));
    if (e != hipSuccess) return static_cast<int>(e);
    e = hipMemset(d, 0, 4 * sizeof(unsigned long long));
    if (e == hipSuccess) {
        const dim3 grid(16384), block(256);
        if (domain == 0) hipLaunchKernelGGL(atlas::enumerate_kernel<0>, grid, block, 0, 0, d);
        if (domain == 1) hipLaunchKernelGGL(atlas::enumerate_kernel<1>, grid, block, 0, 0, d);
        if (domain == 2) hipLaunchKernelGGL(atlas::enumerate_kernel<2>, grid, block, 0, 0, d);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(counts, d, 4 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    const hipError_t f = hipFree(d);
    if (e == hipSuccess) e = f;
    return static_cast<int>(e);
}
