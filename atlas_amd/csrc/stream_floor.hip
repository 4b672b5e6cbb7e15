// stream_floor.hip -- measurement-only streaming kernels for bench.py.
//
// Not part of the operator library (built into libatlas_stream_floor.so,
// loaded only by the benchmark).  For each op the benchmark times, it
// launches kernels that read the op's input bytes and write its output bytes
// as plain contiguous streams, and takes the fastest: its time is what the
// launch path and the memory system give for that many bytes at that size,
// with no arithmetic, no reduction and no gather -- the size-matched floor
// the op's own time is compared against.
//
// Three shapes, the fastest of a sweep over cache policies (plain, nt, sc0,
// sc1 and their combinations on loads and stores) and grid shapes on MI355X:
//   kind 0: one float4 per thread, one thread per float4 of the longer
//           stream, nontemporal loads and stores;
//   kind 1: a grid of 4096 workgroups of 256 threads striding over the
//           streams, nontemporal loads, stores with the sc1 + nt policy
//           (fastest where reads and writes are balanced: 25 + 25 MB in
//           9.06 us against 9.75 for kind 0 on one box);
//   kind 2: kind 0's shape with plain loads and nontemporal stores (fastest
//           for write-dominated streams such as a token gather's).
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
// buffer-instruction cache-policy bits on gfx950: sc0 = 1, nt = 2, sc1 = 16
constexpr int kPolicyPlain = 0;
constexpr int kPolicyNt = 2;
constexpr int kPolicySc1Nt = 18;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// Thread i handles float4 j = i, i + stride, ... of both streams: it loads
// in[j] (j < in4; past the end the buffer load returns 0) and stores it to
// out[j] (j < out4).  Loads past the output's end feed a store under a
// data-dependent guard that never holds for the benchmark's zero-filled
// buffers, so the compiler keeps every load.
template <int LOAD, int STORE>
__global__ __launch_bounds__(kThreads) void stream_floor_kernel(const void* __restrict__ in, uint32_t in4,
                                                                void* __restrict__ out, uint32_t out4,
                                                                uint32_t* __restrict__ sink) {
    const auto ri = rsrc(in, in4 * 16u), ro = rsrc(out, out4 * 16u);
    const uint32_t n4 = in4 > out4 ? in4 : out4;
    const uint32_t stride = gridDim.x * kThreads;
    for (uint32_t j = blockIdx.x * kThreads + threadIdx.x; j < n4; j += stride) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(ri, j * 16u, 0, LOAD);
        if (j < out4)
            __builtin_amdgcn_raw_buffer_store_b128(v, ro, j * 16u, 0, STORE);
        else if (v.x == 0x7fc00001u)
            sink[0] = v.y;
    }
}

// The token gather's dependency chain with no decode: one wavefront per
// token (four per workgroup) reads the token's id (scalar load), then the
// table row it names (16 bytes per lane, lanes past the row re-read it
// modulo its length), then writes out_row4 float4 of the output row, each a
// copy of the lane's loaded chunk -- the id round trip, the row round trip
// and the output stream a quantized gather cannot avoid.
__global__ __launch_bounds__(256) void gather_floor_kernel(const void* __restrict__ table, uint32_t table_bytes,
                                                           uint32_t row_bytes, const uint32_t* __restrict__ ids,
                                                           uint32_t tokens, uint32_t vocab, void* __restrict__ out,
                                                           uint32_t out_row4) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t t = blockIdx.x * 4u + static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
    if (t >= tokens) return;
    const uint32_t id = ids[t];
    if (id >= vocab) return;
    const uint32_t chunks = (row_bytes + 15u) / 16u;
    const auto rt = rsrc(table, table_bytes);
    const uint32_t base = id * row_bytes;
    u32x4 v[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
        v[k] = __builtin_amdgcn_raw_buffer_load_b128(rt, base + 16u * ((lane + 64u * k) % chunks), 0, kPolicyPlain);
    const auto ro = rsrc(static_cast<uint8_t*>(out) + static_cast<size_t>(t) * out_row4 * 16u, out_row4 * 16u);
    for (uint32_t c = lane; c < out_row4; c += 64u)
        __builtin_amdgcn_raw_buffer_store_b128(v[(c >> 6) & 1u], ro, 16u * c, 0, kPolicyNt);
}

// Launch cost alone: one-wavefront workgroups that touch no memory (the
// guard never holds: blockDim.x is 64).
__global__ __launch_bounds__(64) void launch_floor_kernel(float* __restrict__ sink) {
    if (threadIdx.x == 1000u) sink[0] = 1.0f;
}

}  // namespace

extern "C" {

// Enqueue one launch of `blocks` empty one-wavefront workgroups on `stream`.
int atlas_floor_launch(void* stream, uint32_t blocks, float* sink) {
    if (blocks == 0) return 0;
    hipLaunchKernelGGL(launch_floor_kernel, dim3(blocks), dim3(64), 0, static_cast<hipStream_t>(stream), sink);
    return static_cast<int>(hipGetLastError());
}

// Number of streaming shapes atlas_floor_stream_kind accepts (0 .. n-1).
int atlas_floor_kinds(void) { return 3; }

// Enqueue one streaming launch of shape `kind` on `stream` (a hipStream_t;
// NULL = the default stream).  in_bytes / out_bytes are rounded down to whole
// float4 and must each be below 4 GiB; `sink` is a device word.  Returns 0
// or the HIP error code.
int atlas_floor_stream_kind(void* stream, const void* in, size_t in_bytes, void* out, size_t out_bytes,
                            uint32_t* sink, int kind) {
    if (kind < 0 || kind > 2 || in_bytes >= (1ull << 32) || out_bytes >= (1ull << 32))
        return static_cast<int>(hipErrorInvalidValue);
    const uint32_t in4 = static_cast<uint32_t>(in_bytes / 16), out4 = static_cast<uint32_t>(out_bytes / 16);
    const uint32_t n4 = in4 > out4 ? in4 : out4;
    if (n4 == 0) return 0;
    const uint32_t full = (n4 + kThreads - 1) / kThreads;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (kind == 0)
        hipLaunchKernelGGL((stream_floor_kernel<kPolicyNt, kPolicyNt>), dim3(full), dim3(kThreads), 0, s, in, in4,
                           out, out4, sink);
    else if (kind == 1)
        hipLaunchKernelGGL((stream_floor_kernel<kPolicyNt, kPolicySc1Nt>), dim3(full < 4096u ? full : 4096u),
                           dim3(kThreads), 0, s, in, in4, out, out4, sink);
    else
        hipLaunchKernelGGL((stream_floor_kernel<kPolicyPlain, kPolicyNt>), dim3(full), dim3(kThreads), 0, s, in, in4,
                           out, out4, sink);
    return static_cast<int>(hipGetLastError());
}

// Enqueue one gather floor launch: `tokens` ids into a table of `vocab` rows
// of `row_bytes` (<= 2048), writing out_row_bytes (a multiple of 16) per
// token.  The table must hold vocab * row_bytes < 4 GiB.
int atlas_floor_gather(void* stream, const void* table, uint32_t row_bytes, uint32_t vocab, const uint32_t* ids,
                       uint32_t tokens, void* out, uint32_t out_row_bytes) {
    const uint64_t table_bytes = static_cast<uint64_t>(vocab) * row_bytes;
    if (row_bytes == 0 || row_bytes > 2048 || out_row_bytes % 16 != 0 || table_bytes >= (1ull << 32))
        return static_cast<int>(hipErrorInvalidValue);
    if (tokens == 0) return 0;
    hipLaunchKernelGGL(gather_floor_kernel, dim3((tokens + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream),
                       table, static_cast<uint32_t>(table_bytes), row_bytes, ids, tokens, vocab, out,
                       out_row_bytes / 16);
    return static_cast<int>(hipGetLastError());
}

// The cache-policy sweep behind the three shapes above: the same kernel
// with load policy `lp` and store policy `sp` (indices into kPolicies:
// plain, nt, sc1, sc1+nt, sc0+sc1+nt) over `grid` workgroups of 256 threads
// (0: one thread per float4 of the longer stream).
int atlas_floor_policy_count(void) { return 5; }

int atlas_floor_stream_policy(void* stream, const void* in, size_t in_bytes, void* out, size_t out_bytes,
                              uint32_t* sink, int lp, int sp, uint32_t grid) {
    if (lp < 0 || lp > 4 || sp < 0 || sp > 4 || in_bytes >= (1ull << 32) || out_bytes >= (1ull << 32))
        return static_cast<int>(hipErrorInvalidValue);
    const uint32_t in4 = static_cast<uint32_t>(in_bytes / 16), out4 = static_cast<uint32_t>(out_bytes / 16);
    const uint32_t n4 = in4 > out4 ? in4 : out4;
    if (n4 == 0) return 0;
    const uint32_t full = (n4 + kThreads - 1) / kThreads;
    const dim3 g(grid == 0 || grid > full ? full : grid);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // kPolicies: 0 plain, 2 nt, 16 sc1, 18 sc1+nt, 19 sc0+sc1+nt
#define ATLAS_FLOOR_SP(LP, SPV)                                                                               \
    hipLaunchKernelGGL((stream_floor_kernel<LP, SPV>), g, dim3(kThreads), 0, s, in, in4, out, out4, sink); \
    break;
#define ATLAS_FLOOR_LP(LP)                  \
    switch (sp) {                           \
        case 0: ATLAS_FLOOR_SP(LP, 0)       \
        case 1: ATLAS_FLOOR_SP(LP, 2)       \
        case 2: ATLAS_FLOOR_SP(LP, 16)      \
        case 3: ATLAS_FLOOR_SP(LP, 18)      \
        default: ATLAS_FLOOR_SP(LP, 19)     \
    }                                       \
    break;
    switch (lp) {
        case 0: ATLAS_FLOOR_LP(0)
        case 1: ATLAS_FLOOR_LP(2)
        case 2: ATLAS_FLOOR_LP(16)
        case 3: ATLAS_FLOOR_LP(18)
        default: ATLAS_FLOOR_LP(19)
    }
#undef ATLAS_FLOOR_LP
#undef ATLAS_FLOOR_SP
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
