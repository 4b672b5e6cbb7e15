// logits_kernels.hip -- the decode tail of the Gemma executor: the final
// logit soft cap and the greedy argmax.
//
// Reference semantics (bisegni/atlas):
//   softcap_f32  crates/atlas-metal/src/kernels.metal:931-934
//                (v = cap * tanh(v / cap), in place; CPU form
//                gemma4_softcap_logits, crates/atlas-model/src/lib.rs:223-232)
//   argmax_f32   kernels.metal:2033-2066 (one 256-thread threadgroup: each
//                lane scans its stride with `value >= best`, then a tree keeps
//                the larger value or, on equal values, the larger index)
//   callers      gemma4_executor.rs:3673-3683 (prefill), :4678-4688 (decode)
//
// MI355X design.  The vocabulary row (262144 logits = 1 MiB) is split over
// many workgroups instead of one: each thread loads its float4s up front
// (nontemporal, every byte is touched once), caps them, stores them, and
// folds a 64-bit key per value,
//     key = (order(v) << 32) | index,
// where order() maps binary32 to an unsigned order (+0 and -0 share one
// code, NaN maps to 0 and so never wins).  The maximum key is the largest
// value and, among equal values, the largest index: exactly the reference's
// result, independent of how the row is split.  Keys reduce through the
// wavefront (shuffles) and the workgroup (LDS).  A row with one workgroup
// writes its index directly; otherwise every workgroup stores its key into
// its own slot of the context's workspace (plain stores, no atomics: many
// workgroups meeting on one word serialise at the memory-side atomic unit)
// and a second launch, one wavefront per row, reduces the row's slots.  The
// slots are overwritten by every launch, so the workspace needs no clearing.
#include "device_common.hpp"
#include "launch.hpp"

namespace atlas {
namespace {

constexpr int kLogitThreads = 256;

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t index) {
    uint32_t b = __float_as_uint(v);
    b = v == 0.0f ? 0u : b;  // -0 == +0 under the reference's comparisons
    const uint32_t ordered = (b & 0x80000000u) ? ~b : (b | 0x80000000u);  // -inf -> 0x007fffff
    const uint64_t key = (static_cast<uint64_t>(ordered) << 32) | index;
    return v != v ? 0ull : key;  // NaN never compares >= and is never taken
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// cap * tanh(v / cap) for the values of one lane.  The series range is
// evaluated for every value; the exponential range only when some lane of
// the wavefront needs it (a wave-uniform branch), then selected per value.
template <int N>
__device__ __forceinline__ void softcap_lanes(float (&v)[N], float cap) {
    float t[N], a[N], r[N];
    bool need_exp = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        t[i] = fdiv_rn(v[i], cap);
        a[i] = __builtin_fabsf(t[i]);
        need_exp = need_exp || !tanh_series_range(a[i]);
        r[i] = tanh_series_abs(a[i]);
    }
    if (__builtin_amdgcn_ballot_w64(need_exp) != 0) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const float big = tanh_exp_abs(a[i]);
            r[i] = tanh_series_range(a[i]) ? r[i] : big;
        }
    }
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = cap * __builtin_copysignf(r[i], t[i]);
}

// Reduce a workgroup's key and publish it: the row's index when the row has
// one workgroup, otherwise the workgroup's slot of the workspace.
__device__ __forceinline__ void publish_key(uint64_t key, uint32_t row, uint64_t* slots, uint32_t* selected) {
    __shared__ uint64_t wave_keys[kLogitThreads / kWave];
    for (int off = kWave / 2; off > 0; off >>= 1) key = max_u64(key, __shfl_xor(key, off, kWave));
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t wave = threadIdx.x / kWave;
    if (lane == 0) wave_keys[wave] = key;
    __syncthreads();
    if (threadIdx.x != 0) return;
    key = wave_keys[0];
#pragma unroll
    for (int w = 1; w < kLogitThreads / kWave; ++w) key = max_u64(key, wave_keys[w]);
    if (gridDim.x == 1)
        selected[row] = static_cast<uint32_t>(key);
    else
        slots[static_cast<uint64_t>(row) * gridDim.x + blockIdx.x] = key;
}

// One wavefront per row: the maximum of the row's `per_row` slot keys.
__global__ __launch_bounds__(kLogitThreads) void argmax_finish_kernel(const uint64_t* slots, uint32_t per_row,
                                                                      uint32_t rows, uint32_t* selected) {
    const uint32_t row = blockIdx.x * (kLogitThreads / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;  // whole wavefronts leave together
    const uint32_t lane = threadIdx.x % kWave;
    uint64_t key = 0;
    for (uint32_t i = lane; i < per_row; i += kWave) key = max_u64(key, slots[static_cast<uint64_t>(row) * per_row + i]);
    for (int off = kWave / 2; off > 0; off >>= 1) key = max_u64(key, __shfl_xor(key, off, kWave));
    if (lane == 0) selected[row] = static_cast<uint32_t>(key);
}

// Rows of `count` logits; blockIdx.y = row, blockIdx.x = slice of
// `per_block` values (a multiple of 1024 * U), walked in steps of 1024 * U.
// Vector form: count % 4 == 0 and 16-byte aligned rows; every load of a
// step is issued before its first value is processed.
template <bool CAP, bool ARG, int U>
__global__ __launch_bounds__(kLogitThreads) void logits_vec_kernel(const float* in, float* out, uint32_t count,
                                                                   uint32_t per_block, float cap, uint64_t* slots,
                                                                   uint32_t* selected) {
    const uint32_t row = blockIdx.y;
    const uint64_t base = static_cast<uint64_t>(row) * count;
    const uint32_t first = blockIdx.x * per_block;
    const uint32_t last = count - first < per_block ? count : first + per_block;
    uint64_t key = 0;
    for (uint32_t begin = first; begin < last; begin += kLogitThreads * 4 * U) {
        f32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t i = begin + (u * kLogitThreads + threadIdx.x) * 4;
            const uint32_t ic = i < last ? i : last - 4;  // in-bounds duplicate for the idle tail
            v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(in + base + ic));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t i = begin + (u * kLogitThreads + threadIdx.x) * 4;
            float x[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            if (CAP) softcap_lanes(x, cap);
            if (i < last) {
                if (CAP && out)
                    __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f32x4*>(out + base + i));
                if (ARG) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) key = max_u64(key, argmax_key(x[j], i + j));
                }
            }
        }
    }
    if (ARG) publish_key(key, row, slots, selected);
}

// Any width or alignment: one value per thread per step.
template <bool CAP, bool ARG>
__global__ __launch_bounds__(kLogitThreads) void logits_scalar_kernel(const float* in, float* out, uint32_t count,
                                                                      uint32_t per_block, float cap, uint64_t* slots,
                                                                      uint32_t* selected) {
    const uint32_t row = blockIdx.y;
    const uint64_t base = static_cast<uint64_t>(row) * count;
    const uint32_t begin = blockIdx.x * per_block;
    const uint32_t end = count - begin < per_block ? count : begin + per_block;
    uint64_t key = 0;
    for (uint32_t i = begin + threadIdx.x; i < end; i += kLogitThreads) {
        float x[1] = {in[base + i]};
        if (CAP) softcap_lanes(x, cap);
        if (CAP && out) out[base + i] = x[0];
        if (ARG) key = max_u64(key, argmax_key(x[0], i));
    }
    if (ARG) publish_key(key, row, slots, selected);
}

// The grid of a soft cap / argmax over rows x count values: `blocks`
// workgroups per row, each covering `per_block` values.
struct RowSplit {
    bool vec, wide;
    uint32_t blocks, per_block;
};

RowSplit row_split(const float* in, const float* out, uint32_t rows, uint32_t count) {
    RowSplit r;
    r.vec = count % 4 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 &&
            (!out || (reinterpret_cast<uintptr_t>(out) & 15) == 0);
    // large batches: steps of 4096 values; a single row: 1024, for more
    // workgroups in flight.  At most kArgmaxSlotsPerRow workgroups per row:
    // longer rows give each workgroup several steps.
    r.wide = static_cast<uint64_t>(rows) * count >= (1u << 22);
    const uint32_t step = r.vec && r.wide ? 4096u : 1024u;
    r.blocks = (count + step - 1) / step;
    r.per_block = step;
    if (r.blocks > kArgmaxSlotsPerRow) {
        r.per_block = ((count + kArgmaxSlotsPerRow - 1) / kArgmaxSlotsPerRow + step - 1) / step * step;
        r.blocks = (count + r.per_block - 1) / r.per_block;
    }
    return r;
}

// Rows one launch can cover with `slot_count` workspace slots (a row split
// over one workgroup writes its result directly and needs none).
uint32_t row_launch_rows(uint32_t blocks, uint32_t slot_count) {
    return blocks == 1 ? 65535u : slot_count / blocks;
}

template <bool CAP, bool ARG>
hipError_t launch_rows(hipStream_t stream, const float* in, float* out, uint32_t* selected, uint32_t rows,
                       uint32_t count, float cap, uint64_t* slots, uint32_t slot_count) {
    const RowSplit split = row_split(in, out, rows, count);
    const bool vec = split.vec, wide = split.wide;
    const uint32_t blocks = split.blocks, per_block = split.per_block;
    const uint32_t rows_per_launch = row_launch_rows(blocks, slot_count);
    for (uint32_t r0 = 0; r0 < rows; r0 += rows_per_launch) {
        const uint32_t n = rows - r0 < rows_per_launch ? rows - r0 : rows_per_launch;
        const dim3 grid(blocks, n);
        const float* rin = in + static_cast<uint64_t>(r0) * count;
        float* rout = out ? out + static_cast<uint64_t>(r0) * count : nullptr;
        uint32_t* rsel = ARG ? selected + r0 : nullptr;
        if (vec && wide)
            hipLaunchKernelGGL((logits_vec_kernel<CAP, ARG, 4>), grid, dim3(kLogitThreads), 0, stream, rin, rout,
                               count, per_block, cap, slots, rsel);
        else if (vec)
            hipLaunchKernelGGL((logits_vec_kernel<CAP, ARG, 1>), grid, dim3(kLogitThreads), 0, stream, rin, rout,
                               count, per_block, cap, slots, rsel);
        else
            hipLaunchKernelGGL((logits_scalar_kernel<CAP, ARG>), grid, dim3(kLogitThreads), 0, stream, rin, rout,
                               count, per_block, cap, slots, rsel);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (ARG && blocks > 1) {
            const uint32_t waves = kLogitThreads / kWave;
            hipLaunchKernelGGL(argmax_finish_kernel, dim3((n + waves - 1) / waves), dim3(kLogitThreads), 0, stream,
                               slots, blocks, n, rsel);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// Soft cap of a flat array: grid-stride float4 body plus a scalar tail.
__global__ __launch_bounds__(kLogitThreads) void softcap_vec_kernel(const float* in, float* out, uint64_t n4,
                                                                    float cap) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(in) + i);
        float x[4] = {v.x, v.y, v.z, v.w};
        softcap_lanes(x, cap);
        __builtin_nontemporal_store(f32x4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f32x4*>(out) + i);
    }
}

__global__ __launch_bounds__(kLogitThreads) void softcap_scalar_kernel(const float* in, float* out, uint64_t begin,
                                                                       uint64_t n, float cap) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = begin + static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        float x[1] = {in[i]};
        softcap_lanes(x, cap);
        out[i] = x[0];
    }
}

uint32_t grid_for(uint64_t items) {
    const uint64_t blocks = (items + kLogitThreads - 1) / kLogitThreads;
    return static_cast<uint32_t>(blocks < 8192 ? (blocks ? blocks : 1) : 8192);
}

}  // namespace

size_t argmax_workspace_bytes() { return kArgmaxSlots * sizeof(uint64_t); }

hipError_t launch_logits_f32(hipStream_t stream, const float* logits, float* capped, uint32_t* selected,
                             uint32_t rows, uint32_t count, float cap, void* workspace, uint32_t slot_count) {
    uint64_t* slots = static_cast<uint64_t*>(workspace);
    const bool do_cap = cap > 0.0f;
    if (do_cap && selected)
        return launch_rows<true, true>(stream, logits, capped, selected, rows, count, cap, slots, slot_count);
    if (selected)
        return launch_rows<false, true>(stream, logits, nullptr, selected, rows, count, cap, slots, slot_count);
    return launch_rows<true, false>(stream, logits, capped, nullptr, rows, count, cap, slots, slot_count);
}

uint32_t logits_launches(const float* logits, const float* capped, uint32_t rows, uint32_t count,
                         uint32_t slot_count) {
    const RowSplit split = row_split(logits, capped, rows, count);
    const uint32_t per = row_launch_rows(split.blocks, slot_count);
    return per == 0 ? 0u : (rows + per - 1) / per;
}

uint32_t logits_row_blocks(const float* logits, const float* capped, uint32_t rows, uint32_t count) {
    return row_split(logits, capped, rows, count).blocks;
}

// ---------------------------------------------------------------------------
// Scratch of the no-allocation soft cap + argmax entry point: a file-scope
// device array, one per GPU for the life of the process.  Host code never
// passes the symbol itself to a kernel (on the host it is only a stand-in);
// argmax_scratch_address resolves this device's copy once, with the device
// current, and callers pass that address.  Every slot a call reads is
// written by the same call first, so the array needs no clearing; calls
// that overlap on one GPU share it and race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint64_t scratch[kArgmaxScratchSlots];

hipError_t argmax_scratch_address(void** ptr) {
    return hipGetSymbolAddress(ptr, HIP_SYMBOL(scratch));
}

hipError_t launch_softcap_f32(hipStream_t stream, const float* in, float* out, uint64_t n, float cap) {
    const bool vec = (reinterpret_cast<uintptr_t>(in) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    const uint64_t n4 = vec ? n / 4 : 0;
    if (n4) {
        hipLaunchKernelGGL(softcap_vec_kernel, dim3(grid_for(n4)), dim3(kLogitThreads), 0, stream, in, out, n4, cap);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (n4 * 4 < n) {
        hipLaunchKernelGGL(softcap_scalar_kernel, dim3(grid_for(n - n4 * 4)), dim3(kLogitThreads), 0, stream, in, out,
                           n4 * 4, n, cap);
        return hipGetLastError();
    }
    return hipSuccess;
}

}  // namespace atlas
