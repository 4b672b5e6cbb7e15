// capi.hip -- the C ABI of libatlas_hip_ops.so (declared in
// include/atlas_hip_ops.h): context/stream management, argument validation
// with the reference's InvalidInput predicates, the device-pointer ops, and
// the host-slice operator API that mirrors atlas_ops::NeuralOps
// (crates/atlas-ops/src/lib.rs:20-147) over MetalRuntime's wrappers
// (crates/atlas-metal/src/lib.rs:1323-1733, 1897-1926).
#include "../../include/atlas_hip_ops.h"
#include "launch.hpp"

#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>
#include <string>
#include <vector>

struct atlas_hip_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    int reduction = ATLAS_REDUCTION_AUTO;
    bool capturing = false;
    // argmax workspace (per-workgroup partial keys of the rows being
    // reduced): allocated once here, never inside an op
    void* argmax_ws = nullptr;
    // this device's copy of the library's static argmax scratch (the
    // no-allocation soft cap + argmax entry point); resolved at init
    void* argmax_scratch = nullptr;
    std::string last_error;
    atlas_hip_telemetry tel{};
};

namespace {

int fail(atlas_hip_ctx* ctx, int code, const char* fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->last_error = buf;
    }
    return code;
}

int invalid(atlas_hip_ctx* ctx, const char* what) {
    return fail(ctx, ATLAS_ERR_INVALID_INPUT, "invalid buffer/input: %s", what);
}

int hip_fail(atlas_hip_ctx* ctx, hipError_t e, const char* where) {
    const int code = e == hipErrorOutOfMemory ? ATLAS_ERR_OUT_OF_MEMORY : ATLAS_ERR_COMMAND_FAILED;
    return fail(ctx, code, "%s: %s", where, hipGetErrorString(e));
}

// Make ctx->device current (one context per host thread).
int enter(atlas_hip_ctx* ctx) {
    if (!ctx) return ATLAS_ERR_INVALID_INPUT;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != ctx->device) {
        hipError_t e = hipSetDevice(ctx->device);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipSetDevice");
    }
    return ATLAS_OK;
}

int launched(atlas_hip_ctx* ctx, hipError_t e, const char* op) {
    if (e != hipSuccess) return hip_fail(ctx, e, op);
    ctx->tel.dispatches += 1;
    return ATLAS_OK;
}

bool finite_positive(float eps) { return std::isfinite(eps) && eps > 0.0f; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool fits_u32(uint64_t v) { return v <= std::numeric_limits<uint32_t>::max(); }

atlas::Reduction red(const atlas_hip_ctx* ctx) {
    switch (ctx->reduction) {
        case ATLAS_REDUCTION_WIDE: return atlas::kWide;
        case ATLAS_REDUCTION_AUTO: return atlas::kAuto;
        default: return atlas::kSequential;
    }
}

int check_norm(atlas_hip_ctx* ctx, const void* a, const void* b, const void* c, uint32_t rows,
               uint32_t hidden, float eps) {
    if (!a || !b || !c) return invalid(ctx, "RMSNorm buffer is null");
    if (rows == 0 || hidden == 0 || !finite_positive(eps))
        return invalid(ctx, "RMSNorm dimensions or epsilon are invalid");
    return ATLAS_OK;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------

int atlas_hip_device_count(int* count) {
    if (!count) return ATLAS_ERR_INVALID_INPUT;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return ATLAS_OK;
}

namespace {

// The static scratch's address on each device, resolved once per device (with
// that device current) and kept for the life of the process.
hipError_t scratch_address(int device, void** ptr) {
    static std::mutex m;
    static std::vector<void*> addr;
    std::lock_guard<std::mutex> lock(m);
    if (addr.size() <= static_cast<size_t>(device)) addr.resize(device + 1, nullptr);
    if (!addr[device]) {
        void* p = nullptr;
        const hipError_t e = atlas::argmax_scratch_address(&p);
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        addr[device] = p;
    }
    *ptr = addr[device];
    return hipSuccess;
}

}  // namespace

int atlas_hip_init(int device, atlas_hip_ctx** out) {
    if (!out) return ATLAS_ERR_INVALID_INPUT;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return ATLAS_ERR_NO_DEVICE;
    if (device < 0 || device >= n) return ATLAS_ERR_NO_DEVICE;
    if (hipSetDevice(device) != hipSuccess) return ATLAS_ERR_NO_DEVICE;
    auto* ctx = new atlas_hip_ctx;
    ctx->device = device;
    hipError_t e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return ATLAS_ERR_COMMAND_FAILED;
    }
    ctx->stream = ctx->own_stream;
    e = hipMalloc(&ctx->argmax_ws, atlas::argmax_workspace_bytes());
    if (e != hipSuccess) {
        if (ctx->argmax_ws) (void)hipFree(ctx->argmax_ws);
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return e == hipErrorOutOfMemory ? ATLAS_ERR_OUT_OF_MEMORY : ATLAS_ERR_COMMAND_FAILED;
    }
    e = scratch_address(device, &ctx->argmax_scratch);
    if (e != hipSuccess) {
        (void)hipFree(ctx->argmax_ws);
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return ATLAS_ERR_COMMAND_FAILED;
    }
    *out = ctx;
    return ATLAS_OK;
}

void atlas_hip_destroy(atlas_hip_ctx* ctx) {
    if (!ctx) return;
    if (enter(ctx) == ATLAS_OK && ctx->own_stream) {
        (void)hipStreamSynchronize(ctx->own_stream);
        (void)hipStreamDestroy(ctx->own_stream);
    }
    if (ctx->argmax_ws && enter(ctx) == ATLAS_OK) {
        (void)hipDeviceSynchronize();  // a caller stream may still use it
        (void)hipFree(ctx->argmax_ws);
    }
    delete ctx;
}

int atlas_hip_sync(atlas_hip_ctx* ctx) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (ctx->capturing) return invalid(ctx, "not allowed while a graph capture is open");
    hipError_t e = hipStreamSynchronize(ctx->stream);
    ctx->tel.syncs += 1;
    if (e != hipSuccess) return hip_fail(ctx, e, "command failed");
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(ctx, e, "command failed");
    return ATLAS_OK;
}

int atlas_hip_set_stream(atlas_hip_ctx* ctx, void* stream) {
    if (!ctx) return ATLAS_ERR_INVALID_INPUT;
    ctx->stream = stream ? static_cast<hipStream_t>(stream) : ctx->own_stream;
    return ATLAS_OK;
}

void* atlas_hip_get_stream(atlas_hip_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int atlas_hip_set_reduction(atlas_hip_ctx* ctx, int reduction) {
    if (!ctx) return ATLAS_ERR_INVALID_INPUT;
    if (reduction != ATLAS_REDUCTION_SEQUENTIAL && reduction != ATLAS_REDUCTION_WIDE &&
        reduction != ATLAS_REDUCTION_AUTO)
        return invalid(ctx, "unknown reduction order");
    ctx->reduction = reduction;
    return ATLAS_OK;
}

const char* atlas_hip_last_error(const atlas_hip_ctx* ctx) { return ctx ? ctx->last_error.c_str() : ""; }

int atlas_hip_get_telemetry(const atlas_hip_ctx* ctx, atlas_hip_telemetry* out) {
    if (!ctx || !out) return ATLAS_ERR_INVALID_INPUT;
    *out = ctx->tel;
    return ATLAS_OK;
}

// ---------------------------------------------------------------------------
// memory / events
// ---------------------------------------------------------------------------

int atlas_hip_malloc(atlas_hip_ctx* ctx, size_t bytes, void** ptr) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (ctx->capturing) return invalid(ctx, "not allowed while a graph capture is open");
    if (!ptr) return invalid(ctx, "null output pointer");
    *ptr = nullptr;
    hipError_t e = hipMalloc(ptr, bytes ? bytes : 16);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc");
    ctx->tel.allocations += 1;
    ctx->tel.resident_bytes += bytes;
    if (ctx->tel.resident_bytes > ctx->tel.peak_resident_bytes) ctx->tel.peak_resident_bytes = ctx->tel.resident_bytes;
    return ATLAS_OK;
}

int atlas_hip_free(atlas_hip_ctx* ctx, void* ptr) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!ptr) return ATLAS_OK;
    size_t size = 0;
    void* base = nullptr;
    if (hipMemGetAddressRange(&base, &size, ptr) == hipSuccess && ctx->tel.resident_bytes >= size)
        ctx->tel.resident_bytes -= size;
    hipError_t e = hipFree(ptr);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipFree");
    return ATLAS_OK;
}

int atlas_hip_upload(atlas_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (ctx->capturing) return invalid(ctx, "not allowed while a graph capture is open");
    if (!bytes) return ATLAS_OK;
    if (!dst || !src) return invalid(ctx, "null upload pointer");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "upload");
    ctx->tel.upload_bytes += bytes;
    return ATLAS_OK;
}

int atlas_hip_download(atlas_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (ctx->capturing) return invalid(ctx, "not allowed while a graph capture is open");
    if (!bytes) return ATLAS_OK;
    if (!dst || !src) return invalid(ctx, "null download pointer");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "download");
    ctx->tel.readback_bytes += bytes;
    return ATLAS_OK;
}

int atlas_hip_memset(atlas_hip_ctx* ctx, void* dst, int value, size_t bytes) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (ctx->capturing) return invalid(ctx, "not allowed while a graph capture is open");
    if (!bytes) return ATLAS_OK;
    if (!dst) return invalid(ctx, "null memset pointer");
    hipError_t e = hipMemsetAsync(dst, value, bytes, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "memset");
    return ATLAS_OK;
}

int atlas_hip_copy_d2d(atlas_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (ctx->capturing) return invalid(ctx, "not allowed while a graph capture is open");
    if (!bytes) return ATLAS_OK;
    if (!dst || !src) return invalid(ctx, "null copy pointer");
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "copy");
    return ATLAS_OK;
}

int atlas_hip_event_create(atlas_hip_ctx* ctx, void** event) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!event) return invalid(ctx, "null event pointer");
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventCreate");
    *event = ev;
    return ATLAS_OK;
}

int atlas_hip_event_record(atlas_hip_ctx* ctx, void* event) {
    int rc = enter(ctx);
    if (rc) return rc;
    hipError_t e = hipEventRecord(static_cast<hipEvent_t>(event), ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventRecord");
    return ATLAS_OK;
}

int atlas_hip_event_elapsed_ms(atlas_hip_ctx* ctx, void* start, void* stop, float* ms) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!ms) return invalid(ctx, "null output");
    hipError_t e = hipEventSynchronize(static_cast<hipEvent_t>(stop));
    if (e == hipSuccess) e = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop));
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventElapsedTime");
    return ATLAS_OK;
}

int atlas_hip_event_destroy(atlas_hip_ctx* ctx, void* event) {
    int rc = enter(ctx);
    if (rc) return rc;
    hipError_t e = hipEventDestroy(static_cast<hipEvent_t>(event));
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventDestroy");
    return ATLAS_OK;
}

// ---------------------------------------------------------------------------
// graph capture
// ---------------------------------------------------------------------------

int atlas_hip_graph_begin(atlas_hip_ctx* ctx) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (ctx->capturing) return invalid(ctx, "a graph capture is already open on this context");
    hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamBeginCapture");
    ctx->capturing = true;
    return ATLAS_OK;
}

int atlas_hip_graph_end(atlas_hip_ctx* ctx, void** graph) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!graph) return invalid(ctx, "null graph pointer");
    *graph = nullptr;
    if (!ctx->capturing) return invalid(ctx, "no graph capture is open on this context");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphInstantiate");
    *graph = exec;
    return ATLAS_OK;
}

int atlas_hip_graph_launch(atlas_hip_ctx* ctx, void* graph) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!graph) return invalid(ctx, "null graph");
    if (ctx->capturing) return invalid(ctx, "cannot launch a graph while capturing");
    hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(graph), ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphLaunch");
    ctx->tel.dispatches += 1;
    return ATLAS_OK;
}

int atlas_hip_graph_destroy(atlas_hip_ctx* ctx, void* graph) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!graph) return ATLAS_OK;
    hipError_t e = hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph));
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGraphExecDestroy");
    return ATLAS_OK;
}

// ---------------------------------------------------------------------------
// RMSNorm family
// ---------------------------------------------------------------------------

int atlas_hip_rms_norm_f32(atlas_hip_ctx* ctx, const float* input, const float* weight, float* output,
                           uint32_t rows, uint32_t hidden, float epsilon) {
    int rc = enter(ctx);
    if (rc || (rc = check_norm(ctx, input, weight, output, rows, hidden, epsilon))) return rc;
    atlas::NormArgs a{input, weight, nullptr, nullptr, nullptr, output, nullptr, rows, hidden, epsilon};
    return launched(ctx, atlas::launch_rms_norm_f32(ctx->stream, atlas::kNormPlain, red(ctx), a), "rms_norm_f32");
}

int atlas_hip_rms_norm_residual_f32(atlas_hip_ctx* ctx, const float* input, const float* weight,
                                    const float* residual, float* normalized, float* output, uint32_t rows,
                                    uint32_t hidden, float epsilon) {
    int rc = enter(ctx);
    if (rc || (rc = check_norm(ctx, input, weight, output, rows, hidden, epsilon))) return rc;
    if (!residual) return invalid(ctx, "residual buffer is null");
    atlas::NormArgs a{input, weight, residual, normalized, nullptr, output, nullptr, rows, hidden, epsilon};
    return launched(ctx, atlas::launch_rms_norm_f32(ctx->stream, atlas::kNormResidual, red(ctx), a),
                    "rms_norm_residual_f32");
}

int atlas_hip_add_rms_norm_f32(atlas_hip_ctx* ctx, const float* input, const float* residual, const float* weight,
                               float* residual_out, float* output, uint32_t rows, uint32_t hidden, float epsilon) {
    int rc = enter(ctx);
    if (rc || (rc = check_norm(ctx, input, weight, output, rows, hidden, epsilon))) return rc;
    if (!residual || !residual_out) return invalid(ctx, "residual buffer is null");
    atlas::NormArgs a{input, weight, residual, nullptr, residual_out, output, nullptr, rows, hidden, epsilon};
    return launched(ctx, atlas::launch_rms_norm_f32(ctx->stream, atlas::kNormAddNorm, red(ctx), a),
                    "add_rms_norm_f32");
}

int atlas_hip_rms_norm_add_scale_f32(atlas_hip_ctx* ctx, const float* input, const float* weight, float* state,
                                     const float* scale, uint32_t rows, uint32_t hidden, float epsilon) {
    int rc = enter(ctx);
    if (rc || (rc = check_norm(ctx, input, weight, state, rows, hidden, epsilon))) return rc;
    if (!scale) return invalid(ctx, "scale buffer is null");
    atlas::NormArgs a{input, weight, nullptr, nullptr, nullptr, state, scale, rows, hidden, epsilon};
    return launched(ctx, atlas::launch_rms_norm_f32(ctx->stream, atlas::kNormAddScale, red(ctx), a),
                    "rms_norm_add_scale_f32");
}

int atlas_hip_rms_norm_groups_stable_f32(atlas_hip_ctx* ctx, float* values, const float* weight, uint32_t width,
                                         uint32_t groups, float epsilon) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!values || !weight) return invalid(ctx, "group norm buffer is null");
    if (width == 0 || groups == 0 || !finite_positive(epsilon) || width > 16384)
        return invalid(ctx, "group norm dimensions or epsilon are invalid");
    return launched(ctx,
                    atlas::launch_rms_norm_groups_stable_f32(ctx->stream, red(ctx), values, weight, width, groups,
                                                             epsilon),
                    "rms_norm_groups_stable_f32");
}

int atlas_hip_rms_norm_f16(atlas_hip_ctx* ctx, const uint16_t* input, const uint16_t* weight, uint16_t* output,
                           uint32_t rows, uint32_t hidden, float epsilon) {
    int rc = enter(ctx);
    if (rc || (rc = check_norm(ctx, input, weight, output, rows, hidden, epsilon))) return rc;
    if (hidden > 16384) return invalid(ctx, "FP16 RMSNorm hidden width exceeds 16384");
    return launched(ctx,
                    atlas::launch_rms_norm_f16(ctx->stream, red(ctx), input, nullptr, weight, nullptr, output, rows,
                                               hidden, epsilon),
                    "rms_norm_f16");
}

int atlas_hip_add_rms_norm_f16(atlas_hip_ctx* ctx, const uint16_t* input, const uint16_t* residual,
                               const uint16_t* weight, uint16_t* residual_out, uint16_t* output, uint32_t rows,
                               uint32_t hidden, float epsilon) {
    int rc = enter(ctx);
    if (rc || (rc = check_norm(ctx, input, weight, output, rows, hidden, epsilon))) return rc;
    if (!residual || !residual_out) return invalid(ctx, "residual buffer is null");
    if (hidden > 16384) return invalid(ctx, "FP16 RMSNorm hidden width exceeds 16384");
    return launched(ctx,
                    atlas::launch_rms_norm_f16(ctx->stream, red(ctx), input, residual, weight, residual_out, output,
                                               rows, hidden, epsilon),
                    "add_rms_norm_f16");
}

// ---------------------------------------------------------------------------
// RoPE
// ---------------------------------------------------------------------------

int atlas_hip_qk_norm_rope_f32(atlas_hip_ctx* ctx, const float* q, const float* k, const float* q_weight,
                               const float* k_weight, const float* cosine, const float* sine, float* q_out,
                               float* k_out, uint32_t tokens, uint32_t q_heads, uint32_t has_key, uint32_t head_dim,
                               uint32_t rope_stride, float epsilon) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (has_key > 1) return invalid(ctx, "has_key must be 0 or 1");
    if (!q_weight || !cosine || !sine || (q_heads && (!q || !q_out)) || (has_key && (!k || !k_out || !k_weight)))
        return invalid(ctx, "QK-norm RoPE buffer is null");
    if (tokens == 0 || head_dim == 0 || head_dim % 2 != 0 || q_heads + has_key == 0 || rope_stride < head_dim / 2 ||
        !finite_positive(epsilon) || head_dim > 16384)
        return invalid(ctx, "QK-norm RoPE dimensions or epsilon are invalid");
    if (!fits_u32(static_cast<uint64_t>(tokens) * (q_heads + has_key)))
        return invalid(ctx, "QK-norm RoPE unit count overflows");
    return launched(ctx,
                    atlas::launch_qk_norm_rope_f32(ctx->stream, red(ctx), q, k, q_weight, k_weight, cosine, sine,
                                                   q_out, k_out, tokens, q_heads, has_key, head_dim, rope_stride,
                                                   epsilon),
                    "qk_norm_rope_f32");
}

static int check_rope_half(atlas_hip_ctx* ctx, const void* x, const void* c, const void* s, const void* o,
                           uint32_t tokens, uint32_t heads, uint32_t head_dim, uint32_t rope_stride) {
    if (!x || !c || !s || !o) return invalid(ctx, "RoPE buffer is null");
    if (tokens == 0 || heads == 0 || head_dim == 0 || head_dim % 2 != 0 || rope_stride < head_dim / 2)
        return invalid(ctx, "RoPE hidden width must be a non-zero even number");
    return ATLAS_OK;
}

int atlas_hip_rope_half_f32(atlas_hip_ctx* ctx, const float* input, const float* cosine, const float* sine,
                            float* output, uint32_t tokens, uint32_t heads, uint32_t head_dim, uint32_t rope_stride) {
    int rc = enter(ctx);
    if (rc || (rc = check_rope_half(ctx, input, cosine, sine, output, tokens, heads, head_dim, rope_stride)))
        return rc;
    return launched(ctx,
                    atlas::launch_rope_half_f32(ctx->stream, input, cosine, sine, output, tokens, heads, head_dim,
                                                rope_stride),
                    "rope_half_f32");
}

int atlas_hip_rope_half_f16(atlas_hip_ctx* ctx, const uint16_t* input, const float* cosine, const float* sine,
                            uint16_t* output, uint32_t tokens, uint32_t heads, uint32_t head_dim,
                            uint32_t rope_stride) {
    int rc = enter(ctx);
    if (rc || (rc = check_rope_half(ctx, input, cosine, sine, output, tokens, heads, head_dim, rope_stride)))
        return rc;
    return launched(ctx,
                    atlas::launch_rope_half_f16(ctx->stream, input, cosine, sine, output, tokens, heads, head_dim,
                                                rope_stride),
                    "rope_half_f16");
}

int atlas_hip_rope_half_qk_f32(atlas_hip_ctx* ctx, const float* q, const float* k, const float* cosine,
                               const float* sine, float* q_out, float* k_out, uint32_t tokens, uint32_t q_heads,
                               uint32_t k_heads, uint32_t head_dim, uint32_t rope_stride) {
    int rc = enter(ctx);
    if (rc || (rc = check_rope_half(ctx, q, cosine, sine, q_out, tokens, q_heads, head_dim, rope_stride)) ||
        (rc = check_rope_half(ctx, k, cosine, sine, k_out, tokens, k_heads, head_dim, rope_stride)))
        return rc;
    return launched(ctx,
                    atlas::launch_rope_half_pair_f32(ctx->stream, q, q_out, q_heads, k, k_out, k_heads, cosine, sine,
                                                     tokens, head_dim, rope_stride),
                    "rope_half_qk_f32");
}

int atlas_hip_rope_half_qk_f16(atlas_hip_ctx* ctx, const uint16_t* q, const uint16_t* k, const float* cosine,
                               const float* sine, uint16_t* q_out, uint16_t* k_out, uint32_t tokens,
                               uint32_t q_heads, uint32_t k_heads, uint32_t head_dim, uint32_t rope_stride) {
    int rc = enter(ctx);
    if (rc || (rc = check_rope_half(ctx, q, cosine, sine, q_out, tokens, q_heads, head_dim, rope_stride)) ||
        (rc = check_rope_half(ctx, k, cosine, sine, k_out, tokens, k_heads, head_dim, rope_stride)))
        return rc;
    return launched(ctx,
                    atlas::launch_rope_half_pair_f16(ctx->stream, q, q_out, q_heads, k, k_out, k_heads, cosine, sine,
                                                     tokens, head_dim, rope_stride),
                    "rope_half_qk_f16");
}

int atlas_hip_rope_interleaved_f32(atlas_hip_ctx* ctx, const float* input, const float* cosine, const float* sine,
                                   float* output, uint32_t rows, uint32_t hidden) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!input || !cosine || !sine || !output) return invalid(ctx, "RoPE buffer is null");
    if (rows == 0 || hidden == 0 || hidden % 2 != 0) return invalid(ctx, "RoPE hidden width must be a non-zero even number");
    return launched(ctx, atlas::launch_rope_interleaved_f32(ctx->stream, input, cosine, sine, output, rows, hidden),
                    "rope_interleaved_f32");
}

// Host tables: gemma4_rope_angle (gemma4_executor.rs:622-633):
//   pair >= rotary/2 -> 0, else pos / theta^((2*pair)/rotary) / factor  (f32, libm powf)
int atlas_rope_tables_gemma4(const uint32_t* positions, size_t tokens, size_t rope_pairs, size_t rotary, float theta,
                             const float* frequency_factors, float* cos_out, float* sin_out) {
    if (!positions || !cos_out || !sin_out || rope_pairs == 0 || rotary == 0 || !(theta > 0.0f))
        return ATLAS_ERR_INVALID_INPUT;
    for (size_t t = 0; t < tokens; ++t) {
        for (size_t p = 0; p < rope_pairs; ++p) {
            float angle = 0.0f;
            if (p < rotary / 2) {
                const float factor = frequency_factors ? frequency_factors[p] : 1.0f;
                angle = static_cast<float>(positions[t]) /
                        powf(theta, static_cast<float>(p * 2) / static_cast<float>(rotary)) / factor;
            }
            cos_out[t * rope_pairs + p] = cosf(angle);
            sin_out[t * rope_pairs + p] = sinf(angle);
        }
    }
    return ATLAS_OK;
}

// write_rope_tables (executor.rs:632-647): angle = pos / theta^((2*pair)/head_dim).
int atlas_rope_tables_llama(const uint32_t* positions, size_t tokens, size_t head_dim, float theta, float* cos_out,
                            float* sin_out) {
    if (!positions || !cos_out || !sin_out || head_dim == 0 || head_dim % 2 != 0 || !(theta > 0.0f))
        return ATLAS_ERR_INVALID_INPUT;
    const size_t pairs = head_dim / 2;
    for (size_t t = 0; t < tokens; ++t)
        for (size_t p = 0; p < pairs; ++p) {
            const float angle = static_cast<float>(positions[t]) /
                                powf(theta, static_cast<float>(p * 2) / static_cast<float>(head_dim));
            cos_out[t * pairs + p] = cosf(angle);
            sin_out[t * pairs + p] = sinf(angle);
        }
    return ATLAS_OK;
}

// ---------------------------------------------------------------------------
// activations / elementwise
// ---------------------------------------------------------------------------

static int elt(atlas_hip_ctx* ctx, atlas::EltOp op, const float* a, const float* b, float scalar, float* out,
               uint64_t n, bool binary, const char* name) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (n == 0) return ATLAS_OK;
    if (!a || !out || (binary && !b)) return invalid(ctx, "elementwise buffer is null");
    return launched(ctx, atlas::launch_elementwise_f32(ctx->stream, op, a, b, scalar, out, n), name);
}

int atlas_hip_swiglu_f32(atlas_hip_ctx* ctx, const float* gate, const float* up, float* output, uint64_t count) {
    return elt(ctx, atlas::kEltSwiglu, gate, up, 0.0f, output, count, true, "swiglu_f32");
}

int atlas_hip_geglu_f32(atlas_hip_ctx* ctx, const float* gate, const float* up, float* output, uint64_t count) {
    return elt(ctx, atlas::kEltGeglu, gate, up, 0.0f, output, count, true, "geglu_f32");
}

int atlas_hip_silu_f32(atlas_hip_ctx* ctx, const float* input, float* output, uint64_t count) {
    return elt(ctx, atlas::kEltSilu, input, nullptr, 0.0f, output, count, false, "silu_f32");
}

int atlas_hip_gelu_f32(atlas_hip_ctx* ctx, const float* input, float* output, uint64_t count) {
    return elt(ctx, atlas::kEltGelu, input, nullptr, 0.0f, output, count, false, "gelu_f32");
}

int atlas_hip_add_f32(atlas_hip_ctx* ctx, const float* lhs, const float* rhs, float* output, uint64_t count) {
    return elt(ctx, atlas::kEltAdd, lhs, rhs, 0.0f, output, count, true, "add_f32");
}

int atlas_hip_multiply_f32(atlas_hip_ctx* ctx, const float* lhs, const float* rhs, float* output, uint64_t count) {
    return elt(ctx, atlas::kEltMul, lhs, rhs, 0.0f, output, count, true, "multiply_f32");
}

int atlas_hip_scale_f32(atlas_hip_ctx* ctx, const float* input, float scalar, float* output, uint64_t count) {
    return elt(ctx, atlas::kEltScale, input, nullptr, scalar, output, count, false, "scale_f32");
}

int atlas_hip_swiglu_f16(atlas_hip_ctx* ctx, const uint16_t* gate, const uint16_t* up, uint16_t* output,
                         uint64_t count) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (count == 0) return ATLAS_OK;
    if (!gate || !up || !output) return invalid(ctx, "SwiGLU buffer is null");
    return launched(ctx, atlas::launch_swiglu_f16(ctx->stream, gate, up, output, count), "swiglu_f16");
}

int atlas_hip_geglu_offset_f32(atlas_hip_ctx* ctx, const float* gate, const float* ple, float* output,
                               uint32_t ple_offset, uint32_t ple_row_stride, uint32_t width, uint32_t rows) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!gate || !ple || !output) return invalid(ctx, "PLE GeGLU buffer is null");
    if (width == 0 || rows == 0 || (rows > 1 && static_cast<uint64_t>(ple_offset) + width > ple_row_stride))
        return invalid(ctx, "PLE GeGLU offset or width is invalid");
    return launched(ctx,
                    atlas::launch_geglu_offset_f32(ctx->stream, gate, ple, output, ple_offset, ple_row_stride, width,
                                                   rows),
                    "geglu_offset_f32");
}

// ---------------------------------------------------------------------------
// gathers
// ---------------------------------------------------------------------------

int atlas_hip_embed_f32(atlas_hip_ctx* ctx, const float* table, const uint32_t* ids, float* output, uint32_t vocab,
                        uint32_t hidden, uint32_t tokens, float scale) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!table || !ids || !output) return invalid(ctx, "embedding buffer is null");
    if (hidden == 0 || tokens == 0) return invalid(ctx, "embedding dimensions or token IDs are invalid");
    return launched(ctx, atlas::launch_embed_f32(ctx->stream, table, ids, output, vocab, hidden, tokens, scale),
                    "embed_f32");
}

// format: 0 Q4_0, 1 Q6_K, 2 Q8_0 (atlas::launch_embed_quant)
static int embed_quant(atlas_hip_ctx* ctx, int format, const uint8_t* table, const uint32_t* ids, float* output,
                       uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale) {
    static const char* const kNames[] = {"embed_q4_0", "embed_q6_k", "embed_q8_0"};
    static const char* const kBad[] = {"Q4_0 embedding dimensions or token IDs are invalid",
                                       "Q6_K embedding dimensions or token IDs are invalid",
                                       "Q8_0 embedding dimensions or token IDs are invalid"};
    int rc = enter(ctx);
    if (rc) return rc;
    const uint32_t qk = format == 1 ? 256 : 32;
    if (!table || !ids || !output) return invalid(ctx, "quantized embedding buffer is null");
    if (hidden == 0 || hidden % qk != 0 || tokens == 0 || hidden > 65536) return invalid(ctx, kBad[format]);
    if (!aligned16(output)) return invalid(ctx, "embedding output must be 16-byte aligned");
    return launched(ctx,
                    atlas::launch_embed_quant(ctx->stream, format, table, ids, output, vocab, hidden, tokens, scale),
                    kNames[format]);
}

int atlas_hip_embed_q4_0(atlas_hip_ctx* ctx, const uint8_t* table, const uint32_t* ids, float* output,
                         uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale) {
    return embed_quant(ctx, 0, table, ids, output, vocab, hidden, tokens, scale);
}

int atlas_hip_embed_q6_k(atlas_hip_ctx* ctx, const uint8_t* table, const uint32_t* ids, float* output,
                         uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale) {
    return embed_quant(ctx, 1, table, ids, output, vocab, hidden, tokens, scale);
}

int atlas_hip_embed_q8_0(atlas_hip_ctx* ctx, const uint8_t* table, const uint32_t* ids, float* output,
                         uint32_t vocab, uint32_t hidden, uint32_t tokens, float scale) {
    return embed_quant(ctx, 2, table, ids, output, vocab, hidden, tokens, scale);
}

static int ple(atlas_hip_ctx* ctx, int q6, const uint8_t* table, const uint32_t* ids, const float* projection,
               float* output, uint32_t vocab, uint32_t layers, uint32_t width, uint32_t tokens, float es, float os) {
    int rc = enter(ctx);
    if (rc) return rc;
    const uint64_t row = static_cast<uint64_t>(layers) * width;
    const uint32_t qk = q6 ? 256 : 32;
    if (!table || !ids || !projection || !output) return invalid(ctx, "PLE buffer is null");
    if (layers == 0 || width == 0 || tokens == 0 || row % qk != 0)
        return invalid(ctx, "PLE dimensions are invalid");
    if (vocab == 0) return invalid(ctx, "PLE table has no rows (vocab is 0)");
    if (row > 16384) return invalid(ctx, "PLE rows are limited to 16384 values (layers * width)");
    if (!aligned16(projection) || !aligned16(output)) return invalid(ctx, "PLE projection/output must be 16-byte aligned");
    return launched(ctx,
                    atlas::launch_ple_quant(ctx->stream, q6, table, ids, projection, output, vocab, layers, width,
                                            tokens, es, os),
                    q6 ? "ple_q6_k" : "ple_q4_0");
}

static int q4_matvec(atlas_hip_ctx* ctx, const float* input, const float* rms_weight, float epsilon,
                     uint32_t input_width, uint32_t segments, const uint8_t* const* weights, float* const* outputs,
                     const uint32_t* widths, const char* op, const float* ple = nullptr, uint32_t ple_offset = 0) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!input) return invalid(ctx, "matvec input is null");
    if (input_width == 0 || input_width % 32 != 0 || input_width > atlas::q4_0_matvec_max_input())
        return invalid(ctx, "matvec input_width must be a positive multiple of 32, at most 4096");
    if (!aligned16(input) || (rms_weight && !aligned16(rms_weight)))
        return invalid(ctx, "matvec input and rms_weight must be 16-byte aligned");
    if (rms_weight && !finite_positive(epsilon)) return invalid(ctx, "epsilon must be finite and positive");
    atlas::MatvecArgs a{};
    a.input = input;
    a.rms_weight = rms_weight;
    a.epsilon = epsilon;
    a.input_width = input_width;
    a.segments = segments;
    a.ple = ple;
    a.ple_offset = ple_offset;
    for (uint32_t i = 0; i < segments; ++i) {
        if (!weights[i] || !outputs[i]) return invalid(ctx, "matvec weights/output is null");
        if (reinterpret_cast<uintptr_t>(weights[i]) & 1) return invalid(ctx, "Q4_0 weights must be 2-byte aligned");
        if (widths[i] == 0) return invalid(ctx, "matvec output width is zero");
        a.weights[i] = weights[i];
        a.output[i] = outputs[i];
        a.width[i] = widths[i];
    }
    return launched(ctx, atlas::launch_q4_0_matvec(ctx->stream, a), op);
}

int atlas_hip_ple_gate_gelu_f32(atlas_hip_ctx* ctx, const float* input, const uint8_t* weights, const float* ple,
                                uint32_t ple_offset, float* output, uint32_t input_width, uint32_t output_width) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!ple) return invalid(ctx, "PLE buffer is null");
    const uint8_t* w[1] = {weights};
    float* o[1] = {output};
    const uint32_t n[1] = {output_width};
    return q4_matvec(ctx, input, nullptr, 0.0f, input_width, 1, w, o, n, "ple_gate_gelu", ple, ple_offset);
}

int atlas_hip_ple_projection_f16(atlas_hip_ctx* ctx, const float* input, const uint16_t* weights,
                                 const float* norm_weight, float* output, uint32_t hidden, uint32_t width,
                                 uint32_t groups, float scale, float epsilon) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!input || !weights || !norm_weight || !output) return invalid(ctx, "PLE projection buffer is null");
    if (hidden == 0 || hidden % 8 != 0 || hidden > atlas::ple_projection_max_hidden())
        return invalid(ctx, "PLE projection hidden must be a positive multiple of 8, at most 4096");
    if (width == 0 || width % 16 != 0 || width > 1024)
        return invalid(ctx, "PLE projection width must be a positive multiple of 16, at most 1024");
    if (groups == 0 || groups > atlas::ple_projection_max_groups())
        return invalid(ctx, "PLE projection groups must be between 1 and 1024");
    if (!aligned16(input) || !aligned16(weights))
        return invalid(ctx, "PLE projection input and weights must be 16-byte aligned");
    if (!std::isfinite(scale)) return invalid(ctx, "PLE projection scale must be finite");
    if (!finite_positive(epsilon)) return invalid(ctx, "epsilon must be finite and positive");
    atlas::PleProjArgs a{input, weights, norm_weight, output, hidden, width, groups, scale, epsilon};
    return launched(ctx, atlas::launch_ple_projection_f16(ctx->stream, a), "ple_projection_f16");
}

int atlas_hip_matvec_q4_0_rms_f32(atlas_hip_ctx* ctx, const float* input, const uint8_t* weights, float* output,
                                  uint32_t input_width, uint32_t output_width, const float* rms_weight,
                                  float epsilon) {
    const uint8_t* w[1] = {weights};
    float* o[1] = {output};
    const uint32_t n[1] = {output_width};
    return q4_matvec(ctx, input, rms_weight, epsilon, input_width, 1, w, o, n, "matvec_q4_0_rms");
}

int atlas_hip_matmul_q4_0_qkv_rms_f32(atlas_hip_ctx* ctx, const float* input, const uint8_t* q_weights,
                                      const uint8_t* k_weights, const uint8_t* v_weights, float* q_output,
                                      float* k_output, float* v_output, uint32_t input_width, uint32_t q_width,
                                      uint32_t kv_width, const float* rms_weight, float epsilon) {
    const uint8_t* w[3] = {q_weights, k_weights, v_weights};
    float* o[3] = {q_output, k_output, v_output};
    const uint32_t n[3] = {q_width, kv_width, kv_width};
    return q4_matvec(ctx, input, rms_weight, epsilon, input_width, 3, w, o, n, "matmul_q4_0_qkv_rms");
}

int atlas_hip_matmul_q4_0_gate_up_rms_f32(atlas_hip_ctx* ctx, const float* input, const uint8_t* gate_weights,
                                          const uint8_t* up_weights, float* gate_output, float* up_output,
                                          uint32_t input_width, uint32_t output_width, const float* rms_weight,
                                          float epsilon) {
    const uint8_t* w[2] = {gate_weights, up_weights};
    float* o[2] = {gate_output, up_output};
    const uint32_t n[2] = {output_width, output_width};
    return q4_matvec(ctx, input, rms_weight, epsilon, input_width, 2, w, o, n, "matmul_q4_0_gate_up_rms");
}

static int kv_append(atlas_hip_ctx* ctx, int format, const float* key, const float* value, void* cache,
                     uint32_t kv_width, uint32_t capacity, const uint32_t* positions, uint32_t tokens, int vnorm,
                     float epsilon, const char* op) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!key || !value || !cache || !positions) return invalid(ctx, "KV append buffer is null");
    if (kv_width == 0 || kv_width > 4096 || capacity == 0 || tokens == 0)
        return invalid(ctx, "KV append dimensions are invalid (kv_width 1..4096, capacity and tokens > 0)");
    if (format != atlas::kKvF32 && kv_width % 32 != 0) return invalid(ctx, "quantized KV rows need kv_width % 32 == 0");
    if (vnorm && kv_width % 4 != 0) return invalid(ctx, "the V norm needs kv_width % 4 == 0");
    if (vnorm && !finite_positive(epsilon)) return invalid(ctx, "epsilon must be finite and positive");
    if ((reinterpret_cast<uintptr_t>(key) | reinterpret_cast<uintptr_t>(value)) & 3)
        return invalid(ctx, "key/value must be 4-byte aligned");
    if (format == atlas::kKvF32 && (reinterpret_cast<uintptr_t>(cache) & 3)) return invalid(ctx, "f32 cache must be 4-byte aligned");
    atlas::KvAppendArgs a{key, value, static_cast<uint8_t*>(cache), positions, kv_width, capacity, tokens, epsilon};
    return launched(ctx, atlas::launch_kv_append(ctx->stream, format, vnorm != 0, a), op);
}

int atlas_hip_kv_append_f32(atlas_hip_ctx* ctx, const float* key, const float* value, float* cache, uint32_t kv_width,
                            uint32_t capacity, const uint32_t* positions, uint32_t tokens, int vnorm, float epsilon) {
    return kv_append(ctx, atlas::kKvF32, key, value, cache, kv_width, capacity, positions, tokens, vnorm, epsilon,
                     "kv_append_f32");
}

int atlas_hip_kv_append_q8_0(atlas_hip_ctx* ctx, const float* key, const float* value, uint8_t* cache,
                             uint32_t kv_width, uint32_t capacity, const uint32_t* positions, uint32_t tokens,
                             int vnorm, float epsilon) {
    return kv_append(ctx, atlas::kKvQ8_0, key, value, cache, kv_width, capacity, positions, tokens, vnorm, epsilon,
                     "kv_append_q8_0");
}

int atlas_hip_kv_append_q4_0(atlas_hip_ctx* ctx, const float* key, const float* value, uint8_t* cache,
                             uint32_t kv_width, uint32_t capacity, const uint32_t* positions, uint32_t tokens,
                             int vnorm, float epsilon) {
    return kv_append(ctx, atlas::kKvQ4_0, key, value, cache, kv_width, capacity, positions, tokens, vnorm, epsilon,
                     "kv_append_q4_0");
}

// ---------------------------------------------------------------------------
// logits: soft cap and argmax
// ---------------------------------------------------------------------------

static bool finite_cap(float cap) { return std::isfinite(cap) && cap > 0.0f; }

int atlas_hip_softcap_f32(atlas_hip_ctx* ctx, const float* input, float* output, uint64_t count, float cap) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!input || !output) return invalid(ctx, "soft cap buffer is null");
    if (count == 0) return invalid(ctx, "soft cap needs at least one value");
    // gemma4_softcap_logits: "Gemma 4 logit soft cap must be positive"
    if (!finite_cap(cap)) return invalid(ctx, "logit soft cap must be finite and positive");
    if ((reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(output)) & 3)
        return invalid(ctx, "logits must be 4-byte aligned");
    return launched(ctx, atlas::launch_softcap_f32(ctx->stream, input, output, count, cap), "softcap_f32");
}

static int logits_rows(atlas_hip_ctx* ctx, const float* logits, float* capped, uint32_t* selected, uint32_t rows,
                       uint32_t count, float cap, const char* op) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!logits || !selected) return invalid(ctx, "argmax buffer is null");
    // argmax_for_test: "argmax requires at least one value"
    if (rows == 0 || count == 0) return invalid(ctx, "argmax requires at least one value per row");
    if ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(capped) |
         reinterpret_cast<uintptr_t>(selected)) & 3)
        return invalid(ctx, "logits and selected must be 4-byte aligned");
    return launched(ctx,
                    atlas::launch_logits_f32(ctx->stream, logits, capped, selected, rows, count, cap, ctx->argmax_ws,
                                             atlas::kArgmaxSlots),
                    op);
}

int atlas_hip_argmax_f32(atlas_hip_ctx* ctx, const float* values, uint32_t* selected, uint32_t rows, uint32_t count) {
    return logits_rows(ctx, values, nullptr, selected, rows, count, 0.0f, "argmax_f32");
}

int atlas_hip_softcap_argmax_f32(atlas_hip_ctx* ctx, const float* logits, float* capped, uint32_t* selected,
                                 uint32_t rows, uint32_t count, float cap) {
    if (ctx && !finite_cap(cap)) return invalid(ctx, "logit soft cap must be finite and positive");
    return logits_rows(ctx, logits, capped, selected, rows, count, cap, "softcap_argmax_f32");
}

// The same computation with the per-workgroup partial keys in the library's
// static scratch (this device's copy, resolved at init) instead of the
// context's workspace: no allocation of any kind, one launch pair per call.
int atlas_hip_softcap_argmax_f32_noalloc(atlas_hip_ctx* ctx, const float* logits, float* capped,
                                         uint32_t* selected, uint32_t rows, uint32_t count, float cap) {
    int rc = enter(ctx);
    if (rc) return rc;
    if (!finite_cap(cap)) return invalid(ctx, "logit soft cap must be finite and positive");
    if (!logits || !selected) return invalid(ctx, "argmax buffer is null");
    if (rows == 0 || count == 0) return invalid(ctx, "argmax requires at least one value per row");
    if ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(capped) |
         reinterpret_cast<uintptr_t>(selected)) & 3)
        return invalid(ctx, "logits and selected must be 4-byte aligned");
    if (!ctx->argmax_scratch) return invalid(ctx, "the argmax scratch was not resolved for this device");
    // rows that fit one workgroup each never touch the scratch (any row
    // count, in launches of up to 65535 rows); split rows need all their
    // partial keys in the scratch at once, in one launch pair
    if (atlas::logits_row_blocks(logits, capped, rows, count) > 1 &&
        atlas::logits_launches(logits, capped, rows, count, atlas::kArgmaxScratchSlots) != 1)
        return fail(ctx, ATLAS_ERR_INVALID_INPUT,
                    "invalid buffer/input: rows x workgroups per row exceed the no-allocation argmax scratch "
                    "(%u slots; it holds up to 256 rows of 262144 values, 64 rows of 1048576)",
                    atlas::kArgmaxScratchSlots);
    return launched(ctx,
                    atlas::launch_logits_f32(ctx->stream, logits, capped, selected, rows, count, cap,
                                             ctx->argmax_scratch, atlas::kArgmaxScratchSlots),
                    "softcap_argmax_f32_noalloc");
}

int atlas_hip_ple_q4_0(atlas_hip_ctx* ctx, const uint8_t* table, const uint32_t* ids, const float* projection,
                       float* output, uint32_t vocab, uint32_t layers, uint32_t width, uint32_t tokens,
                       float embedding_scale, float output_scale) {
    return ple(ctx, 0, table, ids, projection, output, vocab, layers, width, tokens, embedding_scale, output_scale);
}

int atlas_hip_ple_q6_k(atlas_hip_ctx* ctx, const uint8_t* table, const uint32_t* ids, const float* projection,
                       float* output, uint32_t vocab, uint32_t layers, uint32_t width, uint32_t tokens,
                       float embedding_scale, float output_scale) {
    return ple(ctx, 1, table, ids, projection, output, vocab, layers, width, tokens, embedding_scale, output_scale);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// host-slice operator API (NeuralOps)
// ---------------------------------------------------------------------------

namespace {

// Scoped device buffers for one host-slice call (buffer_from_slice,
// crates/atlas-metal/src/lib.rs:1975-1998).
struct Scratch {
    atlas_hip_ctx* ctx;
    void* ptrs[8] = {};
    int n = 0;
    explicit Scratch(atlas_hip_ctx* c) : ctx(c) {}
    ~Scratch() {
        for (int i = 0; i < n; ++i) atlas_hip_free(ctx, ptrs[i]);
    }
    int alloc(size_t bytes, void** out) {
        int rc = atlas_hip_malloc(ctx, bytes, out);
        if (rc == ATLAS_OK) ptrs[n++] = *out;
        return rc;
    }
    int upload(const void* src, size_t bytes, void** out) {
        int rc = alloc(bytes, out);
        if (rc == ATLAS_OK) rc = atlas_hip_upload(ctx, *out, src, bytes);
        return rc;
    }
};

// Times the enqueued launch with events and the whole call on the host.
template <class F>
int timed(atlas_hip_ctx* ctx, atlas_dispatch_timing* timing, std::chrono::steady_clock::time_point t0, F&& launch) {
    hipEvent_t a = nullptr, b = nullptr;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess)
        return fail(ctx, ATLAS_ERR_COMMAND_FAILED, "command creation failed");
    (void)hipEventRecord(a, ctx->stream);
    int rc = launch();
    (void)hipEventRecord(b, ctx->stream);
    if (rc == ATLAS_OK) rc = atlas_hip_sync(ctx);
    float ms = 0.0f;
    if (rc == ATLAS_OK) (void)hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    if (timing && rc == ATLAS_OK) {
        timing->gpu_ms = ms;
        timing->wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    }
    return rc;
}

bool mul_ok(size_t a, size_t b, size_t* out) {
    if (a != 0 && b > std::numeric_limits<size_t>::max() / a) return false;
    *out = a * b;
    return true;
}

}  // namespace

extern "C" {

int atlas_ops_embedding(atlas_hip_ctx* ctx, const float* table, size_t table_len, size_t vocabulary, size_t hidden,
                        const uint32_t* token_ids, size_t token_count, float* output, size_t output_len,
                        atlas_dispatch_timing* timing) {
    const auto t0 = std::chrono::steady_clock::now();
    int rc = enter(ctx);
    if (rc) return rc;
    size_t table_elems = 0, total = 0;
    if (!mul_ok(vocabulary, hidden, &table_elems) || table_len != table_elems)
        return invalid(ctx, "embedding table has the wrong length");
    if (hidden == 0 || token_count == 0 || !token_ids) return invalid(ctx, "embedding dimensions or token IDs are invalid");
    for (size_t i = 0; i < token_count; ++i)
        if (token_ids[i] >= vocabulary) return invalid(ctx, "embedding dimensions or token IDs are invalid");
    if (!mul_ok(token_count, hidden, &total)) return invalid(ctx, "embedding output length overflow");
    if (!output || output_len != total) return invalid(ctx, "embedding output has the wrong length");
    if (!fits_u32(vocabulary) || !fits_u32(hidden) || !fits_u32(token_count)) return invalid(ctx, "input is too large");
    Scratch s(ctx);
    void *dt, *di, *dout;
    if ((rc = s.upload(table, table_len * 4, &dt)) || (rc = s.upload(token_ids, token_count * 4, &di)) ||
        (rc = s.alloc(total * 4, &dout)))
        return rc;
    rc = timed(ctx, timing, t0, [&] {
        return atlas_hip_embed_f32(ctx, static_cast<float*>(dt), static_cast<uint32_t*>(di), static_cast<float*>(dout),
                                   static_cast<uint32_t>(vocabulary), static_cast<uint32_t>(hidden),
                                   static_cast<uint32_t>(token_count), 1.0f);
    });
    if (rc) return rc;
    return atlas_hip_download(ctx, output, dout, total * 4);
}

int atlas_ops_embedding_q6_k(atlas_hip_ctx* ctx, const uint8_t* weights, size_t weights_len, size_t vocabulary,
                             size_t hidden, const uint32_t* token_ids, size_t token_count, float* output,
                             size_t output_len, atlas_dispatch_timing* timing) {
    const auto t0 = std::chrono::steady_clock::now();
    int rc = enter(ctx);
    if (rc) return rc;
    if (hidden == 0 || hidden % 256 != 0 || token_count == 0 || !token_ids)
        return invalid(ctx, "Q6_K embedding dimensions or token IDs are invalid");
    for (size_t i = 0; i < token_count; ++i)
        if (token_ids[i] >= vocabulary) return invalid(ctx, "Q6_K embedding dimensions or token IDs are invalid");
    size_t elems = 0, bytes = 0, total = 0;
    if (!mul_ok(vocabulary, hidden, &elems) || !mul_ok(elems / 256, 210, &bytes))
        return invalid(ctx, "Q6_K embedding size overflows");
    if (!weights || weights_len != bytes) return invalid(ctx, "Q6_K embedding table has the wrong length");
    if (!mul_ok(token_count, hidden, &total)) return invalid(ctx, "Q6_K embedding output length overflow");
    if (!output || output_len != total) return invalid(ctx, "Q6_K embedding output has the wrong length");
    if (!fits_u32(vocabulary) || !fits_u32(hidden) || !fits_u32(token_count)) return invalid(ctx, "input is too large");
    Scratch s(ctx);
    void *dt, *di, *dout;
    if ((rc = s.upload(weights, weights_len, &dt)) || (rc = s.upload(token_ids, token_count * 4, &di)) ||
        (rc = s.alloc(total * 4, &dout)))
        return rc;
    rc = timed(ctx, timing, t0, [&] {
        return atlas_hip_embed_q6_k(ctx, static_cast<uint8_t*>(dt), static_cast<uint32_t*>(di),
                                    static_cast<float*>(dout), static_cast<uint32_t>(vocabulary),
                                    static_cast<uint32_t>(hidden), static_cast<uint32_t>(token_count), 1.0f);
    });
    if (rc) return rc;
    return atlas_hip_download(ctx, output, dout, total * 4);
}

static int binary_op(atlas_hip_ctx* ctx, int op, const float* lhs, size_t lhs_len, const float* rhs, size_t rhs_len,
                     float* output, size_t output_len, atlas_dispatch_timing* timing) {
    const auto t0 = std::chrono::steady_clock::now();
    int rc = enter(ctx);
    if (rc) return rc;
    if (lhs_len != rhs_len) return invalid(ctx, op == 0 ? "vector lengths differ" : "multiply requires equally sized non-empty vectors");
    if (op == 1 && lhs_len == 0) return invalid(ctx, "multiply requires equally sized non-empty vectors");
    if (!fits_u32(lhs_len)) return invalid(ctx, "vector is too large");
    if (output_len != lhs_len || (lhs_len && (!lhs || !rhs || !output))) return invalid(ctx, "output has the wrong length");
    if (lhs_len == 0) {
        if (timing) *timing = atlas_dispatch_timing{0.0, 0.0};
        return ATLAS_OK;
    }
    Scratch s(ctx);
    void *da, *db, *dout;
    if ((rc = s.upload(lhs, lhs_len * 4, &da)) || (rc = s.upload(rhs, rhs_len * 4, &db)) ||
        (rc = s.alloc(lhs_len * 4, &dout)))
        return rc;
    rc = timed(ctx, timing, t0, [&] {
        return op == 0 ? atlas_hip_add_f32(ctx, static_cast<float*>(da), static_cast<float*>(db),
                                           static_cast<float*>(dout), lhs_len)
                       : atlas_hip_multiply_f32(ctx, static_cast<float*>(da), static_cast<float*>(db),
                                                static_cast<float*>(dout), lhs_len);
    });
    if (rc) return rc;
    return atlas_hip_download(ctx, output, dout, lhs_len * 4);
}

int atlas_ops_add(atlas_hip_ctx* ctx, const float* lhs, size_t lhs_len, const float* rhs, size_t rhs_len,
                  float* output, size_t output_len, atlas_dispatch_timing* timing) {
    return binary_op(ctx, 0, lhs, lhs_len, rhs, rhs_len, output, output_len, timing);
}

int atlas_ops_multiply(atlas_hip_ctx* ctx, const float* lhs, size_t lhs_len, const float* rhs, size_t rhs_len,
                       float* output, size_t output_len, atlas_dispatch_timing* timing) {
    return binary_op(ctx, 1, lhs, lhs_len, rhs, rhs_len, output, output_len, timing);
}

static int unary_op(atlas_hip_ctx* ctx, int op, const float* input, size_t input_len, float scalar, float* output,
                    size_t output_len, atlas_dispatch_timing* timing) {
    const auto t0 = std::chrono::steady_clock::now();
    int rc = enter(ctx);
    if (rc) return rc;
    if (!fits_u32(input_len)) return invalid(ctx, "input is too large");
    if (output_len != input_len || (input_len && (!input || !output))) return invalid(ctx, "output has the wrong length");
    if (input_len == 0) {
        if (timing) *timing = atlas_dispatch_timing{0.0, 0.0};
        return ATLAS_OK;
    }
    Scratch s(ctx);
    void *da, *dout;
    if ((rc = s.upload(input, input_len * 4, &da)) || (rc = s.alloc(input_len * 4, &dout))) return rc;
    rc = timed(ctx, timing, t0, [&] {
        float* a = static_cast<float*>(da);
        float* o = static_cast<float*>(dout);
        if (op == 0) return atlas_hip_silu_f32(ctx, a, o, input_len);
        if (op == 1) return atlas_hip_gelu_f32(ctx, a, o, input_len);
        return atlas_hip_scale_f32(ctx, a, scalar, o, input_len);
    });
    if (rc) return rc;
    return atlas_hip_download(ctx, output, dout, input_len * 4);
}

int atlas_ops_silu(atlas_hip_ctx* ctx, const float* input, size_t input_len, float* output, size_t output_len,
                   atlas_dispatch_timing* timing) {
    return unary_op(ctx, 0, input, input_len, 0.0f, output, output_len, timing);
}

int atlas_ops_gelu(atlas_hip_ctx* ctx, const float* input, size_t input_len, float* output, size_t output_len,
                   atlas_dispatch_timing* timing) {
    return unary_op(ctx, 1, input, input_len, 0.0f, output, output_len, timing);
}

int atlas_ops_scalar_multiply(atlas_hip_ctx* ctx, const float* input, size_t input_len, float scalar, float* output,
                              size_t output_len, atlas_dispatch_timing* timing) {
    return unary_op(ctx, 2, input, input_len, scalar, output, output_len, timing);
}

int atlas_ops_rms_norm(atlas_hip_ctx* ctx, const float* input, size_t input_len, size_t rows, size_t hidden,
                       const float* weight, size_t weight_len, float epsilon, float* output, size_t output_len,
                       atlas_dispatch_timing* timing) {
    const auto t0 = std::chrono::steady_clock::now();
    int rc = enter(ctx);
    if (rc) return rc;
    size_t elements = 0;
    if (!mul_ok(rows, hidden, &elements)) return invalid(ctx, "RMSNorm dimensions overflow");
    if (input_len != elements) return invalid(ctx, "RMSNorm input has the wrong length");
    if (weight_len != hidden) return invalid(ctx, "RMSNorm weight has the wrong length");
    if (rows == 0 || hidden == 0 || !finite_positive(epsilon)) return invalid(ctx, "RMSNorm dimensions or epsilon are invalid");
    if (!input || !weight || !output || output_len != elements) return invalid(ctx, "RMSNorm output has the wrong length");
    if (!fits_u32(rows) || !fits_u32(hidden)) return invalid(ctx, "input is too large");
    Scratch s(ctx);
    void *dx, *dw, *dout;
    if ((rc = s.upload(input, elements * 4, &dx)) || (rc = s.upload(weight, hidden * 4, &dw)) ||
        (rc = s.alloc(elements * 4, &dout)))
        return rc;
    rc = timed(ctx, timing, t0, [&] {
        return atlas_hip_rms_norm_f32(ctx, static_cast<float*>(dx), static_cast<float*>(dw), static_cast<float*>(dout),
                                      static_cast<uint32_t>(rows), static_cast<uint32_t>(hidden), epsilon);
    });
    if (rc) return rc;
    return atlas_hip_download(ctx, output, dout, elements * 4);
}

int atlas_ops_rope(atlas_hip_ctx* ctx, const float* input, size_t input_len, size_t rows, size_t hidden,
                   const float* cosine, size_t cosine_len, const float* sine, size_t sine_len, float* output,
                   size_t output_len, atlas_dispatch_timing* timing) {
    const auto t0 = std::chrono::steady_clock::now();
    int rc = enter(ctx);
    if (rc) return rc;
    size_t elements = 0;
    if (!mul_ok(rows, hidden, &elements)) return invalid(ctx, "RoPE input overflow");
    if (input_len != elements) return invalid(ctx, "RoPE input has the wrong length");
    if (cosine_len != hidden / 2) return invalid(ctx, "RoPE cosine has the wrong length");
    if (sine_len != hidden / 2) return invalid(ctx, "RoPE sine has the wrong length");
    if (rows == 0 || hidden == 0 || hidden % 2 != 0) return invalid(ctx, "RoPE hidden width must be a non-zero even number");
    if (!input || !cosine || !sine || !output || output_len != elements) return invalid(ctx, "RoPE output has the wrong length");
    if (!fits_u32(rows) || !fits_u32(hidden)) return invalid(ctx, "input is too large");
    Scratch s(ctx);
    void *dx, *dc, *ds, *dout;
    if ((rc = s.upload(input, elements * 4, &dx)) || (rc = s.upload(cosine, cosine_len * 4, &dc)) ||
        (rc = s.upload(sine, sine_len * 4, &ds)) || (rc = s.alloc(elements * 4, &dout)))
        return rc;
    rc = timed(ctx, timing, t0, [&] {
        return atlas_hip_rope_interleaved_f32(ctx, static_cast<float*>(dx), static_cast<float*>(dc),
                                              static_cast<float*>(ds), static_cast<float*>(dout),
                                              static_cast<uint32_t>(rows), static_cast<uint32_t>(hidden));
    });
    if (rc) return rc;
    return atlas_hip_download(ctx, output, dout, elements * 4);
}

}  // extern "C"
