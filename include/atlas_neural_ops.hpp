/*
 * atlas_neural_ops.hpp -- C++17 host interface over libatlas_hip_ops.so that
 * mirrors the reference operator API atlas_ops::NeuralOps
 * (crates/atlas-ops/src/lib.rs:20-147) for the fused per-layer ops:
 * the same method names and argument order, host slices in, an owned output
 * plus DispatchTiming out, and failures raised as OperatorError carrying the
 * MetalError kind the reference returns (crates/atlas-metal/src/lib.rs:37-53).
 *
 * Header-only; link with -latlas_hip_ops.  DeviceBuffer<T> is the resident
 * counterpart of GpuBuffer (lib.rs:225-238) for the device-pointer entry
 * points (atlas_hip_*), which callers invoke directly on buffer.data().
 */
#ifndef ATLAS_NEURAL_OPS_HPP
#define ATLAS_NEURAL_OPS_HPP

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "atlas_hip_ops.h"

namespace atlas {

/* DispatchTiming (lib.rs:81-88): host wall time of the call and the GPU time
 * between events around the kernel launch. */
struct DispatchTiming {
    double wall_ms = 0.0;
    double gpu_ms = 0.0;
};

/* MetalError variants the operator path can produce, mapped from atlas_status. */
enum class ErrorKind { NoDevice, InvalidInput, CommandFailed, OutOfMemory };

inline const char* error_kind_name(ErrorKind k) {
    switch (k) {
        case ErrorKind::NoDevice: return "NoDevice";
        case ErrorKind::InvalidInput: return "InvalidInput";
        case ErrorKind::CommandFailed: return "CommandFailed";
        default: return "OutOfMemory";
    }
}

/* OperatorError::Metal(MetalError::...) (crates/atlas-ops/src/lib.rs:14-18). */
class OperatorError : public std::runtime_error {
   public:
    OperatorError(ErrorKind kind, const std::string& message)
        : std::runtime_error(std::string(error_kind_name(kind)) + ": " + message), kind_(kind) {}
    ErrorKind kind() const { return kind_; }

   private:
    ErrorKind kind_;
};

inline ErrorKind kind_of(int status) {
    switch (status) {
        case ATLAS_ERR_NO_DEVICE: return ErrorKind::NoDevice;
        case ATLAS_ERR_INVALID_INPUT: return ErrorKind::InvalidInput;
        case ATLAS_ERR_OUT_OF_MEMORY: return ErrorKind::OutOfMemory;
        default: return ErrorKind::CommandFailed;
    }
}

/* A read-only host slice (&[T]): pointer and length, built from any
 * contiguous container (std::vector, std::array, a C array). */
template <class T>
struct Slice {
    const T* ptr = nullptr;
    std::size_t len = 0;
    Slice() = default;
    Slice(const T* p, std::size_t n) : ptr(p), len(n) {}
    template <class C, class = decltype(std::declval<const C&>().data())>
    Slice(const C& c) : ptr(c.data()), len(c.size()) {}
    template <std::size_t N>
    Slice(const T (&a)[N]) : ptr(a), len(N) {}
};

/* (Vec<T>, DispatchTiming), the reference operators' Ok value. */
template <class T>
using Output = std::pair<std::vector<T>, DispatchTiming>;

class NeuralOps {
   public:
    /* NeuralOps::new -> MetalRuntime::new; throws OperatorError(NoDevice). */
    explicit NeuralOps(int device = 0) {
        const int rc = atlas_hip_init(device, &ctx_);
        if (rc != ATLAS_OK) throw OperatorError(kind_of(rc), "no HIP device is available to this process");
    }
    ~NeuralOps() {
        if (ctx_) atlas_hip_destroy(ctx_);
    }
    NeuralOps(const NeuralOps&) = delete;
    NeuralOps& operator=(const NeuralOps&) = delete;
    NeuralOps(NeuralOps&& o) noexcept : ctx_(o.ctx_) { o.ctx_ = nullptr; }
    NeuralOps& operator=(NeuralOps&& o) noexcept {
        if (this != &o) {
            if (ctx_) atlas_hip_destroy(ctx_);
            ctx_ = o.ctx_;
            o.ctx_ = nullptr;
        }
        return *this;
    }

    /* runtime(): the context the device-pointer entry points take. */
    atlas_hip_ctx* runtime() const { return ctx_; }

    /* NeuralOps::embedding (lib.rs:34-44). */
    Output<float> embedding(Slice<float> table, std::size_t vocabulary, std::size_t hidden,
                            Slice<uint32_t> token_ids) const {
        Output<float> out{std::vector<float>(token_ids.len * hidden), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_embedding(ctx_, table.ptr, table.len, vocabulary, hidden, token_ids.ptr, token_ids.len,
                                  out.first.data(), out.first.size(), &t));
        return finish(std::move(out), t);
    }
    /* NeuralOps::add (lib.rs:45-51). */
    Output<float> add(Slice<float> lhs, Slice<float> rhs) const {
        Output<float> out{std::vector<float>(lhs.len), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_add(ctx_, lhs.ptr, lhs.len, rhs.ptr, rhs.len, out.first.data(), out.first.size(), &t));
        return finish(std::move(out), t);
    }
    /* NeuralOps::multiply (lib.rs:52-58). */
    Output<float> multiply(Slice<float> lhs, Slice<float> rhs) const {
        Output<float> out{std::vector<float>(lhs.len), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_multiply(ctx_, lhs.ptr, lhs.len, rhs.ptr, rhs.len, out.first.data(), out.first.size(),
                                 &t));
        return finish(std::move(out), t);
    }
    /* NeuralOps::silu (lib.rs:59-61). */
    Output<float> silu(Slice<float> input) const {
        Output<float> out{std::vector<float>(input.len), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_silu(ctx_, input.ptr, input.len, out.first.data(), out.first.size(), &t));
        return finish(std::move(out), t);
    }
    /* NeuralOps::rms_norm (lib.rs:62-73). */
    Output<float> rms_norm(Slice<float> input, std::size_t rows, std::size_t hidden, Slice<float> weight,
                           float epsilon) const {
        Output<float> out{std::vector<float>(input.len), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_rms_norm(ctx_, input.ptr, input.len, rows, hidden, weight.ptr, weight.len, epsilon,
                                 out.first.data(), out.first.size(), &t));
        return finish(std::move(out), t);
    }
    /* NeuralOps::rope (lib.rs:74-83): interleaved pairs, cos/sin of hidden/2. */
    Output<float> rope(Slice<float> input, std::size_t rows, std::size_t hidden, Slice<float> cosine,
                       Slice<float> sine) const {
        Output<float> out{std::vector<float>(input.len), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_rope(ctx_, input.ptr, input.len, rows, hidden, cosine.ptr, cosine.len, sine.ptr, sine.len,
                             out.first.data(), out.first.size(), &t));
        return finish(std::move(out), t);
    }
    /* MetalRuntime::gelu (crates/atlas-metal/src/lib.rs:1913-1926). */
    Output<float> gelu(Slice<float> input) const {
        Output<float> out{std::vector<float>(input.len), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_gelu(ctx_, input.ptr, input.len, out.first.data(), out.first.size(), &t));
        return finish(std::move(out), t);
    }
    /* MetalRuntime::scalar_multiply (lib.rs:1348-1366). */
    Output<float> scalar_multiply(Slice<float> input, float scalar) const {
        Output<float> out{std::vector<float>(input.len), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_scalar_multiply(ctx_, input.ptr, input.len, scalar, out.first.data(), out.first.size(),
                                        &t));
        return finish(std::move(out), t);
    }
    /* MetalRuntime::embedding_lookup_q6_k (lib.rs:1437-1483). */
    Output<float> embedding_lookup_q6_k(Slice<uint8_t> weights, std::size_t vocabulary, std::size_t hidden,
                                        Slice<uint32_t> token_ids) const {
        Output<float> out{std::vector<float>(token_ids.len * hidden), {}};
        atlas_dispatch_timing t{};
        check(atlas_ops_embedding_q6_k(ctx_, weights.ptr, weights.len, vocabulary, hidden, token_ids.ptr,
                                       token_ids.len, out.first.data(), out.first.size(), &t));
        return finish(std::move(out), t);
    }

    /* ResidentCommand::finish (lib.rs:743-755) for work enqueued through the
     * device-pointer entry points on runtime(). */
    void finish() const { check(atlas_hip_sync(ctx_)); }

    /* Throws OperatorError for a non-OK atlas_status of this context. */
    void check(int status) const {
        if (status != ATLAS_OK) throw OperatorError(kind_of(status), atlas_hip_last_error(ctx_));
    }

   private:
    static Output<float> finish(Output<float> out, const atlas_dispatch_timing& t) {
        out.second.wall_ms = t.wall_ms;
        out.second.gpu_ms = t.gpu_ms;
        return out;
    }
    atlas_hip_ctx* ctx_ = nullptr;
};

/* A device allocation owned through a NeuralOps context (GpuBuffer,
 * lib.rs:225-238): upload/download by value, freed on destruction. */
template <class T>
class DeviceBuffer {
   public:
    DeviceBuffer(const NeuralOps& ops, std::size_t count) : ops_(&ops), count_(count) {
        void* p = nullptr;
        ops.check(atlas_hip_malloc(ops.runtime(), count * sizeof(T), &p));
        ptr_ = static_cast<T*>(p);
    }
    DeviceBuffer(const NeuralOps& ops, Slice<T> host) : DeviceBuffer(ops, host.len) { upload(host); }
    ~DeviceBuffer() {
        if (ptr_) atlas_hip_free(ops_->runtime(), ptr_);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    T* data() { return ptr_; }
    const T* data() const { return ptr_; }
    std::size_t size() const { return count_; }
    void upload(Slice<T> host) {
        if (host.len > count_) throw OperatorError(ErrorKind::InvalidInput, "upload larger than the buffer");
        ops_->check(atlas_hip_upload(ops_->runtime(), ptr_, host.ptr, host.len * sizeof(T)));
    }
    std::vector<T> download() const {
        std::vector<T> out(count_);
        ops_->check(atlas_hip_download(ops_->runtime(), out.data(), ptr_, count_ * sizeof(T)));
        return out;
    }

   private:
    const NeuralOps* ops_;
    T* ptr_ = nullptr;
    std::size_t count_ = 0;
};

}  // namespace atlas

#endif  // ATLAS_NEURAL_OPS_HPP
