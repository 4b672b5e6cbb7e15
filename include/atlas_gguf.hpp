/*
 * atlas_gguf.hpp -- C++17 mirror of atlas_core::gguf::GgufModel
 * (crates/atlas-core/src/gguf.rs:80-235) over the C reader in
 * libatlas_hip_ops.so (include/atlas_gguf.h): GgufModel::open / from_bytes,
 * `tensors()` (GgufTensor), `metadata()` (scalar values as strings),
 * `metadata_arrays()` (GgufMetadataArray) and `tensor_data()`.  Failures
 * throw atlas::OperatorError(InvalidInput), as the reference returns
 * CoreError::InvalidInput.
 *
 * Header-only; link with -latlas_hip_ops.
 */
#ifndef ATLAS_GGUF_HPP
#define ATLAS_GGUF_HPP

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <map>
#include <string>
#include <utility>
#include <vector>

#include "atlas_gguf.h"
#include "atlas_neural_ops.hpp"

namespace atlas {

/* GgufTensorType (gguf.rs:16-23). */
enum class GgufTensorType : uint32_t { F32 = 0, F16 = 1, Q4_0 = 2, Q8_0 = 8, Q6K = 14 };

/* GgufTensor (gguf.rs:80-87); dims in GGUF order (dims[0] contiguous). */
struct GgufTensor {
    std::string name;
    std::vector<uint64_t> dims;
    GgufTensorType tensor_type;
    uint64_t offset;
    uint64_t bytes;
    uint64_t index;  // position in the file's tensor list
};

/* GgufMetadataArray (gguf.rs:89-100): the element type and either the
 * strings or the packed little-endian elements (bool: one byte each). */
struct GgufMetadataArray {
    uint32_t element_type = 0;
    uint64_t count = 0;
    std::vector<std::string> strings;
    std::vector<uint8_t> packed;
};

class GgufModel {
   public:
    static GgufModel open(const std::string& path) {
        atlas_gguf* h = nullptr;
        char err[512] = {0};
        const int rc = atlas_gguf_open(path.c_str(), &h, err, sizeof err);
        if (rc != ATLAS_OK) throw OperatorError(kind_of(rc), err);
        return GgufModel(h);
    }
    static GgufModel from_bytes(const std::vector<uint8_t>& data) {
        atlas_gguf* h = nullptr;
        char err[512] = {0};
        const int rc = atlas_gguf_from_bytes(data.data(), data.size(), &h, err, sizeof err);
        if (rc != ATLAS_OK) throw OperatorError(kind_of(rc), err);
        return GgufModel(h);
    }
    ~GgufModel() {
        if (h_) atlas_gguf_close(h_);
    }
    GgufModel(const GgufModel&) = delete;
    GgufModel& operator=(const GgufModel&) = delete;
    GgufModel(GgufModel&& o) noexcept : h_(o.h_), tensors_(std::move(o.tensors_)), metadata_(std::move(o.metadata_)),
                                        arrays_(std::move(o.arrays_)) {
        o.h_ = nullptr;
    }

    const std::vector<GgufTensor>& tensors() const { return tensors_; }
    const std::map<std::string, std::string>& metadata() const { return metadata_; }
    const std::map<std::string, GgufMetadataArray>& metadata_arrays() const { return arrays_; }

    /* GgufModel::tensor_data (gguf.rs:226-235): a view of the encoded bytes,
     * valid while the model lives. */
    std::pair<const uint8_t*, std::size_t> tensor_data(const GgufTensor& t) const {
        const void* p = nullptr;
        uint64_t n = 0;
        const int rc = atlas_gguf_tensor_data(h_, t.index, &p, &n);
        if (rc != ATLAS_OK) throw OperatorError(kind_of(rc), "GGUF tensor data is outside file");
        return {static_cast<const uint8_t*>(p), static_cast<std::size_t>(n)};
    }
    const GgufTensor& tensor(const std::string& name) const {
        for (const GgufTensor& t : tensors_)
            if (t.name == name) return t;
        throw OperatorError(ErrorKind::InvalidInput, "GGUF tensor " + name + " is missing");
    }
    /* The resident upload of one tensor into caller-owned device memory. */
    void upload(const NeuralOps& ops, const GgufTensor& t, void* device_dst) const {
        ops.check(atlas_gguf_upload_tensor(ops.runtime(), h_, t.index, device_dst));
    }
    const atlas_gguf* handle() const { return h_; }

   private:
    explicit GgufModel(atlas_gguf* h) : h_(h) {
        const uint64_t n = atlas_gguf_tensor_count(h);
        for (uint64_t i = 0; i < n; ++i) {
            atlas_gguf_tensor info{};
            atlas_gguf_tensor_info(h, i, &info);
            tensors_.push_back(GgufTensor{std::string(info.name, info.name_len),
                                          std::vector<uint64_t>(info.dims, info.dims + info.n_dims),
                                          static_cast<GgufTensorType>(info.type), info.offset, info.bytes, i});
        }
        for (uint64_t i = 0; i < atlas_gguf_metadata_count(h); ++i) {
            const char *k = nullptr, *v = nullptr;
            uint64_t kn = 0, vn = 0;
            atlas_gguf_metadata_entry(h, i, &k, &kn, &v, &vn);
            metadata_.emplace(std::string(k, kn), std::string(v, vn));
        }
        for (uint64_t i = 0; i < atlas_gguf_metadata_array_count(h); ++i) {
            const char* k = nullptr;
            uint64_t kn = 0;
            GgufMetadataArray a;
            const void* values = nullptr;
            atlas_gguf_metadata_array_entry(h, i, &k, &kn, &a.element_type, &a.count, &values);
            if (a.element_type == 8) {
                for (uint64_t e = 0; e < a.count; ++e) {
                    const char* text = nullptr;
                    uint64_t len = 0;
                    atlas_gguf_metadata_array_string(h, i, e, &text, &len);
                    a.strings.emplace_back(text, len);
                }
            } else if (values) {
                const std::size_t width = a.element_type == 7 ? 1 : (a.element_type == 10 || a.element_type == 11 ? 8 : 4);
                const uint8_t* p = static_cast<const uint8_t*>(values);
                a.packed.assign(p, p + a.count * width);
            }
            arrays_.emplace(std::string(k, kn), std::move(a));
        }
    }

    atlas_gguf* h_ = nullptr;
    std::vector<GgufTensor> tensors_;
    std::map<std::string, std::string> metadata_;
    std::map<std::string, GgufMetadataArray> arrays_;
};

}  // namespace atlas

#endif  // ATLAS_GGUF_HPP
