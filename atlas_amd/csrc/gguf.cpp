// gguf.cpp -- the GGUF v3 reader behind include/atlas_gguf.h.
//
// Restates atlas_core::gguf::GgufModel::from_bytes
// (crates/atlas-core/src/gguf.rs:112-225) and its Reader (:439-568): the same
// fields are read in the same order and the same conditions are rejected,
// so a file the reference refuses is refused here and a file it accepts
// yields the same tensors, offsets, sizes and metadata strings.  Host code
// only; the tensor bytes reach the device through atlas_hip_upload.
#include "../../include/atlas_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

namespace {

constexpr uint64_t kAlignment = 32;  // GGUF_ALIGNMENT (gguf.rs:13)

struct GgufError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void reject(const std::string& what) { throw GgufError(what); }

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type;
    uint64_t offset;
    uint64_t bytes;
};

struct MetaArray {
    uint32_t type = 0;
    uint64_t count = 0;
    std::vector<uint8_t> packed;       // numeric / bool elements, little-endian
    std::vector<std::string> strings;  // string elements
};

// GgufTensorType::block_bytes / encoded_bytes (gguf.rs:47-77).
bool known_type(uint32_t t) { return t == 0 || t == 1 || t == 2 || t == 8 || t == 14; }

uint64_t encoded_bytes(uint32_t type, uint64_t elements) {
    switch (type) {
        case 0:
        case 1: {
            const uint64_t width = type == 0 ? 4 : 2;
            if (elements > UINT64_MAX / width) reject("GGUF tensor byte size overflows");
            return elements * width;
        }
        default: {
            const uint64_t block = type == 14 ? 256 : 32;
            const uint64_t bytes = type == 2 ? 18 : (type == 8 ? 34 : 210);
            if (elements % block != 0)
                reject("packed GGUF tensor has " + std::to_string(elements) + " elements, not a multiple of " +
                       std::to_string(block));
            const uint64_t blocks = elements / block;
            if (blocks > UINT64_MAX / bytes) reject("GGUF packed tensor byte size overflows");
            return blocks * bytes;
        }
    }
}

// Strict UTF-8 (the rules of Rust's str::from_utf8): no overlong forms, no
// surrogates, nothing above U+10FFFF.
bool valid_utf8(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        size_t extra;
        uint8_t lo = 0x80, hi = 0xBF;
        if (c >= 0xC2 && c <= 0xDF) {
            extra = 1;
        } else if (c >= 0xE0 && c <= 0xEF) {
            extra = 2;
            if (c == 0xE0) lo = 0xA0;
            if (c == 0xED) hi = 0x9F;
        } else if (c >= 0xF0 && c <= 0xF4) {
            extra = 3;
            if (c == 0xF0) lo = 0x90;
            if (c == 0xF4) hi = 0x8F;
        } else {
            return false;
        }
        if (n - i <= extra) return false;
        if (s[i + 1] < lo || s[i + 1] > hi) return false;
        for (size_t k = 2; k <= extra; ++k)
            if ((s[i + k] & 0xC0) != 0x80) return false;
        i += extra + 1;
    }
    return true;
}

// Rust's Display for floats: the shortest decimal that reads back to the
// same value, never in exponent form; NaN / inf / -inf spelled as Rust does.
// The digits come from std::to_chars' shortest scientific form (d.ddde+X);
// they are then laid out positionally, padded with zeros (fixed-format
// to_chars would print the exact binary expansion of large values instead).
template <typename T>
std::string rust_float(T v) {
    if (std::isnan(v)) return "NaN";
    if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
    char buf[64];
    const auto r = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::scientific);
    const std::string sci(buf, r.ptr);
    const size_t e_at = sci.find('e');
    std::string digits;
    bool negative = false;
    for (size_t i = 0; i < e_at; ++i) {
        if (sci[i] == '-') negative = true;
        else if (sci[i] != '.') digits += sci[i];
    }
    const int exponent = std::stoi(sci.substr(e_at + 1));  // value = d.ddd x 10^exponent
    std::string out = negative ? "-" : "";
    if (exponent < 0) {
        out += "0." + std::string(static_cast<size_t>(-exponent - 1), '0') + digits;
    } else {
        const size_t whole = static_cast<size_t>(exponent) + 1;
        if (digits.size() <= whole) {
            out += digits + std::string(whole - digits.size(), '0');
        } else {
            out += digits.substr(0, whole) + "." + digits.substr(whole);
        }
    }
    return out;
}

// Rust's usize::from_str: an optional '+', then one or more decimal digits.
bool parse_usize(const std::string& s, uint64_t* out) {
    size_t i = s.size() > 0 && s[0] == '+' ? 1 : 0;
    if (i == s.size()) return false;
    uint64_t v = 0;
    for (; i < s.size(); ++i) {
        if (s[i] < '0' || s[i] > '9') return false;
        const uint64_t d = static_cast<uint64_t>(s[i] - '0');
        if (v > (UINT64_MAX - d) / 10) return false;
        v = v * 10 + d;
    }
    *out = v;
    return true;
}

// Reader (gguf.rs:439-568): a cursor that never reads past the buffer.
struct Cursor {
    const uint8_t* data;
    uint64_t len;
    uint64_t at = 0;

    const uint8_t* take(uint64_t n) {
        if (n > UINT64_MAX - at) reject("GGUF cursor overflows");
        if (at + n > len) reject("truncated GGUF");
        const uint8_t* p = data + at;
        at += n;
        return p;
    }
    template <typename T>
    T le() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));  // x86-64 and gfx hosts are little-endian
        return v;
    }
    uint32_t u32() { return le<uint32_t>(); }
    uint64_t u64() { return le<uint64_t>(); }
    std::string string() {
        const uint64_t n = u64();
        const uint8_t* p = take(n);
        if (!valid_utf8(p, n)) reject("GGUF string is not UTF-8");
        return std::string(reinterpret_cast<const char*>(p), n);
    }
    // metadata_value: the scalar kinds Atlas keeps, as their string form.
    std::string value(uint32_t type) {
        switch (type) {
            case 0: return std::to_string(static_cast<unsigned>(take(1)[0]));
            case 1: return std::to_string(static_cast<int>(static_cast<int8_t>(take(1)[0])));
            case 2: return std::to_string(le<uint16_t>());
            case 3: return std::to_string(le<int16_t>());
            case 4: return std::to_string(le<uint32_t>());
            case 5: return std::to_string(le<int32_t>());
            case 6: return rust_float(le<float>());
            case 7: return take(1)[0] != 0 ? "true" : "false";
            case 8: return string();
            case 9: reject("GGUF array must be read through metadata_array");
            case 10: return std::to_string(le<uint64_t>());
            case 11: return std::to_string(le<int64_t>());
            case 12: return rust_float(le<double>());
            default: reject("unsupported GGUF metadata type " + std::to_string(type));
        }
    }
    // metadata_array: strings, f32, i32, u32, u64, i64 and bool are kept;
    // other element kinds are read and dropped (returns false).
    bool array(MetaArray* out) {
        const uint32_t type = u32();
        const uint64_t count = u64();
        out->type = type;
        out->count = count;
        uint64_t width = 0;
        switch (type) {
            case 8:
                for (uint64_t i = 0; i < count; ++i) out->strings.push_back(string());
                return true;
            case 6: case 5: case 4: width = 4; break;
            case 10: case 11: width = 8; break;
            case 7: width = 1; break;
            default:
                for (uint64_t i = 0; i < count; ++i) (void)value(type);
                return false;
        }
        for (uint64_t i = 0; i < count; ++i) {
            const uint8_t* p = take(width);
            if (type == 7)
                out->packed.push_back(p[0] != 0 ? 1 : 0);
            else
                out->packed.insert(out->packed.end(), p, p + width);
        }
        return true;
    }
};

uint64_t align_up(uint64_t v, uint64_t a) {
    if (v > UINT64_MAX - (a - 1)) reject("GGUF alignment overflows");
    return (v + a - 1) / a * a;
}

}  // namespace

struct atlas_gguf {
    void* map = nullptr;
    size_t map_len = 0;
    std::vector<uint8_t> owned;
    const uint8_t* data = nullptr;
    uint64_t len = 0;
    uint64_t data_start = 0;
    std::map<std::string, std::string> metadata;
    std::vector<const std::pair<const std::string, std::string>*> metadata_order;
    std::map<std::string, MetaArray> arrays;
    std::vector<const std::pair<const std::string, MetaArray>*> array_order;
    std::vector<Tensor> tensors;

    ~atlas_gguf() {
        if (map) munmap(map, map_len);
    }

    // GgufModel::from_bytes (gguf.rs:116-225).
    void parse() {
        Cursor r{data, len};
        if (std::memcmp(r.take(4), "GGUF", 4) != 0) reject("GGUF magic is missing");
        if (r.u32() != 3) reject("only GGUF v3 is supported");
        const uint64_t tensor_count = r.u64();
        const uint64_t metadata_count = r.u64();
        if (tensor_count > 1000000 || metadata_count > 1000000) reject("GGUF count is unreasonable");
        for (uint64_t m = 0; m < metadata_count; ++m) {
            std::string key = r.string();
            const uint32_t type = r.u32();
            if (type == 9) {
                MetaArray a;
                if (r.array(&a)) arrays[key] = std::move(a);
            } else {
                metadata[key] = r.value(type);
            }
        }
        tensors.reserve(tensor_count);
        for (uint64_t t = 0; t < tensor_count; ++t) {
            Tensor x;
            x.name = r.string();
            const uint32_t rank = r.u32();
            if (rank == 0 || rank > 4) reject("GGUF tensor " + x.name + " has invalid rank " + std::to_string(rank));
            uint64_t elements = 1;
            for (uint32_t d = 0; d < rank; ++d) {
                const uint64_t dim = r.u64();
                if (dim == 0) reject("GGUF tensor " + x.name + " has zero dimension");
                if (elements > UINT64_MAX / dim) reject("GGUF element count overflows");
                elements *= dim;
                x.dims.push_back(dim);
            }
            x.type = r.u32();
            if (!known_type(x.type)) reject("unsupported GGUF tensor type " + std::to_string(x.type));
            x.offset = r.u64();
            if (x.offset % kAlignment != 0) reject("GGUF tensor " + x.name + " offset is not aligned");
            x.bytes = encoded_bytes(x.type, elements);
            tensors.push_back(std::move(x));
        }
        const auto al = metadata.find("general.alignment");
        if (al != metadata.end()) {
            uint64_t a = 0;
            if (!parse_usize(al->second, &a)) reject("invalid general.alignment");
            if (a != kAlignment)
                reject("Atlas requires GGUF alignment 32, got " + std::to_string(a));
        }
        data_start = align_up(r.at, kAlignment);
        std::vector<std::tuple<uint64_t, uint64_t, const std::string*>> ranges;
        for (const Tensor& x : tensors) {
            if (x.offset > UINT64_MAX - data_start) reject("GGUF tensor offset overflows");
            const uint64_t start = data_start + x.offset;
            if (x.bytes > UINT64_MAX - start) reject("GGUF tensor range overflows");
            const uint64_t end = start + x.bytes;
            if (end > len) reject("GGUF tensor " + x.name + " is outside the file");
            ranges.emplace_back(start, end, &x.name);
        }
        std::stable_sort(ranges.begin(), ranges.end(),
                         [](const auto& a, const auto& b) { return std::get<0>(a) < std::get<0>(b); });
        for (size_t i = 1; i < ranges.size(); ++i)
            if (std::get<1>(ranges[i - 1]) > std::get<0>(ranges[i]))
                reject("GGUF tensors " + *std::get<2>(ranges[i - 1]) + " and " + *std::get<2>(ranges[i]) +
                       " overlap");
        for (const auto& kv : metadata) metadata_order.push_back(&kv);
        for (const auto& kv : arrays) array_order.push_back(&kv);
    }
};

namespace {

int finish(atlas_gguf* model, atlas_gguf** out, char* error, size_t error_len) {
    try {
        model->parse();
    } catch (const GgufError& e) {
        if (error && error_len) std::snprintf(error, error_len, "%s", e.what());
        delete model;
        return ATLAS_ERR_INVALID_INPUT;
    } catch (const std::bad_alloc&) {
        if (error && error_len) std::snprintf(error, error_len, "out of host memory");
        delete model;
        return ATLAS_ERR_OUT_OF_MEMORY;
    }
    *out = model;
    return ATLAS_OK;
}

int fail_open(char* error, size_t error_len, const char* what) {
    if (error && error_len) std::snprintf(error, error_len, "read GGUF: %s", what);
    return ATLAS_ERR_INVALID_INPUT;
}

}  // namespace

extern "C" {

int atlas_gguf_open(const char* path, atlas_gguf** out, char* error, size_t error_len) {
    if (!out) return ATLAS_ERR_INVALID_INPUT;
    *out = nullptr;
    if (!path) return fail_open(error, error_len, "no path");
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail_open(error, error_len, std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int err = errno;
        ::close(fd);
        return fail_open(error, error_len, std::strerror(err));
    }
    auto* model = new atlas_gguf;
    if (st.st_size > 0) {
        void* p = mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            const int err = errno;
            ::close(fd);
            delete model;
            return fail_open(error, error_len, std::strerror(err));
        }
        model->map = p;
        model->map_len = static_cast<size_t>(st.st_size);
        model->data = static_cast<const uint8_t*>(p);
        model->len = static_cast<uint64_t>(st.st_size);
    }
    ::close(fd);
    return finish(model, out, error, error_len);
}

int atlas_gguf_from_bytes(const void* data, size_t bytes, atlas_gguf** out, char* error, size_t error_len) {
    if (!out) return ATLAS_ERR_INVALID_INPUT;
    *out = nullptr;
    if (!data && bytes) return ATLAS_ERR_INVALID_INPUT;
    auto* model = new atlas_gguf;
    model->owned.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + bytes);
    model->data = model->owned.data();
    model->len = bytes;
    return finish(model, out, error, error_len);
}

void atlas_gguf_close(atlas_gguf* model) { delete model; }

uint64_t atlas_gguf_tensor_count(const atlas_gguf* model) { return model ? model->tensors.size() : 0; }

int atlas_gguf_tensor_info(const atlas_gguf* model, uint64_t index, atlas_gguf_tensor* out) {
    if (!model || !out || index >= model->tensors.size()) return ATLAS_ERR_INVALID_INPUT;
    const Tensor& t = model->tensors[index];
    std::memset(out, 0, sizeof *out);
    out->name = t.name.c_str();
    out->name_len = t.name.size();
    out->n_dims = static_cast<uint32_t>(t.dims.size());
    for (size_t d = 0; d < t.dims.size(); ++d) out->dims[d] = t.dims[d];
    out->type = t.type;
    out->offset = t.offset;
    out->bytes = t.bytes;
    return ATLAS_OK;
}

int64_t atlas_gguf_find_tensor(const atlas_gguf* model, const char* name) {
    if (!model || !name) return -1;
    for (size_t i = 0; i < model->tensors.size(); ++i)
        if (model->tensors[i].name == name) return static_cast<int64_t>(i);
    return -1;
}

int atlas_gguf_tensor_data(const atlas_gguf* model, uint64_t index, const void** data, uint64_t* bytes) {
    if (!model || !data || !bytes || index >= model->tensors.size()) return ATLAS_ERR_INVALID_INPUT;
    const Tensor& t = model->tensors[index];
    *data = model->data + model->data_start + t.offset;  // inside the file: checked at open
    *bytes = t.bytes;
    return ATLAS_OK;
}

int atlas_gguf_upload_tensor(atlas_hip_ctx* ctx, const atlas_gguf* model, uint64_t index, void* device_dst) {
    const void* src = nullptr;
    uint64_t bytes = 0;
    const int rc = atlas_gguf_tensor_data(model, index, &src, &bytes);
    if (rc) return rc;
    if (!device_dst) return ATLAS_ERR_INVALID_INPUT;
    return atlas_hip_upload(ctx, device_dst, src, static_cast<size_t>(bytes));
}

uint64_t atlas_gguf_metadata_count(const atlas_gguf* model) { return model ? model->metadata_order.size() : 0; }

int atlas_gguf_metadata_entry(const atlas_gguf* model, uint64_t index, const char** key, uint64_t* key_len,
                              const char** value, uint64_t* value_len) {
    if (!model || index >= model->metadata_order.size()) return ATLAS_ERR_INVALID_INPUT;
    const auto& kv = *model->metadata_order[index];
    if (key) *key = kv.first.c_str();
    if (key_len) *key_len = kv.first.size();
    if (value) *value = kv.second.c_str();
    if (value_len) *value_len = kv.second.size();
    return ATLAS_OK;
}

const char* atlas_gguf_metadata_get(const atlas_gguf* model, const char* key) {
    if (!model || !key) return nullptr;
    const auto it = model->metadata.find(key);
    return it == model->metadata.end() ? nullptr : it->second.c_str();
}

uint64_t atlas_gguf_metadata_array_count(const atlas_gguf* model) { return model ? model->array_order.size() : 0; }

int atlas_gguf_metadata_array_entry(const atlas_gguf* model, uint64_t index, const char** key, uint64_t* key_len,
                                    uint32_t* element_type, uint64_t* count, const void** values) {
    if (!model || index >= model->array_order.size()) return ATLAS_ERR_INVALID_INPUT;
    const auto& kv = *model->array_order[index];
    if (key) *key = kv.first.c_str();
    if (key_len) *key_len = kv.first.size();
    if (element_type) *element_type = kv.second.type;
    if (count) *count = kv.second.count;
    if (values) *values = kv.second.type == 8 || kv.second.packed.empty() ? nullptr : kv.second.packed.data();
    return ATLAS_OK;
}

int atlas_gguf_metadata_array_string(const atlas_gguf* model, uint64_t index, uint64_t element, const char** text,
                                     uint64_t* text_len) {
    if (!model || index >= model->array_order.size()) return ATLAS_ERR_INVALID_INPUT;
    const MetaArray& a = model->array_order[index]->second;
    if (a.type != 8 || element >= a.strings.size()) return ATLAS_ERR_INVALID_INPUT;
    if (text) *text = a.strings[element].c_str();
    if (text_len) *text_len = a.strings[element].size();
    return ATLAS_OK;
}

int64_t atlas_gguf_find_metadata_array(const atlas_gguf* model, const char* key) {
    if (!model || !key) return -1;
    for (size_t i = 0; i < model->array_order.size(); ++i)
        if (model->array_order[i]->first == key) return static_cast<int64_t>(i);
    return -1;
}

}  // extern "C"
