/*
 * atlas_gguf.h -- C ABI of the GGUF v3 reader in libatlas_hip_ops.so: the
 * host side that feeds the model's packed tables (Q4_0 / Q6_K token and PLE
 * embeddings, Q4_0 projections, F32 norm weights) to the device ops in
 * atlas_hip_ops.h without conversion.
 *
 * It restates atlas_core::gguf::GgufModel (crates/atlas-core/src/gguf.rs:
 * 112-235) with the same checks, in the same order, each failing with
 * ATLAS_ERR_INVALID_INPUT and a message (CoreError::InvalidInput):
 *   magic "GGUF"; version 3; tensor and metadata counts <= 1 000 000;
 *   UTF-8 keys and strings; known metadata value types (0-12; arrays of
 *   strings, f32, i32, u32, u64, i64 and bool are kept, arrays of the other
 *   scalar types are read and dropped, nested arrays are rejected);
 *   tensor rank 1..4 with non-zero dimensions and no element-count overflow;
 *   tensor types F32 (0), F16 (1), Q4_0 (2), Q8_0 (8), Q6_K (14) only,
 *   packed element counts a multiple of the block (32, or 256 for Q6_K);
 *   tensor offsets 32-byte aligned; general.alignment absent or 32; every
 *   tensor inside the file; no two tensors overlapping.
 * Scalar metadata values are kept as the reference keeps them, as strings
 * (GgufModel::metadata: integers in decimal, floats as the shortest decimal
 * that reads back to the same value, booleans as true/false).
 *
 * The file is memory-mapped read-only (the reference reads it into memory,
 * GgufModel::open); atlas_gguf_from_bytes copies a caller buffer.  Strings and
 * data pointers returned stay valid until atlas_gguf_close.  A model may be
 * read from several threads; it is never modified after it is opened.
 */
#ifndef ATLAS_GGUF_H
#define ATLAS_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "atlas_hip_ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct atlas_gguf atlas_gguf;

/* GgufTensorType raw codes (crates/atlas-core/src/gguf.rs:16-45). */
enum {
    ATLAS_GGUF_F32 = 0,
    ATLAS_GGUF_F16 = 1,
    ATLAS_GGUF_Q4_0 = 2,
    ATLAS_GGUF_Q8_0 = 8,
    ATLAS_GGUF_Q6_K = 14
};

/* GgufTensor (crates/atlas-core/src/gguf.rs:80-87).  dims are in GGUF order
 * (dims[0] is the contiguous one: a [vocab, hidden] table has dims
 * {hidden, vocab}). */
typedef struct atlas_gguf_tensor {
    const char *name; /* name_len bytes of UTF-8 (may hold NUL), NUL-terminated after them */
    uint64_t name_len;
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t type;
    uint64_t offset; /* from the start of the aligned data section */
    uint64_t bytes;  /* encoded size (GgufTensorType::encoded_bytes, gguf.rs:56-77) */
} atlas_gguf_tensor;

/* GgufModel::open / from_bytes (gguf.rs:112-225).  On failure *out is NULL
 * and, when error is not NULL, the message is copied into error[error_len]. */
int atlas_gguf_open(const char *path, atlas_gguf **out, char *error, size_t error_len);
int atlas_gguf_from_bytes(const void *data, size_t bytes, atlas_gguf **out, char *error, size_t error_len);
void atlas_gguf_close(atlas_gguf *model);

/* GgufModel::tensors, in file order. */
uint64_t atlas_gguf_tensor_count(const atlas_gguf *model);
int atlas_gguf_tensor_info(const atlas_gguf *model, uint64_t index, atlas_gguf_tensor *out);
/* Index of the tensor called `name` (NUL-terminated), or -1. */
int64_t atlas_gguf_find_tensor(const atlas_gguf *model, const char *name);
/* GgufModel::tensor_data (gguf.rs:226-235): the encoded bytes of a tensor. */
int atlas_gguf_tensor_data(const atlas_gguf *model, uint64_t index, const void **data, uint64_t *bytes);
/* Copy a tensor's encoded bytes into device memory (the upload of
 * ensure_resident_weights, crates/atlas-model/src/lib.rs:720-753); the
 * destination holds at least atlas_gguf_tensor.bytes bytes.
 * Synchronous. */
int atlas_gguf_upload_tensor(atlas_hip_ctx *ctx, const atlas_gguf *model, uint64_t index, void *device_dst);

/* Names, keys and strings are UTF-8 and may contain NUL bytes (Rust strings
 * do), so entries are returned as pointer + length; each is also followed by
 * a NUL for callers that know their strings hold none. */

/* GgufModel::metadata (scalar values as strings), in key order. */
uint64_t atlas_gguf_metadata_count(const atlas_gguf *model);
int atlas_gguf_metadata_entry(const atlas_gguf *model, uint64_t index, const char **key, uint64_t *key_len,
                              const char **value, uint64_t *value_len);
/* The value stored under the NUL-terminated `key`, or NULL. */
const char *atlas_gguf_metadata_get(const atlas_gguf *model, const char *key);

/* GgufModel::metadata_arrays (GgufMetadataArray, gguf.rs:89-100), in key
 * order.  *element_type is the GGUF element type (8 strings, 6 f32, 5 i32,
 * 4 u32, 10 u64, 11 i64, 7 bool), *count the length and, for the numeric and
 * bool kinds, *values the packed little-endian elements (bool: one byte, 0
 * or 1); for strings *values is NULL and atlas_gguf_metadata_array_string
 * returns the elements. */
uint64_t atlas_gguf_metadata_array_count(const atlas_gguf *model);
int atlas_gguf_metadata_array_entry(const atlas_gguf *model, uint64_t index, const char **key, uint64_t *key_len,
                                    uint32_t *element_type, uint64_t *count, const void **values);
int atlas_gguf_metadata_array_string(const atlas_gguf *model, uint64_t index, uint64_t element, const char **text,
                                     uint64_t *text_len);
/* Index of the array stored under the NUL-terminated `key`, or -1. */
int64_t atlas_gguf_find_metadata_array(const atlas_gguf *model, const char *key);

#ifdef __cplusplus
}
#endif

#endif /* ATLAS_GGUF_H */
