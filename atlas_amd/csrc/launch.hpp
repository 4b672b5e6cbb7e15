// launch.hpp -- internal (C++) launch entry points between the C-ABI layer
// (capi.hip) and the kernel translation units.  Each launcher assumes its
// arguments were validated by the caller and enqueues work on `stream`.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace atlas {

// Reduction order of the row sums of squares.
enum Reduction : int {
    kSequential = 0,  // left-to-right f32 fold: bit-identical to the CPU operators
    kWide = 1,        // lane-parallel partial sums + cross-lane tree (tolerance-level)
    kAuto = 2,        // tree for plain scaled rows, sequential where an epilogue cancels
};

// RMSNorm family (norm_kernels.hip).  Modes of the row epilogue:
enum NormMode : int {
    kNormPlain = 0,     // y = (x*inv)*w
    kNormResidual = 1,  // n = (x*inv)*w; [normalized = n]; out = residual + n
    kNormAddNorm = 2,   // r = x + residual -> residual_out; y = (r*inv)*w
    kNormAddScale = 3,  // n = (x*inv)*w; state = (state + n) * (*scale)
};

struct NormArgs {
    const float* x;
    const float* weight;
    const float* residual;
    float* normalized;
    float* residual_out;
    float* out;
    const float* scale;
    uint32_t rows;
    uint32_t hidden;
    float epsilon;
};

hipError_t launch_rms_norm_f32(hipStream_t stream, NormMode mode, Reduction red, const NormArgs& a);
hipError_t launch_rms_norm_groups_stable_f32(hipStream_t stream, Reduction red, float* values,
                                             const float* weight, uint32_t width, uint32_t groups,
                                             float epsilon);
hipError_t launch_rms_norm_f16(hipStream_t stream, Reduction red, const uint16_t* x,
                               const uint16_t* residual, const uint16_t* weight,
                               uint16_t* residual_out, uint16_t* out, uint32_t rows,
                               uint32_t hidden, float epsilon);

// RoPE (rope_kernels.hip).
hipError_t launch_qk_norm_rope_f32(hipStream_t stream, Reduction red, const float* q,
                                   const float* k, const float* q_weight, const float* k_weight,
                                   const float* cosine, const float* sine, float* q_out,
                                   float* k_out, uint32_t tokens, uint32_t q_heads,
                                   uint32_t has_key, uint32_t head_dim, uint32_t rope_stride,
                                   float epsilon);
hipError_t launch_rope_half_f32(hipStream_t stream, const float* x, const float* cosine,
                                const float* sine, float* out, uint32_t tokens, uint32_t heads,
                                uint32_t head_dim, uint32_t rope_stride);
hipError_t launch_rope_half_f16(hipStream_t stream, const uint16_t* x, const float* cosine,
                                const float* sine, uint16_t* out, uint32_t tokens, uint32_t heads,
                                uint32_t head_dim, uint32_t rope_stride);
// Q and K (x0: heads0 heads, x1: heads1 heads) of the same tokens in one
// launch, sharing the cos/sin rows; heads1 = 0 rotates x0 alone.
hipError_t launch_rope_half_pair_f32(hipStream_t stream, const float* x0, float* out0, uint32_t heads0,
                                     const float* x1, float* out1, uint32_t heads1, const float* cosine,
                                     const float* sine, uint32_t tokens, uint32_t head_dim, uint32_t rope_stride);
hipError_t launch_rope_half_pair_f16(hipStream_t stream, const uint16_t* x0, uint16_t* out0, uint32_t heads0,
                                     const uint16_t* x1, uint16_t* out1, uint32_t heads1, const float* cosine,
                                     const float* sine, uint32_t tokens, uint32_t head_dim, uint32_t rope_stride);
hipError_t launch_rope_interleaved_f32(hipStream_t stream, const float* x, const float* cosine,
                                       const float* sine, float* out, uint32_t rows,
                                       uint32_t hidden);

// Gated activations and elementwise ops (glu_kernels.hip).
enum EltOp : int {
    kEltSilu = 0,
    kEltGelu = 1,
    kEltSwiglu = 2,
    kEltGeglu = 3,
    kEltAdd = 4,
    kEltMul = 5,
    kEltScale = 6,
};
hipError_t launch_elementwise_f32(hipStream_t stream, EltOp op, const float* a, const float* b,
                                  float scalar, float* out, uint64_t n);
hipError_t launch_swiglu_f16(hipStream_t stream, const uint16_t* gate, const uint16_t* up,
                             uint16_t* out, uint64_t n);
hipError_t launch_geglu_offset_f32(hipStream_t stream, const float* gate, const float* ple,
                                   float* out, uint32_t ple_offset, uint32_t ple_row_stride,
                                   uint32_t width, uint32_t rows);

// Gathers (gather_kernels.hip).
hipError_t launch_embed_f32(hipStream_t stream, const float* table, const uint32_t* ids,
                            float* out, uint32_t vocab, uint32_t hidden, uint32_t tokens,
                            float scale);
// format: 0 Q4_0 (18-byte blocks of 32), 1 Q6_K (210-byte blocks of 256),
// 2 Q8_0 (34-byte blocks of 32).  Rows with id >= vocab are left untouched.
hipError_t launch_embed_quant(hipStream_t stream, int format, const uint8_t* table,
                              const uint32_t* ids, float* out, uint32_t vocab, uint32_t hidden,
                              uint32_t tokens, float scale);
hipError_t launch_ple_quant(hipStream_t stream, int q6k, const uint8_t* table, const uint32_t* ids,
                            const float* projection, float* out, uint32_t vocab, uint32_t layers,
                            uint32_t width, uint32_t tokens, float embedding_scale,
                            float output_scale);

// RMS-folded Q4_0 projections of one token (matvec_kernels.hip).  Up to
// three projections of the same input share one launch (fused QKV, fused
// gate/up); rms_weight == nullptr gives the plain matvec.
struct MatvecArgs {
    const float* input;
    const float* rms_weight;
    // epilogue: out = gelu_tanh(total) * ple[ple_offset + row] when ple is set
    // (the PLE input gate); otherwise out = total (* inv_rms with rms_weight)
    const float* ple;
    uint32_t ple_offset;
    float epsilon;
    uint32_t input_width;  // multiple of 32, <= q4_0_matvec_max_input()
    uint32_t segments;     // 1..3
    const uint8_t* weights[3];
    float* output[3];
    uint32_t width[3];
    uint32_t tile_begin[3];  // filled by the launcher
};
uint32_t q4_0_matvec_max_input();
hipError_t launch_q4_0_matvec(hipStream_t stream, MatvecArgs a);

// The PLE projection of one decode token and its norm (matvec_kernels.hip,
// then the stable group norm of norm_kernels.hip in place):
// out = stable_group_rms_norm(scale * (W . input)), W [groups * width, hidden] F16.
struct PleProjArgs {
    const float* input;        // [hidden], 16-byte aligned
    const uint16_t* weights;   // [groups * width, hidden] F16 bits, 16-byte aligned
    const float* norm_weight;  // [width]
    float* output;             // [groups * width]
    uint32_t hidden;           // multiple of 8, <= ple_projection_max_hidden()
    uint32_t width;            // multiple of 16, <= 1024
    uint32_t groups;           // <= ple_projection_max_groups()
    float scale;
    float epsilon;
};
uint32_t ple_projection_max_hidden();
uint32_t ple_projection_max_groups();
hipError_t launch_ple_projection_f16(hipStream_t stream, const PleProjArgs& a);

// KV-cache append with optional fused V RMSNorm (kv_kernels.hip).
enum KvFormat : int { kKvF32 = 0, kKvQ8_0 = 1, kKvQ4_0 = 2 };
struct KvAppendArgs {
    const float* key;           // [tokens, kv_width]
    const float* value;         // [tokens, kv_width]
    uint8_t* cache;             // [K | V][capacity][row]
    const uint32_t* positions;  // [tokens] cache position of each token (device)
    uint32_t kv_width;          // <= 4096; multiple of 32 for Q8_0/Q4_0
    uint32_t capacity;
    uint32_t tokens;
    float epsilon;
};
hipError_t launch_kv_append(hipStream_t stream, int format, bool vnorm, const KvAppendArgs& a);

// Logit soft cap and argmax (logits_kernels.hip).  The argmax of a row split
// over several workgroups goes through a workspace owned by the context:
// one 64-bit slot per workgroup (at most kArgmaxSlotsPerRow per row), written
// by the streaming launch and reduced by a second launch; every slot read is
// written by the same call first, so the workspace needs no clearing.
constexpr uint32_t kArgmaxSlotsPerRow = 256;
constexpr uint32_t kArgmaxSlots = 65536;  // 512 KiB
size_t argmax_workspace_bytes();
// cap > 0: capped = cap * tanh(logits / cap) (capped may alias logits or be
// null when only the argmax is wanted); selected != null: selected[r] =
// argmax of row r of the (capped) logits.  rows x count values, count >= 1.
// workspace holds slot_count 64-bit slots; rows are split over as many
// launches as that needs.
hipError_t launch_logits_f32(hipStream_t stream, const float* logits, float* capped, uint32_t* selected,
                             uint32_t rows, uint32_t count, float cap, void* workspace, uint32_t slot_count);
// Launches launch_logits_f32 makes for these operands with slot_count slots
// (0 if a row needs more slots than that).
uint32_t logits_launches(const float* logits, const float* capped, uint32_t rows, uint32_t count,
                         uint32_t slot_count);
// Workgroups per row of launch_logits_f32 for these operands: with one, the
// argmax is written directly and the workspace is not used.
uint32_t logits_row_blocks(const float* logits, const float* capped, uint32_t rows, uint32_t count);
// The library's static scratch for the no-allocation soft cap + argmax:
// kArgmaxScratchSlots slots (128 KiB per GPU).  argmax_scratch_address gives
// the current device's copy (hipGetSymbolAddress).
constexpr uint32_t kArgmaxScratchSlots = 16384;
hipError_t argmax_scratch_address(void** ptr);
hipError_t launch_softcap_f32(hipStream_t stream, const float* in, float* out, uint64_t n, float cap);

}  // namespace atlas
