// neural_ops_test.cpp -- the C++ operator API (include/atlas_neural_ops.hpp)
// exercised the way the reference tests its NeuralOps
// (crates/atlas-ops/tests/phase_02_operators.rs): the same known-answer
// inputs, the same inline CPU oracles and tolerances, the NoDevice skip; plus
// bit-exact comparisons against the CPU oracle library (oracle/), the
// reference's InvalidInput predicates, and one resident (device-pointer) call
// with the aliased bindings of the Gemma decode site.
//
// Exit status 0 = all checks passed (or skipped for want of a device, unless
// --require-device is given).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <string>
#include <vector>

#include "atlas_gguf.hpp"
#include "atlas_neural_ops.hpp"
#include "atlas_oracle.h"

namespace {

int failures = 0;

void fail(const std::string& what) {
    std::fprintf(stderr, "FAIL: %s\n", what.c_str());
    ++failures;
}

// assert_close (phase_02_operators.rs:21-40): finite, |actual - expected| <= tolerance.
void assert_close(const char* op, const std::vector<float>& actual, const std::vector<float>& expected,
                  float tolerance) {
    if (actual.size() != expected.size()) return fail(std::string(op) + ": output length");
    float max_abs = 0.0f;
    for (size_t i = 0; i < actual.size(); ++i) {
        if (!std::isfinite(actual[i])) return fail(std::string(op) + ": non-finite output");
        const float d = std::fabs(actual[i] - expected[i]);
        max_abs = std::fmax(max_abs, d);
        if (d > tolerance) return fail(std::string(op) + ": differs by " + std::to_string(d));
    }
    std::fprintf(stderr, "%s: max_abs=%.7f tolerance=%.7f\n", op, max_abs, tolerance);
}

void assert_bits(const char* op, const std::vector<float>& actual, const std::vector<float>& expected) {
    if (actual.size() != expected.size() || std::memcmp(actual.data(), expected.data(), 4 * actual.size()) != 0)
        return fail(std::string(op) + ": not bit-identical to the CPU oracle");
    std::fprintf(stderr, "%s: bit-identical (%zu values)\n", op, actual.size());
}

void expect_invalid(const char* what, const std::function<void()>& call) {
    try {
        call();
    } catch (const atlas::OperatorError& e) {
        if (e.kind() == atlas::ErrorKind::InvalidInput) {
            std::fprintf(stderr, "%s: InvalidInput (%s)\n", what, e.what());
            return;
        }
        return fail(std::string(what) + ": wrong error kind: " + e.what());
    }
    fail(std::string(what) + ": accepted invalid input");
}

// cpu_rms_norm (phase_02_operators.rs:223-242).
std::vector<float> cpu_rms_norm(const std::vector<float>& input, size_t rows, size_t hidden,
                                const std::vector<float>& weight, float epsilon) {
    std::vector<float> out;
    for (size_t r = 0; r < rows; ++r) {
        float sum = 0.0f;
        for (size_t i = 0; i < hidden; ++i) sum += input[r * hidden + i] * input[r * hidden + i];
        const float inverse = 1.0f / std::sqrt(sum / static_cast<float>(hidden) + epsilon);
        for (size_t i = 0; i < hidden; ++i) out.push_back(input[r * hidden + i] * inverse * weight[i]);
    }
    return out;
}

// cpu_rope (phase_02_operators.rs:262-272): interleaved pairs.
std::vector<float> cpu_rope(const std::vector<float>& input, size_t rows, size_t hidden,
                            const std::vector<float>& cosine, const std::vector<float>& sine) {
    std::vector<float> out(input.size());
    for (size_t r = 0; r < rows; ++r)
        for (size_t p = 0; p < hidden / 2; ++p) {
            const size_t b = r * hidden + 2 * p;
            out[b] = input[b] * cosine[p] - input[b + 1] * sine[p];
            out[b + 1] = input[b] * sine[p] + input[b + 1] * cosine[p];
        }
    return out;
}

std::vector<float> normal(std::mt19937& g, size_t n, float mean = 0.0f, float std = 1.0f) {
    std::normal_distribution<float> d(mean, std);
    std::vector<float> v(n);
    for (auto& x : v) x = d(g);
    return v;
}

// fp32_neural_operators_match_cpu_oracles_for_prefill_and_decode
// (phase_02_operators.rs:42-190), the operators on this path.
void reference_known_answers(const atlas::NeuralOps& ops) {
    const std::vector<float> table = {0.0f, 0.1f, 0.2f, 0.3f, 1.0f, 1.1f, 1.2f, 1.3f, 2.0f, 2.1f, 2.2f, 2.3f};
    const std::vector<uint32_t> ids = {2, 0};
    assert_close("embedding", ops.embedding(table, 3, 4, ids).first,
                 {2.0f, 2.1f, 2.2f, 2.3f, 0.0f, 0.1f, 0.2f, 0.3f}, 1e-6f);

    const std::vector<float> lhs = {1.0f, -2.0f, 3.0f, -4.0f};
    const std::vector<float> rhs = {0.5f, 0.25f, -1.0f, -2.0f};
    assert_close("add", ops.add(lhs, rhs).first, {1.5f, -1.75f, 2.0f, -6.0f}, 1e-6f);
    assert_close("multiply", ops.multiply(lhs, rhs).first, {0.5f, -0.5f, -3.0f, 8.0f}, 1e-6f);
    std::vector<float> silu_expected;
    for (float v : lhs) silu_expected.push_back(v / (1.0f + std::exp(-v)));
    assert_close("silu", ops.silu(lhs).first, silu_expected, 1e-6f);

    const std::vector<float> norm_input = {1.0f, 2.0f, 3.0f, 4.0f, -1.0f, 0.5f, 2.0f, -2.5f};
    const std::vector<float> norm_weight = {1.0f, 0.5f, 1.5f, 2.0f};
    assert_close("rms_norm", ops.rms_norm(norm_input, 2, 4, norm_weight, 1e-5f).first,
                 cpu_rms_norm(norm_input, 2, 4, norm_weight, 1e-5f), 1e-5f);

    const std::vector<float> cosine = {0.5f, 0.25f}, sine = {0.25f, 0.5f};
    assert_close("rope", ops.rope(norm_input, 2, 4, cosine, sine).first,
                 cpu_rope(norm_input, 2, 4, cosine, sine), 1e-6f);
}

// first_layer_rms_norm_weights_match_the_cpu_oracle (phase_02_operators.rs:196-217):
// the SmolLM2-135M input_layernorm width with synthetic weights (the model
// fixture is downloaded by the reference's scripts and is not available here).
void first_layer_rms_norm(const atlas::NeuralOps& ops) {
    std::mt19937 g(576);
    const std::vector<float> weights = normal(g, 576, 1.0f, 0.1f);
    std::vector<float> input(576);
    for (size_t i = 0; i < input.size(); ++i) input[i] = std::sin(static_cast<float>(i) * 0.013f);
    assert_close("first_layer_rms_norm", ops.rms_norm(input, 1, 576, weights, 1e-5f).first,
                 cpu_rms_norm(input, 1, 576, weights, 1e-5f), 1e-5f);
}

void bit_exact_against_oracle(const atlas::NeuralOps& ops) {
    std::mt19937 g(2024);
    const size_t rows = 37, hidden = 1536;
    const std::vector<float> x = normal(g, rows * hidden), w = normal(g, hidden, 1.0f, 0.1f);
    std::vector<float> expect(rows * hidden);
    oracle_rms_norm_f32(x.data(), w.data(), expect.data(), rows, hidden, 1e-6f);
    // the default reduction (ATLAS_REDUCTION_AUTO) sums a plain RMSNorm's
    // squares as a tree: within 1e-5 relative of the sequential CPU fold ...
    const std::vector<float> tree = ops.rms_norm(x, rows, hidden, w, 1e-6f).first;
    for (size_t i = 0; i < tree.size(); ++i)
        if (!(std::fabs(tree[i] - expect[i]) <= 1e-5f * std::fabs(expect[i]))) {
            fail("rms_norm[37x1536] (auto): beyond 1e-5 relative of the CPU oracle");
            break;
        }
    // ... and the sequential reduction reproduces the fold's bits
    ops.check(atlas_hip_set_reduction(ops.runtime(), ATLAS_REDUCTION_SEQUENTIAL));
    assert_bits("rms_norm[37x1536] (sequential)", ops.rms_norm(x, rows, hidden, w, 1e-6f).first, expect);
    ops.check(atlas_hip_set_reduction(ops.runtime(), ATLAS_REDUCTION_AUTO));

    const std::vector<float> c = normal(g, hidden / 2), s = normal(g, hidden / 2);
    oracle_rope_interleaved_f32(x.data(), rows, hidden, c.data(), s.data(), expect.data());
    assert_bits("rope[37x1536]", ops.rope(x, rows, hidden, c, s).first, expect);

    std::vector<float> act(x.size());
    oracle_silu_f32(x.data(), act.data(), x.size());
    assert_bits("silu", ops.silu(x).first, act);
    oracle_gelu_f32(x.data(), act.data(), x.size());
    assert_bits("gelu", ops.gelu(x).first, act);
}

// The reference's InvalidInput predicates (crates/atlas-metal/src/lib.rs:
// 1323-1346, 1368-1391, 1400-1408, 1444-1458, 1493-1500, 1705-1713).
void invalid_inputs(const atlas::NeuralOps& ops) {
    const std::vector<float> four = {1.0f, 2.0f, 3.0f, 4.0f}, three = {1.0f, 2.0f, 3.0f}, none;
    expect_invalid("add with unequal lengths", [&] { ops.add(four, three); });
    expect_invalid("multiply of empty vectors", [&] { ops.multiply(none, none); });
    expect_invalid("rms_norm with a short weight", [&] { ops.rms_norm(four, 1, 4, three, 1e-5f); });
    expect_invalid("rms_norm with zero epsilon", [&] { ops.rms_norm(four, 1, 4, four, 0.0f); });
    expect_invalid("rms_norm with zero rows", [&] { ops.rms_norm(none, 0, 4, four, 1e-5f); });
    expect_invalid("rope with an odd width", [&] { ops.rope(three, 1, 3, std::vector<float>{1.0f},
                                                            std::vector<float>{0.0f}); });
    const std::vector<float> table(12, 0.5f);
    expect_invalid("embedding with an out-of-range id",
                   [&] { ops.embedding(table, 3, 4, std::vector<uint32_t>{3}); });
    const std::vector<uint8_t> q6(210, 0);
    expect_invalid("Q6_K embedding with hidden % 256 != 0",
                   [&] { ops.embedding_lookup_q6_k(q6, 1, 128, std::vector<uint32_t>{0}); });
}

// One resident call: the Gemma decode post-attention epilogue binds
// input = normalized = work and residual = state (gemma4_executor.rs:4492-4506).
void resident_aliased_epilogue(const atlas::NeuralOps& ops) {
    std::mt19937 g(4492);
    const size_t rows = 8, hidden = 1536;
    const std::vector<float> work = normal(g, rows * hidden), state = normal(g, rows * hidden),
                             w = normal(g, hidden, 1.0f, 0.1f);
    std::vector<float> n_exp(rows * hidden), out_exp(rows * hidden);
    oracle_rms_norm_residual_f32(work.data(), w.data(), state.data(), n_exp.data(), out_exp.data(), rows, hidden,
                                 1e-6f);
    atlas::DeviceBuffer<float> dwork(ops, work), dstate(ops, state), dw(ops, w), dres(ops, rows * hidden);
    ops.check(atlas_hip_rms_norm_residual_f32(ops.runtime(), dwork.data(), dw.data(), dstate.data(), dwork.data(),
                                              dres.data(), rows, hidden, 1e-6f));
    ops.finish();
    assert_bits("resident rms_residual (normalized)", dwork.download(), n_exp);
    assert_bits("resident rms_residual (residual out)", dres.download(), out_exp);
}

// ---- GGUF (crates/atlas-core/tests/phase_11a_gguf.rs:99-120) -------------

// GgufWriter's layout (crates/atlas-core/src/gguf.rs:237-311), restated for
// the test: string metadata in key order, tensor infos, 32-byte aligned data.
std::vector<uint8_t> write_gguf(const std::vector<std::pair<std::string, std::string>>& metadata,
                                const std::string& name, const std::vector<uint64_t>& dims, uint32_t type,
                                const std::vector<uint8_t>& data) {
    std::vector<uint8_t> out;
    auto u32 = [&](uint32_t v) { for (int i = 0; i < 4; ++i) out.push_back(static_cast<uint8_t>(v >> (8 * i))); };
    auto u64 = [&](uint64_t v) { for (int i = 0; i < 8; ++i) out.push_back(static_cast<uint8_t>(v >> (8 * i))); };
    auto str = [&](const std::string& v) { u64(v.size()); out.insert(out.end(), v.begin(), v.end()); };
    out.insert(out.end(), {'G', 'G', 'U', 'F'});
    u32(3);
    u64(1);
    u64(metadata.size());
    for (const auto& kv : metadata) {
        str(kv.first);
        u32(8);
        str(kv.second);
    }
    str(name);
    u32(static_cast<uint32_t>(dims.size()));
    for (uint64_t d : dims) u64(d);
    u32(type);
    u64(0);
    while (out.size() % 32) out.push_back(0);
    out.insert(out.end(), data.begin(), data.end());
    return out;
}

void gguf_reader() {
    // writer_and_reader_preserve_aligned_packed_tensors
    std::vector<uint8_t> q4(32 * 18);
    for (size_t i = 0; i < q4.size(); ++i) q4[i] = static_cast<uint8_t>(i * 7 + 3);
    const auto bytes = write_gguf({{"general.alignment", "32"}, {"general.architecture", "llama"},
                                   {"llama.block_count", "1"}},
                                  "blk.0.attn_q.weight", {32, 32}, 2, q4);
    try {
        const atlas::GgufModel m = atlas::GgufModel::from_bytes(bytes);
        if (m.metadata().at("general.architecture") != "llama") fail("gguf: architecture metadata");
        const atlas::GgufTensor& t = m.tensor("blk.0.attn_q.weight");
        if (t.tensor_type != atlas::GgufTensorType::Q4_0 || t.dims != std::vector<uint64_t>{32, 32})
            fail("gguf: tensor info");
        const auto data = m.tensor_data(t);
        if (data.second != 32 * 18 || std::memcmp(data.first, q4.data(), q4.size()) != 0) fail("gguf: tensor data");
    } catch (const std::exception& e) {
        fail(std::string("gguf: valid file rejected: ") + e.what());
    }
    // malformed_gguf_is_rejected_before_tensor_access
    expect_invalid("truncated GGUF header", [] { atlas::GgufModel::from_bytes({'G', 'G', 'U', 'F', 3, 0, 0, 0}); });
    auto bad_align = write_gguf({{"general.alignment", "64"}}, "t", {32}, 2, std::vector<uint8_t>(18));
    expect_invalid("GGUF alignment 64", [&] { atlas::GgufModel::from_bytes(bad_align); });
    auto q4_1 = write_gguf({}, "t", {32}, 3, std::vector<uint8_t>(20));
    expect_invalid("GGUF tensor type Q4_1", [&] { atlas::GgufModel::from_bytes(q4_1); });
    expect_invalid("missing GGUF file", [] { atlas::GgufModel::open("/nonexistent/model.gguf"); });
}

// argmax_reduction_preserves_large_vocabulary_and_highest_tie
// (crates/atlas-metal/src/lib.rs:2217-2230), through the device entry point.
void argmax_known_answer(const atlas::NeuralOps& ops) {
    std::vector<float> values(65537, -10.0f);
    values[7] = 3.5f;
    values[31111] = 9.0f;
    values[65536] = 9.0f;
    atlas::DeviceBuffer<float> dv(ops, values);
    atlas::DeviceBuffer<uint32_t> sel(ops, 1);
    ops.check(atlas_hip_argmax_f32(ops.runtime(), dv.data(), sel.data(), 1, static_cast<uint32_t>(values.size())));
    ops.finish();
    if (sel.download()[0] != 65536) fail("argmax: the later of two equal maxima must win");
}

}  // namespace

int main(int argc, char** argv) {
    const bool require_device = argc > 1 && std::strcmp(argv[1], "--require-device") == 0;
    gguf_reader();  // host only: runs with or without a device
    // require_ops (phase_02_operators.rs:8-19)
    atlas::NeuralOps* ops = nullptr;
    try {
        ops = new atlas::NeuralOps(0);
    } catch (const atlas::OperatorError& e) {
        if (e.kind() == atlas::ErrorKind::NoDevice) {
            std::fprintf(stderr, "skipping GPU operator assertions: no HIP device is available to this process\n");
            return require_device ? 2 : (failures ? 1 : 0);
        }
        std::fprintf(stderr, "operators should initialize: %s\n", e.what());
        return 1;
    }
    try {
        reference_known_answers(*ops);
        first_layer_rms_norm(*ops);
        bit_exact_against_oracle(*ops);
        invalid_inputs(*ops);
        resident_aliased_epilogue(*ops);
        argmax_known_answer(*ops);
    } catch (const std::exception& e) {
        fail(std::string("unexpected exception: ") + e.what());
    }
    delete ops;
    std::fprintf(stderr, failures ? "%d check(s) failed\n" : "all operator checks passed\n", failures);
    return failures ? 1 : 0;
}
