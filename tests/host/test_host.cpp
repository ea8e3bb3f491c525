// Tests of the C++ host interface (metal-candle_amd/host/mc_candle.hpp),
// written after the reference's own Rust tests, each citing the test it
// follows. Numerical results are compared with the CPU oracle (oracle/,
// linked here as the checker) on the same inputs and dropout masks.
//
//   test_host --cpu     cases that need no GPU (validation, error strings,
//                       configuration, graph operations, dropout masks)
//   test_host --gpu     every case (needs a HIP device)
//   test_host ... NAME  only cases whose name contains NAME
//
// Exit status 0 iff every selected case passed.
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <functional>
#include <random>
#include <string>
#include <vector>

#include "mc_candle.hpp"
#include "mc_hip.h"
#include "oracle.h"

using namespace mc_candle;

// ------------------------------------------------------------------ harness
namespace {

struct Case {
    const char* name;
    bool gpu;
    std::function<void()> fn;
};
std::vector<Case>& cases() {
    static std::vector<Case> c;
    return c;
}
struct Reg {
    Reg(const char* n, bool gpu, std::function<void()> f) { cases().push_back({n, gpu, std::move(f)}); }
};
int g_failures_in_case = 0;

void fail_at(int line, const std::string& what) {
    ++g_failures_in_case;
    printf("    line %d: %s\n", line, what.c_str());
    fflush(stdout);
}

#define CASE(name, gpu)                          \
    static void name();                          \
    static Reg reg_##name(#name, gpu, name);     \
    static void name()
#define CHECK(...)                                                    \
    do {                                                              \
        if (!(__VA_ARGS__)) fail_at(__LINE__, "CHECK(" #__VA_ARGS__ ")"); \
    } while (0)
#define CHECK_CONTAINS(s, sub)                                                             \
    do {                                                                                    \
        const std::string s_ = (s);                                                         \
        if (s_.find(sub) == std::string::npos)                                              \
            fail_at(__LINE__, std::string("\"") + s_ + "\" does not contain \"" + (sub) + "\""); \
    } while (0)
#define CHECK_LE(a, b)                                                                       \
    do {                                                                                      \
        const double a_ = (a), b_ = (b);                                                      \
        if (!(a_ <= b_)) fail_at(__LINE__, #a " = " + std::to_string(a_) + " > " + std::to_string(b_)); \
    } while (0)
// The text of an error value (the graph's errors are plain strings).
template <class E>
std::string err_text(const E& e) { return e.to_string(); }
inline std::string err_text(const std::string& e) { return e; }
// Unwraps a Result or fails the case (and returns from it).
#define TRY(var, expr)                                                              \
    auto var##_r = (expr);                                                          \
    if (var##_r.is_err()) {                                                         \
        fail_at(__LINE__, std::string(#expr " failed: ") + err_text(var##_r.error())); \
        return;                                                                     \
    }                                                                               \
    auto var = std::move(var##_r.value())

const Device kHip = Device::hip(0);
const Device kCpu = Device::cpu();

std::vector<float> randn(size_t n, float mean, float std, uint64_t seed) {
    std::mt19937_64 g(seed);
    std::normal_distribution<float> d(mean, std);
    std::vector<float> v(n);
    for (float& x : v) x = d(g);
    return v;
}

std::vector<float> ones(size_t n) { return std::vector<float>(n, 1.f); }

// max|a - b| / max|b| (the tolerance measure of the parity bar).
double rel_err(const std::vector<float>& a, const std::vector<float>& b) {
    double num = 0, den = 0;
    for (size_t i = 0; i < a.size() && i < b.size(); ++i) {
        num = fmax(num, fabs((double)a[i] - b[i]));
        den = fmax(den, fabs((double)b[i]));
    }
    return a.size() != b.size() ? 1e30 : num / (den > 0 ? den : 1.0);
}

std::vector<float> round_bf16(const std::vector<float>& v) {
    std::vector<float> o(v.size());
    oracle_round_bf16(v.data(), o.data(), (int64_t)v.size());
    return o;
}

std::vector<float> transpose(const std::vector<float>& m, int64_t rows, int64_t cols) {
    std::vector<float> t(m.size());
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < cols; ++j) t[(size_t)(j * rows + i)] = m[(size_t)(i * cols + j)];
    return t;
}

constexpr double kTolF32 = 1e-5;
constexpr double kTolBf16 = 2e-2;

}  // namespace

// ================================================================== CPU cases
// lora.rs:571-604 (tests module): defaults and scaling().
CASE(lora_config_default_and_scaling, false) {
    LoRAConfig c;
    CHECK(c.rank == 8 && c.alpha == 16.f && c.dropout == 0.f);
    CHECK(c.scaling() == 2.f);
    LoRAConfig d{4, 8.f, 0.f};
    CHECK(d.scaling() == 2.f);
    CHECK(c.validate().is_ok());
}

// lora.rs:97-120: validation messages, and the crate Error display.
CASE(lora_config_validation_messages, false) {
    auto r0 = LoRAConfig{0, 16.f, 0.f}.validate();
    CHECK(r0.is_err());
    if (r0.is_err()) {
        CHECK_CONTAINS(r0.error().to_string(), "LoRA rank must be greater than 0");
        CHECK(r0.error().to_string() ==
              "training error: invalid training configuration: LoRA rank must be greater than 0");
    }
    auto ra = LoRAConfig{8, 0.f, 0.f}.validate();
    CHECK(ra.is_err());
    if (ra.is_err()) CHECK_CONTAINS(ra.error().to_string(), "LoRA alpha must be positive");
    for (float p : {1.0f, -0.1f, 1.5f}) {
        auto rp = LoRAConfig{8, 16.f, p}.validate();
        CHECK(rp.is_err());
        if (rp.is_err()) CHECK_CONTAINS(rp.error().to_string(), "LoRA dropout must be in [0, 1)");
    }
    CHECK(LoRAConfig{8, 16.f, 0.99f}.validate().is_ok());
}

// lora.rs:214-228: rank above min(in, out).
CASE(lora_layer_rank_exceeds_maximum, false) {
    auto r = LoRALayer::create(16, 8, LoRAConfig{16, 32.f, 0.f}, kCpu);
    CHECK(r.is_err());
    if (r.is_err())
        CHECK_CONTAINS(r.error().to_string(),
                       "LoRA rank 16 exceeds maximum rank 8 (min of in_features=16, out_features=8)");
}

// lora.rs:694-707: num_parameters = r (K + N); lora.rs:233-247: shapes, B = 0.
CASE(lora_layer_parameters_and_init, false) {
    TRY(layer, LoRALayer::create(768, 768, LoRAConfig{8, 16.f, 0.f}, kCpu));
    CHECK(layer.num_parameters() == 12288);
    CHECK((layer.lora_a_tensor().dims() == std::vector<int64_t>{768, 8}));
    CHECK((layer.lora_b_tensor().dims() == std::vector<int64_t>{8, 768}));
    TRY(b, layer.lora_b_tensor().to_vec_f32());
    bool all_zero = true;
    for (float v : b) all_zero &= v == 0.f;
    CHECK(all_zero);
    // A ~ N(0, 1/sqrt(8)): sample std within 5% of 0.3536.
    TRY(a, layer.lora_a_tensor().to_vec_f32());
    double s2 = 0;
    for (float v : a) s2 += (double)v * v;
    CHECK(fabs(sqrt(s2 / a.size()) - 1.0 / sqrt(8.0)) < 0.05 / sqrt(8.0));
}

// lora_dropout.rs:102-131: training mode is the default; set_training / eval.
CASE(lora_layer_training_mode, false) {
    TRY(layer, LoRALayer::create(32, 32, LoRAConfig{8, 16.f, 0.1f}, kCpu));
    CHECK(layer.is_training());
    layer.eval();
    CHECK(!layer.is_training());
    layer.set_training(true);
    CHECK(layer.is_training());
    layer.set_training(false);
    CHECK(!layer.is_training());
}

// lora.rs:302-310: the reference layer falls back to the candle composite on
// any Err of the fused op. The mirror has no CPU path: a CPU input gives the
// op's HIP-only error, which the caller's fallback then handles.
CASE(lora_layer_cpu_input_is_an_error, false) {
    TRY(layer, LoRALayer::create(32, 32, LoRAConfig{8, 16.f, 0.f}, kCpu));
    TRY(x, Tensor::from_slice(ones(4 * 32), {4, 32}, kCpu));
    auto y = layer.forward(x);
    CHECK(y.is_err());
    if (y.is_err()) CHECK_CONTAINS(y.error().to_string(), "FusedLoRAOp is HIP-only");
}

// custom_ops.rs:118-150: FusedLoRAOp::new validation.
CASE(fused_lora_op_new_validation, false) {
    TRY(a3, Tensor::zeros({2, 4, 2}, DType::F32, kCpu));
    TRY(a, Tensor::zeros({4, 2}, DType::F32, kCpu));
    TRY(b, Tensor::zeros({2, 4}, DType::F32, kCpu));
    TRY(b_bad, Tensor::zeros({3, 4}, DType::F32, kCpu));
    auto r1 = FusedLoRAOp::create(a3, b, 1.f);
    CHECK(r1.is_err());
    if (r1.is_err()) CHECK(r1.error().to_string() == "LoRA matrices must be 2D, got shapes [2, 4, 2] and [2, 4]");
    auto r2 = FusedLoRAOp::create(a, b_bad, 1.f);
    CHECK(r2.is_err());
    if (r2.is_err()) CHECK(r2.error().to_string() == "Incompatible LoRA matrix dimensions: 4×2 and 3×4");
    CHECK(FusedLoRAOp::create(a, b, 2.f).is_ok());
}

// custom_ops.rs:231-233, 522-524, 715-717: op names.
CASE(op_names, false) {
    TRY(a, Tensor::zeros({4, 2}, DType::F32, kCpu));
    TRY(b, Tensor::zeros({2, 4}, DType::F32, kCpu));
    TRY(lo, FusedLoRAOp::create(a, b, 1.f));
    TRY(rn, FusedRMSNormOp::create(1e-5f));
    TRY(sm, FusedSoftmaxOp::create());
    CHECK(std::string(lo.name()) == "fused_lora_forward");
    CHECK(std::string(rn.name()) == "fused-rms-norm");
    CHECK(std::string(sm.name()) == "fused-softmax");
}

// custom_ops.rs:235-245, 526-532, 719-725: the CPU forward bails; the
// CustomMetalOps wrappers map it to TrainingError::Failed (metal_ops.rs:127-170).
CASE(cpu_forward_bails_with_reference_messages, false) {
    TRY(x, Tensor::from_slice(ones(8), {2, 4}, kCpu));
    TRY(a, Tensor::zeros({4, 2}, DType::F32, kCpu));
    TRY(b, Tensor::zeros({2, 4}, DType::F32, kCpu));
    auto l = lora_forward_fused(x, a, b, 1.f);
    CHECK(l.is_err());
    if (l.is_err()) {
        CHECK_CONTAINS(l.error().to_string(), "training failed: Failed to apply fused LoRA op: FusedLoRAOp is HIP-only");
    }
    auto s = softmax_fused(x);
    CHECK(s.is_err());
    if (s.is_err()) CHECK_CONTAINS(s.error().to_string(), "Fused Softmax kernel execution failed: Fused Softmax kernel not implemented for CPU");
    auto r = rms_norm_fused(x, 1e-5f);
    CHECK(r.is_err());
    if (r.is_err()) CHECK_CONTAINS(r.error().to_string(), "Fused RMS Norm kernel execution failed: Fused RMS Norm kernel not implemented for CPU");
    auto l2 = lora_forward_fused(x, b, a, 1.f);  // A [2,4] with B [4,2]: fine shapes, wrong K
    CHECK(l2.is_err());
}

// executor_direct.rs:11-16, 499-506.
CASE(executor_creation_and_debug, false) {
    TRY(ex, AsyncExecutor::create(kCpu));
    CHECK(ex.synchronize().is_ok());
    CHECK_CONTAINS(ex.debug_string(), "AsyncExecutor");
    CHECK_CONTAINS(ex.debug_string(), "device");
}

// executor_direct.rs:18-121, 180-249, 293-337, 415-432: error strings.
CASE(executor_input_and_count_errors, false) {
    TRY(ex, AsyncExecutor::create(kCpu));
    TRY(t, Tensor::from_slice({1.f, 2.f}, {2}, kCpu));
    auto expect = [&](const Operation& op, size_t n, const char* msg, int line) {
        std::vector<Tensor> in(n, t);
        auto r = ex.execute_operation(op, in);
        if (!r.is_err()) {
            fail_at(line, std::string(op.name()) + " with " + std::to_string(n) + " inputs did not fail");
        } else if (r.error().to_string().find(msg) == std::string::npos) {
            fail_at(line, "\"" + r.error().to_string() + "\" does not contain \"" + msg + "\"");
        }
    };
    expect(Operation::input(), 1, "Cannot execute Input operation", __LINE__);
    for (size_t n : {1, 3}) expect(Operation::matmul(), n, "Matmul requires 2 inputs", __LINE__);
    for (size_t n : {1, 3}) expect(Operation::add(), n, "Add requires 2 inputs", __LINE__);
    for (size_t n : {1, 3}) expect(Operation::mul(), n, "Mul requires 2 inputs", __LINE__);
    for (size_t n : {0, 2}) expect(Operation::mul_scalar(2.5f), n, "MulScalar requires 1 input", __LINE__);
    for (size_t n : {0, 2}) expect(Operation::softmax(0), n, "Softmax requires 1 input", __LINE__);
    for (size_t n : {0, 2}) expect(Operation::rms_norm(1e-5f), n, "RMSNorm requires 1 input", __LINE__);
    for (size_t n : {1, 2, 4}) expect(Operation::lora(NodeId{0}, NodeId{1}, 1.f), n, "LoRA requires 3 inputs", __LINE__);
}

// operation.rs:49-160: names and output shapes.
CASE(operation_names_and_shapes, false) {
    CHECK(std::string(Operation::input().name()) == "input");
    CHECK(std::string(Operation::mul_scalar(1.f).name()) == "mul_scalar");
    CHECK(std::string(Operation::lora(NodeId{0}, NodeId{1}, 1.f).name()) == "lora");
    CHECK(std::string(Operation::softmax(1).name()) == "softmax");
    CHECK(std::string(Operation::rms_norm(1e-5f).name()) == "rms_norm");
    auto mm = Operation::matmul().output_shape({{2, 3}, {3, 4}});
    CHECK(mm.is_ok() && (mm.value() == std::vector<int64_t>{2, 4}));
    auto bad = Operation::matmul().output_shape({{2, 3}, {2, 4}});
    CHECK(bad.is_err());
    if (bad.is_err()) CHECK(bad.error() == "Matmul dimension mismatch: 2×3 @ 2×4");
    auto lo = Operation::lora(NodeId{0}, NodeId{1}, 1.f).output_shape({{2, 5, 4}, {4, 2}, {2, 6}});
    CHECK(lo.is_ok() && (lo.value() == std::vector<int64_t>{2, 5, 6}));
    auto lo_bad = Operation::lora(NodeId{0}, NodeId{1}, 1.f).output_shape({{2, 4}, {4, 2}});
    CHECK(lo_bad.is_err());
    if (lo_bad.is_err()) CHECK(lo_bad.error() == "LoRA requires 3 inputs (input, a, b), got 2");
    auto add_bad = Operation::add().output_shape({{3}, {4}});
    CHECK(add_bad.is_err());
    if (add_bad.is_err()) CHECK(add_bad.error() == "Shape mismatch: [3] vs [4]");
}

// node.rs:363-458 (tests module): graph creation, nodes, order, shape
// inference and the errors of unknown nodes.
CASE(graph_nodes_order_and_errors, false) {
    ComputationGraph g(kCpu);
    CHECK(g.len() == 0 && g.is_empty());
    TRY(a, Tensor::zeros({2, 3}, DType::F32, kCpu));
    TRY(b, Tensor::zeros({2, 3}, DType::F32, kCpu));
    TRY(m, Tensor::zeros({3, 4}, DType::F32, kCpu));
    const NodeId ia = g.add_input(a), ib = g.add_input(b), im = g.add_input(m);
    CHECK(ia.id == 0 && ib.id == 1 && g.len() == 3);
    TRY(ic, g.add_node(Operation::add(), {ia, ib}));
    CHECK(ic.id == 3);
    TRY(nc, g.get_node(ic));
    CHECK(nc->inputs.size() == 2 && nc->inputs[0].id == ia.id && nc->inputs[1].id == ib.id);
    CHECK(!nc->is_available());
    TRY(na, g.get_node(ia));
    CHECK(na->is_available() && na->data == GraphNode::Data::Concrete);
    // a diamond: d = (a + b) * a; dependencies come first, each node once
    TRY(id, g.add_node(Operation::mul(), {ic, ia}));
    TRY(order, g.topological_order(id));
    CHECK(order.size() == 4);
    if (order.size() == 4) CHECK(order[0].id == ia.id && order[1].id == ib.id && order[2].id == ic.id && order[3].id == id.id);
    TRY(mm, g.add_node(Operation::matmul(), {ia, im}));
    TRY(nmm, g.get_node(mm));
    CHECK((nmm->output_shape == std::vector<int64_t>{2, 4}));
    CHECK(nmm->output_dtype == DType::F32);
    auto bad = g.add_node(Operation::add(), {ia, im});
    CHECK(bad.is_err());
    if (bad.is_err()) CHECK(bad.error() == "Shape mismatch: [2, 3] vs [3, 4]");
    auto unknown = g.add_node(Operation::mul_scalar(2.f), {NodeId{99}});
    CHECK(unknown.is_err());
    if (unknown.is_err()) CHECK(unknown.error() == "Input node NodeId(99) not found");
    auto missing = g.get_node(NodeId{999});
    CHECK(missing.is_err());
    if (missing.is_err()) CHECK(missing.error() == "Node NodeId(999) not found");
    CHECK(g.get_node_mut(NodeId{999}).is_err());
}

// node.rs:461-543: merging a node of another graph copies it and everything
// it depends on, inputs renumbered, values kept.
CASE(graph_merge_copies_dependencies, false) {
    ComputationGraph g1(kCpu), g2(kCpu);
    TRY(ta, Tensor::from_slice({1.f, 2.f}, {2}, kCpu));
    TRY(tb, Tensor::from_slice({3.f, 4.f}, {2}, kCpu));
    TRY(tc, Tensor::from_slice({5.f, 6.f}, {2}, kCpu));
    g1.add_input(ta);
    const NodeId b = g2.add_input(tb), c = g2.add_input(tc);
    TRY(d, g2.add_node(Operation::add(), {b, c}));
    const NodeId nd = g1.merge_from(g2, d);
    CHECK(g1.len() == 4 && g2.len() == 3);
    TRY(n, g1.get_node(nd));
    CHECK(n->inputs.size() == 2);
    if (n->inputs.size() == 2) {
        TRY(nb, g1.get_node(n->inputs[0]));
        CHECK(nb->is_available() && nb->tensor.data() == tb.data());  // the same storage, as Arc'd tensors
        CHECK(n->inputs[0].id >= 1 && n->inputs[1].id >= 1);
    }
    // a chain b -> c -> d -> e: merging e brings all four
    ComputationGraph g3(kCpu), g4(kCpu);
    g3.add_input(ta);
    const NodeId e0 = g4.add_input(tb);
    TRY(e1, g4.add_node(Operation::mul_scalar(2.f), {e0}));
    TRY(e2, g4.add_node(Operation::mul_scalar(3.f), {e1}));
    TRY(e3, g4.add_node(Operation::mul_scalar(4.f), {e2}));
    const NodeId ne = g3.merge_from(g4, e3);
    CHECK(g3.len() == 5);
    TRY(order, g3.topological_order(ne));
    CHECK(order.size() == 4);
}

// lazy_tensor.rs:466-530 and lazy_execution.rs:104-170: graph sharing and
// merging, shapes and dtypes known before evaluation.
CASE(lazy_tensor_graphs_and_shapes, false) {
    TRY(a, LazyTensor::from_slice({1.f, 2.f}, {2}, kCpu));
    TRY(b, a.mul_scalar(2.f));
    CHECK(a.shares_graph_with(b) && a.graph_size() == 2);
    TRY(c, a.add(b));  // same graph: no merge
    CHECK(a.graph_size() == 3);
    TRY(x, LazyTensor::from_slice({3.f, 4.f}, {2}, kCpu));
    CHECK(!a.shares_graph_with(x) && x.graph_size() == 1);
    TRY(y, a.add(x));  // x's node is copied into a's graph
    CHECK(a.graph_size() == 5 && x.graph_size() == 1 && y.shares_graph_with(a));
    TRY(m1, LazyTensor::zeros({4, 3}, DType::F32, kCpu));
    TRY(m2, LazyTensor::ones({3, 5}, DType::F32, kCpu));
    TRY(p, m1.matmul(m2));
    CHECK((p.shape() == std::vector<int64_t>{4, 5}) && p.dtype() == DType::F32);
    auto bad = m1.add(m2);
    CHECK(bad.is_err());
    if (bad.is_err()) CHECK(bad.error().msg == "Shape mismatch: [4, 3] vs [3, 5]");
    CHECK(m1.is_evaluated() && !p.is_evaluated());
    TRY(s, p.softmax(1));
    TRY(r, s.rms_norm(1e-5f));
    CHECK((r.shape() == std::vector<int64_t>{4, 5}));
    CHECK_CONTAINS(r.debug_string(), "LazyTensor { node_id: NodeId(");
    CHECK_CONTAINS(r.debug_string(), "shape: [4, 5]");
    (void)c;
}

// lora_lazy.rs:10-160 run on the CPU device: forward_lazy records the
// reference's composite (input A) B * scaling, whose generic ops only candle
// runs, so eval gives the executor's error and the caller's fallback applies.
CASE(lora_forward_lazy_on_cpu_records_the_composite, false) {
    TRY(layer, LoRALayer::create(32, 48, LoRAConfig{4, 8.f, 0.f}, kCpu));
    TRY(x, LazyTensor::zeros({4, 32}, DType::F32, kCpu));
    TRY(y, layer.forward_lazy(x));
    CHECK(y.graph_size() == 6);  // x, A, B, x A, (x A) B, * scaling
    CHECK((y.shape() == std::vector<int64_t>{4, 48}));
    auto v = y.eval();
    CHECK(v.is_err());
    if (v.is_err()) CHECK_CONTAINS(v.error().to_string(), "Matmul is a generic candle op");
}

// The keep-mask generator of the C ABI equals the oracle's, byte for byte.
CASE(dropout_mask_matches_oracle, false) {
    const int64_t T = 1000;
    const int32_t r = 64;
    std::vector<uint8_t> a((size_t)T * r), b((size_t)T * r);
    CHECK(mc_dropout_mask(1234, 0.1f, T, r, a.data()) == MC_OK);
    oracle_dropout_mask(1234, 0.1f, T, r, b.data());
    CHECK(a == b);
    size_t kept = 0;
    for (uint8_t v : a) kept += v;
    CHECK(fabs((double)kept / a.size() - 0.9) < 0.01);
}

// ================================================================== GPU cases
// executor_direct.rs:339-373: the executor's LoRA on the reference's fixed
// inputs; the reference asserts shape and non-zero only, here the
// hand-derived values are asserted too.
CASE(executor_lora_known_answer, true) {
    TRY(ex, AsyncExecutor::create(kHip));
    TRY(x, Tensor::from_slice({1, 2, 3, 4, 5, 6, 7, 8}, {2, 4}, kHip));
    TRY(a, Tensor::from_slice({.1f, .2f, .3f, .4f, .5f, .6f, .7f, .8f}, {4, 2}, kHip));
    TRY(b, Tensor::from_slice({1, 2, 3, 4, 5, 6, 7, 8}, {2, 4}, kHip));
    TRY(y, ex.execute_operation(Operation::lora(NodeId{0}, NodeId{1}, 0.5f), {x, a, b}));
    CHECK((y.dims() == std::vector<int64_t>{2, 4}));
    TRY(v, y.to_vec_f32());
    const std::vector<float> want = {17.5f, 23.f, 28.5f, 34.f, 40.7f, 53.4f, 66.1f, 78.8f};
    CHECK_LE(rel_err(v, want), kTolF32);
    CHECK(ex.synchronize().is_ok());
}

// rmsnorm_lazy.rs:9-205, softmax_lazy.rs:12-250: the fused ops through the
// graph give the eager calls' results (the same kernels, bit for bit) and the
// oracle's; a node is evaluated once.
CASE(lazy_fused_ops_match_eager_and_oracle, true) {
    const int64_t rows = 4, D = 64;
    const std::vector<float> xv = randn(rows * D, 0.f, 1.f, 21);
    TRY(x, Tensor::from_slice(xv, {rows, D}, kHip));
    TRY(lx, LazyTensor::from_tensor(x));
    TRY(ln, lx.rms_norm(1e-5f));
    TRY(ls, ln.softmax(1));
    CHECK(!ls.is_evaluated() && ls.graph_size() == 3);
    TRY(got, ls.eval());
    CHECK(ls.is_evaluated() && ln.is_evaluated());
    TRY(e1, rms_norm_fused(x, 1e-5f));
    TRY(e2, softmax_fused(e1));
    TRY(vg, got.to_vec_f32());
    TRY(ve, e2.to_vec_f32());
    CHECK(vg == ve);
    std::vector<float> n((size_t)(rows * D)), p((size_t)(rows * D));
    oracle_rmsnorm_fwd(rows, D, 1e-5f, xv.data(), nullptr, n.data(), nullptr, 0);
    oracle_softmax_fwd(rows, D, 0, n.data(), p.data(), 0);
    CHECK_LE(rel_err(vg, p), kTolF32);
    TRY(again, ls.eval());  // nothing left to run: the stored value
    CHECK(again.data() == got.data());
    auto wrong_dim = lx.softmax(0);
    CHECK(wrong_dim.is_ok());
    if (wrong_dim.is_ok()) {
        auto r = wrong_dim.value().eval();
        CHECK(r.is_err());
        if (r.is_err()) CHECK_CONTAINS(r.error().to_string(), "only the last dimension has a fused kernel");
    }
}

// lora_lazy.rs:10-160 on the HIP device: forward_lazy is one fused LoRA node
// and its value equals forward's (the same op) and the oracle's; ranks 2-16,
// batched shapes, and a chain of two layers. B is set to random values (the
// reference's tests run with its zero initialisation).
CASE(lora_forward_lazy_matches_forward, true) {
    uint64_t seed = 100;
    for (size_t rank : {2, 4, 8, 16}) {
        TRY(layer, LoRALayer::create(64, 64, LoRAConfig{rank, 2.f * rank, 0.f}, kHip, seed));
        const std::vector<float> bv = randn(rank * 64, 0.f, 0.02f, seed + 1);
        TRY(bt, Tensor::from_slice(bv, {(int64_t)rank, 64}, kHip));
        CHECK(layer.set_lora_b(bt).is_ok());
        layer.eval();
        const std::vector<float> xv = randn(8 * 64, 0.f, 1.f, seed + 2);
        TRY(x, Tensor::from_slice(xv, {8, 64}, kHip));
        TRY(lx, LazyTensor::from_tensor(x));
        TRY(ly, layer.forward_lazy(lx));
        CHECK(ly.graph_size() == 4);  // x, A, B, lora
        TRY(y, ly.eval());
        TRY(ye, layer.forward(x));
        TRY(vy, y.to_vec_f32());
        TRY(ve, ye.to_vec_f32());
        CHECK(vy == ve);
        TRY(av, layer.lora_a_tensor().to_vec_f32());
        std::vector<float> ref(8 * 64);
        oracle_lora_fwd(8, 64, 64, (int32_t)rank, layer.config().scaling(), 0.f, xv.data(), nullptr, nullptr,
                        av.data(), bv.data(), nullptr, ref.data(), nullptr, 0);
        CHECK_LE(rel_err(vy, ref), kTolF32);
        seed += 10;
    }
    // shapes [batch, seq, 128] are kept (lora_lazy.rs:145-165)
    TRY(wide, LoRALayer::create(128, 128, LoRAConfig{}, kHip, 7));
    for (auto bs : {std::pair<int64_t, int64_t>{1, 10}, {4, 20}, {8, 5}}) {
        TRY(x, Tensor::from_slice(randn(bs.first * bs.second * 128, 0.f, 1.f, 9), {bs.first, bs.second, 128}, kHip));
        TRY(lx, LazyTensor::from_tensor(x));
        TRY(ly, wide.forward_lazy(lx));
        CHECK((ly.shape() == std::vector<int64_t>{bs.first, bs.second, 128}));
        TRY(y, ly.eval());
        CHECK((y.dims() == std::vector<int64_t>{bs.first, bs.second, 128}));
    }
    // two layers chained in one graph (lora_lazy.rs:81-112)
    TRY(l1, LoRALayer::create(32, 32, LoRAConfig{4, 8.f, 0.f}, kHip, 31));
    TRY(l2, LoRALayer::create(32, 32, LoRAConfig{4, 8.f, 0.f}, kHip, 32));
    for (LoRALayer* l : {&l1, &l2}) {
        TRY(bt, Tensor::from_slice(randn(4 * 32, 0.f, 0.05f, 33), {4, 32}, kHip));
        CHECK(l->set_lora_b(bt).is_ok());
        l->eval();
    }
    TRY(x, Tensor::from_slice(randn(4 * 32, 0.f, 1.f, 34), {4, 32}, kHip));
    TRY(lx, LazyTensor::from_tensor(x));
    TRY(o1, l1.forward_lazy(lx));
    TRY(o2, l2.forward_lazy(o1));
    CHECK(o2.graph_size() == 7);
    TRY(lazy, o2.eval());
    TRY(e1, l1.forward(x));
    TRY(e2, l2.forward(e1));
    TRY(vl, lazy.to_vec_f32());
    TRY(v2, e2.to_vec_f32());
    CHECK(vl == v2);
}

// A and B from graphs of their own: lora_fused merges them into the input's
// graph, so the node's inputs are A and B (executor_direct.rs:339-373's
// known answer).
CASE(lazy_lora_merges_separate_graphs, true) {
    TRY(lx, LazyTensor::from_slice({1, 2, 3, 4, 5, 6, 7, 8}, {2, 4}, kHip));
    TRY(la, LazyTensor::from_slice({.1f, .2f, .3f, .4f, .5f, .6f, .7f, .8f}, {4, 2}, kHip));
    TRY(lb, LazyTensor::from_slice({1, 2, 3, 4, 5, 6, 7, 8}, {2, 4}, kHip));
    TRY(ly, lx.lora_fused(la, lb, 0.5f));
    CHECK(ly.graph_size() == 4 && la.graph_size() == 1);
    TRY(y, ly.eval());
    TRY(v, y.to_vec_f32());
    const std::vector<float> want = {17.5f, 23.f, 28.5f, 34.f, 40.7f, 53.4f, 66.1f, 78.8f};
    CHECK_LE(rel_err(v, want), kTolF32);
}

// executor_direct.rs:456-495: RMSNorm through the executor; [3, 4] at eps 0
// gives [0.8485, 1.1314].
CASE(executor_rmsnorm_correctness, true) {
    TRY(ex, AsyncExecutor::create(kHip));
    TRY(x, Tensor::from_slice({3.f, 4.f}, {2}, kHip));
    TRY(y, ex.execute_operation(Operation::rms_norm(0.f), {x}));
    TRY(v, y.to_vec_f32());
    CHECK(fabs(v[0] - 0.8485f) < 1e-3 && fabs(v[1] - 1.1314f) < 1e-3);
    TRY(x2, Tensor::from_slice(randn(8, 0, 1, 3), {2, 4}, kHip));
    TRY(y2, ex.execute_operation(Operation::rms_norm(1e-5f), {x2}));
    CHECK((y2.dims() == std::vector<int64_t>{2, 4}));
}

// executor.rs:162-185: last-dim softmax runs fused; another dim is refused
// (the caller's candle softmax handles it).
CASE(executor_softmax_last_dim, true) {
    TRY(ex, AsyncExecutor::create(kHip));
    TRY(x, Tensor::from_slice({1, 2, 3, 4, 5, 6}, {2, 3}, kHip));
    TRY(p, ex.execute_operation(Operation::softmax(1), {x}));
    TRY(v, p.to_vec_f32());
    CHECK(fabs(v[0] + v[1] + v[2] - 1.0) < 1e-6 && fabs(v[3] + v[4] + v[5] - 1.0) < 1e-6);
    CHECK(ex.execute_operation(Operation::softmax(0), {x}).is_err());
}

namespace {
// FusedLoRAOp (delta only, fp32) against the oracle for x [dims..., K].
void check_fused_lora(std::vector<int64_t> xdims, int64_t N, int64_t r, float scaling, uint64_t seed, int line) {
    const int64_t K = xdims.back();
    int64_t T = 1;
    for (size_t i = 0; i + 1 < xdims.size(); ++i) T *= xdims[i];
    const auto x = randn((size_t)(T * K), 0, 1, seed);
    const auto A = randn((size_t)(K * r), 0, 0.01f, seed + 1);
    const auto B = randn((size_t)(r * N), 0, 0.01f, seed + 2);
    auto tx = Tensor::from_slice(x, xdims, kHip);
    auto ta = Tensor::from_slice(A, {K, r}, kHip);
    auto tb = Tensor::from_slice(B, {r, N}, kHip);
    if (tx.is_err() || ta.is_err() || tb.is_err()) return fail_at(line, "tensor upload failed");
    auto op = FusedLoRAOp::create(ta.value(), tb.value(), scaling);
    if (op.is_err()) return fail_at(line, op.error().to_string());
    auto y = op.value().apply(tx.value());
    if (y.is_err()) return fail_at(line, y.error().to_string());
    std::vector<int64_t> want_dims = xdims;
    want_dims.back() = N;
    if (y.value().dims() != want_dims) return fail_at(line, "output shape " + dims_to_string(y.value().dims()));
    auto got = y.value().to_vec_f32();
    std::vector<float> ref((size_t)(T * N));
    oracle_lora_fwd(T, K, N, (int32_t)r, scaling, 0.f, x.data(), nullptr, nullptr, A.data(), B.data(), nullptr,
                    ref.data(), nullptr, 0);
    const double e = rel_err(got.value(), ref);
    if (!(e <= kTolF32))
        fail_at(line, "x " + dims_to_string(xdims) + " r " + std::to_string(r) + ": rel err " + std::to_string(e));
}
}  // namespace

// custom_ops_correctness.rs:16-90.
CASE(fused_lora_correctness_basic, true) { check_fused_lora({2, 64, 512}, 512, 8, 2.f, 11, __LINE__); }

// custom_ops_correctness.rs:92-133.
CASE(fused_lora_various_batch_sizes, true) {
    for (int64_t b : {1, 2, 4, 8}) check_fused_lora({b, 32, 256}, 256, 8, 2.f, 20 + b, __LINE__);
}

// custom_ops_correctness.rs:135-168.
CASE(fused_lora_various_ranks, true) {
    for (int64_t r : {4, 8, 16, 32, 64}) check_fused_lora({1, 64, 512}, 512, r, 2.f, 40 + r, __LINE__);
}

// FusedLoRAOp::new's shape contract on a HIP input (custom_ops.rs:153-174).
CASE(fused_lora_input_mismatch, true) {
    TRY(x, Tensor::from_slice(ones(2 * 5), {2, 5}, kHip));
    TRY(a, Tensor::zeros({4, 2}, DType::F32, kHip));
    TRY(b, Tensor::zeros({2, 4}, DType::F32, kHip));
    TRY(op, FusedLoRAOp::create(a, b, 1.f));
    auto r = op.apply(x);
    CHECK(r.is_err());
    if (r.is_err()) CHECK(r.error().to_string() == "Input feature dimension mismatch: expected 4, got 5");
}

namespace {
void check_rmsnorm(std::vector<int64_t> dims, const std::vector<float>& x, float eps, double tol, int line) {
    const int64_t D = dims.back();
    const int64_t rows = (int64_t)x.size() / D;
    auto tx = Tensor::from_slice(x, dims, kHip);
    if (tx.is_err()) return fail_at(line, tx.error().to_string());
    auto y = rms_norm_fused(tx.value(), eps);
    if (y.is_err()) return fail_at(line, y.error().to_string());
    if (y.value().dims() != dims) return fail_at(line, "shape");
    auto got = y.value().to_vec_f32();
    std::vector<float> ref(x.size());
    oracle_rmsnorm_fwd(rows, D, eps, x.data(), nullptr, ref.data(), nullptr, 0);
    const double e = rel_err(got.value(), ref);
    if (!(e <= tol)) fail_at(line, "rmsnorm " + dims_to_string(dims) + ": rel err " + std::to_string(e));
}

void check_softmax(std::vector<int64_t> dims, const std::vector<float>& x, double tol, int line) {
    const int64_t D = dims.back();
    const int64_t rows = (int64_t)x.size() / D;
    auto tx = Tensor::from_slice(x, dims, kHip);
    if (tx.is_err()) return fail_at(line, tx.error().to_string());
    auto p = softmax_fused(tx.value());
    if (p.is_err()) return fail_at(line, p.error().to_string());
    auto got = p.value().to_vec_f32();
    std::vector<float> ref(x.size());
    oracle_softmax_fwd(rows, D, 0, x.data(), ref.data(), 0);
    const double e = rel_err(got.value(), ref);
    if (!(e <= tol)) fail_at(line, "softmax " + dims_to_string(dims) + ": rel err " + std::to_string(e));
}
}  // namespace

// rmsnorm_correctness.rs:41-116.
CASE(rmsnorm_correctness_2d_3d, true) {
    check_rmsnorm({4, 128}, randn(4 * 128, 0, 1, 1), 1e-5f, kTolF32, __LINE__);
    check_rmsnorm({2, 16, 512}, randn(2 * 16 * 512, 0, 1, 2), 1e-5f, kTolF32, __LINE__);
}

// rmsnorm_correctness.rs:118-147: output RMS is 1 within 1%.
CASE(rmsnorm_numerical_properties, true) {
    const auto x = randn(8 * 256, 0, 3, 5);
    TRY(tx, Tensor::from_slice(x, {8, 256}, kHip));
    TRY(y, rms_norm_fused(tx, 1e-6f));
    TRY(v, y.to_vec_f32());
    for (int r = 0; r < 8; ++r) {
        double s = 0;
        for (int j = 0; j < 256; ++j) s += (double)v[r * 256 + j] * v[r * 256 + j];
        CHECK(fabs(sqrt(s / 256) - 1.0) < 0.01);
    }
}

// rmsnorm_correctness.rs:149-203 (various shapes; extended to rank 4).
CASE(rmsnorm_various_shapes, true) {
    for (int64_t b : {1, 3, 8})
        for (int64_t d : {64, 896, 1536, 4096}) check_rmsnorm({b, d}, randn(b * d, 0, 1, b * d), 1e-6f, kTolF32, __LINE__);
    check_rmsnorm({2, 3, 4, 100}, randn(2400, 0, 1, 77), 1e-6f, kTolF32, __LINE__);
}

// rmsnorm_correctness.rs:205-265: constant rows of 100 and 0.01 at eps 1e-5
// (closed form 0.01 / sqrt(1e-4 + 1e-5) = 0.95346), and mixed magnitudes.
CASE(rmsnorm_extreme_values, true) {
    TRY(big, Tensor::from_slice(std::vector<float>(64, 100.f), {1, 64}, kHip));
    TRY(yb, rms_norm_fused(big, 1e-5f));
    TRY(vb, yb.to_vec_f32());
    CHECK(fabs(vb[0] - 1.0f) < 1e-5);
    TRY(small, Tensor::from_slice(std::vector<float>(64, 0.01f), {1, 64}, kHip));
    TRY(ys, rms_norm_fused(small, 1e-5f));
    TRY(vs, ys.to_vec_f32());
    CHECK(fabs(vs[0] - 0.01 / sqrt(1e-4 + 1e-5)) < 1e-5);
    std::vector<float> mixed(64);
    for (int i = 0; i < 64; ++i) mixed[i] = (i % 2 ? 1e3f : 1e-3f) * (i % 3 ? 1 : -1);
    check_rmsnorm({1, 64}, mixed, 1e-5f, kTolF32, __LINE__);
}

// softmax_correctness.rs:31-106.
CASE(softmax_correctness_2d_3d, true) {
    check_softmax({4, 128}, randn(4 * 128, 0, 1, 3), kTolF32, __LINE__);
    check_softmax({2, 16, 512}, randn(2 * 16 * 512, 0, 1, 4), kTolF32, __LINE__);
}

// softmax_correctness.rs:108-142: values in [0, 1], rows sum to 1 within 1e-5.
CASE(softmax_numerical_properties, true) {
    const auto x = randn(8 * 1000, 0, 3, 9);
    TRY(tx, Tensor::from_slice(x, {8, 1000}, kHip));
    TRY(p, softmax_fused(tx));
    TRY(v, p.to_vec_f32());
    for (int r = 0; r < 8; ++r) {
        double s = 0;
        for (int j = 0; j < 1000; ++j) {
            const float q = v[r * 1000 + j];
            CHECK(q >= 0.f && q <= 1.f);
            s += q;
        }
        CHECK(fabs(s - 1.0) < 1e-5);
    }
}

// softmax_correctness.rs:144-199 (various shapes; extended to rank 4, the
// attention-score shape the Metal kernel refuses).
CASE(softmax_various_shapes, true) {
    for (int64_t b : {1, 3, 8})
        for (int64_t d : {16, 100, 1024, 4096}) check_softmax({b, d}, randn(b * d, 0, 3, b + d), kTolF32, __LINE__);
    check_softmax({2, 3, 8, 64}, randn(2 * 3 * 8 * 64, 0, 3, 5), kTolF32, __LINE__);
}

// softmax_correctness.rs:200-243: constant rows of +-100 give the uniform
// distribution; large spreads stay finite (tensor.rs:146-162).
CASE(softmax_extreme_values, true) {
    for (float c : {100.f, -100.f}) {
        TRY(x, Tensor::from_slice(std::vector<float>(50, c), {1, 50}, kHip));
        TRY(p, softmax_fused(x));
        TRY(v, p.to_vec_f32());
        for (float q : v) CHECK(fabs(q - 0.02f) < 1e-6);
    }
    check_softmax({1, 3}, {100.f, 200.f, 300.f}, kTolF32, __LINE__);
}

// Causal softmax forward and backward (transformer.rs:264-275 mask; the
// backward is the autograd of tensor.rs:91-98), rank 4 [B, H, S, S].
CASE(softmax_causal_forward_backward, true) {
    const int64_t Bt = 2, H = 3, S = 64;
    const int64_t rows = Bt * H * S;
    const auto s = randn((size_t)(rows * S), 0, 3, 31);
    const auto dp = randn((size_t)(rows * S), 0, 0.01f, 32);
    TRY(ts, Tensor::from_slice(s, {Bt, H, S, S}, kHip));
    TRY(tdp, Tensor::from_slice(dp, {Bt, H, S, S}, kHip));
    TRY(op, FusedSoftmaxOp::create());
    TRY(p, op.forward_causal(ts, true));
    TRY(ds, op.backward(p, tdp, true));
    TRY(vp, p.to_vec_f32());
    TRY(vds, ds.to_vec_f32());
    std::vector<float> rp(s.size()), rds(s.size());
    oracle_softmax_fwd(rows, S, S, s.data(), rp.data(), 0);
    oracle_softmax_bwd(rows, S, S, rp.data(), dp.data(), rds.data(), 0);
    CHECK_LE(rel_err(vp, rp), kTolF32);
    CHECK_LE(rel_err(vds, rds), kTolF32);
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = i % S + 1; j < S; ++j) CHECK(vp[(size_t)(i * S + j)] == 0.f && vds[(size_t)(i * S + j)] == 0.f);
}

// Weighted RMSNorm forward and backward (qwen.rs:314-325), bf16 and fp32.
CASE(rmsnorm_weighted_forward_backward, true) {
    const int64_t rows = 64, D = 1536;
    for (DType dt : {DType::F32, DType::BF16}) {
        const bool bf = dt == DType::BF16;
        auto x = randn((size_t)(rows * D), 0, 1, 51), w = randn((size_t)D, 1, 0.1f, 52),
             dy = randn((size_t)(rows * D), 0, 0.01f, 53);
        if (bf) x = round_bf16(x), w = round_bf16(w), dy = round_bf16(dy);
        TRY(tx, Tensor::from_slice(x, {rows, D}, kHip, dt));
        TRY(tw, Tensor::from_slice(w, {D}, kHip, dt));
        TRY(tdy, Tensor::from_slice(dy, {rows, D}, kHip, dt));
        TRY(op, FusedRMSNormOp::create(1e-6f));
        TRY(fw, op.forward_weighted(tx, &tw));
        TRY(bw, op.backward(tx, &tw, fw.second, tdy));
        TRY(vy, fw.first.to_vec_f32());
        TRY(vdx, bw.first.to_vec_f32());
        TRY(vdw, bw.second.to_vec_f32());
        std::vector<float> ry(x.size()), rdx(x.size()), rdw((size_t)D);
        oracle_rmsnorm_fwd(rows, D, 1e-6f, x.data(), w.data(), ry.data(), nullptr, 0);
        oracle_rmsnorm_bwd(rows, D, 1e-6f, x.data(), w.data(), dy.data(), rdx.data(), rdw.data(), 0);
        const double tol = bf ? kTolBf16 : kTolF32;
        CHECK_LE(rel_err(vy, ry), tol);
        CHECK_LE(rel_err(vdx, rdx), tol);
        CHECK_LE(rel_err(vdw, rdw), bf ? kTolBf16 : 1e-4);
    }
}

// lora_dropout.rs:5-69, 197-238: eval mode is deterministic; training mode
// with dropout draws a new mask per forward, and equals the CPU reference fed
// the same mask.
CASE(lora_dropout_train_and_eval, true) {
    TRY(layer, LoRALayer::create(64, 64, LoRAConfig{8, 16.f, 0.5f}, kHip, 7));
    const auto bv = randn(8 * 64, 0, 0.1f, 8);
    TRY(tb, Tensor::from_slice(bv, {8, 64}, kHip));
    CHECK(layer.set_lora_b(tb).is_ok());
    const auto x = randn(4 * 10 * 64, 0, 1, 9);
    TRY(tx, Tensor::from_slice(x, {4, 10, 64}, kHip));
    TRY(av, layer.lora_a_tensor().to_vec_f32());
    // training: two forwards, two masks, each equal to the oracle with its mask
    std::vector<std::vector<float>> outs;
    std::vector<std::vector<float>> masks;
    for (int k = 0; k < 2; ++k) {
        TRY(y, layer.forward(tx));
        TRY(vy, y.to_vec_f32());
        TRY(m, layer.last_mask().to_vec_f32());
        std::vector<uint8_t> mb(m.size());
        for (size_t i = 0; i < m.size(); ++i) mb[i] = (uint8_t)m[i];
        std::vector<float> ref(vy.size());
        oracle_lora_fwd(40, 64, 64, 8, 2.f, 0.5f, x.data(), nullptr, nullptr, av.data(), bv.data(), mb.data(),
                        ref.data(), nullptr, 0);
        CHECK_LE(rel_err(vy, ref), kTolF32);
        outs.push_back(vy);
        masks.push_back(m);
    }
    CHECK(masks[0] != masks[1]);
    CHECK(outs[0] != outs[1]);
    // eval: identical outputs, equal to the no-dropout reference
    layer.eval();
    TRY(e1, layer.forward(tx));
    TRY(e2, layer.forward(tx));
    TRY(v1, e1.to_vec_f32());
    TRY(v2, e2.to_vec_f32());
    CHECK(v1 == v2);
    std::vector<float> ref(v1.size());
    oracle_lora_fwd(40, 64, 64, 8, 2.f, 0.f, x.data(), nullptr, nullptr, av.data(), bv.data(), nullptr,
                    ref.data(), nullptr, 0);
    CHECK_LE(rel_err(v1, ref), kTolF32);
    CHECK((e1.dims() == std::vector<int64_t>{4, 10, 64}));
}

// lora_dropout.rs:69-100: dropout 0 in training mode is deterministic.
CASE(lora_dropout_zero_no_randomness, true) {
    TRY(layer, LoRALayer::create(16, 16, LoRAConfig{4, 8.f, 0.f}, kHip, 3));
    TRY(tb, Tensor::from_slice(randn(4 * 16, 0, 0.1f, 4), {4, 16}, kHip));
    CHECK(layer.set_lora_b(tb).is_ok());
    TRY(x, Tensor::from_slice(ones(16), {1, 16}, kHip));
    TRY(y1, layer.forward(x));
    TRY(y2, layer.forward(x));
    TRY(v1, y1.to_vec_f32());
    TRY(v2, y2.to_vec_f32());
    CHECK(v1 == v2);
}

// gradient_verification.rs:16-89 and lora_dropout.rs:240-263: gradients of
// A and B exist, have A's and B's shapes, are non-zero, and equal the
// closed-form gradients of the oracle (with and without dropout).
CASE(lora_layer_gradient_flow, true) {
    for (float p : {0.f, 0.2f}) {
        TRY(layer, LoRALayer::create(16, 16, LoRAConfig{4, 8.f, p}, kHip, 5));
        const auto bv = randn(4 * 16, 0, 0.1f, 6);
        TRY(tb, Tensor::from_slice(bv, {4, 16}, kHip));
        CHECK(layer.set_lora_b(tb).is_ok());
        const auto x = randn(2 * 16, 0, 1, 7);
        const auto dy = randn(2 * 16, 0, 1, 8);
        TRY(tx, Tensor::from_slice(x, {2, 16}, kHip));
        TRY(tdy, Tensor::from_slice(dy, {2, 16}, kHip));
        TRY(y, layer.forward(tx));
        (void)y;
        TRY(g, layer.backward(tx, tdy));
        CHECK(g.da.dims() == layer.lora_a_tensor().dims());
        CHECK(g.db.dims() == layer.lora_b_tensor().dims());
        CHECK(g.dx.dims() == tx.dims());
        TRY(av, layer.lora_a_tensor().to_vec_f32());
        TRY(vda, g.da.to_vec_f32());
        TRY(vdb, g.db.to_vec_f32());
        TRY(vdx, g.dx.to_vec_f32());
        std::vector<uint8_t> mb;
        if (p > 0) {
            TRY(m, layer.last_mask().to_vec_f32());
            for (float v : m) mb.push_back((uint8_t)v);
        }
        std::vector<float> rdx(x.size()), rda(av.size()), rdb(bv.size());
        oracle_lora_bwd(2, 16, 16, 4, 2.f, p, x.data(), nullptr, av.data(), bv.data(), p > 0 ? mb.data() : nullptr,
                        dy.data(), rdx.data(), rda.data(), rdb.data(), 0);
        CHECK_LE(rel_err(vda, rda), kTolF32);
        CHECK_LE(rel_err(vdb, rdb), kTolF32);
        CHECK_LE(rel_err(vdx, rdx), kTolF32);
        double sa = 0, sb = 0;
        for (float v : vda) sa += fabs(v);
        for (float v : vdb) sb += fabs(v);
        CHECK(sa > 1e-6 && sb > 1e-6);
    }
}

// B = 0 (the initial state, lora.rs:244): the delta is 0, and so is dA
// (G = s dY B^T = 0), while dB is not.
CASE(lora_zero_b_gradients, true) {
    TRY(layer, LoRALayer::create(32, 48, LoRAConfig{8, 16.f, 0.f}, kHip, 1));
    TRY(x, Tensor::from_slice(randn(5 * 32, 0, 1, 2), {5, 32}, kHip));
    TRY(dy, Tensor::from_slice(randn(5 * 48, 0, 1, 3), {5, 48}, kHip));
    TRY(y, layer.forward(x));
    TRY(vy, y.to_vec_f32());
    for (float v : vy) CHECK(v == 0.f);
    TRY(g, layer.backward(x, dy));
    TRY(vda, g.da.to_vec_f32());
    TRY(vdb, g.db.to_vec_f32());
    for (float v : vda) CHECK(v == 0.f);
    double sb = 0;
    for (float v : vdb) sb += fabs(v);
    CHECK(sb > 1e-3);
}

// The fused linear with frozen base weight and bias (the q/k/v projection of
// transformer.rs:189-192 plus its LoRA), bf16 activations, fwd and bwd.
CASE(fused_lora_with_base_bf16, true) {
    const int64_t T = 96, K = 256, N = 192, r = 16;
    const float s = 2.f;
    const auto x = round_bf16(randn((size_t)(T * K), 0, 1, 61));
    const auto W = round_bf16(randn((size_t)(N * K), 0, 0.02f, 62));
    const auto bias = round_bf16(randn((size_t)N, 0, 0.02f, 63));
    const auto A = randn((size_t)(K * r), 0, 1.f / 16, 64);
    const auto B = randn((size_t)(r * N), 0, 0.02f, 65);
    const auto dy = round_bf16(randn((size_t)(T * N), 0, 0.01f, 66));
    TRY(tx, Tensor::from_slice(x, {T, K}, kHip, DType::BF16));
    TRY(tW, Tensor::from_slice(W, {N, K}, kHip, DType::BF16));
    TRY(tb, Tensor::from_slice(bias, {N}, kHip, DType::BF16));
    TRY(tA, Tensor::from_slice(A, {K, r}, kHip));
    TRY(tB, Tensor::from_slice(B, {r, N}, kHip));
    TRY(tdy, Tensor::from_slice(dy, {T, N}, kHip, DType::BF16));
    TRY(op, FusedLoRAOp::create(tA, tB, s));
    TRY(fw, op.forward_with_base(tx, &tW, &tb, nullptr, 0.f));
    TRY(g, op.backward(tx, &tW, fw.second, tdy, nullptr, 0.f));
    TRY(vy, fw.first.to_vec_f32());
    TRY(vdx, g.dx.to_vec_f32());
    TRY(vda, g.da.to_vec_f32());
    TRY(vdb, g.db.to_vec_f32());
    std::vector<float> ry((size_t)(T * N)), rdx(x.size()), rda(A.size()), rdb(B.size());
    oracle_lora_fwd(T, K, N, (int32_t)r, s, 0.f, x.data(), W.data(), bias.data(), A.data(), B.data(), nullptr,
                    ry.data(), nullptr, 0);
    oracle_lora_bwd(T, K, N, (int32_t)r, s, 0.f, x.data(), W.data(), A.data(), B.data(), nullptr, dy.data(),
                    rdx.data(), rda.data(), rdb.data(), 0);
    CHECK_LE(rel_err(vy, ry), kTolBf16);
    CHECK_LE(rel_err(vdx, rdx), kTolBf16);
    CHECK_LE(rel_err(vda, rda), kTolBf16);
    CHECK_LE(rel_err(vdb, rdb), kTolBf16);
    // h_save is Hd^T [r, T]
    TRY(vh, fw.second.hidden_t.to_vec_f32());
    std::vector<float> rh((size_t)(T * r));
    oracle_lora_fwd(T, K, N, (int32_t)r, s, 0.f, x.data(), nullptr, nullptr, A.data(), B.data(), nullptr, ry.data(),
                    rh.data(), 0);
    CHECK_LE(rel_err(vh, transpose(rh, T, r)), kTolF32 * 10);
}

// ================================================================== AdamW
// optimizer.rs:367-375 test_adamw_config_default
CASE(adamw_config_default, false) {
    const AdamWConfig c;
    CHECK(fabs((double)c.learning_rate - 1e-4) < 1e-7);
    CHECK(fabs((double)c.beta1 - 0.9) < 1e-7);
    CHECK(fabs((double)c.beta2 - 0.999) < 1e-7);
    CHECK(fabs((double)c.epsilon - 1e-8) < 1e-7);
    CHECK(fabs((double)c.weight_decay - 0.01) < 1e-7);
}

// optimizer.rs:377-399 test_adamw_config_validation, with the messages of 67-103
CASE(adamw_config_validation, false) {
    CHECK(AdamWConfig().validate().is_ok());
    const char* prefix = "training error: invalid training configuration: ";
    AdamWConfig c;
    c.learning_rate = -1.f;
    CHECK(c.validate().is_err() && c.validate().error().to_string() == std::string(prefix) + "learning rate must be positive");
    c = AdamWConfig();
    c.beta1 = 1.5f;
    CHECK(c.validate().is_err() && c.validate().error().to_string() == std::string(prefix) + "beta1 must be in [0, 1), got 1.5");
    c = AdamWConfig();
    c.beta2 = -0.1f;
    CHECK(c.validate().is_err() && c.validate().error().to_string() == std::string(prefix) + "beta2 must be in [0, 1), got -0.1");
    c = AdamWConfig();
    c.epsilon = 0.f;
    CHECK(c.validate().is_err() && c.validate().error().to_string() == std::string(prefix) + "epsilon must be positive");
    c = AdamWConfig();
    c.weight_decay = -0.5f;
    CHECK(c.validate().is_err() && c.validate().error().to_string() == std::string(prefix) + "weight decay must be non-negative");
}

// optimizer.rs:401-409 test_adamw_creation
CASE(adamw_creation, false) {
    TRY(opt, AdamW::create(AdamWConfig()));
    CHECK(opt.step_count() == 0);
    AdamWConfig bad;
    bad.learning_rate = 0.f;
    CHECK(AdamW::create(bad).is_err());
}

// optimizer.rs:411-420 test_adamw_add_parameter
CASE(adamw_add_parameter, false) {
    TRY(opt, AdamW::create(AdamWConfig()));
    TRY(p, Tensor::zeros({10, 10}, DType::F32, kCpu));
    CHECK(opt.add_parameter("test_param", p).is_ok());
}

// optimizer.rs:490-508 test_adamw_parameter_not_found
CASE(adamw_parameter_not_found, false) {
    TRY(opt, AdamW::create(AdamWConfig()));
    TRY(p, Tensor::from_slice(std::vector<float>(9, 1.f), {3, 3}, kCpu));
    auto r = opt.step("unknown", p, p);
    CHECK(r.is_err());
    if (r.is_err())
        CHECK(r.error().to_string() == "training error: training state error: parameter 'unknown' not found in optimizer");
}

// Runs `steps` AdamW steps of the oracle on host copies; returns the last parameter.
static std::vector<float> adamw_oracle(const AdamWConfig& c, std::vector<float> p, const std::vector<float>& g,
                                       int first_step, int steps) {
    std::vector<float> m(p.size(), 0.f), v(p.size(), 0.f), out(p.size());
    for (int t = first_step; t < first_step + steps; ++t) {
        oracle_adamw_step((int64_t)p.size(), c.learning_rate, c.beta1, c.beta2, c.epsilon, c.weight_decay, t, p.data(),
                          g.data(), m.data(), v.data(), out.data());
        p = out;
    }
    return p;
}

// optimizer.rs:422-446 test_adamw_step
CASE(adamw_step, true) {
    AdamWConfig c;
    c.learning_rate = 0.1f;
    TRY(opt, AdamW::create(c));
    const std::vector<float> ones(25, 1.f);
    TRY(p, Tensor::from_slice(ones, {5, 5}, kHip));
    TRY(g, Tensor::from_slice(ones, {5, 5}, kHip));
    CHECK(opt.add_parameter("param", p).is_ok());
    TRY(p1, opt.step("param", p, g));
    CHECK(p1.dims() == std::vector<int64_t>({5, 5}));
    TRY(v1, p1.to_vec_f32());
    double sum = 0;
    for (float x : v1) sum += x;
    CHECK(fabs(25.0 - sum) > 1e-6);
    CHECK(opt.step_count() == 1);
    CHECK(v1 == adamw_oracle(c, ones, ones, 1, 1));  // bit for bit
}

// optimizer.rs:448-470 test_adamw_multiple_steps
CASE(adamw_multiple_steps, true) {
    const AdamWConfig c;
    TRY(opt, AdamW::create(c));
    const std::vector<float> ones(9, 1.f);
    TRY(p, Tensor::from_slice(ones, {3, 3}, kHip));
    TRY(g, Tensor::from_slice(ones, {3, 3}, kHip));
    CHECK(opt.add_parameter("param", p).is_ok());
    Tensor cur = p;
    for (int i = 0; i < 5; ++i) {
        TRY(next, opt.step("param", cur, g));
        cur = next;
    }
    CHECK(opt.step_count() == 5);
    TRY(v, cur.to_vec_f32());
    double sum = 0;
    for (float x : v) sum += x;
    CHECK(sum < 9.0);
    CHECK(v == adamw_oracle(c, ones, ones, 1, 5));
}

// optimizer.rs:472-488 test_adamw_reset_state
CASE(adamw_reset_state, true) {
    const AdamWConfig c;
    TRY(opt, AdamW::create(c));
    const std::vector<float> ones(9, 1.f);
    TRY(p, Tensor::from_slice(ones, {3, 3}, kHip));
    TRY(g, Tensor::from_slice(ones, {3, 3}, kHip));
    CHECK(opt.add_parameter("param", p).is_ok());
    TRY(a, opt.step("param", p, g));
    TRY(b, opt.step("param", p, g));
    CHECK(opt.step_count() == 2);
    opt.reset_state();
    CHECK(opt.step_count() == 0);
    // after the reset the next step is a first step from zero moments
    TRY(c1, opt.step("param", p, g));
    TRY(vc, c1.to_vec_f32());
    CHECK(vc == adamw_oracle(c, ones, ones, 1, 1));
    (void)a;
    (void)b;
}

// ================================================================== LayerNorm
// custom_ops.rs LayerNormOp: name and the 2-D requirement
CASE(layer_norm_op_name_and_rank, false) {
    const LayerNormOp op = LayerNormOp::create(1e-5);
    CHECK(std::string(op.name()) == "layer-norm");
    TRY(x, Tensor::from_slice(ones(8), {2, 4}, kCpu));
    CHECK(op.apply(x).is_err());  // CPU tensors are not computed here
}

CASE(layer_norm_op_requires_2d, true) {
    const LayerNormOp op = LayerNormOp::create(1e-5);
    TRY(x, Tensor::from_slice(ones(24), {2, 3, 4}, kHip));
    auto r = op.apply(x);
    CHECK(r.is_err());
    if (r.is_err()) CHECK(r.error().to_string() == "LayerNorm expects 2D tensors, got shape [2, 3, 4]");
}

// tensor.rs:165-181 test_layer_norm, 214-228 _with_different_eps, 278-300 _preserves_shape / _with_zeros
CASE(layer_norm_reference_tests, true) {
    TRY(x, Tensor::from_slice({1, 2, 3, 4, 5, 6, 7, 8}, {2, 4}, kHip));
    TRY(y, layer_norm(x, 1e-5));
    TRY(v, y.to_vec_f32());
    for (int r = 0; r < 2; ++r) {
        double m = 0;
        for (int j = 0; j < 4; ++j) m += v[r * 4 + j];
        CHECK(fabs(m / 4) < 1e-4);
    }
    std::vector<float> ref(8);
    const std::vector<float> xs = {1, 2, 3, 4, 5, 6, 7, 8};
    oracle_layernorm_fwd(2, 4, 1e-5f, xs.data(), nullptr, nullptr, ref.data(), nullptr, nullptr, 0);
    CHECK_LE(rel_err(v, ref), kTolF32);
    TRY(x3, Tensor::from_slice({1, 2, 3}, {1, 3}, kHip));
    TRY(a, layer_norm(x3, 1e-5));
    TRY(b, layer_norm(x3, 1e-3));
    CHECK(a.dims() == b.dims());
    TRY(xr, Tensor::from_slice(randn(105, 0, 1, 71), {3, 5, 7}, kHip));
    TRY(yr, layer_norm(xr, 1e-5));
    CHECK(yr.dims() == xr.dims());
    TRY(z, Tensor::from_slice({0, 0, 0}, {1, 3}, kHip));
    TRY(yz, layer_norm(z, 1e-5));
    TRY(vz, yz.to_vec_f32());
    for (float t : vz) CHECK(fabs(t) < 1e-6);
}

// MetalLayerNorm (metal_bert.rs:30-72): weight, bias, and the backward
CASE(layer_norm_affine_forward_backward, true) {
    const int64_t R = 12, D = 384;
    const auto x = randn((size_t)(R * D), 0.2f, 1.5f, 72), w = randn((size_t)D, 1.f, 0.1f, 73),
               b = randn((size_t)D, 0, 0.1f, 74), dy = randn((size_t)(R * D), 0, 1, 75);
    TRY(tx, Tensor::from_slice(x, {R, D}, kHip));
    TRY(tw, Tensor::from_slice(w, {D}, kHip));
    TRY(tb, Tensor::from_slice(b, {D}, kHip));
    TRY(tdy, Tensor::from_slice(dy, {R, D}, kHip));
    const LayerNormOp op = LayerNormOp::create(1e-12);  // BertConfig layer_norm_eps (embeddings/bert.rs:169)
    TRY(f, op.forward_affine(tx, &tw, &tb));
    TRY(g, op.backward(tx, &tw, f.second, tdy));
    std::vector<float> ry(x.size()), rdx(x.size()), rdw(D), rdb(D);
    oracle_layernorm_fwd(R, D, 1e-12f, x.data(), w.data(), b.data(), ry.data(), nullptr, nullptr, 0);
    oracle_layernorm_bwd(R, D, 1e-12f, x.data(), w.data(), dy.data(), rdx.data(), rdw.data(), rdb.data(), 0);
    TRY(vy, f.first.to_vec_f32());
    TRY(vdx, g.dx.to_vec_f32());
    TRY(vdw, g.dw.to_vec_f32());
    TRY(vdb, g.db.to_vec_f32());
    CHECK_LE(rel_err(vy, ry), kTolF32);
    CHECK_LE(rel_err(vdx, rdx), kTolF32);
    CHECK_LE(rel_err(vdw, rdw), kTolF32);
    CHECK_LE(rel_err(vdb, rdb), kTolF32);
}

// ================================================================== cross entropy
static double loss_of(const Result<Tensor, Error>& r) {
    if (r.is_err()) return NAN;
    auto v = r.value().to_vec_f32();
    return v.is_ok() && !v.value().empty() ? v.value()[0] : NAN;
}

// loss.rs:265-278 test_cross_entropy_loss_basic, 281-294 _wrong_prediction
CASE(cross_entropy_basic_and_wrong_prediction, true) {
    TRY(lg, Tensor::from_slice({10, 0, 0}, {1, 1, 3}, kHip));
    TRY(t0, Tensor::from_u32({0}, {1, 1}, kHip));
    TRY(t2, Tensor::from_u32({2}, {1, 1}, kHip));
    const double a = loss_of(cross_entropy_loss(lg, t0, std::nullopt));
    const double b = loss_of(cross_entropy_loss(lg, t2, std::nullopt));
    CHECK(a < 0.1);
    CHECK(b > 5.0);
    const std::vector<float> xs = {10, 0, 0};
    const uint32_t t[1] = {2};
    CHECK(fabs(b - oracle_cross_entropy_fwd(1, 3, xs.data(), t, -1, 0.f, nullptr, nullptr)) < 1e-5);
    auto sc = cross_entropy_loss(lg, t0, std::nullopt);
    CHECK(sc.is_ok() && sc.value().dims().empty());  // a scalar
}

// loss.rs:297-316 test_cross_entropy_loss_with_ignore, and the all-ignored error (loss.rs:123-131)
CASE(cross_entropy_with_ignore, true) {
    TRY(lg, Tensor::from_slice({1, 2, 3, 1, 2, 3, 1, 2, 3, 1, 2, 3}, {2, 2, 3}, kHip));
    TRY(t, Tensor::from_u32({2, 0, 2, 0}, {2, 2}, kHip));
    auto r = cross_entropy_loss(lg, t, 0u);
    CHECK(r.is_ok());
    const double want = log(exp(1.0) + exp(2.0) + exp(3.0)) - 3.0;
    CHECK(fabs(loss_of(r) - want) < 1e-5);
    TRY(t0, Tensor::from_u32({0, 0, 0, 0}, {2, 2}, kHip));
    auto e = cross_entropy_loss(lg, t0, 0u);
    CHECK(e.is_err());
    if (e.is_err())
        CHECK(e.error().to_string() ==
              "training error: invalid training configuration: all tokens are ignored, cannot compute loss");
}

// loss.rs:319-341 test_cross_entropy_loss_invalid_shapes, _shape_mismatch
CASE(cross_entropy_shape_errors, true) {
    TRY(l2, Tensor::zeros({2, 10}, DType::F32, kHip));
    TRY(t2, Tensor::from_u32(std::vector<uint32_t>(20, 0), {2, 10}, kHip));
    auto a = cross_entropy_loss(l2, t2, std::nullopt);
    CHECK(a.is_err());
    if (a.is_err())
        CHECK(a.error().to_string() == "training error: invalid training configuration: logits must be 3D (batch, "
                                       "seq_len, vocab_size), got shape [2, 10]");
    TRY(l3, Tensor::zeros({2, 10, 100}, DType::F32, kHip));
    TRY(t5, Tensor::from_u32(std::vector<uint32_t>(10, 0), {2, 5}, kHip));
    auto b = cross_entropy_loss(l3, t5, std::nullopt);
    CHECK(b.is_err());
    if (b.is_err())
        CHECK(b.error().to_string() == "training error: invalid training configuration: logits and targets "
                                       "batch/seq_len mismatch: logits [2, 10] vs targets [2, 5]");
}

// loss.rs:344-380 label smoothing: zero equals plain, 0.1 raises the loss, 1.0 and -0.1 are rejected
CASE(cross_entropy_label_smoothing, true) {
    TRY(lg, Tensor::from_slice({1, 2, 3}, {1, 1, 3}, kHip));
    TRY(t, Tensor::from_u32({2}, {1, 1}, kHip));
    CHECK(fabs(loss_of(cross_entropy_loss(lg, t, std::nullopt)) -
               loss_of(cross_entropy_loss_with_smoothing(lg, t, 0.f, std::nullopt))) < 1e-6);
    TRY(lg2, Tensor::from_slice({10, 0, 0}, {1, 1, 3}, kHip));
    TRY(t0, Tensor::from_u32({0}, {1, 1}, kHip));
    CHECK(loss_of(cross_entropy_loss_with_smoothing(lg2, t0, 0.1f, std::nullopt)) >
          loss_of(cross_entropy_loss(lg2, t0, std::nullopt)));
    auto a = cross_entropy_loss_with_smoothing(lg, t, 1.f, std::nullopt);
    auto b = cross_entropy_loss_with_smoothing(lg, t, -0.1f, std::nullopt);
    CHECK(a.is_err() && b.is_err());
    if (a.is_err())
        CHECK(a.error().to_string() == "training error: invalid training configuration: smoothing must be in [0, 1), got 1");
    if (b.is_err())
        CHECK(b.error().to_string() == "training error: invalid training configuration: smoothing must be in [0, 1), got -0.1");
}

// the gradient extension against the oracle
CASE(cross_entropy_backward, true) {
    const int64_t B = 2, S = 8, V = 50;
    const auto x = randn((size_t)(B * S * V), 0, 2, 76);
    std::vector<uint32_t> t((size_t)(B * S));
    for (size_t i = 0; i < t.size(); ++i) t[i] = (uint32_t)((i * 7) % V);
    t[3] = 0;
    TRY(lg, Tensor::from_slice(x, {B, S, V}, kHip));
    TRY(tt, Tensor::from_u32(t, {B, S}, kHip));
    TRY(g, cross_entropy_loss_backward(lg, tt, 0.1f, 0u, 2.0f));
    TRY(vg, g.to_vec_f32());
    std::vector<float> rg(x.size());
    oracle_cross_entropy_bwd(B * S, V, x.data(), t.data(), 0, 0.1f, 2.0f, rg.data());
    CHECK_LE(rel_err(vg, rg), kTolF32);
}

// ================================================================== adapter
// adapter.rs:358-372 test_target_module_name / _from_name
CASE(adapter_target_modules, false) {
    CHECK(std::string(target_module_name(TargetModule::QProj)) == "q_proj");
    CHECK(std::string(target_module_name(TargetModule::VProj)) == "v_proj");
    CHECK(std::string(target_module_name(TargetModule::GateProj)) == "gate_proj");
    CHECK(target_module_from_name("q_proj") == TargetModule::QProj);
    CHECK(target_module_from_name("v_proj") == TargetModule::VProj);
    CHECK(!target_module_from_name("invalid").has_value());
}

// adapter.rs:375-384 test_lora_adapter_config_default; creation and parameter counts
CASE(adapter_config_and_creation, false) {
    const LoRAAdapterConfig c;
    CHECK(c.rank == 8 && fabs(c.alpha - 16.0) < 1e-7 && c.target_modules.size() == 2);
    CHECK(c.is_target(TargetModule::QProj) && c.is_target(TargetModule::VProj) && !c.is_target(TargetModule::KProj));
    LoRAAdapterConfig all = c;
    all.rank = 4;
    all.target_modules = {TargetModule::QProj, TargetModule::GateProj, TargetModule::DownProj};
    TRY(a, LoRAAdapter::create(32, 128, 2, all, kCpu));
    CHECK(a.layers().size() == 6 && a.num_layers() == 2);
    const LoRALayer* q = a.get_layer(1, TargetModule::QProj);
    const LoRALayer* g = a.get_layer(0, TargetModule::GateProj);
    const LoRALayer* d = a.get_layer(1, TargetModule::DownProj);
    CHECK(q && g && d && !a.get_layer(0, TargetModule::VProj));
    if (q && g && d) {
        CHECK(q->lora_a_tensor().dims() == std::vector<int64_t>({32, 4}));
        CHECK(g->lora_b_tensor().dims() == std::vector<int64_t>({4, 128}));
        CHECK(d->lora_a_tensor().dims() == std::vector<int64_t>({128, 4}));
    }
    // q: 4 (32 + 32), gate: 4 (32 + 128), down: 4 (128 + 32), two layers
    CHECK(a.num_trainable_parameters() == 2 * (4 * 64 + 4 * 160 + 4 * 160));
    CHECK(a.num_frozen_parameters(10) == 0);
    CHECK(a.num_frozen_parameters(1000000) == 1000000 - a.num_trainable_parameters());
}

// The device pool: a released block of a size is reused by the next
// allocation of that size (no hipMalloc, no hipFree in a steady loop).
CASE(device_pool_reuses_blocks, true) {
    const size_t hits0 = device_pool_hits();
    void* first = nullptr;
    {
        TRY(t, Tensor::empty({1024, 1024}, DType::F32, kHip));
        first = t.data();
    }
    CHECK(cached_device_bytes() >= (size_t)4 << 20);
    TRY(u, Tensor::empty({1024, 1024}, DType::F32, kHip));
    CHECK(u.data() == first);
    CHECK(device_pool_hits() == hits0 + 1);
    // ops that need workspace draw it from the pool as well: two identical
    // backward calls, the second served from cached blocks
    TRY(op, FusedRMSNormOp::create(1e-6f));
    std::vector<float> xv(64 * 256, 0.5f);
    TRY(x, Tensor::from_slice(xv, {64, 256}, kHip));
    TRY(fw, op.forward_weighted(x, nullptr));
    TRY(g1, op.backward(x, nullptr, fw.second, x));
    const size_t hits1 = device_pool_hits();
    TRY(g2, op.backward(x, nullptr, fw.second, x));
    CHECK(device_pool_hits() > hits1);
    release_cached_device_memory();
    CHECK(cached_device_bytes() == 0);
}

// ================================================================== checkpoints
static std::string tmp_path(const char* name) {
    const char* d = getenv("MC_CKPT_DIR");
    return std::string(d && *d ? d : "/tmp") + "/" + name;
}

static LoRAAdapterConfig ckpt_config() {
    LoRAAdapterConfig c;  // checkpoint.rs tests: rank 4, alpha 8, q_proj
    c.rank = 4;
    c.alpha = 8.f;
    c.target_modules = {TargetModule::QProj};
    return c;
}

// checkpoint.rs:113-150 test_save_and_load_checkpoint
CASE(checkpoint_save_and_load, false) {
    TRY(a, LoRAAdapter::create(32, 128, 2, ckpt_config(), kCpu, 1));
    const std::string path = tmp_path("mc_ckpt_meta.safetensors");
    const CheckpointMetadata md{100, 1.5f, 1e-4f, 1234567890ull};
    CHECK(save_checkpoint(a, path, &md).is_ok());
    TRY(b, LoRAAdapter::create(32, 128, 2, ckpt_config(), kCpu, 2));
    auto r = load_checkpoint(b, path);
    CHECK(r.is_ok() && !r.value().has_value());  // metadata is not loaded (checkpoint.rs:80-82)
    auto m = read_checkpoint_metadata(path);
    CHECK(m.is_ok() && m.value().has_value());
    if (m.is_ok() && m.value()) {
        CHECK(m.value()->global_step == 100 && m.value()->loss == 1.5f && m.value()->learning_rate == 1e-4f &&
              m.value()->timestamp == 1234567890ull);
    }
    CHECK(md.to_json() == "{\"global_step\":100,\"loss\":1.5,\"learning_rate\":0.0001,\"timestamp\":1234567890}");
    remove(path.c_str());
}

// checkpoint.rs:153-177 test_save_checkpoint_without_metadata, 180-221 test_checkpoint_preserves_weights
CASE(checkpoint_preserves_weights, false) {
    TRY(a, LoRAAdapter::create(32, 128, 1, ckpt_config(), kCpu, 3));
    const std::string path = tmp_path("mc_ckpt_plain.safetensors");
    CHECK(save_checkpoint(a, path, nullptr).is_ok());
    TRY(b, LoRAAdapter::create(32, 128, 1, ckpt_config(), kCpu, 4));
    auto r = load_checkpoint(b, path);
    CHECK(r.is_ok() && !r.value().has_value());
    auto m = read_checkpoint_metadata(path);
    CHECK(m.is_ok() && !m.value().has_value());
    TRY(va, a.get_layer(0, TargetModule::QProj)->lora_a_tensor().to_vec_f32());
    TRY(vb, b.get_layer(0, TargetModule::QProj)->lora_a_tensor().to_vec_f32());
    CHECK(va == vb);  // bit for bit
    remove(path.c_str());
}

// A HIP adapter round trip, and errors: missing file, truncated file, wrong shape
CASE(checkpoint_hip_and_errors, true) {
    LoRAAdapterConfig c = ckpt_config();
    c.target_modules = {TargetModule::QProj, TargetModule::DownProj};
    TRY(a, LoRAAdapter::create(64, 96, 2, c, kHip, 5));
    const std::string path = tmp_path("mc_ckpt_hip.safetensors");
    CHECK(save_checkpoint(a, path, nullptr).is_ok());
    TRY(b, LoRAAdapter::create(64, 96, 2, c, kHip, 6));
    CHECK(load_checkpoint(b, path).is_ok());
    for (const auto& kv : a.layers()) {
        TRY(x, kv.second.lora_b_tensor().to_vec_f32());
        TRY(y, b.layers().at(kv.first).lora_b_tensor().to_vec_f32());
        CHECK(x == y);
    }
    TRY(wrong, LoRAAdapter::create(32, 96, 2, c, kHip, 7));  // different hidden size: shapes differ
    CHECK(load_checkpoint(wrong, path).is_err());
    CHECK(load_checkpoint(b, tmp_path("mc_no_such_file.safetensors")).is_err());
    FILE* f = fopen(path.c_str(), "r+b");
    if (f) {
        fseek(f, 0, SEEK_END);
        const long n = ftell(f);
        fclose(f);
        CHECK(truncate(path.c_str(), n - 5) == 0);
        CHECK(load_checkpoint(b, path).is_err());
    }
    remove(path.c_str());
}

// Malformed headers are errors, never exceptions: numbers past 2^64, a bad
// \u escape, a non-number loss, and a shape whose element count overflows
// (the safetensors crate rejects all of them with a validation error).
static void write_raw_safetensors(const std::string& path, std::string header, size_t data_bytes) {
    while (header.size() % 8) header += ' ';
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) return;
    const uint64_t n = header.size();
    unsigned char len[8];
    for (int i = 0; i < 8; ++i) len[i] = (unsigned char)(n >> (8 * i));
    fwrite(len, 1, 8, f);
    fwrite(header.data(), 1, header.size(), f);
    for (size_t i = 0; i < data_bytes; ++i) fputc(0, f);
    fclose(f);
}

CASE(checkpoint_malformed_headers, false) {
    const std::string path = tmp_path("mc_ckpt_bad.safetensors");
    const char* bad[] = {
        "{\"t\":{\"dtype\":\"F32\",\"shape\":[12345678901234567890123],\"data_offsets\":[0,0]}}",
        "{\"a\\uZZZZ\":{\"dtype\":\"F32\",\"shape\":[1],\"data_offsets\":[0,4]}}",
        "{\"t\":{\"dtype\":\"F32\",\"shape\":[4294967296,4294967296],\"data_offsets\":[0,0]}}",
        "{\"t\":{\"dtype\":\"F32\",\"shape\":[1],\"data_offsets\":[0,99999999999999999999999]}}",
    };
    for (const char* h : bad) {
        write_raw_safetensors(path, h, 4);
        auto r = safetensors_load(path, kCpu);
        CHECK(r.is_err());
    }
    // metadata with a loss that is not a number
    write_raw_safetensors(path,
                          "{\"__metadata__\":{\"checkpoint_metadata\":\"{\\\"global_step\\\":1,\\\"loss\\\":-,"
                          "\\\"learning_rate\\\":0.1,\\\"timestamp\\\":1}\"},"
                          "\"t\":{\"dtype\":\"F32\",\"shape\":[1],\"data_offsets\":[0,4]}}",
                          4);
    CHECK(safetensors_load(path, kCpu).is_ok());  // the container itself is valid
    CHECK(read_checkpoint_metadata(path).is_err());
    remove(path.c_str());
}

// Mutations of a valid checkpoint file: every truncation of the header and
// its length prefix, and byte substitutions at every header position with
// characters that matter to the JSON reader (quotes, brackets, digits,
// escapes, control bytes). Each load must return Ok or Err, never throw or
// read out of bounds (the sanitizer build of this program checks the
// latter). Deterministic; the file is small, so this runs in seconds.
CASE(checkpoint_mutated_files, false) {
    TRY(a, LoRAAdapter::create(8, 12, 1, ckpt_config(), kCpu, 21));
    const std::string good = tmp_path("mc_ckpt_mut_src.safetensors");
    const CheckpointMetadata md{7, 0.25f, 1e-3f, 42ull};
    CHECK(save_checkpoint(a, good, &md).is_ok());
    std::vector<unsigned char> bytes;
    if (FILE* f = fopen(good.c_str(), "rb")) {
        int ch;
        while ((ch = fgetc(f)) != EOF) bytes.push_back((unsigned char)ch);
        fclose(f);
    }
    CHECK(bytes.size() > 16);
    if (bytes.size() <= 16) return;
    uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= (uint64_t)bytes[(size_t)i] << (8 * i);
    const size_t hend = (size_t)std::min<uint64_t>(8 + hlen, bytes.size());
    const std::string path = tmp_path("mc_ckpt_mut.safetensors");
    auto write = [&](const std::vector<unsigned char>& b) {
        FILE* f = fopen(path.c_str(), "wb");
        if (!f) return false;
        if (!b.empty()) fwrite(b.data(), 1, b.size(), f);
        fclose(f);
        return true;
    };
    int loads = 0, errs = 0;
    auto try_load = [&](const std::vector<unsigned char>& b) {
        if (!write(b)) return;
        ++loads;
        auto r = safetensors_load(path, kCpu);
        auto m = read_checkpoint_metadata(path);
        TRY(dst, LoRAAdapter::create(8, 12, 1, ckpt_config(), kCpu, 22));
        auto l = load_checkpoint(dst, path);
        if (r.is_err() || m.is_err() || l.is_err()) ++errs;
    };
    for (size_t n = 0; n < hend; ++n) try_load(std::vector<unsigned char>(bytes.begin(), bytes.begin() + (long)n));
    const unsigned char subs[] = {'"', '{', '}', '[', ']', ',', ':', '\\', '-', '0', '9', 'e', 'u', 'E', ' ', 0, 0x7f,
                                  0xff};
    for (size_t i = 0; i < hend; ++i)
        for (unsigned char s : subs) {
            if (bytes[i] == s) continue;
            std::vector<unsigned char> b = bytes;
            b[i] = s;
            try_load(b);
        }
    // length prefixes past the file, at the file, and 0
    for (uint64_t v : {(uint64_t)0, (uint64_t)bytes.size(), (uint64_t)bytes.size() - 8, ~(uint64_t)0,
                       (uint64_t)1 << 40}) {
        std::vector<unsigned char> b = bytes;
        for (int i = 0; i < 8; ++i) b[(size_t)i] = (unsigned char)(v >> (8 * i));
        try_load(b);
    }
    CHECK(loads > 1000 && errs > 0);
    remove(path.c_str());
    remove(good.c_str());
}

// The file format against the safetensors library: tests/test_checkpoint_cpu.py
// writes py.safetensors with safetensors.numpy for the tensors below and runs
// this case with MC_CKPT_DIR set; this case writes cpp.safetensors for the same
// tensors (the Python side compares the bytes) and reads py.safetensors.
CASE(checkpoint_format, false) {
    if (!getenv("MC_CKPT_DIR")) return;  // driven by the Python test
    LoRAAdapterConfig c = ckpt_config();
    c.target_modules = {TargetModule::QProj, TargetModule::VProj, TargetModule::GateProj, TargetModule::DownProj};
    TRY(a, LoRAAdapter::create(16, 24, 2, c, kCpu, 8));
    // tensor k of the name-sorted list holds ((131 k + 17 i + 3 j) % 97) / 100 - 0.5 at [i][j]
    int k = 0;
    for (auto& kv : a.layers_mut()) {
        for (int ab = 0; ab < 2; ++ab, ++k) {
            const Tensor& t = ab == 0 ? kv.second.lora_a_tensor() : kv.second.lora_b_tensor();
            const int64_t R = t.dims()[0], C = t.dims()[1];
            std::vector<float> v((size_t)(R * C));
            for (int64_t i = 0; i < R; ++i)
                for (int64_t j = 0; j < C; ++j)
                    v[(size_t)(i * C + j)] = (float)((131 * k + 17 * i + 3 * j) % 97) / 100.f - 0.5f;
            TRY(nt, Tensor::from_slice(v, {R, C}, kCpu));
            CHECK((ab == 0 ? kv.second.set_lora_a(nt) : kv.second.set_lora_b(nt)).is_ok());
        }
    }
    const CheckpointMetadata md{100, 1.5f, 1e-4f, 1234567890ull};
    CHECK(save_checkpoint(a, tmp_path("cpp.safetensors"), &md).is_ok());
    TRY(b, LoRAAdapter::create(16, 24, 2, c, kCpu, 9));
    CHECK(load_checkpoint(b, tmp_path("py.safetensors")).is_ok());
    for (const auto& kv : a.layers()) {
        TRY(x, kv.second.lora_a_tensor().to_vec_f32());
        TRY(y, b.layers().at(kv.first).lora_a_tensor().to_vec_f32());
        TRY(x2, kv.second.lora_b_tensor().to_vec_f32());
        TRY(y2, b.layers().at(kv.first).lora_b_tensor().to_vec_f32());
        CHECK(x == y && x2 == y2);
    }
    auto m = read_checkpoint_metadata(tmp_path("py.safetensors"));
    CHECK(m.is_ok() && m.value().has_value() && m.value()->global_step == 100 && m.value()->timestamp == 1234567890ull);
}

// ================================================================== main
int main(int argc, char** argv) {
    bool gpu = false;
    std::string filter;
    for (int i = 1; i < argc; ++i) {
        if (!strcmp(argv[i], "--gpu")) gpu = true;
        else if (!strcmp(argv[i], "--cpu")) gpu = false;
        else filter = argv[i];
    }
    int run = 0, failed = 0;
    for (const Case& c : cases()) {
        if (c.gpu && !gpu) continue;
        if (!filter.empty() && std::string(c.name).find(filter) == std::string::npos) continue;
        printf("[ RUN    ] %s\n", c.name);
        fflush(stdout);
        g_failures_in_case = 0;
        c.fn();
        ++run;
        if (g_failures_in_case) {
            ++failed;
            printf("[ FAILED ] %s\n", c.name);
        } else {
            printf("[     OK ] %s\n", c.name);
        }
        fflush(stdout);
    }
    printf("%d cases, %d failed\n", run, failed);
    return failed ? 1 : 0;
}
