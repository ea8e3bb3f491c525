// mc_candle.hpp - C++ host side of the MI355X fused-op path, mirroring the
// operator / layer / executor interface of GarthDB/metal-candle v1.3.0 above
// the C ABI of libmc_hip.so (include/mc_hip.h).
//
// The reference is Rust over candle; this is the same interface in C++, so a
// caller (and the parity tests) use the names, argument meanings and error
// strings of the reference:
//
//   FusedLoRAOp, FusedRMSNormOp, FusedSoftmaxOp  src/backend/custom_ops.rs:73-824
//   lora_forward_fused / softmax_fused /
//   rms_norm_fused (CustomMetalOps)              src/backend/metal_ops.rs:33-171
//   LoRAConfig, LoRALayer                        src/training/lora.rs:49-560
//   Operation                                    src/graph/operation.rs:5-181
//   AsyncExecutor::execute_operation             src/graph/executor.rs:40-226
//   ComputationGraph, GraphNode                  src/graph/node.rs:1-300
//   LazyTensor, LoRALayer::forward_lazy          src/graph/lazy_tensor.rs:1-460,
//                                                src/training/lora.rs:372-439
//   TrainingError / Error display strings        src/error.rs:10-117
//
// Differences from the reference, all additive:
//   * ops run on HIP device tensors; a CPU tensor gets the reference's
//     "not implemented for CPU" error (there is no CPU compute here: on any
//     error the caller's own fallback applies, as in lora.rs:302-310);
//   * FusedLoRAOp also takes the frozen base weight, bias and a dropout mask,
//     and has a backward (dX, dA, dB); RMSNorm takes a weight and has a
//     backward; softmax takes a causal mask and has a backward;
//   * RMSNorm and softmax accept any rank >= 1 (leading dims are folded into
//     rows); the Metal kernels stop at rank 3 (custom_ops.rs:548-556, 741-749);
//   * Operation::output_shape of LoRA returns [..., out_features] (the
//     reference returns the input shape, operation.rs:139-150);
//   * LazyTensor::lora_fused merges the graphs of A and B into the input's,
//     as the binary ops do (the reference takes their node ids as they are,
//     lazy_tensor.rs:317-331, which is only right when A and B were added to
//     the input's graph, as forward_lazy does).
//
// All device work is enqueued on the null stream and every call that returns
// a host value synchronises through hipMemcpy. Output tensors are allocated
// here with hipMalloc (like the reference's op allocates its output buffer,
// custom_ops.rs:395-397); the C ABI underneath allocates nothing.
#pragma once

#include <stdint.h>

#include <map>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <vector>

namespace mc_candle {

// ------------------------------------------------------------------ errors
// candle_core::Error::Msg: the op-level error.
struct CandleError {
    std::string msg;
    std::string to_string() const { return msg; }
};

// crate::error::TrainingError (src/error.rs:94-117).
struct TrainingError {
    enum class Kind { InvalidLoRAConfig, InvalidConfig, Failed, StateError };
    Kind kind = Kind::Failed;
    std::string reason;
    static TrainingError failed(std::string r) { return {Kind::Failed, std::move(r)}; }
    static TrainingError invalid_config(std::string r) { return {Kind::InvalidConfig, std::move(r)}; }
    static TrainingError state_error(std::string r) { return {Kind::StateError, std::move(r)}; }
    std::string to_string() const;
};

// crate::error::Error: a candle error or a training error (src/error.rs:10-50).
struct Error {
    enum class Kind { Candle, Training };
    Kind kind = Kind::Candle;
    CandleError candle;
    TrainingError training;
    static Error from(CandleError e) { Error x; x.kind = Kind::Candle; x.candle = std::move(e); return x; }
    static Error from(TrainingError e) { Error x; x.kind = Kind::Training; x.training = std::move(e); return x; }
    std::string to_string() const;
};

// Rust's Result<T, E>.
template <class T, class E>
class Result {
public:
    Result(T v) : v_(std::move(v)) {}                      // NOLINT: implicit like Ok(v)
    Result(E e) : e_(std::move(e)) {}                      // NOLINT: implicit like Err(e)
    bool is_ok() const { return v_.has_value(); }
    bool is_err() const { return !v_.has_value(); }
    T& value() { return *v_; }
    const T& value() const { return *v_; }
    const E& error() const { return *e_; }
    T unwrap() && { return std::move(*v_); }
private:
    std::optional<T> v_;
    std::optional<E> e_;
};

template <class E>
class Result<void, E> {
public:
    Result() = default;
    Result(E e) : e_(std::move(e)) {}                      // NOLINT
    bool is_ok() const { return !e_.has_value(); }
    bool is_err() const { return e_.has_value(); }
    const E& error() const { return *e_; }
private:
    std::optional<E> e_;
};

// ------------------------------------------------------------------ tensors
enum class DType { F32, BF16, U8, U32 };

struct Device {
    enum class Kind { Cpu, Hip };
    Kind kind = Kind::Cpu;
    int ordinal = 0;
    static Device cpu() { return {Kind::Cpu, 0}; }
    static Device hip(int ordinal = 0) { return {Kind::Hip, ordinal}; }
    bool is_cpu() const { return kind == Kind::Cpu; }
    bool is_hip() const { return kind == Kind::Hip; }
};

std::string dims_to_string(const std::vector<int64_t>& dims);  // "[2, 3]", as {:?} of a dims slice

// Device memory of HIP tensors and op workspaces comes from a per-device
// caching pool (candle's Metal device pools its buffers likewise): released
// blocks are kept for reuse in stream order instead of being freed, so ops in
// a steady loop neither allocate nor synchronise the device. These return the
// cached blocks to the runtime, and report the bytes cached and the number of
// allocations served from the cache.
void release_cached_device_memory();
size_t cached_device_bytes();
size_t device_pool_hits();

// A contiguous row-major tensor in host memory (Device::cpu) or HIP device
// memory (Device::hip). Copies share storage, like candle's Arc'd storage.
class Tensor {
public:
    Tensor() = default;
    // Tensor::from_slice: values given as fp32, stored as `dtype` (bf16 is
    // rounded to nearest even; U8 truncates).
    static Result<Tensor, CandleError> from_slice(const std::vector<float>& data, std::vector<int64_t> dims,
                                                  const Device& device, DType dtype = DType::F32);
    static Result<Tensor, CandleError> from_bytes(const std::vector<uint8_t>& data, std::vector<int64_t> dims,
                                                  const Device& device);
    // U32 tensor (token ids), as Tensor::new(&[u32]) in candle.
    static Result<Tensor, CandleError> from_u32(const std::vector<uint32_t>& data, std::vector<int64_t> dims,
                                                const Device& device);
    static Result<Tensor, CandleError> zeros(std::vector<int64_t> dims, DType dtype, const Device& device);
    // Uninitialised storage (for outputs).
    static Result<Tensor, CandleError> empty(std::vector<int64_t> dims, DType dtype, const Device& device);

    Result<Tensor, CandleError> to_device(const Device& device) const;
    // Host copy as fp32 (the to_vec1 / flatten_all().to_vec1() of candle).
    Result<std::vector<float>, CandleError> to_vec_f32() const;

    const std::vector<int64_t>& dims() const { return dims_; }
    Result<int64_t, CandleError> dim(int64_t i) const;  // negative i counts from the end
    size_t rank() const { return dims_.size(); }
    int64_t elem_count() const;
    DType dtype() const { return dtype_; }
    const Device& device() const { return device_; }
    size_t size_bytes() const;
    void* data() const { return storage_.get(); }
    bool defined() const { return storage_ != nullptr || elem_count() == 0; }

private:
    std::vector<int64_t> dims_;
    DType dtype_ = DType::F32;
    Device device_;
    std::shared_ptr<void> storage_;
};

// ------------------------------------------------------------------ ops
// Saved state of a LoRA forward that the backward needs.
struct LoRASaved {
    Tensor hidden_t;   // Hd^T [r, T] fp32 (post-dropout, pre-scale hidden)
};

struct LoRAGrads {
    Tensor dx;         // like the input
    Tensor da;         // [K, r] fp32
    Tensor db;         // [r, N] fp32
};

// FusedLoRAOp (custom_ops.rs:73-431): y = scaling * (x A) B, extended with
// an optional frozen base linear (x W^T + b) and a dropout keep-mask.
class FusedLoRAOp {
public:
    // FusedLoRAOp::new (custom_ops.rs:118-150): A [K, r], B [r, N].
    static Result<FusedLoRAOp, CandleError> create(Tensor lora_a, Tensor lora_b, float scaling);
    const char* name() const { return "fused_lora_forward"; }

    // candle's apply_op1: dispatch on the input's device.
    Result<Tensor, CandleError> apply(const Tensor& input) const;
    Result<Tensor, CandleError> cpu_fwd(const Tensor& input) const;
    Result<Tensor, CandleError> hip_fwd(const Tensor& input) const;

    // Extensions. W [N, K] and bias [N] in the input's dtype (may be
    // undefined Tensors); mask [T, r] uint8 (1 = keep) with dropout_p > 0.
    Result<std::pair<Tensor, LoRASaved>, CandleError> forward_with_base(const Tensor& input, const Tensor* weight,
                                                                        const Tensor* bias, const Tensor* mask,
                                                                        float dropout_p) const;
    Result<LoRAGrads, CandleError> backward(const Tensor& input, const Tensor* weight, const LoRASaved& saved,
                                            const Tensor& grad_output, const Tensor* mask,
                                            float dropout_p) const;

    const Tensor& lora_a() const { return lora_a_; }
    const Tensor& lora_b() const { return lora_b_; }
    float scaling() const { return scaling_; }

private:
    // compute_output_shape (custom_ops.rs:153-174).
    Result<std::vector<int64_t>, CandleError> compute_output_shape(const std::vector<int64_t>& dims) const;
    Tensor lora_a_, lora_b_;
    float scaling_ = 1.f;
};

// FusedRMSNormOp (custom_ops.rs:443-632): y = x / sqrt(mean(x^2) + eps) [* w].
class FusedRMSNormOp {
public:
    static Result<FusedRMSNormOp, CandleError> create(float eps);
    const char* name() const { return "fused-rms-norm"; }
    Result<Tensor, CandleError> apply(const Tensor& input) const;
    Result<Tensor, CandleError> cpu_fwd(const Tensor& input) const;
    Result<Tensor, CandleError> hip_fwd(const Tensor& input) const;
    // Extensions: weight [dim] (Qwen RMSNorm, qwen.rs:314-325), saved rstd,
    // backward (dx, dw).
    Result<std::pair<Tensor, Tensor>, CandleError> forward_weighted(const Tensor& input, const Tensor* weight) const;
    Result<std::pair<Tensor, Tensor>, CandleError> backward(const Tensor& input, const Tensor* weight,
                                                            const Tensor& rstd, const Tensor& grad_output) const;
    float eps() const { return eps_; }

private:
    float eps_ = 1e-6f;
};

// FusedSoftmaxOp (custom_ops.rs:644-824): last-dim softmax.
class FusedSoftmaxOp {
public:
    static Result<FusedSoftmaxOp, CandleError> create();
    const char* name() const { return "fused-softmax"; }
    Result<Tensor, CandleError> apply(const Tensor& input) const;
    Result<Tensor, CandleError> cpu_fwd(const Tensor& input) const;
    Result<Tensor, CandleError> hip_fwd(const Tensor& input) const;
    // Extensions: causal mask over the last two dims (S = dims[-2]; the mask
    // of Attention::forward, transformer.rs:264-275) and the backward.
    Result<Tensor, CandleError> forward_causal(const Tensor& input, bool causal) const;
    Result<Tensor, CandleError> backward(const Tensor& probs, const Tensor& grad_output, bool causal) const;
};

// LayerNormOp (custom_ops.rs:826-1079): y = (x - mean) / sqrt(var + eps) over
// the last dim of a 2-D input, as the reference's op requires.
class LayerNormOp {
public:
    static LayerNormOp create(double eps) { return LayerNormOp(eps); }  // LayerNormOp::new
    const char* name() const { return "layer-norm"; }
    Result<Tensor, CandleError> apply(const Tensor& input) const;
    Result<Tensor, CandleError> cpu_fwd(const Tensor& input) const;
    Result<Tensor, CandleError> hip_fwd(const Tensor& input) const;
    // Extensions: the weight and bias of MetalLayerNorm (src/embeddings/
    // metal_bert.rs:30-72), any rank (leading dims folded), the saved
    // statistics and the backward.
    struct Saved {
        Tensor mean, rstd;  // fp32 [rows]
    };
    struct Grads {
        Tensor dx, dw, db;  // dw, db fp32 [dim] (undefined without weight / bias)
    };
    Result<std::pair<Tensor, Saved>, CandleError> forward_affine(const Tensor& input, const Tensor* weight,
                                                                 const Tensor* bias) const;
    Result<Grads, CandleError> backward(const Tensor& input, const Tensor* weight, const Saved& saved,
                                        const Tensor& grad_output) const;
    double eps() const { return eps_; }

private:
    explicit LayerNormOp(double eps) : eps_(eps) {}
    double eps_;
};

// TensorExt::layer_norm (tensor.rs:100-109): any rank, last dim, no affine.
Result<Tensor, CandleError> layer_norm(const Tensor& input, double eps);

// cross_entropy_loss (loss.rs:58-148) and cross_entropy_loss_with_smoothing
// (loss.rs:208-245) over HIP tensors: logits [batch, seq, vocab] (F32 or
// BF16), targets [batch, seq] U32; the scalar loss as a fp32 tensor of shape
// []. The reference's validation messages and its "all tokens are ignored"
// error (the count is read back, as the reference's to_scalar does).
Result<Tensor, Error> cross_entropy_loss(const Tensor& logits, const Tensor& targets,
                                         std::optional<uint32_t> ignore_index);
Result<Tensor, Error> cross_entropy_loss_with_smoothing(const Tensor& logits, const Tensor& targets, float smoothing,
                                                        std::optional<uint32_t> ignore_index);
// Extension: d loss / d logits for a loss gradient dloss (the reference has no backward).
Result<Tensor, Error> cross_entropy_loss_backward(const Tensor& logits, const Tensor& targets, float smoothing,
                                                  std::optional<uint32_t> ignore_index, float dloss = 1.0f);

// CustomMetalOps (metal_ops.rs:33-171), as free functions over HIP tensors.
Result<Tensor, TrainingError> lora_forward_fused(const Tensor& input, const Tensor& lora_a, const Tensor& lora_b,
                                                 float scaling);
Result<Tensor, TrainingError> softmax_fused(const Tensor& input);
Result<Tensor, TrainingError> rms_norm_fused(const Tensor& input, float eps);

class LazyTensor;

// ------------------------------------------------------------------ LoRA layer
// LoRAConfig (lora.rs:49-121).
struct LoRAConfig {
    size_t rank = 8;
    float alpha = 16.f;
    float dropout = 0.f;
    float scaling() const { return alpha / (float)rank; }
    Result<void, Error> validate() const;
};

// LoRALayer (lora.rs:123-560). A is initialised N(0, 1/sqrt(rank)) from a
// seeded host generator, B with zeros (lora.rs:233-247). In training mode with
// dropout > 0 the keep-mask of each forward is drawn with mc_dropout_mask from
// (seed, forward counter), so a CPU reference fed the same bytes reproduces it.
class LoRALayer {
public:
    static Result<LoRALayer, Error> create(size_t in_features, size_t out_features, const LoRAConfig& config,
                                           const Device& device, uint64_t seed = 0);
    // forward (lora.rs:292-342): scaling * (input A) B, dropout in training mode.
    Result<Tensor, Error> forward(const Tensor& input);
    // forward_lazy (lora.rs:372-439): records the forward into the input's
    // graph. On a HIP device with dropout 0 it is one fused LoRA node (A and B
    // added as inputs); otherwise the reference's composite (input A) B *
    // scaling, with no dropout, whose generic ops this library does not run.
    Result<LazyTensor, Error> forward_lazy(const LazyTensor& input) const;
    // Gradients of the most recent forward for grad_output = dL/dy (the candle
    // autograd of lora.rs:323-339): dX, dA, dB.
    Result<LoRAGrads, Error> backward(const Tensor& input, const Tensor& grad_output);

    size_t num_parameters() const { return config_.rank * (in_features_ + out_features_); }
    void set_training(bool training) { training_ = training; }
    void eval() { training_ = false; }
    bool is_training() const { return training_; }
    const Tensor& lora_a_tensor() const { return lora_a_; }
    const Tensor& lora_b_tensor() const { return lora_b_; }
    // Replaces A or B (same shape), e.g. after an optimizer step or a load.
    Result<void, Error> set_lora_a(Tensor a);
    Result<void, Error> set_lora_b(Tensor b);
    const LoRAConfig& config() const { return config_; }
    size_t in_features() const { return in_features_; }
    size_t out_features() const { return out_features_; }
    // Keep-mask [T, rank] of the most recent training-mode forward (undefined otherwise).
    const Tensor& last_mask() const { return mask_; }

private:
    Tensor lora_a_, lora_b_;
    LoRAConfig config_;
    size_t in_features_ = 0, out_features_ = 0;
    bool training_ = true;
    uint64_t seed_ = 0, step_ = 0;
    LoRASaved saved_;
    Tensor mask_;
    bool have_saved_ = false;
};

// ------------------------------------------------------------------ AdamW
// AdamWConfig (optimizer.rs:33-104): defaults and validate() with the
// reference's messages.
struct AdamWConfig {
    float learning_rate = 1e-4f;
    float beta1 = 0.9f;
    float beta2 = 0.999f;
    float epsilon = 1e-8f;
    float weight_decay = 0.01f;
    Result<void, Error> validate() const;
};

// AdamW (optimizer.rs:130-362) over fp32 HIP tensors. Like the reference,
// step() returns the updated parameter as a new tensor, keeps the moments per
// parameter name, and counts one step per step() call (the count is shared
// by all parameters and drives the bias correction). The update itself is
// one mc_adamw_step launch.
class AdamW {
public:
    static Result<AdamW, Error> create(const AdamWConfig& config);
    // add_parameter (optimizer.rs:196-205): zero moments of the param's shape.
    Result<void, Error> add_parameter(const std::string& name, const Tensor& param);
    // step (optimizer.rs:227-281).
    Result<Tensor, Error> step(const std::string& name, const Tensor& param, const Tensor& grad);
    void set_lr(float lr) { config_.learning_rate = lr; }
    float learning_rate() const { return config_.learning_rate; }
    size_t step_count() const { return step_count_; }
    const AdamWConfig& config() const { return config_; }
    // reset_state (optimizer.rs:333-349): step count 0, moments zeroed.
    void reset_state();

private:
    struct State {
        Tensor m, v;
    };
    AdamWConfig config_;
    std::vector<std::pair<std::string, State>> state_;
    size_t step_count_ = 0;
    State* find(const std::string& name);
};

// ------------------------------------------------------------------ adapter
// TargetModule (adapter.rs:12-58).
enum class TargetModule { QProj, KProj, VProj, OProj, GateProj, UpProj, DownProj };
const char* target_module_name(TargetModule m);
std::optional<TargetModule> target_module_from_name(const std::string& name);

// LoRAAdapterConfig (adapter.rs:60-100): defaults rank 8, alpha 16, q and v.
struct LoRAAdapterConfig {
    size_t rank = 8;
    float alpha = 16.f;
    float dropout = 0.f;
    std::vector<TargetModule> target_modules{TargetModule::QProj, TargetModule::VProj};
    LoRAConfig to_lora_config() const { return LoRAConfig{rank, alpha, dropout}; }
    bool is_target(TargetModule m) const;
};

// LoRAAdapter (adapter.rs:102-258): one LoRALayer per (layer, target module),
// keyed "layers.{i}.{module}"; q/k/v/o are hidden x hidden, gate/up hidden x
// intermediate, down intermediate x hidden (adapter.rs:193-206). layers()
// iterates in key order (the reference's HashMap has none).
class LoRAAdapter {
public:
    static Result<LoRAAdapter, Error> create(size_t hidden_size, size_t intermediate_size, size_t num_layers,
                                             const LoRAAdapterConfig& config, const Device& device,
                                             uint64_t seed = 0);
    // forward (adapter.rs:215-231): the layer's delta, or nullopt when the
    // module is not adapted.
    Result<std::optional<Tensor>, Error> forward(size_t layer_idx, TargetModule module, const Tensor& input);
    size_t num_trainable_parameters() const;
    size_t num_frozen_parameters(size_t total_model_params) const;
    const LoRAAdapterConfig& config() const { return config_; }
    size_t num_layers() const { return num_layers_; }
    const std::map<std::string, LoRALayer>& layers() const { return layers_; }
    std::map<std::string, LoRALayer>& layers_mut() { return layers_; }
    const LoRALayer* get_layer(size_t layer_idx, TargetModule module) const;
    LoRALayer* get_layer_mut(size_t layer_idx, TargetModule module);

private:
    std::map<std::string, LoRALayer> layers_;
    LoRAAdapterConfig config_;
    size_t num_layers_ = 0;
};

// ------------------------------------------------------------------ checkpoints
// CheckpointMetadata (checkpoint.rs:11-27), stored as the JSON string of the
// safetensors metadata entry "checkpoint_metadata" in serde_json's form.
struct CheckpointMetadata {
    uint64_t global_step = 0;
    float loss = 0.f;
    float learning_rate = 0.f;
    uint64_t timestamp = 0;
    std::string to_json() const;
    static std::optional<CheckpointMetadata> from_json(const std::string& json);
};

// save_checkpoint (checkpoint.rs:29-66): every layer's A and B as
// "{key}.lora_a" / "{key}.lora_b" (F32) in one safetensors file, with the
// metadata entry when given. The file's bytes are what the safetensors crate
// writes for the same tensors (header, order, padding).
Result<void, Error> save_checkpoint(const LoRAAdapter& adapter, const std::string& path,
                                    const CheckpointMetadata* metadata);
// load_checkpoint (checkpoint.rs:68-103): sets A and B of every layer whose
// keys are in the file (others keep their values) and, as the reference,
// returns no metadata (read_checkpoint_metadata reads it).
Result<std::optional<CheckpointMetadata>, Error> load_checkpoint(LoRAAdapter& adapter, const std::string& path);
Result<std::optional<CheckpointMetadata>, Error> read_checkpoint_metadata(const std::string& path);

// The safetensors container (the format of the safetensors crate): an 8-byte
// little-endian header length, a JSON header (optional "__metadata__" string
// map, then per tensor dtype / shape / data_offsets) padded with spaces to a
// multiple of 8, then the tensors' little-endian bytes. Tensors are written
// in the crate's order: dtype descending, then name.
Result<void, Error> safetensors_save(const std::vector<std::pair<std::string, Tensor>>& tensors,
                                     const std::map<std::string, std::string>* metadata, const std::string& path);
Result<std::map<std::string, Tensor>, Error> safetensors_load(const std::string& path, const Device& device,
                                                              std::map<std::string, std::string>* metadata = nullptr);

// ------------------------------------------------------------------ graph
struct NodeId {
    size_t id = 0;
};

// Operation (operation.rs:5-181).
struct Operation {
    enum class Kind { Input, Matmul, Add, Mul, MulScalar, LoRA, Softmax, RMSNorm };
    Kind kind = Kind::Input;
    float value = 0.f;      // MulScalar
    NodeId a, b;            // LoRA
    float scale = 1.f;      // LoRA
    size_t dim = 0;         // Softmax
    float eps = 1e-5f;      // RMSNorm

    static Operation input() { return {}; }
    static Operation matmul() { Operation o; o.kind = Kind::Matmul; return o; }
    static Operation add() { Operation o; o.kind = Kind::Add; return o; }
    static Operation mul() { Operation o; o.kind = Kind::Mul; return o; }
    static Operation mul_scalar(float v) { Operation o; o.kind = Kind::MulScalar; o.value = v; return o; }
    static Operation lora(NodeId a, NodeId b, float scale) {
        Operation o; o.kind = Kind::LoRA; o.a = a; o.b = b; o.scale = scale; return o;
    }
    static Operation softmax(size_t dim) { Operation o; o.kind = Kind::Softmax; o.dim = dim; return o; }
    static Operation rms_norm(float eps) { Operation o; o.kind = Kind::RMSNorm; o.eps = eps; return o; }

    const char* name() const;
    Result<std::vector<int64_t>, std::string> output_shape(const std::vector<std::vector<int64_t>>& input_shapes) const;
    // operation.rs:170-180: the first input's dtype.
    DType output_dtype(const std::vector<DType>& input_dtypes) const;
};

std::string node_id_string(NodeId id);  // "NodeId(3)", as {:?} of a NodeId

// AsyncExecutor (executor.rs:20-226). The fused ops (LoRA, Softmax, RMSNorm)
// run on HIP tensors through libmc_hip.so; the generic ops (Matmul, Add, Mul,
// MulScalar) are candle's and return an error here after the reference's
// input-count checks.
class AsyncExecutor {
public:
    static Result<AsyncExecutor, TrainingError> create(const Device& device);
    Result<Tensor, TrainingError> execute_operation(const Operation& op, const std::vector<Tensor>& inputs);
    Result<void, TrainingError> synchronize();
    const Device& device() const { return device_; }
    std::string debug_string() const;

private:
    Device device_;
};

// ------------------------------------------------------------------ lazy graph
// GraphNode and NodeData (node.rs:1-120): an input node holds its tensor
// (Concrete); an operation node is Lazy until eval stores its result
// (Available).
struct GraphNode {
    enum class Data { Concrete, Lazy, Available };
    NodeId id;
    Operation operation;
    std::vector<NodeId> inputs;
    std::vector<int64_t> output_shape;
    DType output_dtype = DType::F32;
    Data data = Data::Lazy;
    Tensor tensor;  // the node's value when data != Lazy
    bool is_available() const { return data != Data::Lazy; }
};

// ComputationGraph (node.rs:122-300): nodes in insertion order, a node's id
// is its index.
class ComputationGraph {
public:
    explicit ComputationGraph(const Device& device) : device_(device) {}
    const Device& device() const { return device_; }
    size_t len() const { return nodes_.size(); }
    bool is_empty() const { return nodes_.empty(); }
    Result<const GraphNode*, std::string> get_node(NodeId id) const;
    Result<GraphNode*, std::string> get_node_mut(NodeId id);
    NodeId add_input(const Tensor& tensor);
    // Shape and dtype inference from the inputs; an unknown input is an error.
    Result<NodeId, std::string> add_node(const Operation& op, const std::vector<NodeId>& inputs);
    // Dependencies first (post-order depth-first from `output`).
    Result<std::vector<NodeId>, std::string> topological_order(NodeId output) const;
    // Copies `target` and everything it depends on from `other` into this
    // graph; returns target's id here.
    NodeId merge_from(const ComputationGraph& other, NodeId target);

private:
    std::vector<GraphNode> nodes_;
    Device device_;
};

// LazyTensor (lazy_tensor.rs): records operations into a graph shared by the
// tensors built from one another (copies share it, as the reference's
// Arc<RwLock<ComputationGraph>>) and runs them through AsyncExecutor on
// eval(). Shape and dtype are known without evaluating.
class LazyTensor {
public:
    static Result<LazyTensor, CandleError> from_slice(const std::vector<float>& data, std::vector<int64_t> dims,
                                                      const Device& device);
    static Result<LazyTensor, CandleError> from_tensor(const Tensor& tensor);
    static Result<LazyTensor, CandleError> zeros(std::vector<int64_t> dims, DType dtype, const Device& device);
    static Result<LazyTensor, CandleError> ones(std::vector<int64_t> dims, DType dtype, const Device& device);
    // A tensor as a new input node of this tensor's graph.
    Result<LazyTensor, CandleError> add_tensor_to_graph(const Tensor& tensor) const;

    const std::vector<int64_t>& shape() const { return shape_; }
    DType dtype() const { return dtype_; }
    const Device& device() const { return device_; }
    NodeId node_id() const { return node_; }
    size_t graph_size() const;
    bool is_evaluated() const;
    bool shares_graph_with(const LazyTensor& other) const { return graph_ == other.graph_; }

    Result<LazyTensor, CandleError> matmul(const LazyTensor& other) const;
    Result<LazyTensor, CandleError> add(const LazyTensor& other) const;
    Result<LazyTensor, CandleError> mul(const LazyTensor& other) const;
    Result<LazyTensor, CandleError> mul_scalar(float value) const;
    Result<LazyTensor, CandleError> softmax(size_t dim) const;
    Result<LazyTensor, CandleError> rms_norm(float eps) const;
    Result<LazyTensor, CandleError> lora_fused(const LazyTensor& lora_a, const LazyTensor& lora_b, float scale) const;

    // Runs every node this one depends on that has no value yet, in
    // dependency order, then synchronises (lazy_tensor.rs:342-424).
    Result<Tensor, TrainingError> eval() const;
    std::string debug_string() const;

    struct Shared;  // the graph and its lock

private:
    LazyTensor() = default;
    NodeId merge_graph_from(const LazyTensor& other) const;
    Result<LazyTensor, CandleError> add_operation(const Operation& op, const std::vector<NodeId>& inputs) const;

    NodeId node_;
    std::shared_ptr<Shared> graph_;
    std::vector<int64_t> shape_;
    DType dtype_ = DType::F32;
    Device device_;
};

}  // namespace mc_candle
