// mc_candle.cpp - implementation of the C++ host interface (mc_candle.hpp)
// over the C ABI of libmc_hip.so. No arithmetic on tensor data happens here
// (apart from dtype conversion of host copies): every op is one or more
// mc_* calls, and an mc_* error becomes the op's error.
#include "mc_candle.hpp"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <string.h>

#include <functional>
#include <mutex>
#include <random>
#include <sstream>
#include <unordered_map>
#include <unordered_set>

#include "mc_hip.h"

namespace mc_candle {

// ------------------------------------------------------------------ errors
std::string TrainingError::to_string() const {
    switch (kind) {  // src/error.rs:97-114
        case Kind::InvalidLoRAConfig: return "invalid LoRA configuration: " + reason;
        case Kind::InvalidConfig: return "invalid training configuration: " + reason;
        case Kind::StateError: return "training state error: " + reason;
        default: return "training failed: " + reason;
    }
}

std::string Error::to_string() const {
    // src/error.rs:18-44: "training error: {0}", "candle error: {0}".
    return kind == Kind::Training ? "training error: " + training.to_string() : "candle error: " + candle.to_string();
}

namespace {

CandleError bail(std::string msg) { return CandleError{std::move(msg)}; }

CandleError mc_error(const char* what, mc_status st) {
    std::ostringstream s;
    s << what << " failed (status " << (int)st << "): " << mc_last_error();
    return bail(s.str());
}

CandleError hip_error(const char* what, hipError_t e) {
    std::ostringstream s;
    s << what << ": " << hipGetErrorString(e);
    return bail(s.str());
}

size_t dtype_size(DType d) { return d == DType::F32 || d == DType::U32 ? 4 : d == DType::BF16 ? 2 : 1; }

int32_t mc_dtype_of(DType d) { return d == DType::BF16 ? MC_BF16 : MC_F32; }

uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);                                             // round to nearest even
    return (uint16_t)(u >> 16);
}

float bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int64_t product(const std::vector<int64_t>& d, size_t from, size_t to) {
    int64_t p = 1;
    for (size_t i = from; i < to; ++i) p *= d[i];
    return p;
}

// Caching allocator of device memory, as candle's Metal device keeps a pool
// of buffers instead of allocating per op. Blocks are sized in 256-byte
// units below 1 MiB and in 1/8-octave steps above, and a released block goes
// back to its device's free list rather than to hipFree, which would wait for
// the device. Every op of this interface enqueues on the null stream, so a
// block released after its last op and handed to a later op is reused in
// stream order: the later op's kernels run after the earlier ones finish.
// The pool lives until the process ends (release_cached_device_memory()
// returns its free blocks to the runtime).
class DevicePool {
  public:
    static DevicePool& get() {
        static DevicePool* pool = new DevicePool();  // never destroyed: tensors may outlive static teardown
        return *pool;
    }
    static size_t bucket(size_t bytes) {
        if (bytes <= ((size_t)1 << 20)) return (bytes + 255) & ~(size_t)255;
        size_t p = (size_t)1 << 20;
        while (p * 2 <= bytes) p *= 2;
        const size_t step = p / 8;
        return (bytes + step - 1) / step * step;
    }
    hipError_t alloc(int device, size_t bytes, void** out) {
        const size_t b = bucket(bytes);
        {
            std::lock_guard<std::mutex> lk(mu_);
            auto& fl = free_[device];
            auto it = fl.find(b);
            if (it != fl.end() && !it->second.empty()) {
                *out = it->second.back();
                it->second.pop_back();
                cached_ -= b;
                ++hits_;
                return hipSuccess;
            }
        }
        hipError_t e = hipMalloc(out, b);
        if (e == hipErrorOutOfMemory) {  // give the cached blocks back and try once more
            release();
            e = hipMalloc(out, b);
        }
        return e;
    }
    void free(int device, size_t bytes, void* p) {
        std::lock_guard<std::mutex> lk(mu_);
        free_[device][bucket(bytes)].push_back(p);
        cached_ += bucket(bytes);
    }
    void release() {
        std::lock_guard<std::mutex> lk(mu_);
        for (auto& dev : free_)
            for (auto& kv : dev.second)
                for (void* p : kv.second) (void)hipFree(p);
        free_.clear();
        cached_ = 0;
    }
    size_t cached() {
        std::lock_guard<std::mutex> lk(mu_);
        return cached_;
    }
    size_t hits() {
        std::lock_guard<std::mutex> lk(mu_);
        return hits_;
    }

  private:
    std::mutex mu_;
    std::unordered_map<int, std::unordered_map<size_t, std::vector<void*>>> free_;
    size_t cached_ = 0, hits_ = 0;
};

// Device-resident workspace for one call, from the pool.
struct Workspace {
    void* p = nullptr;
    int device = 0;
    size_t bytes = 0;
    ~Workspace() {
        if (p) DevicePool::get().free(device, bytes, p);
    }
};

Result<void, CandleError> alloc_ws(Workspace& ws, size_t bytes) {
    if (bytes == 0) return {};
    hipError_t e = hipGetDevice(&ws.device);
    if (e != hipSuccess) return hip_error("workspace allocation", e);
    e = DevicePool::get().alloc(ws.device, bytes, &ws.p);
    if (e != hipSuccess) return hip_error("workspace allocation", e);
    ws.bytes = bytes;
    return {};
}

bool same_device(const Tensor& a, const Tensor& b) {
    return a.device().kind == b.device().kind && a.device().ordinal == b.device().ordinal;
}

}  // namespace

void release_cached_device_memory() { DevicePool::get().release(); }
size_t cached_device_bytes() { return DevicePool::get().cached(); }
size_t device_pool_hits() { return DevicePool::get().hits(); }

std::string dims_to_string(const std::vector<int64_t>& dims) {
    std::ostringstream s;
    s << "[";
    for (size_t i = 0; i < dims.size(); ++i) s << (i ? ", " : "") << dims[i];
    s << "]";
    return s.str();
}

// ------------------------------------------------------------------ tensors
int64_t Tensor::elem_count() const { return product(dims_, 0, dims_.size()); }

size_t Tensor::size_bytes() const { return (size_t)elem_count() * dtype_size(dtype_); }

Result<int64_t, CandleError> Tensor::dim(int64_t i) const {
    const int64_t r = (int64_t)dims_.size();
    const int64_t j = i < 0 ? r + i : i;
    if (j < 0 || j >= r) return bail("DimOutOfRange: dim " + std::to_string(i) + " of shape " + dims_to_string(dims_));
    return dims_[(size_t)j];
}

Result<Tensor, CandleError> Tensor::empty(std::vector<int64_t> dims, DType dtype, const Device& device) {
    for (int64_t d : dims)
        if (d < 0) return bail("negative dimension in shape " + dims_to_string(dims));
    Tensor t;
    t.dims_ = std::move(dims);
    t.dtype_ = dtype;
    t.device_ = device;
    const size_t bytes = t.size_bytes();
    if (bytes == 0) return t;
    if (device.is_cpu()) {
        void* p = ::operator new(bytes);
        t.storage_ = std::shared_ptr<void>(p, [](void* q) { ::operator delete(q); });
    } else {
        hipError_t e = hipSetDevice(device.ordinal);
        if (e != hipSuccess) return hip_error("hipSetDevice", e);
        void* p = nullptr;
        e = DevicePool::get().alloc(device.ordinal, bytes, &p);
        if (e != hipSuccess) return hip_error("hipMalloc", e);
        const int ord = device.ordinal;
        t.storage_ = std::shared_ptr<void>(p, [ord, bytes](void* q) { DevicePool::get().free(ord, bytes, q); });
    }
    return t;
}

Result<Tensor, CandleError> Tensor::zeros(std::vector<int64_t> dims, DType dtype, const Device& device) {
    auto r = empty(std::move(dims), dtype, device);
    if (r.is_err() || r.value().size_bytes() == 0) return r;
    Tensor& t = r.value();
    if (device.is_cpu()) {
        memset(t.data(), 0, t.size_bytes());
    } else {
        hipError_t e = hipMemset(t.data(), 0, t.size_bytes());
        if (e != hipSuccess) return hip_error("hipMemset", e);
    }
    return r;
}

Result<Tensor, CandleError> Tensor::from_slice(const std::vector<float>& data, std::vector<int64_t> dims,
                                               const Device& device, DType dtype) {
    if ((int64_t)data.size() != product(dims, 0, dims.size()))
        return bail("shape mismatch in from_slice, got buffer of size " + std::to_string(data.size()) +
                    " which is incompatible with shape " + dims_to_string(dims));
    std::vector<uint8_t> host(data.size() * dtype_size(dtype));
    for (size_t i = 0; i < data.size(); ++i) {
        if (dtype == DType::F32) {
            memcpy(&host[i * 4], &data[i], 4);
        } else if (dtype == DType::BF16) {
            const uint16_t h = f32_to_bf16(data[i]);
            memcpy(&host[i * 2], &h, 2);
        } else if (dtype == DType::U32) {
            const uint32_t u = (uint32_t)data[i];
            memcpy(&host[i * 4], &u, 4);
        } else {
            host[i] = (uint8_t)data[i];
        }
    }
    auto r = empty(std::move(dims), dtype, device);
    if (r.is_err() || host.empty()) return r;
    Tensor& t = r.value();
    if (device.is_cpu()) {
        memcpy(t.data(), host.data(), host.size());
    } else {
        hipError_t e = hipMemcpy(t.data(), host.data(), host.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_error("hipMemcpy H2D", e);
    }
    return r;
}

Result<Tensor, CandleError> Tensor::from_bytes(const std::vector<uint8_t>& data, std::vector<int64_t> dims,
                                               const Device& device) {
    if ((int64_t)data.size() != product(dims, 0, dims.size()))
        return bail("shape mismatch in from_bytes for shape " + dims_to_string(dims));
    auto r = empty(std::move(dims), DType::U8, device);
    if (r.is_err() || data.empty()) return r;
    Tensor& t = r.value();
    if (device.is_cpu()) {
        memcpy(t.data(), data.data(), data.size());
    } else {
        hipError_t e = hipMemcpy(t.data(), data.data(), data.size(), hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_error("hipMemcpy H2D", e);
    }
    return r;
}

Result<Tensor, CandleError> Tensor::from_u32(const std::vector<uint32_t>& data, std::vector<int64_t> dims,
                                             const Device& device) {
    if ((int64_t)data.size() != product(dims, 0, dims.size()))
        return bail("shape mismatch in from_u32 for shape " + dims_to_string(dims));
    auto r = empty(std::move(dims), DType::U32, device);
    if (r.is_err() || data.empty()) return r;
    Tensor& t = r.value();
    const size_t bytes = data.size() * 4;
    if (device.is_cpu()) {
        memcpy(t.data(), data.data(), bytes);
    } else {
        hipError_t e = hipMemcpy(t.data(), data.data(), bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_error("hipMemcpy H2D", e);
    }
    return r;
}

Result<Tensor, CandleError> Tensor::to_device(const Device& device) const {
    auto r = empty(dims_, dtype_, device);
    if (r.is_err() || size_bytes() == 0) return r;
    Tensor& t = r.value();
    hipMemcpyKind kind = device_.is_cpu() ? (device.is_cpu() ? hipMemcpyHostToHost : hipMemcpyHostToDevice)
                                          : (device.is_cpu() ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice);
    if (kind == hipMemcpyHostToHost) {
        memcpy(t.data(), data(), size_bytes());
        return r;
    }
    hipError_t e = hipMemcpy(t.data(), data(), size_bytes(), kind);
    if (e != hipSuccess) return hip_error("hipMemcpy", e);
    return r;
}

Result<std::vector<float>, CandleError> Tensor::to_vec_f32() const {
    std::vector<uint8_t> host(size_bytes());
    if (!host.empty()) {
        if (device_.is_cpu()) {
            memcpy(host.data(), data(), host.size());
        } else {
            hipError_t e = hipMemcpy(host.data(), data(), host.size(), hipMemcpyDeviceToHost);
            if (e != hipSuccess) return hip_error("hipMemcpy D2H", e);
        }
    }
    std::vector<float> out((size_t)elem_count());
    for (size_t i = 0; i < out.size(); ++i) {
        if (dtype_ == DType::F32) {
            memcpy(&out[i], &host[i * 4], 4);
        } else if (dtype_ == DType::BF16) {
            uint16_t h;
            memcpy(&h, &host[i * 2], 2);
            out[i] = bf16_to_f32(h);
        } else if (dtype_ == DType::U32) {
            uint32_t u;
            memcpy(&u, &host[i * 4], 4);
            out[i] = (float)u;
        } else {
            out[i] = (float)host[i];
        }
    }
    return out;
}

// ------------------------------------------------------------------ FusedLoRAOp
Result<FusedLoRAOp, CandleError> FusedLoRAOp::create(Tensor lora_a, Tensor lora_b, float scaling) {
    // custom_ops.rs:118-150
    if (lora_a.rank() != 2 || lora_b.rank() != 2)
        return bail("LoRA matrices must be 2D, got shapes " + dims_to_string(lora_a.dims()) + " and " +
                    dims_to_string(lora_b.dims()));
    if (lora_a.dims()[1] != lora_b.dims()[0]) {
        std::ostringstream s;
        s << "Incompatible LoRA matrix dimensions: " << lora_a.dims()[0] << "×" << lora_a.dims()[1] << " and "
          << lora_b.dims()[0] << "×" << lora_b.dims()[1];
        return bail(s.str());
    }
    FusedLoRAOp op;
    op.lora_a_ = std::move(lora_a);
    op.lora_b_ = std::move(lora_b);
    op.scaling_ = scaling;
    return op;
}

Result<std::vector<int64_t>, CandleError> FusedLoRAOp::compute_output_shape(const std::vector<int64_t>& dims) const {
    if (dims.empty()) return bail("Input must have at least 1 dimension");
    const int64_t in_features = dims.back();
    const int64_t expected_in = lora_a_.dims()[0];
    if (in_features != expected_in)
        return bail("Input feature dimension mismatch: expected " + std::to_string(expected_in) + ", got " +
                    std::to_string(in_features));
    std::vector<int64_t> out = dims;
    out.back() = lora_b_.dims()[1];
    return out;
}

Result<Tensor, CandleError> FusedLoRAOp::apply(const Tensor& input) const {
    return input.device().is_hip() ? hip_fwd(input) : cpu_fwd(input);
}

Result<Tensor, CandleError> FusedLoRAOp::cpu_fwd(const Tensor&) const {
    // custom_ops.rs:235-245
    return bail("FusedLoRAOp is HIP-only. Use standard LoRA operations on CPU or move tensors to a HIP device.");
}

Result<Tensor, CandleError> FusedLoRAOp::hip_fwd(const Tensor& input) const {
    auto r = forward_with_base(input, nullptr, nullptr, nullptr, 0.f);
    if (r.is_err()) return r.error();
    return std::move(r.value().first);
}

Result<std::pair<Tensor, LoRASaved>, CandleError> FusedLoRAOp::forward_with_base(const Tensor& input,
                                                                                 const Tensor* weight,
                                                                                 const Tensor* bias,
                                                                                 const Tensor* mask,
                                                                                 float dropout_p) const {
    if (!input.device().is_hip()) return cpu_fwd(input).error();
    auto shape = compute_output_shape(input.dims());
    if (shape.is_err()) return shape.error();
    if (!lora_a_.device().is_hip() || !same_device(lora_a_, input)) return bail("LoRA_A must be on HIP device");
    if (!lora_b_.device().is_hip() || !same_device(lora_b_, input)) return bail("LoRA_B must be on HIP device");
    if (lora_a_.dtype() != DType::F32 || lora_b_.dtype() != DType::F32)
        return bail("LoRA_A and LoRA_B must be F32");
    if (input.dtype() == DType::U8) return bail("fused_lora: input must be F32 or BF16");
    const int64_t K = lora_a_.dims()[0], r = lora_a_.dims()[1], N = lora_b_.dims()[1];
    const int64_t T = input.elem_count() / (K ? K : 1);
    if (weight && (weight->dims() != std::vector<int64_t>{N, K} || weight->dtype() != input.dtype() ||
                   !same_device(*weight, input)))
        return bail("fused_lora: weight must be [" + std::to_string(N) + ", " + std::to_string(K) +
                    "] in the input's dtype on its device, got " + dims_to_string(weight->dims()));
    if (bias && (bias->dims() != std::vector<int64_t>{N} || bias->dtype() != input.dtype() ||
                 !same_device(*bias, input)))
        return bail("fused_lora: bias must be [" + std::to_string(N) + "] in the input's dtype on its device");
    if (mask && (mask->dims() != std::vector<int64_t>{T, r} || mask->dtype() != DType::U8 ||
                 !same_device(*mask, input)))
        return bail("fused_lora: dropout mask must be U8 [" + std::to_string(T) + ", " + std::to_string(r) + "]");

    auto y = Tensor::empty(shape.value(), input.dtype(), input.device());
    if (y.is_err()) return y.error();
    auto h = Tensor::empty({r, T}, DType::F32, input.device());
    if (h.is_err()) return h.error();
    mc_lora_desc d{T, K, N, (int32_t)r, scaling_, dropout_p, mc_dtype_of(input.dtype())};
    Workspace ws;
    const size_t ws_bytes = mc_lora_fwd_workspace_size(&d);
    auto a = alloc_ws(ws, ws_bytes);
    if (a.is_err()) return a.error();
    const mc_status st = mc_lora_fwd(&d, input.data(), weight ? weight->data() : nullptr,
                                     bias ? bias->data() : nullptr, static_cast<const float*>(lora_a_.data()),
                                     static_cast<const float*>(lora_b_.data()),
                                     mask ? static_cast<const uint8_t*>(mask->data()) : nullptr, y.value().data(),
                                     static_cast<float*>(h.value().data()), ws.p, ws_bytes, nullptr);
    if (st != MC_OK) return mc_error("fused_lora_forward", st);
    return std::make_pair(std::move(y.value()), LoRASaved{std::move(h.value())});
}

Result<LoRAGrads, CandleError> FusedLoRAOp::backward(const Tensor& input, const Tensor* weight,
                                                     const LoRASaved& saved, const Tensor& grad_output,
                                                     const Tensor* mask, float dropout_p) const {
    if (!input.device().is_hip()) return cpu_fwd(input).error();
    auto shape = compute_output_shape(input.dims());
    if (shape.is_err()) return shape.error();
    if (grad_output.dims() != shape.value() || grad_output.dtype() != input.dtype())
        return bail("fused_lora backward: grad_output must have shape " + dims_to_string(shape.value()) +
                    " and the input's dtype, got " + dims_to_string(grad_output.dims()));
    const int64_t K = lora_a_.dims()[0], r = lora_a_.dims()[1], N = lora_b_.dims()[1];
    const int64_t T = input.elem_count() / (K ? K : 1);
    if (saved.hidden_t.dims() != std::vector<int64_t>{r, T} || saved.hidden_t.dtype() != DType::F32)
        return bail("fused_lora backward: saved hidden must be F32 [" + std::to_string(r) + ", " +
                    std::to_string(T) + "]");
    if (weight && (weight->dims() != std::vector<int64_t>{N, K} || weight->dtype() != input.dtype()))
        return bail("fused_lora backward: weight must be [" + std::to_string(N) + ", " + std::to_string(K) + "]");
    if (mask && (mask->dims() != std::vector<int64_t>{T, r} || mask->dtype() != DType::U8))
        return bail("fused_lora backward: dropout mask must be U8 [" + std::to_string(T) + ", " +
                    std::to_string(r) + "]");
    auto dx = Tensor::empty(input.dims(), input.dtype(), input.device());
    auto da = Tensor::empty({K, r}, DType::F32, input.device());
    auto db = Tensor::empty({r, N}, DType::F32, input.device());
    if (dx.is_err()) return dx.error();
    if (da.is_err()) return da.error();
    if (db.is_err()) return db.error();
    mc_lora_desc d{T, K, N, (int32_t)r, scaling_, dropout_p, mc_dtype_of(input.dtype())};
    Workspace ws;
    const size_t ws_bytes = mc_lora_bwd_workspace_size(&d);
    auto a = alloc_ws(ws, ws_bytes);
    if (a.is_err()) return a.error();
    const mc_status st = mc_lora_bwd(
        &d, input.data(), weight ? weight->data() : nullptr, static_cast<const float*>(lora_a_.data()),
        static_cast<const float*>(lora_b_.data()), mask ? static_cast<const uint8_t*>(mask->data()) : nullptr,
        static_cast<const float*>(saved.hidden_t.data()), grad_output.data(), dx.value().data(),
        static_cast<float*>(da.value().data()), static_cast<float*>(db.value().data()), ws.p, ws_bytes, nullptr);
    if (st != MC_OK) return mc_error("fused_lora_backward", st);
    return LoRAGrads{std::move(dx.value()), std::move(da.value()), std::move(db.value())};
}

// ------------------------------------------------------------------ FusedRMSNormOp
Result<FusedRMSNormOp, CandleError> FusedRMSNormOp::create(float eps) {
    FusedRMSNormOp op;
    op.eps_ = eps;
    return op;
}

Result<Tensor, CandleError> FusedRMSNormOp::apply(const Tensor& input) const {
    return input.device().is_hip() ? hip_fwd(input) : cpu_fwd(input);
}

Result<Tensor, CandleError> FusedRMSNormOp::cpu_fwd(const Tensor&) const {
    // custom_ops.rs:526-532
    return bail("Fused RMS Norm kernel not implemented for CPU. Use a HIP device.");
}

Result<Tensor, CandleError> FusedRMSNormOp::hip_fwd(const Tensor& input) const {
    auto r = forward_weighted(input, nullptr);
    if (r.is_err()) return r.error();
    return std::move(r.value().first);
}

Result<std::pair<Tensor, Tensor>, CandleError> FusedRMSNormOp::forward_weighted(const Tensor& input,
                                                                                const Tensor* weight) const {
    if (!input.device().is_hip()) return cpu_fwd(input).error();
    if (input.rank() == 0)
        return bail("Input tensor for FusedRMSNormOp must have at least 1 dimension, got " +
                    dims_to_string(input.dims()));
    if (input.dtype() == DType::U8) return bail("fused-rms-norm: input must be F32 or BF16");
    const int64_t dim = input.dims().back();
    const int64_t rows = dim ? input.elem_count() / dim : 0;
    if (weight && (weight->dims() != std::vector<int64_t>{dim} || weight->dtype() != input.dtype() ||
                   !same_device(*weight, input)))
        return bail("fused-rms-norm: weight must be [" + std::to_string(dim) + "] in the input's dtype");
    auto y = Tensor::empty(input.dims(), input.dtype(), input.device());
    auto rstd = Tensor::empty({rows}, DType::F32, input.device());
    if (y.is_err()) return y.error();
    if (rstd.is_err()) return rstd.error();
    const mc_status st = mc_rmsnorm_fwd(rows, dim, eps_, mc_dtype_of(input.dtype()), input.data(),
                                        weight ? weight->data() : nullptr, y.value().data(),
                                        static_cast<float*>(rstd.value().data()), nullptr);
    if (st != MC_OK) return mc_error("fused-rms-norm", st);
    return std::make_pair(std::move(y.value()), std::move(rstd.value()));
}

Result<std::pair<Tensor, Tensor>, CandleError> FusedRMSNormOp::backward(const Tensor& input, const Tensor* weight,
                                                                        const Tensor& rstd,
                                                                        const Tensor& grad_output) const {
    if (!input.device().is_hip()) return cpu_fwd(input).error();
    if (input.rank() == 0)
        return bail("Input tensor for FusedRMSNormOp must have at least 1 dimension, got " +
                    dims_to_string(input.dims()));
    const int64_t dim = input.dims().back();
    const int64_t rows = dim ? input.elem_count() / dim : 0;
    if (grad_output.dims() != input.dims() || grad_output.dtype() != input.dtype())
        return bail("fused-rms-norm backward: grad_output must match the input, got " +
                    dims_to_string(grad_output.dims()));
    if (rstd.defined() && rstd.rank() && (rstd.dims() != std::vector<int64_t>{rows} || rstd.dtype() != DType::F32))
        return bail("fused-rms-norm backward: rstd must be F32 [" + std::to_string(rows) + "]");
    if (weight && (weight->dims() != std::vector<int64_t>{dim} || weight->dtype() != input.dtype()))
        return bail("fused-rms-norm backward: weight must be [" + std::to_string(dim) + "]");
    auto dx = Tensor::empty(input.dims(), input.dtype(), input.device());
    auto dw = Tensor::empty({dim}, DType::F32, input.device());
    if (dx.is_err()) return dx.error();
    if (dw.is_err()) return dw.error();
    Workspace ws;
    const size_t ws_bytes = mc_rmsnorm_bwd_workspace_size(rows, dim);
    auto a = alloc_ws(ws, ws_bytes);
    if (a.is_err()) return a.error();
    const mc_status st = mc_rmsnorm_bwd(rows, dim, eps_, mc_dtype_of(input.dtype()), input.data(),
                                        weight ? weight->data() : nullptr,
                                        rstd.rank() ? static_cast<const float*>(rstd.data()) : nullptr,
                                        grad_output.data(), dx.value().data(), static_cast<float*>(dw.value().data()),
                                        ws.p, ws_bytes, nullptr);
    if (st != MC_OK) return mc_error("fused-rms-norm backward", st);
    return std::make_pair(std::move(dx.value()), std::move(dw.value()));
}

// ------------------------------------------------------------------ FusedSoftmaxOp
Result<FusedSoftmaxOp, CandleError> FusedSoftmaxOp::create() { return FusedSoftmaxOp{}; }

Result<Tensor, CandleError> FusedSoftmaxOp::apply(const Tensor& input) const {
    return input.device().is_hip() ? hip_fwd(input) : cpu_fwd(input);
}

Result<Tensor, CandleError> FusedSoftmaxOp::cpu_fwd(const Tensor&) const {
    // custom_ops.rs:719-725
    return bail("Fused Softmax kernel not implemented for CPU. Use a HIP device.");
}

Result<Tensor, CandleError> FusedSoftmaxOp::hip_fwd(const Tensor& input) const { return forward_causal(input, false); }

namespace {
Result<int64_t, CandleError> causal_rows_of(const Tensor& t, bool causal) {
    if (!causal) return (int64_t)0;
    if (t.rank() < 2) return bail("fused-softmax: a causal mask needs at least 2 dimensions, got " +
                                  dims_to_string(t.dims()));
    const int64_t S = t.dims()[t.rank() - 2], D = t.dims().back();
    if (S > D) return bail("fused-softmax: causal mask needs dims[-2] <= dims[-1], got " + dims_to_string(t.dims()));
    return S;
}
}  // namespace

Result<Tensor, CandleError> FusedSoftmaxOp::forward_causal(const Tensor& input, bool causal) const {
    if (!input.device().is_hip()) return cpu_fwd(input).error();
    if (input.rank() == 0)
        return bail("Input tensor for FusedSoftmaxOp must have at least 1 dimension, got " +
                    dims_to_string(input.dims()));
    if (input.dtype() == DType::U8) return bail("fused-softmax: input must be F32 or BF16");
    auto S = causal_rows_of(input, causal);
    if (S.is_err()) return S.error();
    const int64_t dim = input.dims().back();
    const int64_t rows = dim ? input.elem_count() / dim : 0;
    auto p = Tensor::empty(input.dims(), input.dtype(), input.device());
    if (p.is_err()) return p.error();
    const mc_status st = mc_softmax_fwd(rows, dim, S.value(), mc_dtype_of(input.dtype()), input.data(),
                                        p.value().data(), nullptr);
    if (st != MC_OK) return mc_error("fused-softmax", st);
    return p;
}

Result<Tensor, CandleError> FusedSoftmaxOp::backward(const Tensor& probs, const Tensor& grad_output,
                                                     bool causal) const {
    if (!probs.device().is_hip()) return cpu_fwd(probs).error();
    if (probs.rank() == 0)
        return bail("Input tensor for FusedSoftmaxOp must have at least 1 dimension, got " +
                    dims_to_string(probs.dims()));
    if (grad_output.dims() != probs.dims() || grad_output.dtype() != probs.dtype())
        return bail("fused-softmax backward: grad_output must match the probabilities, got " +
                    dims_to_string(grad_output.dims()));
    auto S = causal_rows_of(probs, causal);
    if (S.is_err()) return S.error();
    const int64_t dim = probs.dims().back();
    const int64_t rows = dim ? probs.elem_count() / dim : 0;
    auto ds = Tensor::empty(probs.dims(), probs.dtype(), probs.device());
    if (ds.is_err()) return ds.error();
    const mc_status st = mc_softmax_bwd(rows, dim, S.value(), mc_dtype_of(probs.dtype()), probs.data(),
                                        grad_output.data(), ds.value().data(), nullptr);
    if (st != MC_OK) return mc_error("fused-softmax backward", st);
    return ds;
}

// ------------------------------------------------------------------ CustomMetalOps mirror
Result<Tensor, TrainingError> lora_forward_fused(const Tensor& input, const Tensor& lora_a, const Tensor& lora_b,
                                                 float scaling) {
    // metal_ops.rs:127-144
    auto op = FusedLoRAOp::create(lora_a, lora_b, scaling);
    if (op.is_err()) return TrainingError::failed("Failed to create FusedLoRAOp: " + op.error().to_string());
    auto y = op.value().apply(input);
    if (y.is_err()) return TrainingError::failed("Failed to apply fused LoRA op: " + y.error().to_string());
    return std::move(y.value());
}

Result<Tensor, TrainingError> softmax_fused(const Tensor& input) {
    // metal_ops.rs:146-157
    auto op = FusedSoftmaxOp::create();
    if (op.is_err()) return TrainingError::failed("Failed to create FusedSoftmaxOp: " + op.error().to_string());
    auto y = op.value().apply(input);
    if (y.is_err()) return TrainingError::failed("Fused Softmax kernel execution failed: " + y.error().to_string());
    return std::move(y.value());
}

Result<Tensor, TrainingError> rms_norm_fused(const Tensor& input, float eps) {
    // metal_ops.rs:159-170
    auto op = FusedRMSNormOp::create(eps);
    if (op.is_err()) return TrainingError::failed("Failed to create FusedRMSNormOp: " + op.error().to_string());
    auto y = op.value().apply(input);
    if (y.is_err()) return TrainingError::failed("Fused RMS Norm kernel execution failed: " + y.error().to_string());
    return std::move(y.value());
}

// ------------------------------------------------------------------ LoRAConfig / LoRALayer
Result<void, Error> LoRAConfig::validate() const {
    // lora.rs:97-120
    if (rank == 0) return Error::from(TrainingError::invalid_config("LoRA rank must be greater than 0"));
    if (!(alpha > 0.f)) return Error::from(TrainingError::invalid_config("LoRA alpha must be positive"));
    if (!(dropout >= 0.f && dropout < 1.f))
        return Error::from(TrainingError::invalid_config("LoRA dropout must be in [0, 1)"));
    return {};
}

// ------------------------------------------------------------------ LayerNorm
Result<Tensor, CandleError> LayerNormOp::apply(const Tensor& input) const {
    return input.device().is_hip() ? hip_fwd(input) : cpu_fwd(input);
}

Result<Tensor, CandleError> LayerNormOp::cpu_fwd(const Tensor&) const {
    return bail("LayerNorm: the CPU path stays with candle; this op runs on HIP tensors");
}

Result<Tensor, CandleError> LayerNormOp::hip_fwd(const Tensor& input) const {
    // custom_ops.rs (metal_fwd): "LayerNorm expects 2D tensors, got shape {:?}"
    if (input.rank() != 2) return bail("LayerNorm expects 2D tensors, got shape " + dims_to_string(input.dims()));
    auto r = forward_affine(input, nullptr, nullptr);
    if (r.is_err()) return r.error();
    return std::move(r.value().first);
}

Result<std::pair<Tensor, LayerNormOp::Saved>, CandleError> LayerNormOp::forward_affine(const Tensor& input,
                                                                                     const Tensor* weight,
                                                                                     const Tensor* bias) const {
    if (!input.device().is_hip()) return cpu_fwd(input).error();
    if (input.rank() == 0) return bail("LayerNorm: input must have at least 1 dimension");
    if (input.dtype() != DType::F32 && input.dtype() != DType::BF16) return bail("layer-norm: input must be F32 or BF16");
    const int64_t dim = input.dims().back();
    const int64_t rows = dim ? input.elem_count() / dim : 0;
    for (const Tensor* p : {weight, bias})
        if (p && (p->dims() != std::vector<int64_t>{dim} || p->dtype() != input.dtype() || !same_device(*p, input)))
            return bail("layer-norm: weight and bias must be [" + std::to_string(dim) + "] in the input's dtype");
    auto y = Tensor::empty(input.dims(), input.dtype(), input.device());
    auto m = Tensor::empty({rows}, DType::F32, input.device());
    auto r = Tensor::empty({rows}, DType::F32, input.device());
    if (y.is_err()) return y.error();
    if (m.is_err()) return m.error();
    if (r.is_err()) return r.error();
    const mc_status st = mc_layernorm_fwd(rows, dim, (float)eps_, mc_dtype_of(input.dtype()), input.data(),
                                          weight ? weight->data() : nullptr, bias ? bias->data() : nullptr,
                                          y.value().data(), static_cast<float*>(m.value().data()),
                                          static_cast<float*>(r.value().data()), nullptr);
    if (st != MC_OK) return mc_error("layer-norm", st);
    return std::make_pair(std::move(y.value()), Saved{std::move(m.value()), std::move(r.value())});
}

Result<LayerNormOp::Grads, CandleError> LayerNormOp::backward(const Tensor& input, const Tensor* weight,
                                                              const Saved& saved, const Tensor& grad_output) const {
    if (!input.device().is_hip()) return cpu_fwd(input).error();
    const int64_t dim = input.dims().empty() ? 0 : input.dims().back();
    const int64_t rows = dim ? input.elem_count() / dim : 0;
    if (grad_output.dims() != input.dims() || grad_output.dtype() != input.dtype())
        return bail("layer-norm backward: grad_output must match the input");
    Grads g;
    auto dx = Tensor::empty(input.dims(), input.dtype(), input.device());
    auto dw = Tensor::empty({dim}, DType::F32, input.device());
    auto db = Tensor::empty({dim}, DType::F32, input.device());
    if (dx.is_err()) return dx.error();
    if (dw.is_err()) return dw.error();
    if (db.is_err()) return db.error();
    Workspace ws;
    const size_t need = mc_layernorm_bwd_workspace_size(rows, dim);
    if (auto e = alloc_ws(ws, need); e.is_err()) return e.error();
    const mc_status st = mc_layernorm_bwd(rows, dim, (float)eps_, mc_dtype_of(input.dtype()), input.data(),
                                          weight ? weight->data() : nullptr,
                                          static_cast<const float*>(saved.mean.data()),
                                          static_cast<const float*>(saved.rstd.data()), grad_output.data(),
                                          dx.value().data(), static_cast<float*>(dw.value().data()),
                                          static_cast<float*>(db.value().data()), ws.p, need, nullptr);
    if (st != MC_OK) return mc_error("layer-norm backward", st);
    g.dx = std::move(dx.value());
    g.dw = std::move(dw.value());
    g.db = std::move(db.value());
    return g;
}

Result<Tensor, CandleError> layer_norm(const Tensor& input, double eps) {
    auto r = LayerNormOp::create(eps).forward_affine(input, nullptr, nullptr);
    if (r.is_err()) return r.error();
    return std::move(r.value().first);
}

// ---------------------------------------------------------------- cross entropy
namespace {

struct XentPrep {
    mc_xent_desc desc{};
    Tensor stats;
};

// loss.rs:66-95: the shape checks, with the reference's messages.
Result<XentPrep, Error> xent_prepare(const Tensor& logits, const Tensor& targets,
                                     std::optional<uint32_t> ignore_index, float smoothing) {
    const auto& ls = logits.dims();
    const auto& ts = targets.dims();
    if (ls.size() != 3)
        return Error::from(TrainingError::invalid_config("logits must be 3D (batch, seq_len, vocab_size), got shape " +
                                                         dims_to_string(ls)));
    if (ts.size() != 2)
        return Error::from(TrainingError::invalid_config("targets must be 2D (batch, seq_len), got shape " +
                                                         dims_to_string(ts)));
    if (ls[0] != ts[0] || ls[1] != ts[1])
        return Error::from(TrainingError::invalid_config("logits and targets batch/seq_len mismatch: logits " +
                                                         dims_to_string({ls[0], ls[1]}) + " vs targets " +
                                                         dims_to_string(ts)));
    if (!logits.device().is_hip() || !targets.device().is_hip())
        return Error::from(bail("cross_entropy_loss runs on HIP tensors"));
    if (logits.dtype() != DType::F32 && logits.dtype() != DType::BF16)
        return Error::from(bail("cross_entropy_loss: logits must be F32 or BF16"));
    if (targets.dtype() != DType::U32) return Error::from(bail("cross_entropy_loss: targets must be U32"));
    XentPrep p;
    p.desc = {ls[0] * ls[1], ls[2], ignore_index ? (int64_t)*ignore_index : -1, smoothing,
              mc_dtype_of(logits.dtype())};
    // gather_last_dim (loss.rs:160-185) fails on a target past the vocabulary
    auto tv = targets.to_vec_f32();
    if (tv.is_err()) return Error::from(tv.error());
    for (float t : tv.value())
        if ((int64_t)t >= ls[2])
            return Error::from(bail("index out of range: target " + std::to_string((int64_t)t) + " for vocab size " +
                                    std::to_string(ls[2])));
    return p;
}

Result<Tensor, Error> xent_forward(const Tensor& logits, const Tensor& targets, std::optional<uint32_t> ignore_index,
                                   float smoothing) {
    auto p = xent_prepare(logits, targets, ignore_index, smoothing);
    if (p.is_err()) return p.error();
    const mc_xent_desc& d = p.value().desc;
    auto loss = Tensor::empty({}, DType::F32, logits.device());
    auto stats = Tensor::empty({d.rows + 1}, DType::F32, logits.device());
    if (loss.is_err()) return Error::from(loss.error());
    if (stats.is_err()) return Error::from(stats.error());
    Workspace ws;
    const size_t need = mc_cross_entropy_workspace_size(&d);
    if (auto e = alloc_ws(ws, need); e.is_err()) return Error::from(e.error());
    const mc_status st = mc_cross_entropy_fwd(&d, logits.data(), static_cast<const uint32_t*>(targets.data()),
                                              static_cast<float*>(loss.value().data()),
                                              static_cast<float*>(stats.value().data()), ws.p, need, nullptr);
    if (st != MC_OK) return Error::from(mc_error("cross_entropy_loss", st));
    if (ignore_index) {  // loss.rs:123-131: the count, read back
        float cnt = 0.f;
        hipError_t e = hipMemcpy(&cnt, static_cast<float*>(stats.value().data()) + d.rows, 4, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return Error::from(hip_error("hipMemcpy D2H", e));
        if (cnt == 0.f)
            return Error::from(TrainingError::invalid_config("all tokens are ignored, cannot compute loss"));
    }
    return std::move(loss.value());
}

}  // namespace

Result<Tensor, Error> cross_entropy_loss(const Tensor& logits, const Tensor& targets,
                                         std::optional<uint32_t> ignore_index) {
    return xent_forward(logits, targets, ignore_index, 0.f);
}

Result<Tensor, Error> cross_entropy_loss_with_smoothing(const Tensor& logits, const Tensor& targets, float smoothing,
                                                        std::optional<uint32_t> ignore_index) {
    if (!(smoothing >= 0.f && smoothing < 1.f)) {  // loss.rs:214-219
        std::ostringstream m;
        m << "smoothing must be in [0, 1), got " << smoothing;
        return Error::from(TrainingError::invalid_config(m.str()));
    }
    return xent_forward(logits, targets, ignore_index, smoothing);
}

Result<Tensor, Error> cross_entropy_loss_backward(const Tensor& logits, const Tensor& targets, float smoothing,
                                                  std::optional<uint32_t> ignore_index, float dloss) {
    if (!(smoothing >= 0.f && smoothing < 1.f)) {
        std::ostringstream m;
        m << "smoothing must be in [0, 1), got " << smoothing;
        return Error::from(TrainingError::invalid_config(m.str()));
    }
    auto p = xent_prepare(logits, targets, ignore_index, smoothing);
    if (p.is_err()) return p.error();
    const mc_xent_desc& d = p.value().desc;
    auto loss = Tensor::empty({}, DType::F32, logits.device());
    auto stats = Tensor::empty({d.rows + 1}, DType::F32, logits.device());
    auto g = Tensor::from_slice({dloss}, {1}, logits.device());
    auto dl = Tensor::empty(logits.dims(), logits.dtype(), logits.device());
    if (loss.is_err()) return Error::from(loss.error());
    if (stats.is_err()) return Error::from(stats.error());
    if (g.is_err()) return Error::from(g.error());
    if (dl.is_err()) return Error::from(dl.error());
    Workspace ws;
    const size_t need = mc_cross_entropy_workspace_size(&d);
    if (auto e = alloc_ws(ws, need); e.is_err()) return Error::from(e.error());
    mc_status st = mc_cross_entropy_fwd(&d, logits.data(), static_cast<const uint32_t*>(targets.data()),
                                        static_cast<float*>(loss.value().data()),
                                        static_cast<float*>(stats.value().data()), ws.p, need, nullptr);
    if (st == MC_OK)
        st = mc_cross_entropy_bwd(&d, logits.data(), static_cast<const uint32_t*>(targets.data()),
                                  static_cast<const float*>(stats.value().data()),
                                  static_cast<const float*>(g.value().data()), dl.value().data(), nullptr);
    if (st != MC_OK) return Error::from(mc_error("cross_entropy_loss backward", st));
    return std::move(dl.value());
}

// ------------------------------------------------------------------ AdamW
Result<void, Error> AdamWConfig::validate() const {
    // optimizer.rs:67-103, with its comparisons (a NaN learning rate passes, as there)
    if (learning_rate <= 0.f) return Error::from(TrainingError::invalid_config("learning rate must be positive"));
    if (!(beta1 >= 0.f && beta1 < 1.f)) {
        std::ostringstream m;
        m << "beta1 must be in [0, 1), got " << beta1;
        return Error::from(TrainingError::invalid_config(m.str()));
    }
    if (!(beta2 >= 0.f && beta2 < 1.f)) {
        std::ostringstream m;
        m << "beta2 must be in [0, 1), got " << beta2;
        return Error::from(TrainingError::invalid_config(m.str()));
    }
    if (epsilon <= 0.f) return Error::from(TrainingError::invalid_config("epsilon must be positive"));
    if (weight_decay < 0.f) return Error::from(TrainingError::invalid_config("weight decay must be non-negative"));
    return {};
}

Result<AdamW, Error> AdamW::create(const AdamWConfig& config) {
    auto v = config.validate();
    if (v.is_err()) return v.error();
    AdamW a;
    a.config_ = config;
    return a;
}

AdamW::State* AdamW::find(const std::string& name) {
    for (auto& kv : state_)
        if (kv.first == name) return &kv.second;
    return nullptr;
}

Result<void, Error> AdamW::add_parameter(const std::string& name, const Tensor& param) {
    auto m = Tensor::zeros(param.dims(), DType::F32, param.device());
    if (m.is_err()) return Error::from(m.error());
    auto v = Tensor::zeros(param.dims(), DType::F32, param.device());
    if (v.is_err()) return Error::from(v.error());
    State st{std::move(m.value()), std::move(v.value())};
    if (State* old = find(name)) *old = std::move(st);  // HashMap::insert replaces
    else state_.emplace_back(name, std::move(st));
    return {};
}

Result<Tensor, Error> AdamW::step(const std::string& name, const Tensor& param, const Tensor& grad) {
    State* st = find(name);
    if (!st) return Error::from(TrainingError::state_error("parameter '" + name + "' not found in optimizer"));
    ++step_count_;  // optimizer.rs:235-237: counted per call, before the update
    if (!param.device().is_hip() || !grad.device().is_hip())
        return Error::from(bail("AdamW step is implemented for HIP tensors only"));
    if (param.dtype() != DType::F32 || grad.dtype() != DType::F32)
        return Error::from(bail("AdamW step: parameters and gradients must be f32"));
    if (param.elem_count() != grad.elem_count() || param.elem_count() != st->m.elem_count())
        return Error::from(bail("shape mismatch in AdamW step: param " + dims_to_string(param.dims()) + ", grad " +
                                dims_to_string(grad.dims()) + ", state " + dims_to_string(st->m.dims())));
    auto out = Tensor::empty(param.dims(), DType::F32, param.device());
    if (out.is_err()) return Error::from(out.error());
    const mc_adamw_config cfg{config_.learning_rate, config_.beta1, config_.beta2, config_.epsilon,
                              config_.weight_decay};
    const mc_adamw_tensor t{static_cast<const float*>(param.data()), static_cast<const float*>(grad.data()),
                            static_cast<float*>(st->m.data()), static_cast<float*>(st->v.data()),
                            static_cast<float*>(out.value().data()), param.elem_count(), (int64_t)step_count_};
    const mc_status rc = mc_adamw_step(&cfg, &t, 1, nullptr);
    if (rc != MC_OK) return Error::from(mc_error("mc_adamw_step", rc));
    return std::move(out.value());
}

void AdamW::reset_state() {
    step_count_ = 0;
    for (auto& kv : state_) {
        auto m = Tensor::zeros(kv.second.m.dims(), DType::F32, kv.second.m.device());
        auto v = Tensor::zeros(kv.second.v.dims(), DType::F32, kv.second.v.device());
        if (m.is_ok()) kv.second.m = std::move(m.value());
        if (v.is_ok()) kv.second.v = std::move(v.value());
    }
}

Result<LoRALayer, Error> LoRALayer::create(size_t in_features, size_t out_features, const LoRAConfig& config,
                                           const Device& device, uint64_t seed) {
    auto v = config.validate();
    if (v.is_err()) return v.error();
    const size_t max_rank = in_features < out_features ? in_features : out_features;
    if (config.rank > max_rank) {
        std::ostringstream s;  // lora.rs:219-228
        s << "LoRA rank " << config.rank << " exceeds maximum rank " << max_rank << " (min of in_features="
          << in_features << ", out_features=" << out_features << ")";
        return Error::from(TrainingError::invalid_config(s.str()));
    }
    // A ~ N(0, 1/sqrt(rank)), B = 0 (lora.rs:233-247). Host initialisation.
    std::mt19937_64 gen(seed);
    std::normal_distribution<float> nd(0.f, 1.f / sqrtf((float)config.rank));
    std::vector<float> a(in_features * config.rank);
    for (float& x : a) x = nd(gen);
    auto ta = Tensor::from_slice(a, {(int64_t)in_features, (int64_t)config.rank}, device);
    if (ta.is_err()) return Error::from(ta.error());
    auto tb = Tensor::zeros({(int64_t)config.rank, (int64_t)out_features}, DType::F32, device);
    if (tb.is_err()) return Error::from(tb.error());
    LoRALayer l;
    l.lora_a_ = std::move(ta.value());
    l.lora_b_ = std::move(tb.value());
    l.config_ = config;
    l.in_features_ = in_features;
    l.out_features_ = out_features;
    l.seed_ = seed;
    return l;
}

Result<void, Error> LoRALayer::set_lora_a(Tensor a) {
    if (a.dims() != lora_a_.dims() || a.dtype() != DType::F32)
        return Error::from(bail("set_lora_a: expected F32 " + dims_to_string(lora_a_.dims()) + ", got " +
                                dims_to_string(a.dims())));
    lora_a_ = std::move(a);
    have_saved_ = false;
    return {};
}

Result<void, Error> LoRALayer::set_lora_b(Tensor b) {
    if (b.dims() != lora_b_.dims() || b.dtype() != DType::F32)
        return Error::from(bail("set_lora_b: expected F32 " + dims_to_string(lora_b_.dims()) + ", got " +
                                dims_to_string(b.dims())));
    lora_b_ = std::move(b);
    have_saved_ = false;
    return {};
}

Result<Tensor, Error> LoRALayer::forward(const Tensor& input) {
    auto op = FusedLoRAOp::create(lora_a_, lora_b_, config_.scaling());
    if (op.is_err()) return Error::from(op.error());
    const bool drop = training_ && config_.dropout > 0.f;
    mask_ = Tensor();
    if (drop) {
        if (input.rank() == 0) return Error::from(bail("Input must have at least 1 dimension"));
        const int64_t T = input.dims().back() ? input.elem_count() / input.dims().back() : 0;
        std::vector<uint8_t> m((size_t)T * config_.rank);
        const mc_status st = mc_dropout_mask(seed_ + step_, config_.dropout, T, (int32_t)config_.rank, m.data());
        if (st != MC_OK) return Error::from(mc_error("dropout mask", st));
        ++step_;
        auto tm = Tensor::from_bytes(m, {T, (int64_t)config_.rank}, input.device());
        if (tm.is_err()) return Error::from(tm.error());
        mask_ = std::move(tm.value());
    }
    auto r = op.value().forward_with_base(input, nullptr, nullptr, drop ? &mask_ : nullptr,
                                          drop ? config_.dropout : 0.f);
    if (r.is_err()) return Error::from(r.error());
    saved_ = std::move(r.value().second);
    have_saved_ = true;
    return std::move(r.value().first);
}

Result<LoRAGrads, Error> LoRALayer::backward(const Tensor& input, const Tensor& grad_output) {
    if (!have_saved_) return Error::from(TrainingError::failed("LoRALayer::backward needs a forward first"));
    auto op = FusedLoRAOp::create(lora_a_, lora_b_, config_.scaling());
    if (op.is_err()) return Error::from(op.error());
    const bool drop = mask_.rank() != 0;
    auto g = op.value().backward(input, nullptr, saved_, grad_output, drop ? &mask_ : nullptr,
                                 drop ? config_.dropout : 0.f);
    if (g.is_err()) return Error::from(g.error());
    return std::move(g.value());
}

// ------------------------------------------------------------------ Operation
const char* Operation::name() const {
    switch (kind) {  // operation.rs:49-63
        case Kind::Input: return "input";
        case Kind::Matmul: return "matmul";
        case Kind::Add: return "add";
        case Kind::Mul: return "mul";
        case Kind::MulScalar: return "mul_scalar";
        case Kind::LoRA: return "lora";
        case Kind::Softmax: return "softmax";
        case Kind::RMSNorm: return "rms_norm";
    }
    return "unknown";
}

Result<std::vector<int64_t>, std::string> Operation::output_shape(
    const std::vector<std::vector<int64_t>>& in) const {
    // operation.rs:66-160
    switch (kind) {
        case Kind::Input:
            if (in.empty()) return std::string("Input operation requires shape");
            return in[0];
        case Kind::Matmul: {
            if (in.size() != 2) return "Matmul requires 2 inputs, got " + std::to_string(in.size());
            const auto &a = in[0], &b = in[1];
            if (a.size() < 2 || b.size() < 2) return std::string("Matmul requires at least 2D tensors");
            const int64_t ar = a[a.size() - 2], ac = a.back(), br = b[b.size() - 2], bc = b.back();
            if (ac != br) {
                std::ostringstream s;
                s << "Matmul dimension mismatch: " << ar << "×" << ac << " @ " << br << "×" << bc;
                return s.str();
            }
            std::vector<int64_t> out(a.begin(), a.end() - 2);
            out.push_back(ar);
            out.push_back(bc);
            return out;
        }
        case Kind::Add:
        case Kind::Mul:
            if (in.size() != 2) return std::string(name()) + " requires 2 inputs, got " + std::to_string(in.size());
            if (in[0] != in[1])
                return "Shape mismatch: " + dims_to_string(in[0]) + " vs " + dims_to_string(in[1]);
            return in[0];
        case Kind::MulScalar:
            if (in.size() != 1) return "MulScalar requires 1 input, got " + std::to_string(in.size());
            return in[0];
        case Kind::LoRA: {
            if (in.size() != 3) return "LoRA requires 3 inputs (input, a, b), got " + std::to_string(in.size());
            std::vector<int64_t> out = in[0];
            if (!out.empty() && !in[2].empty()) out.back() = in[2].back();
            return out;
        }
        case Kind::Softmax:
        case Kind::RMSNorm:
            if (in.size() != 1) return std::string(name()) + " requires 1 input, got " + std::to_string(in.size());
            return in[0];
    }
    return std::string("unknown operation");
}

// ------------------------------------------------------------------ AsyncExecutor
Result<AsyncExecutor, TrainingError> AsyncExecutor::create(const Device& device) {
    AsyncExecutor e;
    e.device_ = device;
    return e;
}

Result<Tensor, TrainingError> AsyncExecutor::execute_operation(const Operation& op,
                                                               const std::vector<Tensor>& inputs) {
    using K = Operation::Kind;
    const std::string n = std::to_string(inputs.size());
    auto candle_only = [&](const char* what) {
        return TrainingError::failed(std::string(what) +
                                     " is a generic candle op; libmc_hip.so only provides the fused ops");
    };
    switch (op.kind) {  // executor.rs:48-66
        case K::Input: return TrainingError::failed("Cannot execute Input operation");
        case K::Matmul:
            if (inputs.size() != 2) return TrainingError::failed("Matmul requires 2 inputs, got " + n);
            return candle_only("Matmul");
        case K::Add:
            if (inputs.size() != 2) return TrainingError::failed("Add requires 2 inputs, got " + n);
            return candle_only("Add");
        case K::Mul:
            if (inputs.size() != 2) return TrainingError::failed("Mul requires 2 inputs, got " + n);
            return candle_only("Mul");
        case K::MulScalar:
            if (inputs.size() != 1) return TrainingError::failed("MulScalar requires 1 input, got " + n);
            return candle_only("MulScalar");
        case K::LoRA:
            // executor.rs:123-159 (fused path; the candle composite fallback belongs to the caller)
            if (inputs.size() != 3) return TrainingError::failed("LoRA requires 3 inputs (input, a, b), got " + n);
            return lora_forward_fused(inputs[0], inputs[1], inputs[2], op.scale);
        case K::Softmax:
            // executor.rs:162-185: the fused kernel is for the last dim only
            if (inputs.size() != 1) return TrainingError::failed("Softmax requires 1 input, got " + n);
            if (inputs[0].rank() == 0 || op.dim != inputs[0].rank() - 1)
                return TrainingError::failed("Softmax failed: only the last dimension has a fused kernel, got dim " +
                                             std::to_string(op.dim) + " of shape " +
                                             dims_to_string(inputs[0].dims()));
            return softmax_fused(inputs[0]);
        case K::RMSNorm:
            // executor.rs:188-215
            if (inputs.size() != 1) return TrainingError::failed("RMSNorm requires 1 input, got " + n);
            return rms_norm_fused(inputs[0], op.eps);
    }
    return TrainingError::failed("unknown operation");
}

Result<void, TrainingError> AsyncExecutor::synchronize() {
    if (device_.is_cpu()) return {};
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return TrainingError::failed(std::string("synchronize: ") + hipGetErrorString(e));
    return {};
}

// ------------------------------------------------------------------ lazy graph
std::string node_id_string(NodeId id) { return "NodeId(" + std::to_string(id.id) + ")"; }

DType Operation::output_dtype(const std::vector<DType>& in) const {
    return in.empty() ? DType::F32 : in[0];  // operation.rs:170-180
}

Result<const GraphNode*, std::string> ComputationGraph::get_node(NodeId id) const {
    if (id.id >= nodes_.size()) return "Node " + node_id_string(id) + " not found";  // node.rs:150-156
    return &nodes_[id.id];
}

Result<GraphNode*, std::string> ComputationGraph::get_node_mut(NodeId id) {
    if (id.id >= nodes_.size()) return "Node " + node_id_string(id) + " not found";
    return &nodes_[id.id];
}

NodeId ComputationGraph::add_input(const Tensor& tensor) {
    GraphNode n;  // node.rs:97-110
    n.id = NodeId{nodes_.size()};
    n.operation = Operation::input();
    n.output_shape = tensor.dims();
    n.output_dtype = tensor.dtype();
    n.data = GraphNode::Data::Concrete;
    n.tensor = tensor;
    nodes_.push_back(std::move(n));
    return nodes_.back().id;
}

Result<NodeId, std::string> ComputationGraph::add_node(const Operation& op, const std::vector<NodeId>& inputs) {
    std::vector<std::vector<int64_t>> shapes;  // node.rs:175-215
    std::vector<DType> dtypes;
    for (NodeId i : inputs) {
        if (i.id >= nodes_.size()) return "Input node " + node_id_string(i) + " not found";
        shapes.push_back(nodes_[i.id].output_shape);
        dtypes.push_back(nodes_[i.id].output_dtype);
    }
    auto shape = op.output_shape(shapes);
    if (shape.is_err()) return shape.error();
    GraphNode n;
    n.id = NodeId{nodes_.size()};
    n.operation = op;
    n.inputs = inputs;
    n.output_shape = std::move(shape.value());
    n.output_dtype = op.output_dtype(dtypes);
    nodes_.push_back(std::move(n));
    return nodes_.back().id;
}

Result<std::vector<NodeId>, std::string> ComputationGraph::topological_order(NodeId output) const {
    // node.rs:222-265: depth-first, each node after its inputs; a node met
    // again while its own inputs are being visited is a cycle
    std::vector<NodeId> order;
    std::unordered_set<size_t> done, active;
    std::function<Result<void, std::string>(NodeId)> visit = [&](NodeId id) -> Result<void, std::string> {
        if (done.count(id.id)) return {};
        if (active.count(id.id)) return "Circular dependency detected at node " + node_id_string(id);
        auto node = get_node(id);
        if (node.is_err()) return node.error();
        active.insert(id.id);
        for (NodeId in : node.value()->inputs) {
            auto r = visit(in);
            if (r.is_err()) return r;
        }
        active.erase(id.id);
        done.insert(id.id);
        order.push_back(id);
        return {};
    };
    auto r = visit(output);
    if (r.is_err()) return r.error();
    return order;
}

NodeId ComputationGraph::merge_from(const ComputationGraph& other, NodeId target) {
    // node.rs:275-300: dependencies first, each node copied once (with its
    // value, if it has one) and its inputs renumbered. `target` must be a
    // node of `other` (the reference panics otherwise; here std::out_of_range).
    std::unordered_map<size_t, NodeId> copied;
    std::function<NodeId(NodeId)> copy = [&](NodeId id) -> NodeId {
        auto it = copied.find(id.id);
        if (it != copied.end()) return it->second;
        GraphNode n = other.nodes_.at(id.id);
        for (NodeId& in : n.inputs) in = copy(in);
        n.id = NodeId{nodes_.size()};
        nodes_.push_back(std::move(n));
        copied[id.id] = nodes_.back().id;
        return nodes_.back().id;
    };
    return copy(target);
}

struct LazyTensor::Shared {
    explicit Shared(const Device& d) : graph(d) {}
    std::mutex mu;
    ComputationGraph graph;
};

Result<LazyTensor, CandleError> LazyTensor::from_tensor(const Tensor& tensor) {
    LazyTensor t;  // lazy_tensor.rs:95-108: a new graph with one input node
    t.graph_ = std::make_shared<Shared>(tensor.device());
    t.node_ = t.graph_->graph.add_input(tensor);
    t.shape_ = tensor.dims();
    t.dtype_ = tensor.dtype();
    t.device_ = tensor.device();
    return t;
}

Result<LazyTensor, CandleError> LazyTensor::from_slice(const std::vector<float>& data, std::vector<int64_t> dims,
                                                       const Device& device) {
    auto t = Tensor::from_slice(data, std::move(dims), device);
    if (t.is_err()) return t.error();
    return from_tensor(t.value());
}

Result<LazyTensor, CandleError> LazyTensor::zeros(std::vector<int64_t> dims, DType dtype, const Device& device) {
    auto t = Tensor::zeros(std::move(dims), dtype, device);
    if (t.is_err()) return t.error();
    return from_tensor(t.value());
}

Result<LazyTensor, CandleError> LazyTensor::ones(std::vector<int64_t> dims, DType dtype, const Device& device) {
    int64_t n = 1;
    for (int64_t d : dims) {
        if (d < 0) return CandleError{"ones: negative dimension in " + dims_to_string(dims)};
        n *= d;
    }
    auto t = Tensor::from_slice(std::vector<float>((size_t)n, 1.f), std::move(dims), device, dtype);
    if (t.is_err()) return t.error();
    return from_tensor(t.value());
}

Result<LazyTensor, CandleError> LazyTensor::add_tensor_to_graph(const Tensor& tensor) const {
    LazyTensor t = *this;  // lazy_tensor.rs:120-131
    {
        std::lock_guard<std::mutex> lk(graph_->mu);
        t.node_ = graph_->graph.add_input(tensor);
    }
    t.shape_ = tensor.dims();
    t.dtype_ = tensor.dtype();
    t.device_ = tensor.device();
    return t;
}

size_t LazyTensor::graph_size() const {
    std::lock_guard<std::mutex> lk(graph_->mu);
    return graph_->graph.len();
}

bool LazyTensor::is_evaluated() const {
    std::lock_guard<std::mutex> lk(graph_->mu);
    auto n = graph_->graph.get_node(node_);
    return n.is_ok() && n.value()->is_available();
}

Result<LazyTensor, CandleError> LazyTensor::add_operation(const Operation& op,
                                                          const std::vector<NodeId>& inputs) const {
    LazyTensor t = *this;  // lazy_tensor.rs:214-236
    std::lock_guard<std::mutex> lk(graph_->mu);
    auto id = graph_->graph.add_node(op, inputs);
    if (id.is_err()) return CandleError{id.error()};
    const GraphNode* n = graph_->graph.get_node(id.value()).value();
    t.node_ = id.value();
    t.shape_ = n->output_shape;
    t.dtype_ = n->output_dtype;
    return t;
}

NodeId LazyTensor::merge_graph_from(const LazyTensor& other) const {
    if (graph_ == other.graph_) return other.node_;  // lazy_tensor.rs:238-250
    std::scoped_lock lk(graph_->mu, other.graph_->mu);
    return graph_->graph.merge_from(other.graph_->graph, other.node_);
}

Result<LazyTensor, CandleError> LazyTensor::matmul(const LazyTensor& other) const {
    return add_operation(Operation::matmul(), {node_, merge_graph_from(other)});
}
Result<LazyTensor, CandleError> LazyTensor::add(const LazyTensor& other) const {
    return add_operation(Operation::add(), {node_, merge_graph_from(other)});
}
Result<LazyTensor, CandleError> LazyTensor::mul(const LazyTensor& other) const {
    return add_operation(Operation::mul(), {node_, merge_graph_from(other)});
}
Result<LazyTensor, CandleError> LazyTensor::mul_scalar(float value) const {
    return add_operation(Operation::mul_scalar(value), {node_});
}
Result<LazyTensor, CandleError> LazyTensor::softmax(size_t dim) const {
    return add_operation(Operation::softmax(dim), {node_});
}
Result<LazyTensor, CandleError> LazyTensor::rms_norm(float eps) const {
    return add_operation(Operation::rms_norm(eps), {node_});
}
Result<LazyTensor, CandleError> LazyTensor::lora_fused(const LazyTensor& lora_a, const LazyTensor& lora_b,
                                                       float scale) const {
    const NodeId a = merge_graph_from(lora_a), b = merge_graph_from(lora_b);
    return add_operation(Operation::lora(a, b, scale), {node_, a, b});
}

Result<Tensor, TrainingError> LazyTensor::eval() const {
    // lazy_tensor.rs:342-424, with the reference's error texts
    std::vector<NodeId> order;
    {
        std::lock_guard<std::mutex> lk(graph_->mu);
        auto o = graph_->graph.topological_order(node_);
        if (o.is_err()) return TrainingError::failed("Failed to compute execution order: " + o.error());
        order = std::move(o.value());
    }
    auto ex = AsyncExecutor::create(device_);
    if (ex.is_err()) return ex.error();
    for (NodeId id : order) {
        Operation op;
        std::vector<Tensor> inputs;
        {
            std::lock_guard<std::mutex> lk(graph_->mu);
            auto n = graph_->graph.get_node(id);
            if (n.is_err()) return TrainingError::failed("Failed to get node: " + n.error());
            if (n.value()->is_available()) continue;
            op = n.value()->operation;
            for (NodeId in : n.value()->inputs) {
                auto i = graph_->graph.get_node(in);
                if (i.is_err()) return TrainingError::failed("Failed to get input node: " + i.error());
                if (!i.value()->is_available())
                    return TrainingError::failed("Input not available: Data not yet available");
                inputs.push_back(i.value()->tensor);
            }
        }
        auto out = ex.value().execute_operation(op, inputs);  // the device work runs outside the lock
        if (out.is_err()) return out.error();
        std::lock_guard<std::mutex> lk(graph_->mu);
        auto n = graph_->graph.get_node_mut(id);
        if (n.is_err()) return TrainingError::failed("Failed to get node for result: " + n.error());
        n.value()->tensor = std::move(out.value());
        n.value()->data = GraphNode::Data::Available;
    }
    auto sync = ex.value().synchronize();
    if (sync.is_err()) return sync.error();
    std::lock_guard<std::mutex> lk(graph_->mu);
    auto n = graph_->graph.get_node(node_);
    if (n.is_err()) return TrainingError::failed("Failed to get output node: " + n.error());
    if (!n.value()->is_available()) return TrainingError::failed("Failed to get output tensor: Data not yet available");
    return n.value()->tensor;
}

std::string LazyTensor::debug_string() const {
    std::ostringstream s;  // lazy_tensor.rs:428-438
    s << "LazyTensor { node_id: " << node_id_string(node_) << ", shape: " << dims_to_string(shape_)
      << ", device: " << (device_.is_cpu() ? "Cpu" : "Hip(" + std::to_string(device_.ordinal) + ")")
      << ", graph_size: " << graph_size() << ", .. }";
    return s.str();
}

// ------------------------------------------------------------------ LoRALayer::forward_lazy
Result<LazyTensor, Error> LoRALayer::forward_lazy(const LazyTensor& input) const {
    // lora.rs:372-439
    auto a = input.add_tensor_to_graph(lora_a_);
    if (a.is_err()) return Error::from(TrainingError::failed("Failed to add LoRA A to graph: " + a.error().msg));
    auto b = input.add_tensor_to_graph(lora_b_);
    if (b.is_err()) return Error::from(TrainingError::failed("Failed to add LoRA B to graph: " + b.error().msg));
    if (input.device().is_hip() && config_.dropout == 0.f) {
        auto y = input.lora_fused(a.value(), b.value(), config_.scaling());
        if (y.is_err()) return Error::from(TrainingError::failed("Fused LoRA operation failed: " + y.error().msg));
        return std::move(y.value());
    }
    auto hidden = input.matmul(a.value());
    if (hidden.is_err()) return Error::from(TrainingError::failed("LoRA matmul A failed: " + hidden.error().msg));
    auto out = hidden.value().matmul(b.value());
    if (out.is_err()) return Error::from(TrainingError::failed("LoRA matmul B failed: " + out.error().msg));
    auto scaled = out.value().mul_scalar(config_.scaling());
    if (scaled.is_err()) return Error::from(TrainingError::failed("LoRA scaling failed: " + scaled.error().msg));
    return std::move(scaled.value());
}

std::string AsyncExecutor::debug_string() const {
    std::ostringstream s;
    s << "AsyncExecutor { device: " << (device_.is_cpu() ? "Cpu" : "Hip(") ;
    if (device_.is_hip()) s << device_.ordinal << ")";
    s << " }";
    return s.str();
}

}  // namespace mc_candle
