// LoRA adapter container and adapter checkpoints (safetensors) of the C++
// host interface.
//
// LoRAAdapter mirrors src/training/adapter.rs; save_checkpoint /
// load_checkpoint mirror src/training/checkpoint.rs:29-103, which write and
// read through the safetensors crate (0.4, not vendored) and candle's
// safetensors loader. The container format is restated here from its
// published description: an 8-byte little-endian header length N, N bytes of
// JSON (an optional "__metadata__" map of strings, then one entry per tensor:
// {"dtype": ..., "shape": [...], "data_offsets": [begin, end]}, offsets
// relative to the data section), padded with spaces so that 8 + N is a
// multiple of 8, then the data. The crate writes the JSON without whitespace,
// the metadata first, and the tensors ordered by dtype (descending in its
// dtype list) and then by name; this writer does the same, so a checkpoint's
// bytes equal the crate's for the same tensors.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cerrno>
#include <charconv>
#include <cmath>
#include <sstream>

#include <hip/hip_runtime_api.h>

#include "mc_candle.hpp"

namespace mc_candle {

namespace {

Error io_error(const std::string& msg) {
    // checkpoint.rs:62-63 maps the crate's errors to Error::Io ("io error: {0}")
    return Error::from(CandleError{"io error: " + msg});
}

Error load_error(const std::string& msg) { return Error::from(CandleError{msg}); }

// The safetensors dtype names and their place in the crate's dtype order
// (the order its Dtype enum declares them in; higher sorts first).
struct DtypeInfo {
    DType dtype;
    const char* name;
    int rank;
    size_t size;
};
constexpr DtypeInfo kDtypes[] = {
    {DType::U8, "U8", 1, 1},
    {DType::BF16, "BF16", 8, 2},
    {DType::U32, "U32", 10, 4},
    {DType::F32, "F32", 11, 4},
};

const DtypeInfo* dtype_info(DType d) {
    for (const auto& i : kDtypes)
        if (i.dtype == d) return &i;
    return nullptr;
}

const DtypeInfo* dtype_info(const std::string& name) {
    for (const auto& i : kDtypes)
        if (name == i.name) return &i;
    return nullptr;
}

// JSON string as serde_json writes it: ", \, and control characters escaped.
void json_string(std::string& out, const std::string& s) {
    out += '"';
    for (unsigned char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            default:
                if (c < 0x20) {
                    char buf[8];
                    snprintf(buf, sizeof(buf), "\\u%04x", c);
                    out += buf;
                } else {
                    out += (char)c;
                }
        }
    }
    out += '"';
}

// An f32 as serde_json prints it: the shortest digits that round-trip,
// laid out as the ryu crate does (plain decimals for exponents -5 .. 16,
// scientific beyond, a ".0" on integral values).
std::string json_f32(float v) {
    if (!std::isfinite(v)) return "null";
    if (v == 0.f) return std::signbit(v) ? "-0.0" : "0.0";
    char buf[64];
    auto r = std::to_chars(buf, buf + sizeof(buf), v, std::chars_format::scientific);
    std::string sci(buf, r.ptr);  // [-]d[.ddd]e[+-]XX
    std::string out;
    size_t p = 0;
    if (sci[0] == '-') {
        out += '-';
        p = 1;
    }
    const size_t e = sci.find('e');
    std::string digits;
    for (size_t i = p; i < e; ++i)
        if (sci[i] != '.') digits += sci[i];
    const int exp10 = std::stoi(sci.substr(e + 1));
    const int n = (int)digits.size();
    const int kk = exp10 + 1;  // value = 0.d1d2..dn x 10^kk
    if (0 <= exp10 && kk <= 16) {
        if (n <= kk) {
            out += digits + std::string((size_t)(kk - n), '0') + ".0";
        } else {
            out += digits.substr(0, (size_t)kk) + "." + digits.substr((size_t)kk);
        }
    } else if (-5 < kk && kk <= 0) {
        out += "0." + std::string((size_t)(-kk), '0') + digits;
    } else if (n == 1) {
        out += digits + "e" + std::to_string(kk - 1);
    } else {
        out += digits.substr(0, 1) + "." + digits.substr(1) + "e" + std::to_string(kk - 1);
    }
    return out;
}

// ------------------------------------------------------------- JSON reader
// Enough JSON for a safetensors header: objects, strings, integer arrays,
// numbers (kept as text).
struct JVal {
    enum Kind { Null, Str, Num, Arr, Obj, Bool } kind = Null;
    std::string s;
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;
};

struct JParser {
    const std::string& t;
    size_t i = 0;
    bool ok = true;
    explicit JParser(const std::string& text) : t(text) {}
    void ws() {
        while (i < t.size() && (t[i] == ' ' || t[i] == '\n' || t[i] == '\r' || t[i] == '\t')) ++i;
    }
    bool eat(char c) {
        ws();
        if (i < t.size() && t[i] == c) {
            ++i;
            return true;
        }
        return false;
    }
    std::string str() {
        std::string out;
        if (!eat('"')) {
            ok = false;
            return out;
        }
        while (i < t.size() && t[i] != '"') {
            char c = t[i++];
            if (c == '\\' && i < t.size()) {
                char e = t[i++];
                switch (e) {
                    case 'n': out += '\n'; break;
                    case 'r': out += '\r'; break;
                    case 't': out += '\t'; break;
                    case 'b': out += '\b'; break;
                    case 'f': out += '\f'; break;
                    case 'u': {
                        if (i + 4 > t.size()) {
                            ok = false;
                            return out;
                        }
                        unsigned cp = 0;
                        const char* h0 = t.data() + i;
                        const auto hr = std::from_chars(h0, h0 + 4, cp, 16);
                        if (hr.ec != std::errc() || hr.ptr != h0 + 4) {  // four hex digits, nothing else
                            ok = false;
                            return out;
                        }
                        i += 4;
                        if (cp < 0x80) {
                            out += (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xC0 | (cp >> 6));
                            out += (char)(0x80 | (cp & 0x3F));
                        } else {
                            out += (char)(0xE0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3F));
                            out += (char)(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: out += e;
                }
            } else {
                out += c;
            }
        }
        if (i >= t.size()) ok = false;
        ++i;
        return out;
    }
    JVal value(int depth = 0) {
        JVal v;
        ws();
        if (i >= t.size() || depth > 8) {
            ok = false;
            return v;
        }
        const char c = t[i];
        if (c == '"') {
            v.kind = JVal::Str;
            v.s = str();
        } else if (c == '{') {
            ++i;
            v.kind = JVal::Obj;
            if (eat('}')) return v;
            do {
                std::string k = str();
                if (!eat(':')) {
                    ok = false;
                    return v;
                }
                v.o.emplace_back(k, value(depth + 1));
            } while (ok && eat(','));
            if (!eat('}')) ok = false;
        } else if (c == '[') {
            ++i;
            v.kind = JVal::Arr;
            if (eat(']')) return v;
            do v.a.push_back(value(depth + 1));
            while (ok && eat(','));
            if (!eat(']')) ok = false;
        } else if (c == 't' || c == 'f' || c == 'n') {
            const char* w = c == 't' ? "true" : c == 'f' ? "false" : "null";
            if (t.compare(i, strlen(w), w) != 0) ok = false;
            i += strlen(w);
            v.kind = c == 'n' ? JVal::Null : JVal::Bool;
            v.s = w;
        } else {
            size_t j = i;
            while (j < t.size() && (isdigit((unsigned char)t[j]) || t[j] == '-' || t[j] == '+' || t[j] == '.' ||
                                    t[j] == 'e' || t[j] == 'E'))
                ++j;
            if (j == i) ok = false;
            v.kind = JVal::Num;
            v.s = t.substr(i, j - i);
            i = j;
        }
        return v;
    }
};

// A JSON number that is a whole decimal in [0, 2^64): no sign, fraction or
// exponent, and no overflow (from_chars reports it instead of throwing).
bool to_u64(const JVal& v, uint64_t& out) {
    if (v.kind != JVal::Num || v.s.empty()) return false;
    for (char c : v.s)
        if (!isdigit((unsigned char)c)) return false;
    const char* b = v.s.data();
    const char* e = b + v.s.size();
    const auto r = std::from_chars(b, e, out);
    return r.ec == std::errc() && r.ptr == e;
}

// A JSON number as f32: the whole text must parse (strtod, then rounded to
// f32 as serde does for an f32 field); out-of-range magnitudes fail.
bool to_f32(const JVal& v, float& out) {
    if (v.kind != JVal::Num || v.s.empty()) return false;
    const char* b = v.s.c_str();
    char* end = nullptr;
    errno = 0;
    const double d = std::strtod(b, &end);
    if (end != b + v.s.size() || !std::isfinite(d) || std::fabs(d) > 3.4028234663852886e38) return false;
    if (errno == ERANGE && d != 0.0) return false;
    out = (float)d;
    return true;
}

Result<std::vector<uint8_t>, Error> host_bytes(const Tensor& t) {
    std::vector<uint8_t> b(t.size_bytes());
    if (b.empty()) return b;
    if (t.device().is_cpu()) {
        memcpy(b.data(), t.data(), b.size());
    } else {
        hipError_t e = hipMemcpy(b.data(), t.data(), b.size(), hipMemcpyDeviceToHost);
        if (e != hipSuccess) return io_error(std::string("hipMemcpy D2H: ") + hipGetErrorString(e));
    }
    return b;
}

}  // namespace

// ------------------------------------------------------------------ adapter
const char* target_module_name(TargetModule m) {
    switch (m) {  // adapter.rs:36-45
        case TargetModule::QProj: return "q_proj";
        case TargetModule::KProj: return "k_proj";
        case TargetModule::VProj: return "v_proj";
        case TargetModule::OProj: return "o_proj";
        case TargetModule::GateProj: return "gate_proj";
        case TargetModule::UpProj: return "up_proj";
        default: return "down_proj";
    }
}

std::optional<TargetModule> target_module_from_name(const std::string& name) {
    for (TargetModule m : {TargetModule::QProj, TargetModule::KProj, TargetModule::VProj, TargetModule::OProj,
                           TargetModule::GateProj, TargetModule::UpProj, TargetModule::DownProj})
        if (name == target_module_name(m)) return m;
    return std::nullopt;
}

bool LoRAAdapterConfig::is_target(TargetModule m) const {
    return std::find(target_modules.begin(), target_modules.end(), m) != target_modules.end();
}

static std::string layer_key(size_t layer_idx, TargetModule m) {
    return "layers." + std::to_string(layer_idx) + "." + target_module_name(m);
}

Result<LoRAAdapter, Error> LoRAAdapter::create(size_t hidden_size, size_t intermediate_size, size_t num_layers,
                                               const LoRAAdapterConfig& config, const Device& device,
                                               uint64_t seed) {
    LoRAAdapter a;
    a.config_ = config;
    a.num_layers_ = num_layers;
    const LoRAConfig lc = config.to_lora_config();
    uint64_t n = 0;
    for (size_t l = 0; l < num_layers; ++l) {
        for (TargetModule m : config.target_modules) {
            size_t in = hidden_size, out = hidden_size;  // adapter.rs:193-206
            if (m == TargetModule::GateProj || m == TargetModule::UpProj) out = intermediate_size;
            if (m == TargetModule::DownProj) in = intermediate_size;
            auto layer = LoRALayer::create(in, out, lc, device, seed + 1000003ull * (++n));
            if (layer.is_err()) return layer.error();
            a.layers_.emplace(layer_key(l, m), std::move(layer.value()));
        }
    }
    return a;
}

Result<std::optional<Tensor>, Error> LoRAAdapter::forward(size_t layer_idx, TargetModule module,
                                                          const Tensor& input) {
    auto it = layers_.find(layer_key(layer_idx, module));
    if (it == layers_.end()) return std::optional<Tensor>();
    auto d = it->second.forward(input);
    if (d.is_err()) return d.error();
    return std::optional<Tensor>(std::move(d.value()));
}

size_t LoRAAdapter::num_trainable_parameters() const {
    size_t n = 0;
    for (const auto& kv : layers_) n += kv.second.num_parameters();
    return n;
}

size_t LoRAAdapter::num_frozen_parameters(size_t total) const {
    const size_t t = num_trainable_parameters();
    return total > t ? total - t : 0;  // saturating_sub
}

const LoRALayer* LoRAAdapter::get_layer(size_t layer_idx, TargetModule module) const {
    auto it = layers_.find(layer_key(layer_idx, module));
    return it == layers_.end() ? nullptr : &it->second;
}

LoRALayer* LoRAAdapter::get_layer_mut(size_t layer_idx, TargetModule module) {
    auto it = layers_.find(layer_key(layer_idx, module));
    return it == layers_.end() ? nullptr : &it->second;
}

// ------------------------------------------------------------------ metadata
std::string CheckpointMetadata::to_json() const {
    // serde_json of the struct: fields in declaration order (checkpoint.rs:14-26)
    return "{\"global_step\":" + std::to_string(global_step) + ",\"loss\":" + json_f32(loss) +
           ",\"learning_rate\":" + json_f32(learning_rate) + ",\"timestamp\":" + std::to_string(timestamp) + "}";
}

std::optional<CheckpointMetadata> CheckpointMetadata::from_json(const std::string& json) {
    JParser p(json);
    JVal v = p.value();
    if (!p.ok || v.kind != JVal::Obj) return std::nullopt;
    CheckpointMetadata m;
    int seen = 0;
    for (const auto& kv : v.o) {
        if (kv.first == "global_step" && to_u64(kv.second, m.global_step)) seen |= 1;
        if (kv.first == "timestamp" && to_u64(kv.second, m.timestamp)) seen |= 8;
        if (kv.first == "loss") {
            if (!to_f32(kv.second, m.loss)) return std::nullopt;
            seen |= 2;
        }
        if (kv.first == "learning_rate") {
            if (!to_f32(kv.second, m.learning_rate)) return std::nullopt;
            seen |= 4;
        }
    }
    if (seen != 15) return std::nullopt;
    return m;
}

// ------------------------------------------------------------------ safetensors
Result<void, Error> safetensors_save(const std::vector<std::pair<std::string, Tensor>>& tensors,
                                     const std::map<std::string, std::string>* metadata, const std::string& path) {
    std::vector<const std::pair<std::string, Tensor>*> order;
    for (const auto& t : tensors) {
        if (!dtype_info(t.second.dtype())) return io_error("unsupported dtype for tensor " + t.first);
        order.push_back(&t);
    }
    std::sort(order.begin(), order.end(), [](const auto* a, const auto* b) {
        const int ra = dtype_info(a->second.dtype())->rank, rb = dtype_info(b->second.dtype())->rank;
        if (ra != rb) return ra > rb;
        return a->first < b->first;
    });
    for (size_t i = 1; i < order.size(); ++i)
        if (order[i]->first == order[i - 1]->first) return io_error("duplicate tensor name " + order[i]->first);
    std::string h = "{";
    bool first = true;
    if (metadata) {
        h += "\"__metadata__\":{";
        bool f2 = true;
        for (const auto& kv : *metadata) {
            if (!f2) h += ',';
            f2 = false;
            json_string(h, kv.first);
            h += ':';
            json_string(h, kv.second);
        }
        h += '}';
        first = false;
    }
    uint64_t off = 0;
    for (const auto* t : order) {
        if (!first) h += ',';
        first = false;
        json_string(h, t->first);
        h += ":{\"dtype\":\"";
        h += dtype_info(t->second.dtype())->name;
        h += "\",\"shape\":[";
        for (size_t d = 0; d < t->second.dims().size(); ++d) {
            if (d) h += ',';
            h += std::to_string(t->second.dims()[d]);
        }
        const uint64_t n = t->second.size_bytes();
        h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + n) + "]}";
        off += n;
    }
    h += '}';
    h.append((8 - h.size() % 8) % 8, ' ');
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) return io_error("cannot create " + path + ": " + strerror(errno));
    uint8_t len[8];
    const uint64_t hn = h.size();
    for (int i = 0; i < 8; ++i) len[i] = (uint8_t)(hn >> (8 * i));
    bool ok = fwrite(len, 1, 8, f) == 8 && fwrite(h.data(), 1, h.size(), f) == h.size();
    for (const auto* t : order) {
        if (!ok) break;
        auto b = host_bytes(t->second);
        if (b.is_err()) {
            fclose(f);
            return b.error();
        }
        ok = b.value().empty() || fwrite(b.value().data(), 1, b.value().size(), f) == b.value().size();
    }
    if (fclose(f) != 0) ok = false;
    if (!ok) return io_error("write to " + path + " failed");
    return {};
}

Result<std::map<std::string, Tensor>, Error> safetensors_load(const std::string& path, const Device& device,
                                                              std::map<std::string, std::string>* metadata) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return load_error("cannot open " + path + ": " + strerror(errno));
    std::vector<uint8_t> file;
    uint8_t buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), f)) > 0) file.insert(file.end(), buf, buf + n);
    fclose(f);
    if (file.size() < 8) return load_error("safetensors: header too small");
    uint64_t hn = 0;
    for (int i = 0; i < 8; ++i) hn |= (uint64_t)file[i] << (8 * i);
    if (hn > file.size() - 8 || hn > 100000000) return load_error("safetensors: invalid header length");
    const std::string header((const char*)file.data() + 8, (size_t)hn);
    JParser p(header);
    JVal root = p.value();
    if (!p.ok || root.kind != JVal::Obj) return load_error("safetensors: invalid header JSON");
    const uint64_t data0 = 8 + hn, data_len = file.size() - data0;
    std::map<std::string, Tensor> out;
    std::vector<std::pair<uint64_t, uint64_t>> spans;
    for (const auto& kv : root.o) {
        if (kv.first == "__metadata__") {
            if (kv.second.kind != JVal::Obj) return load_error("safetensors: invalid __metadata__");
            if (metadata)
                for (const auto& m : kv.second.o) {
                    if (m.second.kind != JVal::Str) return load_error("safetensors: metadata values must be strings");
                    (*metadata)[m.first] = m.second.s;
                }
            continue;
        }
        const JVal& t = kv.second;
        const JVal *dt = nullptr, *sh = nullptr, *of = nullptr;
        for (const auto& e : t.o) {
            if (e.first == "dtype") dt = &e.second;
            if (e.first == "shape") sh = &e.second;
            if (e.first == "data_offsets") of = &e.second;
        }
        if (!dt || !sh || !of || dt->kind != JVal::Str || sh->kind != JVal::Arr || of->kind != JVal::Arr ||
            of->a.size() != 2)
            return load_error("safetensors: invalid entry for tensor " + kv.first);
        const DtypeInfo* di = dtype_info(dt->s);
        if (!di) return load_error("safetensors: unsupported dtype " + dt->s + " for tensor " + kv.first);
        std::vector<int64_t> dims;
        uint64_t count = 1;
        for (const JVal& d : sh->a) {
            uint64_t v;
            if (!to_u64(d, v) || v > (uint64_t)INT64_MAX)
                return load_error("safetensors: invalid shape for tensor " + kv.first);
            dims.push_back((int64_t)v);
            if (__builtin_mul_overflow(count, v, &count))
                return load_error("safetensors: element count of tensor " + kv.first + " overflows");
        }
        uint64_t nbytes = 0;
        if (__builtin_mul_overflow(count, (uint64_t)di->size, &nbytes))
            return load_error("safetensors: byte size of tensor " + kv.first + " overflows");
        uint64_t b0, b1;
        if (!to_u64(of->a[0], b0) || !to_u64(of->a[1], b1) || b1 < b0 || b1 > data_len)
            return load_error("safetensors: invalid data_offsets for tensor " + kv.first);
        if (b1 - b0 != nbytes)
            return load_error("safetensors: tensor " + kv.first + " has " + std::to_string(b1 - b0) +
                              " bytes for its shape " + dims_to_string(dims));
        spans.emplace_back(b0, b1);
        auto tt = Tensor::empty(dims, di->dtype, device);
        if (tt.is_err()) return Error::from(tt.error());
        if (b1 > b0) {
            const uint8_t* src = file.data() + data0 + b0;
            if (device.is_cpu()) {
                memcpy(tt.value().data(), src, (size_t)(b1 - b0));
            } else {
                hipError_t e = hipMemcpy(tt.value().data(), src, (size_t)(b1 - b0), hipMemcpyHostToDevice);
                if (e != hipSuccess) return load_error(std::string("hipMemcpy H2D: ") + hipGetErrorString(e));
            }
        }
        out.emplace(kv.first, std::move(tt.value()));
    }
    // the data section is covered exactly, without overlaps
    std::sort(spans.begin(), spans.end());
    uint64_t end = 0;
    for (const auto& s : spans) {
        if (s.first != end) return load_error("safetensors: data_offsets leave gaps or overlap");
        end = s.second;
    }
    if (end != data_len) return load_error("safetensors: data section length does not match the header");
    return out;
}

// ------------------------------------------------------------------ checkpoints
Result<void, Error> save_checkpoint(const LoRAAdapter& adapter, const std::string& path,
                                    const CheckpointMetadata* metadata) {
    std::vector<std::pair<std::string, Tensor>> tensors;
    for (const auto& kv : adapter.layers()) {  // checkpoint.rs:36-45
        tensors.emplace_back(kv.first + ".lora_a", kv.second.lora_a_tensor());
        tensors.emplace_back(kv.first + ".lora_b", kv.second.lora_b_tensor());
    }
    std::map<std::string, std::string> meta;
    if (metadata) meta["checkpoint_metadata"] = metadata->to_json();  // checkpoint.rs:48-55
    return safetensors_save(tensors, metadata ? &meta : nullptr, path);
}

Result<std::optional<CheckpointMetadata>, Error> load_checkpoint(LoRAAdapter& adapter, const std::string& path) {
    if (adapter.layers().empty()) return load_error("load_checkpoint: the adapter has no layers");
    const Device device = adapter.layers().begin()->second.lora_a_tensor().device();  // checkpoint.rs:74-75
    auto tensors = safetensors_load(path, device);
    if (tensors.is_err()) return tensors.error();
    for (auto& kv : adapter.layers_mut()) {  // checkpoint.rs:84-96
        auto a = tensors.value().find(kv.first + ".lora_a");
        if (a != tensors.value().end()) {
            auto r = kv.second.set_lora_a(a->second);
            if (r.is_err()) return r.error();
        }
        auto b = tensors.value().find(kv.first + ".lora_b");
        if (b != tensors.value().end()) {
            auto r = kv.second.set_lora_b(b->second);
            if (r.is_err()) return r.error();
        }
    }
    return std::optional<CheckpointMetadata>();  // checkpoint.rs:80-82: metadata is not loaded
}

Result<std::optional<CheckpointMetadata>, Error> read_checkpoint_metadata(const std::string& path) {
    std::map<std::string, std::string> meta;
    auto t = safetensors_load(path, Device::cpu(), &meta);
    if (t.is_err()) return t.error();
    auto it = meta.find("checkpoint_metadata");
    if (it == meta.end()) return std::optional<CheckpointMetadata>();
    auto m = CheckpointMetadata::from_json(it->second);
    if (!m) return load_error("safetensors: checkpoint_metadata is not a valid CheckpointMetadata");
    return m;
}

}  // namespace mc_candle
