// Checkpoint loading (include/mrun_load.h): the counterpart of crates/mrun-engine/src/load.rs
// and SparseMoe::load (models/moe.rs:120-147), for MLX and Hugging Face safetensors checkpoints.
//
//   json        — the subset of JSON that config.json and safetensors headers use
//   Weights     — tensor headers of every *.safetensors file (data mapped, read when taken); a
//                 tensor is a list of byte ranges, so the Hugging Face restatements (stacked
//                 per-expert weights, split gate_up) need no copies until the device upload
//   Quantization— config.json `quantization` with per-path overrides, resolve and infer
//   load_moe    — Linear::load / SwitchLinear::load for each projection, then device copies
#include <dirent.h>
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "mrun_load.h"
#include "mrun_moe.h"
#include "status.hpp"

namespace mrun {
namespace json {

struct Value {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<Value> arr;
    std::vector<std::pair<std::string, Value>> obj;  // in file order

    const Value *get(const std::string &key) const {
        if (kind != Obj) return nullptr;
        for (const auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
    bool is_int() const { return kind == Num && std::floor(num) == num && std::fabs(num) < 9e15; }
};

class Parser {
  public:
    Parser(const char *p, size_t n) : p_(p), end_(p + n) {}

    bool parse(Value &v, std::string &err) {
        if (!value(v, 0)) {
            err = err_.empty() ? "malformed JSON" : err_;
            return false;
        }
        ws();
        if (p_ != end_) {
            err = "trailing characters after JSON";
            return false;
        }
        return true;
    }

  private:
    const char *p_, *end_;
    std::string err_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool lit(const char *s) {
        const size_t n = std::strlen(s);
        if ((size_t)(end_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(uint32_t c, std::string &out) {
        if (c < 0x80) {
            out += (char)c;
        } else if (c < 0x800) {
            out += (char)(0xC0 | (c >> 6));
            out += (char)(0x80 | (c & 0x3F));
        } else if (c < 0x10000) {
            out += (char)(0xE0 | (c >> 12));
            out += (char)(0x80 | ((c >> 6) & 0x3F));
            out += (char)(0x80 | (c & 0x3F));
        } else {
            out += (char)(0xF0 | (c >> 18));
            out += (char)(0x80 | ((c >> 12) & 0x3F));
            out += (char)(0x80 | ((c >> 6) & 0x3F));
            out += (char)(0x80 | (c & 0x3F));
        }
    }
    bool hex4(uint32_t &c) {
        if (end_ - p_ < 4) return false;
        c = 0;
        for (int i = 0; i < 4; ++i) {
            const char h = *p_++;
            c <<= 4;
            if (h >= '0' && h <= '9') c |= (uint32_t)(h - '0');
            else if (h >= 'a' && h <= 'f') c |= (uint32_t)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') c |= (uint32_t)(h - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string &out) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (p_ >= end_) return false;
            c = *p_++;
            switch (c) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        uint32_t lo;
                        if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(cp, out);
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool number(double &v) {
        const char *s = p_;
        if (p_ < end_ && (*p_ == '-' || *p_ == '+')) ++p_;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                             *p_ == '-' || *p_ == '+'))
            ++p_;
        if (p_ == s) return false;
        const std::string t(s, p_);
        char *e = nullptr;
        v = std::strtod(t.c_str(), &e);
        return e && *e == '\0';
    }
    bool value(Value &v, int depth) {
        if (depth > 64) {
            err_ = "JSON nested too deeply";
            return false;
        }
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Value::Obj;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                Value item;
                if (!value(item, depth + 1)) return false;
                v.obj.emplace_back(std::move(key), std::move(item));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == '}') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = Value::Arr;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                Value item;
                if (!value(item, depth + 1)) return false;
                v.arr.push_back(std::move(item));
                ws();
                if (p_ < end_ && *p_ == ',') {
                    ++p_;
                    continue;
                }
                if (p_ < end_ && *p_ == ']') {
                    ++p_;
                    return true;
                }
                return false;
            }
        }
        if (c == '"') {
            v.kind = Value::Str;
            return string(v.str);
        }
        if (lit("true")) {
            v.kind = Value::Bool, v.b = true;
            return true;
        }
        if (lit("false")) {
            v.kind = Value::Bool, v.b = false;
            return true;
        }
        if (lit("null")) {
            v.kind = Value::Null;
            return true;
        }
        v.kind = Value::Num;
        return number(v.num);
    }
};

}  // namespace json

namespace load {

static Status invalid(const std::string &key, const std::string &reason) {
    return Err(MRUN_ERR_INVALID, key + ": " + reason);
}

static std::string shape_str(const std::vector<int64_t> &s) {
    std::string out = "[";
    for (size_t i = 0; i < s.size(); ++i) out += (i ? ", " : "") + std::to_string(s[i]);
    return out + "]";
}

// ---------------------------------------------------------------------------------------------
// Weights (load.rs:158-256)

struct Mapped {
    std::string path;
    const char *base = nullptr;
    size_t size = 0;
};

struct Range {
    int file;
    size_t begin, bytes;  // absolute offsets in the mapped file
};

struct Tensor {
    std::string dtype;
    std::vector<int64_t> shape;
    std::vector<Range> parts;  // concatenated in order

    size_t bytes() const {
        size_t n = 0;
        for (const Range &r : parts) n += r.bytes;
        return n;
    }
    int64_t dim(int i) const { return shape[i < 0 ? (int)shape.size() + i : i]; }
};

static size_t dtype_size(const std::string &d) {
    if (d == "BF16" || d == "F16" || d == "I16" || d == "U16") return 2;
    if (d == "F32" || d == "U32" || d == "I32") return 4;
    if (d == "F64" || d == "I64" || d == "U64") return 8;
    if (d == "U8" || d == "I8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    return 0;
}

// unused_tensor (load.rs:164-173)
static bool unused_tensor(const std::string &name) {
    return name.rfind("vision_tower", 0) == 0 || name.rfind("model.visual", 0) == 0 ||
           name.find("mtp.") != std::string::npos ||
           name.find("rotary_emb.inv_freq") != std::string::npos;
}

struct QParams {
    int group_size, bits;
};

// Quantization (load.rs:44-126)
struct Quantization {
    std::map<std::string, std::optional<QParams>> overrides;
};

}  // namespace load
}  // namespace mrun

struct mrun_weights {
    std::vector<mrun::load::Mapped> files;
    std::map<std::string, mrun::load::Tensor> tensors;
    mrun::json::Value config;
    bool has_config = false;
    mrun::load::Quantization quant;
    std::vector<void *> device;  // allocations owned by the checkpoint

    ~mrun_weights() {
        for (void *p : device) (void)hipFree(p);
        for (auto &f : files)
            if (f.base) munmap((void *)f.base, f.size);
    }
};

namespace mrun {
namespace load {

static Status map_file(const std::string &path, Mapped &m) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return invalid("weights", "cannot open " + path);
    struct stat st{};
    if (fstat(fd, &st) != 0 || st.st_size < 8) {
        ::close(fd);
        return invalid("weights", path + ": not a safetensors file");
    }
    void *base = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (base == MAP_FAILED) return invalid("weights", "cannot map " + path);
    m.path = path, m.base = (const char *)base, m.size = (size_t)st.st_size;
    return Ok();
}

// One safetensors file: u64 header length, JSON header {name: {dtype, shape, data_offsets}},
// then the data region the offsets are relative to.
static Status read_header(mrun_weights &w, int fi) {
    const Mapped &m = w.files[fi];
    uint64_t n = 0;
    std::memcpy(&n, m.base, 8);
    if (n > m.size - 8) return invalid("weights", m.path + ": header past the end of the file");
    json::Value h;
    std::string err;
    if (!json::Parser(m.base + 8, (size_t)n).parse(h, err) || h.kind != json::Value::Obj)
        return invalid("weights", m.path + ": bad header (" + err + ")");
    const size_t data = 8 + (size_t)n;
    for (const auto &kv : h.obj) {
        if (kv.first == "__metadata__") continue;
        const json::Value &t = kv.second;
        const json::Value *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
        if (!dt || dt->kind != json::Value::Str || !sh || sh->kind != json::Value::Arr || !off ||
            off->kind != json::Value::Arr || off->arr.size() != 2 || !off->arr[0].is_int() ||
            !off->arr[1].is_int())
            return invalid("weights", m.path + ": bad entry for " + kv.first);
        Tensor ten;
        ten.dtype = dt->str;
        int64_t count = 1;
        for (const json::Value &d : sh->arr) {
            if (!d.is_int() || d.num < 0) return invalid("weights", m.path + ": bad shape of " + kv.first);
            ten.shape.push_back((int64_t)d.num);
            count *= (int64_t)d.num;
        }
        const size_t b = (size_t)off->arr[0].num, e = (size_t)off->arr[1].num;
        const size_t es = dtype_size(ten.dtype);
        if (e < b || data + e > m.size || (es && (size_t)count * es != e - b))
            return invalid("weights", m.path + ": data of " + kv.first + " does not match its header");
        if (unused_tensor(kv.first)) continue;
        ten.parts.push_back(Range{fi, data + b, e - b});
        w.tensors.emplace(kv.first, std::move(ten));  // the first file holding a name keeps it
    }
    return Ok();
}

// Quantization::from_config (load.rs:52-103)
static Status params(const std::string &path, const json::Value &v, std::optional<QParams> base,
                     std::optional<QParams> &out) {
    if (const json::Value *mode = v.get("mode"); mode && mode->kind == json::Value::Str &&
                                                 mode->str != "affine")
        return invalid("quantization", path + ": quantization mode " + mode->str +
                                           " cannot be loaded; this build reads affine codes");
    std::optional<int> g, b;
    if (const json::Value *x = v.get("group_size"); x && x->is_int()) g = (int)x->num;
    else if (base) g = base->group_size;
    if (const json::Value *x = v.get("bits"); x && x->is_int()) b = (int)x->num;
    else if (base) b = base->bits;
    out = (g && b) ? std::optional<QParams>(QParams{*g, *b}) : std::nullopt;
    return Ok();
}

// QParams::checked (load.rs:26-41)
static Status checked(const std::string &path, QParams q) {
    const bool bits = q.bits == 4 || q.bits == 8;
    const bool group = q.group_size == 32 || q.group_size == 64 || q.group_size == 128;
    if (!bits || !group)
        return invalid("quantization", path + ": affine codes of " + std::to_string(q.bits) +
                                           " bits in groups of " + std::to_string(q.group_size) +
                                           " cannot be loaded; accepted: 4- or 8-bit codes, "
                                           "groups of 32/64/128");
    return Ok();
}

static Status quantization_from_config(const json::Value &config, Quantization &q) {
    const json::Value *root = config.get("quantization");
    if (!root || root->kind != json::Value::Obj) root = config.get("quantization_config");
    if (!root || root->kind != json::Value::Obj) return Ok();
    std::optional<QParams> def;
    TRY(params("quantization", *root, std::nullopt, def));
    for (const auto &kv : root->obj) {
        if (kv.second.kind == json::Value::Obj) {
            std::optional<QParams> named;
            TRY(params(kv.first, kv.second, def, named));
            if (named) {
                TRY(checked(kv.first, *named));
                q.overrides[kv.first] = named;
            }
        } else if (kv.second.kind == json::Value::Bool && !kv.second.b) {
            q.overrides[kv.first] = std::nullopt;
        }
    }
    return Ok();
}

// infer (load.rs:128-156)
static Status infer(const std::string &path, const Tensor &weight, const Tensor &scales,
                    int in_dims, QParams &out) {
    if (scales.dtype == "U8")
        return invalid("quantization", path + ": U8 scales belong to a microscaling format; "
                                           "this build reads affine codes with bf16 scales");
    if (weight.shape.empty() || scales.shape.empty())
        return invalid("quantization", path + ": weight and scales need at least one dimension");
    const int64_t groups = scales.dim(-1);
    if (in_dims <= 0 || groups <= 0 || in_dims % groups != 0)
        return invalid("quantization", path + ": an input width of " + std::to_string(in_dims) +
                                           " is no whole number of " + std::to_string(groups) +
                                           " groups");
    const int64_t packed = weight.dim(-1) * 32;
    if (packed % in_dims != 0)
        return invalid("quantization", path + ": a row of " + std::to_string(weight.dim(-1)) +
                                           " u32 words packs no whole number of bits per code "
                                           "for an input width of " +
                                           std::to_string(in_dims));
    out = QParams{(int)(in_dims / groups), (int)(packed / in_dims)};
    return checked(path, out);
}

// Quantization::resolve (load.rs:105-126)
static Status resolve(const Quantization &q, const std::string &path, const Tensor &weight,
                      const Tensor &scales, int in_dims, QParams &out) {
    auto it = q.overrides.find(path);
    if (it != q.overrides.end()) {
        if (!it->second)
            return invalid("quantization", path + " has codes and scales on disk, while "
                                                  "config.json lists it as a plain tensor");
        out = *it->second;
        return Ok();
    }
    return infer(path, weight, scales, in_dims, out);
}

// ---------------------------------------------------------------------------------------------
// Hugging Face layouts at a MoE prefix

// qwen3_moe.rs:39-58: experts.<e>.<proj>.weight [out, in] -> switch_mlp.<proj>.weight [E, out, in]
static Status stack_experts(mrun_weights &w, const std::string &prefix, int experts) {
    if (!w.tensors.count(prefix + ".experts.0.up_proj.weight")) return Ok();
    for (const char *name : {"up_proj", "down_proj", "gate_proj"}) {
        Tensor st;
        for (int e = 0; e < experts; ++e) {
            const std::string n = prefix + ".experts." + std::to_string(e) + "." + name + ".weight";
            auto it = w.tensors.find(n);
            if (it == w.tensors.end()) return invalid("weights", "missing tensor " + n);
            const Tensor &t = it->second;
            if (e == 0) {
                st.dtype = t.dtype;
                st.shape = t.shape;
                st.shape.insert(st.shape.begin(), experts);
            } else if (t.dtype != st.dtype ||
                       !std::equal(t.shape.begin(), t.shape.end(), st.shape.begin() + 1,
                                   st.shape.end())) {
                return invalid("weights", prefix + ".experts: expert " + std::to_string(e) +
                                              " differs in shape or dtype");
            }
            st.parts.insert(st.parts.end(), t.parts.begin(), t.parts.end());
            w.tensors.erase(it);
        }
        w.tensors[prefix + ".switch_mlp." + name + ".weight"] = std::move(st);
    }
    return Ok();
}

// qwen3_5_moe.rs:391-405: experts.gate_up_proj [E, 2I, D] -> gate [E, I, D] and up [E, I, D]
// (the halves of axis -2), experts.down_proj -> switch_mlp.down_proj.weight
static Status split_gate_up(mrun_weights &w, const std::string &prefix) {
    auto it = w.tensors.find(prefix + ".experts.gate_up_proj");
    if (it == w.tensors.end()) return Ok();
    const Tensor gu = it->second;
    w.tensors.erase(it);
    if (gu.shape.size() != 3 || gu.shape[1] % 2 != 0 || gu.parts.size() != 1)
        return invalid("weights", prefix + ".experts.gate_up_proj: gate_up_proj does not split in two");
    const int64_t E = gu.shape[0], half = gu.shape[1] / 2, D = gu.shape[2];
    const size_t es = dtype_size(gu.dtype), row = (size_t)D * es, blk = (size_t)half * row;
    Tensor gate{gu.dtype, {E, half, D}, {}}, up{gu.dtype, {E, half, D}, {}};
    for (int64_t e = 0; e < E; ++e) {
        const size_t base = gu.parts[0].begin + (size_t)e * 2 * blk;
        gate.parts.push_back(Range{gu.parts[0].file, base, blk});
        up.parts.push_back(Range{gu.parts[0].file, base + blk, blk});
    }
    w.tensors[prefix + ".switch_mlp.gate_proj.weight"] = std::move(gate);
    w.tensors[prefix + ".switch_mlp.up_proj.weight"] = std::move(up);
    auto dn = w.tensors.find(prefix + ".experts.down_proj");
    if (dn == w.tensors.end()) return invalid("weights", "missing tensor " + prefix + ".experts.down_proj");
    w.tensors[prefix + ".switch_mlp.down_proj.weight"] = std::move(dn->second);
    w.tensors.erase(dn);
    return Ok();
}

// ---------------------------------------------------------------------------------------------
// Linear::load (load.rs:274-292), kept on the host until every projection of the block checks

struct HostLinear {
    std::string path;
    std::optional<Tensor> weight, scales, biases, bias;
    QParams q{0, 0};
    bool quantized = false;
};

static Status take(mrun_weights &w, const std::string &name, Tensor &out) {
    auto it = w.tensors.find(name);
    if (it == w.tensors.end()) return invalid("weights", "missing tensor " + name);
    out = std::move(it->second);
    w.tensors.erase(it);
    return Ok();
}

static std::optional<Tensor> take_opt(mrun_weights &w, const std::string &name) {
    auto it = w.tensors.find(name);
    if (it == w.tensors.end()) return std::nullopt;
    Tensor t = std::move(it->second);
    w.tensors.erase(it);
    return t;
}

static Status linear_load(mrun_weights &w, const std::string &path, int in_dims, HostLinear &l) {
    l.path = path;
    Tensor weight;
    TRY(take(w, path + ".weight", weight));
    l.weight = std::move(weight);
    l.bias = take_opt(w, path + ".bias");
    l.scales = take_opt(w, path + ".scales");
    if (l.scales) {
        TRY(resolve(w.quant, path, *l.weight, *l.scales, in_dims, l.q));
        l.biases = take_opt(w, path + ".biases");
        l.quantized = true;
    }
    return Ok();
}

// Shape and dtype rules of the device view (Quantized::new, nuvec.rs:609-626): codes U32
// [E?, out, in*bits/32], scales and biases BF16 [E?, out, in/group]; dense weights BF16 [out, in].
static Status check_linear(const HostLinear &l, int experts, int out, int in, bool stacked,
                           bool allow_bias) {
    const std::vector<int64_t> lead = stacked ? std::vector<int64_t>{experts} : std::vector<int64_t>{};
    auto want = [&](std::vector<int64_t> tail) {
        std::vector<int64_t> s = lead;
        s.insert(s.end(), tail.begin(), tail.end());
        return s;
    };
    if (l.bias && !allow_bias) return invalid("weights", l.path + ".bias is not supported");
    if (!l.quantized) {
        // dense bf16, or f32 (an f32 checkpoint's block runs through mrun_moe_forward_f32)
        const bool f32 = l.weight->dtype == "F32";
        if (stacked && l.weight->dtype != "BF16" && !f32)
            return Err(MRUN_ERR_UNSUPPORTED,
                       l.path + ": dense " + l.weight->dtype + " " + shape_str(l.weight->shape) +
                           " experts (gather_mm) are not run by this build (bf16 or f32 only)");
        if (l.weight->dtype != "BF16" && !f32)
            return Err(MRUN_ERR_UNSUPPORTED, l.path + ": dense " + l.weight->dtype +
                                                 " weights are not run by this build (bf16 or "
                                                 "f32 only)");
        if (f32 && l.bias)
            return Err(MRUN_ERR_UNSUPPORTED, l.path + ".bias: f32 Linear biases are not run");
        if (l.weight->shape != want({out, in}))
            return invalid("weights", l.path + ".weight: shape " + shape_str(l.weight->shape) +
                                          ", expected " + shape_str(want({out, in})));
    } else {
        const int64_t words = (int64_t)in * l.q.bits / 32, groups = in / l.q.group_size;
        if (l.weight->dtype != "U32")
            return invalid("weights", l.path + ".weight: packed codes must be U32, not " + l.weight->dtype);
        if (l.weight->shape != want({out, words}))
            return invalid("weights", l.path + ".weight: shape " + shape_str(l.weight->shape) +
                                          ", expected " + shape_str(want({out, words})) + " for " +
                                          std::to_string(l.q.bits) + "-bit codes");
        if (l.scales->dtype != "BF16")
            return Err(MRUN_ERR_UNSUPPORTED,
                       l.path + ".scales: " + l.scales->dtype + " scales are not run by this build");
        if (l.scales->shape != want({out, groups}))
            return invalid("weights", l.path + ".scales: shape " + shape_str(l.scales->shape) +
                                          ", expected " + shape_str(want({out, groups})));
        if (l.biases && (l.biases->dtype != "BF16" || l.biases->shape != l.scales->shape))
            return invalid("weights", l.path + ".biases must be BF16 shaped like the scales");
    }
    if (l.bias && (l.bias->dtype != "BF16" || l.bias->shape != std::vector<int64_t>{out}))
        return invalid("weights", l.path + ".bias must be BF16 [" + std::to_string(out) + "]");
    return Ok();
}

static Status upload(mrun_weights &w, const Tensor &t, const void **out) {
    const size_t n = t.bytes();
    void *d = nullptr;
    TRY_HIP(hipMalloc(&d, n ? n : 16), "hipMalloc");
    w.device.push_back(d);
    size_t at = 0;
    for (const Range &r : t.parts) {
        TRY_HIP(hipMemcpy((char *)d + at, w.files[r.file].base + r.begin, r.bytes,
                          hipMemcpyHostToDevice),
                "hipMemcpy");
        at += r.bytes;
    }
    *out = d;
    return Ok();
}

static Status to_device(mrun_weights &w, const HostLinear &l, int experts, int out, int in,
                        mrun_linear *lin, mrun_quantized *q) {
    const void *p = nullptr;
    if (l.quantized) {
        mrun_quantized v{};
        TRY(upload(w, *l.weight, &p));
        v.weight = (const uint32_t *)p;
        TRY(upload(w, *l.scales, &p));
        v.scales = (const mrun_bf16 *)p;
        if (l.biases) {
            TRY(upload(w, *l.biases, &p));
            v.biases = (const mrun_bf16 *)p;
        }
        v.experts = experts, v.out = out, v.in = in, v.group_size = l.q.group_size, v.bits = l.q.bits;
        if (q) *q = v;
        if (lin) lin->q = v;
    } else if (q || l.weight->dtype == "F32") {
        // dense experts (gather_mm) as a 16-bit (bf16) or 32-bit (f32) stacked weight; an f32
        // Linear carries its weight the same way, in its `q`
        TRY(upload(w, *l.weight, &p));
        mrun_quantized v{};
        v.weight = (const uint32_t *)p, v.experts = experts, v.out = out, v.in = in;
        v.bits = l.weight->dtype == "F32" ? 32 : 16;
        if (q) *q = v;
        if (lin) lin->q = v;
    } else {
        TRY(upload(w, *l.weight, &p));
        lin->weight = (const mrun_bf16 *)p;
    }
    if (lin) {
        lin->out = out, lin->in = in;
        if (l.bias) {
            TRY(upload(w, *l.bias, &p));
            lin->bias = (const mrun_bf16 *)p;
        }
    }
    return Ok();
}

static Status int_field(const json::Value &c, const char *key, std::optional<int> def, int &out) {
    const json::Value *v = c.get(key);
    if (!v || v->kind == json::Value::Null) {
        if (!def) return invalid(key, "missing from config.json");
        out = *def;
        return Ok();
    }
    if (!v->is_int()) return invalid(key, "must be an integer");
    out = (int)v->num;
    return Ok();
}

static const json::Value &text_config(const mrun_weights &w) {
    const json::Value *t = w.config.get("text_config");
    return (t && t->kind == json::Value::Obj) ? *t : w.config;
}

}  // namespace load
}  // namespace mrun

using namespace mrun;
using namespace mrun::load;

extern "C" {

int mrun_weights_open(const char *dir, mrun_weights **out) {
    if (!dir || !out) return report(Err(MRUN_ERR_INVALID, "weights: null argument"));
    *out = nullptr;
    auto w = std::make_unique<mrun_weights>();
    const std::string d(dir);
    // config.json first: its quantization is refused before any tensor is read
    {
        const std::string cp = d + "/config.json";
        if (access(cp.c_str(), R_OK) == 0) {
            FILE *f = fopen(cp.c_str(), "rb");
            if (!f) return report(invalid("config", "cannot read " + cp));
            std::string text;
            char buf[65536];
            size_t n;
            while ((n = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
            fclose(f);
            std::string err;
            if (!json::Parser(text.data(), text.size()).parse(w->config, err) ||
                w->config.kind != json::Value::Obj)
                return report(invalid("config", cp + ": " + (err.empty() ? "not an object" : err)));
            w->has_config = true;
            Status st = quantization_from_config(w->config, w->quant);
            if (!st.ok()) return report(st);
        }
    }
    std::vector<std::string> files;
    if (DIR *dp = opendir(dir)) {
        while (dirent *e = readdir(dp)) {
            const std::string n = e->d_name;
            if (n.size() > 12 && n.compare(n.size() - 12, 12, ".safetensors") == 0)
                files.push_back(d + "/" + n);
        }
        closedir(dp);
    } else {
        return report(invalid("weights", "cannot read " + d));
    }
    std::sort(files.begin(), files.end());
    if (files.empty() && !w->has_config) return report(invalid("weights", "no *.safetensors files"));
    for (const std::string &f : files) {
        Mapped m;
        Status st = map_file(f, m);
        if (!st.ok()) return report(st);
        w->files.push_back(m);
        st = read_header(*w, (int)w->files.size() - 1);
        if (!st.ok()) return report(st);
    }
    if (files.empty()) return report(invalid("weights", "no *.safetensors files"));
    *out = w.release();
    return report(Ok());
}

void mrun_weights_close(mrun_weights *w) { delete w; }

int mrun_weights_moe_config(const mrun_weights *w, mrun_moe_config *cfg, float *eps) {
    if (!w || !cfg) return report(Err(MRUN_ERR_INVALID, "weights: null argument"));
    if (!w->has_config) return report(invalid("config", "config.json is missing"));
    const json::Value &c = text_config(*w);
    mrun_moe_config m{};
    Status st = int_field(c, "hidden_size", std::nullopt, m.hidden);
    if (st.ok()) st = int_field(c, "num_experts", std::nullopt, m.experts);
    if (st.ok()) st = int_field(c, "num_experts_per_tok", std::nullopt, m.top_k);
    if (st.ok()) st = int_field(c, "moe_intermediate_size", std::nullopt, m.intermediate);
    if (st.ok()) st = int_field(c, "shared_expert_intermediate_size", 0, m.shared_intermediate);
    if (st.ok() && (m.top_k < 1 || m.top_k > m.experts))
        st = invalid("num_experts_per_tok", "must be in 1..=" + std::to_string(m.experts));
    if (!st.ok()) return report(st);
    const json::Value *nt = c.get("norm_topk_prob");
    m.norm_topk_prob = (nt && nt->kind == json::Value::Bool) ? (int)nt->b : 1;
    if (eps) {
        const json::Value *e = c.get("rms_norm_eps");
        *eps = (e && e->kind == json::Value::Num) ? (float)e->num : 1e-6f;
    }
    *cfg = m;
    return report(Ok());
}

int mrun_weights_tensor_info(const mrun_weights *w, const char *name, char *dtype, int64_t *shape,
                             int32_t *ndim) {
    if (!w || !name) return report(Err(MRUN_ERR_INVALID, "weights: null argument"));
    auto it = w->tensors.find(name);
    if (it == w->tensors.end()) return report(invalid("weights", std::string("missing tensor ") + name));
    const Tensor &t = it->second;
    if (dtype) {
        std::strncpy(dtype, t.dtype.c_str(), 7);
        dtype[7] = '\0';
    }
    if (ndim) *ndim = (int32_t)t.shape.size();
    if (shape)
        for (size_t i = 0; i < t.shape.size() && i < 8; ++i) shape[i] = t.shape[i];
    return report(Ok());
}

int32_t mrun_weights_remaining(const mrun_weights *w) { return w ? (int32_t)w->tensors.size() : 0; }

int mrun_weights_resolve_quant(const mrun_weights *w, const char *path, int32_t in_dims,
                               int32_t *group_size, int32_t *bits) {
    if (!w || !path) return report(Err(MRUN_ERR_INVALID, "weights: null argument"));
    const std::string p(path);
    auto wt = w->tensors.find(p + ".weight"), sc = w->tensors.find(p + ".scales");
    if (wt == w->tensors.end()) return report(invalid("weights", "missing tensor " + p + ".weight"));
    if (sc == w->tensors.end()) return report(invalid("quantization", p + " is not quantized"));
    QParams q{0, 0};
    Status st = resolve(w->quant, p, wt->second, sc->second, in_dims, q);
    if (st.ok()) {
        if (group_size) *group_size = q.group_size;
        if (bits) *bits = q.bits;
    }
    return report(st);
}

int mrun_weights_load_moe(mrun_weights *w, const char *prefix, const mrun_moe_config *cfg,
                          mrun_sparse_moe *out) {
    if (!w || !prefix || !cfg || !out) return report(Err(MRUN_ERR_INVALID, "weights: null argument"));
    const std::string p(prefix);
    const int D = cfg->hidden, E = cfg->experts, I = cfg->intermediate, S = cfg->shared_intermediate;
    Status st = stack_experts(*w, p, E);
    if (st.ok()) st = split_gate_up(*w, p);
    HostLinear gate, sw[3], sh[3], sh_gate;
    const char *sw_names[3] = {"gate_proj", "up_proj", "down_proj"};
    // SparseMoe::load order (moe.rs:131-146): the shared expert, then the router and the experts
    if (st.ok() && S > 0) {
        for (int i = 0; st.ok() && i < 3; ++i)
            st = linear_load(*w, p + ".shared_expert." + sw_names[i], i == 2 ? S : D, sh[i]);
        if (st.ok()) st = linear_load(*w, p + ".shared_expert_gate", D, sh_gate);
    }
    if (st.ok()) st = linear_load(*w, p + ".gate", D, gate);
    for (int i = 0; st.ok() && i < 3; ++i)
        st = linear_load(*w, p + ".switch_mlp." + sw_names[i], i == 2 ? I : D, sw[i]);
    // every check before the first device allocation (experts first: their layout decides
    // whether this build runs the checkpoint at all)
    for (int i = 0; st.ok() && i < 3; ++i)
        st = check_linear(sw[i], E, i == 2 ? D : I, i == 2 ? I : D, true, false);
    if (st.ok()) st = check_linear(gate, 1, E, D, false, true);
    if (st.ok() && S > 0) {
        for (int i = 0; st.ok() && i < 3; ++i)
            st = check_linear(sh[i], 1, i == 2 ? D : S, i == 2 ? S : D, false, false);
        if (st.ok()) st = check_linear(sh_gate, 1, 1, D, false, true);
    }
    mrun_sparse_moe m{};
    m.cfg = *cfg;
    if (st.ok()) st = to_device(*w, gate, 1, E, D, &m.gate, nullptr);
    mrun_quantized *swq[3] = {&m.switch_gate_proj, &m.switch_up_proj, &m.switch_down_proj};
    for (int i = 0; st.ok() && i < 3; ++i)
        st = to_device(*w, sw[i], E, i == 2 ? D : I, i == 2 ? I : D, nullptr, swq[i]);
    if (st.ok() && S > 0) {
        mrun_linear *shl[3] = {&m.shared_gate_proj, &m.shared_up_proj, &m.shared_down_proj};
        for (int i = 0; st.ok() && i < 3; ++i)
            st = to_device(*w, sh[i], 1, i == 2 ? D : S, i == 2 ? S : D, shl[i], nullptr);
        if (st.ok()) st = to_device(*w, sh_gate, 1, 1, D, &m.shared_expert_gate, nullptr);
    }
    if (!st.ok()) return report(st);
    const int rc = mrun_moe_check(&m);
    if (rc == MRUN_OK) *out = m;
    return rc;
}

int mrun_weights_load_bf16(mrun_weights *w, const char *name, int64_t n, const mrun_bf16 **out) {
    if (!w || !name || !out) return report(Err(MRUN_ERR_INVALID, "weights: null argument"));
    Tensor t;
    Status st = take(*w, name, t);
    if (st.ok() && t.dtype != "BF16")
        st = Err(MRUN_ERR_UNSUPPORTED, std::string(name) + ": " + t.dtype + " (bf16 only)");
    if (st.ok() && (int64_t)(t.bytes() / 2) != n)
        st = invalid("weights", std::string(name) + ": " + std::to_string(t.bytes() / 2) +
                                    " elements, expected " + std::to_string(n));
    const void *p = nullptr;
    if (st.ok()) st = upload(*w, t, &p);
    if (st.ok()) *out = (const mrun_bf16 *)p;
    return report(st);
}

}  // extern "C"
