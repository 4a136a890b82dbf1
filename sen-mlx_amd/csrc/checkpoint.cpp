// checkpoint.cpp -- reading MLX's on-disk quantized checkpoints: which modules
// are quantized, with which bits and group size, and where their packed
// weights, scales and biases live in the safetensors shards.
//
// The format and the rules follow the reference's loaders:
//   - shards: model.safetensors, or model.safetensors.index.json's weight_map
//     naming several (src/engine/mlx_native.rs:3603-3623);
//   - a module is stored quantized iff a "<path>.scales" tensor exists; its
//     bits / group size come from config.json's "quantization" (or
//     "quantization_config") object, a per-module object keyed by the path
//     overriding the top-level default (src/engine/mlx_lm/models/gemma4.rs:
//     1755-1834, src/engine/mlx_lm/models/qwen3_5.rs:722-760);
//   - the codes are "<path>.weight", which mlx-rs's parameter tree names
//     "<path>.inner.weight" (src/engine/mlx_native.rs:3684-3703); both spellings
//     are accepted, as is "<path>.bias" / "<path>.inner.bias".
// Unlike the reference, the bits and group size are checked against the
// tensor shapes (codes [.., N, K*bits/32], scales [.., N, K/g] must imply the
// same K): a mismatch is a load error here instead of silently misread words
// (the risk noted at src/engine/mlx_lm/models/gemma4.rs:160-166).  Shapes
// only fix the product bits * group_size, so a misdescription that keeps it
// (8-bit g32 read as 4-bit g64) still passes.
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/miqmm.h"
#include "../../include/miqmm_checkpoint.h"

namespace {

thread_local std::string g_ckpt_error;

int ckpt_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int ckpt_fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_ckpt_error = buf;
    return code;
}

// ---------------------------------------------------------------- JSON
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;  // insertion order kept

    const Json* get(const std::string& k) const {
        if (kind != Object) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    bool is_int() const { return kind == Number && num == (double)(long long)num; }
};

class JsonParser {
   public:
    JsonParser(const char* s, size_t n) : p_(s), end_(s + n) {}
    bool parse(Json& out, std::string& err) {
        if (!value(out, 0)) {
            err = err_.empty() ? "malformed JSON" : err_;
            return false;
        }
        ws();
        if (p_ != end_) {
            err = "trailing characters after JSON value";
            return false;
        }
        return true;
    }

   private:
    const char* p_;
    const char* end_;
    std::string err_;

    void ws() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if ((size_t)(end_ - p_) < n || memcmp(p_, w, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(std::string& s, unsigned cp) {
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(unsigned& v) {
        if (end_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; ++i) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            const char c = *p_++;
            if ((unsigned char)c < 0x20) return false;
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) return false;
            const char e = *p_++;
            switch (e) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    unsigned cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
                        unsigned lo;
                        if (!lit("\\u") || !hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(s, cp);
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool number(double& v) {
        const char* s = p_;
        if (p_ < end_ && *p_ == '-') ++p_;
        if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                             *p_ == '-'))
            ++p_;
        const std::string t(s, p_);
        char* e = nullptr;
        v = strtod(t.c_str(), &e);
        return e && *e == '\0';
    }
    bool value(Json& v, int depth) {
        if (depth > 64) {
            err_ = "JSON nested too deeply";
            return false;
        }
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Json::Object;
            ws();
            if (p_ < end_ && *p_ == '}') {
                ++p_;
                return true;
            }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                Json item;
                if (!value(item, depth + 1)) return false;
                v.obj.emplace_back(std::move(k), std::move(item));
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
            v.kind = Json::Array;
            ws();
            if (p_ < end_ && *p_ == ']') {
                ++p_;
                return true;
            }
            for (;;) {
                Json item;
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
            v.kind = Json::String;
            return string(v.str);
        }
        if (lit("true")) {
            v.kind = Json::Bool;
            v.b = true;
            return true;
        }
        if (lit("false")) {
            v.kind = Json::Bool;
            return true;
        }
        if (lit("null")) return true;
        v.kind = Json::Number;
        return number(v.num);
    }
};

bool read_file(const std::string& path, std::string& out, std::string& err) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) {
        err = "cannot open " + path + ": " + strerror(errno);
        return false;
    }
    out.clear();
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    fclose(f);
    return true;
}

// ---------------------------------------------------------------- safetensors
struct Tensor {
    std::string name, dtype, file;
    std::vector<int64_t> shape;
    int64_t offset = 0, nbytes = 0;  // absolute byte offset in `file`
};

int64_t dtype_size(const std::string& d) {
    if (d == "U8" || d == "I8" || d == "BOOL" || d == "F8_E4M3" || d == "F8_E5M2") return 1;
    if (d == "U16" || d == "I16" || d == "F16" || d == "BF16") return 2;
    if (d == "U32" || d == "I32" || d == "F32") return 4;
    if (d == "U64" || d == "I64" || d == "F64") return 8;
    return 0;
}

// header of one shard: u64 little-endian length, then a JSON object mapping
// tensor names to {dtype, shape, data_offsets: [begin, end)} relative to the
// byte after the header
int parse_shard(const std::string& path, std::vector<Tensor>& out) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return ckpt_fail(MIQMM_EINVAL, "cannot open shard %s: %s", path.c_str(), strerror(errno));
    unsigned char lenb[8];
    if (fread(lenb, 1, 8, f) != 8) {
        fclose(f);
        return ckpt_fail(MIQMM_EINVAL, "%s: shorter than a safetensors header", path.c_str());
    }
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | lenb[i];
    fseek(f, 0, SEEK_END);
    const long fsize = ftell(f);
    if (hlen == 0 || hlen > (uint64_t)100 << 20 || (long)(8 + hlen) > fsize) {
        fclose(f);
        return ckpt_fail(MIQMM_EINVAL, "%s: bad safetensors header length %llu", path.c_str(),
                         (unsigned long long)hlen);
    }
    std::string hdr(hlen, '\0');
    fseek(f, 8, SEEK_SET);
    const size_t got = fread(&hdr[0], 1, hlen, f);
    fclose(f);
    if (got != hlen) return ckpt_fail(MIQMM_EINVAL, "%s: truncated header", path.c_str());
    Json j;
    std::string err;
    if (!JsonParser(hdr.data(), hdr.size()).parse(j, err) || j.kind != Json::Object)
        return ckpt_fail(MIQMM_EINVAL, "%s: header is not a JSON object (%s)", path.c_str(), err.c_str());
    const int64_t data0 = 8 + (int64_t)hlen;
    for (const auto& kv : j.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& t = kv.second;
        const Json* dt = t.get("dtype");
        const Json* sh = t.get("shape");
        const Json* off = t.get("data_offsets");
        if (!dt || dt->kind != Json::String || !sh || sh->kind != Json::Array || !off || off->kind != Json::Array ||
            off->arr.size() != 2 || !off->arr[0].is_int() || !off->arr[1].is_int())
            return ckpt_fail(MIQMM_EINVAL, "%s: tensor %s has a malformed entry", path.c_str(), kv.first.c_str());
        Tensor x;
        x.name = kv.first;
        x.dtype = dt->str;
        x.file = path;
        int64_t count = 1;
        for (const Json& d : sh->arr) {
            if (!d.is_int() || d.num < 0)
                return ckpt_fail(MIQMM_EINVAL, "%s: tensor %s has a bad shape", path.c_str(), kv.first.c_str());
            x.shape.push_back((int64_t)d.num);
            // a product past INT64_MAX / 8 would wrap and could match the byte range by accident
            if (__builtin_mul_overflow(count, (int64_t)d.num, &count) || count > INT64_MAX / 8)
                return ckpt_fail(MIQMM_EINVAL, "%s: tensor %s has a shape too large", path.c_str(), kv.first.c_str());
        }
        const int64_t b = (int64_t)off->arr[0].num, e = (int64_t)off->arr[1].num;
        const int64_t es = dtype_size(x.dtype);
        if (es == 0)
            return ckpt_fail(MIQMM_EINVAL, "%s: tensor %s has unknown dtype %s", path.c_str(), kv.first.c_str(),
                             x.dtype.c_str());
        if (b < 0 || e < b || data0 + e > fsize || e - b != count * es)
            return ckpt_fail(MIQMM_EINVAL, "%s: tensor %s has data offsets [%lld, %lld) that do not fit its shape",
                             path.c_str(), kv.first.c_str(), (long long)b, (long long)e);
        x.offset = data0 + b;
        x.nbytes = e - b;
        out.push_back(std::move(x));
    }
    return MIQMM_OK;
}

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

}  // namespace

// ---------------------------------------------------------------- the checkpoint
struct miqmm_checkpoint {
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> by_name;
    struct Module {
        std::string path, weight, scales, biases, bias;
        int bits = 0, group_size = 0, sb_dtype = 0;
        int64_t experts = 0, rows = 0, cols = 0;
    };
    std::vector<Module> modules;
};

namespace {

const Tensor* find(const miqmm_checkpoint* c, const std::string& n) {
    auto it = c->by_name.find(n);
    return it == c->by_name.end() ? nullptr : &c->tensors[it->second];
}

int build_plan(miqmm_checkpoint* c, const Json& cfg) {
    const Json* q = cfg.get("quantization");
    if (!q) q = cfg.get("quantization_config");
    int def_g = 64, def_b = 4;
    std::map<std::string, std::pair<int, int>> overrides;  // path -> (group_size, bits)
    std::string def_mode = "affine";
    if (q && q->kind == Json::Object) {
        if (const Json* g = q->get("group_size"); g && g->is_int()) def_g = (int)g->num;
        if (const Json* b = q->get("bits"); b && b->is_int()) def_b = (int)b->num;
        if (const Json* m = q->get("mode"); m && m->kind == Json::String) def_mode = m->str;
        for (const auto& kv : q->obj) {
            if (kv.first == "group_size" || kv.first == "bits" || kv.first == "mode") continue;
            if (kv.second.kind != Json::Object) continue;  // e.g. "path": false -- left to the default rule
            int g = def_g, b = def_b;
            if (const Json* x = kv.second.get("group_size"); x && x->is_int()) g = (int)x->num;
            if (const Json* x = kv.second.get("bits"); x && x->is_int()) b = (int)x->num;
            if (const Json* m = kv.second.get("mode"); m && m->kind == Json::String && m->str != "affine")
                return ckpt_fail(MIQMM_ENOTSUP, "module %s uses quantization mode '%s'; only affine is provided",
                                 kv.first.c_str(), m->str.c_str());
            overrides[kv.first] = {g, b};
        }
    }
    if (def_mode != "affine")
        return ckpt_fail(MIQMM_ENOTSUP, "quantization mode '%s'; only affine is provided", def_mode.c_str());

    for (const Tensor& t : c->tensors) {
        if (!ends_with(t.name, ".scales")) continue;
        miqmm_checkpoint::Module m;
        m.path = t.name.substr(0, t.name.size() - 7);
        for (const char* suf : {".weight", ".inner.weight"})
            if (find(c, m.path + suf)) {
                m.weight = m.path + suf;
                break;
            }
        for (const char* suf : {".bias", ".inner.bias"})
            if (find(c, m.path + suf)) {
                m.bias = m.path + suf;
                break;
            }
        m.scales = t.name;
        m.biases = m.path + ".biases";
        const Tensor* w = m.weight.empty() ? nullptr : find(c, m.weight);
        const Tensor* b = find(c, m.biases);
        if (!w) return ckpt_fail(MIQMM_EINVAL, "module %s has scales but no .weight codes", m.path.c_str());
        if (!b) return ckpt_fail(MIQMM_EINVAL, "module %s has scales but no .biases", m.path.c_str());
        auto ov = overrides.find(m.path);
        m.group_size = ov != overrides.end() ? ov->second.first : def_g;
        m.bits = ov != overrides.end() ? ov->second.second : def_b;
        if (w->dtype != "U32")
            return ckpt_fail(MIQMM_EINVAL, "module %s: codes are %s, expected U32 packed words", m.path.c_str(),
                             w->dtype.c_str());
        if (t.dtype != b->dtype || (t.dtype != "BF16" && t.dtype != "F16"))
            return ckpt_fail(MIQMM_ENOTSUP, "module %s: scales %s / biases %s (bf16 or fp16 pairs are provided)",
                             m.path.c_str(), t.dtype.c_str(), b->dtype.c_str());
        m.sb_dtype = t.dtype == "F16" ? MIQMM_DT_F16 : MIQMM_DT_BF16;
        if (w->shape.size() != t.shape.size() || t.shape != b->shape || (w->shape.size() != 2 && w->shape.size() != 3))
            return ckpt_fail(MIQMM_EINVAL, "module %s: codes, scales and biases must be 2-D (or 3-D stacked experts) "
                                           "with equal scales/biases shapes", m.path.c_str());
        const size_t nd = w->shape.size();
        for (size_t i = 0; i + 1 < nd; ++i)
            if (w->shape[i] != t.shape[i])
                return ckpt_fail(MIQMM_EINVAL, "module %s: codes and scales disagree on dim %zu", m.path.c_str(), i);
        if (m.bits <= 0 || 32 % m.bits != 0 || m.group_size <= 0)
            return ckpt_fail(MIQMM_EINVAL, "module %s: bits=%d group_size=%d", m.path.c_str(), m.bits, m.group_size);
        const int64_t k_codes = w->shape[nd - 1] * (32 / m.bits);
        const int64_t k_scales = t.shape[nd - 1] * m.group_size;
        if (k_codes != k_scales)
            return ckpt_fail(MIQMM_EINVAL,
                             "module %s: bits=%d group_size=%d do not fit the tensors (codes give K=%lld, "
                             "scales K=%lld): the quantization section does not describe this checkpoint",
                             m.path.c_str(), m.bits, m.group_size, (long long)k_codes, (long long)k_scales);
        m.experts = nd == 3 ? w->shape[0] : 0;
        m.rows = w->shape[nd - 2];
        m.cols = k_codes;
        if (!m.bias.empty()) {
            const Tensor* bb = find(c, m.bias);
            if (bb->shape.size() != nd - 1 || bb->shape.back() != m.rows)
                return ckpt_fail(MIQMM_EINVAL, "module %s: bias shape does not match %lld rows", m.path.c_str(),
                                 (long long)m.rows);
        }
        c->modules.push_back(std::move(m));
    }
    return MIQMM_OK;
}

}  // namespace

extern "C" {

int miqmm_checkpoint_open(const char* model_dir, miqmm_checkpoint** out) {
    if (!model_dir || !out) return ckpt_fail(MIQMM_EINVAL, "null argument");
    *out = nullptr;
    const std::string dir(model_dir);
    std::string text, err;
    Json cfg;
    if (read_file(dir + "/config.json", text, err)) {
        if (!JsonParser(text.data(), text.size()).parse(cfg, err) || cfg.kind != Json::Object)
            return ckpt_fail(MIQMM_EINVAL, "config.json: %s", err.empty() ? "not a JSON object" : err.c_str());
    } else {
        return ckpt_fail(MIQMM_EINVAL, "%s", err.c_str());
    }
    std::vector<std::string> shards;
    if (read_file(dir + "/model.safetensors.index.json", text, err)) {
        Json idx;
        if (!JsonParser(text.data(), text.size()).parse(idx, err) || !idx.get("weight_map") ||
            idx.get("weight_map")->kind != Json::Object)
            return ckpt_fail(MIQMM_EINVAL, "model.safetensors.index.json has no weight_map object");
        std::set<std::string> files;
        for (const auto& kv : idx.get("weight_map")->obj)
            if (kv.second.kind == Json::String) files.insert(kv.second.str);
        for (const auto& f : files) shards.push_back(dir + "/" + f);
    } else {
        shards.push_back(dir + "/model.safetensors");
    }
    std::unique_ptr<miqmm_checkpoint> c(new miqmm_checkpoint);
    for (const auto& s : shards) {
        const int st = parse_shard(s, c->tensors);
        if (st != MIQMM_OK) return st;
    }
    for (size_t i = 0; i < c->tensors.size(); ++i) {
        if (!c->by_name.emplace(c->tensors[i].name, i).second)
            return ckpt_fail(MIQMM_EINVAL, "tensor %s appears in two shards", c->tensors[i].name.c_str());
    }
    const int st = build_plan(c.get(), cfg);
    if (st != MIQMM_OK) return st;
    *out = c.release();
    g_ckpt_error.clear();
    return MIQMM_OK;
}

void miqmm_checkpoint_close(miqmm_checkpoint* c) { delete c; }

int64_t miqmm_checkpoint_num_modules(const miqmm_checkpoint* c) { return c ? (int64_t)c->modules.size() : 0; }

int64_t miqmm_checkpoint_num_tensors(const miqmm_checkpoint* c) { return c ? (int64_t)c->tensors.size() : 0; }

int miqmm_checkpoint_module(const miqmm_checkpoint* c, int64_t i, miqmm_qmodule* out) {
    if (!c || !out) return ckpt_fail(MIQMM_EINVAL, "null argument");
    if (i < 0 || i >= (int64_t)c->modules.size())
        return ckpt_fail(MIQMM_EINVAL, "module index %lld out of range", (long long)i);
    const auto& m = c->modules[(size_t)i];
    out->path = m.path.c_str();
    out->weight = m.weight.c_str();
    out->scales = m.scales.c_str();
    out->biases = m.biases.c_str();
    out->bias = m.bias.empty() ? nullptr : m.bias.c_str();
    out->bits = m.bits;
    out->group_size = m.group_size;
    out->sb_dtype = m.sb_dtype;
    out->experts = m.experts;
    out->rows = m.rows;
    out->cols = m.cols;
    return MIQMM_OK;
}

int miqmm_checkpoint_tensor(const miqmm_checkpoint* c, const char* name, int64_t index, miqmm_tensor_info* out) {
    if (!c || !out) return ckpt_fail(MIQMM_EINVAL, "null argument");
    const Tensor* t = nullptr;
    if (name) {
        t = find(c, name);
        if (!t) return ckpt_fail(MIQMM_EINVAL, "no tensor named %s", name);
    } else {
        if (index < 0 || index >= (int64_t)c->tensors.size())
            return ckpt_fail(MIQMM_EINVAL, "tensor index %lld out of range", (long long)index);
        t = &c->tensors[(size_t)index];
    }
    if (t->shape.size() > 8) return ckpt_fail(MIQMM_ENOTSUP, "tensor %s has more than 8 dims", t->name.c_str());
    out->name = t->name.c_str();
    out->dtype = t->dtype.c_str();
    out->file = t->file.c_str();
    out->ndim = (int)t->shape.size();
    for (int i = 0; i < 8; ++i) out->shape[i] = i < out->ndim ? t->shape[(size_t)i] : 0;
    out->offset = t->offset;
    out->nbytes = t->nbytes;
    return MIQMM_OK;
}

int miqmm_checkpoint_read(const miqmm_checkpoint* c, const char* name, void* dst, int64_t bytes) {
    if (!c || !name || !dst) return ckpt_fail(MIQMM_EINVAL, "null argument");
    const Tensor* t = find(c, name);
    if (!t) return ckpt_fail(MIQMM_EINVAL, "no tensor named %s", name);
    if (bytes != t->nbytes)
        return ckpt_fail(MIQMM_EINVAL, "tensor %s holds %lld bytes, buffer has %lld", name, (long long)t->nbytes,
                         (long long)bytes);
    FILE* f = fopen(t->file.c_str(), "rb");
    if (!f) return ckpt_fail(MIQMM_EINVAL, "cannot open %s: %s", t->file.c_str(), strerror(errno));
    const bool ok = fseek(f, (long)t->offset, SEEK_SET) == 0 && fread(dst, 1, (size_t)bytes, f) == (size_t)bytes;
    fclose(f);
    if (!ok) return ckpt_fail(MIQMM_EINVAL, "short read of %s from %s", name, t->file.c_str());
    return MIQMM_OK;
}

const char* miqmm_checkpoint_last_error(void) { return g_ckpt_error.c_str(); }

}  // extern "C"
