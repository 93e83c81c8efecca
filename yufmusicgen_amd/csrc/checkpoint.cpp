// .yuf checkpoint loader (host side of libyufhip.so).
//
// Container (vulkan/scripts/export_checkpoint.py:32-146; checks of
// vulkan/src/checkpoint.rs:90-149):
//   b"YUFM" | u32 LE version (1 or 2) | u64 LE header_len | UTF-8 JSON | payload
// Version 1: an f32 LE payload whose size must equal 4 * sum(tensors[].count).
// Version 2 (this build's extension for bf16 weights): tensor entries carry a
// "dtype" ("f32" | "bf16") and a byte "offset" into the payload (a multiple of
// the element size), the header a "payload_bytes" that the file size must
// match; bf16 tensors are widened to f32 on load (exact).  The model
// config is validated like ModelConfig::validate (checkpoint.rs:32-47) except
// that the low-rank width is read from the w1 tensor's shape instead of the
// Rust rounding formula, which disagrees with Python's at d_model = 1024.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/yuf_engine.h"
#include "checkpoint.h"

namespace yuf {

int fail(int status, const std::string &msg);

// ------------------------------------------------------------ minimal JSON
namespace json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Value> arr;
    std::map<std::string, Value> obj;

    const Value *get(const std::string &key) const {
        if (kind != Object) return nullptr;
        auto it = obj.find(key);
        return it == obj.end() ? nullptr : &it->second;
    }
};

class Parser {
  public:
    Parser(const char *p, const char *end) : p_(p), end_(end) {}
    bool parse(Value &out, std::string &err) {
        if (!value(out, 0)) {
            err = err_.empty() ? "invalid JSON" : err_;
            return false;
        }
        ws();
        if (p_ != end_) {
            err = "trailing characters after JSON header";
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
        size_t n = std::strlen(s);
        if ((size_t)(end_ - p_) < n || std::strncmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    static void utf8(std::string &out, unsigned cp) {
        if (cp < 0x80) out += (char)cp;
        else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) {
            out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 0x3F)); out += (char)(0x80 | (cp & 0x3F));
        } else {
            out += (char)(0xF0 | (cp >> 18)); out += (char)(0x80 | ((cp >> 12) & 0x3F));
            out += (char)(0x80 | ((cp >> 6) & 0x3F)); out += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(unsigned &cp) {
        if (end_ - p_ < 4) return false;
        cp = 0;
        for (int i = 0; i < 4; ++i) {
            char c = *p_++;
            cp <<= 4;
            if (c >= '0' && c <= '9') cp |= c - '0';
            else if (c >= 'a' && c <= 'f') cp |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') cp |= c - 'A' + 10;
            else return false;
        }
        return true;
    }
    bool string(std::string &out) {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if (c != '\\') { out += c; continue; }
            if (p_ >= end_) return false;
            char e = *p_++;
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    unsigned cp;
                    if (!hex4(cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                        p_ += 2;
                        unsigned lo;
                        if (!hex4(lo)) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(out, cp);
                    break;
                }
                default: return false;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool value(Value &v, int depth) {
        if (depth > 64) { err_ = "JSON nested too deeply"; return false; }
        ws();
        if (p_ >= end_) return false;
        char c = *p_;
        if (c == '{') {
            ++p_;
            v.kind = Value::Object;
            ws();
            if (p_ < end_ && *p_ == '}') { ++p_; return true; }
            while (true) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                Value child;
                if (!value(child, depth + 1)) return false;
                v.obj[key] = std::move(child);
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') { ++p_; return true; }
                return false;
            }
        }
        if (c == '[') {
            ++p_;
            v.kind = Value::Array;
            ws();
            if (p_ < end_ && *p_ == ']') { ++p_; return true; }
            while (true) {
                Value child;
                if (!value(child, depth + 1)) return false;
                v.arr.push_back(std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') { ++p_; return true; }
                return false;
            }
        }
        if (c == '"') { v.kind = Value::String; return string(v.str); }
        if (lit("true")) { v.kind = Value::Bool; v.b = true; return true; }
        if (lit("false")) { v.kind = Value::Bool; v.b = false; return true; }
        if (lit("null")) { v.kind = Value::Null; return true; }
        const char *start = p_;
        if (p_ < end_ && (*p_ == '-' || *p_ == '+')) ++p_;
        while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '-' ||
                             *p_ == '+'))
            ++p_;
        if (p_ == start) return false;
        std::string num(start, p_);
        char *endp = nullptr;
        v.num = std::strtod(num.c_str(), &endp);
        v.kind = Value::Number;
        return endp && *endp == '\0';
    }
};

}  // namespace json

namespace {

bool get_int(const json::Value *obj, const char *key, long long &out) {
    const json::Value *v = obj ? obj->get(key) : nullptr;
    if (!v || v->kind != json::Value::Number || v->num != std::floor(v->num)) return false;
    out = (long long)v->num;
    return true;
}

}  // namespace

int load_checkpoint(const char *path, Checkpoint &ck) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail(YUF_ERR_IO, std::string("cannot open checkpoint ") + path);
    f.seekg(0, std::ios::end);
    const long long file_len = (long long)f.tellg();
    f.seekg(0);
    char magic[4];
    if (!f.read(magic, 4)) return fail(YUF_ERR_FORMAT, "cannot read checkpoint magic");
    if (std::memcmp(magic, "YUFM", 4) != 0)
        return fail(YUF_ERR_FORMAT, std::string(path) + " is not a .yuf checkpoint (bad magic)");
    uint32_t version = 0;
    uint64_t header_len = 0;
    unsigned char b4[4], b8[8];
    if (!f.read((char *)b4, 4)) return fail(YUF_ERR_FORMAT, "truncated header");
    version = b4[0] | (b4[1] << 8) | (b4[2] << 16) | ((uint32_t)b4[3] << 24);
    if (version != 1 && version != 2) return fail(YUF_ERR_FORMAT, "unsupported .yuf version " + std::to_string(version));
    if (!f.read((char *)b8, 8)) return fail(YUF_ERR_FORMAT, "truncated header");
    for (int i = 7; i >= 0; --i) header_len = (header_len << 8) | b8[i];
    if (header_len > (uint64_t)file_len - 16) return fail(YUF_ERR_FORMAT, "header length exceeds file size");
    std::string header(header_len, '\0');
    if (!f.read(&header[0], (std::streamsize)header_len)) return fail(YUF_ERR_FORMAT, "truncated JSON header");

    json::Value root;
    std::string err;
    json::Parser parser(header.data(), header.data() + header.size());
    if (!parser.parse(root, err)) return fail(YUF_ERR_FORMAT, "invalid .yuf header JSON: " + err);
    ck.version = version;
    const json::Value *fmt = root.get("format");
    if (!fmt || fmt->kind != json::Value::String || fmt->str != "yufmusicgen-checkpoint")
        return fail(YUF_ERR_FORMAT, "unexpected .yuf payload format");
    long long hdr_version = 0;
    if (!get_int(&root, "version", hdr_version) || hdr_version < 0)
        return fail(YUF_ERR_FORMAT, "header has no integer version field");
    const json::Value *mc = root.get("model_config");
    long long vocab, d, layers, heads, hs, rosa;
    if (!get_int(mc, "vocab_size", vocab) || !get_int(mc, "d_model", d) || !get_int(mc, "n_layers", layers) ||
        !get_int(mc, "n_heads", heads) || !get_int(mc, "head_size", hs) || !get_int(mc, "rosa_size", rosa))
        return fail(YUF_ERR_FORMAT, "model_config is missing integer fields");
    ModelShape &s = ck.shape;
    s.vocab = (int)vocab; s.d = (int)d; s.layers = (int)layers; s.heads = (int)heads; s.head_size = (int)hs;
    s.rosa = (int)rosa;
    // Required fields and checks of the Rust loader: ModelConfig and MidiHeader
    // are deserialized without defaults (vulkan/src/checkpoint.rs:14-24,
    // :58-80), then ModelConfig::validate (:33-47) runs.
    const json::Value *tie = mc->get("tie_embeddings");
    if (!tie || tie->kind != json::Value::Bool) return fail(YUF_ERR_FORMAT, "model_config.tie_embeddings must be a bool");
    s.tie = tie->b;
    const json::Value *drop = mc->get("dropout");
    if (!drop || drop->kind != json::Value::Number) return fail(YUF_ERR_FORMAT, "model_config.dropout must be a number");
    s.dropout = (float)drop->num;
    if (s.d != s.heads * s.head_size)
        return fail(YUF_ERR_FORMAT, "d_model " + std::to_string(s.d) + " must equal n_heads * head_size");
    if (s.d < 32 || s.layers < 1) return fail(YUF_ERR_FORMAT, "model is too small to be useful");
    if (s.rosa < 1) return fail(YUF_ERR_FORMAT, "rosa_size must be positive");
    if (s.vocab < s.d)
        return fail(YUF_ERR_FORMAT, "vocab_size " + std::to_string(s.vocab) + " looks wrong for d_model " +
                                        std::to_string(s.d));
    const json::Value *midi = root.get("midi");
    long long mo = 0, mv = 0;
    const json::Value *tok = midi ? midi->get("tokenization") : nullptr;
    const json::Value *mvocab = midi ? midi->get("vocab") : nullptr;
    if (!midi || midi->kind != json::Value::Object || !tok || tok->kind != json::Value::String ||
        !get_int(midi, "midi_offset", mo) || !get_int(midi, "midi_vocab_size", mv) || mo < 0 || mv < 0 || !mvocab ||
        mvocab->kind != json::Value::Array)
        return fail(YUF_ERR_FORMAT, "midi header needs tokenization, midi_offset, midi_vocab_size and vocab");
    s.midi_offset = (int)mo;
    s.midi_vocab = (int)mv;

    const json::Value *tensors = root.get("tensors");
    if (!tensors || tensors->kind != json::Value::Array) return fail(YUF_ERR_FORMAT, "header has no tensors array");
    long long total = 0;
    std::vector<std::pair<std::string, long long>> byte_offsets;  // version 2: payload byte offset per tensor
    for (const json::Value &t : tensors->arr) {
        TensorInfo info;
        const json::Value *name = t.get("name");
        const json::Value *shape = t.get("shape");
        long long off, cnt;
        if (!name || name->kind != json::Value::String || !shape || shape->kind != json::Value::Array ||
            !get_int(&t, "offset", off) || !get_int(&t, "count", cnt) || off < 0 || cnt < 0)
            return fail(YUF_ERR_FORMAT, "malformed tensor entry in header");
        if (version == 2) {
            const json::Value *dt = t.get("dtype");
            if (!dt || dt->kind != json::Value::String || (dt->str != "f32" && dt->str != "bf16"))
                return fail(YUF_ERR_FORMAT, "tensor " + name->str + ": dtype must be \"f32\" or \"bf16\"");
            info.bf16 = dt->str == "bf16";
            if (off % (info.bf16 ? 2 : 4) != 0)
                return fail(YUF_ERR_FORMAT, "tensor " + name->str + ": offset is not a multiple of its element size");
            byte_offsets.emplace_back(name->str, off);
            off = total;  // position in the widened f32 copy
        }
        info.offset = off;
        info.count = cnt;
        long long prod = 1;
        for (const json::Value &dim : shape->arr) {
            if (dim.kind != json::Value::Number || dim.num < 0) return fail(YUF_ERR_FORMAT, "bad tensor shape");
            info.dims.push_back((long long)dim.num);
            prod *= (long long)dim.num;
        }
        if (prod != cnt) return fail(YUF_ERR_FORMAT, "tensor " + name->str + ": shape does not match count");
        total += cnt;
        ck.tensors[name->str] = info;
    }
    const long long data_start = 16 + (long long)header_len;
    if (version == 1) {
        const long long expected = data_start + total * 4;
        if (file_len != expected)
            return fail(YUF_ERR_FORMAT, "checkpoint size mismatch: file has " + std::to_string(file_len) +
                                            " bytes, header expects " + std::to_string(expected));
        for (const auto &kv : ck.tensors)
            if (kv.second.offset + kv.second.count > total)
                return fail(YUF_ERR_FORMAT, "tensor " + kv.first + " lies outside the payload");
        ck.data.resize((size_t)total);
        if (total > 0 && !f.read(reinterpret_cast<char *>(ck.data.data()), (std::streamsize)(total * 4)))
            return fail(YUF_ERR_IO, "cannot read tensor payload");
    } else {
        long long payload = -1;
        if (!get_int(&root, "payload_bytes", payload) || payload < 0)
            return fail(YUF_ERR_FORMAT, "version 2 header needs payload_bytes");
        if (file_len != data_start + payload)
            return fail(YUF_ERR_FORMAT, "checkpoint size mismatch: file has " + std::to_string(file_len) +
                                            " bytes, header expects " + std::to_string(data_start + payload));
        std::vector<unsigned char> raw((size_t)payload);
        if (payload > 0 && !f.read(reinterpret_cast<char *>(raw.data()), (std::streamsize)payload))
            return fail(YUF_ERR_IO, "cannot read tensor payload");
        ck.data.resize((size_t)total);
        for (const auto &no : byte_offsets) {
            const TensorInfo &info = ck.tensors[no.first];
            const long long width = info.bf16 ? 2 : 4;
            if (no.second + width * info.count > payload)
                return fail(YUF_ERR_FORMAT, "tensor " + no.first + " lies outside the payload");
            float *dst = ck.data.data() + info.offset;
            const unsigned char *src = raw.data() + no.second;
            for (long long i = 0; i < info.count; ++i) {
                uint32_t u;
                if (info.bf16) {
                    u = ((uint32_t)src[2 * i] | ((uint32_t)src[2 * i + 1] << 8)) << 16;
                } else {
                    u = (uint32_t)src[4 * i] | ((uint32_t)src[4 * i + 1] << 8) | ((uint32_t)src[4 * i + 2] << 16) |
                        ((uint32_t)src[4 * i + 3] << 24);
                }
                std::memcpy(dst + i, &u, 4);
            }
        }
    }

    // Low-rank width from the w1 tensor ([d, L]).
    auto it = ck.tensors.find("blocks.0.time_mix.w1");
    if (it == ck.tensors.end() || it->second.dims.size() != 2 || it->second.dims[0] != s.d)
        return fail(YUF_ERR_FORMAT, "checkpoint has no usable blocks.0.time_mix.w1");
    s.low_rank = (int)it->second.dims[1];
    ck.header_json = std::move(header);
    return YUF_OK;
}

const float *Checkpoint::tensor(const std::string &name, const std::vector<long long> &dims, std::string &err) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) {
        err = "checkpoint has no tensor " + name;
        return nullptr;
    }
    if (!dims.empty() && it->second.dims != dims) {
        std::string want, got;
        for (long long x : dims) want += std::to_string(x) + ",";
        for (long long x : it->second.dims) got += std::to_string(x) + ",";
        err = "tensor " + name + " has shape [" + got + "], expected [" + want + "]";
        return nullptr;
    }
    return data.data() + it->second.offset;
}

}  // namespace yuf

// --------------------------------------------------------------------- C ABI
struct yuf_ckpt {
    yuf::Checkpoint ck;
};

extern "C" int yuf_ckpt_load(const char *path, yuf_ckpt **out) {
    if (!path || !out) return yuf::fail(YUF_ERR_INVALID, "yuf_ckpt_load: null argument");
    *out = nullptr;
    std::unique_ptr<yuf_ckpt> h;
    try {
        h.reset(new yuf_ckpt());
        int st = yuf::load_checkpoint(path, h->ck);
        if (st != YUF_OK) return st;
    } catch (const std::bad_alloc &) {
        return yuf::fail(YUF_ERR_OOM, "out of host memory loading checkpoint");
    } catch (const std::exception &e) {
        return yuf::fail(YUF_ERR_FORMAT, std::string("checkpoint load failed: ") + e.what());
    }
    *out = h.release();
    return YUF_OK;
}

extern "C" void yuf_ckpt_free(yuf_ckpt *ckpt) { delete ckpt; }

extern "C" int yuf_ckpt_config(const yuf_ckpt *ckpt, yuf_model_config *out) {
    if (!ckpt || !out) return yuf::fail(YUF_ERR_INVALID, "yuf_ckpt_config: null argument");
    yuf::fill_config(ckpt->ck.shape, *out);
    return YUF_OK;
}

extern "C" int yuf_ckpt_tensor(const yuf_ckpt *ckpt, const char *name, const float **data, int64_t *count,
                               int32_t *ndim, int64_t dims[8]) {
    if (!ckpt || !name) return yuf::fail(YUF_ERR_INVALID, "yuf_ckpt_tensor: null argument");
    auto it = ckpt->ck.tensors.find(name);
    if (it == ckpt->ck.tensors.end()) return yuf::fail(YUF_ERR_RANGE, std::string("checkpoint has no tensor ") + name);
    if (data) *data = ckpt->ck.data.data() + it->second.offset;
    if (count) *count = it->second.count;
    if (ndim) *ndim = (int32_t)it->second.dims.size();
    if (dims)
        for (size_t i = 0; i < it->second.dims.size() && i < 8; ++i) dims[i] = it->second.dims[i];
    return YUF_OK;
}

extern "C" int yuf_ckpt_header_json(const yuf_ckpt *ckpt, const char **json, size_t *len, uint32_t *version) {
    if (!ckpt || !json) return yuf::fail(YUF_ERR_INVALID, "yuf_ckpt_header_json: null argument");
    *json = ckpt->ck.header_json.c_str();
    if (len) *len = ckpt->ck.header_json.size();
    if (version) *version = ckpt->ck.version;
    return YUF_OK;
}

namespace yuf {
void fill_config(const ModelShape &s, yuf_model_config &c) {
    c.vocab_size = s.vocab;
    c.d_model = s.d;
    c.n_layers = s.layers;
    c.n_heads = s.heads;
    c.head_size = s.head_size;
    c.rosa_size = s.rosa;
    c.low_rank = s.low_rank;
    c.tie_embeddings = s.tie ? 1 : 0;
    c.dropout = s.dropout;
    c.midi_offset = s.midi_offset;
    c.midi_vocab_size = s.midi_vocab;
}
const Checkpoint &checkpoint_of(const yuf_ckpt *h) { return h->ck; }
}  // namespace yuf
