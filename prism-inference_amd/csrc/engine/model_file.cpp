/*
 * model_file.cpp - the on-disk model: a flat fp16 `.weights` file plus a
 * `.json` sidecar (host only).
 *
 * The reference's exporter writes exactly this pair for its conv layers
 * (vulkan_engine/export_weights.py:96-120: flat fp16 values, JSON with
 * total_fp16_values, total_bytes and per-layer weight/bias offsets and
 * counts) and its engine uploads the flat file as is
 * (prism_vulkan.cpp:558-611). The transformer adds layer kinds, per-block
 * tensors and the model shape to the sidecar; prism-inference_amd's
 * export_weights.py writes it. This file reads it back: a small JSON parser,
 * the mapping from layers to prism_block_offsets / prism_adapter_offsets, and
 * the one-call loader.
 */
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "engine_internal.h"

namespace prism {
namespace {

/* ---- a minimal JSON value + recursive-descent parser -------------------- */

struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    double num = 0;
    bool is_int = false;
    int64_t inum = 0;
    bool b = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json* get(const char* key) const {
        if (kind != Object) return nullptr;
        for (const auto& kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class Parser {
public:
    explicit Parser(const std::string& s) : s_(s) {}

    bool parse(Json& out, std::string* why) {
        if (!value(out, 0) || (ws(), p_ != s_.size())) {
            if (why) *why = "malformed JSON near byte " + std::to_string(p_) + (err_.empty() ? "" : ": " + err_);
            return false;
        }
        return true;
    }

private:
    const std::string& s_;
    size_t p_ = 0;
    std::string err_;

    void ws() {
        while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\t' || s_[p_] == '\n' || s_[p_] == '\r')) ++p_;
    }
    bool lit(const char* w) {
        const size_t n = strlen(w);
        if (s_.compare(p_, n, w) != 0) return false;
        p_ += n;
        return true;
    }
    bool value(Json& v, int depth) {
        if (depth > 64) return err_ = "nested too deeply", false;
        ws();
        if (p_ >= s_.size()) return err_ = "unexpected end", false;
        const char c = s_[p_];
        if (c == '{') return object(v, depth);
        if (c == '[') return array(v, depth);
        if (c == '"') {
            v.kind = Json::String;
            return string(v.str);
        }
        if (lit("true")) { v.kind = Json::Bool; v.b = true; return true; }
        if (lit("false")) { v.kind = Json::Bool; v.b = false; return true; }
        if (lit("null")) { v.kind = Json::Null; return true; }
        return number(v);
    }
    bool string(std::string& out) {
        ++p_; /* opening quote */
        while (p_ < s_.size() && s_[p_] != '"') {
            char c = s_[p_++];
            if (c == '\\') {
                if (p_ >= s_.size()) return err_ = "bad escape", false;
                const char e = s_[p_++];
                switch (e) {
                    case '"': case '\\': case '/': c = e; break;
                    case 'n': c = '\n'; break;
                    case 't': c = '\t'; break;
                    case 'r': c = '\r'; break;
                    case 'b': c = '\b'; break;
                    case 'f': c = '\f'; break;
                    case 'u': /* names here are ASCII; keep the code point's low byte */
                        if (p_ + 4 > s_.size()) return err_ = "bad \\u escape", false;
                        c = (char)strtol(s_.substr(p_, 4).c_str(), nullptr, 16);
                        p_ += 4;
                        break;
                    default: return err_ = "bad escape", false;
                }
            }
            out.push_back(c);
        }
        if (p_ >= s_.size()) return err_ = "unterminated string", false;
        ++p_;
        return true;
    }
    bool number(Json& v) {
        const size_t b = p_;
        bool frac = false;
        if (p_ < s_.size() && (s_[p_] == '-' || s_[p_] == '+')) ++p_;
        while (p_ < s_.size()) {
            const char c = s_[p_];
            if (c >= '0' && c <= '9') { ++p_; continue; }
            if (c == '.' || c == 'e' || c == 'E' || c == '-' || c == '+') { frac = true; ++p_; continue; }
            break;
        }
        if (p_ == b) return err_ = "expected a value", false;
        const std::string t = s_.substr(b, p_ - b);
        v.kind = Json::Number;
        errno = 0;
        char* end = nullptr;
        v.num = strtod(t.c_str(), &end);
        if (end != t.c_str() + t.size()) return err_ = "bad number", false;
        if (!frac) {
            const long long i = strtoll(t.c_str(), &end, 10);
            if (errno == ERANGE) return err_ = "integer out of range", false;
            v.is_int = true;
            v.inum = i;
        }
        return true;
    }
    bool array(Json& v, int depth) {
        v.kind = Json::Array;
        ++p_;
        ws();
        if (p_ < s_.size() && s_[p_] == ']') { ++p_; return true; }
        for (;;) {
            v.arr.emplace_back();
            if (!value(v.arr.back(), depth + 1)) return false;
            ws();
            if (p_ < s_.size() && s_[p_] == ',') { ++p_; continue; }
            if (p_ < s_.size() && s_[p_] == ']') { ++p_; return true; }
            return err_ = "expected , or ]", false;
        }
    }
    bool object(Json& v, int depth) {
        v.kind = Json::Object;
        ++p_;
        ws();
        if (p_ < s_.size() && s_[p_] == '}') { ++p_; return true; }
        for (;;) {
            ws();
            if (p_ >= s_.size() || s_[p_] != '"') return err_ = "expected a key", false;
            std::string key;
            if (!string(key)) return false;
            ws();
            if (p_ >= s_.size() || s_[p_] != ':') return err_ = "expected :", false;
            ++p_;
            v.obj.emplace_back(key, Json());
            if (!value(v.obj.back().second, depth + 1)) return false;
            ws();
            if (p_ < s_.size() && s_[p_] == ',') { ++p_; continue; }
            if (p_ < s_.size() && s_[p_] == '}') { ++p_; return true; }
            return err_ = "expected , or }", false;
        }
    }
};

bool get_int(const Json& o, const char* key, int64_t* out, std::string* why, const std::string& where) {
    const Json* v = o.get(key);
    if (!v || v->kind != Json::Number || !v->is_int) {
        if (why) *why = where + ": integer field \"" + key + "\" missing";
        return false;
    }
    *out = v->inum;
    return true;
}

}  // namespace

/* Parses a model sidecar into a description, per-block offsets and
 * (optionally) adapter offsets. Layer kinds (field "kind"):
 *   ln1, ln2      weight = gamma, bias = beta           [dim]
 *   qkv           weight [3*dim][dim], bias [3*dim]
 *   out           weight [dim][dim], bias [dim]
 *   router        weight [n_experts][dim], bias [n_experts] (MoE blocks)
 *   experts       w1/b1/w2/b2 offsets of expert 0 and expert_stride
 *   proj_up       weight [dim][in_dim], bias [dim]      (block -1)
 *   proj_down     weight [in_dim][dim], bias [in_dim]   (block -1) */
int read_model_json(const std::string& text, prism_model_desc* desc, std::vector<prism_block_offsets>* offs,
                    prism_adapter_offsets* ad, bool* has_adapters, int64_t* total, std::string* why) {
    Json root;
    Parser ps(text);
    if (!ps.parse(root, why)) return PRISM_ERR_BLOB;
    if (root.kind != Json::Object) { if (why) *why = "sidecar is not a JSON object"; return PRISM_ERR_BLOB; }
    const Json* fmt = root.get("format");
    if (!fmt || fmt->kind != Json::String || fmt->str != "prism-transformer-v1") {
        if (why) *why = "sidecar format is not \"prism-transformer-v1\"";
        return PRISM_ERR_BLOB;
    }
    int64_t tv = 0, tb = 0;
    if (!get_int(root, "total_fp16_values", &tv, why, "sidecar") || !get_int(root, "total_bytes", &tb, why, "sidecar"))
        return PRISM_ERR_BLOB;
    if (tv < 0 || tb != 2 * tv) { if (why) *why = "total_bytes != 2 * total_fp16_values"; return PRISM_ERR_BLOB; }
    const Json* m = root.get("model");
    if (!m || m->kind != Json::Object) { if (why) *why = "sidecar has no \"model\" object"; return PRISM_ERR_BLOB; }
    int64_t v[8];
    const char* keys[8] = {"dim", "n_blocks", "n_heads", "head_dim", "n_experts", "spatial_h", "spatial_w", "window"};
    for (int i = 0; i < 8; ++i) {
        if (!get_int(*m, keys[i], &v[i], why, "model")) return PRISM_ERR_BLOB;
        if (v[i] < 0 || v[i] > 1000000) { if (why) *why = std::string("model.") + keys[i] + " out of range"; return PRISM_ERR_BLOB; }
    }
    *desc = prism_model_desc{(int32_t)v[0], (int32_t)v[1], (int32_t)v[2], (int32_t)v[3],
                             (int32_t)v[4], (int32_t)v[5], (int32_t)v[6], (int32_t)v[7]};
    if (!shape_supported(desc, why)) return PRISM_ERR_UNSUPPORTED;
    const int NB = desc->n_blocks;
    const bool moe = desc->n_experts > 1;
    offs->assign(NB, prism_block_offsets{});
    /* which kinds each block has seen: bit per kind */
    std::vector<int> seen(NB, 0);
    enum { K_LN1 = 1, K_QKV = 2, K_OUT = 4, K_LN2 = 8, K_ROUTER = 16, K_EXPERTS = 32 };
    int adapters_seen = 0;
    prism_adapter_offsets a{};
    a.in_dim = 0;
    const Json* layers = root.get("layers");
    if (!layers || layers->kind != Json::Array) { if (why) *why = "sidecar has no \"layers\" array"; return PRISM_ERR_BLOB; }
    for (size_t li = 0; li < layers->arr.size(); ++li) {
        const Json& L = layers->arr[li];
        const std::string where = "layers[" + std::to_string(li) + "]";
        if (L.kind != Json::Object) { if (why) *why = where + " is not an object"; return PRISM_ERR_BLOB; }
        const Json* kind = L.get("kind");
        if (!kind || kind->kind != Json::String) { if (why) *why = where + ": no \"kind\""; return PRISM_ERR_BLOB; }
        int64_t blk = 0;
        if (!get_int(L, "block", &blk, why, where)) return PRISM_ERR_BLOB;
        const std::string& k = kind->str;
        if (k == "proj_up" || k == "proj_down") {
            int64_t w = 0, b = 0, in_dim = 0;
            if (!get_int(L, "weight_offset_fp16", &w, why, where) || !get_int(L, "bias_offset_fp16", &b, why, where) ||
                !get_int(L, "in_dim", &in_dim, why, where))
                return PRISM_ERR_BLOB;
            if (a.in_dim && a.in_dim != in_dim) { if (why) *why = where + ": adapters disagree on in_dim"; return PRISM_ERR_BLOB; }
            a.in_dim = (int32_t)in_dim;
            if (k == "proj_up") { a.up_w = w; a.up_b = b; adapters_seen |= 1; }
            else { a.down_w = w; a.down_b = b; adapters_seen |= 2; }
            continue;
        }
        if (blk < 0 || blk >= NB) { if (why) *why = where + ": block " + std::to_string(blk) + " out of range"; return PRISM_ERR_BLOB; }
        prism_block_offsets& o = (*offs)[blk];
        int bit = 0;
        if (k == "experts") {
            bit = K_EXPERTS;
            if (!get_int(L, "w1_offset_fp16", &o.exp_w1, why, where) || !get_int(L, "b1_offset_fp16", &o.exp_b1, why, where) ||
                !get_int(L, "w2_offset_fp16", &o.exp_w2, why, where) || !get_int(L, "b2_offset_fp16", &o.exp_b2, why, where) ||
                !get_int(L, "expert_stride", &o.exp_stride, why, where))
                return PRISM_ERR_BLOB;
            int64_t ne = 0;
            if (!get_int(L, "n_experts", &ne, why, where)) return PRISM_ERR_BLOB;
            if (ne != desc->n_experts) { if (why) *why = where + ": n_experts differs from the model's"; return PRISM_ERR_BLOB; }
        } else {
            int64_t w = 0, b = 0;
            if (!get_int(L, "weight_offset_fp16", &w, why, where) || !get_int(L, "bias_offset_fp16", &b, why, where))
                return PRISM_ERR_BLOB;
            if (k == "ln1") { bit = K_LN1; o.ln1_g = w; o.ln1_b = b; }
            else if (k == "qkv") { bit = K_QKV; o.qkv_w = w; o.qkv_b = b; }
            else if (k == "out") { bit = K_OUT; o.out_w = w; o.out_b = b; }
            else if (k == "ln2") { bit = K_LN2; o.ln2_g = w; o.ln2_b = b; }
            else if (k == "router") { bit = K_ROUTER; o.router_w = w; o.router_b = b; }
            else { if (why) *why = where + ": unknown layer kind \"" + k + "\""; return PRISM_ERR_BLOB; }
        }
        if (seen[blk] & bit) { if (why) *why = where + ": duplicate " + k + " for block " + std::to_string(blk); return PRISM_ERR_BLOB; }
        seen[blk] |= bit;
    }
    const int need = K_LN1 | K_QKV | K_OUT | K_LN2 | K_EXPERTS | (moe ? K_ROUTER : 0);
    for (int b = 0; b < NB; ++b)
        if ((seen[b] & need) != need) {
            if (why) *why = "block " + std::to_string(b) + " is missing layers";
            return PRISM_ERR_BLOB;
        }
    if (adapters_seen != 0 && adapters_seen != 3) { if (why) *why = "only one of proj_up / proj_down present"; return PRISM_ERR_BLOB; }
    int rc = validate_blocks(desc, offs->data(), tv, why);
    if (rc) return rc;
    if (adapters_seen == 3) {
        rc = validate_adapters(desc, &a, tv, why);
        if (rc) return rc;
    }
    if (ad) *ad = a;
    if (has_adapters) *has_adapters = adapters_seen == 3;
    if (total) *total = tv;
    return PRISM_OK;
}

bool read_text_file(const char* path, std::string* out) {
    std::ifstream f(path, std::ios::binary);
    if (!f.is_open()) return false;
    std::ostringstream ss;
    ss << f.rdbuf();
    *out = ss.str();
    return true;
}

std::string sidecar_path(const char* weights_path) {
    std::string p(weights_path);
    const std::string ext = ".weights";
    if (p.size() >= ext.size() && p.compare(p.size() - ext.size(), ext.size(), ext) == 0)
        return p.substr(0, p.size() - ext.size()) + ".json";
    return p + ".json";
}

}  // namespace prism

using namespace prism;

extern "C" int prism_read_model_json(const char* json_path, prism_model_desc* desc, prism_block_offsets* offs,
                                     int32_t offs_capacity, prism_adapter_offsets* adapters, int32_t* has_adapters,
                                     int64_t* total_elems) {
    if (!json_path || !desc) {
        set_global_error("prism_read_model_json: json_path or desc is NULL");
        return PRISM_ERR_INVALID;
    }
    std::string text, why;
    if (!read_text_file(json_path, &text)) {
        set_global_error(std::string("cannot read ") + json_path);
        return PRISM_ERR_INVALID;
    }
    std::vector<prism_block_offsets> o;
    bool had = false;
    const int rc = read_model_json(text, desc, &o, adapters, &had, total_elems, &why);
    if (rc) {
        set_global_error(std::string(json_path) + ": " + why);
        return rc;
    }
    if (offs) {
        if (offs_capacity < desc->n_blocks) {
            set_global_error("prism_read_model_json: offs has room for " + std::to_string(offs_capacity) + " blocks, the model has " +
                             std::to_string(desc->n_blocks));
            return PRISM_ERR_INVALID;
        }
        for (int b = 0; b < desc->n_blocks; ++b) offs[b] = o[b];
    }
    if (has_adapters) *has_adapters = had ? 1 : 0;
    return PRISM_OK;
}
