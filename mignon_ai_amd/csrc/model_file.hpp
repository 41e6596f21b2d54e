// Host-side decoding of the reference's INT8 model file into plain arrays.
//
// Binary container (internal/binfmt/binfmt.go:1-144): "MGNN", uint16 version 1, uint8 kind (2 = INT8),
// uint8 reserved, uint32 header length, JSON header, then uint32-count-prefixed int8 / float32 arrays in
// the order of quant.CheckpointJSON.arrays (internal/quant/checkpoint.go:74-89). Legacy JSON files carry
// the arrays inline (internal/quant/checkpoint.go:162-180). Shape check: checkBlockShapes
// (internal/quant/checkpoint.go:214-225). Errors reuse the reference's wording.
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"

namespace mg {

struct HostBlock {
    int steps = 1, dilation_base = 2, initial_dilation = 1;
    std::vector<int8_t> w1, w2, wsel;
    float s1 = 0, s2 = 0, ssel = 0;
    std::vector<float> b1, b2, gamma;
    bool has_attn = false;
    std::vector<float> attn_norm;
    std::vector<int8_t> qkv, wo;
    float sqkv = 0, so = 0;
};

struct HostModel {
    int V = 0, D = 0, H = 0;
    bool tied = false;
    std::vector<int8_t> embed;
    float embed_scale = 0;
    std::vector<HostBlock> blocks;
    std::vector<float> final_norm;
    std::vector<int8_t> head_w;
    float head_scale = 0;
    std::vector<float> head_b;
    int attn_heads = 0, attn_window = 0, context_size = 0;
    std::string task;
    long long num_params = 0;  // quant.Model.NumParams (internal/quant/checkpoint.go:91-104)
};

class FormatError : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

namespace detail {

inline uint32_t rd32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

struct ArrayReader {
    const uint8_t* p;
    size_t n, off = 0;
    int index = 0;
    template <class T>
    void read(std::vector<T>& out) {
        if (n - off < 4) throw FormatError("binary model file is truncated (array " + std::to_string(index) + ")");
        uint32_t cnt = rd32(p + off);
        off += 4;
        if ((size_t)cnt > (n - off) / sizeof(T))
            throw FormatError("binary model file is truncated (array " + std::to_string(index) + ")");
        out.resize(cnt);
        if (cnt) std::memcpy(out.data(), p + off, (size_t)cnt * sizeof(T));  // little-endian host
        off += (size_t)cnt * sizeof(T);
        index++;
    }
};

template <class T>
void json_array(const mgjson::Value* v, std::vector<T>& out) {
    out.clear();
    if (!v || v->is_null()) return;
    if (v->kind != mgjson::Value::Array) throw FormatError("expected an array in the model file");
    out.reserve(v->arr.size());
    for (auto& e : v->arr) out.push_back((T)e.num);
}

inline float tensor_scale(const mgjson::Value* t) {
    if (!t || t->kind != mgjson::Value::Object) return 0.0f;
    return (float)t->number_or("scale", 0.0);
}

inline const mgjson::Value* tensor_data(const mgjson::Value* t) { return t ? t->get("data") : nullptr; }

}  // namespace detail

// The container of a model file (internal/binfmt/binfmt.go; legacy JSON files are the header alone):
// returns the parsed JSON header and, for binary files, where the arrays begin.
inline mgjson::Value parse_model_header(const uint8_t* data, size_t n, const uint8_t** arrays_out,
                                        size_t* arrays_n_out) {
    using namespace detail;
    mgjson::Value cp;
    bool binary = n >= 4 && std::memcmp(data, "MGNN", 4) == 0;
    const uint8_t* arrays = nullptr;
    size_t arrays_n = 0;
    if (binary) {
        if (n < 12) throw FormatError("binary model file is truncated");
        uint16_t version = (uint16_t)(data[4] | (data[5] << 8));
        if (version != 1)
            throw FormatError("binary model file version " + std::to_string(version) +
                              " is not supported (this build reads version 1)");
        int kind = data[6];
        if (kind != 1 && kind != 2) throw FormatError("unknown model kind " + std::to_string(kind));
        uint32_t hn = rd32(data + 8);
        if ((size_t)hn > n - 12) throw FormatError("binary model file is truncated (header)");
        if (kind != 2) throw FormatError("not an INT8 model file");
        cp = mgjson::parse((const char*)data + 12, hn);
        arrays = data + 12 + hn;
        arrays_n = n - 12 - hn;
    } else {
        cp = mgjson::parse((const char*)data, n);
    }
    if (cp.kind != mgjson::Value::Object) throw FormatError("model file header is not an object");
    if (arrays_out) *arrays_out = arrays;
    if (arrays_n_out) *arrays_n_out = arrays_n;
    return cp;
}

// quant.Decode (internal/quant/checkpoint.go:162-212).
inline HostModel decode_model_file(const uint8_t* data, size_t n) {
    using namespace detail;
    HostModel m;
    const uint8_t* arrays = nullptr;
    size_t arrays_n = 0;
    const mgjson::Value cp = parse_model_header(data, n, &arrays, &arrays_n);
    const bool binary = arrays != nullptr;
    m.V = (int)cp.number_or("vocab_size", 0);
    m.D = (int)cp.number_or("state_size", 0);
    m.H = (int)cp.number_or("hidden_size", 0);
    m.tied = cp.bool_or("tied_embed", false);
    const mgjson::Value* meta = cp.get("metadata");
    if (meta) {
        m.attn_heads = (int)meta->number_or("attn_heads", 0);
        m.attn_window = (int)meta->number_or("attn_window", 0);
        m.context_size = (int)meta->number_or("context_size", 0);
        const mgjson::Value* t = meta->get("task");
        if (t && t->kind == mgjson::Value::String) m.task = t->str;
    }
    const mgjson::Value* emb = cp.get("embed");
    m.embed_scale = tensor_scale(emb);
    const mgjson::Value* blocks = cp.get("blocks");
    size_t nb = (blocks && blocks->kind == mgjson::Value::Array) ? blocks->arr.size() : 0;
    m.blocks.resize(nb);
    for (size_t b = 0; b < nb; b++) {
        const mgjson::Value& jb = blocks->arr[b];
        HostBlock& hb = m.blocks[b];
        hb.steps = (int)jb.number_or("steps", 0);
        hb.dilation_base = (int)jb.number_or("dilation_base", 0);
        hb.initial_dilation = (int)jb.number_or("initial_dilation", 0);
        hb.s1 = tensor_scale(jb.get("rule_w1"));
        hb.s2 = tensor_scale(jb.get("rule_w2"));
        hb.ssel = tensor_scale(jb.get("rule_w_select"));
        const mgjson::Value* a = jb.get("attn");
        hb.has_attn = a && !a->is_null();
        if (hb.has_attn) {
            hb.sqkv = tensor_scale(a->get("qkv"));
            hb.so = tensor_scale(a->get("out"));
        }
    }
    const mgjson::Value* hw = cp.get("head_w");
    m.head_scale = tensor_scale(hw);

    if (binary) {
        ArrayReader r{arrays, arrays_n};
        r.read(m.embed);
        for (auto& hb : m.blocks) {
            r.read(hb.w1); r.read(hb.b1); r.read(hb.w2); r.read(hb.b2); r.read(hb.gamma); r.read(hb.wsel);
            if (hb.has_attn) { r.read(hb.attn_norm); r.read(hb.qkv); r.read(hb.wo); }
        }
        r.read(m.final_norm); r.read(m.head_w); r.read(m.head_b);
        if (r.off != arrays_n)
            throw FormatError("binary model file has " + std::to_string(arrays_n - r.off) + " unexpected trailing bytes");
    } else {
        json_array(tensor_data(emb), m.embed);
        for (size_t b = 0; b < nb; b++) {
            const mgjson::Value& jb = blocks->arr[b];
            HostBlock& hb = m.blocks[b];
            json_array(tensor_data(jb.get("rule_w1")), hb.w1);
            json_array(jb.get("rule_b1"), hb.b1);
            json_array(tensor_data(jb.get("rule_w2")), hb.w2);
            json_array(jb.get("rule_b2"), hb.b2);
            json_array(jb.get("gamma"), hb.gamma);
            json_array(tensor_data(jb.get("rule_w_select")), hb.wsel);
            if (hb.has_attn) {
                const mgjson::Value* a = jb.get("attn");
                json_array(a->get("norm"), hb.attn_norm);
                json_array(tensor_data(a->get("qkv")), hb.qkv);
                json_array(tensor_data(a->get("out")), hb.wo);
            }
        }
        json_array(cp.get("final_norm"), m.final_norm);
        json_array(tensor_data(hw), m.head_w);
        json_array(cp.get("head_b"), m.head_b);
    }

    // checkBlockShapes (internal/quant/checkpoint.go:214-225)
    size_t want = (size_t)2 * m.H * 3 * m.D;
    for (size_t b = 0; b < nb; b++) {
        if (m.blocks[b].w1.size() != want)
            throw FormatError("block " + std::to_string(b) + " rule_w1 has " + std::to_string(m.blocks[b].w1.size()) +
                              " weights, want " + std::to_string(want) + " (2*hidden*" + std::to_string(3 * m.D) +
                              "): trained with a different CA neighbourhood, retrain the model");
    }
    long long np = (long long)m.embed.size();
    for (auto& hb : m.blocks) {
        np += hb.w1.size() + hb.b1.size() + hb.w2.size() + hb.b2.size() + hb.gamma.size() + hb.wsel.size();
        if (hb.has_attn) np += hb.attn_norm.size() + hb.qkv.size() + hb.wo.size();
    }
    np += m.final_norm.size() + (m.tied ? 0 : m.head_w.size()) + m.head_b.size();
    m.num_params = np;
    return m;
}

// Sizes the engine relies on beyond the reference's own shape check; the reference would index out of
// range (a Go panic) on these, the engine reports them instead.
inline void validate_for_engine(const HostModel& m) {
    auto need = [](bool ok, const std::string& what) {
        if (!ok) throw FormatError("model file: " + what);
    };
    need(m.V > 0 && m.D > 0 && m.H > 0, "vocab, state and hidden sizes must be positive");
    need(m.D <= 1024 && m.H <= 2048, "state size above 1024 or hidden size above 2048 is not supported");
    need(m.embed.size() == (size_t)m.V * m.D, "embed has the wrong size");
    for (size_t b = 0; b < m.blocks.size(); b++) {
        const HostBlock& hb = m.blocks[b];
        std::string p = "block " + std::to_string(b) + " ";
        need(hb.steps >= 0, p + "has negative steps");
        need(hb.b1.size() == (size_t)2 * m.H, p + "rule_b1 has the wrong size");
        need(hb.w2.size() == (size_t)2 * m.D * m.H, p + "rule_w2 has the wrong size");
        need(hb.b2.size() == (size_t)2 * m.D, p + "rule_b2 has the wrong size");
        need(hb.wsel.size() == (size_t)m.D * m.D, p + "rule_w_select has the wrong size");
        if (hb.has_attn) {
            need(m.attn_heads > 0 && m.D % m.attn_heads == 0, "attention heads must divide the state size");
            need(hb.attn_norm.size() == (size_t)m.D, p + "attention norm has the wrong size");
            need(hb.qkv.size() == (size_t)3 * m.D * m.D, p + "attention qkv has the wrong size");
            need(hb.wo.size() == (size_t)m.D * m.D, p + "attention out has the wrong size");
        }
    }
    if (!m.tied) need(m.head_w.size() == (size_t)m.V * m.D, "head_w has the wrong size");
    need(m.head_b.empty() || m.head_b.size() == (size_t)m.V, "head_b has the wrong size");
}

}  // namespace mg
