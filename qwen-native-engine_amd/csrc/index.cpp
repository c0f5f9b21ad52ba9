// index.json parsing and validation (generalises Index::validate, kernels/src/model.rs:51-86).
#include "index.hpp"

#include <cmath>

#include "error.hpp"
#include "json.hpp"

namespace qne {

static const int kGemvK[] = {512, 1024, 2048, 3072, 3584, 4096, 6144};

bool gemv_k_supported(int k) {
    for (int v : kGemvK)
        if (v == k) return true;
    return false;
}

const MatInfo& ModelIndex::mat(const std::string& n) const {
    auto it = mats.find(n);
    if (it == mats.end()) throw Error(QNE_EFORMAT, "missing matrix " + n);
    return it->second;
}

const TensorRef& ModelIndex::tensor(const std::string& n) const {
    auto it = tensors.find(n);
    if (it == tensors.end()) throw Error(QNE_EFORMAT, "missing tensor " + n);
    return it->second;
}

static int geti(const Json& o, const char* k) {
    uint64_t v = o.at(k).u64(k);
    if (v > (1u << 30)) throw Error(QNE_EFORMAT, std::string("value out of range: ") + k);
    return (int)v;
}

ModelIndex parse_index(const char* text, size_t n, uint64_t weights_len) {
    Json j = Json::parse(text, n);
    ModelIndex ix;
    ModelConfig& c = ix.cfg;
    c.format_version = j.has("format_version") ? (int)j.at("format_version").u64("format_version") : 1;
    if (c.format_version != 1 && c.format_version != 2)
        throw Error(QNE_EFORMAT, "unsupported format_version " + std::to_string(c.format_version));
    const Json& jc = j.at("config");
    c.layers = geti(jc, "layers");
    c.full_attention_every = geti(jc, "full_attention_every");
    c.hidden = geti(jc, "hidden");
    c.vocab = geti(jc, "vocab");
    c.rope_theta = jc.at("rope_theta").number();
    c.rope_dim = geti(jc, "rope_dim");
    // model.rs:48-51: a missing or zero intermediate follows the hidden size.
    c.intermediate = jc.has("intermediate") ? geti(jc, "intermediate") : 0;
    if (c.intermediate == 0) c.intermediate = c.hidden == 1024 ? 3584 : 6144;

    if (c.format_version == 1) {
        // model.rs:53-56: only the Qwen3.5-0.8B / 2B architecture.
        bool ok = c.layers == 24 && c.full_attention_every == 4 &&
                  ((c.hidden == 1024 && c.intermediate == 3584) || (c.hidden == 2048 && c.intermediate == 6144)) &&
                  c.vocab == 248320 && c.rope_dim == 64 && c.rope_theta == 10000000.0;
        if (!ok)
            throw Error(QNE_EFORMAT, "unsupported model architecture: these kernels require Qwen3.5-0.8B or Qwen3.5-2B");
        c.n_q_heads = 8; c.n_kv_heads = 2; c.head_dim = 256;
        c.gdn_heads = 16; c.gdn_dk = 128; c.gdn_dv = 128; c.conv_kernel = 4; c.eps = 1e-6f;
    } else {
        c.n_q_heads = geti(jc, "n_q_heads");
        c.n_kv_heads = geti(jc, "n_kv_heads");
        c.head_dim = geti(jc, "head_dim");
        c.gdn_heads = geti(jc, "gdn_heads");
        c.gdn_dk = geti(jc, "gdn_dk");
        c.gdn_dv = geti(jc, "gdn_dv");
        c.conv_kernel = jc.has("conv_kernel") ? geti(jc, "conv_kernel") : 4;
        c.eps = jc.has("rms_eps") ? (float)jc.at("rms_eps").number() : 1e-6f;
    }
    // Shapes the kernels are built for.
    auto need = [](bool ok, const std::string& what) {
        if (!ok) throw Error(QNE_EFORMAT, "unsupported model architecture: " + what);
    };
    need(c.layers >= 1 && c.layers <= 256, "layers must be 1..256");
    need(c.full_attention_every >= 1, "full_attention_every must be >= 1");
    need(c.head_dim == 256, "head_dim must be 256");
    need(c.gdn_dk == 128 && c.gdn_dv == 128, "gdn_dk and gdn_dv must be 128");
    need(c.conv_kernel == 4, "conv_kernel must be 4");
    need(c.n_kv_heads >= 1 && c.n_q_heads % c.n_kv_heads == 0 &&
             (c.n_q_heads / c.n_kv_heads == 1 || c.n_q_heads / c.n_kv_heads == 2 || c.n_q_heads / c.n_kv_heads == 4),
         "n_q_heads must be 1, 2 or 4 times n_kv_heads");
    need(c.n_q_heads <= 64 && c.gdn_heads >= 1 && c.gdn_heads <= 64, "too many heads");
    need(c.rope_dim >= 2 && c.rope_dim % 2 == 0 && c.rope_dim <= c.head_dim, "rope_dim must be even and <= head_dim");
    need(c.vocab >= 1 && c.hidden >= 1, "empty vocab or hidden size");
    need(std::isfinite(c.rope_theta) && c.rope_theta > 1.0, "rope_theta must be > 1");
    need(c.eps > 0.0f && c.eps < 1.0f, "rms eps must be in (0, 1)");

    // Tensor table: ranges inside weights.bin, 4-byte aligned, non-empty (model.rs:57-61).
    const Json& jt = j.at("tensors");
    if (jt.type != Json::Object) throw Error(QNE_EFORMAT, "tensors must be an object");
    for (const auto& kv : jt.obj) {
        TensorRef t;
        t.offset = kv.second.at("offset").u64("offset");
        t.bytes = kv.second.at("bytes").u64("bytes");
        bool ok = t.offset + t.bytes >= t.offset && t.offset + t.bytes <= weights_len && t.offset % 4 == 0 &&
                  t.bytes > 0 && t.bytes % 4 == 0;
        if (!ok) throw Error(QNE_EFORMAT, "invalid tensor range: " + kv.first);
        ix.tensors[kv.first] = t;
    }
    auto tensor = [&](const std::string& name, uint64_t expected) -> TensorRef {
        auto it = ix.tensors.find(name);
        if (it == ix.tensors.end() || it->second.bytes != expected)
            throw Error(QNE_EFORMAT, "invalid tensor size: " + name);
        return it->second;
    };
    const Json& jm = j.at("matrices");
    auto matrix = [&](const std::string& name, int rows, int k) {
        if (!jm.has(name)) throw Error(QNE_EFORMAT, "invalid matrix shape: " + name);
        const Json& e = jm.at(name);
        MatInfo m;
        m.rows = geti(e, "rows");
        m.k = geti(e, "k");
        if (m.rows != rows || m.k != k) throw Error(QNE_EFORMAT, "invalid matrix shape: " + name);
        std::string dtype = c.format_version == 1 ? "q4" : (e.has("dtype") ? e.at("dtype").string() : "q4");
        uint64_t el = (uint64_t)rows * (uint64_t)k;
        if (dtype == "f16") {
            m.kind = MAT_F16;
            m.w = tensor(name + ".w", el * 2);
        } else if (dtype == "q4") {
            m.kind = MAT_Q4;
            if (c.format_version == 1) {
                m.group = 32;
                m.zero_u4 = true;
            } else {
                m.group = e.has("group") ? geti(e, "group") : 64;
                std::string zk = e.has("zero") ? e.at("zero").string() : "f16";
                if (zk != "f16" && zk != "u4") throw Error(QNE_EFORMAT, "unknown zero kind for " + name);
                m.zero_u4 = zk == "u4";
            }
            if (m.group != 32 && m.group != 64 && m.group != 128)
                throw Error(QNE_EFORMAT, "unsupported quantisation group for " + name);
            if (k % 512 != 0) throw Error(QNE_EFORMAT, "invalid matrix shape: " + name + " (k % 512)");
            uint64_t groups = el / (uint64_t)m.group;
            m.w = tensor(name + ".w", el / 2);
            m.s = tensor(name + ".s", groups * 2);
            // u4 zero points: ceil(groups per row / 2) bytes per row (model.rs:69-71 with block 32).
            uint64_t zb = m.zero_u4 ? (uint64_t)rows * (((uint64_t)k / m.group + 1) / 2) : groups * 2;
            m.z = tensor(name + ".z", zb);
        } else {
            throw Error(QNE_EFORMAT, "unknown dtype for " + name);
        }
        ix.mats[name] = m;
    };
    const uint64_t H = (uint64_t)c.hidden;
    matrix("embed", c.vocab, c.hidden);
    matrix("lm_head", c.vocab, c.hidden);
    tensor("final_norm", H * 4);
    for (int i = 0; i < c.layers; i++) {
        std::string p = "layer" + std::to_string(i) + ".";
        bool attn = c.is_attn(i);
        tensor(p + "input_norm", H * 4);
        tensor(p + "post_norm", H * 4);
        matrix(p + "mixer_in", attn ? c.attn_proj() : c.gdn_proj(), c.hidden);
        matrix(p + "mixer_out", c.hidden, attn ? c.attn_out() : c.gdn_out());
        matrix(p + "gate_up", 2 * c.intermediate, c.hidden);
        matrix(p + "down", c.hidden, c.intermediate);
        if (attn) {
            tensor(p + "attn_norms", (uint64_t)c.head_dim * 2 * 4);
        } else {
            tensor(p + "conv_w", (uint64_t)c.conv_channels() * c.conv_kernel * 4);
            tensor(p + "gdn_params", (uint64_t)(2 * c.gdn_heads + c.gdn_dv) * 4);
        }
    }
    // Every matrix width must be one the GEMV kernels are built for.
    for (const auto& kv : ix.mats) {
        if (kv.first == "embed") continue;  // gathered by rows, never multiplied
        if (!gemv_k_supported(kv.second.k))
            throw Error(QNE_EFORMAT, "unsupported matrix width k=" + std::to_string(kv.second.k) + " for " + kv.first);
    }
    return ix;
}

}  // namespace qne
