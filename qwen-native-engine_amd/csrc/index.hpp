// index.json: the tensor map written next to weights.bin, and its validation.
//
// format_version 1 is the reference's file (scripts/convert_weights.py:134-141, validated by
// Index::validate, kernels/src/model.rs:51-86): fixed Qwen3.5-0.8B/2B architecture, every matrix
// int4 in the ONNX MatMulNBits layout (block 32, f16 scale, u4 zero point).
// format_version 2 adds config-driven shapes (heads, kv heads, head_dim, GDN heads and dims,
// conv kernel, rms eps) and a per-matrix encoding: "f16", or "q4" with a group size and an
// "f16" or "u4" zero point.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace qne {

enum MatKind { MAT_F16 = 0, MAT_Q4 = 1 };

struct TensorRef {
    uint64_t offset = 0, bytes = 0;
};

struct MatInfo {
    int kind = MAT_Q4;
    int rows = 0, k = 0, group = 0;
    bool zero_u4 = false;  // zero point as packed u4 (format 1) instead of f16
    TensorRef w, s, z;
};

struct ModelConfig {
    int format_version = 2;
    int layers = 0, full_attention_every = 4, hidden = 0, intermediate = 0, vocab = 0;
    int n_q_heads = 8, n_kv_heads = 2, head_dim = 256, rope_dim = 64;
    double rope_theta = 1e7;
    int gdn_heads = 16, gdn_dk = 128, gdn_dv = 128, conv_kernel = 4;
    float eps = 1e-6f;

    bool is_attn(int i) const { return (i + 1) % full_attention_every == 0; }
    int attn_proj() const { return 2 * n_q_heads * head_dim + 2 * n_kv_heads * head_dim; }
    int gdn_proj() const { return 2 * gdn_heads * gdn_dk + 2 * gdn_heads * gdn_dv + 2 * gdn_heads; }
    int attn_out() const { return n_q_heads * head_dim; }
    int gdn_out() const { return gdn_heads * gdn_dv; }
    int conv_channels() const { return 2 * gdn_heads * gdn_dk + gdn_heads * gdn_dv; }
    int n_attn_layers() const {
        int n = 0;
        for (int i = 0; i < layers; i++) n += is_attn(i);
        return n;
    }
};

struct ModelIndex {
    ModelConfig cfg;
    std::map<std::string, TensorRef> tensors;
    std::map<std::string, MatInfo> mats;
    const MatInfo& mat(const std::string& n) const;
    const TensorRef& tensor(const std::string& n) const;
};

// Parses index.json and checks it against a weights blob of `weights_len` bytes. Throws
// Error(QNE_EFORMAT) with the reference's messages where they exist.
ModelIndex parse_index(const char* json, size_t n, uint64_t weights_len);

// The matrix widths (k) that the GEMV kernels are built for.
bool gemv_k_supported(int k);

}  // namespace qne
