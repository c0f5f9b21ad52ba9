// Token sampling on the device (src/sampling.rs Sampler): the O(vocab) work -- fail-closed checks,
// presence penalty, grammar mask, greedy pick or top-k candidates -- runs in one kernel over the
// logits where they lie; only the pick or the k best (value, token) pairs come back, and the
// O(k) tail (softmax weights, top-p prefix, the xorshift draw) runs here in the reference's f32
// arithmetic and order, so a draw picks the token the reference picks from the same logits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace qne {

struct SamplingOptions {
    float temperature = 0.6f;  // <= 0: greedy
    uint32_t top_k = 20;       // 0 is taken as 1, as by the reference; at most 1024 here
    float top_p = 0.95f;
    uint64_t seed = 42;
    float presence_penalty = 0.0f;  // subtracted from generated tokens' logits (not under a mask)
};

class DeviceSampler {
  public:
    DeviceSampler(const SamplingOptions& o, uint32_t vocab);
    ~DeviceSampler();
    DeviceSampler(const DeviceSampler&) = delete;
    DeviceSampler& operator=(const DeviceSampler&) = delete;

    // Sampler::try_sample (src/sampling.rs:58-67) over `vocab` device logits, with `bias` added to
    // `bias_token`'s logit first (the caller's tool-call bias; bias_token >= vocab: none). mask:
    // host bitset of mask_len tokens (bit i%32 of word i/32 allows token i), or null. Throws
    // QNE_EINVAL for a distribution the reference rejects. Ends synchronised with `st`.
    uint32_t sample(const float* logits, const uint32_t* mask, uint32_t mask_len, uint32_t bias_token, float bias,
                    hipStream_t st);
    uint64_t state() const { return state_; }

  private:
    float next_f32();
    void release();

    SamplingOptions o_;
    uint32_t V_;
    uint64_t state_;
    std::vector<uint32_t> seen_host_;  // bitset of the generated tokens
    uint32_t* seen_ = nullptr;         // device copy
    uint32_t* mask_ = nullptr;         // device mask upload
    float* out_v_ = nullptr;
    uint32_t* out_i_ = nullptr;
    uint32_t* info_ = nullptr;
    void* scratch_ = nullptr;   // the kernels' counters, sampled keys and candidates
    uint32_t* host_ = nullptr;  // pinned: info (4 words) + k values + k tokens
};

}  // namespace qne
