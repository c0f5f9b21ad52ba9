// DeviceSampler: src/sampling.rs Sampler with the O(vocab) part on the device (kernels/sample.hip).
#include "sample.hpp"

#include <cmath>
#include <cstring>

#include "error.hpp"
#include "hip_util.hpp"
#include "kernels/launch.hpp"

namespace qne {

DeviceSampler::DeviceSampler(const SamplingOptions& o, uint32_t vocab) : o_(o), V_(vocab) {
    if (vocab == 0) throw Error(QNE_EINVAL, "empty vocabulary");
    if (o.top_k > kSampleMaxK) throw Error(QNE_EINVAL, "top_k above 1024 is not supported by the device sampler");
    if (!(o.temperature == o.temperature) || !(o.top_p == o.top_p) || !(o.presence_penalty == o.presence_penalty))
        throw Error(QNE_EINVAL, "NaN sampling option");
    // Sampler::new (src/sampling.rs:42-46): xorshift has a fixed point at zero
    state_ = (o.seed * 0x9E3779B97F4A7C15ull) | 1ull;
    const size_t words = ((size_t)vocab + 31) / 32;
    seen_host_.assign(words, 0u);
    try {
        QNE_HIP(hipMalloc((void**)&seen_, words * 4));
        QNE_HIP(hipMemset(seen_, 0, words * 4));
        QNE_HIP(hipMalloc((void**)&mask_, words * 4));
        QNE_HIP(hipMalloc((void**)&out_v_, kSampleMaxK * 4));
        QNE_HIP(hipMalloc((void**)&out_i_, kSampleMaxK * 4));
        QNE_HIP(hipMalloc((void**)&info_, 16));
        QNE_HIP(hipMalloc(&scratch_, sample_scratch_bytes()));
        QNE_HIP(hipHostMalloc((void**)&host_, (4 + 2 * kSampleMaxK) * 4, hipHostMallocDefault));
    } catch (...) {
        release();
        throw;
    }
}

DeviceSampler::~DeviceSampler() { release(); }

void DeviceSampler::release() {
    for (void* p : {(void*)seen_, (void*)mask_, (void*)out_v_, (void*)out_i_, (void*)info_, scratch_})
        if (p) (void)hipFree(p);
    if (host_) (void)hipHostFree(host_);
    seen_ = mask_ = out_i_ = info_ = host_ = nullptr;
    out_v_ = nullptr;
    scratch_ = nullptr;
}

// src/sampling.rs:48-55
float DeviceSampler::next_f32() {
    uint64_t x = state_;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    state_ = x;
    return (float)(x >> 40) / (float)(1ull << 24);
}

uint32_t DeviceSampler::sample(const float* logits, const uint32_t* mask, uint32_t mask_len, uint32_t bias_token,
                               float bias, hipStream_t st) {
    if (!logits) throw Error(QNE_EINVAL, "null logits");
    SampleArgs a;
    a.logits = logits;
    a.V = V_;
    if (mask) {
        const uint32_t covered = mask_len < V_ ? mask_len : V_;  // tokens past the vocabulary are never read
        if (covered) QNE_HIP(hipMemcpyAsync(mask_, mask, ((size_t)covered + 31) / 32 * 4, hipMemcpyHostToDevice, st));
        a.mask = mask_;
        a.mask_len = covered;
    }
    // choose (:81-86): the presence penalty does not apply under a grammar mask
    const float penalty = mask ? 0.0f : o_.presence_penalty;
    a.seen = penalty != 0.0f ? seen_ : nullptr;
    a.penalty = penalty;
    a.bias_token = bias_token;
    a.bias = bias;
    const bool greedy = o_.temperature <= 0.0f;
    a.k = greedy ? 0u : (o_.top_k < 1 ? 1u : o_.top_k);
    a.out_v = out_v_;
    a.out_i = out_i_;
    a.info = info_;
    launch_sample(a, scratch_, st);
    QNE_HIP(hipGetLastError());
    // the pick or the candidates come back with the flags in one synchronisation (up to a.k
    // candidates are copied; host_[0] says how many are valid)
    float* v = (float*)(host_ + 4);
    uint32_t* id = host_ + 4 + kSampleMaxK;
    QNE_HIP(hipMemcpyAsync(host_, info_, 16, hipMemcpyDeviceToHost, st));
    if (a.k) {
        QNE_HIP(hipMemcpyAsync(v, out_v_, (size_t)a.k * 4, hipMemcpyDeviceToHost, st));
        QNE_HIP(hipMemcpyAsync(id, out_i_, (size_t)a.k * 4, hipMemcpyDeviceToHost, st));
    }
    QNE_HIP(hipStreamSynchronize(st));
    const uint32_t n = host_[0], flags = host_[1];
    // try_sample (:58-67): fail closed
    if (flags & 1u) throw Error(QNE_EINVAL, "non-finite model logits");
    if (!(flags & 2u)) throw Error(QNE_EINVAL, "no finite token is allowed by the sampling mask");
    uint32_t token = 0;
    if (greedy) {
        token = host_[2];
    } else if (n > 0) {
        // choose (:104-133), in the reference's f32 order
        const float t = o_.temperature, top = v[0];
        float w[kSampleMaxK];
        for (uint32_t j = 0; j < n; j++) w[j] = std::exp((v[j] - top) / t);
        float total = 0.0f;
        for (uint32_t j = 0; j < n; j++) total += w[j];
        float kept = 0.0f;
        uint32_t m = 0;
        for (uint32_t j = 0; j < n; j++) {
            kept += w[j];
            m++;
            if (kept >= o_.top_p * total) break;
        }
        float r = next_f32() * kept;
        token = id[m - 1];
        for (uint32_t j = 0; j < m; j++) {
            r -= w[j];
            if (r <= 0.0f) {
                token = id[j];
                break;
            }
        }
    }
    // sample (:69-79): remember the token for the presence penalty
    if (o_.presence_penalty != 0.0f && token < V_) {
        uint32_t& word = seen_host_[token >> 5];
        const uint32_t nw = word | (1u << (token & 31));
        if (nw != word) {
            word = nw;
            QNE_HIP(hipMemcpyAsync(seen_ + (token >> 5), &seen_host_[token >> 5], 4, hipMemcpyHostToDevice, st));
            QNE_HIP(hipStreamSynchronize(st));
        }
    }
    return token;
}

}  // namespace qne
