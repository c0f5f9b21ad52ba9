// Seeded synthetic weights and the int4 quantiser used to build test and benchmark models.
//
// Generator: value i of stream `stream` under `seed` is the Box-Muller transform of two SplitMix64
// outputs on a counter, so any tensor (or any slice of one) can be produced independently and in
// parallel: key = mix(seed ^ mix(stream)); a = mix(key + 2p), b = mix(key + 2p + 1) for pair p;
// u1 = ((a >> 11) + 1) / 2^53, u2 = (b >> 11) / 2^53; r = sqrt(-2 ln u1);
// value[2p] = r cos(2 pi u2), value[2p+1] = r sin(2 pi u2).
// Quantiser (per group of `group` values along a row): s = (max - min) / 15 rounded to f16
// (1 if max == min), z = -min / s rounded to f16, q = clamp(round_half_even(w / s + z), 0, 15);
// the dequantised weight is (q - z) * s with the stored f16 s and z.
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/qne.h"

namespace {

inline uint64_t mix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

inline void normal_pair(uint64_t key, uint64_t p, double* z0, double* z1) {
    const uint64_t a = mix(key + 2 * p), b = mix(key + 2 * p + 1);
    const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53, u2 = (double)(b >> 11) * 0x1.0p-53;
    const double r = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586476925286766559 * u2;
    *z0 = r * std::cos(th);
    *z1 = r * std::sin(th);
}

uint16_t to_f16(float f) {  // round to nearest even
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)(ax >> 23);
        uint32_t v = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (v & 1u))) v++;
        return (uint16_t)(sign | v);
    }
    uint32_t v = (ax >> 13) - (112u << 10);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) v++;
    return (uint16_t)(sign | v);
}

float from_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, f = h & 0x3ffu;
    if (e == 0) {
        const float v = (float)f * 5.9604644775390625e-8f;
        return (h & 0x8000u) ? -v : v;
    }
    const uint32_t bits = e == 31 ? (sign | 0x7f800000u | (f << 13)) : (sign | ((e + 112u) << 23) | (f << 13));
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

template <typename Out>
int fill_normal(uint64_t seed, uint64_t stream, size_t n, float std_, Out out) {
    const uint64_t key = mix(seed ^ mix(stream));
    const int64_t pairs = (int64_t)((n + 1) / 2);
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < pairs; p++) {
        double z0, z1;
        normal_pair(key, (uint64_t)p, &z0, &z1);
        out((size_t)(2 * p), (float)(z0 * std_));
        if ((size_t)(2 * p + 1) < n) out((size_t)(2 * p + 1), (float)(z1 * std_));
    }
    return QNE_OK;
}

}  // namespace

extern "C" {

int qne_synth_normal_f32(uint64_t seed, uint64_t stream, size_t n, float std_, float* out) {
    if (!out && n) return QNE_EINVAL;
    return fill_normal(seed, stream, n, std_, [out](size_t i, float v) { out[i] = v; });
}

int qne_synth_normal_f16(uint64_t seed, uint64_t stream, size_t n, float std_, uint16_t* out) {
    if (!out && n) return QNE_EINVAL;
    return fill_normal(seed, stream, n, std_, [out](size_t i, float v) { out[i] = to_f16(v); });
}

int qne_quantize_q4g(const float* w, size_t rows, size_t k, size_t group, uint32_t* q, uint16_t* scales,
                     uint16_t* zeros) {
    if (!w || !q || !scales || !zeros || group == 0 || k % group != 0 || k % 8 != 0 || group % 8 != 0)
        return QNE_EINVAL;
    const size_t gpr = k / group;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; r++) {
        for (size_t g = 0; g < gpr; g++) {
            const float* src = w + (size_t)r * k + g * group;
            float mn = src[0], mx = src[0];
            for (size_t i = 1; i < group; i++) {
                mn = src[i] < mn ? src[i] : mn;
                mx = src[i] > mx ? src[i] : mx;
            }
            float s = (mx - mn) / 15.0f;
            if (!(s > 0.0f)) s = 1.0f;
            const uint16_t s16 = to_f16(s);
            const float sf = from_f16(s16);
            const uint16_t z16 = to_f16(-mn / sf);
            const float zf = from_f16(z16);
            scales[(size_t)r * gpr + g] = s16;
            zeros[(size_t)r * gpr + g] = z16;
            uint32_t* dst = q + ((size_t)r * k + g * group) / 8;
            for (size_t wi = 0; wi < group / 8; wi++) {
                uint32_t word = 0;
                for (int j = 0; j < 8; j++) {
                    float v = std::nearbyint(src[wi * 8 + j] / sf + zf);
                    v = v < 0.0f ? 0.0f : (v > 15.0f ? 15.0f : v);
                    word |= (uint32_t)v << (4 * j);
                }
                dst[wi] = word;
            }
        }
    }
    return QNE_OK;
}

}  // extern "C"
