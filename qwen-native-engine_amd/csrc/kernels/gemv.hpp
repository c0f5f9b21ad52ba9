// Matrix-vector products for batch-1 decode on gfx950 (device side).
//
// Restates the reference's GEMV family (kernels/src/shaders.rs:45-376: gemv, gemv_f16,
// gemv_split_f16 + split_reduce) for MI355X instead of translating it:
//  - one wave64 owns whole rows; each lane streams a contiguous slice of the row with 16-byte
//    loads (a wave reads 1 KiB of a q4 row, or 1 KiB of an f16 row, per instruction), so every
//    row is one coalesced sweep and no LDS tree reduction is needed;
//  - the lane keeps its slice of x in VGPRs for every row it visits (K/64 floats), so x is read
//    once per wave instead of once per row;
//  - int4 nibbles become f32 with v_cvt_f32_ubyte (after two masks per 8 values) and are
//    accumulated in f32 against f32 x, so the result keeps f32 accuracy; per group the lane
//    applies acc += s * (sum q*x - z * sum x);
//  - several rows per wave are loaded before any is reduced, to keep bytes in flight;
//  - the row total is a wave reduction; epilogues Store / Accumulate / SwiGlu (rows r and
//    r + rows/2) and an argmax-tracking Store for the LM head are fused.
// Weight layouts in HBM:
//  - q4: u32 [rows][K/8], value c at bits 4*(c%8) of word c/8 (the file layout); scale and zero
//    interleaved as an f16 pair per group: u32 [rows][K/G] (scale in the low half);
//  - f16: [rows][K].
#pragma once

#include "common.hpp"
#include "launch.hpp"

namespace qne {


// Slab plan of a q4 row of compile-time width K: 2048-column slabs read with 16-byte loads
// (32 values per lane), then at most one 1024-column slab (8-byte loads) and one 512-column slab
// (4-byte loads). K must be a multiple of 512.
template <int K>
struct Q4Plan {
    static_assert(K % 512 == 0, "q4 rows must be a multiple of 512 values");
    static constexpr int N4 = K / 2048;
    static constexpr int N2 = (K % 2048) / 1024;
    static constexpr int N1 = (K % 1024) / 512;
    static constexpr int NS = N4 + N2 + N1;
    static constexpr int CPL = K / 64;  // values per lane
    static constexpr int WPL = K / 512; // u32 words per lane
    __host__ __device__ static constexpr int cols(int s) { return s < N4 ? 32 : (s < N4 + N2 ? 16 : 8); }
    __host__ __device__ static constexpr int base(int s) {
        return s < N4 ? 2048 * s : (s < N4 + N2 ? 2048 * N4 + 1024 * (s - N4) : 2048 * N4 + 1024 * N2 + 512 * (s - N4 - N2));
    }
    __host__ __device__ static constexpr int roff(int s) { return s == 0 ? 0 : roff(s - 1) + cols(s - 1); }
};

// Slab plan of an f16 row: 512-column slabs, 8 values (16 bytes) per lane.
template <int K>
struct F16Plan {
    static_assert(K % 512 == 0, "f16 rows must be a multiple of 512 values");
    static constexpr int NS = K / 512;
    static constexpr int CPL = K / 64;
};

// Lane slice of x (optionally RMS-normalised with `gain`), in the column order of the plan.
// Returns nothing; every lane of the wave must call it (it contains a wave reduction).
template <int KIND, int K>
__device__ __forceinline__ void load_x(const float* __restrict__ x, const float* __restrict__ gain, float eps,
                                       float (&xr)[K / 64], int lane) {
    if constexpr (KIND == KIND_Q4) {
        using P = Q4Plan<K>;
#pragma unroll
        for (int s = 0; s < P::NS; s++) {
            const float* src = x + P::base(s) + P::cols(s) * lane;
#pragma unroll
            for (int i = 0; i < P::cols(s); i += 4) {
                float4 v = *(const float4*)(src + i);
                xr[P::roff(s) + i] = v.x; xr[P::roff(s) + i + 1] = v.y;
                xr[P::roff(s) + i + 2] = v.z; xr[P::roff(s) + i + 3] = v.w;
            }
        }
    } else {
#pragma unroll
        for (int s = 0; s < F16Plan<K>::NS; s++) {
            const float* src = x + 512 * s + 8 * lane;
            float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
            xr[8 * s] = a.x; xr[8 * s + 1] = a.y; xr[8 * s + 2] = a.z; xr[8 * s + 3] = a.w;
            xr[8 * s + 4] = b.x; xr[8 * s + 5] = b.y; xr[8 * s + 6] = b.z; xr[8 * s + 7] = b.w;
        }
    }
    if (gain) {
        // y = x * rsqrt(sum(x^2)/K + eps) * g (kernels/src/shaders.rs:378-403); the lanes of one
        // wave hold all K values, so the sum is a wave reduction.
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < K / 64; i++) ss = fmaf(xr[i], xr[i], ss);
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)K + eps);
        if constexpr (KIND == KIND_Q4) {
            using P = Q4Plan<K>;
#pragma unroll
            for (int s = 0; s < P::NS; s++) {
                const float* gs = gain + P::base(s) + P::cols(s) * lane;
#pragma unroll
                for (int i = 0; i < P::cols(s); i += 4) {
                    float4 g = *(const float4*)(gs + i);
                    const int o = P::roff(s) + i;
                    xr[o] = xr[o] * inv * g.x; xr[o + 1] = xr[o + 1] * inv * g.y;
                    xr[o + 2] = xr[o + 2] * inv * g.z; xr[o + 3] = xr[o + 3] * inv * g.w;
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < F16Plan<K>::NS; s++) {
                const float* gs = gain + 512 * s + 8 * lane;
                float4 a = *(const float4*)gs, b = *(const float4*)(gs + 4);
                const int o = 8 * s;
                xr[o] = xr[o] * inv * a.x; xr[o + 1] = xr[o + 1] * inv * a.y;
                xr[o + 2] = xr[o + 2] * inv * a.z; xr[o + 3] = xr[o + 3] * inv * a.w;
                xr[o + 4] = xr[o + 4] * inv * b.x; xr[o + 5] = xr[o + 5] * inv * b.y;
                xr[o + 6] = xr[o + 6] * inv * b.z; xr[o + 7] = xr[o + 7] * inv * b.w;
            }
        }
    }
}

// Per-slab sums of the lane's x values (the zero-point term of each q4 group).
template <int K>
__device__ __forceinline__ void slab_sums(const float (&xr)[K / 64], float (&xs)[Q4Plan<K>::NS]) {
    using P = Q4Plan<K>;
#pragma unroll
    for (int s = 0; s < P::NS; s++) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < P::cols(s); i++) a += xr[P::roff(s) + i];
        xs[s] = a;
    }
}

// Raw bytes of one row held by one lane.
template <int KIND, int K>
struct RowRaw;
template <int K>
struct RowRaw<KIND_Q4, K> {
    uint32_t w[Q4Plan<K>::WPL];
    uint32_t sz[Q4Plan<K>::NS];
};
template <int K>
struct RowRaw<KIND_F16, K> {
    uint32_t w[K / 128];
};

template <int KIND, int K, int G>
__device__ __forceinline__ void load_row(RowRaw<KIND, K>& r, const void* __restrict__ W, const uint32_t* __restrict__ SZ,
                                         int row, int lane) {
    if constexpr (KIND == KIND_Q4) {
        using P = Q4Plan<K>;
        const uint32_t* wr = (const uint32_t*)W + (size_t)row * (K / 8);
        const uint32_t* sr = SZ + (size_t)row * (K / G);
        int wi = 0;
#pragma unroll
        for (int s = 0; s < P::NS; s++) {
            const int first = P::base(s) + P::cols(s) * lane;
            const uint32_t* src = wr + first / 8;
            if (P::cols(s) == 32) {
                u32x4 v = __builtin_nontemporal_load((const u32x4*)src);
                r.w[wi] = v.x; r.w[wi + 1] = v.y; r.w[wi + 2] = v.z; r.w[wi + 3] = v.w;
                wi += 4;
            } else if (P::cols(s) == 16) {
                u32x2 v = __builtin_nontemporal_load((const u32x2*)src);
                r.w[wi] = v.x; r.w[wi + 1] = v.y;
                wi += 2;
            } else {
                r.w[wi] = __builtin_nontemporal_load(src);
                wi += 1;
            }
            r.sz[s] = sr[first / G];
        }
    } else {
        const u32x4* wr = (const u32x4*)((const uint16_t*)W + (size_t)row * K);
#pragma unroll
        for (int s = 0; s < F16Plan<K>::NS; s++) {
            u32x4 v = __builtin_nontemporal_load(wr + 64 * s + lane);
            r.w[4 * s] = v.x; r.w[4 * s + 1] = v.y; r.w[4 * s + 2] = v.z; r.w[4 * s + 3] = v.w;
        }
    }
}

// sum_{i<8} nibble_i * x[i] for one u32 word of a q4 row.
__device__ __forceinline__ float dot8_q4(uint32_t w, const float* x) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    float a = (float)(lo & 0xFFu) * x[0];
    float b = (float)(hi & 0xFFu) * x[1];
    a = fmaf((float)((lo >> 8) & 0xFFu), x[2], a);
    b = fmaf((float)((hi >> 8) & 0xFFu), x[3], b);
    a = fmaf((float)((lo >> 16) & 0xFFu), x[4], a);
    b = fmaf((float)((hi >> 16) & 0xFFu), x[5], b);
    a = fmaf((float)(lo >> 24), x[6], a);
    b = fmaf((float)(hi >> 24), x[7], b);
    return a + b;
}

// The lane's share of one row's dot product.
template <int KIND, int K>
__device__ __forceinline__ float row_partial(const RowRaw<KIND, K>& r, const float (&xr)[K / 64],
                                             const float* xs) {
    if constexpr (KIND == KIND_Q4) {
        using P = Q4Plan<K>;
        float acc = 0.0f;
        int wi = 0;
#pragma unroll
        for (int s = 0; s < P::NS; s++) {
            float dq = 0.0f;
#pragma unroll
            for (int j = 0; j < P::cols(s) / 8; j++) dq += dot8_q4(r.w[wi + j], &xr[P::roff(s) + 8 * j]);
            wi += P::cols(s) / 8;
            const float sc = lo_h(r.sz[s]), z = hi_h(r.sz[s]);
            acc = fmaf(sc, dq - z * xs[s], acc);
        }
        return acc;
    } else {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int i = 0; i < K / 128; i++) {
            a = fmaf(lo_h(r.w[i]), xr[2 * i], a);
            b = fmaf(hi_h(r.w[i]), xr[2 * i + 1], b);
        }
        return a + b;
    }
}

}  // namespace qne
