// The x operand of the batched GEMM (k_gemm) in memory, and the device helpers that write and read
// it: the kernels that produce a GEMM's input (the embedding, the split reduce, the GDN step, the
// attention combine) stage it directly in this form.
//
// x is staged in chunks of 64 columns for tiles of 64 rows: per chunk the f16 halves hi = f16(x),
// lo = f16(x - hi) in v_mfma_f32_32x32x16_f16 A-operand order, then each row's sum of hi + lo and
// sum of x^2 over the chunk.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace qne {

constexpr int kBM = 64;            // rows of x per GEMM (sequences)
constexpr int kChunk = 64;         // columns per staged chunk
constexpr int kFragBytes = 8192;   // one half (hi or lo) of a chunk: 4 k-steps x 2 row tiles x 64 lanes x 16 B
constexpr int kXsumOff = 2 * kFragBytes;           // per-row sums of hi + lo over the chunk
constexpr int kSsOff = kXsumOff + kBM * 4;           // per-row sums of x^2 (raw x) over the chunk
constexpr int kChunkBytes = kSsOff + kBM * 4;        // a staged chunk in memory

// Operand layout of v_mfma_f32_32x32x16_f16 (lane l): A[l % 32][8 (l / 32) + i], B[8 (l / 32) + i][l % 32],
// D register j = [8 (j / 4) + 4 (l / 32) + j % 4][l % 32]. The 16 k-slots of k-step s of a chunk are
// chunk columns 32 (l / 32) + 8 s + i, the same for A and B, so a lane's q4 bytes of a chunk (16) are
// contiguous. In a staged chunk, fragment (s, row tile mt) of a half is 64 lanes x 16 bytes.
__device__ __forceinline__ int frag_offset(int s, int mt, int lane) { return ((s * 2 + mt) * 64 + lane) * 16; }

// Writes one value of the x operand of a GEMM: row r, column c, value v (times gain g). The 64
// lanes of the calling wave hold the 64 columns of one chunk of row r (all lanes call it), so the
// chunk's sums of hi + lo and of v^2 are wave sums. q4order: the column order of the q4 GEMM's B
// operand within each 8 columns, [0, 4, 1, 5, 2, 6, 3, 7] (nibbles8); else natural. Rows come in
// tiles of 64: tile r / 64 of the operand starts tile_bytes (the K / 64 chunks of one tile) after
// the previous one.
__device__ __forceinline__ void emit_x(uint8_t* __restrict__ frag, size_t tile_bytes, int r, int c, float v, float g,
                                       int q4order, int lane) {
    const float xg = v * g;
    const float hi = (float)(_Float16)xg;
    const float lo = (float)(_Float16)(xg - hi);
    const int chunk = c / kChunk, kk = c % kChunk, hf = kk / 32, st = (kk % 32) / 8, i = kk % 8;
    const int slot = q4order ? 2 * (i % 4) + i / 4 : i;
    const int rr = r & (kBM - 1);
    uint8_t* tile = frag + (size_t)(r / kBM) * tile_bytes + (size_t)chunk * kChunkBytes;
    uint8_t* dst = tile + frag_offset(st, rr >> 5, 32 * hf + (rr & 31)) + 2 * slot;
    *(uint16_t*)dst = __builtin_bit_cast(uint16_t, (_Float16)hi);
    *(uint16_t*)(dst + kFragBytes) = __builtin_bit_cast(uint16_t, (_Float16)lo);
    const float xs = wave_sum_dpp(hi + lo), ss = wave_sum_dpp(v * v);
    if (lane == 0) {
        float* sums = (float*)tile;
        sums[kXsumOff / 4 + rr] = xs;
        sums[kSsOff / 4 + rr] = ss;
    }
}

// 1 / rms of row r from the staged chunk sums of x^2 (the RMSNorm of the GEMM's input, applied to
// its output: y = (1 / rms) W (x * gain)). Called by every one of the NT threads of the workgroup
// (a multiple of 256: with K <= 16384 the wave sums and their order are those of a 256-thread
// workgroup, the waves past the fourth adding zeros).
template <int NT>
__device__ __forceinline__ float row_inv_rms(const uint8_t* __restrict__ frag, int nchunks, int K, float eps, int r,
                                             float* red) {
    const uint8_t* tile = frag + (size_t)(r / kBM) * nchunks * kChunkBytes;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < nchunks; c += NT) ss += ((const float*)(tile + (size_t)c * kChunkBytes))[kSsOff / 4 + (r & (kBM - 1))];
    ss = block_sum<NT>(ss, red);
    return 1.0f / sqrtf(ss / (float)K + eps);
}

// Up to 8 split partials of one output value in flight at once, summed in split order (the order
// of k_gemm_reduce: terms past the splits are +0 and leave the sum unchanged).
constexpr int kFoldSplits = 8;
struct Split8 {
    float v[kFoldSplits];
    __device__ __forceinline__ void load(const float* p, int splits, size_t stride) {
#pragma unroll
        for (int s = 0; s < kFoldSplits; s++) v[s] = s < splits ? p[s * stride] : 0.0f;
    }
    __device__ __forceinline__ float sum(const float* p, int splits, size_t stride) const {
        float g = v[0];
#pragma unroll
        for (int s = 1; s < kFoldSplits; s++) g += v[s];
        for (int s = kFoldSplits; s < splits; s++) g += p[s * stride];
        return g;
    }
};

}  // namespace qne
