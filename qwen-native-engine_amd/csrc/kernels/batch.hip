// Batched decode (up to 64 sequences per step): the GEMM that replaces the GEMV, and the small
// per-row kernels around it.
//
// Reference: the 16-token prefill GEMM `gemm` (kernels/src/batch.rs:12-99, launched by `Gpu::gemm`,
// lib.rs:341-347) and its embed / argmax companions (shaders.rs:405-434, 635-699), generalised to M
// rows of one decode step each. Design for gfx950:
//  - the x operand (f32 activations, times the RMSNorm gain when the matrix follows a norm) is
//    written once per GEMM as f16 halves hi = f16(x), lo = f16(x - hi), already in
//    v_mfma_f32_32x32x16_f16 operand order, with each row's sums of hi + lo and of x^2 over every
//    64-column chunk: two MFMAs (hi, lo) reproduce f32 products to about 2^-22. The kernels that
//    produce an activation write it (the reduce kernels, the embedding); k_stage_x does it for the
//    others. The norm's 1 / rms is a per-row scalar, applied to the GEMM's output from the sums of
//    x^2;
//  - k_gemm: a workgroup (4 or 8 waves) computes a 64 x (32 waves) tile of y = x W^T over a slice
//    of K (split-K). x chunks and W chunks stream into a ring of LDS slots by LDS DMA
//    (global_load_lds) with explicit vmcnt waits, so the compiler inserts no waits that would drain
//    the pipeline;
//  - q4 weights are dequantised in registers as exact f16 integers (0x6400 | q is 1024 + q, minus
//    1024 is exact); every chunk's sum is scaled once: y += s (sum q x) - s z (sum x), with sum x
//    from the staged chunk sums. f16 weights go to the MFMA as they are;
//  - with one split the GEMM applies the epilogue itself; otherwise it writes partials and
//    k_gemm_reduce sums them in split order (so the result does not depend on timing) and applies
//    the epilogue (store, residual add, SwiGLU).
#include <algorithm>

#include "../error.hpp"
#include "common.hpp"
#include "launch.hpp"
#include "lds_dma.hpp"
#include "operand.hpp"

namespace qne {

namespace {

using namespace lds_dma;


typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// The 8 nibbles of a q4 word (nibble i at bits 4i: column 8j + i of word j) as exact f16 values, in
// the order [q0, q4, q1, q5, q2, q6, q3, q7]: 0x6400 | q is the f16 1024 + q, and 0x6400 | (q << 4)
// is 1024 + 16 q, so four and-or, one shift, two packed subtracts and two packed fmas (x / 16 - 64)
// give all eight. The x operand of a q4 GEMM is staged in the same column order.
__device__ __forceinline__ half8_t nibbles8(uint32_t v) {
    typedef uint32_t u32;
    const u32 v2 = v >> 8;
    const u32 t0 = (v & 0x000F000Fu) | 0x64006400u;
    const u32 t1 = (v & 0x00F000F0u) | 0x64006400u;
    const u32 t2 = (v2 & 0x000F000Fu) | 0x64006400u;
    const u32 t3 = (v2 & 0x00F000F0u) | 0x64006400u;
    const half2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const half2_t k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const half2_t k64 = {(_Float16)-64.0f, (_Float16)-64.0f};
    const half2_t h0 = __builtin_bit_cast(half2_t, t0) - k1024;
    const half2_t h1 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t1), k16, k64);
    const half2_t h2 = __builtin_bit_cast(half2_t, t2) - k1024;
    const half2_t h3 = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, t3), k16, k64);
    return half8_t{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
}
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

}  // namespace

// Grid (ceil(K / 256), rows rounded up to 64): the x operand of a GEMM from f32 rows
// (x + r * x_stride; rows >= m are zero), times `gain` when set; the row's RMSNorm factor is applied
// by the GEMM's epilogue.
__global__ __launch_bounds__(256) void k_stage_x(const float* __restrict__ x, int x_stride, int m, int K,
                                                 const float* __restrict__ gain, int q4order, uint8_t* __restrict__ frag) {
    const int c = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (blockIdx.x * 256 >= K) return;  // whole workgroup; K is a multiple of 64, so waves are whole chunks
    if ((threadIdx.x & ~63) + blockIdx.x * 256 >= K) return;  // whole wave
    const float v = r < m ? x[(size_t)r * x_stride + c] : 0.0f;
    emit_x(frag, (size_t)(K / kChunk) * kChunkBytes, r, c, v, gain ? gain[c] : 1.0f, q4order, threadIdx.x & 63);
}

// Until at most n of the wave's vector-memory operations are outstanding (n wave-uniform; counts
// past 31 wait for 31, which is only stricter).
__device__ __forceinline__ void wait_vm_upto(int n) {
    switch (n < 31 ? n : 31) {
#define QNE_WAIT_CASE(k) \
    case k: wait_vm<k>(); break;
        QNE_WAIT_CASE(0) QNE_WAIT_CASE(1) QNE_WAIT_CASE(2) QNE_WAIT_CASE(3) QNE_WAIT_CASE(4) QNE_WAIT_CASE(5)
        QNE_WAIT_CASE(6) QNE_WAIT_CASE(7) QNE_WAIT_CASE(8) QNE_WAIT_CASE(9) QNE_WAIT_CASE(10) QNE_WAIT_CASE(11)
        QNE_WAIT_CASE(12) QNE_WAIT_CASE(13) QNE_WAIT_CASE(14) QNE_WAIT_CASE(15) QNE_WAIT_CASE(16) QNE_WAIT_CASE(17)
        QNE_WAIT_CASE(18) QNE_WAIT_CASE(19) QNE_WAIT_CASE(20) QNE_WAIT_CASE(21) QNE_WAIT_CASE(22) QNE_WAIT_CASE(23)
        QNE_WAIT_CASE(24) QNE_WAIT_CASE(25) QNE_WAIT_CASE(26) QNE_WAIT_CASE(27) QNE_WAIT_CASE(28) QNE_WAIT_CASE(29)
        QNE_WAIT_CASE(30)
#undef QNE_WAIT_CASE
        default: wait_vm<31>();
    }
}

// Grid (ceil(N / (32 WAVES CF)), splits, row tiles); split s covers chunks [s * cps, (s + 1) * cps)
// of the x rows 64 blockIdx.z .. + 63. The workgroup's W rows come in TW = WAVES CF tiles of 32;
// compute wave w < WAVES owns tiles w CF .. w CF + CF - 1, so every A fragment it reads from LDS
// feeds CF MFMAs. The chunks stream through a ring of D LDS slots, each holding one x chunk and
// every W tile's chunk; D - 1 chunks are in flight while one is computed. With DW > 0 the workgroup
// has DW more waves that only issue the LDS DMA (x, chunk sums, every W tile), so a compute wave's
// instruction stream holds LDS reads, MFMAs and VALU only and the transfers overlap the
// computation; with DW = 0 every compute wave sends a share of the W tiles and of x. The row tiles
// of one W tile read the same W chunks, which the MALL serves after the first.
// Epilogues: partials (split-K, or an epilogue the GEMM does not apply); `direct` (one split: store
// or residual add); `fuse` 1 (one split, SwiGLU): tiles [0, TW / 2) are gate rows and [TW / 2, TW)
// the matching up rows (n_out further), and the workgroup writes silu(gate) * up and stages it as
// the next GEMM's operand; `fuse` 2 (one split, store or residual add with the result staged as the
// next GEMM's operand). Both compute exactly what k_gemm_reduce does with one split.
template <int KIND, int WAVES, int D, int DW, int CF>
__global__ __launch_bounds__(64 * (WAVES + DW)) void k_gemm(const GemmArgs a) {
    constexpr int TW = WAVES * CF;                                  // 32-row W tiles per workgroup
    // A ring slot: the x chunk's fragments (hi, lo), every W tile's chunk (1 KiB q4 or 4 KiB f16),
    // then (q4) the x chunk's 64 row sums (256 B) and every tile's 32 scale/zero words (128 B
    // each). A sender copies its tiles' words with one 16-byte-per-lane DMA from the tile-major
    // copy (8 lanes a tile), the first sender the row sums in the same DMA (16 lanes in front):
    // every workgroup of a row tile reads those two lines at about the same time, and 4-byte
    // lanes would make 4x the requests to them (measured: -9 % GEMM time). An LDS DMA costs its
    // issuing wave about the same however little it moves, so this adds none. The f16 GEMM needs
    // no row sums.
    constexpr int kWTile = KIND == KIND_Q4 ? 1024 : 4096;           // one W tile's chunk
    constexpr int kSzOff = 2 * kFragBytes + TW * kWTile;            // q4: row sums, then words
    constexpr int kSlot = kSzOff + (KIND == KIND_Q4 ? 256 + TW * 128 : 0);
    constexpr int kSenders = DW > 0 ? DW : WAVES;                   // waves that issue the DMA
    constexpr int kXPart = 2 * kFragBytes / kSenders;               // x bytes each sender copies
    constexpr int kTilesPer = TW / kSenders;                        // W tiles each sender sends
    constexpr int kWDmas = KIND == KIND_Q4 ? 1 : 4;                 // DMAs of one W tile chunk
    static_assert(kXPart % 1024 == 0 && TW % kSenders == 0, "the senders split x and W evenly");
    static_assert(16 + 8 * kTilesPer <= 64, "the first sender's words DMA holds the row sums and its tiles");
    // DMAs per sender per chunk: its x part, its W tiles, (q4) its tiles' words (+ row sums)
    constexpr int kPer = kXPart / 1024 + kTilesPer * kWDmas + (KIND == KIND_Q4 ? 1 : 0);
    __shared__ __attribute__((aligned(16))) uint8_t ring[D][kSlot];
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool computes = w < WAVES;
    const int sender = DW > 0 ? w - WAVES : w;  // index among the senders (< 0: none)
    const int hf = lane >> 5, l32 = lane & 31;
    const int K = a.K, nchunks = K / kChunk;
    const int cpg = KIND == KIND_Q4 ? a.group / kChunk : 1;
    const int ngroups = nchunks / cpg;
    const int c0 = blockIdx.y * a.cps, c1 = min(nchunks, c0 + a.cps);
    const int nch = max(0, c1 - c0);
    const int mt = blockIdx.z;  // row tile
    const uint8_t* xfrag = a.frag + (size_t)mt * nchunks * kChunkBytes;
    // first W row (= output column) of tile t of this workgroup; lane l32 has row + l32
    auto wrow0 = [&](int t) -> int {
        constexpr int half = TW / 2;
        if (a.fuse == 1) return t < half ? (blockIdx.x * half + t) * 32 : a.n_out + (blockIdx.x * half + t - half) * 32;
        return (blockIdx.x * TW + t) * 32;
    };
    auto wrow = [&](int t) -> int { return wrow0(t) + l32; };

    auto issue = [&](int j, int slot) {  // senders only
        uint8_t* base = ring[slot];
        const uint8_t* src = xfrag + (size_t)(c0 + j) * kChunkBytes;
#pragma unroll
        for (int u = 0; u < kXPart / 1024; u++) dma16(src + kXPart * sender + 1024 * u + 16 * lane, base + kXPart * sender + 1024 * u);
        const int c = c0 + j;
#pragma unroll
        for (int i = 0; i < kTilesPer; i++) {
            const int wt = sender * kTilesPer + i;  // W tile sent
            const int nr = min(wrow(wt), a.N - 1);  // rows past N: row N - 1, not stored
            uint8_t* dst = base + 2 * kFragBytes + wt * kWTile;
            if (KIND == KIND_Q4) {
                dma16((const uint8_t*)a.W + (size_t)nr * (K / 2) + c * 32 + 16 * hf, dst);
            } else {
#pragma unroll
                for (int s = 0; s < 4; s++) dma16((const uint16_t*)a.W + (size_t)nr * K + c * kChunk + 32 * hf + 8 * s, dst + 1024 * s);
            }
        }
        if (KIND == KIND_Q4) {
            // lanes [0, lead): row sums (first sender); then 8 lanes (16 B of words) per tile
            const int lead = sender == 0 ? 16 : 0, li = lane - lead;
            if (lane < lead + 8 * kTilesPer) {
                const int t = sender * kTilesPer + (li >> 3);
                const int tb = min(wrow0(t), a.N - 1) >> 5;  // tiles past N: the last one, not stored
                const void* sp = lane < lead ? (const void*)(src + kXsumOff + 16 * lane)
                                             : (const void*)(a.SZT + ((size_t)tb * ngroups + c / cpg) * 32 + 4 * (li & 7));
                dma16(sp, base + kSzOff + (sender == 0 ? 0 : 256 + 128 * kTilesPer * sender));
            }
        }
    };
    static_assert(D >= 2 && (D - 2) * kPer <= 31, "ring deeper than the waits cover");

    float16_t acc[CF][2], grp[CF][2];
#pragma unroll
    for (int cf = 0; cf < CF; cf++)
#pragma unroll
        for (int j = 0; j < 16; j++) acc[cf][0][j] = acc[cf][1][j] = grp[cf][0][j] = grp[cf][1][j] = 0.0f;

    if (sender >= 0)
        for (int j = 0; j < min(D - 1, nch); j++) issue(j, j);
    int slot = 0;           // slot of chunk j
    int next_slot = D - 1;  // slot of chunk j + D - 1
    for (int j = 0; j < nch; j++) {
        if (sender >= 0) wait_vm_upto(kPer * (min(j + D - 2, nch - 1) - j));  // this sender's part of chunk j is in
        __syncthreads();  // every part of chunk j has landed; every wave is done with chunk j - 1
        if (sender >= 0 && j + D - 1 < nch) issue(j + D - 1, next_slot);
        if (computes) {
            const uint8_t* xs = ring[slot];
            const uint8_t* ws = ring[slot] + 2 * kFragBytes + w * CF * kWTile;
            const uint8_t* wsz = ring[slot] + kSzOff + 256 + w * CF * 128;
            uint4 wq[CF];
            if (KIND == KIND_Q4)
#pragma unroll
                for (int cf = 0; cf < CF; cf++) wq[cf] = *(const uint4*)(ws + cf * kWTile + 16 * lane);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const half8_t a0h = *(const half8_t*)(xs + frag_offset(s, 0, lane));
                const half8_t a1h = *(const half8_t*)(xs + frag_offset(s, 1, lane));
                const half8_t a0l = *(const half8_t*)(xs + kFragBytes + frag_offset(s, 0, lane));
                const half8_t a1l = *(const half8_t*)(xs + kFragBytes + frag_offset(s, 1, lane));
#pragma unroll
                for (int cf = 0; cf < CF; cf++) {
                    half8_t b;
                    if (KIND == KIND_Q4) b = nibbles8(s == 0 ? wq[cf].x : s == 1 ? wq[cf].y : s == 2 ? wq[cf].z : wq[cf].w);
                    else b = *(const half8_t*)(ws + cf * kWTile + 1024 * s + 16 * lane);
                    if (KIND == KIND_Q4 && s == 0) {  // a fresh tile per chunk: C = 0
                        const float16_t zero = {};
                        grp[cf][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0h, b, zero, 0, 0, 0);
                        grp[cf][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1h, b, zero, 0, 0, 0);
                    } else {
                        grp[cf][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0h, b, grp[cf][0], 0, 0, 0);
                        grp[cf][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1h, b, grp[cf][1], 0, 0, 0);
                    }
                    grp[cf][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0l, b, grp[cf][0], 0, 0, 0);
                    grp[cf][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1l, b, grp[cf][1], 0, 0, 0);
                }
            }
            if (KIND == KIND_Q4) {
                // y += s (sum q x) - s z (sum x) over the chunk (scale and zero of the chunk's group)
                const float* xsum0 = (const float*)(xs + kSzOff);  // rows 0..31
                const float* xsum1 = xsum0 + 32;                     // rows 32..63
#pragma unroll
                for (int cf = 0; cf < CF; cf++) {
                    const uint32_t szw = *(const uint32_t*)(wsz + cf * 128 + 4 * l32);
                    const float sc = lo_h(szw), sz = sc * hi_h(szw);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 s0 = *(const float4*)(xsum0 + 8 * q + 4 * hf);
                        const float4 s1 = *(const float4*)(xsum1 + 8 * q + 4 * hf);
                        const float v0[4] = {s0.x, s0.y, s0.z, s0.w}, v1[4] = {s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            acc[cf][0][4 * q + e] = fmaf(sc, grp[cf][0][4 * q + e], fmaf(-sz, v0[e], acc[cf][0][4 * q + e]));
                            acc[cf][1][4 * q + e] = fmaf(sc, grp[cf][1][4 * q + e], fmaf(-sz, v1[e], acc[cf][1][4 * q + e]));
                        }
                    }
                }
            }
        }
        slot = slot + 1 == D ? 0 : slot + 1;
        next_slot = next_slot + 1 == D ? 0 : next_slot + 1;
    }
    if (KIND != KIND_Q4) {
#pragma unroll
        for (int cf = 0; cf < CF; cf++) {
            acc[cf][0] = grp[cf][0];
            acc[cf][1] = grp[cf][1];
        }
    }
    if (!a.direct && !a.fuse) {
        if (!computes) return;
#pragma unroll
        for (int cf = 0; cf < CF; cf++) {
            const int n = wrow(w * CF + cf);
            if (n >= a.N) continue;
            float* pp = a.part + ((size_t)blockIdx.y * a.mpad + (size_t)kBM * mt) * a.N + n;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int m = 8 * (j / 4) + 4 * hf + (j % 4);
                store_through(pp + (size_t)m * a.N, acc[cf][0][j]);
                store_through(pp + (size_t)(32 + m) * a.N, acc[cf][1][j]);
            }
        }
        return;
    }
    // one split: 1 / rms of the rows (normed input), then the epilogue
    float* sinv = (float*)ring[0];
    __syncthreads();  // ring no longer read
    if (a.fuse) {
        // as k_gemm_reduce computes it (row_inv_rms<256>), so the result is the same: with at most
        // 64 chunks the first wave's lanes hold one chunk each and the other waves add +0, so the
        // sum is one wave_sum; every row's loads are in flight at once
        if (computes) {
            constexpr int kRows = kBM / WAVES;  // rows per wave
            float v[kRows];
#pragma unroll
            for (int j = 0; j < kRows; j++)
                v[j] = a.norm && lane < nchunks ? ((const float*)(xfrag + (size_t)lane * kChunkBytes))[kSsOff / 4 + w + WAVES * j] : 0.0f;
#pragma unroll
            for (int j = 0; j < kRows; j++) {
                const float inv = a.norm ? 1.0f / sqrtf(wave_sum(v[j]) / (float)K + a.eps) : 1.0f;
                if (lane == 0) sinv[w + WAVES * j] = inv;
            }
        }
    } else if (a.norm) {
        if (threadIdx.x < kBM) {
            float ss = 0.0f;
            for (int c = 0; c < nchunks; c++) ss += ((const float*)(xfrag + (size_t)c * kChunkBytes))[kSsOff / 4 + threadIdx.x];
            sinv[threadIdx.x] = 1.0f / sqrtf(ss / (float)K + a.eps);
        }
    } else if (threadIdx.x < kBM) {
        sinv[threadIdx.x] = 1.0f;
    }
    __syncthreads();
    const int rows = a.m - kBM * mt;  // rows of this tile
    if (a.direct) {
        if (!computes) return;
#pragma unroll
        for (int cf = 0; cf < CF; cf++) {
            const int n = wrow(w * CF + cf);
            if (n >= a.N) continue;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int m = 8 * (j / 4) + 4 * hf + (j % 4);
                if (m < rows) {
                    float* d = a.y + (size_t)(kBM * mt + m) * a.y_stride + n;
                    const float v = acc[cf][0][j] * sinv[m];
                    store_through(d, a.epi == EPI_ACCUMULATE ? *d + v : v);
                }
                if (32 + m < rows) {
                    float* d = a.y + (size_t)(kBM * mt + 32 + m) * a.y_stride + n;
                    const float v = acc[cf][1][j] * sinv[32 + m];
                    store_through(d, a.epi == EPI_ACCUMULATE ? *d + v : v);
                }
            }
        }
        return;
    }
    if (a.fuse == 2) {
        // the tile through LDS ([row][column]) times the rows' 1 / rms, then every wave takes whole
        // 64-column chunks of rows (lanes = columns): residual add or store, and the staged operand
        constexpr int kOut = TW * 32;  // output columns of the workgroup
        static_assert(kOut % kChunk == 0 && (kBM * kOut + kBM) * 4 <= D * kSlot, "fused epilogue tile");
        float* so = sinv + kBM;  // [kBM][kOut]
        if (computes) {
#pragma unroll
            for (int cf = 0; cf < CF; cf++) {
                const int col = (w * CF + cf) * 32 + l32;
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const int m = 8 * (j / 4) + 4 * hf + (j % 4);
                    so[m * kOut + col] = acc[cf][0][j] * sinv[m];
                    so[(32 + m) * kOut + col] = acc[cf][1][j] * sinv[32 + m];
                }
            }
        }
        __syncthreads();
        if (!computes) return;
        constexpr int nck = kOut / kChunk;
        constexpr int kIt = kBM * nck / WAVES;  // (row, chunk) items per wave: item w + WAVES q
        static_assert(kBM * nck % WAVES == 0, "fused epilogue items");
        const size_t tile_bytes = (size_t)(a.n_out / kChunk) * kChunkBytes;
        const int nrow = min(rows, kBM), col0 = blockIdx.x * kOut;
        // every item's residual and gain loads in flight before the first is used
        float hv[kIt], gv[kIt];
#pragma unroll
        for (int q = 0; q < kIt; q++) {
            const int it = w + WAVES * q, r = it / nck, ch = it % nck, c = col0 + ch * kChunk + lane;
            const bool live = r < nrow && col0 + ch * kChunk < a.n_out;  // else a whole chunk past the outputs
            hv[q] = live && a.epi == EPI_ACCUMULATE ? a.y[(size_t)(kBM * mt + r) * a.y_stride + c] : 0.0f;
            gv[q] = live && a.gain_out ? a.gain_out[c] : 1.0f;
        }
#pragma unroll
        for (int q = 0; q < kIt; q++) {
            const int it = w + WAVES * q, r = it / nck, ch = it % nck, c = col0 + ch * kChunk + lane;
            if (r >= nrow || col0 + ch * kChunk >= a.n_out) continue;  // wave-uniform
            const float g = so[r * kOut + ch * kChunk + lane];
            const float v = a.epi == EPI_ACCUMULATE ? hv[q] + g : g;
            if (a.y) store_through(a.y + (size_t)(kBM * mt + r) * a.y_stride + c, v);
            emit_x(a.frag_out, tile_bytes, kBM * mt + r, c, v, gv[q], a.order_out, lane);
        }
        return;
    }
    // fused SwiGLU: the up tiles go through LDS ([row][column of the workgroup's gate columns]),
    // the gate tiles' lanes form silu(g / rms) * (u / rms) in place, then every wave stages whole
    // 64-column chunks of rows (lanes = columns), as the reduce does
    constexpr int kCols = TW / 2 * 32;  // output columns of the workgroup
    static_assert(kCols % kChunk == 0 && (kBM * kCols + kBM) * 4 <= D * kSlot, "fused SwiGLU tile");
    float* sv = sinv + kBM;  // [kBM][kCols]
    if (computes) {
#pragma unroll
        for (int cf = 0; cf < CF; cf++) {
            const int t = w * CF + cf;
            if (t < TW / 2) continue;
            const int col = (t - TW / 2) * 32 + l32;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int m = 8 * (j / 4) + 4 * hf + (j % 4);
                sv[m * kCols + col] = acc[cf][0][j];
                sv[(32 + m) * kCols + col] = acc[cf][1][j];
            }
        }
    }
    __syncthreads();
    if (computes) {
#pragma unroll
        for (int cf = 0; cf < CF; cf++) {
            const int t = w * CF + cf;
            if (t >= TW / 2) continue;
            const int col = t * 32 + l32;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int m = 8 * (j / 4) + 4 * hf + (j % 4);
                sv[m * kCols + col] = silu(acc[cf][0][j] * sinv[m]) * (sv[m * kCols + col] * sinv[m]);
                sv[(32 + m) * kCols + col] = silu(acc[cf][1][j] * sinv[32 + m]) * (sv[(32 + m) * kCols + col] * sinv[32 + m]);
            }
        }
    }
    __syncthreads();
    if (!computes) return;
    constexpr int nck = kCols / kChunk;
    const size_t tile_bytes = (size_t)(a.n_out / kChunk) * kChunkBytes;
    for (int it = w; it < min(rows, kBM) * nck; it += WAVES) {  // wave-uniform
        const int r = it / nck, ch = it % nck;
        const int c = blockIdx.x * kCols + ch * kChunk + lane;
        const float v = sv[r * kCols + ch * kChunk + lane];
        if (a.y) store_through(a.y + (size_t)(kBM * mt + r) * a.y_stride + c, v);
        if (a.frag_out) emit_x(a.frag_out, tile_bytes, kBM * mt + r, c, v, a.gain_out ? a.gain_out[c] : 1.0f, a.order_out, lane);
    }
}

// Grid (ceil(n_out / 256), m). Output row r, columns c < n_out, from the split partials summed in
// split order, times 1 / rms of the row when the GEMM's input was normed: store, residual add, or
// SwiGLU silu(gate) * up with gate = column c and up = column c + n_out (matrix rows [gate; up],
// shaders.rs gemv epilogues). With frag_out, the result (times gain_out) is also written as the x
// operand of the next GEMM (n_out is a multiple of 64, so every wave holds whole chunks).
__global__ __launch_bounds__(256) void k_gemm_reduce(const GemmArgs a) {
    __shared__ float red[16];
    const int c = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    const bool wave_live = (threadIdx.x & ~63) + blockIdx.x * 256 < a.n_out;  // false: whole waves past the outputs
    const bool live = c < a.n_out;
    // The partials' loads go first and the row's sums of x^2 (1 / rms, a workgroup sum) after
    // them, so the two round trips overlap; the arithmetic and its order are unchanged.
    float* d = a.y && live ? a.y + (size_t)r * a.y_stride + c : nullptr;
    const float* p = a.part + (size_t)r * a.N + c;
    const size_t ss = (size_t)a.mpad * a.N;  // between splits
    // every split's load in flight at once (up to kSplitsInFlight), then the sum in split order
    constexpr int kSplitsInFlight = 24;
    const bool swiglu = a.epi == EPI_SWIGLU;
    float gv[kSplitsInFlight], uv[kSplitsInFlight], hv = 0.0f;
#pragma unroll
    for (int s = 0; s < kSplitsInFlight; s++) {
        gv[s] = live && s < a.splits ? p[s * ss] : 0.0f;
        uv[s] = live && s < a.splits && swiglu ? p[s * ss + a.n_out] : 0.0f;
    }
    if (live && a.epi == EPI_ACCUMULATE) hv = *d;
    const float inv = a.norm ? row_inv_rms<256>(a.frag, a.K / kChunk, a.K, a.eps, r, red) : 1.0f;
    if (!wave_live) return;
    float v = 0.0f;
    if (live) {
        float g = gv[0], u = uv[0];  // a.splits >= 1
#pragma unroll
        for (int s = 1; s < kSplitsInFlight; s++) {  // past a.splits the terms are +0: g and u unchanged
            g += gv[s];
            u += uv[s];
        }
        for (int s = kSplitsInFlight; s < a.splits; s++) {
            g += p[s * ss];
            if (swiglu) u += p[s * ss + a.n_out];
        }
        g *= inv;
        u *= inv;
        if (a.epi == EPI_STORE) v = g;
        else if (a.epi == EPI_ACCUMULATE) v = hv + g;
        else v = silu(g) * u;
        if (d) store_through(d, v);
    }
    if (a.frag_out)
        emit_x(a.frag_out, (size_t)(a.n_out / kChunk) * kChunkBytes, r, c, v, a.gain_out ? a.gain_out[live ? c : 0] : 1.0f,
               a.order_out, threadIdx.x & 63);
}

// h[r] = embedding row tokens[r] (f16 row, or q4 values (q - z) s), shaders.rs:405-434 per row.
// Grid (ceil(hidden / 256), m). With frag, h * gain is also written as the x operand of the first
// GEMM.
__global__ __launch_bounds__(256) void k_embed_rows(int kind, const void* __restrict__ W, const uint32_t* __restrict__ SZ,
                                                    int group, int hidden, const uint32_t* __restrict__ tokens,
                                                    float* __restrict__ h, uint8_t* __restrict__ frag,
                                                    const float* __restrict__ gain, int q4order,
                                                    const int32_t* __restrict__ pos, int32_t* __restrict__ order) {
    const int r = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
    if (order && blockIdx.x == 0 && blockIdx.y == 0 && (int)threadIdx.x < (int)gridDim.y) {
        // rank of row t by decreasing position, ties to the lower row
        const int t = threadIdx.x, m = gridDim.y;
        const int pt = pos[t];
        int rank = 0;
        for (int u = 0; u < m; u++) {
            const int pu = pos[u];
            rank += pu > pt || (pu == pt && u < t);
        }
        order[rank] = t;
    }
    if ((threadIdx.x & ~63) + blockIdx.x * 256 >= hidden) return;  // whole waves
    const size_t tok = tokens[r];
    float v;
    if (kind == KIND_F16) {
        v = h2f(((const uint16_t*)W)[tok * hidden + c]);
    } else {
        const uint32_t word = ((const uint32_t*)W)[tok * (hidden / 8) + c / 8];
        const uint32_t sz = SZ[tok * (hidden / group) + c / group];
        v = ((float)((word >> (4 * (c % 8))) & 15u) - hi_h(sz)) * lo_h(sz);
    }
    store_through(h + (size_t)r * hidden + c, v);
    if (frag) emit_x(frag, (size_t)(hidden / kChunk) * kChunkBytes, r, c, v, gain ? gain[c] : 1.0f, q4order, threadIdx.x & 63);
}

// Greedy pick of every logits row (argmax_partial / argmax_final, shaders.rs:635-699): the largest
// value, ties to the lower index (a NaN never wins). Pass 1, grid (kArgParts, m): the best of each
// 1/kArgParts of a row. Pass 2, one wave per row: the best of the parts, in part order; with
// `tokens`, row r's pick becomes its next token and its position advances (pos[r] += 1), so decode
// steps chain on the device.
constexpr int kArgParts = 32;

__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ logits, int V, float* __restrict__ pv,
                                                     uint32_t* __restrict__ pi) {
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    const int part = blockIdx.x, r = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int per = (V + kArgParts - 1) / kArgParts, c0 = part * per, c1 = min(V, c0 + per);
    const float* row = logits + (size_t)r * V;
    float best = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (int c = c0 + t; c < c1; c += 256) {
        const float v = row[c];
        if (better(v, (uint32_t)c, best, bi)) {
            best = v;
            bi = (uint32_t)c;
        }
    }
#pragma unroll
    for (int mk = 32; mk >= 1; mk >>= 1) {
        const float ov = __shfl_xor(best, mk, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, mk, 64);
        if (better(ov, oi, best, bi)) {
            best = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        sv[w] = best;
        si[w] = bi;
    }
    __syncthreads();
    if (t == 0) {
        float b = sv[0];
        uint32_t bix = si[0];
        for (int i = 1; i < 4; i++)
            if (better(sv[i], si[i], b, bix)) {
                b = sv[i];
                bix = si[i];
            }
        pv[r * kArgParts + part] = b;
        pi[r * kArgParts + part] = bix;
    }
}

__global__ __launch_bounds__(64) void k_argmax_final(const float* __restrict__ pv, const uint32_t* __restrict__ pi,
                                                     uint32_t* __restrict__ out, uint32_t* __restrict__ tokens,
                                                     int32_t* __restrict__ pos) {
    const int r = blockIdx.x, lane = threadIdx.x;
    float best = lane < kArgParts ? pv[r * kArgParts + lane] : -INFINITY;
    uint32_t bi = lane < kArgParts ? pi[r * kArgParts + lane] : 0xFFFFFFFFu;
#pragma unroll
    for (int mk = 32; mk >= 1; mk >>= 1) {
        const float ov = __shfl_xor(best, mk, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, mk, 64);
        if (better(ov, oi, best, bi)) {
            best = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        const uint32_t pick = bi == 0xFFFFFFFFu ? 0u : bi;  // all NaN: token 0
        if (out) out[r] = pick;
        if (tokens) {
            tokens[r] = pick;
            pos[r] += 1;
        }
    }
}

// Workgroup width: 8 waves (256 W rows) for q4 and wide f16 matrices, else 4 (128 rows). At the
// 2B model's M = 64 shapes (W streamed from HBM), 8 waves with a 3-deep ring (two workgroups fit a
// CU) beat 4 waves by 8-20 % including the reduce.
static int gemm_waves(int kind, int N) { return kind == KIND_Q4 || N > 4096 ? 8 : 4; }

int gemm_splits(int kind, int N, int K, int group, int row_tiles) {
    (void)group;
    const int waves = gemm_waves(kind, N);
    const int tiles = (N + 32 * waves - 1) / (32 * waves) * std::max(1, row_tiles);
    const int nch = K / kChunk;
    // as many splits as keep the grid within one workgroup per CU (a second one on a CU shares its
    // chunk throughput), at least 2 chunks per split, at most 24 (the reduce reads every split's
    // 64 x N partials)
    int splits = std::min(256 / tiles, std::min(24, nch / 2));
    splits = std::max(1, splits);
    const int per = (nch + splits - 1) / splits;
    return (nch + per - 1) / per;  // no empty split
}

bool gemm_shape_ok(int kind, int N, int K, int group, int m) {
    if (m < 1 || m > kGemmRowsMax || N < 1 || K < kChunk || K % kChunk != 0) return false;
    if (kind == KIND_Q4 && (group < kChunk || group % kChunk != 0 || K % group != 0)) return false;
    return true;
}

size_t gemm_frag_bytes(int K, int m) { return (size_t)((m + kBM - 1) / kBM) * (K / kChunk) * kChunkBytes; }

void launch_stage_x(const float* x, int x_stride, int m, int K, const float* gain, int q4order, uint8_t* frag,
                    hipStream_t st) {
    const int mpad = (m + kBM - 1) / kBM * kBM;
    hipLaunchKernelGGL(k_stage_x, dim3((K + 255) / 256, mpad), dim3(256), 0, st, x, x_stride, m, K, gain, q4order, frag);
}

// The tile-major copy of a q4 matrix's (scale, zero) words: szt[(t G + g) 32 + r] = sz[(32 t + r) G + g]
// (zero for rows past the matrix). Grid (ceil(rows / 32) G / 8), 256 threads.
__global__ __launch_bounds__(256) void k_tile_sz(const uint32_t* __restrict__ sz, int rows, int ngroups,
                                                 uint32_t* __restrict__ szt) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, tiles = ((size_t)rows + 31) / 32;
    if (i >= tiles * ngroups * 32) return;
    const size_t r = (i / ((size_t)ngroups * 32)) * 32 + i % 32, g = (i / 32) % ngroups;
    szt[i] = r < (size_t)rows ? sz[r * ngroups + g] : 0u;
}

size_t tile_sz_words(int rows, int ngroups) { return ((size_t)rows + 31) / 32 * ngroups * 32; }

void launch_tile_sz(const uint32_t* sz, int rows, int ngroups, uint32_t* szt, hipStream_t st) {
    const size_t n = tile_sz_words(rows, ngroups);
    hipLaunchKernelGGL(k_tile_sz, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, sz, rows, ngroups, szt);
}

void launch_gemm(GemmArgs a, hipStream_t st) {
    if (a.kind == KIND_Q4 && !a.SZT) throw Error(QNE_EINVAL, "q4 GEMM needs the tile-major scale/zero words");
    const int nch = a.K / kChunk;
    a.cps = (nch + a.splits - 1) / a.splits;
    a.mpad = (a.m + kBM - 1) / kBM * kBM;
    if (a.x) {  // stage the x operand here (RMSNorm gain folded in, 1 / rms deferred to the epilogue)
        launch_stage_x(a.x, a.x_stride, a.m, a.K, a.gain, a.kind == KIND_Q4 ? 1 : 0, a.frag, st);
        a.norm = a.gain ? 1 : 0;
    }
    const int waves = gemm_waves(a.kind, a.N);
    const dim3 grid((a.N + 32 * waves - 1) / (32 * waves), a.splits, a.mpad / kBM);
    // One row tile (a batched decode step): about one workgroup per CU, so 4 DMA waves beside the
    // 8 compute waves let the transfers overlap the computation (64 rows: gate_up 23.9 -> 22.4 us,
    // LM head 222 -> 205 us). Several row tiles (a prefill pass): two 8-wave workgroups per CU
    // (125 VGPRs in a 12-wave workgroup leave room for one). Measured and not kept for the prefill:
    // 4 compute waves of 64 columns each (every A fragment read from LDS feeding two MFMAs), slower
    // on every shape (gate_up 68 -> 108 us): each wave then issues 9 LDS DMAs per chunk instead of
    // 5, and a DMA holds its wave for about the transfer time.
    const bool dma_waves = a.mpad == kBM;
    // One split over several row tiles: the GEMM applies the SwiGLU, or the store / residual add,
    // and stages the output itself, with no partials and no reduce pass
    const bool one = a.fuse == 0 && a.kind == KIND_Q4 && !dma_waves && a.splits == 1 && !a.partials_only;
    a.fuse = 0;
    if (one && a.epi == EPI_SWIGLU && a.N == 2 * a.n_out && a.n_out % (32 * waves / 2) == 0 && a.K <= 64 * kChunk &&
        (a.y || a.frag_out))
        a.fuse = 1;
    // store or residual add staged as the next operand (with a normed input its 1 / rms needs K <= 4096)
    else if (one && a.epi != EPI_SWIGLU && a.frag_out && a.n_out == a.N && a.N % kChunk == 0 &&
             (a.epi == EPI_STORE || a.y) && (!a.norm || a.K <= 64 * kChunk))
        a.fuse = 2;
    a.direct = a.splits == 1 && a.epi != EPI_SWIGLU && !a.frag_out && !a.partials_only;
    if (a.kind == KIND_Q4) {
        // 3 chunk slots (77.6 KiB): deeper rings measured slower, and two workgroups fit a CU
        if (dma_waves) hipLaunchKernelGGL((k_gemm<KIND_Q4, 8, 3, 4, 1>), grid, dim3(768), 0, st, a);
        else hipLaunchKernelGGL((k_gemm<KIND_Q4, 8, 3, 0, 1>), grid, dim3(512), 0, st, a);
    } else {
        // f16: as many chunk slots as fit in 160 KiB of LDS
        if (waves == 8 && dma_waves) hipLaunchKernelGGL((k_gemm<KIND_F16, 8, 3, 4, 1>), grid, dim3(768), 0, st, a);
        else if (waves == 8) hipLaunchKernelGGL((k_gemm<KIND_F16, 8, 3, 0, 1>), grid, dim3(512), 0, st, a);
        else hipLaunchKernelGGL((k_gemm<KIND_F16, 4, 4, 0, 1>), grid, dim3(256), 0, st, a);
    }
    if (!a.direct && !a.fuse && !a.partials_only)
        hipLaunchKernelGGL(k_gemm_reduce, dim3((a.n_out + 255) / 256, a.m), dim3(256), 0, st, a);
}

void launch_embed_rows(int kind, const void* W, const uint32_t* SZ, int group, int hidden, const uint32_t* tokens, int m,
                       float* h, uint8_t* frag, const float* gain, int q4order, hipStream_t st, const int32_t* pos,
                       int32_t* order) {
    if (order && m > 256) order = nullptr;  // one thread per row: larger batches keep the row order
    hipLaunchKernelGGL(k_embed_rows, dim3((hidden + 255) / 256, m), dim3(256), 0, st, kind, W, SZ, group, hidden, tokens,
                       h, frag, gain, q4order, order ? pos : nullptr, order);
}

size_t argmax_rows_scratch(int m) { return (size_t)m * kArgParts * 8; }

void launch_argmax_rows(const float* logits, int m, int V, uint32_t* out, uint32_t* tokens, int32_t* pos, void* scratch,
                        hipStream_t st) {
    float* pv = (float*)scratch;
    uint32_t* pi = (uint32_t*)(pv + (size_t)m * kArgParts);
    hipLaunchKernelGGL(k_argmax_part, dim3(kArgParts, m), dim3(256), 0, st, logits, V, pv, pi);
    hipLaunchKernelGGL(k_argmax_final, dim3(m), dim3(64), 0, st, pv, pi, out, tokens, pos);
}

}  // namespace qne
