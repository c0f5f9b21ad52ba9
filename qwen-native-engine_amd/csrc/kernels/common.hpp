// Device helpers shared by the gfx950 kernels: f16 conversion, wave64 reductions, activations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qne {

constexpr int kWave = 64;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// A store written through to memory at device scope (sc1) instead of left dirty in this XCD's L2.
// For data the next kernel reads: the kernel-end release then has fewer dirty lines to write back.
template <class T>
__device__ __forceinline__ void store_through(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float lo_h(uint32_t w) { return h2f((uint16_t)(w & 0xFFFFu)); }
__device__ __forceinline__ float hi_h(uint32_t w) { return h2f((uint16_t)(w >> 16)); }

// Accurate expf (not the fast exp2 form): the oracle evaluates the same expressions with libm.
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// Cross-lane moves without the LDS crossbar: DPP within rows of 16 lanes, and the gfx950
// permlane swaps across rows (v_permlane16_swap: lane ^ 16, v_permlane32_swap: lane ^ 32).
#define QNE_DPP(v, ctrl) __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), (ctrl), 0xF, 0xF, false))
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within 16
constexpr int kDppRor8 = 0x128;        // lane i <- (i + 8) % 16 within 16, i.e. lane ^ 8
__device__ __forceinline__ float lane_xor32(float v, int lane) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((lane & 32) ? p[0] : p[1]);
}
__device__ __forceinline__ float lane_xor16(float v, int lane) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((lane & 16) ? p[0] : p[1]);
}
// Sum over the 64 lanes of a wave with DPP and permlane swaps; every lane receives the total.
__device__ __forceinline__ float wave_sum_dpp(float v) {
    const int lane = (int)__lane_id();
    v += QNE_DPP(v, kDppXor1);
    v += QNE_DPP(v, kDppXor2);
    v += QNE_DPP(v, kDppHalfMirror);
    v += QNE_DPP(v, kDppMirror);
    v += lane_xor16(v, lane);
    v += lane_xor32(v, lane);
    return v;
}

// Sum over each half (32 lanes) of a wave; every lane receives its half's total.
__device__ __forceinline__ float half_sum_dpp(float v, int lane) {
    v += QNE_DPP(v, kDppXor1);
    v += QNE_DPP(v, kDppXor2);
    v += QNE_DPP(v, kDppHalfMirror);
    v += QNE_DPP(v, kDppMirror);
    v += lane_xor16(v, lane);
    return v;
}

// Sums 8 per-lane partials across the wave: after the call, lanes 8r..8r+7 hold the total of
// partial r. Halving steps over lane bits 5, 4, 3 (each lane keeps the half its bit selects and
// adds its partner's copy of it, exchanged with permlane swaps and DPP), then a plain sum over
// lane bits 2, 1, 0 with DPP.
__device__ __forceinline__ float reduce8(float (&v)[8], int lane) {
    float h4[4], h2[2];
    const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float send = b5 ? v[i] : v[i + 4], keep = b5 ? v[i + 4] : v[i];
        h4[i] = keep + lane_xor32(send, lane);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const float send = b4 ? h4[i] : h4[i + 2], keep = b4 ? h4[i + 2] : h4[i];
        h2[i] = keep + lane_xor16(send, lane);
    }
    const float send = b3 ? h2[0] : h2[1], keep = b3 ? h2[1] : h2[0];
    float t = keep + QNE_DPP(send, kDppRor8);
    t += QNE_DPP(t, kDppXor1);
    t += QNE_DPP(t, kDppXor2);
    t += QNE_DPP(t, kDppHalfMirror);
    return t;
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}
// The same butterfly as wave_sum (lane xor 32, 16, 8, 4, 2, 1), so the same bits, with permlane
// swaps, LDS swizzles and DPP: no per-lane shuffle addresses for the compiler to keep live.
__device__ __forceinline__ float wave_sum_xor(float v) {
    const int lane = (int)__lane_id();
    v += lane_xor32(v, lane);
    v += lane_xor16(v, lane);
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (8 << 10)));
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (4 << 10)));
    v += QNE_DPP(v, kDppXor2);
    v += QNE_DPP(v, kDppXor1);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
    return v;
}
// Sum over aligned groups of 16 lanes.
__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Block-wide sum over the NT threads of the workgroup (NT, the launch's block size, a multiple of
// 64, at most 1024: a constant, as blockDim.x costs two dependent loads of the dispatch's implicit
// arguments). `red` needs 16 floats of LDS.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    static_assert(NT % kWave == 0 && NT <= 1024, "whole waves, at most 16");
    v = wave_sum(v);
    const int w = threadIdx.x / kWave;
    constexpr int nw = NT / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) red[w] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

// Greedy-pick order: larger value wins, ties go to the lower index, NaN never wins.
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

}  // namespace qne
