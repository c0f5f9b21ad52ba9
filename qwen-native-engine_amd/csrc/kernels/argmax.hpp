// Device side of the LM-head greedy pick: per-block argmax, then the last block reduces.
#pragma once

#include "common.hpp"
#include "launch.hpp"

namespace qne {

// Block-level argmax of per-lane candidates, then the last block to finish reduces the per-block
// results and publishes the pick. Candidates: larger value, then lower index.
__device__ __forceinline__ void argmax_block_and_finish(float best, uint32_t best_i, const ArgmaxOut& am) {
    __shared__ float sv[16];
    __shared__ uint32_t si[16];
    __shared__ bool last;
    // wave reduction of (value, index)
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float ov = __shfl_xor(best, m, kWave);
        uint32_t oi = (uint32_t)__shfl_xor((int)best_i, m, kWave);
        if (better(ov, oi, best, best_i)) { best = ov; best_i = oi; }
    }
    const int w = threadIdx.x / kWave, nw = blockDim.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) { sv[w] = best; si[w] = best_i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = sv[0];
        uint32_t bi = si[0];
        for (int i = 1; i < nw; i++)
            if (better(sv[i], si[i], b, bi)) { b = sv[i]; bi = si[i]; }
        am.part_val[blockIdx.x] = b;
        am.part_idx[blockIdx.x] = bi;
        __threadfence();
        const unsigned prev = atomicAdd(am.counter, 1u);
        last = prev == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    float b = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (unsigned i = threadIdx.x; i < gridDim.x; i += blockDim.x) {
        const float v = __builtin_nontemporal_load(am.part_val + i);
        const uint32_t ix = __builtin_nontemporal_load(am.part_idx + i);
        if (better(v, ix, b, bi)) { b = v; bi = ix; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float ov = __shfl_xor(b, m, kWave);
        uint32_t oi = (uint32_t)__shfl_xor((int)bi, m, kWave);
        if (better(ov, oi, b, bi)) { b = ov; bi = oi; }
    }
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) { sv[w] = b; si[w] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < nw; i++)
            if (better(sv[i], si[i], sv[0], si[0])) { sv[0] = sv[i]; si[0] = si[i]; }
        const uint32_t pick = si[0] == 0xFFFFFFFFu ? 0u : si[0];
        am.tok[0] = pick;
        am.tok[1] = am.tok[1] + 1u;
        if (am.ids) {
            const uint32_t n = am.tok[2];
            if (n < am.ids_cap) am.ids[n] = pick;
            am.tok[2] = n + 1u;
        }
        *am.counter = 0u;
    }
}

}  // namespace qne
