// Standalone GEMV kernels (one launch per matrix) and their host-side dispatcher.
#include "gemv.hpp"
#include "argmax.hpp"

namespace qne {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

// rows_out outputs (SwiGlu: rows/2), R rows (or gate/up pairs) per wave iteration.
template <int KIND, int K, int G, int EPI, int R>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(const void* __restrict__ W, const uint32_t* __restrict__ SZ,
                                                        const float* __restrict__ x, const float* __restrict__ gain,
                                                        float eps, float* __restrict__ y, int rows_out, ArgmaxOut am) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    float xr[K / 64];
    load_x<KIND, K>(x, gain, eps, xr, lane);
    float xs[KIND == KIND_Q4 ? Q4Plan<K>::NS : 1];
    if constexpr (KIND == KIND_Q4) slab_sums<K>(xr, xs);
    float best = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    const int gw = blockIdx.x * kGemvWaves + wave, nw = gridDim.x * kGemvWaves;
    constexpr int NR = EPI == EPI_SWIGLU ? 2 * R : R;
    for (int r0 = gw * R; r0 < rows_out; r0 += nw * R) {
        RowRaw<KIND, K> raw[NR];
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int row = min(r0 + i, rows_out - 1);
            load_row<KIND, K, G>(raw[i], W, SZ, row, lane);
            if constexpr (EPI == EPI_SWIGLU) load_row<KIND, K, G>(raw[R + i], W, SZ, row + rows_out, lane);
        }
        float part[NR];
#pragma unroll
        for (int i = 0; i < NR; i++) part[i] = wave_sum(row_partial<KIND, K>(raw[i], xr, xs));
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int row = r0 + i;
                if (row < rows_out) {
                    if constexpr (EPI == EPI_STORE || EPI == EPI_ARGMAX) y[row] = part[i];
                    else if constexpr (EPI == EPI_ACCUMULATE) y[row] = y[row] + part[i];
                    else y[row] = silu(part[i]) * part[R + i];
                    if constexpr (EPI == EPI_ARGMAX) {
                        if (better(part[i], (uint32_t)row, best, best_i)) { best = part[i]; best_i = (uint32_t)row; }
                    }
                }
            }
        }
    }
    if constexpr (EPI == EPI_ARGMAX) argmax_block_and_finish(best, best_i, am);
}

template <int KIND, int K, int G, int EPI>
static void launch_one(const void* W, const uint32_t* SZ, const float* x, const float* gain, float eps, float* y,
                       int rows_out, const ArgmaxOut& am, hipStream_t st) {
    constexpr int R = (K >= 4096) ? 2 : 4;
    int blocks = (rows_out + kGemvWaves * R - 1) / (kGemvWaves * R);
    const int cap = EPI == EPI_ARGMAX ? kArgmaxMaxBlocks : 1024;
    if (blocks > cap) blocks = cap;
    hipLaunchKernelGGL((k_gemv<KIND, K, G, EPI, R>), dim3(blocks), dim3(kGemvThreads), 0, st, W, SZ, x, gain, eps, y,
                       rows_out, am);
}

template <int KIND, int K, int G>
static void by_epi(int epi, const void* W, const uint32_t* SZ, const float* x, const float* gain, float eps, float* y,
                   int rows_out, const ArgmaxOut& am, hipStream_t st) {
    switch (epi) {
        case EPI_STORE: launch_one<KIND, K, G, EPI_STORE>(W, SZ, x, gain, eps, y, rows_out, am, st); break;
        case EPI_ACCUMULATE: launch_one<KIND, K, G, EPI_ACCUMULATE>(W, SZ, x, gain, eps, y, rows_out, am, st); break;
        case EPI_SWIGLU: launch_one<KIND, K, G, EPI_SWIGLU>(W, SZ, x, gain, eps, y, rows_out, am, st); break;
        default: launch_one<KIND, K, G, EPI_ARGMAX>(W, SZ, x, gain, eps, y, rows_out, am, st); break;
    }
}

template <int K>
static bool by_kind(int kind, int group, int epi, const void* W, const uint32_t* SZ, const float* x, const float* gain,
                    float eps, float* y, int rows_out, const ArgmaxOut& am, hipStream_t st) {
    if (kind == KIND_F16) { by_epi<KIND_F16, K, 64>(epi, W, SZ, x, gain, eps, y, rows_out, am, st); return true; }
    switch (group) {
        case 32: by_epi<KIND_Q4, K, 32>(epi, W, SZ, x, gain, eps, y, rows_out, am, st); return true;
        case 64: by_epi<KIND_Q4, K, 64>(epi, W, SZ, x, gain, eps, y, rows_out, am, st); return true;
        case 128: by_epi<KIND_Q4, K, 128>(epi, W, SZ, x, gain, eps, y, rows_out, am, st); return true;
        default: return false;
    }
}

bool launch_gemv(int kind, const void* W, const uint32_t* SZ, int rows, int k, int group, const float* x,
                 const float* gain, float eps, float* y, int epi, const ArgmaxOut& am, hipStream_t st) {
    const int rows_out = epi == EPI_SWIGLU ? rows / 2 : rows;
    if (rows_out <= 0) return false;
    switch (k) {
        case 512: return by_kind<512>(kind, group, epi, W, SZ, x, gain, eps, y, rows_out, am, st);
        case 1024: return by_kind<1024>(kind, group, epi, W, SZ, x, gain, eps, y, rows_out, am, st);
        case 2048: return by_kind<2048>(kind, group, epi, W, SZ, x, gain, eps, y, rows_out, am, st);
        case 3072: return by_kind<3072>(kind, group, epi, W, SZ, x, gain, eps, y, rows_out, am, st);
        case 3584: return by_kind<3584>(kind, group, epi, W, SZ, x, gain, eps, y, rows_out, am, st);
        case 4096: return by_kind<4096>(kind, group, epi, W, SZ, x, gain, eps, y, rows_out, am, st);
        case 6144: return by_kind<6144>(kind, group, epi, W, SZ, x, gain, eps, y, rows_out, am, st);
        default: return false;
    }
}

}  // namespace qne
