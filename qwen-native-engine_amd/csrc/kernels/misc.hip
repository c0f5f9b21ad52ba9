// Small kernels: embedding row gather (kernels/src/shaders.rs:405-434 reads the row index on the
// device so a GPU-resident decode loop never needs the host), token-slot updates.
#include "gemv.hpp"
#include "launch.hpp"

namespace qne {

// h[c] = W[tok[0]][c] for an f16 table, or the dequantised q4 row (value (q - z) * s).
__global__ void k_embed(int kind, const void* __restrict__ W, const uint32_t* __restrict__ SZ, int group, int hidden,
                        const uint32_t* __restrict__ tok, float* __restrict__ h) {
    const size_t row = tok[0];
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < hidden; c += gridDim.x * blockDim.x) {
        if (kind == KIND_F16) {
            h[c] = h2f(((const uint16_t*)W)[row * hidden + c]);
        } else {
            const uint32_t word = ((const uint32_t*)W)[row * (hidden / 8) + c / 8];
            const float q = (float)((word >> (4 * (c % 8))) & 15u);
            const uint32_t sz = SZ[row * (hidden / group) + c / group];
            h[c] = (q - hi_h(sz)) * lo_h(sz);
        }
    }
}

// tok = {ids[i], pos, tok[2], tok[3]}: the host writes of tok in Model::prefill (model.rs:329),
// done on the device so a whole prompt is one upload.
__global__ void k_set_tok(uint32_t* __restrict__ tok, const uint32_t* __restrict__ ids, int i, uint32_t pos) {
    tok[0] = ids[i];
    tok[1] = pos;
}

// Pseudo-random fill for benchmark state: value i is uniform in [-amp, amp) from a SplitMix64 hash
// of (seed, i).
__global__ void k_fill_uniform(void* __restrict__ p, size_t n, int f16, uint64_t seed, float amp) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        const float v = ((float)(z >> 40) * (1.0f / 8388608.0f) - 1.0f) * amp;
        if (f16) ((uint16_t*)p)[i] = f2h(v);
        else ((float*)p)[i] = v;
    }
}

// Streaming-read probe (the reference's `bandwidth` shader, kernels/src/shaders.rs:701-717): every
// 16-byte word of `data` is read once, non-temporal, and xor-folded into one word per thread, so
// nothing but the loads costs time. Four loads per thread are in flight per iteration.
__global__ __launch_bounds__(256) void k_stream_read(const u32x4* __restrict__ data, size_t n, uint32_t* __restrict__ sink) {
    const size_t threads = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (; i + 3 * threads < n; i += 4 * threads) {
        const u32x4 a = __builtin_nontemporal_load(data + i), b = __builtin_nontemporal_load(data + i + threads);
        const u32x4 c = __builtin_nontemporal_load(data + i + 2 * threads), d = __builtin_nontemporal_load(data + i + 3 * threads);
        acc ^= a ^ b ^ c ^ d;
    }
    for (; i < n; i += threads) acc ^= __builtin_nontemporal_load(data + i);
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

// A dispatch that does almost nothing (the reference's `noop`, kernels/src/shaders.rs:719-729): the
// fixed cost of one dispatch.
__global__ void k_noop(float* y) {
    if (threadIdx.x == 0) y[0] = y[0] + 1.0f;
}

// Hand-over probe: the all-to-all exchange the persistent decode kernel pays at every phase, without
// its compute or its weight stream. Each of the (co-resident) workgroups publishes its share of an
// n-value vector every round: value o = round + o next to the 32-bit tag `round`, one 8-byte
// agent-scope store per value, the workgroups interleaved (o = wg + workgroups * k). Then every
// workgroup polls all n / 2 pairs with agent-scope 16-byte loads (up to 6 per thread in flight)
// until each carries the round's tag, and ends the round with a barrier. Rounds alternate between
// two buffers of n entries. ticks[0] = wall-clock ticks of workgroup 0 over rounds 3..rounds;
// err[0] = 1 after a poll spins 2^20 times (then every workgroup stops).
__global__ __launch_bounds__(512, 1) void k_exchange_probe(uint64_t* __restrict__ buf, int n, int rounds,
                                                           unsigned long long* __restrict__ ticks, unsigned* __restrict__ err) {
    constexpr int kT = 512, kP = 6;
    const int wg = blockIdx.x, nwg = gridDim.x, np = n / 2;
    __shared__ int bail;
    __shared__ float sink[2 * kT * kP];
    if (threadIdx.x == 0) bail = 0;
    __syncthreads();
    unsigned long long t0 = 0;
    for (int r = 1; r <= rounds; r++) {
        if (r == 3) t0 = __builtin_amdgcn_s_memrealtime();
        uint64_t* b = buf + (size_t)(r & 1) * n;
        for (int o = wg + nwg * (int)threadIdx.x; o < n; o += nwg * kT)
            __hip_atomic_store(b + o, ((uint64_t)r << 32) | __float_as_uint((float)(r + o)), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(b, (short)0, n * 8, 0x00020000);
        unsigned pend = 0;
#pragma unroll
        for (int j = 0; j < kP; j++)
            if (j * kT + (int)threadIdx.x < np) pend |= 1u << j;
        unsigned spins = 0;
        while (pend) {
            u32x4 v[kP];
#pragma unroll
            for (int j = 0; j < kP; j++)
                if ((pend >> j) & 1u) v[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * (j * kT + (int)threadIdx.x), 0, 16);
#pragma unroll
            for (int j = 0; j < kP; j++) {
                if (((pend >> j) & 1u) && v[j].y == (unsigned)r && v[j].w == (unsigned)r) {
                    const int q = j * kT + (int)threadIdx.x;
                    sink[2 * q] = __uint_as_float(v[j].x);
                    sink[2 * q + 1] = __uint_as_float(v[j].z);
                    pend &= ~(1u << j);
                }
            }
            asm volatile("" ::: "memory");  // every spin loads again
            if (pend && ++spins > (1u << 20)) {
                err[0] = 1u;
                bail = 1;
                break;
            }
        }
        __syncthreads();
        if (bail) break;
    }
    if (wg == 0 && threadIdx.x == 0) ticks[0] = __builtin_amdgcn_s_memrealtime() - t0;
}

hipError_t launch_exchange_probe(uint64_t* buf, int n, int rounds, int workgroups, unsigned long long* ticks, unsigned* err,
                                 hipStream_t st) {
    void* args[] = {&buf, &n, &rounds, &ticks, &err};
    return hipLaunchCooperativeKernel((const void*)k_exchange_probe, dim3(workgroups), dim3(512), args, 0, st);
}

void launch_stream_read(const void* data, size_t bytes, uint32_t* sink, int workgroups, hipStream_t st) {
    hipLaunchKernelGGL(k_stream_read, dim3(workgroups), dim3(256), 0, st, (const u32x4*)data, bytes / 16, sink);
}

void launch_noop(float* y, hipStream_t st) { hipLaunchKernelGGL(k_noop, dim3(1), dim3(64), 0, st, y); }

void launch_fill_uniform(void* p, size_t n, bool f16, uint64_t seed, float amp, hipStream_t st) {
    if (n == 0) return;
    const size_t blocks = std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(k_fill_uniform, dim3((unsigned)blocks), dim3(256), 0, st, p, n, f16 ? 1 : 0, seed, amp);
}

void launch_set_tok(uint32_t* tok, const uint32_t* ids, int i, uint32_t pos, hipStream_t st) {
    hipLaunchKernelGGL(k_set_tok, dim3(1), dim3(1), 0, st, tok, ids, i, pos);
}

void launch_embed(int kind, const void* W, const uint32_t* SZ, int group, int hidden, const uint32_t* tok, float* h,
                  hipStream_t st) {
    const int blocks = (hidden + 255) / 256;
    hipLaunchKernelGGL(k_embed, dim3(blocks), dim3(256), 0, st, kind, W, SZ, group, hidden, tok, h);
}

}  // namespace qne
