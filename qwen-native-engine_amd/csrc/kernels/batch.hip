// Batched decode (up to 64 sequences per step): the GEMM that replaces the GEMV, and the small
// per-row kernels around it.
//
// Reference: the 16-token prefill GEMM `gemm` (kernels/src/batch.rs:12-99, launched by `Gpu::gemm`,
// lib.rs:341-347) and its embed / argmax companions (shaders.rs:405-434, 635-699), generalised to M
// rows of one decode step each. Design for gfx950:
//  - a workgroup (4 waves) computes a 64 x 128 tile of y = x W^T (64 rows of x, 32 W rows per
//    wave) over a slice of K (split-K), with v_mfma_f32_32x32x16_f16;
//  - x chunks of 64 columns are staged in LDS once per workgroup from the f32 activations: scaled
//    by the RMSNorm gain when the matrix follows a norm (the row's 1 / rms is a scalar per row and
//    is applied after the sum), then split into f16 halves hi = f16(x), lo = f16(x - hi), so that
//    the two MFMAs over hi and lo reproduce f32 products to about 2^-22;
//  - q4 weights are dequantised in registers as exact f16 integers (0x6400 | q is 1024 + q, minus
//    1024 is exact); each quantisation group is summed into a fresh f32 tile and its scale and zero
//    applied once: y += s (sum q x - z sum x), with the group sums of x taken from the staged
//    values. f16 weights go to the MFMA as they are;
//  - with one split the workgroup applies the epilogue itself; otherwise it writes partials and
//    k_gemm_reduce sums them in split order (so the result does not depend on timing) and applies
//    1 / rms and the epilogue (store, residual add, SwiGLU).
#include "common.hpp"
#include "launch.hpp"

namespace qne {

namespace {

constexpr int kBM = 64;            // rows of x per GEMM (sequences)
constexpr int kTileN = 128;        // W rows per workgroup, 32 per wave
constexpr int kChunk = 64;         // columns of x per staged chunk
constexpr int kXRow = kChunk + 8;  // f16 per LDS row of a chunk (16 bytes of padding)
constexpr int kGemmThreads = 256;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// The 8 nibbles of a q4 word (nibble i at bits 4i, column 8j + i of word j) as exact f16 values.
__device__ __forceinline__ half8_t nibbles8(uint32_t v) {
    const half2_t bias = {(_Float16)1024.0f, (_Float16)1024.0f};
    half8_t r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t nb = v >> (8 * i);
        const uint32_t p = (nb & 0xFu) | ((nb & 0xF0u) << 12) | 0x64006400u;
        const half2_t x = __builtin_bit_cast(half2_t, p) - bias;
        r[2 * i] = x.x;
        r[2 * i + 1] = x.y;
    }
    return r;
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

}  // namespace

// Grid (ceil(N / 128), splits); split s covers quantisation groups [s * gps, (s + 1) * gps) (for f16
// weights a "group" is one 64-column chunk). Lane layout of v_mfma_f32_32x32x16_f16 (lane l):
// A[l % 32][8 (l / 32) + i], B[8 (l / 32) + i][l % 32], D register j = [8 (j / 4) + 4 (l / 32) + j % 4][l % 32].
// The 16 MFMA k-slots of step s of a chunk map to chunk columns 32 (l / 32) + 8 s + i, the same for
// A and B, so a lane's W bytes of a chunk are contiguous (16 bytes of q4, 64 of f16).
template <int KIND>
__global__ __launch_bounds__(kGemmThreads, 2) void k_gemm(const GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sx[2][kBM * kXRow];  // hi, lo of one chunk
    __shared__ float ssum[kBM];                                          // group sums of x (q4)
    __shared__ float sinv[kBM];                                          // 1 / rms per row
    const int t = threadIdx.x, lane = t & 63, w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int hf = lane >> 5, l32 = lane & 31;
    const int n = blockIdx.x * kTileN + 32 * w + l32;
    const int nr = min(n, a.N - 1);  // rows past N compute on row N - 1 and are not stored
    const int K = a.K;
    const int cpg = KIND == KIND_Q4 ? a.group / kChunk : 1;
    const int ngroups = K / (cpg * kChunk);
    const int g0 = blockIdx.y * a.gps, g1 = min(ngroups, g0 + a.gps);
    const int c0 = g0 * cpg, c1 = g1 * cpg;

    // staging: thread t copies row sm, columns sk .. sk + 15 of each chunk
    const int sm = t >> 2, sk = 16 * (t & 3);
    const bool live = sm < a.m;
    const float* xr = a.x + (size_t)(live ? sm : 0) * a.x_stride + sk;
    const float* gr = a.gain ? a.gain + sk : nullptr;

    const uint8_t* wq = (const uint8_t*)a.W + (size_t)nr * (K / 2) + 16 * hf;  // q4: 16 bytes per chunk
    const uint16_t* wf = (const uint16_t*)a.W + (size_t)nr * K + 32 * hf;      // f16: 64 bytes per chunk

    float16_t acc0, acc1, grp0, grp1;
#pragma unroll
    for (int j = 0; j < 16; j++) acc0[j] = acc1[j] = grp0[j] = grp1[j] = 0.0f;
    float ss = 0.0f, gsum = 0.0f;

    constexpr int kWv = KIND == KIND_Q4 ? 1 : 4;
    float4 xv[4];
    uint4 wv[kWv];
    auto load = [&](int c) {
        const int k0 = c * kChunk;
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = live ? *(const float4*)(xr + k0 + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (KIND == KIND_Q4) {
            wv[0] = *(const uint4*)(wq + (size_t)k0 / 2);
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) wv[i] = *(const uint4*)(wf + k0 + 8 * i);
        }
    };
    if (c0 < c1) load(c0);
    for (int c = c0; c < c1; c++) {
        const int k0 = c * kChunk;
        // x chunk -> hi / lo (times the gain), sums of squares of the raw x, group sums of hi + lo
        uint32_t ph[8], pl[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float v[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
            float4 gv = make_float4(1.f, 1.f, 1.f, 1.f);
            if (gr) gv = *(const float4*)(gr + k0 + 4 * i);
            const float g[4] = {gv.x, gv.y, gv.z, gv.w};
            float hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                ss = fmaf(v[e], v[e], ss);
                const float xg = v[e] * g[e];
                hi[e] = (float)(_Float16)xg;
                lo[e] = (float)(_Float16)(xg - hi[e]);
                gsum += hi[e] + lo[e];
            }
            ph[2 * i] = pack_h2(hi[0], hi[1]);
            ph[2 * i + 1] = pack_h2(hi[2], hi[3]);
            pl[2 * i] = pack_h2(lo[0], lo[1]);
            pl[2 * i + 1] = pack_h2(lo[2], lo[3]);
        }
        uint4 wcur[kWv];
#pragma unroll
        for (int i = 0; i < kWv; i++) wcur[i] = wv[i];
        const bool group_end = KIND == KIND_Q4 && (c + 1 - c0) % cpg == 0;
        float gtot = 0.0f;
        if (group_end) {
            gtot = gsum + __shfl_xor(gsum, 1, 64);
            gtot += __shfl_xor(gtot, 2, 64);
            gsum = 0.0f;
        }
        __syncthreads();  // every wave is done with the previous chunk
        uint4* dh = (uint4*)&sx[0][sm * kXRow + sk];
        uint4* dl = (uint4*)&sx[1][sm * kXRow + sk];
        dh[0] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
        dh[1] = make_uint4(ph[4], ph[5], ph[6], ph[7]);
        dl[0] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
        dl[1] = make_uint4(pl[4], pl[5], pl[6], pl[7]);
        if (group_end && (t & 3) == 0) ssum[sm] = gtot;
        __syncthreads();
        if (c + 1 < c1) load(c + 1);  // next chunk in flight during the MFMAs
#pragma unroll
        for (int s = 0; s < 4; s++) {
            half8_t b;
            if (KIND == KIND_Q4) {
                const uint32_t word = s == 0 ? wcur[0].x : s == 1 ? wcur[0].y : s == 2 ? wcur[0].z : wcur[0].w;
                b = nibbles8(word);
            } else {
                b = __builtin_bit_cast(half8_t, wcur[s]);
            }
            const int o = l32 * kXRow + 32 * hf + 8 * s;
            const half8_t a0h = *(const half8_t*)&sx[0][o];
            const half8_t a0l = *(const half8_t*)&sx[1][o];
            const half8_t a1h = *(const half8_t*)&sx[0][o + 32 * kXRow];
            const half8_t a1l = *(const half8_t*)&sx[1][o + 32 * kXRow];
            grp0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0h, b, grp0, 0, 0, 0);
            grp1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1h, b, grp1, 0, 0, 0);
            grp0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0l, b, grp0, 0, 0, 0);
            grp1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1l, b, grp1, 0, 0, 0);
        }
        if (group_end) {
            const uint32_t szw = a.SZ[(size_t)nr * ngroups + (c / cpg)];
            const float sc = lo_h(szw), z = hi_h(szw);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int m = 8 * (j / 4) + 4 * hf + (j % 4);
                acc0[j] = fmaf(sc, grp0[j] - z * ssum[m], acc0[j]);
                acc1[j] = fmaf(sc, grp1[j] - z * ssum[32 + m], acc1[j]);
                grp0[j] = 0.0f;
                grp1[j] = 0.0f;
            }
        }
    }
    if (KIND != KIND_Q4) {
        acc0 = grp0;
        acc1 = grp1;
    }
    // sums of squares of the rows over this split's columns
    ss += __shfl_xor(ss, 1, 64);
    ss += __shfl_xor(ss, 2, 64);
    if (!a.direct) {
        if (blockIdx.x == 0 && (t & 3) == 0) a.ss_part[(size_t)blockIdx.y * kBM + sm] = ss;
        if (n < a.N) {
            float* pp = a.part + (size_t)blockIdx.y * kBM * a.N + n;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int m = 8 * (j / 4) + 4 * hf + (j % 4);
                pp[(size_t)m * a.N] = acc0[j];
                pp[(size_t)(32 + m) * a.N] = acc1[j];
            }
        }
        return;
    }
    // direct (one split, no SwiGLU): 1 / rms and the epilogue here (store or residual add)
    if ((t & 3) == 0) sinv[sm] = a.gain ? 1.0f / sqrtf(ss / (float)K + a.eps) : 1.0f;
    __syncthreads();
    if (n < a.N) {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int m = 8 * (j / 4) + 4 * hf + (j % 4);
            if (m < a.m) {
                float* d = a.y + (size_t)m * a.y_stride + n;
                const float v = acc0[j] * sinv[m];
                *d = a.epi == EPI_ACCUMULATE ? *d + v : v;
            }
            if (32 + m < a.m) {
                float* d = a.y + (size_t)(32 + m) * a.y_stride + n;
                const float v = acc1[j] * sinv[32 + m];
                *d = a.epi == EPI_ACCUMULATE ? *d + v : v;
            }
        }
    }
}

// y rows r < m, columns c < n_out, from the split partials summed in split order, times 1 / rms of
// the row when the GEMM followed a norm: store, residual add, or SwiGLU silu(gate) * up with gate =
// column c and up = column c + n_out (matrix rows [gate; up], shaders.rs gemv epilogues).
__global__ __launch_bounds__(256) void k_gemm_reduce(const GemmArgs a) {
    const int c = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (c >= a.n_out || r >= a.m) return;
    float inv = 1.0f;
    if (a.gain) {
        float ss = 0.0f;
        for (int s = 0; s < a.splits; s++) ss += a.ss_part[(size_t)s * kBM + r];
        inv = 1.0f / sqrtf(ss / (float)a.K + a.eps);
    }
    float g = 0.0f, u = 0.0f;
    for (int s = 0; s < a.splits; s++) {
        const float* p = a.part + ((size_t)s * kBM + r) * a.N;
        g += p[c];
        if (a.epi == EPI_SWIGLU) u += p[c + a.n_out];
    }
    g *= inv;
    u *= inv;
    float* d = a.y + (size_t)r * a.y_stride + c;
    if (a.epi == EPI_STORE) *d = g;
    else if (a.epi == EPI_ACCUMULATE) *d += g;
    else *d = silu(g) * u;
}

// h[r] = embedding row tokens[r] (f16 row, or q4 values (q - z) s), shaders.rs:405-434 per row.
__global__ __launch_bounds__(256) void k_embed_rows(int kind, const void* __restrict__ W, const uint32_t* __restrict__ SZ,
                                                    int group, int hidden, const uint32_t* __restrict__ tokens,
                                                    float* __restrict__ h) {
    const int r = blockIdx.y;
    const size_t tok = tokens[r];
    for (int c = blockIdx.x * 256 + threadIdx.x; c < hidden; c += gridDim.x * 256) {
        float v;
        if (kind == KIND_F16) {
            v = h2f(((const uint16_t*)W)[tok * hidden + c]);
        } else {
            const uint32_t word = ((const uint32_t*)W)[tok * (hidden / 8) + c / 8];
            const uint32_t sz = SZ[tok * (hidden / group) + c / group];
            v = ((float)((word >> (4 * (c % 8))) & 15u) - hi_h(sz)) * lo_h(sz);
        }
        h[(size_t)r * hidden + c] = v;
    }
}

// Greedy pick of every logits row (argmax_partial / argmax_final, shaders.rs:635-699): the largest
// value, ties to the lower index. With `tokens`, row r's pick becomes its next token and its
// position advances (pos[r] += 1), so decode steps chain on the device.
__global__ __launch_bounds__(512) void k_argmax_rows(const float* __restrict__ logits, int V, uint32_t* __restrict__ out,
                                                     uint32_t* __restrict__ tokens, int32_t* __restrict__ pos) {
    __shared__ float sv[8];
    __shared__ uint32_t si[8];
    const int r = blockIdx.x, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const float* row = logits + (size_t)r * V;
    float best = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (int c = t; c < V; c += 512) {
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
        for (int i = 1; i < 8; i++)
            if (better(sv[i], si[i], b, bix)) {
                b = sv[i];
                bix = si[i];
            }
        const uint32_t pick = bix == 0xFFFFFFFFu ? 0u : bix;  // all NaN: token 0
        if (out) out[r] = pick;
        if (tokens) {
            tokens[r] = pick;
            pos[r] += 1;
        }
    }
}

int gemm_splits(int kind, int N, int K, int group) {
    const int tiles = (N + kTileN - 1) / kTileN;
    const int units = kind == KIND_Q4 ? K / group : K / kChunk;
    int splits = (512 + tiles - 1) / tiles;  // about 512 workgroups
    if (splits > units) splits = units;
    if (splits < 1) splits = 1;
    const int per = (units + splits - 1) / splits;
    return (units + per - 1) / per;  // no empty split
}

bool gemm_shape_ok(int kind, int N, int K, int group, int m) {
    if (m < 1 || m > kBM || N < 1 || K < kChunk || K % kChunk != 0) return false;
    if (kind == KIND_Q4 && (group < kChunk || group % kChunk != 0 || K % group != 0)) return false;
    return true;
}

void launch_gemm(GemmArgs a, hipStream_t st) {
    const int units = a.kind == KIND_Q4 ? a.K / a.group : a.K / kChunk;
    a.gps = (units + a.splits - 1) / a.splits;
    a.direct = a.splits == 1 && a.epi != EPI_SWIGLU;
    const dim3 grid((a.N + kTileN - 1) / kTileN, a.splits);
    if (a.kind == KIND_Q4) hipLaunchKernelGGL((k_gemm<KIND_Q4>), grid, dim3(kGemmThreads), 0, st, a);
    else hipLaunchKernelGGL((k_gemm<KIND_F16>), grid, dim3(kGemmThreads), 0, st, a);
    if (!a.direct) hipLaunchKernelGGL(k_gemm_reduce, dim3((a.n_out + 255) / 256, a.m), dim3(256), 0, st, a);
}

void launch_embed_rows(int kind, const void* W, const uint32_t* SZ, int group, int hidden, const uint32_t* tokens, int m,
                       float* h, hipStream_t st) {
    hipLaunchKernelGGL(k_embed_rows, dim3((hidden + 255) / 256, m), dim3(256), 0, st, kind, W, SZ, group, hidden, tokens, h);
}

void launch_argmax_rows(const float* logits, int m, int V, uint32_t* out, uint32_t* tokens, int32_t* pos,
                        hipStream_t st) {
    hipLaunchKernelGGL(k_argmax_rows, dim3(m), dim3(512), 0, st, logits, V, out, tokens, pos);
}

}  // namespace qne
