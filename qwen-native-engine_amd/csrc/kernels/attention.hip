// GQA attention decode over a paged f16 KV cache (head_dim 256, 16-token blocks).
//
// Reference: the decode kernel `attention` (kernels/src/shaders.rs:522-633), which runs one
// workgroup per query head over an f32 cache with all scores in LDS. Design for gfx950:
//  - the cache is paged: pools [block][kv_head][16][256] f16, a block table maps logical blocks;
//  - split-context ("flash decoding") partials: workgroup (split, kv_head, seq) streams a slice
//    of the context once for all query heads that share the kv head (GQA reuse);
//  - a wave covers 4 positions per step, 16 lanes per position, 16 dims (32 bytes of K and of V)
//    per lane; scores are 16-lane reductions; softmax is online (running max / sum);
//  - a combine kernel merges the splits (and applies the sigmoid output gate of the model).
// The current token's k and v are appended (rounded to f16) before the partials run, so the
// current position is read back exactly as every later step will read it.
#include "common.hpp"
#include "launch.hpp"

namespace qne {

constexpr int kHD = 256, kBlock = 16, kAttnThreads = 256;

__device__ __forceinline__ size_t kv_index(const int32_t* bt, int pos, int nkv, int g) {
    const int blk = bt[pos / kBlock];
    return (((size_t)blk * nkv + g) * kBlock + (pos % kBlock)) * kHD;
}

// RMSNorm (weight w) and rotate-half RoPE on the first rope_dim dims of one 256-vector held one
// value per thread (shaders.rs:575-593). Returns the thread's output value.
__device__ __forceinline__ float norm_rope(float x, const float* __restrict__ w, const float* __restrict__ inv_freq,
                                           int rope_dim, uint32_t pos, float* sh, float* red) {
    const int t = threadIdx.x;
    const float ss = block_sum(x * x, red);
    const float y = x * (1.0f / sqrtf(ss / (float)kHD + 1e-6f)) * w[t];
    sh[t] = y;
    __syncthreads();
    const int half = rope_dim / 2;
    float r = y;
    if (t < rope_dim) {
        const int i = t < half ? t : t - half;
        const float angle = (float)pos * inv_freq[i];
        float sn, cs;
        sincosf(angle, &sn, &cs);
        r = t < half ? y * cs - sh[t + half] * sn : y * cs + sh[t - half] * sn;
    }
    __syncthreads();
    return r;
}

// Model form, grid nq + nkv: query heads are normed/rotated into qbuf; kv heads are normed,
// rotated and appended with their values at position tok[1].
__global__ __launch_bounds__(kAttnThreads) void k_attn_prep(AttnModelArgs a) {
    __shared__ float sh[kHD];
    __shared__ float red[16];
    const int t = threadIdx.x, hb = blockIdx.x;
    const uint32_t pos = a.tok[1];
    if (hb < a.nq) {
        const float x = a.proj[hb * kHD + t];
        a.qbuf[hb * kHD + t] = norm_rope(x, a.norms, a.inv_freq, a.rope_dim, pos, sh, red);
    } else {
        const int g = hb - a.nq;
        const float* kp = a.proj + 2 * a.nq * kHD;
        const float kr = norm_rope(kp[g * kHD + t], a.norms + kHD, a.inv_freq, a.rope_dim, pos, sh, red);
        const size_t at = kv_index(a.block_table, (int)pos, a.nkv, g) + t;
        a.k_pool[at] = f2h(kr);
        a.v_pool[at] = f2h(kp[a.nkv * kHD + g * kHD + t]);
    }
}

// Raw form: append k_new / v_new of sequence blockIdx.y, kv head blockIdx.x at ctx[b].
__global__ __launch_bounds__(kAttnThreads) void k_kv_append(const float* __restrict__ k_new, const float* __restrict__ v_new,
                                                            uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
                                                            const int32_t* __restrict__ bt, int max_blocks,
                                                            const int32_t* __restrict__ ctx, int nkv) {
    const int g = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    if (ctx[b] < 0 || ctx[b] >= max_blocks * kBlock) return;  // beyond the table: nothing to write
    const size_t at = kv_index(bt + (size_t)b * max_blocks, ctx[b], nkv, g) + t;
    const size_t src = ((size_t)b * nkv + g) * kHD + t;
    k_pool[at] = f2h(k_new[src]);
    v_pool[at] = f2h(v_new[src]);
}

// Split-context partials. Grid (splits, nkv, batch). Sequence b attends positions 0..len-1 with
// len = lens[b] + 1 (lens = tok + 1 for the model, ctx for the raw form).
template <int G>
__global__ __launch_bounds__(kAttnThreads) void k_attn_partial(const float* __restrict__ q, const uint16_t* __restrict__ k_pool,
                                                               const uint16_t* __restrict__ v_pool,
                                                               const int32_t* __restrict__ block_table, int max_blocks,
                                                               const int32_t* __restrict__ lens, int nkv,
                                                               float* __restrict__ part_ml, float* __restrict__ part_acc) {
    __shared__ float s_ml[4][G][2];
    __shared__ float s_acc[4][G][kHD];
    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z, splits = gridDim.x;
    const int t = threadIdx.x, lane = t % kWave, w = t / kWave, pg = lane / 16, li = lane % 16;
    const int len = max(1, min(lens[b] + 1, max_blocks * kBlock));  // never past the block table
    int per = (len + splits - 1) / splits;
    per = (per + kBlock - 1) / kBlock * kBlock;
    const int p0 = split * per, p1 = min(len, p0 + per);
    const int32_t* bt = block_table + (size_t)b * max_blocks;
    const int nq = nkv * G;

    float qr[G][16], acc[G][16], m[G], l[G];
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        const float* qs = q + ((size_t)b * nq + g * G + gi) * kHD + 16 * li;
#pragma unroll
        for (int d = 0; d < 16; d += 4) {
            float4 v = *(const float4*)(qs + d);
            qr[gi][d] = v.x * 0.0625f; qr[gi][d + 1] = v.y * 0.0625f;  // 1/sqrt(256), exact
            qr[gi][d + 2] = v.z * 0.0625f; qr[gi][d + 3] = v.w * 0.0625f;
        }
#pragma unroll
        for (int d = 0; d < 16; d++) acc[gi][d] = 0.0f;
        m[gi] = -INFINITY;
        l[gi] = 0.0f;
    }
    for (int p = p0 + 4 * w + pg; p < p1; p += 16) {
        const size_t at = kv_index(bt, p, nkv, g) + 16 * li;
        const u32x4* kp = (const u32x4*)(k_pool + at);
        const u32x4* vp = (const u32x4*)(v_pool + at);
        const u32x4 k0 = __builtin_nontemporal_load(kp), k1 = __builtin_nontemporal_load(kp + 1);
        const u32x4 v0 = __builtin_nontemporal_load(vp), v1 = __builtin_nontemporal_load(vp + 1);
        const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        const uint32_t vw[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        float kf[16], vf[16];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            kf[2 * i] = lo_h(kw[i]); kf[2 * i + 1] = hi_h(kw[i]);
            vf[2 * i] = lo_h(vw[i]); vf[2 * i + 1] = hi_h(vw[i]);
        }
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < 16; d++) s = fmaf(qr[gi][d], kf[d], s);
            s = group16_sum(s);
            float pw;
            if (s > m[gi]) {
                const float corr = expf(m[gi] - s);
                m[gi] = s;
                l[gi] *= corr;
#pragma unroll
                for (int d = 0; d < 16; d++) acc[gi][d] *= corr;
                pw = 1.0f;
            } else {
                pw = expf(s - m[gi]);
            }
            l[gi] += pw;
#pragma unroll
            for (int d = 0; d < 16; d++) acc[gi][d] = fmaf(pw, vf[d], acc[gi][d]);
        }
    }
    // merge the 4 position groups of the wave (lanes li, li+16, li+32, li+48)
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
#pragma unroll
        for (int mask = 16; mask <= 32; mask <<= 1) {
            const float mo = __shfl_xor(m[gi], mask, kWave), lo = __shfl_xor(l[gi], mask, kWave);
            const float mn = fmaxf(m[gi], mo);
            const float ca = mn == -INFINITY ? 0.0f : expf(m[gi] - mn), cb = mn == -INFINITY ? 0.0f : expf(mo - mn);
#pragma unroll
            for (int d = 0; d < 16; d++) {
                const float ao = __shfl_xor(acc[gi][d], mask, kWave);
                acc[gi][d] = acc[gi][d] * ca + ao * cb;
            }
            l[gi] = l[gi] * ca + lo * cb;
            m[gi] = mn;
        }
        if (pg == 0) {
#pragma unroll
            for (int d = 0; d < 16; d++) s_acc[w][gi][16 * li + d] = acc[gi][d];
            if (li == 0) { s_ml[w][gi][0] = m[gi]; s_ml[w][gi][1] = l[gi]; }
        }
    }
    __syncthreads();
    // merge the 4 waves: thread t owns dim t for every head of the group
    const size_t pbase = (((size_t)b * nkv + g) * splits + split) * G;
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        float mn = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) mn = fmaxf(mn, s_ml[i][gi][0]);
        float lsum = 0.0f, a = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float c = mn == -INFINITY ? 0.0f : expf(s_ml[i][gi][0] - mn);
            lsum += s_ml[i][gi][1] * c;
            a += s_acc[i][gi][t] * c;
        }
        part_acc[(pbase + gi) * kHD + t] = a;
        if (t == 0) { part_ml[(pbase + gi) * 2] = mn; part_ml[(pbase + gi) * 2 + 1] = lsum; }
    }
}

// Merge the splits of query head blockIdx.x of sequence blockIdx.y; with `gate`, multiply by
// sigmoid(gate) (shaders.rs:626-629).
__global__ __launch_bounds__(kAttnThreads) void k_attn_combine(const float* __restrict__ part_ml, const float* __restrict__ part_acc,
                                                               int nkv, int G, int splits, const float* __restrict__ gate,
                                                               float* __restrict__ out) {
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x, g = h / G, gi = h % G, nq = nkv * G;
    float mn = -INFINITY;
    for (int s = 0; s < splits; s++) mn = fmaxf(mn, part_ml[((((size_t)b * nkv + g) * splits + s) * G + gi) * 2]);
    float lsum = 0.0f, a = 0.0f;
    for (int s = 0; s < splits; s++) {
        const size_t i = (((size_t)b * nkv + g) * splits + s) * G + gi;
        const float ms = part_ml[i * 2];
        if (ms == -INFINITY) continue;
        const float c = expf(ms - mn);
        lsum += part_ml[i * 2 + 1] * c;
        a += part_acc[i * kHD + t] * c;
    }
    float o = a / lsum;
    if (gate) o = o / (1.0f + expf(-gate[h * kHD + t]));
    out[((size_t)b * nq + h) * kHD + t] = o;
}

template <int G>
static void launch_partial(const float* q, const uint16_t* kp, const uint16_t* vp, const int32_t* bt, int max_blocks,
                           const int32_t* lens, int nkv, float* ml, float* acc, int splits, int batch, hipStream_t st) {
    hipLaunchKernelGGL((k_attn_partial<G>), dim3(splits, nkv, batch), dim3(kAttnThreads), 0, st, q, kp, vp, bt,
                       max_blocks, lens, nkv, ml, acc);
}

static void partial_by_g(int G, const float* q, const uint16_t* kp, const uint16_t* vp, const int32_t* bt, int max_blocks,
                         const int32_t* lens, int nkv, float* ml, float* acc, int splits, int batch, hipStream_t st) {
    switch (G) {
        case 1: launch_partial<1>(q, kp, vp, bt, max_blocks, lens, nkv, ml, acc, splits, batch, st); break;
        case 2: launch_partial<2>(q, kp, vp, bt, max_blocks, lens, nkv, ml, acc, splits, batch, st); break;
        default: launch_partial<4>(q, kp, vp, bt, max_blocks, lens, nkv, ml, acc, splits, batch, st); break;
    }
}

void launch_attention_model(const AttnModelArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(k_attn_prep, dim3(a.nq + a.nkv), dim3(kAttnThreads), 0, st, a);
    const int G = a.nq / a.nkv;
    // tok[1] is the position; the partial kernel attends lens[0] + 1 = pos + 1 positions.
    partial_by_g(G, a.qbuf, a.k_pool, a.v_pool, a.block_table, a.max_blocks, (const int32_t*)(a.tok + 1), a.nkv,
                 a.part_ml, a.part_acc, a.splits, 1, st);
    hipLaunchKernelGGL(k_attn_combine, dim3(a.nq, 1), dim3(kAttnThreads), 0, st, a.part_ml, a.part_acc, a.nkv, G,
                       a.splits, a.proj + a.nq * kHD, a.out);
}

void launch_paged_attn(const float* q, const float* k_new, const float* v_new, uint16_t* k_pool, uint16_t* v_pool,
                       const int32_t* block_table, int max_blocks, const int32_t* ctx, float* out, int batch, int nq,
                       int nkv, float* part_ml, float* part_acc, int splits, hipStream_t st) {
    hipLaunchKernelGGL(k_kv_append, dim3(nkv, batch), dim3(kAttnThreads), 0, st, k_new, v_new, k_pool, v_pool,
                       block_table, max_blocks, ctx, nkv);
    const int G = nq / nkv;
    partial_by_g(G, q, k_pool, v_pool, block_table, max_blocks, ctx, nkv, part_ml, part_acc, splits, batch, st);
    hipLaunchKernelGGL(k_attn_combine, dim3(nq, batch), dim3(kAttnThreads), 0, st, part_ml, part_acc, nkv, G, splits,
                       (const float*)nullptr, out);
}

}  // namespace qne
