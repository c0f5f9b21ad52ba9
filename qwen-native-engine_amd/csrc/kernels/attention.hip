// GQA attention decode over a paged f16 KV cache (head_dim 256, 16-token blocks).
//
// Reference: the decode kernel `attention` (kernels/src/shaders.rs:522-633), which runs one
// workgroup per query head over an f32 cache with all scores in LDS. Design for gfx950:
//  - the cache is paged: pools [block][kv_head][16][256] f16, a block table maps logical blocks;
//  - split-context ("flash decoding") partials: workgroup (split, kv_head, seq) streams a slice
//    of the context once for all query heads that share the kv head (GQA reuse);
//  - a wave covers 2 positions per step, 32 lanes per position, 8 dims (16 bytes of K and of V)
//    per lane, with the next step's rows in flight; scores are half-wave DPP sums; softmax is
//    online (running max / sum) in base 2;
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

// Batched model form, grid (nq + nkv, rows): row b reads its projection at proj + b * proj_stride,
// sits at position pos[b] and appends through block table row block_table + b * bt_stride (rows of
// one sequence share a row: bt_stride 0).
__global__ __launch_bounds__(kAttnThreads) void k_attn_prep_rows(AttnRowsArgs a) {
    __shared__ float sh[kHD];
    __shared__ float red[16];
    const int t = threadIdx.x, hb = blockIdx.x, b = blockIdx.y;
    const uint32_t pos = (uint32_t)a.pos[b];
    const float* proj = a.proj + (size_t)b * a.proj_stride;
    if (hb < a.nq) {
        const float x = proj[hb * kHD + t];
        a.qbuf[((size_t)b * a.nq + hb) * kHD + t] = norm_rope(x, a.norms, a.inv_freq, a.rope_dim, pos, sh, red);
    } else {
        const int g = hb - a.nq;
        const float* kp = proj + 2 * a.nq * kHD;
        const float kr = norm_rope(kp[g * kHD + t], a.norms + kHD, a.inv_freq, a.rope_dim, pos, sh, red);
        const size_t at = kv_index(a.block_table + (size_t)b * a.bt_stride, (int)pos, a.nkv, g) + t;
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

// Split-context partials. Grid (splits, nkv, batch), 4 waves. Sequence b attends positions
// 0..len-1 with len = lens[b] + 1 (lens = tok + 1 for the model, ctx for the raw form). A wave takes
// two positions per step (one per 32-lane half; a lane holds 8 dims, 16 bytes of K and of V) and
// loads the next step's rows while it computes the current ones. Scores are half-wave DPP sums.
// The softmax runs in base 2: q is pre-scaled by log2(e) / sqrt(256), so each weight is one
// exp2, and the partial maxima and sums are in that base (the combine uses the same base).
template <int G>
__global__ __launch_bounds__(kAttnThreads) void k_attn_partial(const float* __restrict__ q, const uint16_t* __restrict__ k_pool,
                                                               const uint16_t* __restrict__ v_pool,
                                                               const int32_t* __restrict__ block_table, int max_blocks,
                                                               int bt_stride, const int32_t* __restrict__ lens, int nkv,
                                                               float* __restrict__ part_ml, float* __restrict__ part_acc) {
    __shared__ float s_ml[4][G][2];
    __shared__ __attribute__((aligned(16))) float s_acc[4][G][kHD];
    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z, splits = gridDim.x;
    const int t = threadIdx.x, lane = t % kWave, w = t / kWave, half = lane >> 5, li = lane & 31;
    const int len = max(1, min(lens[b] + 1, max_blocks * kBlock));  // never past the block table
    int per = (len + splits - 1) / splits;
    per = (per + kBlock - 1) / kBlock * kBlock;
    const int p0 = split * per, p1 = min(len, p0 + per);
    const int32_t* bt = block_table + (size_t)b * bt_stride;
    const int nq = nkv * G;
    constexpr float kScale = 1.4426950408889634f * 0.0625f;  // log2(e) / sqrt(256)

    float qr[G][8], acc[G][8], m[G], l[G];
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        const float* qs = q + ((size_t)b * nq + g * G + gi) * kHD + 8 * li;
        const float4 a0 = *(const float4*)qs, a1 = *(const float4*)(qs + 4);
        qr[gi][0] = a0.x * kScale; qr[gi][1] = a0.y * kScale; qr[gi][2] = a0.z * kScale; qr[gi][3] = a0.w * kScale;
        qr[gi][4] = a1.x * kScale; qr[gi][5] = a1.y * kScale; qr[gi][6] = a1.z * kScale; qr[gi][7] = a1.w * kScale;
#pragma unroll
        for (int d = 0; d < 8; d++) acc[gi][d] = 0.0f;
        m[gi] = -INFINITY;
        l[gi] = 0.0f;
    }
    auto load = [&](int p, u32x4& kw, u32x4& vw) {
        if (p < p1) {
            const size_t at = kv_index(bt, p, nkv, g) + 8 * li;
            kw = __builtin_nontemporal_load((const u32x4*)(k_pool + at));
            vw = __builtin_nontemporal_load((const u32x4*)(v_pool + at));
        } else {
            kw = u32x4{0u, 0u, 0u, 0u};
            vw = kw;
        }
    };
    u32x4 kc, vc, kn, vn;
    load(p0 + 2 * w + half, kc, vc);
    for (int base = p0 + 2 * w; base < p1; base += 8) {  // wave-uniform
        const int pc = base + half;
        const bool valid = pc < p1;
        load(pc + 8, kn, vn);
        float kf[8], vf[8];
        kf[0] = lo_h(kc.x); kf[1] = hi_h(kc.x); kf[2] = lo_h(kc.y); kf[3] = hi_h(kc.y);
        kf[4] = lo_h(kc.z); kf[5] = hi_h(kc.z); kf[6] = lo_h(kc.w); kf[7] = hi_h(kc.w);
        vf[0] = lo_h(vc.x); vf[1] = hi_h(vc.x); vf[2] = lo_h(vc.y); vf[3] = hi_h(vc.y);
        vf[4] = lo_h(vc.z); vf[5] = hi_h(vc.z); vf[6] = lo_h(vc.w); vf[7] = hi_h(vc.w);
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            float s = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; d++) s = fmaf(qr[gi][d], kf[d], s);
            s = half_sum_dpp(s, lane);
            s = valid ? s : -INFINITY;
            // The running sum and accumulators are kept relative to m; m moves (and they are
            // rescaled) only when a score exceeds it by more than 8 (a weight of 2^8 at most),
            // which after the first positions is rare, so most positions cost one exp2 (the
            // hardware v_exp_f32: weights below 2^-126 flush to 0).
            if (__builtin_amdgcn_ballot_w64(s > m[gi] + 8.0f)) {  // wave-uniform branch
                const float mn = fmaxf(m[gi], s);
                const float corr = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[gi] - mn);
                m[gi] = mn;
                l[gi] *= corr;
#pragma unroll
                for (int d = 0; d < 8; d++) acc[gi][d] *= corr;
            }
            const float pw = s == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s - m[gi]);  // an invalid position weighs 0
            l[gi] += pw;
#pragma unroll
            for (int d = 0; d < 8; d++) acc[gi][d] = fmaf(pw, vf[d], acc[gi][d]);
        }
        kc = kn;
        vc = vn;
    }
    // merge the two halves of the wave, then the 4 waves through LDS
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        const float mo = lane_xor32(m[gi], lane), lo = lane_xor32(l[gi], lane);
        const float mn = fmaxf(m[gi], mo);
        const float ca = mn == -INFINITY ? 0.0f : exp2f(m[gi] - mn), cb = mn == -INFINITY ? 0.0f : exp2f(mo - mn);
#pragma unroll
        for (int d = 0; d < 8; d++) acc[gi][d] = acc[gi][d] * ca + lane_xor32(acc[gi][d], lane) * cb;
        l[gi] = l[gi] * ca + lo * cb;
        m[gi] = mn;
        if (half == 0) {
            *(float4*)&s_acc[w][gi][8 * li] = make_float4(acc[gi][0], acc[gi][1], acc[gi][2], acc[gi][3]);
            *(float4*)&s_acc[w][gi][8 * li + 4] = make_float4(acc[gi][4], acc[gi][5], acc[gi][6], acc[gi][7]);
            if (li == 0) { s_ml[w][gi][0] = m[gi]; s_ml[w][gi][1] = l[gi]; }
        }
    }
    __syncthreads();
    // thread t owns dim t for every head of the group
    const size_t pbase = (((size_t)b * nkv + g) * splits + split) * G;
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        float mn = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) mn = fmaxf(mn, s_ml[i][gi][0]);
        float lsum = 0.0f, a = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float c = mn == -INFINITY ? 0.0f : exp2f(s_ml[i][gi][0] - mn);
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
                                                               int gate_stride, float* __restrict__ out) {
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x, g = h / G, gi = h % G, nq = nkv * G;
    float mn = -INFINITY;
    for (int s = 0; s < splits; s++) mn = fmaxf(mn, part_ml[((((size_t)b * nkv + g) * splits + s) * G + gi) * 2]);
    float lsum = 0.0f, a = 0.0f;
    for (int s = 0; s < splits; s++) {
        const size_t i = (((size_t)b * nkv + g) * splits + s) * G + gi;
        const float ms = part_ml[i * 2];
        if (ms == -INFINITY) continue;
        const float c = exp2f(ms - mn);  // the partials' maxima are in base 2
        lsum += part_ml[i * 2 + 1] * c;
        a += part_acc[i * kHD + t] * c;
    }
    float o = a / lsum;
    if (gate) o = o / (1.0f + expf(-gate[(size_t)b * gate_stride + h * kHD + t]));
    out[((size_t)b * nq + h) * kHD + t] = o;
}

template <int G>
static void launch_partial(const float* q, const uint16_t* kp, const uint16_t* vp, const int32_t* bt, int max_blocks,
                           int bt_stride, const int32_t* lens, int nkv, float* ml, float* acc, int splits, int batch,
                           hipStream_t st) {
    hipLaunchKernelGGL((k_attn_partial<G>), dim3(splits, nkv, batch), dim3(kAttnThreads), 0, st, q, kp, vp, bt,
                       max_blocks, bt_stride, lens, nkv, ml, acc);
}

static void partial_by_g(int G, const float* q, const uint16_t* kp, const uint16_t* vp, const int32_t* bt, int max_blocks,
                         int bt_stride, const int32_t* lens, int nkv, float* ml, float* acc, int splits, int batch,
                         hipStream_t st) {
    switch (G) {
        case 1: launch_partial<1>(q, kp, vp, bt, max_blocks, bt_stride, lens, nkv, ml, acc, splits, batch, st); break;
        case 2: launch_partial<2>(q, kp, vp, bt, max_blocks, bt_stride, lens, nkv, ml, acc, splits, batch, st); break;
        default: launch_partial<4>(q, kp, vp, bt, max_blocks, bt_stride, lens, nkv, ml, acc, splits, batch, st); break;
    }
}

void launch_attention_model(const AttnModelArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(k_attn_prep, dim3(a.nq + a.nkv), dim3(kAttnThreads), 0, st, a);
    const int G = a.nq / a.nkv;
    // tok[1] is the position; the partial kernel attends lens[0] + 1 = pos + 1 positions.
    partial_by_g(G, a.qbuf, a.k_pool, a.v_pool, a.block_table, a.max_blocks, a.max_blocks, (const int32_t*)(a.tok + 1),
                 a.nkv, a.part_ml, a.part_acc, a.splits, 1, st);
    hipLaunchKernelGGL(k_attn_combine, dim3(a.nq, 1), dim3(kAttnThreads), 0, st, a.part_ml, a.part_acc, a.nkv, G,
                       a.splits, a.proj + a.nq * kHD, 0, a.out);
}

void launch_attention_rows(const AttnRowsArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(k_attn_prep_rows, dim3(a.nq + a.nkv, a.rows), dim3(kAttnThreads), 0, st, a);
    const int G = a.nq / a.nkv;
    partial_by_g(G, a.qbuf, a.k_pool, a.v_pool, a.block_table, a.max_blocks, a.bt_stride, a.pos, a.nkv, a.part_ml,
                 a.part_acc, a.splits, a.rows, st);
    hipLaunchKernelGGL(k_attn_combine, dim3(a.nq, a.rows), dim3(kAttnThreads), 0, st, a.part_ml, a.part_acc, a.nkv, G,
                       a.splits, a.proj + a.nq * kHD, (int)a.proj_stride, a.out);
}

void launch_paged_attn(const float* q, const float* k_new, const float* v_new, uint16_t* k_pool, uint16_t* v_pool,
                       const int32_t* block_table, int max_blocks, const int32_t* ctx, float* out, int batch, int nq,
                       int nkv, float* part_ml, float* part_acc, int splits, hipStream_t st) {
    hipLaunchKernelGGL(k_kv_append, dim3(nkv, batch), dim3(kAttnThreads), 0, st, k_new, v_new, k_pool, v_pool,
                       block_table, max_blocks, ctx, nkv);
    const int G = nq / nkv;
    partial_by_g(G, q, k_pool, v_pool, block_table, max_blocks, max_blocks, ctx, nkv, part_ml, part_acc, splits, batch, st);
    hipLaunchKernelGGL(k_attn_combine, dim3(nq, batch), dim3(kAttnThreads), 0, st, part_ml, part_acc, nkv, G, splits,
                       (const float*)nullptr, 0, out);
}

}  // namespace qne
