// Gated DeltaNet kernels (dk = dv = 128).
//
// Reference: the decode step `gdn` (kernels/src/shaders.rs:436-520) and the chunk kernel `gdn_b`
// (kernels/src/batch.rs:166-255). Design for gfx950: the decode step runs one 512-thread
// workgroup per (sequence, head) and reads the head's 64 KiB value-major state tile once, in
// address order (each wave instruction one contiguous KiB), into registers: thread t holds keys
// 4 (t % 32)..+3 of the value columns t / 32 + 16 r, so a column lies in one half-wave and S^T k,
// S^T q are half-wave DPP sums; the tile is written back from the same registers. The
// multi-token kernels keep the tile in registers across all tokens of the launch.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"
#include "operand.hpp"

namespace qne {

constexpr int kDK = 128, kDV = 128, kGdnThreads = 512;
constexpr int kNT = 2;  // buffer cache policy: non-temporal (the state is streamed once per step)

struct DeltaShared {
    float q[kDK], k[kDK], v[kDV];
    float part[2][4][kDV];
    float dv[kDV];
    float o[kDV];
    float z[kDV];
    float red[16];
    float kq, g, beta;
};

// The model keeps each head's state value-major, S_T[t][j] = S[j][t]: the 128 keys of one value
// column are contiguous, so a column (what one wave updates in the persistent decode kernel) is a
// single 512-byte read.
// The decode step reads the value-major tile as 16-byte pieces in address order (piece f of the
// tile: column f / 32, keys 4 (f % 32)..+3; each wave instruction one contiguous KiB) and keeps
// them in that layout: thread t owns piece t + 512 r (r = 0..7). The pieces go through one buffer
// resource (the tile's base in scalar registers, piece r at a scalar offset of 8 KiB r),
// non-temporal: no 64-bit address per piece for the compiler to keep live, which holds the kernel
// to 64 VGPRs, so four 8-wave workgroups fit a CU and a 64-sequence batch (1024 workgroups) runs
// in one round.
typedef float f4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(float* S) {
    return __builtin_amdgcn_make_buffer_rsrc(S, (short)0, kDK * kDV * 4, 0x00020000);
}
__device__ __forceinline__ void load_tile_rs(f4v (&v)[8], __amdgpu_buffer_rsrc_t rs) {
#pragma unroll
    for (int r = 0; r < 8; r++)
        v[r] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * threadIdx.x, 16 * kGdnThreads * r, kNT));
}
__device__ __forceinline__ void store_tile_rs(const f4v (&v)[8], __amdgpu_buffer_rsrc_t rs) {
#pragma unroll
    for (int r = 0; r < 8; r++)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[r]), rs, 16 * threadIdx.x, 16 * kGdnThreads * r, kNT);
}

// Model decode step for head blockIdx.x: conv + SiLU on the head's q, k, v channels, L2 norms,
// gates, delta rule, gated RMSNorm (shaders.rs:436-520).
// proj = [q(H*dk) k(H*dk) v(H*dv) z(H*dv) a(H) b(H)], prm = [dt_bias(H) A_neg_exp(H) norm_w(dv)].
__global__ __launch_bounds__(kGdnThreads, 8) void k_gdn_decode(const float* __restrict__ proj, float* __restrict__ conv_state,
                                                            const float* __restrict__ conv_w, float* __restrict__ state,
                                                            float* __restrict__ out, const float* __restrict__ prm, int H,
                                                            GdnRowStrides rs, GdnRowsIO io) {
    __shared__ DeltaShared sh;
    const int h = blockIdx.x, t = threadIdx.x, lane = t % kWave, w = t / kWave, b = blockIdx.y;
    // row b of a batch: its own projection, conv and recurrent state, output
    proj += (size_t)b * rs.proj;
    conv_state += (size_t)b * rs.conv;
    state += (size_t)b * rs.state;
    if (out) out += (size_t)b * rs.out;
    const int col = t & (kDV - 1);
    float* S = state + (size_t)h * kDK * kDV;
    f4v tv[8];
    // The row's projection values this thread reads: channel ch (q, k or v; threads < 384; z of
    // column t - 384 for threads 384..511) and a (thread 0) or b (thread 1). Stored, or the
    // in-projection's split partials summed in split order times the row's 1 / rms from the sums
    // of x^2 of its operand, as k_gemm_reduce computes them. Loads complete in order: the
    // channel's partials and its conv state and weights are issued before the state tile, so the
    // conv does not wait for the tile; the gates' partials (threads 0 and 1) after it, as they are
    // summed only after the conv's barrier.
    const int zoff = 2 * H * kDK + 2 * H * kDV;  // a[H] then b[H] follow z
    const int ch = t < 128 ? h * kDK + t
                           : (t < 256 ? H * kDK + h * kDK + (t - 128)
                                      : (t < 384 ? 2 * H * kDK + h * kDV + (t - 256) : 2 * H * kDK + H * kDV + h * kDV + col));
    const int gch = zoff + (t == 0 ? h : H + h);
    const int nchunks_in = io.k_in / kChunk;
    const float ss_in = io.part && t < nchunks_in ? ((const float*)(io.x_in + (size_t)t * kChunkBytes))[kSsOff / 4 + b] : 0.0f;
    const float* pbase = io.part ? io.part + (size_t)b * io.n : proj;
    const int nsp = io.part ? io.splits : 1;
    Split8 pc;
    pc.load(pbase + ch, nsp, io.split_stride);
    float* st = conv_state + (size_t)(t < 384 ? ch : 0) * 4;
    const float* cw = conv_w + (size_t)(t < 384 ? ch : 0) * 4;
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, w0 = 0.0f, w1 = 0.0f, w2 = 0.0f, w3 = 0.0f;
    if (t < 384) {
        s0 = st[0]; s1 = st[1]; s2 = st[2];
        w0 = cw[0]; w1 = cw[1]; w2 = cw[2]; w3 = cw[3];
    }
    asm volatile("" ::: "memory");  // keeps the loads above ahead of the tile's
    const __amdgpu_buffer_rsrc_t trs = tile_rsrc(S);
    load_tile_rs(tv, trs);  // in flight while the conv runs
    float inv = 1.0f;
    if (io.part) {
        // row_inv_rms: one chunk sum per thread (nchunks_in <= 256), the block sum in wave order
        inv = 1.0f / sqrtf(block_sum<kGdnThreads>(ss_in, sh.red) / (float)io.k_in + io.eps);
        __syncthreads();  // sh.red is reused below
    }
    const float x = pc.sum(pbase + ch, nsp, io.split_stride) * inv;
    if (t >= 384) sh.z[t - 384] = x;

    float val = 0.0f;
    if (t < 384) {
        const float y = s0 * w0 + s1 * w1 + s2 * w2 + x * w3;
        st[0] = s1; st[1] = s2; st[2] = x;
        val = silu(y);
    }
    const float ss = wave_sum_xor(val * val);
    if (lane == 0) sh.red[w] = ss;
    __syncthreads();
    if (t < 128) sh.q[t] = val * (1.0f / sqrtf(sh.red[0] + sh.red[1] + 1e-6f)) * 0.08838834764831845f;
    else if (t < 256) sh.k[t - 128] = val * (1.0f / sqrtf(sh.red[2] + sh.red[3] + 1e-6f));
    else if (t < 384) sh.v[t - 256] = val;
    if (t < 2) {  // the gates: issued after the tile, summed in split order like the channels
        Split8 pg;
        pg.load(pbase + gch, nsp, io.split_stride);
        const float gx = pg.sum(pbase + gch, nsp, io.split_stride) * inv;
        if (t == 0) sh.g = expf(prm[H + h] * logf(1.0f + expf(gx + prm[h])));
        else sh.beta = 1.0f / (1.0f + expf(-gx));
    }
    __syncthreads();
    if (w == 0) {
        float p = sh.k[lane] * sh.q[lane] + sh.k[lane + 64] * sh.q[lane + 64];
        p = wave_sum_xor(p);
        if (lane == 0) sh.kq = p;
    }
    __syncthreads();
    // The delta rule on the tile as loaded: thread t holds keys 4 (t % 32)..+3 of the value
    // columns t / 32 + 16 r (r = 0..7), so each column lies in one half-wave and its S^T k and
    // S^T q are half-wave sums; the updated pieces are stored back where they were read.
    {
        const int kb = 4 * (t & 31), hw = t >> 5;
        const f4v k4 = *(const f4v*)&sh.k[kb], q4 = *(const f4v*)&sh.q[kb];
        const float g = sh.g, beta = sh.beta, kq = sh.kq;
#pragma unroll
        for (int r = 0; r < 8; r++) {
            float sk = tv[r].x * k4.x, sq = tv[r].x * q4.x;
            sk = fmaf(tv[r].y, k4.y, sk);
            sq = fmaf(tv[r].y, q4.y, sq);
            sk = fmaf(tv[r].z, k4.z, sk);
            sq = fmaf(tv[r].z, q4.z, sq);
            sk = fmaf(tv[r].w, k4.w, sk);
            sq = fmaf(tv[r].w, q4.w, sq);
            sk = half_sum_dpp(sk, lane);
            sq = half_sum_dpp(sq, lane);
            const int c = hw + 16 * r;
            const float d = beta * (sh.v[c] - g * sk);
            tv[r].x = fmaf(g, tv[r].x, d * k4.x);
            tv[r].y = fmaf(g, tv[r].y, d * k4.y);
            tv[r].z = fmaf(g, tv[r].z, d * k4.z);
            tv[r].w = fmaf(g, tv[r].w, d * k4.w);
            if ((t & 31) == 0) sh.o[c] = g * sq + d * kq;
        }
        store_tile_rs(tv, trs);
    }
    __syncthreads();
    // gated RMSNorm over the head's dv outputs (threads 0..127 = waves 0 and 1, one column each)
    const float o = t < kDV ? sh.o[t] : 0.0f;
    const float oo = wave_sum_xor(o * o);
    if (lane == 0) sh.red[w] = oo;
    __syncthreads();
    if (t < kDV) {
        const float rinv = 1.0f / sqrtf((sh.red[0] + sh.red[1]) / (float)kDV + 1e-6f);
        const float y = o * rinv * silu(sh.z[col]) * prm[2 * H + col];
        if (out) out[h * kDV + col] = y;
        if (io.frag_out)  // waves 0 and 1: 64 columns of the row each
            emit_x(io.frag_out, (size_t)(H * kDV / kChunk) * kChunkBytes, b, h * kDV + col, y, 1.0f, io.order_out, lane);
    }
}

// The bare delta rule for one token of sequence blockIdx.y, head blockIdx.x, on the key-major
// tile S[j][c] (key j, value column c): thread t holds columns 4 (t % 32)..+3 of keys t / 32 + 16 r
// (r = 0..7) as 16-byte pieces, so every wave instruction moves one contiguous KiB. Each thread
// dots its 8 keys with k and q for its 4 columns; the 16 key groups' partial sums meet in LDS and
// are added in key-group order; then every thread updates its pieces with the column's dv.
__global__ __launch_bounds__(kGdnThreads) void k_delta_rule(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v, const float* __restrict__ beta,
                                                            const float* __restrict__ g, float* __restrict__ state,
                                                            float* __restrict__ out, int H) {
    constexpr int kGroups = kGdnThreads / 32;  // key groups: 16
    __shared__ float sq_[kDK], sk_[kDK], sv_[kDV], sdv[kDV];
    __shared__ f4v spart[2][kGroups][kDV / 4];
    __shared__ float sred[2], skq;
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int c4 = t & 31, kg = t >> 5;
    const size_t bh = (size_t)b * H + h;
    f4v* S = (f4v*)(state + bh * kDK * kDV) + c4;
    f4v s[8];
#pragma unroll
    for (int r = 0; r < 8; r++) s[r] = __builtin_nontemporal_load(S + (size_t)(kg + kGroups * r) * (kDV / 4));
    if (t < 128) sq_[t] = q[bh * kDK + t];
    else if (t < 256) sk_[t - 128] = k[bh * kDK + t - 128];
    else if (t < 384) sv_[t - 256] = v[bh * kDV + t - 256];
    if (t == 0) { sred[0] = g[bh]; sred[1] = beta[bh]; }
    __syncthreads();
    if (t < kWave) {
        float p = sk_[t] * sq_[t] + sk_[t + 64] * sq_[t + 64];
        p = wave_sum(p);
        if (t == 0) skq = p;
    }
    f4v pk = {0.0f, 0.0f, 0.0f, 0.0f}, pq = pk;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const float kj = sk_[kg + kGroups * r], qj = sq_[kg + kGroups * r];
        pk += s[r] * kj;
        pq += s[r] * qj;
    }
    spart[0][kg][c4] = pk;
    spart[1][kg][c4] = pq;
    __syncthreads();
    if (t < kDV) {
        // column t: S^T k and S^T q summed over the key groups in order
        float sk = 0.0f, sq = 0.0f;
#pragma unroll
        for (int gi = 0; gi < kGroups; gi++) {
            sk += ((const float*)spart[0][gi])[t];
            sq += ((const float*)spart[1][gi])[t];
        }
        const float gg = sred[0], d = sred[1] * (sv_[t] - gg * sk);
        sdv[t] = d;
        out[bh * kDV + t] = gg * sq + d * skq;
    }
    __syncthreads();
    const float gg = sred[0];
    const f4v d4 = *(const f4v*)&sdv[4 * c4];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const float kj = sk_[kg + kGroups * r];
        s[r] = gg * s[r] + d4 * kj;
        __builtin_nontemporal_store(s[r], S + (size_t)(kg + kGroups * r) * (kDV / 4));
    }
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the row's total.
__device__ __forceinline__ float row16_sum(float v) {
    v += QNE_DPP(v, kDppXor1);
    v += QNE_DPP(v, kDppXor2);
    v += QNE_DPP(v, kDppHalfMirror);
    v += QNE_DPP(v, kDppMirror);
    return v;
}

// The delta rule over T tokens with the value columns split across waves: a wave owns (sequence
// b, head h, columns 4c..4c+3); row r of the wave (lanes 16r..16r+15) owns column 4c + r, and lane
// i of the row keeps keys 8i..8i+7 of it in registers for the whole launch. A token costs 8 FMAs
// each for the lane's shares of (S^T k)_col and (S^T q)_col and of k.q, three 16-lane DPP sums
// (no cross-row traffic), and 8 state FMAs; the next tokens' inputs load while one runs. The
// waves are independent (no LDS, no barrier), so B * H * 32 of them run at once.
// Layouts: q,k [B][T][H][dk], v,out [B][T][H][dv], beta,g [B][T][H], state [B][H][dk][dv], or with
// value_major the model's [B][H][dv][dk] (a lane's 8 keys then contiguous).
__global__ __launch_bounds__(256) void k_delta_rule_cols(const float* __restrict__ q, const float* __restrict__ k,
                                                         const float* __restrict__ v, const float* __restrict__ beta,
                                                         const float* __restrict__ g, float* __restrict__ state,
                                                         float* __restrict__ out, int T, int H, int waves,
                                                         int value_major) {
    const int lane = threadIdx.x & (kWave - 1), r = lane >> 4, i = lane & 15;
    const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (gw >= waves) return;
    constexpr int kGroups = kDV / 4;
    const int col = 4 * (gw % kGroups) + r, bh = gw / kGroups, h = bh % H, b = bh / H;
    const size_t jstride = value_major ? 1 : kDV;
    float* S = state + (size_t)bh * kDK * kDV + (value_major ? (size_t)col * kDK + 8 * i : (size_t)(8 * i) * kDV + col);
    float s[8];
#pragma unroll
    for (int j = 0; j < 8; j++) s[j] = S[j * jstride];
    struct In {
        float4 k0, k1, q0, q1;
        float v, beta, g;
    };
    auto load = [&](int n, In& x) {
        const size_t bth = ((size_t)b * T + n) * H + h;
        const float4* kp = (const float4*)(k + bth * kDK + 8 * i);
        const float4* qp = (const float4*)(q + bth * kDK + 8 * i);
        x.k0 = kp[0]; x.k1 = kp[1];
        x.q0 = qp[0]; x.q1 = qp[1];
        x.v = v[bth * kDV + col];
        x.beta = beta[bth];
        x.g = g[bth];
    };
    // kAhead tokens' inputs in flight in a register ring used in place (no copies, which would
    // make each token wait for the next one's loads); slot d is refilled after its token ran
    constexpr int kAhead = 4;
    In ring[kAhead];
#pragma unroll
    for (int d = 0; d < kAhead; d++)
        if (d < T) load(d, ring[d]);
    for (int n0 = 0; n0 < T; n0 += kAhead) {
#pragma unroll
        for (int d = 0; d < kAhead; d++) {
            const int n = n0 + d;
            if (n >= T) break;
            In& cur = ring[d];
            const float kk[8] = {cur.k0.x, cur.k0.y, cur.k0.z, cur.k0.w, cur.k1.x, cur.k1.y, cur.k1.z, cur.k1.w};
            const float qq[8] = {cur.q0.x, cur.q0.y, cur.q0.z, cur.q0.w, cur.q1.x, cur.q1.y, cur.q1.z, cur.q1.w};
            const float vv = cur.v, bb = cur.beta, gg = cur.g;
            if (n + kAhead < T) load(n + kAhead, cur);
            float sk = 0.0f, sq = 0.0f, kq = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                sk = fmaf(s[j], kk[j], sk);
                sq = fmaf(s[j], qq[j], sq);
                kq = fmaf(kk[j], qq[j], kq);
            }
            sk = row16_sum(sk);
            sq = row16_sum(sq);
            kq = row16_sum(kq);
            const float dv = bb * (vv - gg * sk);
#pragma unroll
            for (int j = 0; j < 8; j++) s[j] = fmaf(gg, s[j], kk[j] * dv);
            if (i == 0) out[(((size_t)b * T + n) * H + h) * kDV + col] = fmaf(gg, sq, dv * kq);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) S[j * jstride] = s[j];
}

// Tokens per workgroup of the chunk prep / post kernels: the conv window slides along them, so a
// channel's inputs are loaded once each (plus three), and their loads are all in flight at once.
constexpr int kChunkTok = 8;

// Prefill of a chunk of T tokens of one sequence, before the recurrence. Grid (ceil(T / 8), H, 3),
// 128 threads: workgroup (x, h, z) takes tokens 8 x .. + 7 of head h's q (z = 0), k (1) or v (2)
// channels, one per thread, so a 2048-token pass's 12288 two-wave workgroups run in three full
// rounds. Token n's projection row is proj + n * proj_stride. Causal conv + SiLU
// (shaders.rs:457-468) with the inputs of tokens n-3..n-1 taken from the chunk or, before it, from
// conv_state (read only; k_gdn_chunk_post shifts it); L2 norms of q (times 128^-1/2) and k; the q
// workgroup also computes g = exp(A_neg_exp ln(1 + e^(a + dt_bias))), beta = sigmoid(b)
// (:489-496). Outputs in the layouts of k_delta_rule_cols: q, k [T][H][dk], v [T][H][dv], g, beta
// [T][H]. Each token's arithmetic is that of one token per workgroup.
__global__ __launch_bounds__(kDK) void k_gdn_chunk_prep(const float* __restrict__ proj, int proj_stride,
                                                        const float* __restrict__ conv_state,
                                                        const float* __restrict__ conv_w, const float* __restrict__ prm,
                                                        int H, int T, float* __restrict__ qo, float* __restrict__ ko,
                                                        float* __restrict__ vo, float* __restrict__ go,
                                                        float* __restrict__ bo) {
    __shared__ float red[kChunkTok][2];
    const int n0 = blockIdx.x * kChunkTok, h = blockIdx.y, z = blockIdx.z, t = threadIdx.x, lane = t % kWave,
              w = t / kWave;
    const int ch = z == 0 ? h * kDK + t : (z == 1 ? H * kDK + h * kDK + t : 2 * H * kDK + h * kDV + t);
    const float* st = conv_state + (size_t)ch * 4;
    const float* cw = conv_w + (size_t)ch * 4;
    // inputs of tokens n0 - 3 .. n0 + 7 (before the chunk: the conv state; past T: unused)
    float in[kChunkTok + 3];
#pragma unroll
    for (int j = 0; j < kChunkTok + 3; j++) {
        const int m = n0 - 3 + j;
        in[j] = m < 0 ? st[3 + m] : (m < T ? proj[(size_t)m * proj_stride + ch] : 0.0f);
    }
    const float w0 = cw[0], w1 = cw[1], w2 = cw[2], w3 = cw[3];
    float val[kChunkTok];
#pragma unroll
    for (int i = 0; i < kChunkTok; i++) {
        const float y = in[i] * w0 + in[i + 1] * w1 + in[i + 2] * w2 + in[i + 3] * w3;
        val[i] = silu(y);
        if (z < 2) {
            const float ss = wave_sum(val[i] * val[i]);
            if (lane == 0) red[i][w] = ss;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kChunkTok; i++) {
        const int n = n0 + i;
        if (n >= T) break;
        const size_t nh = (size_t)n * H + h;
        if (z == 0) qo[nh * kDK + t] = val[i] * (1.0f / sqrtf(red[i][0] + red[i][1] + 1e-6f)) * 0.08838834764831845f;
        else if (z == 1) ko[nh * kDK + t] = val[i] * (1.0f / sqrtf(red[i][0] + red[i][1] + 1e-6f));
        else vo[nh * kDV + t] = val[i];
    }
    if (z == 0 && t < kChunkTok && n0 + t < T) {
        const int n = n0 + t;
        const size_t nh = (size_t)n * H + h;
        const float* row = proj + (size_t)n * proj_stride;
        const int zoff = 2 * H * kDK + 2 * H * kDV;  // a[H] then b[H] follow z
        const float a = row[zoff + h], b = row[zoff + H + h];
        go[nh] = expf(prm[H + h] * logf(1.0f + expf(a + prm[h])));
        bo[nh] = 1.0f / (1.0f + expf(-b));
    }
}

// After the recurrence. Grid (ceil(T / 8), H), 128 threads (one per value column), tokens
// 8 blockIdx.x .. + 7: two waves a workgroup, so every workgroup of a 2048-token pass is resident at
// once (the q, k, v channels of the conv-state shift are three per thread). Gated
// RMSNorm of token n's head output (shaders.rs:514-516) into mixed + n * mixed_stride (when set)
// and, with frag_out, staged as the out-projection's GEMM operand (column order order_out); the
// workgroup of the last token also shifts the conv state by the chunk (the inputs of the chunk's
// last three tokens).
__global__ __launch_bounds__(kDV) void k_gdn_chunk_post(const float* __restrict__ proj, int proj_stride,
                                                        float* __restrict__ conv_state, const float* __restrict__ prm,
                                                        int H, int T, const float* __restrict__ o,
                                                        float* __restrict__ mixed, int mixed_stride,
                                                        uint8_t* __restrict__ frag_out, int order_out) {
    __shared__ float red[kChunkTok][2];
    const int n0 = blockIdx.x * kChunkTok, h = blockIdx.y, t = threadIdx.x, lane = t % kWave, w = t / kWave;
    float v[kChunkTok], z[kChunkTok];
#pragma unroll
    for (int i = 0; i < kChunkTok; i++) {
        const int n = n0 + i;
        const bool live = n < T;
        v[i] = live ? o[((size_t)n * H + h) * kDV + t] : 0.0f;
        z[i] = live ? proj[(size_t)n * proj_stride + 2 * H * kDK + H * kDV + h * kDV + t] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kChunkTok; i++) {
        const float ss = wave_sum(v[i] * v[i]);
        if (lane == 0) red[i][w] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kChunkTok; i++) {
        const int n = n0 + i;
        if (n >= T) break;
        const float inv = 1.0f / sqrtf((red[i][0] + red[i][1]) / (float)kDV + 1e-6f);
        const float y = v[i] * inv * silu(z[i]) * prm[2 * H + t];
        if (mixed) mixed[(size_t)n * mixed_stride + h * kDV + t] = y;
        if (frag_out)  // the two waves: the two 64-column chunks of head h in row n
            emit_x(frag_out, (size_t)(H * kDV / kChunk) * kChunkBytes, n, h * kDV + t, y, 1.0f, order_out, lane);
    }
    if (n0 <= T - 1 && T - 1 < n0 + kChunkTok) {
        // channels q t, k t, v t of head h
        const int chs[3] = {h * kDK + t, H * kDK + h * kDK + t, 2 * H * kDK + h * kDV + t};
        float in[3][3];
#pragma unroll
        for (int u = 0; u < 3; u++) {
            const float* st = conv_state + (size_t)chs[u] * 4;
#pragma unroll
            for (int j = 0; j < 3; j++) {
                const int m = T - 3 + j;
                in[u][j] = m >= 0 ? proj[(size_t)m * proj_stride + chs[u]] : st[3 + m];
            }
        }
#pragma unroll
        for (int u = 0; u < 3; u++) {
            float* st = conv_state + (size_t)chs[u] * 4;
#pragma unroll
            for (int j = 0; j < 3; j++) st[j] = in[u][j];
        }
    }
}

void launch_gdn_chunk(const float* proj, int proj_stride, float* conv_state, const float* conv_w, float* state,
                      const float* prm, int heads, int tokens, float* q, float* k, float* v, float* g, float* beta,
                      float* o, float* mixed, int mixed_stride, hipStream_t st, int lead, float* wy_ws,
                      uint8_t* frag_out, int order_out) {
    const int tb = (tokens + kChunkTok - 1) / kChunkTok;
    hipLaunchKernelGGL(k_gdn_chunk_prep, dim3(tb, heads, 3), dim3(kDK), 0, st, proj, proj_stride, conv_state, conv_w,
                       prm, heads, tokens, q, k, v, g, beta);
    const int waves = heads * (kDV / 4);
    const size_t hk = (size_t)heads * kDK;  // floats of q, k, v, o per token
    // tokens [t0, t0 + n) in order on the state, one wave per 4 value columns
    auto sequential = [&](int t0, int n) {
        if (n > 0)
            hipLaunchKernelGGL(k_delta_rule_cols, dim3((waves + 3) / 4), dim3(256), 0, st, q + t0 * hk, k + t0 * hk,
                               v + t0 * hk, beta + (size_t)t0 * heads, g + (size_t)t0 * heads, state, o + t0 * hk, n,
                               heads, waves, 1);
    };
    const int head = wy_ws ? std::min(std::max(lead, 0), tokens) : tokens;
    const int blocks = wy_ws ? (tokens - head) / 64 : 0;
    sequential(0, head);
    if (blocks > 0)
        launch_delta_rule_wy(q + head * hk, k + head * hk, v + head * hk, beta + (size_t)head * heads,
                             g + (size_t)head * heads, state, o + head * hk, 1, 64 * blocks, heads, wy_ws, st, 1);
    sequential(head + 64 * blocks, tokens - head - 64 * blocks);
    hipLaunchKernelGGL(k_gdn_chunk_post, dim3(tb, heads), dim3(kDV), 0, st, proj, proj_stride, conv_state, prm,
                       heads, tokens, o, mixed, mixed_stride, frag_out, order_out);
}

void launch_gdn_decode(const float* proj, float* conv_state, const float* conv_w, float* state, float* out,
                       const float* prm, int heads, hipStream_t st) {
    hipLaunchKernelGGL(k_gdn_decode, dim3(heads), dim3(kGdnThreads), 0, st, proj, conv_state, conv_w, state, out, prm,
                       heads, GdnRowStrides{}, GdnRowsIO{});
}

void launch_gdn_decode_rows(const float* proj, float* conv_state, const float* conv_w, float* state, float* out,
                            const float* prm, int heads, int rows, const GdnRowStrides& rs, hipStream_t st,
                            const GdnRowsIO& io) {
    hipLaunchKernelGGL(k_gdn_decode, dim3(heads, rows), dim3(kGdnThreads), 0, st, proj, conv_state, conv_w, state, out,
                       prm, heads, rs, io);
}

void launch_delta_rule(const float* q, const float* k, const float* v, const float* beta, const float* g, float* state,
                       float* out, int batch, int heads, hipStream_t st) {
    hipLaunchKernelGGL(k_delta_rule, dim3(heads, batch), dim3(kGdnThreads), 0, st, q, k, v, beta, g, state, out, heads);
}

void launch_delta_rule_chunked(const float* q, const float* k, const float* v, const float* beta, const float* g,
                               float* state, float* out, int batch, int tokens, int heads, hipStream_t st) {
    const int waves = batch * heads * (kDV / 4);
    hipLaunchKernelGGL(k_delta_rule_cols, dim3((waves + 3) / 4), dim3(256), 0, st, q, k, v, beta, g, state, out, tokens,
                       heads, waves, 0);
}

}  // namespace qne
