// GQA attention decode over a paged f16 KV cache (head_dim 256, 16-token blocks).
//
// Reference: the decode kernel `attention` (kernels/src/shaders.rs:522-633), which runs one
// workgroup per query head over an f32 cache with all scores in LDS. Design for gfx950:
//  - the cache is paged: pools [block][kv_head][16][256] f16, a block table maps logical blocks;
//  - split-context ("flash decoding") partials: workgroup (split, kv_head, seq) streams a slice
//    of the context once for all query heads that share the kv head (GQA reuse);
//  - a wave takes 16-position blocks with all of a block's K and V rows in flight at once; scores
//    on the matrix cores (f16 MFMA, q as two f16 halves), values on the vector ALUs; softmax is
//    online (running max / sum) in base 2;
//  - a combine kernel merges the splits (and applies the sigmoid output gate of the model).
// The current token's k and v are appended (rounded to f16) before the partials run, so the
// current position is read back exactly as every later step will read it.
#include <mutex>
#include <string>

#include "../error.hpp"
#include "common.hpp"
#include "launch.hpp"
#include "operand.hpp"

namespace qne {

constexpr int kHD = 256, kBlock = 16, kAttnThreads = 256;

// The split partials of qne_paged_attn_decode_noalloc ((maximum, sum) pairs, then 256-float
// accumulators) live here instead of in memory the library allocates. Each GPU holds its own copy
// for the life of the process. In host code `scratch` names a host-side stand-in, never the
// device memory: host code uses the address noalloc_scratch() looked up.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

float* noalloc_scratch() {
    static std::mutex mu;
    static void* per_device[256] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) throw Error(QNE_EDEVICE, std::string("HIP error in hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= 256) throw Error(QNE_EDEVICE, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (!per_device[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw Error(QNE_EDEVICE, std::string("HIP error in hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        per_device[dev] = p;
    }
    return (float*)per_device[dev];
}

__device__ __forceinline__ size_t kv_index(const int32_t* bt, int pos, int nkv, int g) {
    const int blk = bt[pos / kBlock];
    return (((size_t)blk * nkv + g) * kBlock + (pos % kBlock)) * kHD;
}

// RMSNorm (weight w) and rotate-half RoPE on the first rope_dim dims of one 256-vector held one
// value per thread (shaders.rs:575-593). Returns the thread's output value.
__device__ __forceinline__ float norm_rope(float x, const float* __restrict__ w, const float* __restrict__ inv_freq,
                                           int rope_dim, uint32_t pos, float* sh, float* red) {
    const int t = threadIdx.x;
    const float ss = block_sum<kAttnThreads>(x * x, red);
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
    // The row's projection values: stored, or the in-projection's split partials (every load in
    // flight at once) summed in split order times the row's 1 / rms from the sums of x^2 of its
    // operand, as k_gemm_reduce computes them.
    const int k0 = 2 * a.nq * kHD, g = hb - a.nq;
    const int c0 = hb < a.nq ? hb * kHD + t : k0 + g * kHD + t;                      // q, or k
    const int c1 = hb < a.nq ? (a.nq + hb) * kHD + t : k0 + (a.nkv + g) * kHD + t;  // the gate, or v
    const int nchunks_in = a.k_in / kChunk;
    const float ss_in = a.part && t < nchunks_in ? ((const float*)(a.x_in + (size_t)t * kChunkBytes))[kSsOff / 4 + b] : 0.0f;
    const float* pbase = a.part ? a.part + (size_t)b * a.in_n : proj;
    const int nsp = a.part ? a.in_splits : 1;
    Split8 p0, p1;
    p0.load(pbase + c0, nsp, a.split_stride);
    if (a.part || hb >= a.nq) p1.load(pbase + c1, nsp, a.split_stride);
    float inv = 1.0f;
    if (a.part) {
        inv = 1.0f / sqrtf(block_sum<kAttnThreads>(ss_in, red) / (float)a.k_in + a.eps);  // row_inv_rms
        __syncthreads();  // red is reused below
    }
    const float x0 = p0.sum(pbase + c0, nsp, a.split_stride) * inv;
    if (hb < a.nq) {
        a.qbuf[((size_t)b * a.nq + hb) * kHD + t] = norm_rope(x0, a.norms, a.inv_freq, a.rope_dim, pos, sh, red);
        if (a.part) a.gate_dst[(size_t)b * a.proj_stride + c1] = p1.sum(pbase + c1, nsp, a.split_stride) * inv;
    } else {
        const float kr = norm_rope(x0, a.norms + kHD, a.inv_freq, a.rope_dim, pos, sh, red);
        const size_t at = kv_index(a.block_table + (size_t)b * a.bt_stride, (int)pos, a.nkv, g) + t;
        a.k_pool[at] = f2h(kr);
        a.v_pool[at] = f2h(p1.sum(pbase + c1, nsp, a.split_stride) * inv);
    }
}

// Raw form: append k_new / v_new of sequence blockIdx.y, kv head blockIdx.x at ctx[b].
__global__ __launch_bounds__(kAttnThreads) void k_kv_append(const float* __restrict__ k_new, const float* __restrict__ v_new,
                                                            uint16_t* __restrict__ k_pool, uint16_t* __restrict__ v_pool,
                                                            const int32_t* __restrict__ bt, int max_blocks,
                                                            const int32_t* __restrict__ ctx, int nkv, int32_t* __restrict__ order) {
    const int g = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    if (order && g == 0 && b == 0 && t < (int)gridDim.y) {
        // rank of sequence t by decreasing context, ties to the lower index
        const int m = gridDim.y, ct = ctx[t];
        int rank = 0;
        for (int u = 0; u < m; u++) {
            const int cu = ctx[u];
            rank += cu > ct || (cu == ct && u < t);
        }
        order[rank] = t;
    }
    if (ctx[b] < 0 || ctx[b] >= max_blocks * kBlock) return;  // beyond the table: nothing to write
    const size_t at = kv_index(bt + (size_t)b * max_blocks, ctx[b], nkv, g) + t;
    const size_t src = ((size_t)b * nkv + g) * kHD + t;
    k_pool[at] = f2h(k_new[src]);
    v_pool[at] = f2h(v_new[src]);
}

typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h4v as_h4(uint32_t a, uint32_t b) { return __builtin_bit_cast(h4v, u32x2{a, b}); }

// Split-context partials. Grid (splits, nkv, batch), 4 waves. Sequence b attends positions
// 0..len-1 with len = lens[b] + 1 (lens = tok + 1 for the model, ctx for the raw form). A wave takes
// blocks of 16 positions (the waves interleave blocks); per block:
//  - scores on the matrix cores: S[position][column] = K[16 x 256] . Qc[256 x 16] with
//    v_mfma_f32_16x16x16_f16, K as stored (f16) and the columns 2h, 2h + 1 holding query head h as
//    two f16 halves, hi = f16(x) and lo = f16((x - hi) * 2^11), so q keeps ~22 bits and the
//    products are exact in f32. Lane l loads 16 bytes of row l % 16 at byte 64 i + 16 (l / 16)
//    (i = 0..7): the 16 rows of a block are one contiguous 8 KB, each load instruction covers 16
//    whole 64-byte segments, and the k slots of the two MFMAs fed by one load are the dims it holds;
//  - the hi and lo columns are added across the lane pair, the block's per-head maximum and weight
//    sum are reduced over the 4 lane groups, and the weights go through LDS ([position][head]);
//  - values on the vector ALUs: lane l accumulates dims 4l..4l+3 of every head, reading one
//    512-byte row per position (all 16 rows are loaded with the K rows, before the scores).
// Rows past the sequence end in its last block are read (they lie in the block) but weigh 0 and
// their values are replaced by 0. The softmax runs in base 2: q is pre-scaled by
// log2(e) / sqrt(256), so each weight is one exp2 (the combine uses the same base).
template <int G>
__global__ __launch_bounds__(kAttnThreads) void k_attn_partial(const float* __restrict__ q, const uint16_t* __restrict__ k_pool,
                                                               const uint16_t* __restrict__ v_pool,
                                                               const int32_t* __restrict__ block_table, int max_blocks,
                                                               int bt_stride, const int32_t* __restrict__ lens, int nkv,
                                                               const int32_t* __restrict__ order,
                                                               float* __restrict__ part_ml, float* __restrict__ part_acc) {
    __shared__ __attribute__((aligned(16))) uint16_t s_q[G][2][kHD];  // per head: hi, lo halves as f16
    __shared__ __attribute__((aligned(16))) float s_p[4][16][4];      // per wave: weights [position][head]
    __shared__ float s_ml[4][G][2];
    __shared__ __attribute__((aligned(16))) float s_acc[4][G][kHD];
    const int split = blockIdx.x, g = blockIdx.y, b = order ? order[blockIdx.z] : (int)blockIdx.z, splits = gridDim.x;
    const int t = threadIdx.x, lane = t % kWave, w = t / kWave;
    const int len = max(1, min(lens[b] + 1, max_blocks * kBlock));  // never past the block table
    int per = (len + splits - 1) / splits;
    per = (per + kBlock - 1) / kBlock * kBlock;
    const int p0 = split * per, p1 = min(len, p0 + per);
    const int32_t* bt = block_table + (size_t)b * bt_stride;
    const int nq = nkv * G;
    constexpr float kScale = 1.4426950408889634f * 0.0625f;  // log2(e) / sqrt(256)

#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        const float x = q[((size_t)b * nq + g * G + gi) * kHD + t] * kScale;
        const _Float16 hi = (_Float16)x;
        s_q[gi][0][t] = __builtin_bit_cast(uint16_t, hi);
        s_q[gi][1][t] = __builtin_bit_cast(uint16_t, (_Float16)((x - (float)hi) * 2048.0f));
    }
    __syncthreads();

    const int c = lane & 15, kq = lane >> 4;  // row (position) / column of the MFMA tiles, k group
    // B operands, read from LDS per block: column c (zero past 2G), k slots = the dims lane loads
    const uint16_t* qcol = &s_q[(c >> 1) % G][c & 1][8 * kq];

    float m = -INFINITY, l = 0.0f;  // lanes c = 2h: head h's running maximum and weight sum
    float acc[G][4];
#pragma unroll
    for (int gi = 0; gi < G; gi++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[gi][e] = 0.0f;

    int bnext = p0 + 16 * w < p1 ? bt[(p0 + 16 * w) / kBlock] : 0;  // block table entries run one block ahead
    for (int pb = p0 + 16 * w; pb < p1; pb += 64) {                  // wave-uniform
        const int bcur = bnext;
        if (pb + 64 < p1) bnext = bt[(pb + 64) / kBlock];
        const size_t blk = ((size_t)bcur * nkv + g) * kBlock * kHD;  // the block's 16 rows, contiguous
        u32x4 kw[8];
#pragma unroll
        for (int i = 0; i < 8; i++) kw[i] = __builtin_nontemporal_load((const u32x4*)(k_pool + blk + c * kHD + 32 * i + 8 * kq));
        u32x2 vw[16];
#pragma unroll
        for (int j = 0; j < 16; j++) vw[j] = __builtin_nontemporal_load((const u32x2*)(v_pool + blk + j * kHD + 4 * lane));
        __builtin_amdgcn_sched_barrier(0);  // all 24 loads in flight before the first MFMA waits
        f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            u32x4 qw = *(const u32x4*)(qcol + 32 * i);
            if (c >= 2 * G) qw = u32x4{0u, 0u, 0u, 0u};
            sc = __builtin_amdgcn_mfma_f32_16x16x16f16(as_h4(kw[i].x, kw[i].y), as_h4(qw.x, qw.y), sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_16x16x16f16(as_h4(kw[i].z, kw[i].w), as_h4(qw.z, qw.w), sc, 0, 0, 0);
        }
        // lane (c, kq) reg r holds column c of position pb + 4 kq + r; even lanes take hi + lo
        float s[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float v = sc[r] + QNE_DPP(sc[r], kDppXor1) * (1.0f / 2048.0f);
            s[r] = pb + 4 * kq + r < p1 ? v : -INFINITY;
        }
        float bm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        bm = fmaxf(bm, lane_xor16(bm, lane));
        bm = fmaxf(bm, lane_xor32(bm, lane));
        const float mn = fmaxf(m, bm);                      // finite: position pb is in range
        const float corr = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first block
        float p[4], ps = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            p[r] = __builtin_amdgcn_exp2f(s[r] - mn);  // 0 past the range
            ps += p[r];
        }
        ps += lane_xor16(ps, lane);
        ps += lane_xor32(ps, lane);
        l = l * corr + ps;
        m = mn;
        if (c < 2 * G && (c & 1) == 0) {
#pragma unroll
            for (int r = 0; r < 4; r++) s_p[w][4 * kq + r][c >> 1] = p[r];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            const float cg = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), 2 * gi));
#pragma unroll
            for (int e = 0; e < 4; e++) acc[gi][e] *= cg;
        }
        const int nj = p1 - pb;  // rows at or past nj weigh 0; their values may be anything
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const uint32_t x0 = j < nj ? vw[j].x : 0u, x1 = j < nj ? vw[j].y : 0u;
            const float v0 = lo_h(x0), v1 = hi_h(x0), v2 = lo_h(x1), v3 = hi_h(x1);
            const float4 pw = *(const float4*)s_p[w][j];
            const float pj[4] = {pw.x, pw.y, pw.z, pw.w};
#pragma unroll
            for (int gi = 0; gi < G; gi++) {
                acc[gi][0] = fmaf(pj[gi], v0, acc[gi][0]);
                acc[gi][1] = fmaf(pj[gi], v1, acc[gi][1]);
                acc[gi][2] = fmaf(pj[gi], v2, acc[gi][2]);
                acc[gi][3] = fmaf(pj[gi], v3, acc[gi][3]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();  // s_p is rewritten by the next block
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // the wave's partial: (m, l) of head h from lane 2h, acc for dims 4 lane..4 lane + 3
    if (lane < 2 * G && (lane & 1) == 0) {
        s_ml[w][lane >> 1][0] = m;
        s_ml[w][lane >> 1][1] = l;
    }
#pragma unroll
    for (int gi = 0; gi < G; gi++) *(float4*)&s_acc[w][gi][4 * lane] = make_float4(acc[gi][0], acc[gi][1], acc[gi][2], acc[gi][3]);
    __syncthreads();
    // merge the 4 waves: thread t owns dim t for every head of the group
    const size_t pbase = (((size_t)b * nkv + g) * splits + split) * G;
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) mx = fmaxf(mx, s_ml[i][gi][0]);
        float lsum = 0.0f, a = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float cw = mx == -INFINITY ? 0.0f : exp2f(s_ml[i][gi][0] - mx);
            lsum += s_ml[i][gi][1] * cw;
            a += s_acc[i][gi][t] * cw;
        }
        part_acc[(pbase + gi) * kHD + t] = a;
        if (t == 0) { part_ml[(pbase + gi) * 2] = mx; part_ml[(pbase + gi) * 2 + 1] = lsum; }
    }
}

typedef _Float16 h8v __attribute__((ext_vector_type(8)));

constexpr int kPfUnit = 32;       // positions per step of the prefill kernel: two cache blocks
constexpr int kPfKStride = 528;   // bytes per K row in LDS: 512 + 16, so the 16 rows of a column read hit distinct banks
constexpr int kPfVStride = 80;    // bytes per dim of the transposed V in LDS: 32 positions (64 B) + 16

__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) { return (a & 0xFFFFu) | (b << 16); }
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xFFFF0000u); }

// Causal attention of the rows of a prompt chunk (consecutive tokens of one sequence, row b at
// position pos[b], cache rows already appended): the same partials as k_attn_partial, computed for
// a tile of query rows at a time so that every K/V row is read once per tile instead of once per
// row. Grid (tiles, nkv, splits), 4 waves; a tile is 16 * (4 / G) rows and wave w takes query head
// g * G + w % G of the 16 rows 16 * (w / G)...; split s covers positions [s * split_len,
// (s + 1) * split_len), cut at the tile's last position.
// Per step of 32 positions (two 16-position blocks) the workgroup stages the K rows (as stored,
// rows padded to 528 B) and V transposed (dim-major: for every dim the 8 positions k-slot group kq
// of the MFMA takes, {4 kq..4 kq + 3, 16 + 4 kq..16 + 4 kq + 3}) in LDS, double-buffered, with the
// next step's global loads in flight during this step's math:
//  - scores S[position][row] = K . Q^T on v_mfma_f32_16x16x32_f16, q as two f16 terms in registers,
//    hi = f16(x) and lo = f16(x - hi) (often subnormal: the matrix cores take f16 subnormals
//    exactly), so q keeps ~22 bits; both terms accumulate into the same scores;
//  - the score tile's layout (lane: row lane % 16, positions 4 (lane / 16) + r) is the B operand of
//    O^T[dim][row] += V^T . P^T, so the weights go to the matrix cores without a shuffle, again as
//    hi and lo f16 terms into one accumulator; the running maximum / sum and the rescale are per
//    lane (= per row). 64 accumulator registers per lane leave room for two waves per SIMD.
// Masked entries (past the row's position or the split) weigh exactly 0 and leave the row's
// maximum alone, so a row's partial does not depend on the other rows of its tile: a token's
// result does not depend on how the prompt was cut into calls. V rows past the split end are
// zeroed in LDS (a block may hold rows never written).
template <int G>
__global__ __launch_bounds__(kAttnThreads, 2) void k_attn_prefill(const float* __restrict__ q, const uint16_t* __restrict__ k_pool,
                                                               const uint16_t* __restrict__ v_pool,
                                                               const int32_t* __restrict__ bt, int max_blocks,
                                                               const int32_t* __restrict__ pos, int rows, int nkv, int split_len,
                                                               float* __restrict__ part_ml, float* __restrict__ part_acc) {
    constexpr int RT = 4 / G;  // 16-row subtiles per tile
    __shared__ __attribute__((aligned(16))) uint8_t s_k[2][kPfUnit * kPfKStride];
    __shared__ __attribute__((aligned(16))) uint8_t s_v[2][kHD * kPfVStride];
    const int split = blockIdx.z, g = blockIdx.y, splits = gridDim.z;
    const int t = threadIdx.x, lane = t % kWave, w = t / kWave;
    const int gi = w % G, n = lane & 15, kq = lane >> 4;
    const int row0 = blockIdx.x * 16 * RT;
    const int b = row0 + 16 * (w / G) + n;  // this lane's row (column of the score tile)
    const int rpos = b < rows ? pos[b] : -1;
    const int tpos = lane < 16 * RT && row0 + lane < rows ? pos[row0 + lane] : -1;
    const int tile_len = min((int)wave_max((float)tpos) + 1, max_blocks * kBlock);
    const int p0 = split * split_len;
    if (p0 >= tile_len) return;  // the whole workgroup: nothing of this split is attended
    const int p1 = min(tile_len, p0 + split_len);
    const int steps = (p1 - p0 + kPfUnit - 1) / kPfUnit;
    const int nq = nkv * G, h = g * G + gi;
    constexpr float kScale = 1.4426950408889634f * 0.0625f;  // log2(e) / sqrt(256)

    // q as the B operand: lane (n, kq) holds dims 32 i + 8 kq .. + 7 of row b, hi and lo terms
    h8v qh[8], ql[8];
    {
        const float* qr = q + ((size_t)b * nq + h) * kHD + 8 * kq;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
            if (b < rows) {
                x0 = *(const float4*)(qr + 32 * i);
                x1 = *(const float4*)(qr + 32 * i + 4);
            }
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float x = xs[e] * kScale;
                const _Float16 hi = (_Float16)x;
                qh[i][e] = hi;
                ql[i][e] = (_Float16)(x - (float)hi);
            }
        }
    }

    // The split's block table entries, lane i holding entry p0 / 16 + i (a split spans at most 64
    // blocks): every step picks its two with readlane, so no load waits on a table entry. A block
    // past the split end (the second of a last step) reads the first block instead; those rows
    // weigh 0 and their values are zeroed below.
    const int nblk = (p1 - p0 + kBlock - 1) / kBlock;
    const int btv = lane < nblk ? bt[p0 / kBlock + lane] : 0;
    // staging assignment: K row kr (of the step's 32), bytes 64 kp..64 kp + 63; V positions
    // {4 w + j, 16 + 4 w + j} (j = 0..3) of dims 4 lane..4 lane + 3
    const int kr = t >> 3, kp = t & 7;
    u32x4 kw[4];
    u32x2 vr[8];
    auto load = [&](int base) {
        const int j0 = (base - p0) / kBlock;
        const int blk0 = __builtin_amdgcn_readlane(btv, j0);
        const int blk1 = j0 + 1 < nblk ? __builtin_amdgcn_readlane(btv, j0 + 1) : blk0;
        const uint16_t* src = k_pool + (((size_t)(kr < kBlock ? blk0 : blk1) * nkv + g) * kBlock + kr % kBlock) * kHD + 32 * kp;
#pragma unroll
        for (int j = 0; j < 4; j++) kw[j] = __builtin_nontemporal_load((const u32x4*)(src + 8 * j));
        const uint16_t* v0 = v_pool + (((size_t)blk0 * nkv + g) * kBlock + 4 * w) * kHD + 4 * lane;
        const uint16_t* v1 = v_pool + (((size_t)blk1 * nkv + g) * kBlock + 4 * w) * kHD + 4 * lane;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            vr[j] = __builtin_nontemporal_load((const u32x2*)(v0 + j * kHD));
            vr[4 + j] = __builtin_nontemporal_load((const u32x2*)(v1 + j * kHD));
        }
    };
    auto stage = [&](int buf, int base) {
#pragma unroll
        for (int j = 0; j < 8; j++) {  // rows past the split end weigh 0: zero their values
            const int pv = base + (j < 4 ? 4 * w + j : 16 + 4 * w + j - 4);
            if (pv >= p1) vr[j] = u32x2{0u, 0u};
        }
        uint8_t* kd = s_k[buf] + kr * kPfKStride + 64 * kp;
#pragma unroll
        for (int j = 0; j < 4; j++) *(u32x4*)(kd + 16 * j) = kw[j];
        uint8_t* vd = s_v[buf] + (4 * lane) * kPfVStride + 16 * w;
        *(u32x4*)(vd) = u32x4{pack_lo16(vr[0].x, vr[1].x), pack_lo16(vr[2].x, vr[3].x), pack_lo16(vr[4].x, vr[5].x),
                              pack_lo16(vr[6].x, vr[7].x)};
        *(u32x4*)(vd + kPfVStride) = u32x4{pack_hi16(vr[0].x, vr[1].x), pack_hi16(vr[2].x, vr[3].x),
                                           pack_hi16(vr[4].x, vr[5].x), pack_hi16(vr[6].x, vr[7].x)};
        *(u32x4*)(vd + 2 * kPfVStride) = u32x4{pack_lo16(vr[0].y, vr[1].y), pack_lo16(vr[2].y, vr[3].y),
                                               pack_lo16(vr[4].y, vr[5].y), pack_lo16(vr[6].y, vr[7].y)};
        *(u32x4*)(vd + 3 * kPfVStride) = u32x4{pack_hi16(vr[0].y, vr[1].y), pack_hi16(vr[2].y, vr[3].y),
                                               pack_hi16(vr[4].y, vr[5].y), pack_hi16(vr[6].y, vr[7].y)};
    };

    float m = -INFINITY, l = 0.0f;  // this lane's row: running maximum (base 2) and weight sum
    f32x4 o[16];                    // O^T: dims 16 d + 4 kq + r of row b
#pragma unroll
    for (int d = 0; d < 16; d++) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};

    load(p0);
    for (int it = 0; it < steps; it++) {
        const int buf = it & 1, base = p0 + kPfUnit * it;
        stage(buf, base);
        __syncthreads();  // also: every wave is done with the step that last read this buffer
        if (it + 1 < steps) load(base + kPfUnit);
        float s[8];
#pragma unroll
        for (int hb = 0; hb < 2; hb++) {
            f32x4 sh = {0.f, 0.f, 0.f, 0.f}, sl = sh;
            const uint8_t* kb = s_k[buf] + (16 * hb + n) * kPfKStride + 16 * kq;
            h8v a[8];  // all eight K fragments in flight before the first MFMA needs one
#pragma unroll
            for (int i = 0; i < 8; i++) a[i] = *(const h8v*)(kb + 64 * i);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                sh = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], qh[i], sh, 0, 0, 0);
                sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], ql[i], sl, 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // the 8 LDS reads first,
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);  // then the 16 MFMAs
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int pp = base + 16 * hb + 4 * kq + r;
                s[4 * hb + r] = pp < p1 && pp <= rpos ? sh[r] + sl[r] : -INFINITY;
            }
        }
        float bm = s[0];
#pragma unroll
        for (int e = 1; e < 8; e++) bm = fmaxf(bm, s[e]);
        bm = fmaxf(bm, lane_xor16(bm, lane));
        bm = fmaxf(bm, lane_xor32(bm, lane));
        const float mn = fmaxf(m, bm);
        const float ms = mn == -INFINITY ? 0.0f : mn;  // a row with nothing attended yet stays (-inf, 0)
        const float corr = __builtin_amdgcn_exp2f(m - ms);
        float ps = 0.0f;
        h8v ph, pl;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float p = __builtin_amdgcn_exp2f(s[e] - ms);  // 0 where masked
            ps += p;
            const _Float16 hi = (_Float16)p;
            ph[e] = hi;
            pl[e] = (_Float16)(p - (float)hi);
        }
        ps += lane_xor16(ps, lane);
        ps += lane_xor32(ps, lane);
        l = l * corr + ps;
        m = mn;
        if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {  // multiplying by exactly 1 changes nothing
#pragma unroll
            for (int d = 0; d < 16; d++) o[d] *= corr;
        }
        const uint8_t* vb = s_v[buf] + n * kPfVStride + 16 * kq;
#pragma unroll
        for (int d0 = 0; d0 < 16; d0 += 8) {
            h8v a[8];  // eight V fragments in flight at a time
#pragma unroll
            for (int d = 0; d < 8; d++) a[d] = *(const h8v*)(vb + 16 * (d0 + d) * kPfVStride);
#pragma unroll
            for (int d = 0; d < 8; d++) {
                o[d0 + d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[d], ph, o[d0 + d], 0, 0, 0);
                o[d0 + d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[d], pl, o[d0 + d], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 1);
        }
    }
    if (b >= rows || rpos < p0) return;  // no partial for a row that attends nothing here
    const size_t pi = (((size_t)b * nkv + g) * splits + split) * G + gi;
    float* dst = part_acc + pi * kHD + 4 * kq;
#pragma unroll
    for (int d = 0; d < 16; d++) *(f32x4*)(dst + 16 * d) = o[d];
    if (kq == 0) {
        part_ml[pi * 2] = m;
        part_ml[pi * 2 + 1] = l;
    }
}

// Merge the splits of query head blockIdx.x of sequence blockIdx.y; with `gate`, multiply by
// sigmoid(gate) (shaders.rs:626-629). With split_len, row b merges only the splits that hold its
// positions 0..pos[b] (the prefill kernel writes no others).
__global__ __launch_bounds__(kAttnThreads) void k_attn_combine(const float* __restrict__ part_ml, const float* __restrict__ part_acc,
                                                               int nkv, int G, int splits, const float* __restrict__ gate,
                                                               int gate_stride, float* __restrict__ out, uint8_t* __restrict__ frag_out,
                                                               int order_out, const int32_t* __restrict__ pos = nullptr,
                                                               int split_len = 0) {
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x, g = h / G, gi = h % G, nq = nkv * G;
    const int used = split_len ? min(splits, pos[b] / split_len + 1) : splits;  // splits holding row b's positions
    float mn = -INFINITY;
    for (int s = 0; s < used; s++) mn = fmaxf(mn, part_ml[((((size_t)b * nkv + g) * splits + s) * G + gi) * 2]);
    // every merged split wrote its partial (an empty one: maximum -inf, sum 0, acc 0), and split 0
    // holds position 0, so mn is finite and an empty split weighs exp2(-inf) = 0
    float lsum = 0.0f, a = 0.0f;
#pragma unroll 8
    for (int s = 0; s < used; s++) {
        const size_t i = (((size_t)b * nkv + g) * splits + s) * G + gi;
        const float c = exp2f(part_ml[i * 2] - mn);  // the partials' maxima are in base 2
        lsum += part_ml[i * 2 + 1] * c;
        a += part_acc[i * kHD + t] * c;
    }
    float o = a / lsum;
    if (gate) o = o / (1.0f + expf(-gate[(size_t)b * gate_stride + h * kHD + t]));
    if (out) out[((size_t)b * nq + h) * kHD + t] = o;
    if (frag_out)  // each wave: 64 columns of row b
        emit_x(frag_out, (size_t)(nq * kHD / kChunk) * kChunkBytes, b, h * kHD + t, o, 1.0f, order_out, t & (kWave - 1));
}

template <int G>
static void launch_partial(const float* q, const uint16_t* kp, const uint16_t* vp, const int32_t* bt, int max_blocks,
                           int bt_stride, const int32_t* lens, int nkv, float* ml, float* acc, int splits, int batch,
                           hipStream_t st, const int32_t* order = nullptr) {
    hipLaunchKernelGGL((k_attn_partial<G>), dim3(splits, nkv, batch), dim3(kAttnThreads), 0, st, q, kp, vp, bt,
                       max_blocks, bt_stride, lens, nkv, order, ml, acc);
}

static void partial_by_g(int G, const float* q, const uint16_t* kp, const uint16_t* vp, const int32_t* bt, int max_blocks,
                         int bt_stride, const int32_t* lens, int nkv, float* ml, float* acc, int splits, int batch,
                         hipStream_t st, const int32_t* order = nullptr) {
    switch (G) {
        case 1: launch_partial<1>(q, kp, vp, bt, max_blocks, bt_stride, lens, nkv, ml, acc, splits, batch, st, order); break;
        case 2: launch_partial<2>(q, kp, vp, bt, max_blocks, bt_stride, lens, nkv, ml, acc, splits, batch, st, order); break;
        default: launch_partial<4>(q, kp, vp, bt, max_blocks, bt_stride, lens, nkv, ml, acc, splits, batch, st, order); break;
    }
}

void launch_attention_model(const AttnModelArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(k_attn_prep, dim3(a.nq + a.nkv), dim3(kAttnThreads), 0, st, a);
    const int G = a.nq / a.nkv;
    // tok[1] is the position; the partial kernel attends lens[0] + 1 = pos + 1 positions.
    partial_by_g(G, a.qbuf, a.k_pool, a.v_pool, a.block_table, a.max_blocks, a.max_blocks, (const int32_t*)(a.tok + 1),
                 a.nkv, a.part_ml, a.part_acc, a.splits, 1, st);
    hipLaunchKernelGGL(k_attn_combine, dim3(a.nq, 1), dim3(kAttnThreads), 0, st, a.part_ml, a.part_acc, a.nkv, G,
                       a.splits, a.proj + a.nq * kHD, 0, a.out, (uint8_t*)nullptr, 0);
}

template <int G>
static void launch_prefill(const AttnRowsArgs& a, hipStream_t st) {
    const int tile = 16 * (4 / G);
    // Tiles in x: consecutive workgroups go to different XCDs, so each XCD gets every 8th tile and
    // an even share of the work. (With splits in x each XCD would hold one split, and the early
    // splits, which every tile needs, would all land on the same few XCDs.)
    hipLaunchKernelGGL((k_attn_prefill<G>), dim3((a.rows + tile - 1) / tile, a.nkv, a.splits), dim3(kAttnThreads), 0, st,
                       a.qbuf, a.k_pool, a.v_pool, a.block_table, a.max_blocks, a.pos, a.rows, a.nkv, a.split_len,
                       a.part_ml, a.part_acc);
}

bool prefill_attention_supported(int nq, int nkv) {
    // the groupings the model configurations have (and the tests run); others take the per-row
    // partials
    const int G = nkv > 0 && nq % nkv == 0 ? nq / nkv : 0;
    return G == 2 || G == 4;
}

void launch_attention_rows(const AttnRowsArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(k_attn_prep_rows, dim3(a.nq + a.nkv, a.rows), dim3(kAttnThreads), 0, st, a);
    const int G = a.nq / a.nkv;
    if (a.split_len) {
        // rows of one sequence (a prompt chunk): query tiles; the host checked the shape
        if (a.bt_stride != 0 || a.split_len % kPfUnit != 0 || a.split_len > kWave * kBlock ||
            !prefill_attention_supported(a.nq, a.nkv) ||
            (long)a.splits * a.split_len < (long)a.max_blocks * kBlock)
            throw Error(QNE_EINVAL, "prefill attention: rows must share one block table, split_len must be a multiple "
                                    "of 32 up to 1024 covering the context, and 2 or 4 query heads per kv head");
        if (G == 2) launch_prefill<2>(a, st);
        else launch_prefill<4>(a, st);
    } else {
        partial_by_g(G, a.qbuf, a.k_pool, a.v_pool, a.block_table, a.max_blocks, a.bt_stride, a.pos, a.nkv, a.part_ml,
                     a.part_acc, a.splits, a.rows, st, a.order);
    }
    const float* gate = a.part ? a.gate_dst + a.nq * kHD : a.proj + a.nq * kHD;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.nq, a.rows), dim3(kAttnThreads), 0, st, a.part_ml, a.part_acc, a.nkv, G,
                       a.splits, gate, (int)a.proj_stride, a.out, a.frag_out, a.order_out,
                       a.split_len ? a.pos : (const int32_t*)nullptr, a.split_len);
}

void launch_paged_attn(const float* q, const float* k_new, const float* v_new, uint16_t* k_pool, uint16_t* v_pool,
                       const int32_t* block_table, int max_blocks, const int32_t* ctx, float* out, int batch, int nq,
                       int nkv, float* part_ml, float* part_acc, int splits, hipStream_t st, int32_t* order) {
    if (batch > kAttnThreads) order = nullptr;  // one thread per sequence ranks them
    hipLaunchKernelGGL(k_kv_append, dim3(nkv, batch), dim3(kAttnThreads), 0, st, k_new, v_new, k_pool, v_pool,
                       block_table, max_blocks, ctx, nkv, order);
    const int G = nq / nkv;
    partial_by_g(G, q, k_pool, v_pool, block_table, max_blocks, max_blocks, ctx, nkv, part_ml, part_acc, splits, batch, st,
                 order);
    hipLaunchKernelGGL(k_attn_combine, dim3(nq, batch), dim3(kAttnThreads), 0, st, part_ml, part_acc, nkv, G, splits,
                       (const float*)nullptr, 0, out, (uint8_t*)nullptr, 0);
}

}  // namespace qne
