// Persistent decode engine: every decode step of the hybrid decoder in ONE cooperative launch.
//
// Reference: the per-token dispatch list of Model::load (kernels/src/model.rs:220-269) and its
// kernels (kernels/src/shaders.rs): embed, 24-28 x [rmsnorm, mixer_in GEMV, gdn | attention,
// mixer_out GEMV (+=), rmsnorm, gate_up GEMV (SwiGLU), down GEMV (+=)], rmsnorm, lm_head GEMV,
// argmax. A batch-1 decode step moves ~1.7 GB in ~150 dependent pieces of ~10 MB; as separate
// launches each piece is bound by launch and memory latency, not bandwidth. Design for MI355X:
//  - one workgroup of 512 threads per CU, all co-resident (cooperative launch); phases are
//    separated by a grid barrier (one agent-scope counter, bounded spin);
//  - every weight matrix is split by rows across workgroups; a workgroup streams its rows in
//    chunks of up to 60 KiB into a 2-slot LDS ring with global_load_lds_dwordx4 (DMA into LDS,
//    no VGPRs). Wave 7 is the copy wave: it issues the next chunk (possibly of the next phase,
//    across the grid barrier and the attention / GDN phase) while waves 0-6 compute the current
//    one, so HBM keeps streaming while the grid synchronises;
//  - compute waves keep their slice of the input vector in VGPRs (K/64 values per lane), read
//    weights from LDS with 16-byte reads (conflict-free), dequantise int4 with v_cvt_f32_ubyte and
//    accumulate in f32; RMSNorm is fused into the x load (its 1/rms is applied to the row sums);
//  - the GDN causal conv + SiLU runs in the epilogue of the in-projection rows that produce it;
//    the GDN step runs one wave per value column (state kept value-major, 512 B per column); its
//    output RMSNorm is completed by the next phase from per-block sums of squares;
//  - attention: split-context partials per (kv head, split) with GQA reuse, merged by the last
//    workgroup to finish its kv head (arrival counter), then the sigmoid gate;
//  - the LM head tracks a per-workgroup argmax; after its barrier every workgroup reduces the
//    partials itself, so the next step starts without another barrier.
#include "common.hpp"
#include "engine.hpp"

namespace qne {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kEW = kEngineThreads / kWave;  // 8 waves
constexpr int kCW = 7;                      // compute waves
constexpr int kDmaWave = 7;
constexpr int kBuf = 60 * 1024;             // bytes per LDS chunk slot
constexpr int kMaxR = 8;                    // output rows per compute wave per chunk
constexpr int kMiscFloats = 4096;  // also holds the embedding row of the step (hidden <= 3968)
constexpr int kHD = 256, kBlk = 16;
constexpr int kDK = 128;

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] at 3:0 and [5:4] at 15:14, expcnt 6:4,
// lgkmcnt 11:8).
constexpr int kWaitVm0 = 0x0F70;
constexpr int kWaitLgkm0 = 0xC07F;
constexpr int kWaitAll = 0x0000;

enum { E_STORE = 0, E_ACC = 1, E_SWIGLU = 2, E_CONV = 3, E_ARGMAX = 4 };
enum { X_PLAIN = 0, X_NORM = 1, X_EMBED = 2, X_GDN = 3 };

struct Job {
    EMat m;
    const float* x;
    const float* gain;
    float* y;
    const float* conv_w;
    float* conv;
    int epi, xmode, rows_out, conv_ch;
    int r0, r1, cap, nchunks;
    int rb, szb;
};

__device__ __forceinline__ void cbar() { asm volatile("" ::: "memory"); }
__device__ __forceinline__ void sbarrier() {
    cbar();
    __builtin_amdgcn_s_barrier();
    cbar();
}

__device__ __forceinline__ int njobs(const EngineArgs& a, int step) {
    const bool head = a.head == 1 || (a.head == 2 && step == a.n_steps - 1);
    return 4 * a.n_layers + (head ? 1 : 0);
}

__device__ __forceinline__ Job make_job(const EngineArgs& a, int j, int wg, int nwg) {
    Job J;
    J.gain = nullptr;
    J.conv_w = nullptr;
    J.conv = nullptr;
    J.conv_ch = 0;
    if (j < 4 * a.n_layers) {
        const ELayer& L = a.layers[j >> 2];
        switch (j & 3) {
            case 0:
                J.m = L.in;
                J.epi = L.attn ? E_STORE : E_CONV;
                J.xmode = (j >> 2) == 0 ? X_EMBED : X_NORM;
                J.x = a.h;
                J.gain = L.in_norm;
                J.y = a.proj;
                J.rows_out = L.in.rows;
                J.conv_w = L.conv_w;
                J.conv = L.conv;
                J.conv_ch = L.attn ? 0 : 3 * a.gdn_heads * kDK;
                break;
            case 1:
                J.m = L.out;
                J.epi = E_ACC;
                J.xmode = L.attn ? X_PLAIN : X_GDN;
                J.x = a.mixed;
                J.y = a.h;
                J.rows_out = L.out.rows;
                break;
            case 2:
                J.m = L.gu;
                J.epi = E_SWIGLU;
                J.xmode = X_NORM;
                J.x = a.h;
                J.gain = L.post_norm;
                J.y = a.act;
                J.rows_out = L.gu.rows / 2;
                break;
            default:
                J.m = L.down;
                J.epi = E_ACC;
                J.xmode = X_PLAIN;
                J.x = a.act;
                J.y = a.h;
                J.rows_out = L.down.rows;
                break;
        }
    } else {
        J.m = a.lm;
        J.epi = a.argmax ? E_ARGMAX : E_STORE;
        J.xmode = X_NORM;
        J.x = a.h;
        J.gain = a.final_norm;
        J.y = a.logits;
        J.rows_out = a.lm.rows;
    }
    J.rb = J.m.kind ? J.m.k / 2 : J.m.k * 2;
    J.szb = J.m.kind ? (J.m.k / J.m.group) * 4 : 0;
    const int per = (J.rows_out + nwg - 1) / nwg;
    J.r0 = min(wg * per, J.rows_out);
    J.r1 = min(J.r0 + per, J.rows_out);
    const int unit = (J.rb + J.szb) * (J.epi == E_SWIGLU ? 2 : 1);
    J.cap = min(kCW * kMaxR, kBuf / unit);
    J.nchunks = J.r1 > J.r0 ? (J.r1 - J.r0 + J.cap - 1) / J.cap : 0;
    return J;
}

// ---- weight streaming (copy wave only) ----

__device__ __forceinline__ void dma_range(const uint8_t* src, int bytes, uint8_t* dst, int lane) {
    for (int u = 0; u * 1024 < bytes; u++) {
        const int off = u * 1024 + lane * 16;
        if (off < bytes)
            __builtin_amdgcn_global_load_lds((const void*)(src + off), (lds_ptr_t)(dst + u * 1024), 16, 0, 0);
    }
}

__device__ __forceinline__ void dma_chunk(const Job& J, int c, uint8_t* buf, int lane) {
    const int a0 = J.r0 + c * J.cap, n = min(J.cap, J.r1 - a0);
    const int nm = J.epi == E_SWIGLU ? 2 : 1;
    const uint8_t* w = (const uint8_t*)J.m.w;
    dma_range(w + (size_t)a0 * J.rb, n * J.rb, buf, lane);
    if (nm == 2) dma_range(w + (size_t)(a0 + J.rows_out) * J.rb, n * J.rb, buf + n * J.rb, lane);
    if (J.szb) {
        const uint8_t* sz = (const uint8_t*)J.m.sz;
        dma_range(sz + (size_t)a0 * J.szb, n * J.szb, buf + nm * n * J.rb, lane);
        if (nm == 2) dma_range(sz + (size_t)(a0 + J.rows_out) * J.szb, n * J.szb, buf + nm * n * J.rb + n * J.szb, lane);
    }
}

// Cursor over every chunk this workgroup will compute, in order: steps, jobs, chunks.
struct Cursor {
    int step, job, chunk;
    bool done;
};

__device__ __forceinline__ void cursor_settle(const EngineArgs& a, Cursor& k, int wg, int nwg) {
    while (!k.done) {
        if (k.job >= njobs(a, k.step)) {
            k.job = 0;
            k.chunk = 0;
            if (++k.step >= a.n_steps) k.done = true;
            continue;
        }
        const Job J = make_job(a, k.job, wg, nwg);
        if (k.chunk < J.nchunks) return;
        k.chunk = 0;
        k.job++;
    }
}

__device__ __forceinline__ void dma_next(const EngineArgs& a, Cursor& k, int seq, uint8_t* smem, int wg, int nwg, int lane) {
    cursor_settle(a, k, wg, nwg);
    if (k.done) return;
    const Job J = make_job(a, k.job, wg, nwg);
    dma_chunk(J, k.chunk, smem + (seq & 1) * kBuf, lane);
    k.chunk++;
}

// ---- grid barrier ----

__device__ __forceinline__ bool grid_sync(const EngineArgs& a, unsigned& epoch, int nwg, int wave, bool drain_copy_wave, int* flag) {
    if (wave != kDmaWave || drain_copy_wave) __builtin_amdgcn_s_waitcnt(kWaitAll);
    else __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    sbarrier();
    epoch++;
    if (threadIdx.x == 0) {
        __atomic_thread_fence(__ATOMIC_RELEASE);  // make this workgroup's stores visible device-wide
        __hip_atomic_fetch_add(a.bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned target = epoch * (unsigned)nwg;
        unsigned spins = 0;
        int ok = 1;
        while (__hip_atomic_load(a.bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > a.spin_limit || __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
        }
        __atomic_thread_fence(__ATOMIC_ACQUIRE);
        *flag = ok;
    }
    sbarrier();
    return *(volatile int*)flag != 0;
}

// ---- input vector in registers ----

struct XRegs {
    float x4[3][32];
    float x2[16];
    float x1[8];
    float s4[3], s2, s1;  // per-slab sums (q4 zero-point term)
    float inv;            // 1/rms for normalised inputs, else 1
};

__device__ __forceinline__ float embed_val(const EMat& e, uint32_t tok, int c) {
    if (e.kind == 0) return h2f(((const uint16_t*)e.w)[(size_t)tok * e.k + c]);
    const uint32_t word = ((const uint32_t*)e.w)[(size_t)tok * (e.k / 8) + c / 8];
    const uint32_t sz = e.sz[(size_t)tok * (e.k / e.group) + c / e.group];
    return ((float)((word >> (4 * (c % 8))) & 15u) - hi_h(sz)) * lo_h(sz);
}

// Loads x (and gain) for columns [c0, c0 + N) with N a multiple of 4; returns sum of raw^2.
template <int N>
__device__ __forceinline__ float x_span(const EngineArgs& a, const Job& J, uint32_t tok, int c0, float* out,
                                        const float* gdn_r) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        float v[4];
        const float4 f = *(const float4*)(J.x + c0 + i);  // global, or the LDS copy of the embedding row
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        if (J.xmode == X_NORM || J.xmode == X_EMBED) {
            const float4 g = *(const float4*)(J.gain + c0 + i);
            ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
            v[0] *= g.x; v[1] *= g.y; v[2] *= g.z; v[3] *= g.w;
        } else if (J.xmode == X_GDN) {
            const float r = *gdn_r;
            v[0] *= r; v[1] *= r; v[2] *= r; v[3] *= r;
        }
        out[i] = v[0]; out[i + 1] = v[1]; out[i + 2] = v[2]; out[i + 3] = v[3];
    }
    return ss;
}

// misc[kRnorm + h]: 1/rms of GDN head h's outputs, staged by run_job before an X_GDN load.
constexpr int kRnorm = 3968;

__device__ __forceinline__ void load_x(const EngineArgs& a, const Job& J, uint32_t tok, XRegs& X, int lane,
                                       const float* rn) {
    const int K = J.m.k;
    float ss = 0.0f;
    if (J.m.kind == 1) {
        const int n4 = K / 2048, n2 = (K % 2048) / 1024, n1 = (K % 1024) / 512;
#pragma unroll
        for (int s = 0; s < 3; s++) {
            if (s < n4) {
                const int c0 = 2048 * s + 32 * lane;
                float r = 1.0f;
                if (J.xmode == X_GDN) r = rn[c0 / kDK];
                ss += x_span<32>(a, J, tok, c0, X.x4[s], &r);
            }
        }
        if (n2) {
            const int c0 = 2048 * n4 + 16 * lane;
            float r = 1.0f;
            if (J.xmode == X_GDN) r = rn[c0 / kDK];
            ss += x_span<16>(a, J, tok, c0, X.x2, &r);
        }
        if (n1) {
            const int c0 = 2048 * n4 + 1024 * n2 + 8 * lane;
            float r = 1.0f;
            if (J.xmode == X_GDN) r = rn[c0 / kDK];
            ss += x_span<8>(a, J, tok, c0, X.x1, &r);
        }
#pragma unroll
        for (int s = 0; s < 3; s++) {
            float t = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) t += X.x4[s][i];
            X.s4[s] = t;
        }
        float t2 = 0.0f, t1 = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) t2 += X.x2[i];
#pragma unroll
        for (int i = 0; i < 8; i++) t1 += X.x1[i];
        X.s2 = t2;
        X.s1 = t1;
    } else {
        const int ns = K / 512;
#pragma unroll
        for (int s = 0; s < 12; s++) {
            if (s < ns) {
                const int c0 = 512 * s + 8 * lane;
                float r = 1.0f;
                if (J.xmode == X_GDN) r = rn[c0 / kDK];
                ss += x_span<8>(a, J, tok, c0, &X.x4[s / 4][8 * (s % 4)], &r);
            }
        }
    }
    X.inv = 1.0f;
    if (J.xmode == X_NORM || J.xmode == X_EMBED) {
        ss = wave_sum(ss);
        X.inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    }
}

__device__ __forceinline__ float dot8(uint32_t w, const float* x) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    float p = (float)(lo & 0xFFu) * x[0];
    float q = (float)(hi & 0xFFu) * x[1];
    p = fmaf((float)((lo >> 8) & 0xFFu), x[2], p);
    q = fmaf((float)((hi >> 8) & 0xFFu), x[3], q);
    p = fmaf((float)((lo >> 16) & 0xFFu), x[4], p);
    q = fmaf((float)((hi >> 16) & 0xFFu), x[5], q);
    p = fmaf((float)(lo >> 24), x[6], p);
    q = fmaf((float)(hi >> 24), x[7], q);
    return p + q;
}

// Lane's partial dot product of one row held in LDS at `row` (weights) / `szr` (scale, zero).
__device__ __forceinline__ float row_dot(const Job& J, const uint8_t* row, const uint8_t* szr, const XRegs& X,
                                         int lane) {
    const int K = J.m.k;
    float acc = 0.0f;
    if (J.m.kind == 1) {
        const int G = J.m.group, n4 = K / 2048, n2 = (K % 2048) / 1024, n1 = (K % 1024) / 512;
#pragma unroll
        for (int s = 0; s < 3; s++) {
            if (s < n4) {
                const u32x4 w = *(const u32x4*)(row + 1024 * s + 16 * lane);
                const uint32_t sz = *(const uint32_t*)(szr + 4 * ((2048 * s + 32 * lane) / G));
                const float dq = dot8(w.x, &X.x4[s][0]) + dot8(w.y, &X.x4[s][8]) + dot8(w.z, &X.x4[s][16]) +
                                 dot8(w.w, &X.x4[s][24]);
                acc = fmaf(lo_h(sz), dq - hi_h(sz) * X.s4[s], acc);
            }
        }
        if (n2) {
            const u32x2 w = *(const u32x2*)(row + 1024 * n4 + 8 * lane);
            const uint32_t sz = *(const uint32_t*)(szr + 4 * ((2048 * n4 + 16 * lane) / G));
            const float dq = dot8(w.x, &X.x2[0]) + dot8(w.y, &X.x2[8]);
            acc = fmaf(lo_h(sz), dq - hi_h(sz) * X.s2, acc);
        }
        if (n1) {
            const uint32_t w = *(const uint32_t*)(row + 1024 * n4 + 512 * n2 + 4 * lane);
            const uint32_t sz = *(const uint32_t*)(szr + 4 * ((2048 * n4 + 1024 * n2 + 8 * lane) / G));
            acc = fmaf(lo_h(sz), dot8(w, X.x1) - hi_h(sz) * X.s1, acc);
        }
    } else {
        const int ns = K / 512;
        float b = 0.0f;
#pragma unroll
        for (int s = 0; s < 12; s++) {
            if (s < ns) {
                const u32x4 w = *(const u32x4*)(row + 1024 * s + 16 * lane);
                const float* x = &X.x4[s / 4][8 * (s % 4)];
                acc = fmaf(lo_h(w.x), x[0], acc); b = fmaf(hi_h(w.x), x[1], b);
                acc = fmaf(lo_h(w.y), x[2], acc); b = fmaf(hi_h(w.y), x[3], b);
                acc = fmaf(lo_h(w.z), x[4], acc); b = fmaf(hi_h(w.z), x[5], b);
                acc = fmaf(lo_h(w.w), x[6], acc); b = fmaf(hi_h(w.w), x[7], b);
            }
        }
        acc += b;
    }
    return acc;
}

// ---- GEMV job ----

struct JobState {
    float best;
    uint32_t best_i;
};

// Prologue values for the rows a compute wave owns in one chunk: lane t holds row slot t.
struct Pro {
    float yold;
    float st[3];
    float cw[4];
};

__device__ __forceinline__ void run_job(const EngineArgs& a, int j, uint32_t tok, int wg, int nwg, int wave, int lane, uint8_t* smem,
                        int& cseq, Cursor& cur, float* misc) {
    Job J = make_job(a, j, wg, nwg);
    if (J.nchunks == 0) return;
    if (J.xmode == X_EMBED) J.x = misc;  // the step's embedding row, staged in LDS
    if (J.xmode == X_GDN) {
        // 1/rms of every GDN head from its 16 column-block sums of squares
        if (threadIdx.x < a.gdn_heads) {
            float s = 0.0f;
            for (int b = 0; b < 16; b++) s += a.gdn_sq[threadIdx.x * 16 + b];
            misc[kRnorm + threadIdx.x] = 1.0f / sqrtf(s / (float)kDK + 1e-6f);
        }
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        sbarrier();
    }
    XRegs X;
    if (wave < kCW) load_x(a, J, tok, X, lane, misc + kRnorm);
    JobState js{-INFINITY, 0xFFFFFFFFu};
    const int nm = J.epi == E_SWIGLU ? 2 : 1;
    for (int c = 0; c < J.nchunks; c++) {
        const int a0 = J.r0 + c * J.cap, n = min(J.cap, J.r1 - a0);
        Pro p;
        const int my_row = a0 + wave + kCW * lane;  // row slot `lane` of this wave
        const bool has = wave < kCW && lane < kMaxR && wave + kCW * lane < n;
        if (has) {
            if (J.epi == E_ACC) p.yold = J.y[my_row];
            if (J.epi == E_CONV && my_row < J.conv_ch) {
                const float* s = J.conv + (size_t)my_row * 3;
                const float* w = J.conv_w + (size_t)my_row * 4;
                p.st[0] = s[0]; p.st[1] = s[1]; p.st[2] = s[2];
                p.cw[0] = w[0]; p.cw[1] = w[1]; p.cw[2] = w[2]; p.cw[3] = w[3];
            }
        }
        // every load of this chunk's compute is done before the copy wave queues more DMA
        __builtin_amdgcn_s_waitcnt(kWaitAll);
        sbarrier();
        if (wave == kDmaWave) dma_next(a, cur, cseq + 1, smem, wg, nwg, lane);
        if (wave < kCW) {
            const uint8_t* buf = smem + (cseq & 1) * kBuf;
            const uint8_t* szb = buf + nm * n * J.rb;
            // each row is reduced as soon as its dot product is done; lane t keeps row slot t
            float mine_g = 0.0f, mine_u = 0.0f;
            for (int t = 0; t < kMaxR; t++) {
                const int i = wave + kCW * t;
                if (i >= n) break;  // wave-uniform
                const float sg = wave_sum(row_dot(J, buf + i * J.rb, szb + i * J.szb, X, lane)) * X.inv;
                float su = 0.0f;
                if (nm == 2) su = wave_sum(row_dot(J, buf + (n + i) * J.rb, szb + (n + i) * J.szb, X, lane)) * X.inv;
                if (lane == t) { mine_g = sg; mine_u = su; }
            }
            if (has) {
                float out = mine_g;
                if (J.epi == E_ACC) out = p.yold + mine_g;
                else if (J.epi == E_SWIGLU) out = silu(mine_g) * mine_u;
                else if (J.epi == E_CONV && my_row < J.conv_ch) {
                    const float yv = p.st[0] * p.cw[0] + p.st[1] * p.cw[1] + p.st[2] * p.cw[2] + mine_g * p.cw[3];
                    float* s = J.conv + (size_t)my_row * 3;
                    s[0] = p.st[1]; s[1] = p.st[2]; s[2] = mine_g;
                    out = silu(yv);
                }
                J.y[my_row] = out;
                if (J.epi == E_ARGMAX && better(out, (uint32_t)my_row, js.best, js.best_i)) {
                    js.best = out;
                    js.best_i = (uint32_t)my_row;
                }
            }
        }
        cseq++;
    }
    if (J.epi == E_ARGMAX) {
        float b = js.best;
        uint32_t bi = js.best_i;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(b, m, kWave);
            const uint32_t oi = (uint32_t)__shfl_xor((int)bi, m, kWave);
            if (better(ov, oi, b, bi)) { b = ov; bi = oi; }
        }
        float* mv = misc + 1800;
        uint32_t* mi = (uint32_t*)(misc + 1816);
        if (lane == 0) { mv[wave] = b; mi[wave] = bi; }
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        sbarrier();
        if (threadIdx.x == 0) {
            float bb = mv[0];
            uint32_t bbi = mi[0];
            for (int w = 1; w < kCW; w++)
                if (better(mv[w], mi[w], bb, bbi)) { bb = mv[w]; bbi = mi[w]; }
            a.am_val[wg] = bb;
            a.am_idx[wg] = bbi;
        }
    }
}

// ---- Gated DeltaNet step: one wave per value column ----

__device__ __forceinline__ void gdn_phase(const EngineArgs& a, const ELayer& L, int wg, int nwg, int wave, int lane, float* misc) {
    const int H = a.gdn_heads;
    const float* P = a.proj;
    for (int it = wg; it < H * 16; it += nwg) {
        const int h = it / 16, cb = it % 16, t = cb * 8 + wave;
        const float2 q = *(const float2*)(P + h * kDK + 2 * lane);
        const float2 k = *(const float2*)(P + H * kDK + h * kDK + 2 * lane);
        const float v = P[2 * H * kDK + h * kDK + t];
        const float z = P[3 * H * kDK + h * kDK + t];
        const float av = P[4 * H * kDK + h], bv = P[4 * H * kDK + H + h];
        float* S = L.rec + ((size_t)h * kDK + t) * kDK + 2 * lane;
        const float2 s = *(const float2*)S;
        const float nq = 1.0f / sqrtf(wave_sum(q.x * q.x + q.y * q.y) + 1e-6f) * 0.08838834764831845f;
        const float nk = 1.0f / sqrtf(wave_sum(k.x * k.x + k.y * k.y) + 1e-6f);
        const float qx = q.x * nq, qy = q.y * nq, kx = k.x * nk, ky = k.y * nk;
        const float kq = wave_sum(kx * qx + ky * qy);
        const float g = expf(L.prm[H + h] * logf(1.0f + expf(av + L.prm[h])));
        const float beta = 1.0f / (1.0f + expf(-bv));
        const float sk = wave_sum(s.x * kx + s.y * ky);
        const float sq = wave_sum(s.x * qx + s.y * qy);
        const float d = beta * (v - g * sk);
        float2 sn;
        sn.x = fmaf(g, s.x, d * kx);
        sn.y = fmaf(g, s.y, d * ky);
        *(float2*)S = sn;
        const float out = g * sq + d * kq;
        if (lane == 0) {
            a.mixed[h * kDK + t] = out * silu(z) * L.prm[2 * H + t];
            misc[wave] = out * out;
        }
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        sbarrier();
        if (threadIdx.x == 0) {
            float ss = 0.0f;
            for (int w = 0; w < kEW; w++) ss += misc[w];
            a.gdn_sq[h * 16 + cb] = ss;
        }
        sbarrier();
    }
}

// ---- attention: split-context partials + last-arriver merge ----

// RMSNorm (weight w) + rotate-half RoPE of one 256-vector held 4 values per lane.
__device__ __forceinline__ void norm_rope4(float (&v)[4], const float* w, const EngineArgs& a, uint32_t pos,
                                           int lane) {
    float ss = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)kHD + 1e-6f);
    const float4 g = *(const float4*)(w + 4 * lane);
    v[0] = v[0] * inv * g.x; v[1] = v[1] * inv * g.y; v[2] = v[2] * inv * g.z; v[3] = v[3] * inv * g.w;
    const int half = a.rope_dim / 2, partner = half / 4;
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int d = 4 * lane + e;
        const float other_lo = __shfl_down(v[e], partner, kWave);  // value at d + half
        const float other_hi = __shfl_up(v[e], partner, kWave);    // value at d - half
        o[e] = v[e];
        if (d < a.rope_dim) {
            const int i = d < half ? d : d - half;
            float sn, cs;
            sincosf((float)pos * a.inv_freq[i], &sn, &cs);
            o[e] = d < half ? v[e] * cs - other_lo * sn : v[e] * cs + other_hi * sn;
        }
    }
    v[0] = o[0]; v[1] = o[1]; v[2] = o[2]; v[3] = o[3];
}

__device__ __forceinline__ void attn_phase(const EngineArgs& a, const ELayer& L, uint32_t pos, int wg, int wave, int lane,
                           float* misc, float* scratch, int* flag) {
    const int G = a.nq / a.nkv, S = a.splits;
    if (wg >= a.nkv * S) return;
    const int g = wg / S, sp = wg % S;
    const int len = (int)pos + 1;
    const int per = (len + S - 1) / S;
    const int p0 = sp * per, p1 = min(len, p0 + per);
    float* qs = misc;          // [G][256], pre-scaled by 1/sqrt(256)
    float* kc = misc + 1024;   // current key, f16-rounded
    float* vc = misc + 1280;   // current value, f16-rounded
    const float* P = a.proj;
    const int nq = a.nq, nkv = a.nkv;
    if (wave < G) {
        float v[4];
        const float4 f = *(const float4*)(P + (g * G + wave) * kHD + 4 * lane);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        norm_rope4(v, L.norms, a, pos, lane);
#pragma unroll
        for (int e = 0; e < 4; e++) qs[wave * kHD + 4 * lane + e] = v[e] * 0.0625f;
    } else if (wave == G) {
        float v[4];
        const float4 f = *(const float4*)(P + 2 * nq * kHD + g * kHD + 4 * lane);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        norm_rope4(v, L.norms + kHD, a, pos, lane);
        const float4 vv = *(const float4*)(P + 2 * nq * kHD + nkv * kHD + g * kHD + 4 * lane);
        const float val[4] = {vv.x, vv.y, vv.z, vv.w};
        const size_t at = (((size_t)a.block_table[pos / kBlk] * nkv + g) * kBlk + pos % kBlk) * kHD + 4 * lane;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint16_t kh = f2h(v[e]), vh = f2h(val[e]);
            kc[4 * lane + e] = h2f(kh);
            vc[4 * lane + e] = h2f(vh);
            if (sp == 0) { L.k_pool[at + e] = kh; L.v_pool[at + e] = vh; }
        }
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    sbarrier();
    // 8 waves x 2 positions, 32 lanes per position, 8 dims (16 bytes of K and of V) per lane
    const int pg = lane / 32, li = lane % 32;
    float qr[4][8], acc[4][8], m[4], l[4];
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
        m[gi] = -INFINITY;
        l[gi] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; d++) {
            qr[gi][d] = gi < G ? qs[gi * kHD + 8 * li + d] : 0.0f;
            acc[gi][d] = 0.0f;
        }
    }
    for (int p = p0 + 2 * wave + pg; p < p1; p += 2 * kEW) {
        float kf[8], vf[8];
        if (p == (int)pos) {
#pragma unroll
            for (int d = 0; d < 8; d++) { kf[d] = kc[8 * li + d]; vf[d] = vc[8 * li + d]; }
        } else {
            const size_t at = (((size_t)a.block_table[p / kBlk] * nkv + g) * kBlk + p % kBlk) * kHD + 8 * li;
            const u32x4 kw = *(const u32x4*)(L.k_pool + at);
            const u32x4 vw = *(const u32x4*)(L.v_pool + at);
            kf[0] = lo_h(kw.x); kf[1] = hi_h(kw.x); kf[2] = lo_h(kw.y); kf[3] = hi_h(kw.y);
            kf[4] = lo_h(kw.z); kf[5] = hi_h(kw.z); kf[6] = lo_h(kw.w); kf[7] = hi_h(kw.w);
            vf[0] = lo_h(vw.x); vf[1] = hi_h(vw.x); vf[2] = lo_h(vw.y); vf[3] = hi_h(vw.y);
            vf[4] = lo_h(vw.z); vf[5] = hi_h(vw.z); vf[6] = lo_h(vw.w); vf[7] = hi_h(vw.w);
        }
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            if (gi < G) {
                float s = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; d++) s = fmaf(qr[gi][d], kf[d], s);
#pragma unroll
                for (int mk = 16; mk >= 1; mk >>= 1) s += __shfl_xor(s, mk, kWave);  // 32-lane sum
                float pw;
                if (s > m[gi]) {
                    const float corr = expf(m[gi] - s);
                    m[gi] = s;
                    l[gi] *= corr;
#pragma unroll
                    for (int d = 0; d < 8; d++) acc[gi][d] *= corr;
                    pw = 1.0f;
                } else {
                    pw = expf(s - m[gi]);
                }
                l[gi] += pw;
#pragma unroll
                for (int d = 0; d < 8; d++) acc[gi][d] = fmaf(pw, vf[d], acc[gi][d]);
            }
        }
    }
    // merge the 2 position groups of each wave
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
        if (gi < G) {
            const float mo = __shfl_xor(m[gi], 32, kWave), lo = __shfl_xor(l[gi], 32, kWave);
            const float mn = fmaxf(m[gi], mo);
            const float ca = mn == -INFINITY ? 0.0f : expf(m[gi] - mn), cb = mn == -INFINITY ? 0.0f : expf(mo - mn);
#pragma unroll
            for (int d = 0; d < 8; d++) acc[gi][d] = acc[gi][d] * ca + __shfl_xor(acc[gi][d], 32, kWave) * cb;
            l[gi] = l[gi] * ca + lo * cb;
            m[gi] = mn;
            if (pg == 0) {
#pragma unroll
                for (int d = 0; d < 8; d++) scratch[(wave * 4 + gi) * kHD + 8 * li + d] = acc[gi][d];
                if (li == 0) { misc[1536 + (wave * 4 + gi) * 2] = m[gi]; misc[1536 + (wave * 4 + gi) * 2 + 1] = l[gi]; }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    sbarrier();
    // merge the waves; waves 0-3 write this workgroup's partial
    if (wave < 4) {
        const int t = threadIdx.x;  // 0..255 = dim
        const size_t base = ((size_t)g * S + sp) * G;
        for (int gi = 0; gi < G; gi++) {
            float mn = -INFINITY;
            for (int w = 0; w < kEW; w++) mn = fmaxf(mn, misc[1536 + (w * 4 + gi) * 2]);
            float ls = 0.0f, ac = 0.0f;
            for (int w = 0; w < kEW; w++) {
                const float mw = misc[1536 + (w * 4 + gi) * 2];
                const float c = mw == -INFINITY ? 0.0f : expf(mw - mn);
                ls += misc[1536 + (w * 4 + gi) * 2 + 1] * c;
                ac += scratch[(w * 4 + gi) * kHD + t] * c;
            }
            a.att_acc[(base + gi) * kHD + t] = ac;
            if (t == 0) { a.att_ml[(base + gi) * 2] = mn; a.att_ml[(base + gi) * 2 + 1] = ls; }
        }
        __builtin_amdgcn_s_waitcnt(kWaitAll);
    }
    sbarrier();
    if (threadIdx.x == 0) {
        __atomic_thread_fence(__ATOMIC_RELEASE);
        const unsigned prev = __hip_atomic_fetch_add(a.att_cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == (unsigned)(S - 1);
        if (last) {
            __atomic_thread_fence(__ATOMIC_ACQUIRE);
            __hip_atomic_store(a.att_cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        *flag = last;
    }
    sbarrier();
    if (*(volatile int*)flag && wave < 4) {
        const int t = threadIdx.x;
        for (int gi = 0; gi < G; gi++) {
            float mn = -INFINITY;
            for (int s = 0; s < S; s++) mn = fmaxf(mn, a.att_ml[(((size_t)g * S + s) * G + gi) * 2]);
            float ls = 0.0f, ac = 0.0f;
            for (int s = 0; s < S; s++) {
                const size_t i = ((size_t)g * S + s) * G + gi;
                const float ms = a.att_ml[i * 2];
                if (ms == -INFINITY) continue;
                const float c = expf(ms - mn);
                ls += a.att_ml[i * 2 + 1] * c;
                ac += a.att_acc[i * kHD + t] * c;
            }
            const int h = g * G + gi;
            const float gate = P[nq * kHD + h * kHD + t];
            a.mixed[h * kHD + t] = ac / ls / (1.0f + expf(-gate));
        }
    }
}

// ---- the kernel ----

__global__ __launch_bounds__(kEngineThreads, 1) void k_engine(EngineArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kBuf];
    __shared__ __attribute__((aligned(16))) float misc[kMiscFloats];
    __shared__ int flag;
    const int wg = blockIdx.x, nwg = gridDim.x, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    unsigned epoch = 0;
    int cseq = 0;
    Cursor cur{0, 0, 0, false};
    if (wave == kDmaWave) dma_next(a, cur, 0, smem, wg, nwg, lane);
    uint32_t token = a.feed ? a.tok[0] : a.ids[0];
    for (int step = 0; step < a.n_steps; step++) {
        const uint32_t pos = a.pos0 + (uint32_t)step;
        if (step > 0 && !a.feed) token = a.ids[step];
        const bool head = a.head == 1 || (a.head == 2 && step == a.n_steps - 1);
        // embedding row of the token (kernels/src/shaders.rs:405-434): staged in LDS as the
        // in-projection input of layer 0; workgroup 0 also writes it to the residual stream h
        for (int c = threadIdx.x; c < a.hidden; c += kEngineThreads) {
            const float v = embed_val(a.embed, token, c);
            misc[c] = v;
            if (wg == 0) a.h[c] = v;
        }
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        sbarrier();
        // phases of the step: per layer [in-proj, mixer, out-proj, gate_up, down], then the head;
        // each phase function has a single call site so it is inlined once
        const int nph = 5 * a.n_layers + (head ? 1 : 0);
        for (int ph = 0; ph < nph; ph++) {
            const int l = ph / 5, k = ph % 5;
            const bool mixer = l < a.n_layers && k == 1;
            if (mixer) {
                const ELayer& L = a.layers[l];
                float* scratch = (float*)(smem + ((cseq + 1) & 1) * kBuf);  // slot not being filled
                if (L.attn) attn_phase(a, L, pos, wg, wave, lane, misc, scratch, &flag);
                else gdn_phase(a, L, wg, nwg, wave, lane, misc);
            } else {
                const int j = l < a.n_layers ? 4 * l + (k == 0 ? 0 : k - 1) : 4 * a.n_layers;
                run_job(a, j, token, wg, nwg, wave, lane, smem, cseq, cur, misc);
            }
            if (!grid_sync(a, epoch, nwg, wave, mixer, &flag)) {
                // no LDS DMA may still be in flight when the workgroup ends
                __builtin_amdgcn_s_waitcnt(kWaitAll);
                return;
            }
        }
        if (head) {
            if (a.argmax) {
                // every workgroup reduces the per-workgroup picks itself
                float b = -INFINITY;
                uint32_t bi = 0xFFFFFFFFu;
                for (int i = threadIdx.x; i < nwg; i += kEngineThreads) {
                    const float v = a.am_val[i];
                    const uint32_t ix = a.am_idx[i];
                    if (better(v, ix, b, bi)) { b = v; bi = ix; }
                }
#pragma unroll
                for (int m = 32; m >= 1; m >>= 1) {
                    const float ov = __shfl_xor(b, m, kWave);
                    const uint32_t oi = (uint32_t)__shfl_xor((int)bi, m, kWave);
                    if (better(ov, oi, b, bi)) { b = ov; bi = oi; }
                }
                float* mv = misc + 1900;
                uint32_t* mi = (uint32_t*)(misc + 1916);
                if (lane == 0) { mv[wave] = b; mi[wave] = bi; }
                __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
                sbarrier();
                float bb = mv[0];
                uint32_t bbi = mi[0];
                for (int w = 1; w < kEW; w++)
                    if (better(mv[w], mi[w], bb, bbi)) { bb = mv[w]; bbi = mi[w]; }
                const uint32_t pick = bbi == 0xFFFFFFFFu ? 0u : bbi;
                token = pick;
                if (wg == 0 && threadIdx.x == 0) {
                    a.tok[0] = pick;
                    a.tok[1] = pos + 1;
                    if (a.out_ids) {
                        const uint32_t n = a.tok[2];
                        if (n < a.out_cap) a.out_ids[n] = pick;
                        a.tok[2] = n + 1;
                    }
                }
                sbarrier();
            }
        }
    }
    // drain the copy wave (a prefetch past the last chunk is never issued, but be explicit)
    __builtin_amdgcn_s_waitcnt(kWaitAll);
}

hipError_t launch_engine(const EngineArgs& a, int grid, hipStream_t st) {
    void* args[] = {(void*)&a};
    return hipLaunchCooperativeKernel((const void*)k_engine, dim3(grid), dim3(kEngineThreads), args, 0, st);
}

int engine_max_grid() {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void*)k_engine, kEngineThreads, 0) != hipSuccess)
        return 0;
    return cus * (per > 1 ? 1 : per);
}

}  // namespace qne
