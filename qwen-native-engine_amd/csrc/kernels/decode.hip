// Persistent decode kernel: every decode step of the hybrid decoder in ONE cooperative launch.
//
// Reference: the per-token dispatch list of Model::load (kernels/src/model.rs:220-269) and its
// kernels (kernels/src/shaders.rs): embed, per layer [rmsnorm, mixer_in GEMV, gdn | attention,
// mixer_out GEMV (+=), rmsnorm, gate_up GEMV (SwiGLU), down GEMV (+=)], rmsnorm, lm_head GEMV,
// argmax. A batch-1 token of the 2B-shaped int4 model moves ~1.74 GB in ~150 dependent pieces of
// 2-14 MB, so a token is latency-bound unless (1) the hand-over between pieces is cheap and
// (2) HBM keeps streaming while the chip waits for it. Design for MI355X (256 CUs, 8 XCDs with
// private L2s):
//  - one workgroup of 8 waves per CU, all co-resident (cooperative launch). The phases of a token
//    form a fixed program (decode.hpp `Phase`, built once at load);
//  - hand-over by tagged values: a phase publishes each output f32 together with a 32-bit tag
//    (its sequence number) in one 8-byte agent-scope store; the next phase polls with agent-scope
//    16-byte loads until every tag it needs is current. There is no grid barrier and no release /
//    acquire fence, so no L2 writeback or invalidate: on MI355X those cost ~10 us per barrier
//    against ~2.4 us for a tagged exchange of a 2048-vector;
//  - each wave owns 16 KiB of LDS in two 8 KiB halves; the phases that read prefetched data
//    ("region phases": LDS GEMVs, GDN, attention) alternate between the halves. When a region
//    phase has done its last LDS read it sends the data of the region phase two ahead into the
//    half it just freed (global_load_lds_dwordx4), and only then waits for the next phase's input:
//    the weight stream then overlaps the hand-over, and nothing the phase computes waits behind it
//    (vector-memory completion is in order, and the compiler makes any LDS read that follows an
//    LDS DMA wait for it). A wave only ever reads what it loaded itself: no cross-wave handshake;
//  - rows are spread over waves wave-major (wave w of every workgroup before wave w+1), so every
//    workgroup owns rows of every vector that all workgroups consume;
//  - RMSNorm is folded into the input exchange (the poll multiplies by the gain and sums the
//    squares of the raw values); the GDN causal conv + SiLU runs in the epilogue of the
//    in-projection rows that own those channels; the residual stream h lives in the registers of
//    the waves that own its rows and is published after each residual add;
//  - GDN: one workgroup per (head, 8 value columns), one wave per column, its 512-byte state column
//    prefetched into LDS; the layer's in-projection rows run in the same phase (PH_GDNF), each
//    head's q / k exchanged among its 16 workgroups. Attention: split-context partials per (kv
//    head, split) with GQA reuse, K/V rows prefetched into LDS through the block table, merged per
//    (q head, 64 dims) with the sigmoid gate by the split workgroups in the same phase (fold), or
//    in a combine phase of its own for shapes with fewer splits than 4 per q head;
//  - the q4 GEMVs run on v_mfma_i32_16x16x64_i8: rows tiled per workgroup, K split over waves, x
//    as three signed base-256 digits of a 22-bit fixed point per 64 columns;
//  - the LM head tracks a per-wave argmax; workgroups publish their best and every workgroup
//    reduces all of them, so the next step needs no separate broadcast.
#include <cstddef>
#include <cstring>

#include "common.hpp"
#include "decode.hpp"
#include "gemv.hpp"

namespace qne {

namespace {

constexpr int kT = kDecodeThreads;
constexpr int kNW = kT / kWave;        // 8 waves
constexpr int kXs = 6144;              // floats of LDS input staging
constexpr int kHalf = 8 * 1024;        // bytes of one half of a wave's LDS region
constexpr int kWaveLds = 2 * kHalf;    // a wave's region: the running phase's half and the next one's
constexpr int kConvSlots = 5;          // EP_CONV outputs per wave and half whose conv state / weights sit in LDS
constexpr int kExtraBytes = 2304;      // the workgroup's extra GEMV output slot (rows [nm][rb], then [nm][szb])
constexpr int kPoll = 6;               // tagged pairs a thread polls at once
constexpr int kSC1 = 16;               // cache policy: agent-scope coherent access
constexpr int kNT = 2;                 // cache policy: non-temporal (streamed once; keeps L2 for reused data)
constexpr int kBlk = 16;               // KV block size (positions)
constexpr int kDK = 128;               // GDN dk = dv
constexpr int kAttnU = kHalf / 2048;   // prefetched K/V wave-loads (2 positions each) per wave
// Attention scores are kept in base 2: q is pre-scaled by log2(e) / sqrt(256), so every softmax
// weight is one hardware exp2 (v_exp_f32) instead of a range-reduced expf.
constexpr float kScoreScale = 1.4426950408889634f * 0.0625f;

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// s_waitcnt until at most N vector-memory operations of this wave are outstanding. Written as
// asm with a memory clobber: the compiler then keeps every load of LDS data the wait protects
// (rows landed by LDS DMA) after it.
template <int N>
__device__ __forceinline__ void wait_vm_n() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Every counter to zero (all of this wave's memory operations done), with the same ordering.
__device__ __forceinline__ void wait_all() { asm volatile("s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0)" ::: "memory"); }
// Rounds n down to a supported count, so the wait is never shorter than asked for.
__device__ __forceinline__ void wait_vm(int n) {
    if (n >= 48) wait_vm_n<48>();
    else if (n >= 32) wait_vm_n<32>();
    else if (n >= 24) wait_vm_n<24>();
    else if (n >= 16) wait_vm_n<16>();
    else if (n >= 12) wait_vm_n<12>();
    else if (n >= 8) wait_vm_n<8>();
    else if (n >= 6) wait_vm_n<6>();
    else if (n >= 4) wait_vm_n<4>();
    else if (n >= 3) wait_vm_n<3>();
    else if (n >= 2) wait_vm_n<2>();
    else if (n >= 1) wait_vm_n<1>();
    else wait_vm_n<0>();
}

// The program and the per-layer parameters are read through the constant address space: they do
// not change during a launch, so the compiler reads them with scalar loads, which do not wait
// behind the wave's outstanding weight DMA (vector-memory completion is in order).
typedef const __attribute__((address_space(4))) Phase CPhase;
typedef const __attribute__((address_space(4))) PhaseBufs CBufs;
typedef const __attribute__((address_space(4))) float cfloat;
typedef const __attribute__((address_space(4))) GdnExtra CGdnX;

__device__ __forceinline__ void cbar() { asm volatile("" ::: "memory"); }
// The lane id computed where it is used (volatile: the compiler does not hoist it, or values derived
// from it, out of the phase loop, where they would hold registers for the whole launch).
__device__ __forceinline__ int lane_here() {
    uint32_t l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return (int)l;
}
// 2^x on the hardware unit (exp2(-inf) = 0).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }
// Workgroup barrier for LDS hand-offs only. Unlike __syncthreads it does not wait for the wave's
// outstanding global loads (the prefetch of the next phase stays in flight).
__device__ __forceinline__ void bar() {
    cbar();
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    cbar();
}

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Publishes value v at index i of a tagged buffer (write-through to the device coherence point).
__device__ __forceinline__ void put(uint64_t* buf, uint32_t i, float v, uint32_t tag) {
    __hip_atomic_store(buf + i, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// 16 bytes of K or V stored with an agent-scope (write-through) store at byte `off` of a 512-byte
// row. `row` is the same in every lane: one buffer resource serves the wave, so the store is one
// instruction (a resource that differs between lanes makes the compiler loop over them).
__device__ __forceinline__ void st16_agent(uint16_t* row, uint32_t off, u32x4 v) {
    const rsrc_t r = make_rsrc(row, 2 * kHeadDim);
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kSC1);
}

struct Ctl {
    unsigned* err;
    unsigned spin;
    int* bail;  // LDS
};

// Polls n tagged pairs of `buf` (cap readable u64 entries). Pair q lives at u64 index src(q)
// (even); fn(q, v0, v1) consumes it. Every thread of the workgroup calls this; the caller ends
// with a barrier. On a timeout the error flag is raised and *bail set.
template <class Src, class Fn>
__device__ __forceinline__ void poll_pairs(const uint64_t* buf, uint32_t cap, int n, uint32_t tag, Src src, Fn fn,
                                           const Ctl& c) {
    const rsrc_t rs = make_rsrc(buf, cap * 8u);
    for (int base = 0; base < n; base += kT * kPoll) {
        unsigned pend = 0;
#pragma unroll
        for (int j = 0; j < kPoll; j++)
            if (base + j * kT + (int)threadIdx.x < n) pend |= 1u << j;
        unsigned spins = 0;
        while (pend) {
            u32x4 v[kPoll];
#pragma unroll
            for (int j = 0; j < kPoll; j++)
                if ((pend >> j) & 1u) v[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, 8 * src(base + j * kT + (int)threadIdx.x), 0, kSC1);
#pragma unroll
            for (int j = 0; j < kPoll; j++) {
                if (((pend >> j) & 1u) && v[j].y == tag && v[j].w == tag) {
                    fn(base + j * kT + (int)threadIdx.x, __uint_as_float(v[j].x), __uint_as_float(v[j].z));
                    pend &= ~(1u << j);
                }
            }
            if (pend && (++spins > c.spin || ((spins & 31u) == 0 && ld_agent(c.err)))) {
                st_agent(c.err, 1u);
                *c.bail = 1;
                return;
            }
        }
    }
}

// Contiguous share of `rows` for global wave index gw of nw.
struct Rows {
    int r0, n;
};
__device__ __forceinline__ Rows part(int rows, int gw, int nw) {
    const int per = rows / nw, rem = rows % nw;
    return {gw * per + min(gw, rem), per + (gw < rem ? 1 : 0)};
}
// The same for a phase's outputs (rows / waves precomputed on the host).
__device__ __forceinline__ Rows part_p(CPhase& P, int gw) {
    return {gw * P.rper + min(gw, P.rrem), P.rper + (gw < P.rrem ? 1 : 0)};
}

// ---- DMA into the wave's LDS region ----

// Weights and recurrent state are streamed once per token, so they are loaded non-temporal: the
// L2 then keeps the small data every phase re-reads (program, norms, block table, conv weights).
// One LDS DMA of 16 bytes per active lane (global_load_lds_dwordx4: lane l lands at dst + 16 l),
// written as asm so that the compiler does not see an LDS write: it then does not make the LDS reads
// of the running phase wait for the next phase's transfer. Readers of dst wait for it explicitly
// (wait_all / wait_vm). m0 carries the LDS address; its previous value is restored.
template <bool NT>
__device__ __forceinline__ void lds_dma16(const void* src, void* dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_ptr_t)dst);
    uint32_t saved;
    if (NT)
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(src), "s"(lds) : "memory");
    else
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(src), "s"(lds) : "memory");
}

// 4 bytes per active lane (global_load_lds_dword: lane l lands at dst + 4 l), as lds_dma16.
template <bool NT>
__device__ __forceinline__ void lds_dma4(const void* src, void* dst) {
    const uint32_t lds = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(lds_ptr_t)dst);
    uint32_t saved;
    if (NT)
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off nt\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(src), "s"(lds) : "memory");
    else
        asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                     : "=&s"(saved) : "v"(src), "s"(lds) : "memory");
}

// `bytes` (a multiple of 16) from src to dst in 1 KiB wave transfers.
__device__ __forceinline__ void dma_bytes(const uint8_t* src, int bytes, uint8_t* dst, int lane) {
    for (int u = 0; u * 1024 < bytes; u++) {
        const int off = u * 1024 + lane * 16;
        if (off < bytes) lds_dma16<true>(src + off, dst + u * 1024);
    }
}

// Geometry of a GEMV phase's rows in a region.
struct GemvGeo {
    int rb, szb, stride, nm, cap;  // row bytes, scale/zero bytes, bytes per row, rows per output, outputs per half
    int per;                       // DMA instructions per output
    int conv;                      // EP_CONV: bytes of conv state + weights per output (16 + 16)
    int extra;                     // one output past cap in the workgroup's extra slot (P.extra)
};
__device__ __forceinline__ GemvGeo geo(CPhase& P) {
    GemvGeo g;
    g.rb = P.rb;
    g.szb = P.szb;
    g.stride = P.stride;
    g.nm = P.nm;
    g.conv = P.convb;
    g.cap = P.cap;
    g.per = P.dper;
    g.extra = P.extra;
    return g;
}

// DMA of outputs [o0, o0 + cnt) (row pairs for SwiGLU) into region slots starting at `slot`.
// LDS layout of a GEMV phase in a half: the nibble (or f16) rows [nm][cap][rb], then the q4
// (scale, zero) rows [nm][cap][szb]. With P.extra, output cap of wave 0 sits in the workgroup's
// extra slot ([nm][rb], then [nm][szb]). The in-projection's conv states and weights sit in the
// wave's conv area of the half ([kConvSlots][16 B] states, then [kConvSlots][16 B] weights).
// Row m of the output in slot s:
__device__ __forceinline__ int lds_w(const GemvGeo& g, int s, int m) { return (m * g.cap + s) * g.rb; }
__device__ __forceinline__ int lds_sz(const GemvGeo& g, int s, int m) {
    return g.nm * g.cap * g.rb + (m * g.cap + s) * g.szb;
}


// DMA of output o into the workgroup's extra slot.
__device__ __forceinline__ void dma_extra(CPhase& P, CBufs& B, const GemvGeo& g, int o, uint8_t* __restrict__ ex, int lane) {
    const uint8_t* w = (const uint8_t*)B.w;
    const uint8_t* sz = (const uint8_t*)B.sz;
    for (int m = 0; m < g.nm; m++) {
        const size_t row = (size_t)o + (size_t)m * P.rows;
        dma_bytes(w + row * g.rb, g.rb, ex + m * g.rb, lane);
        if (g.szb) dma_bytes(sz + row * g.szb, g.szb, ex + g.nm * g.rb + m * g.szb, lane);
    }
}

// DMA of outputs [o0, o0 + cnt) into slots [slot, slot + cnt). Consecutive outputs are consecutive
// rows of each of the nm matrices, so each block is one contiguous transfer.
__device__ __forceinline__ void dma_rows(CPhase& P, CBufs& B, const GemvGeo& g, int o0, int cnt, int slot,
                                         uint8_t* __restrict__ reg, int lane) {
    const uint8_t* w = (const uint8_t*)B.w;
    const uint8_t* sz = (const uint8_t*)B.sz;
    for (int m = 0; m < g.nm; m++) {
        const size_t row = (size_t)o0 + (size_t)m * P.rows;
        dma_bytes(w + row * g.rb, cnt * g.rb, reg + lds_w(g, slot, m), lane);
        if (g.szb) dma_bytes(sz + row * g.szb, cnt * g.szb, reg + lds_sz(g, slot, m), lane);
    }
}

// ---- input vector slice in registers ----

// The input vector is consumed in steps of at most 32 values per lane, so that only one step's
// slice of x lives in registers while it is applied to a group of up to 8 rows:
//  - q4 rows (K <= 6144): step s < n4 is the 2048-column slab s (32 values per lane, 16 bytes of
//    nibbles), then at most one 1024-column slab (16 values, 8 bytes) and one 512-column slab
//    (8 values, 4 bytes);
//  - f16 rows: step j is the 512-column slab j (8 values, 16 bytes per lane).
struct Step {
    int kind, K, n4, n2, n1, nsteps;
    int gdn;  // the input is a GDN output: each lane's slice is scaled by its head's 1/rms
};
__device__ __forceinline__ Step make_step(CPhase& P) {
    Step t;
    t.kind = P.mkind;
    t.K = P.k;
    t.n4 = P.n4;
    t.n2 = P.n2;
    t.n1 = P.n1;
    t.nsteps = P.nsteps;
    t.gdn = P.xnorm == XN_GDN;
    return t;
}

// Position in xs of input value k of a GEMV of this shape. Each slab's lane slices are stored
// chunk-major: chunk c (4 values) of lane l at slab_base + 256c + 4l, so a wave reading chunk c of
// its slices touches 64 consecutive 16-byte words (no LDS bank conflicts). Values past K (the GDN
// partial sums of squares) keep their index.
__device__ __forceinline__ int xs_slot(const Step& t, int k) {
    if (k >= t.K) return k;
    int base, sh;  // slab base and log2(values per lane)
    if (t.kind == 1) {
        if (k < 2048 * t.n4) { base = k & ~2047; sh = 5; }
        else if (k < 2048 * t.n4 + 1024 * t.n2) { base = 2048 * t.n4; sh = 4; }
        else { base = 2048 * t.n4 + 1024 * t.n2; sh = 3; }
    } else {
        base = k & ~511;
        sh = 3;
    }
    const int w = k - base, l = w >> sh, i = w & ((1 << sh) - 1);
    return base + ((i >> 2) << 8) + (l << 2) + (i & 3);
}

struct XC {
    float x[32];
    float sum;    // q4: sum of the step's values (the zero-point term)
    float scale;  // the slice's factor: 1, or its head's 1/rms for a GDN output
};

// Inverse of xs_slot for a position d < K of the chunk-major staging.
__device__ __forceinline__ int xs_value(const Step& t, int d) {
    int base, sh;
    if (t.kind == 1) {
        if (d < 2048 * t.n4) { base = d & ~2047; sh = 5; }
        else if (d < 2048 * t.n4 + 1024 * t.n2) { base = 2048 * t.n4; sh = 4; }
        else { base = 2048 * t.n4 + 1024 * t.n2; sh = 3; }
    } else {
        base = d & ~511;
        sh = 3;
    }
    const int w = d - base, i = ((w >> 8) << 2) + (w & 3), l = (w >> 2) & 63;
    return base + (l << sh) + i;
}

// Slab of step j: base, chunks of 4 values per lane.
__device__ __forceinline__ void step_slab(const Step& t, int j, int& base, int& nch) {
    if (t.kind == 1) {
        if (j < t.n4) { base = 2048 * j; nch = 8; }
        else if (j < t.n4 + t.n2) { base = 2048 * t.n4; nch = 4; }
        else { base = 2048 * t.n4 + 1024 * t.n2; nch = 2; }
    } else {
        base = 512 * j;
        nch = 2;
    }
}

// The lane's values of step j from xs, and (q4) their sum.
__device__ __forceinline__ void load_step(const float* xs, const Step& t, int j, XC& X, int lane) {
    int base, nch;
    step_slab(t, j, base, nch);
    float sm = 0.0f;  // q4: the slice's sum (the zero-point term), chunk by chunk
#pragma unroll
    for (int c = 0; c < 8; c++) {
        if (c < nch) {
            const float4 f = *(const float4*)(xs + base + 256 * c + 4 * lane);
            X.x[4 * c] = f.x; X.x[4 * c + 1] = f.y; X.x[4 * c + 2] = f.z; X.x[4 * c + 3] = f.w;
            sm += (f.x + f.y) + (f.z + f.w);
        }
    }
    X.sum = t.kind == 1 ? sm : 0.0f;
    X.scale = 1.0f;
    if (t.gdn) {
        // GDN output norm (kernels/src/shaders.rs:514): the lane's slice lies in one 128-value head;
        // its 1/rms comes from the head's 16 published partial sums of squares (staged past K)
        const int h = (base + lane * 4 * nch) / kDK;
        const float4* ps = (const float4*)(xs + t.K + 16 * h);
        const float4 a = ps[0], b = ps[1], c = ps[2], d = ps[3];
        const float ssum = (((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w))) +
                           (((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w)));
        X.scale = 1.0f / sqrtf(ssum / (float)kDK + 1e-6f);
    }
}

// Nibble c of w times x[c], c = 0..7. The even and odd nibbles are masked into bytes once, and the
// empty asm keeps the compiler from folding the mask back into a bit-field extract per nibble: each
// value then costs one v_cvt_f32_ubyteN and one FMA.
__device__ __forceinline__ float dot8(uint32_t w, const float* x) {
    uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    asm("" : "+v"(lo), "+v"(hi));
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

// The lane's share, over every step of x, of the dot products of NR rows held in LDS at
// cur + roff[r] (q4: the row's (scale, zero) pairs at cur + soff[r]; gs = log2 of the group size). Each slab type has its own loop with the NR rows unrolled and no branch between
// them, so a step's LDS reads for all rows issue together. X holds step 0 when nsteps is 1.
template <int NR>
__device__ __forceinline__ void rows_dot(const Step& t, int gs, const uint8_t* cur, const int (&roff)[8],
                                         const int (&soff)[8], const float* xs, XC& X, int lane,
                                         float (&acc)[8]) {
    const bool reload = t.nsteps > 1;
    if (t.kind == 1) {
        for (int j = 0; j < t.n4; j++) {
            if (reload) load_step(xs, t, j, X, lane);
            u32x4 w[NR];
            uint32_t sz[NR];
#pragma unroll
            for (int r = 0; r < NR; r++) {
                w[r] = *(const u32x4*)(cur + roff[r] + 1024 * j + 16 * lane);
                sz[r] = *(const uint32_t*)(cur + soff[r] + 4 * ((2048 * j + 32 * lane) >> gs));
            }
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const float dq = dot8(w[r].x, &X.x[0]) + dot8(w[r].y, &X.x[8]) + dot8(w[r].z, &X.x[16]) + dot8(w[r].w, &X.x[24]);
                acc[r] += (X.scale * lo_h(sz[r])) * (dq - hi_h(sz[r]) * X.sum);
            }
        }
        if (t.n2) {
            const int j = t.n4;
            if (reload) load_step(xs, t, j, X, lane);
            u32x2 w[NR];
            uint32_t sz[NR];
#pragma unroll
            for (int r = 0; r < NR; r++) {
                w[r] = *(const u32x2*)(cur + roff[r] + 1024 * t.n4 + 8 * lane);
                sz[r] = *(const uint32_t*)(cur + soff[r] + 4 * ((2048 * t.n4 + 16 * lane) >> gs));
            }
#pragma unroll
            for (int r = 0; r < NR; r++)
                acc[r] += (X.scale * lo_h(sz[r])) * (dot8(w[r].x, &X.x[0]) + dot8(w[r].y, &X.x[8]) - hi_h(sz[r]) * X.sum);
        }
        if (t.n1) {
            const int j = t.n4 + t.n2;
            if (reload) load_step(xs, t, j, X, lane);
            uint32_t w[NR], sz[NR];
#pragma unroll
            for (int r = 0; r < NR; r++) {
                w[r] = *(const uint32_t*)(cur + roff[r] + 1024 * t.n4 + 512 * t.n2 + 4 * lane);
                sz[r] = *(const uint32_t*)(cur + soff[r] + 4 * ((2048 * t.n4 + 1024 * t.n2 + 8 * lane) >> gs));
            }
#pragma unroll
            for (int r = 0; r < NR; r++) acc[r] += (X.scale * lo_h(sz[r])) * (dot8(w[r], &X.x[0]) - hi_h(sz[r]) * X.sum);
        }
    } else {
        for (int j = 0; j < t.nsteps; j++) {
            if (reload) load_step(xs, t, j, X, lane);
            u32x4 w[NR];
#pragma unroll
            for (int r = 0; r < NR; r++) w[r] = *(const u32x4*)(cur + roff[r] + 1024 * j + 16 * lane);
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const float* x = &X.x[0];
                float a = lo_h(w[r].x) * x[0], b = hi_h(w[r].x) * x[1];
                a = fmaf(lo_h(w[r].y), x[2], a); b = fmaf(hi_h(w[r].y), x[3], b);
                a = fmaf(lo_h(w[r].z), x[4], a); b = fmaf(hi_h(w[r].z), x[5], b);
                a = fmaf(lo_h(w[r].w), x[6], a); b = fmaf(hi_h(w[r].w), x[7], b);
                acc[r] += X.scale * (a + b);
            }
        }
    }
}

// Per-wave state carried across phases.
struct WaveState {
    float hown[2];   // residual rows this wave owns (uniform across lanes)
    float best;      // argmax of the LM head rows this lane reduced
    uint32_t best_i;
};

struct Env {
    const DecodeArgs* a;
    int wg, nwg, wave, lane, gwm, nw;
    float* xs;
    uint8_t* regs;  // all waves' regions
    float* red;
    int* bail;
    unsigned long long* tt;  // profiling: the running phase's sub-step timestamps (thread 0's, in LDS)
};

__device__ __forceinline__ uint32_t tag_of(const DecodeArgs& a, int step, int p) {
    return a.tag_base + (uint32_t)step * (uint32_t)a.nph + (uint32_t)p;
}

// Profiling only: timestamp k (0..7) of the running phase, kept in registers until the phase ends.
__device__ __forceinline__ void mark(const Env& e, int k) {
    if (e.a->sub && threadIdx.x == 0) e.tt[k] = __builtin_amdgcn_s_memrealtime();
}

// Whether the LM head has a register-streaming path (else it goes through the LDS region).
__device__ __forceinline__ bool head_fast(CPhase& P) { return P.fast_head != 0; }
// Phases whose data is prefetched into a wave's LDS half.
__device__ __forceinline__ bool uses_region(CPhase& P) { return P.region != 0; }
__device__ __forceinline__ bool head_at(const DecodeArgs& a, int step) {
    return a.head == 1 || (a.head == 2 && step == a.n_steps - 1);
}
// The k-th (1 or 2) region phase after phase p of `step`, from the links set on the host: the
// step's own next region phases, then the LM head when it runs on this step, then the next step's
// first two. False past the window.
__device__ __forceinline__ bool region_after(const DecodeArgs& a, CPhase& P, int step, int p, int k, int& ns, int& np) {
    int c = 0;
    for (int i = 0; i < 2; i++) {
        if (P.nr[i] < 0) break;
        if (++c == k) { ns = step; np = p + P.nr[i]; return true; }
    }
    if (a.head_reg >= 0 && p < a.head_reg && head_at(a, step) && ++c == k) { ns = step; np = a.head_reg; return true; }
    if (step + 1 < a.n_steps) {
        if (++c == k) { ns = step + 1; np = a.reg0; return true; }
        if (++c == k) { ns = step + 1; np = a.reg1; return true; }
    }
    return false;
}

// First position of context split sp of S over len positions (sp * len < 2^32: len <= 2^16, S <= 92).
__device__ __forceinline__ int split_at(int sp, uint32_t len, int S) { return (int)(((uint32_t)sp * len) / (uint32_t)S); }

// ---- the fused GDN phase (PH_GDNF): geometry ----
// Workgroup w takes item (head h, value columns 8cb..8cb+7); with P.xcd the 16 items of a head go
// to workgroups of one w % 8 class, which the dispatcher places on one XCD, so the head's q / k
// exchange stays in that XCD's L2. Wave `wave` of the item owns channel t = 8cb + wave of the head:
// its projection rows q_t, k_t, v_t, z_t (slots 0..3) and, for cb 0 and waves 0 / 1, the head's
// a / b row (slot 4). LDS half: the slots' rows [5][rb], their (scale, zero) rows [5][szb], the
// conv state and weights of slots 0..2 (6 x 16 bytes), then the 512-byte state column t.
constexpr int kGfSlots = 5;
__device__ __forceinline__ int gf_item(CPhase& P, int w) {
    if (!P.xcd) return w;
    const int x = w & 7, j = w >> 3;
    return (x * (P.heads >> 3) + (j >> 4)) * 16 + (j & 15);
}
__device__ __forceinline__ int gf_nrows(int cb, int wave) { return cb == 0 && wave < 2 ? 5 : 4; }
__device__ __forceinline__ int gf_row(int H, int h, int t, int wave, int slot) {
    return slot < 4 ? slot * H * kDK + h * kDK + t : 4 * H * kDK + wave * H + h;
}
__device__ __forceinline__ int gf_conv(CPhase& P) { return kGfSlots * P.stride; }
__device__ __forceinline__ int gf_state(CPhase& P) { return (kGfSlots * P.stride + 96 + 127) & ~127; }

// ---- the tiled q4 GEMV (PH_GEMV with P.tiled): geometry ----
// Workgroup g owns outputs [o0, o0 + n) (rper / rrem per workgroup), in tiles of 16 matrix rows
// (16 outputs, or 8 gate rows then the same 8 outputs' up rows), each tile two groups of 8 rows. K is
// cut into 64-column chunks (one q4 group of 64, or half of a group of 128); wave w takes the
// contiguous chunks [w Cw, (w + 1) Cw) of every tile, in blocks of 4 (128 bytes of a row: one cache
// line). It prefetches exactly those into its half: nibbles [tile][block][row group 2][16-byte piece
// 8][row 8][16 B] (one DMA instruction per (tile, block, row group): 8 whole lines; a chunk's 64-lane
// B operand is then 512 contiguous bytes), then (scale, zero) pairs [tile][chunk][row 16][4 B].
typedef int i32x4 __attribute__((ext_vector_type(4)));
// the workgroup's residual rows in the tiled layout (h_tiled), and the waves' partial row sums of a
// tiled GEMV [kNW][4 tiles][16 rows]: fixed LDS addresses, no register holds them
__shared__ float s_hres[kTiledMaxRes];
__shared__ float s_tsum[kNW * 4 * 16];
// EP_CONV conv state and weights: [half][wave][16 B state x kConvSlots, 16 B weights x kConvSlots];
// and the workgroup's extra GEMV output slot (wave 0 of a phase with P.extra). At file scope their
// LDS addresses are constants, so no register holds them.
__shared__ __attribute__((aligned(16))) uint8_t s_conv[2 * kNW * kConvSlots * 32];
__shared__ __attribute__((aligned(16))) uint8_t s_extra[kExtraBytes];
__device__ __forceinline__ uint8_t* conv_area(int half, int wave) { return s_conv + (half * kNW + wave) * (kConvSlots * 32); }
__device__ __forceinline__ void t_outputs(CPhase& P, int g, int& o0, int& n) {
    o0 = g * P.rper + min(g, P.rrem);
    n = P.rper + (g < P.rrem ? 1 : 0);
}
// Matrix row of tile slot (t, j), or -1 for a padding slot.
__device__ __forceinline__ int t_row(CPhase& P, int o0, int n, int t, int j) {
    if (P.epi == EP_SWIGLU) {
        const int o = 8 * t + (j & 7);
        return o < n ? (j < 8 ? 0 : P.rows) + o0 + o : -1;
    }
    const int o = 16 * t + j;
    return o < n ? o0 + o : -1;
}
__device__ __forceinline__ int t_blocks(CPhase& P) { return (P.tcw + 3) >> 2; }
__device__ __forceinline__ int t_pairs(CPhase& P) { return P.ttiles * t_blocks(P) * 2048; }

// ---- prefetch of a region phase's data into one half of the wave's LDS region ----
// GEMV: the wave's first outputs (rows, then their scale/zero pairs; for the GDN in-projection the
// conv state and conv weights of those rows after them). GDN: the wave's 512-byte state column.
// Attention: the K/V rows of the wave's positions, through the block table.
__device__ __forceinline__ void prefetch(const Env& e, CPhase& P, CBufs& B, int step, uint8_t* __restrict__ nxt, int half) {
    const DecodeArgs& a = *e.a;
    const int lane = lane_here();
    if (P.kind == PH_GEMV && P.tiled) {
        int o0, n;
        t_outputs(P, e.wg, o0, n);
        const int T = P.ttiles, Cw = P.tcw, NB = t_blocks(P), c0 = e.wave * Cw;
        const uint8_t* W = (const uint8_t*)B.w;
        const uint8_t* SZ = (const uint8_t*)B.sz;
        for (int t = 0; t < T; t++) {
            // nibbles: per block of 4 chunks and group of 8 rows, lane l carries piece l / 8 of row l % 8
            for (int b = 0; b < NB; b++) {
                const int pc = 8 * b + (lane >> 3);  // piece of the wave's 32 Cw bytes of a row
#pragma unroll
                for (int g = 0; g < 2; g++) {
                    const int r = t_row(P, o0, n, t, 8 * g + (lane & 7));
                    if (pc < 2 * Cw && r >= 0)
                        lds_dma16<true>(W + (size_t)r * P.rb + 32 * c0 + 16 * pc, nxt + ((t * NB + b) * 2 + g) * 1024);
                }
            }
            // (scale, zero) pairs, four chunks per transfer: lane l carries chunk i0 + l / 16 of row l % 16
            const int r = t_row(P, o0, n, t, lane & 15);
            for (int i0 = 0; i0 < Cw; i0 += 4) {
                const int i = i0 + (lane >> 4);
                if (i < Cw && r >= 0)
                    lds_dma4<true>(SZ + (size_t)r * P.szb + 4 * ((64 * (c0 + i)) >> P.gshift),
                                   nxt + t_pairs(P) + (t * Cw + i0) * 64);
            }
        }
    } else if (P.kind == PH_GEMV) {
        const GemvGeo g = geo(P);
        const Rows R = part_p(P, e.gwm);
        const int cnt = min(R.n, g.cap);
        dma_rows(P, B, g, R.r0, cnt, 0, nxt, lane);
        const int ex = g.extra && R.n > g.cap ? 1 : 0;  // wave 0 only (rrem <= workgroups)
        if (ex) dma_extra(P, B, g, R.r0 + g.cap, s_extra, lane);
        if (P.epi == EP_CONV && cnt + ex > 0) {
            // conv state [ch][4] and weights [ch][4] of the prefetched rows, 16 bytes each
            uint8_t* cv = conv_area(half, e.wave);
            const int row = min(R.r0 + lane, P.conv_ch - 1);
            if (lane < cnt + ex) {
                lds_dma16<false>(B.conv + (size_t)row * 4, cv);
                lds_dma16<false>((const float*)B.aux + (size_t)row * 4, cv + 16 * kConvSlots);
            }
        }
    } else if (P.kind == PH_GDNF) {
        const int it = gf_item(P, e.wg), H = P.heads, h = it >> 4, cb = it & 15, t = cb * 8 + e.wave;
        const int nr = gf_nrows(cb, e.wave);
        const uint8_t* w = (const uint8_t*)B.w;
        for (int sl = 0; sl < nr; sl++) dma_bytes(w + (size_t)gf_row(H, h, t, e.wave, sl) * P.rb, P.rb, nxt + sl * P.rb, lane);
        // every slot's (scale, zero) row in one transfer: lane l carries 16 bytes of slot l / (szb / 16)
        const int per = P.szb >> 4;
        if (lane < nr * per) {
            const int sl = lane / per, part = lane - sl * per;
            lds_dma16<true>((const uint8_t*)B.sz + (size_t)gf_row(H, h, t, e.wave, sl) * P.szb + 16 * part,
                            nxt + kGfSlots * P.rb);
        }
        // conv state (lanes 0..2) and conv weights (lanes 3..5) of the q, k, v channels
        if (lane < 6) {
            const int sl = lane < 3 ? lane : lane - 3;
            const size_t ch = (size_t)gf_row(H, h, t, e.wave, sl) * 4;
            lds_dma16<false>(lane < 3 ? (const void*)(B.conv + ch) : (const void*)((const float*)B.aux + ch),
                             nxt + gf_conv(P));
        }
        const float* rec = ((CGdnX*)a.gdnx)[B.xi].rec;
        dma_bytes((const uint8_t*)(rec + ((size_t)h * kDK + t) * kDK), 512, nxt + gf_state(P), lane);
    } else if (P.kind == PH_GDN) {
        const int it = e.wg;
        const float* rec = (const float*)B.w;
        if (it < P.heads * 16) {
            const int h = it / 16, t = (it % 16) * 8 + e.wave;
            // state column t of head h: S[h][t][0..127] (value-major), 512 bytes
            dma_bytes((const uint8_t*)(rec + ((size_t)h * kDK + t) * kDK), 512, nxt, lane);
        }
    } else if (P.kind == PH_ATTN) {
        const int nkv = P.kv_heads, S = P.splits;
        if (e.wg < nkv * S) {
            const int g = e.wg / S, sp = e.wg % S;
            const uint32_t pos = a.pos0 + (uint32_t)step, len = pos + 1;
            const int p0 = split_at(sp, len, S), p1 = split_at(sp + 1, len, S);
            const int half = lane / 32, li = lane % 32;
            int bid[kAttnU];
#pragma unroll
            for (int u = 0; u < kAttnU; u++) {
                const int pp = p0 + 2 * (e.wave + kNW * u) + half;
                bid[u] = pp < p1 && pp < (int)pos ? a.block_table[pp / kBlk] : -1;
            }
#pragma unroll
            for (int u = 0; u < kAttnU; u++) {
                const int pp = p0 + 2 * (e.wave + kNW * u) + half;
                if (bid[u] >= 0) {
                    const size_t at = (((size_t)bid[u] * nkv + g) * kBlk + pp % kBlk) * kHeadDim + 8 * li;
                    lds_dma16<false>((const uint16_t*)B.w + at, nxt + u * 2048);
                    lds_dma16<false>((const uint16_t*)B.sz + at, nxt + u * 2048 + 1024);
                }
            }
        }
    }
}

// ---- phases ----

// Waits for the GEMV input vector and stages it in xs (times the RMSNorm gain); returns 1/rms (or 1).
__device__ __forceinline__ float gemv_input(const Env& e, CPhase& P, CBufs& B, int step, int p, const Ctl& c) {
    const DecodeArgs& a = *e.a;
    if (P.xin == XI_EMBED) return e.red[2 * kNW - 1];  // staged with the embedding row
    const uint32_t tag = tag_of(a, step, p - P.in_rel);
    const uint64_t* in = B.in + (size_t)(step & 1) * P.in_stride;
    float ss = 0.0f;
    float* xs = e.xs;
    const bool norm = P.xnorm == XN_NORM;
    const Step st = make_step(P);
    const bool cm = !head_fast(P) && !P.tiled;  // the LDS-region GEMV reads chunk-major slices
    // the RMSNorm gains of the pairs this thread will poll, loaded before the poll so that their
    // latency overlaps it (norm inputs fit one polling round: in_n <= 2 * kT * kPoll)
    float2 gn[kPoll];
    if (norm) {
#pragma unroll
        for (int j = 0; j < kPoll; j++) {
            const int q = j * kT + (int)threadIdx.x;
            gn[j] = 2 * q < P.in_n ? *(const float2*)(B.gain + 2 * q) : make_float2(1.0f, 1.0f);
        }
    }
    poll_pairs(in, P.in_cap, (P.in_n + 1) / 2, tag, [](int q) { return 2 * q; },
               [&](int q, float v0, float v1) {
                   if (norm) {
                       const int j = (q - (int)threadIdx.x) / kT;
                       float2 g = gn[0];
#pragma unroll
                       for (int jj = 1; jj < kPoll; jj++)
                           if (jj == j) g = gn[jj];
                       ss += v0 * v0 + v1 * v1;
                       v0 *= g.x;
                       v1 *= g.y;
                   }
                   const int d = cm ? xs_slot(st, 2 * q) : 2 * q;  // 2q even: 2q + 1 is the next slot
                   xs[d] = v0;
                   xs[d + 1] = v1;
               },
               c);
    if (norm) {
        ss = wave_sum_dpp(ss);
        if (e.lane == 0) e.red[e.wave] = ss;
    }
    bar();
    if (!norm) return 1.0f;
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kNW; w++) t += e.red[w];
    return 1.0f / sqrtf(t / (float)P.k + a.eps);
}

// LM head rows streamed straight into registers (the kernel's longest phase: vocab rows of width
// hidden). Two rows are computed while the next two load; the register file, not the LDS region,
// holds the bytes in flight.
template <int KIND, int K>
__device__ __forceinline__ void head_rows(const Env& e, CPhase& P, CBufs& B, WaveState& ws, float inv, const Rows& R,
                                          const float* __restrict__ xs) {
    const DecodeArgs& a = *e.a;
    const int lane = e.lane;
    float xr[K / 64];
    load_x<KIND, K>(xs, nullptr, 0.0f, xr, lane);
    float xsum[KIND == KIND_Q4 ? Q4Plan<K>::NS : 1];
    if constexpr (KIND == KIND_Q4) slab_sums<K>(xr, xsum);
    // Rows per group, two groups in flight per wave: ~48 registers of rows a group (f16 K = 2048:
    // 3 rows, 24 KiB in flight per wave). With 2 rows a group the head streamed at 0.78 of HBM,
    // waiting on load latency; 4 rows of K = 2048 spill.
    constexpr int kRowRegs = (int)(sizeof(RowRaw<KIND, K>) / 4);
    constexpr int NB = 48 / kRowRegs < 2 ? 2 : (48 / kRowRegs > 8 ? 8 : 48 / kRowRegs);
    RowRaw<KIND, K> cur[NB], nxt[NB];
#pragma unroll
    for (int k = 0; k < NB; k++) load_row<KIND, K, 64>(cur[k], B.w, (const uint32_t*)B.sz, R.r0 + min(k, R.n - 1), lane);
    for (int i = 0; i < R.n; i += NB) {
        if (i + NB < R.n) {
#pragma unroll
            for (int k = 0; k < NB; k++) load_row<KIND, K, 64>(nxt[k], B.w, (const uint32_t*)B.sz, R.r0 + min(i + NB + k, R.n - 1), lane);
        }
#pragma unroll
        for (int k = 0; k < NB; k++) {
            const float v = wave_sum_dpp(row_partial<KIND, K>(cur[k], xr, xsum)) * inv;
            const int o = R.r0 + i + k;
            if (i + k < R.n) {
                if (lane == 0) a.logits[o] = v;
                if (better(v, (uint32_t)o, ws.best, ws.best_i)) { ws.best = v; ws.best_i = (uint32_t)o; }
            }
        }
#pragma unroll
        for (int k = 0; k < NB; k++) cur[k] = nxt[k];
    }
}

__device__ __forceinline__ void head_phase(const Env& e, CPhase& P, CBufs& B, WaveState& ws, float inv) {
    const Rows R = part_p(P, e.gwm);
    if (R.n == 0) return;
    if (P.mkind == 0) {
        if (P.k == 512) head_rows<KIND_F16, 512>(e, P, B, ws, inv, R, e.xs);
        else if (P.k == 1024) head_rows<KIND_F16, 1024>(e, P, B, ws, inv, R, e.xs);
        else head_rows<KIND_F16, 2048>(e, P, B, ws, inv, R, e.xs);
    } else {
        if (P.k == 512) head_rows<KIND_Q4, 512>(e, P, B, ws, inv, R, e.xs);
        else if (P.k == 1024) head_rows<KIND_Q4, 1024>(e, P, B, ws, inv, R, e.xs);
        else head_rows<KIND_Q4, 2048>(e, P, B, ws, inv, R, e.xs);
    }
}

// One GEMV phase for this wave's outputs, rows read from `cur` (this phase's half). Output i sits
// in slot i % cap; the first min(n, cap) were prefetched (with more outputs than fit, slots are
// refilled as groups finish). Outputs are computed in groups of up to 8 rows (8 / nm outputs): for
// every step of x, the step's slice is read from LDS once and applied to the whole group, then the
// group is reduced together. The caller then sends the data of the region phase two ahead into `cur`.
__device__ __forceinline__ void gemv_body(const Env& e, CPhase& P, CBufs& B, int step, int p, WaveState& ws, float inv,
                                          uint8_t* cur, const float* xs, int half) {
    const DecodeArgs& a = *e.a;
    const int lane = e.lane;
    mark(e, 0);
    wait_all();  // this phase's rows (issued two region phases ago) are in
    const GemvGeo g = geo(P);
    const Rows R = part_p(P, e.gwm);
    if (R.n > 0) {
        const uint32_t tag = tag_of(a, step, p);
        uint64_t* out = B.out ? B.out + (size_t)(step & 1) * P.out_stride : nullptr;
        const Step t = make_step(P);
        const int gmax = 8 / g.nm;  // outputs per group
        const int ex = g.extra && R.n > g.cap ? 1 : 0;  // output cap in the workgroup's extra slot
        const int pre = min(R.n, g.cap + ex);  // outputs prefetched
        const bool stream = R.n > pre;
        const int go = stream ? max(1, min(gmax, g.cap / 2)) : min(gmax, R.n);
        const uint8_t* cvs = conv_area(half, e.wave);  // EP_CONV: conv state / weights of the prefetched rows
        const int xoff = (int)(s_extra - cur);  // the extra slot relative to this half
        int issued = pre;
        XC X;
        if (t.nsteps == 1) load_step(xs, t, 0, X, lane);
        asm volatile("" ::"v"(X.x[0]), "v"(X.x[31]));
        mark(e, 1);
        const int ns = g.nm - 1;  // log2(rows per output): 0 or 1 (SwiGLU)
        for (int o0 = 0; o0 < R.n; o0 += go) {
            const int ng = min(go, R.n - o0), nr = ng << ns;
            if (o0 + ng > pre) wait_vm((issued - o0 - ng) * g.per);  // refilled group
            // LDS offsets of the group's rows and their (scale, zero) rows (row r = row m of output i);
            // padding rows repeat row 0
            int roff[8], soff[8];
#pragma unroll
            for (int r = 0; r < 8; r++) {
                int slot = o0 + (r >> ns);
                if (stream) slot = slot < g.cap ? slot : slot % g.cap;
                if (ex && slot == g.cap) {
                    roff[r] = xoff + (r & ns) * g.rb;
                    soff[r] = xoff + g.nm * g.rb + (r & ns) * g.szb;
                } else {
                    roff[r] = lds_w(g, slot, r & ns);
                    soff[r] = lds_sz(g, slot, r & ns);
                }
            }
#pragma unroll
            for (int r = 1; r < 8; r++) {
                if (r >= nr) {
                    roff[r] = roff[0];
                    soff[r] = soff[0];
                }
            }
            float acc[8];
#pragma unroll
            for (int r = 0; r < 8; r++) acc[r] = 0.0f;
            if (nr == 1) rows_dot<1>(t, P.gshift, cur, roff, soff, xs, X, lane, acc);
            else if (nr == 2) rows_dot<2>(t, P.gshift, cur, roff, soff, xs, X, lane, acc);
            else if (nr <= 4) rows_dot<4>(t, P.gshift, cur, roff, soff, xs, X, lane, acc);
            else if (nr <= 6) rows_dot<6>(t, P.gshift, cur, roff, soff, xs, X, lane, acc);
            else rows_dot<8>(t, P.gshift, cur, roff, soff, xs, X, lane, acc);
            if (o0 == 0) {
                asm volatile("" ::"v"(acc[0]), "v"(acc[1]), "v"(acc[7]));
                mark(e, 2);
            }
            // refill the group's slots with the outputs cap further on
            for (int i = 0; i < ng && issued < R.n; i++, issued++) dma_rows(P, B, g, R.r0 + issued, 1, issued % g.cap, cur, lane);
            const float tot = reduce8(acc, lane) * inv;   // lanes 8r..8r+7: row r of the group
            const float up = __shfl_down(tot, 8, kWave);  // SwiGLU: the up row of the output
            const int r = lane >> 3;
            const int i = r >> ns;
            const bool lead = (lane & 7) == 0 && (r & ns) == 0 && i < ng;
            const int o = R.r0 + o0 + i;
            float y = tot;
            if (P.epi == EP_RESID) {
                // rows of h owned by this wave: outputs 0 and 1
                const float t0 = __shfl(tot, 0, kWave), t1 = __shfl(tot, 8 * g.nm, kWave);
                if (o0 == 0) {
                    ws.hown[0] += t0;
                    if (ng > 1) ws.hown[1] += t1;
                } else {
                    ws.hown[1] += t0;
                }
                y = i == 0 && o0 == 0 ? ws.hown[0] : ws.hown[1];
            }
            if (lead) {
                if (P.epi == EP_SWIGLU) y = silu(tot) * up;
                else if (P.epi == EP_CONV && o < P.conv_ch) {
                    // conv state s0..s2 and weights w0..w3 of the output's channel
                    const int k = o0 + i;
                    float4 st, cw;
                    if (k < pre) {
                        st = *(const float4*)(cvs + 16 * k);
                        cw = *(const float4*)(cvs + 16 * kConvSlots + 16 * k);
                    } else {
                        st = *(const float4*)(B.conv + (size_t)o * 4);
                        cw = *(const float4*)((const float*)B.aux + (size_t)o * 4);
                    }
                    const float cv = st.x * cw.x + st.y * cw.y + st.z * cw.z + tot * cw.w;
                    float* sp = B.conv + (size_t)o * 4;
                    sp[0] = st.y; sp[1] = st.z; sp[2] = tot;
                    y = silu(cv);
                }
                if (P.epi == EP_HEAD) {
                    a.logits[o] = y;
                    if (better(y, (uint32_t)o, ws.best, ws.best_i)) { ws.best = y; ws.best_i = (uint32_t)o; }
                } else {
                    put(out, (uint32_t)o, y, tag);
                }
            }
        }
        mark(e, 3);
    }
}

// The tiled q4 GEMV phase (the GEMV of kernels/src/shaders.rs:45-376 with the Store / Accumulate /
// SwiGlu epilogues) on v_mfma_i32_16x16x64_i8. x (staged in xs in column order, times the RMSNorm
// gain) becomes, per 64-column chunk and in place, a fixed-point vector X = rint(x * 2^(22 - e))
// (e: the chunk's exponent, so |X| < 2^22) held as three signed base-256 digits, X = d0 + 256 d1 +
// 65536 d2. Those digits are the MFMA's A rows 0..2, the tile's 16 rows of nibbles (q in 0..15 as
// int8) its B columns: D[d][row] = sum_k d_k q_k exactly, and per chunk and row
//   y += s * 2^(e - 22) * (D0 + 256 D1 + 65536 D2 - z * sum_k X_k)
// is sum_k s (q_k - z) x_k to within the quantisation of x (2^-23 of the chunk's largest value).
// Chunk layout after the conversion (256 bytes, was 64 floats): [k group 0..3][digit 0..2][16 bytes,
// columns in the order the nibble unpacking gives: 0 2 4 6 1 3 5 7 8 10 12 14 9 11 13 15], then
// sum X (int) at byte 192 and 2^(e - 22) (float) at 196.
// Each wave converts only the Cw chunks its own MFMAs read (chunks wave Cw .. + Cw - 1, four per
// pass: lanes 16 m .. 16 m + 15 take chunk 4 pass + m), so no workgroup barrier follows.
__device__ __forceinline__ void tiled_digits(const Env& e, CPhase& P) {
    float* xs = e.xs;
    const int Cw = P.tcw;
    const bool gdn = P.xnorm == XN_GDN;
    for (int base = 0; base < Cw; base += 4) {
        const int row = e.lane >> 4;
        if (base + row >= Cw) break;  // whole DPP rows (16 lanes per chunk)
        const int c = e.wave * Cw + base + row, i = e.lane & 15;
        // thread i takes the 4 columns whose digits form one word of the A layout: k group kq = i / 4,
        // columns 16 kq + {0, 2, 4, 6}, {1, 3, 5, 7}, {8, 10, 12, 14} or {9, 11, 13, 15} (sub = i % 4)
        const int kq = i >> 2, sub = i & 3, col = 64 * c + 16 * kq + 8 * (sub >> 1) + (sub & 1);
        float4 v;
        v.x = xs[col];
        v.y = xs[col + 2];
        v.z = xs[col + 4];
        v.w = xs[col + 6];
        if (gdn) {
            // GDN output norm (kernels/src/shaders.rs:514): the chunk lies in head (64 c) / 128, whose
            // 1/rms comes from the head's 16 published partial sums of squares (staged past K)
            const float4* ps = (const float4*)(xs + P.k + 16 * ((64 * c) / kDK));
            const float4 a0 = ps[0], a1 = ps[1], a2 = ps[2], a3 = ps[3];
            const float ssum = (((a0.x + a0.y) + (a0.z + a0.w)) + ((a1.x + a1.y) + (a1.z + a1.w))) +
                               (((a2.x + a2.y) + (a2.z + a2.w)) + ((a3.x + a3.y) + (a3.z + a3.w)));
            const float sc = 1.0f / sqrtf(ssum / (float)kDK + 1e-6f);
            v.x *= sc; v.y *= sc; v.z *= sc; v.w *= sc;
        }
        float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        // the chunk's 16 threads (a DPP row): every lane receives the maximum
        m = fmaxf(m, QNE_DPP(m, kDppXor1));
        m = fmaxf(m, QNE_DPP(m, kDppXor2));
        m = fmaxf(m, QNE_DPP(m, kDppHalfMirror));
        m = fmaxf(m, QNE_DPP(m, kDppMirror));
        int ex = 0;
        (void)frexpf(m, &ex);  // m < 2^ex (m = 0: ex = 0, every digit 0)
        const float f = ldexpf(1.0f, 22 - ex);
        const int x0 = (int)rintf(v.x * f), x1 = (int)rintf(v.y * f), x2 = (int)rintf(v.z * f), x3 = (int)rintf(v.w * f);
        int sx = (x0 + x1) + (x2 + x3);
        sx += __builtin_amdgcn_update_dpp(0, sx, kDppXor1, 0xF, 0xF, false);
        sx += __builtin_amdgcn_update_dpp(0, sx, kDppXor2, 0xF, 0xF, false);
        sx += __builtin_amdgcn_update_dpp(0, sx, kDppHalfMirror, 0xF, 0xF, false);
        sx += __builtin_amdgcn_update_dpp(0, sx, kDppMirror, 0xF, 0xF, false);
        // signed base-256 digits: the bytes of (X + 0x808080) ^ 0x808080
        const uint32_t z0 = (uint32_t)(x0 + 0x808080) ^ 0x808080u, z1 = (uint32_t)(x1 + 0x808080) ^ 0x808080u;
        const uint32_t z2 = (uint32_t)(x2 + 0x808080) ^ 0x808080u, z3 = (uint32_t)(x3 + 0x808080) ^ 0x808080u;
        cbar();  // every value of the chunk is read before its bytes are overwritten (one wave, in order)
        uint8_t* ch = (uint8_t*)(xs + 64 * c);
#pragma unroll
        for (int d = 0; d < 3; d++) {
            const uint32_t sh = 8 * d;
            *(uint32_t*)(ch + (kq * 3 + d) * 16 + 4 * sub) = ((z0 >> sh) & 0xFFu) | (((z1 >> sh) & 0xFFu) << 8) |
                                                             (((z2 >> sh) & 0xFFu) << 16) | (((z3 >> sh) & 0xFFu) << 24);
        }
        if (i == 0) {
            *(int*)(ch + 192) = sx;
            *(float*)(ch + 196) = ldexpf(1.0f, ex - 22);
        }
    }
}

__device__ __forceinline__ void tiled_body(const Env& e, CPhase& P, CBufs& B, int step, int p, float inv, uint8_t* cur) {
    const DecodeArgs& a = *e.a;
    const int lane = lane_here();
    mark(e, 0);
    wait_all();  // this wave's chunks (issued two region phases ago) are in
    tiled_digits(e, P);  // the wave's own chunks: its LDS writes precede its reads in order
    mark(e, 1);
    int o0, n;
    t_outputs(P, e.wg, o0, n);
    const int T = P.ttiles, Cw = P.tcw, j = lane & 15, kq = lane >> 4;
    const uint8_t* xb = (const uint8_t*)e.xs + 256 * (e.wave * Cw);  // the wave's first chunk
    const i32x4 zero = {0, 0, 0, 0};
    const int NB = t_blocks(P);
    static_assert(12 * 64 * kNW >= 6144, "the widest q4 GEMV: 12 chunks per wave");
    // B operand of lane (j, kq) for chunk i of tile t: row group j / 8, row j % 8, piece 2 (i % 4) + kq / 2
    const int boff = (j >> 3) * 1024 + (kq >> 1) * 128 + (j & 7) * 16 + 8 * (kq & 1);
    // Blocks of four chunks outside, tiles (T <= 4) inside: a block's x digits and exponents are
    // read once for every tile, and the tiles' loads and MFMAs are independent of each other. Each
    // tile still adds its blocks in block order, so the sums are those of a tile-by-tile loop.
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i0 = 0; i0 < Cw; i0 += 4) {
        i32x4 A[4];
        float sxf[4], xf[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = min(i0 + u, Cw - 1);
            const uint8_t* ch = xb + 256 * i;
            // A rows 3..15 are zero (their lanes read row 0 and drop it)
            const i32x4 a = *(const i32x4*)(ch + (kq * 3 + (j < 3 ? j : 0)) * 16);
            A[u] = j < 3 ? a : zero;
            const u32x2 hx = *(const u32x2*)(ch + 192);
            sxf[u] = (float)(int)hx.x;
            xf[u] = __uint_as_float(hx.y);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (t >= T) break;  // wave-uniform
            // the tile's four chunks of the block: every load issued before the first MFMA waits
            const uint8_t* blk = cur + (t * NB + (i0 >> 2)) * 2048 + boff;
            i32x4 Bv[4];
            uint32_t pr[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int i = min(i0 + u, Cw - 1);
                pr[u] = *(const uint32_t*)(cur + t_pairs(P) + ((t * Cw + i) * 16 + j) * 4);
                const u32x2 w = *(const u32x2*)(blk + 256 * (i - i0));
                Bv[u].x = (int)(w.x & 0x0F0F0F0Fu);
                Bv[u].y = (int)((w.x >> 4) & 0x0F0F0F0Fu);
                Bv[u].z = (int)(w.y & 0x0F0F0F0Fu);
                Bv[u].w = (int)((w.y >> 4) & 0x0F0F0F0Fu);
            }
            i32x4 D[4];
#pragma unroll
            for (int u = 0; u < 4; u++) D[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[u], Bv[u], zero, 0, 0, 0);
            // lanes 0..15: D[digit 0..2][row j] in D.x, D.y, D.z
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (i0 + u < Cw) {
                    const float comb = fmaf(65536.0f, (float)D[u].z, fmaf(256.0f, (float)D[u].y, (float)D[u].x));
                    acc[t] = fmaf(lo_h(pr[u]) * xf[u], comb - hi_h(pr[u]) * sxf[u], acc[t]);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < 4; t++)
        if (t < T && lane < 16) s_tsum[(e.wave * 4 + t) * 16 + lane] = acc[t];
    mark(e, 2);
    bar();
    // one thread per output: the waves' partials in wave order, then the epilogue
    const int o = (int)threadIdx.x;
    if (o < n) {
        const uint32_t tag = tag_of(a, step, p);
        uint64_t* out = B.out + (size_t)(step & 1) * P.out_stride;
        auto rowsum = [&](int slot) {
            float s = 0.0f;
            for (int w = 0; w < kNW; w++) s += s_tsum[(w * 4 + (slot >> 4)) * 16 + (slot & 15)];
            return s * inv;
        };
        float y;
        if (P.epi == EP_SWIGLU) {
            const int t = o >> 3, jj = o & 7;
            y = silu(rowsum(16 * t + jj)) * rowsum(16 * t + 8 + jj);
        } else {
            y = rowsum(o);
            if (P.epi == EP_RESID) {
                s_hres[o] += y;
                y = s_hres[o];
            }
        }
        put(out, (uint32_t)(o0 + o), y, tag);
    }
    mark(e, 3);
}

// The inputs of GDN item `it` (head h, value columns 8cb..8cb+7): q_h, k_h (64 pairs each), v and
// z of the 8 columns (4 pairs each), a_h and b_h; staged at xs[0..276).
__device__ __forceinline__ void gdn_input(const Env& e, CPhase& P, CBufs& B, int step, int p, int it, const Ctl& c) {
    const DecodeArgs& a = *e.a;
    const int H = P.heads, h = it / 16, cb = it % 16;
    const uint32_t tin = tag_of(a, step, p - P.in_rel);
    const uint64_t* in = B.in + (size_t)(step & 1) * P.in_stride;
    const int qa = h * kDK, ka = H * kDK + h * kDK, va = 2 * H * kDK + h * kDK + cb * 8;
    const int za = 3 * H * kDK + h * kDK + cb * 8, aa = 4 * H * kDK + h, ba = 4 * H * kDK + H + h;
    float* xs = e.xs;
    poll_pairs(in, P.in_cap, 138, tin,
               [&](int q) {
                   if (q < 64) return qa + 2 * q;
                   if (q < 128) return ka + 2 * (q - 64);
                   if (q < 132) return va + 2 * (q - 128);
                   if (q < 136) return za + 2 * (q - 132);
                   return q == 136 ? (aa & ~1) : (ba & ~1);
               },
               [&](int q, float v0, float v1) {
                   xs[2 * q] = v0;
                   xs[2 * q + 1] = v1;
               },
               c);
    bar();
}

// Gated DeltaNet step (kernels/src/shaders.rs:436-520 after the conv): workgroup = (head, 8 value
// columns), wave = one value column t, lane = keys 2l, 2l+1 of the value-major state column.
// The first item's inputs are staged by gdn_input and its state column is in `cur`.
__device__ __forceinline__ void gdn_body(const Env& e, CPhase& P, CBufs& B, int step, int p, const Ctl& c, const uint8_t* cur,
                                         const float* xs, float* red) {
    const DecodeArgs& a = *e.a;
    wait_all();  // the state column (issued two region phases ago) is in
    const int H = P.heads, lane = e.lane;
    const uint32_t tag = tag_of(a, step, p);
    uint64_t* out = B.out + (size_t)(step & 1) * P.out_stride;
    cfloat* prm = (cfloat*)B.gain;
    for (int it = e.wg; it < H * 16; it += e.nwg) {
        if (it != e.wg) {
            gdn_input(e, P, B, step, p, it, c);
            if (*e.bail) break;
        }
        const int h = it / 16, cb = it % 16;
        const int aa = 4 * H * kDK + h, ba = 4 * H * kDK + H + h;
        const int t = cb * 8 + e.wave;
        const float2 q2 = *(const float2*)(xs + 2 * lane);
        const float2 k2 = *(const float2*)(xs + 128 + 2 * lane);
        const float v = xs[256 + e.wave], z = xs[264 + e.wave];
        const float av = xs[272 + (aa & 1)], bv = xs[274 + (ba & 1)];
        float* Sg = (float*)B.w + ((size_t)h * kDK + t) * kDK + 2 * lane;
        const float2 s = it == e.wg ? *(const float2*)(cur + 8 * lane) : *(const float2*)Sg;
        const float nq = 1.0f / sqrtf(wave_sum_dpp(q2.x * q2.x + q2.y * q2.y) + 1e-6f) * rsqrtf((float)kDK);
        const float nk = 1.0f / sqrtf(wave_sum_dpp(k2.x * k2.x + k2.y * k2.y) + 1e-6f);
        const float qx = q2.x * nq, qy = q2.y * nq, kx = k2.x * nk, ky = k2.y * nk;
        const float kq = wave_sum_dpp(kx * qx + ky * qy);
        const float gg = expf(prm[H + h] * logf(1.0f + expf(av + prm[h])));
        const float beta = 1.0f / (1.0f + expf(-bv));
        const float sk = wave_sum_dpp(s.x * kx + s.y * ky);
        const float sq = wave_sum_dpp(s.x * qx + s.y * qy);
        const float d = beta * (v - gg * sk);
        float2 sn;
        sn.x = fmaf(gg, s.x, d * kx);
        sn.y = fmaf(gg, s.y, d * ky);
        *(float2*)Sg = sn;
        const float o = gg * sq + d * kq;
        if (lane == 0) {
            put(out, (uint32_t)(h * kDK + t), o * silu(z) * prm[2 * H + t], tag);
            red[e.wave] = o * o;
        }
        bar();
        if (threadIdx.x == 0) {
            float ss = 0.0f;
            for (int w = 0; w < kNW; w++) ss += red[w];
            put(out, (uint32_t)(H * kDK + h * 16 + cb), ss, tag);
        }
        bar();
    }
}

// The fused GDN phase (PH_GDNF): kernels/src/model.rs:233-241 for one GDN layer up to the mixer
// output, i.e. the in-projection GEMV (shaders.rs:45-376) with the causal conv + SiLU epilogue,
// then the gated delta rule step (shaders.rs:436-520). The input vector (1 / rms in `inv`) is staged
// in xs; the wave's projection rows, conv state and state column were prefetched into `cur`.
//  1. each wave dots its 4 (or 5) rows with x; q_t and k_t (and a / b) are published to the
//     head-group buffer, v_t and z_t stay in the wave;
//  2. the workgroup polls the head's 128 q, 128 k, a and b from the 16 workgroups of the head;
//  3. each wave steps value column t of the head's state and publishes o_t * silu(z_t) * norm_w[t];
//     the workgroup publishes the sum of its 8 o_t^2 (the out-projection folds the output norm).
__device__ __forceinline__ void gdnf_phase(const Env& e, CPhase& P, CBufs& B, int step, int p, float inv, uint8_t* cur,
                                           const Ctl& c) {
    const DecodeArgs& a = *e.a;
    const int lane = lane_here(), H = P.heads;
    mark(e, 0);
    wait_all();  // rows, conv and state column (issued two region phases ago) are in
    const int it = gf_item(P, e.wg), h = it >> 4, cb = it & 15, t = cb * 8 + e.wave;
    const int nr = gf_nrows(cb, e.wave);
    const uint32_t tag = tag_of(a, step, p);
    CGdnX& X = ((CGdnX*)a.gdnx)[B.xi];
    uint64_t* grp = X.grp + (size_t)(step & 1) * X.grp_stride;
    uint64_t* out = B.out + (size_t)(step & 1) * P.out_stride;
    // 1. the rows
    const Step st = make_step(P);
    XC xc;
    if (st.nsteps == 1) load_step(e.xs, st, 0, xc, lane);
    int roff[8], soff[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int sl = r < nr ? r : nr - 1;
        roff[r] = sl * P.rb;
        soff[r] = kGfSlots * P.rb + sl * P.szb;
    }
    float acc[8];
#pragma unroll
    for (int r = 0; r < 8; r++) acc[r] = 0.0f;
    if (nr == 5) rows_dot<5>(st, P.gshift, cur, roff, soff, e.xs, xc, lane, acc);
    else rows_dot<4>(st, P.gshift, cur, roff, soff, e.xs, xc, lane, acc);
    const float tot = reduce8(acc, lane) * inv;  // lanes 8r..8r+7: row r
    const int r = lane >> 3;
    float y = tot;
    if ((lane & 7) == 0 && r < 3) {
        // causal conv (kernel 4) + SiLU of the q / k / v channel (shaders.rs:457-468)
        const float4 sv = *(const float4*)(cur + gf_conv(P) + 16 * r);
        const float4 cw = *(const float4*)(cur + gf_conv(P) + 48 + 16 * r);
        const float cv = sv.x * cw.x + sv.y * cw.y + sv.z * cw.z + tot * cw.w;
        float* sp = B.conv + (size_t)gf_row(H, h, t, e.wave, r) * 4;
        sp[0] = sv.y;
        sp[1] = sv.z;
        sp[2] = tot;
        y = silu(cv);
    }
    if ((lane & 7) == 0) {
        if (r == 0) put(grp, (uint32_t)(h * 258 + t), y, tag);
        else if (r == 1) put(grp, (uint32_t)(h * 258 + 128 + t), y, tag);
        else if (r == 4 && r < nr) put(grp, (uint32_t)(h * 258 + 256 + e.wave), y, tag);
    }
    const float v = __shfl(y, 16, kWave), z = __shfl(y, 24, kWave);
    mark(e, 1);
    // 2. the head's q, k, a, b
    float* gs = e.xs + 4096;
    poll_pairs(grp, X.grp_stride, 129, tag, [&](int q) { return h * 258 + 2 * q; },
               [&](int q, float v0, float v1) {
                   gs[2 * q] = v0;
                   gs[2 * q + 1] = v1;
               },
               c);
    bar();
    if (*e.bail) return;
    mark(e, 2);
    // 3. the delta rule step of value column t (the same arithmetic as gdn_body)
    cfloat* prm = (cfloat*)X.prm;
    const float2 q2 = *(const float2*)(gs + 2 * lane);
    const float2 k2 = *(const float2*)(gs + 128 + 2 * lane);
    const float av = gs[256], bv = gs[257];
    const float2 sc = *(const float2*)(cur + gf_state(P) + 8 * lane);
    const float nq = 1.0f / sqrtf(wave_sum_dpp(q2.x * q2.x + q2.y * q2.y) + 1e-6f) * rsqrtf((float)kDK);
    const float nk = 1.0f / sqrtf(wave_sum_dpp(k2.x * k2.x + k2.y * k2.y) + 1e-6f);
    const float qx = q2.x * nq, qy = q2.y * nq, kx = k2.x * nk, ky = k2.y * nk;
    const float kq = wave_sum_dpp(kx * qx + ky * qy);
    const float gg = expf(prm[H + h] * logf(1.0f + expf(av + prm[h])));
    const float beta = 1.0f / (1.0f + expf(-bv));
    const float sk = wave_sum_dpp(sc.x * kx + sc.y * ky);
    const float sq = wave_sum_dpp(sc.x * qx + sc.y * qy);
    const float d = beta * (v - gg * sk);
    float2 sn;
    sn.x = fmaf(gg, sc.x, d * kx);
    sn.y = fmaf(gg, sc.y, d * ky);
    *(float2*)(X.rec + ((size_t)h * kDK + t) * kDK + 2 * lane) = sn;
    const float o = gg * sq + d * kq;
    if (lane == 0) {
        put(out, (uint32_t)(h * kDK + t), o * silu(z) * prm[2 * H + t], tag);
        e.red[e.wave] = o * o;
    }
    bar();
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (int w = 0; w < kNW; w++) ss += e.red[w];
        put(out, (uint32_t)(H * kDK + h * 16 + cb), ss, tag);
    }
    mark(e, 3);
}

// Combine of the attention partials (the merge of shaders.rs:522-633's split form): item = (q head
// h, 64 dims c); the S splits' (max, sum, acc) of the head, times sigmoid(gate). `part` holds the
// partials (tag tin), `gsrc` the in-projection output with the gate (tag tin2); the 64 outputs go to
// `out` with `tag`. Every thread of the workgroup takes part (polls end with barriers).
static_assert(66 * kMaxSplits + 64 + 64 * kNW + kNW <= kXs, "the combine's staging must fit in xs");
__device__ __forceinline__ void comb_core(const Env& e, int nq, int G, int S, int h, int cq, const uint64_t* part,
                                          uint32_t part_cap, uint32_t tin, const uint64_t* gsrc, uint32_t g_cap,
                                          uint32_t tin2, uint64_t* out, uint32_t tag, const Ctl& c) {
    const int g = h / G, gi = h % G;
    float* xs = e.xs;
    // xs: ml[2S] then acc[S][64] then gate[64]
    poll_pairs(part, part_cap, S * 33, tin,
               [&](int q) {
                   const int s = q / 33, j = q % 33;
                   const int base = ((g * S + s) * G + gi) * 258;
                   return j == 0 ? base : base + 2 + 64 * cq + 2 * (j - 1);
               },
               [&](int q, float v0, float v1) {
                   const int s = q / 33, j = q % 33;
                   const int d = j == 0 ? 2 * s : 2 * S + 64 * s + 2 * (j - 1);
                   xs[d] = v0;
                   xs[d + 1] = v1;
               },
               c);
    const int ga = nq * kHeadDim + h * kHeadDim + 64 * cq;
    poll_pairs(gsrc, g_cap, 32, tin2, [&](int q) { return ga + 2 * q; },
               [&](int q, float v0, float v1) {
                   xs[2 * S + 64 * S + 2 * q] = v0;
                   xs[2 * S + 64 * S + 2 * q + 1] = v1;
               },
               c);
    bar();
    if (*e.bail) return;
    {
        // wave sg takes splits sg, sg + 8, ...; lane = dim. Their sums meet in xs after the gate.
        const int d = threadIdx.x & 63, sg = threadIdx.x >> 6;
        // every wave finds the maximum over the splits with its lanes (one split each), in parallel
        float mm = -INFINITY;
        for (int s = d; s < S; s += kWave) mm = fmaxf(mm, xs[2 * s]);
        const float mn = wave_max(mm);
        float ls = 0.0f, ac = 0.0f;
        for (int s = sg; s < S; s += kNW) {
            const float ms = xs[2 * s];
            if (ms == -INFINITY) continue;
            const float cw = exp2_hw(ms - mn);  // the partials' maxima and sums are in base 2
            ls += xs[2 * s + 1] * cw;
            ac += xs[2 * S + 64 * s + d] * cw;
        }
        float* rd = xs + 2 * S + 64 * S + 64;  // [kNW][64] sums of acc, then [kNW] sums of l
        rd[64 * sg + d] = ac;
        if (d == 0) rd[64 * kNW + sg] = ls;
        bar();
        if (threadIdx.x < 64) {
            float at = 0.0f, lt = 0.0f;
#pragma unroll
            for (int w = 0; w < kNW; w++) {
                at += rd[64 * w + d];
                lt += rd[64 * kNW + w];
            }
            const float gate = xs[2 * S + 64 * S + d];
            put(out, (uint32_t)(h * kHeadDim + 64 * cq + d), at / lt / (1.0f + expf(-gate)), tag);
        }
    }
    bar();
}

// RMSNorm (weight w) + rotate-half RoPE of one 256-vector held 4 values per lane
// (kernels/src/shaders.rs:575-593). rope = {cos[64], sin[64]} of the step's angles.
__device__ __forceinline__ void norm_rope4(float (&v)[4], const float* w, const DecodeArgs& a, const float* rope,
                                           int) {
    const int lane = lane_here();
    float ss = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
    ss = wave_sum_dpp(ss);
    const float inv = 1.0f / sqrtf(ss / (float)kHeadDim + 1e-6f);
    const float4 g = *(const float4*)(w + 4 * lane);
    v[0] = v[0] * inv * g.x; v[1] = v[1] * inv * g.y; v[2] = v[2] * inv * g.z; v[3] = v[3] * inv * g.w;
    const int half = a.rope_dim / 2, partner = half / 4;
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = 4 * lane + i;
        const float other_lo = __shfl_down(v[i], partner, kWave);  // value at d + half
        const float other_hi = __shfl_up(v[i], partner, kWave);    // value at d - half
        o[i] = v[i];
        if (d < a.rope_dim) {
            const int fi = d < half ? d : d - half;
            const float cs = rope[fi], sn = rope[64 + fi];
            o[i] = d < half ? v[i] * cs - other_lo * sn : v[i] * cs + other_hi * sn;
        }
    }
    v[0] = o[0]; v[1] = o[1]; v[2] = o[2]; v[3] = o[3];
}

// Attention partials (kernels/src/shaders.rs:522-633 split over the context): workgroup =
// (kv head g, split sp) over positions [p0, p1) of 0..pos; publishes (max, sum, acc[256]) per
// q head of the group. The K/V rows prefetched into half `rh` are read from it and the waves'
// partials merged through it.
__device__ __forceinline__ void attn_phase(const Env& e, CPhase& P, CBufs& B, int step, int p, const Ctl& c, int rh,
                                           const float* rope) {
    uint8_t* cur = e.regs + e.wave * kWaveLds + rh * kHalf;
    const DecodeArgs& a = *e.a;
    const int nq = P.heads, nkv = P.kv_heads, G = nq / nkv, S = P.splits, lane = e.lane;
    if (e.wg >= nkv * S) return;
    mark(e, 0);
    const int g = e.wg / S, sp = e.wg % S;
    const uint32_t pos = a.pos0 + (uint32_t)step, len = pos + 1;
    const int p0 = split_at(sp, len, S), p1 = split_at(sp + 1, len, S);
    const uint32_t tin = tag_of(a, step, p - P.in_rel), tag = tag_of(a, step, p);
    const uint64_t* in = B.in + (size_t)(step & 1) * P.in_stride;
    // the partials: this phase's output, or with the combine folded in, the phase's own exchange
    // buffer (B.aux) and the combined vector its output
    uint64_t* out = P.fold ? (uint64_t*)B.aux + (size_t)(step & 1) * P.part_stride : B.out + (size_t)(step & 1) * P.out_stride;
    uint16_t* kp = (uint16_t*)B.w;
    uint16_t* vp = (uint16_t*)B.sz;
    float* xs = e.xs;
    // q of the group's heads -> xs[0, G*256), k -> xs[1024, 1280), v -> xs[1280, 1536)
    const int qa = g * G * kHeadDim, ka = 2 * nq * kHeadDim + g * kHeadDim, va = ka + nkv * kHeadDim;
    const int nqp = G * kHeadDim / 2;
    poll_pairs(in, P.in_cap, nqp + 256, tin,
               [&](int q) { return q < nqp ? qa + 2 * q : (q < nqp + 128 ? ka + 2 * (q - nqp) : va + 2 * (q - nqp - 128)); },
               [&](int q, float v0, float v1) {
                   const int d = q < nqp ? 2 * q : 1024 + 2 * (q - nqp);
                   xs[d] = v0;
                   xs[d + 1] = v1;
               },
               c);
    bar();
    if (*e.bail) return;
    mark(e, 1);
    float* qs = xs + 1536;  // [G][256], normed, rotated, pre-scaled by log2(e) / sqrt(256)
    float* kc = xs + 2560;  // current key and value, f16-rounded
    float* vc = xs + 2816;
    if (e.wave < G) {
        float v[4];
        const float4 f = *(const float4*)(xs + e.wave * kHeadDim + 4 * lane);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        norm_rope4(v, B.gain, a, rope, lane);
#pragma unroll
        for (int i = 0; i < 4; i++) qs[e.wave * kHeadDim + 4 * lane + i] = v[i] * kScoreScale;
    } else if (e.wave == G) {
        float v[4];
        const float4 f = *(const float4*)(xs + 1024 + 4 * lane);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        norm_rope4(v, B.gain + kHeadDim, a, rope, lane);
        const float4 vv = *(const float4*)(xs + 1280 + 4 * lane);
        const float val[4] = {vv.x, vv.y, vv.z, vv.w};
        uint16_t kh[4], vh[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kh[i] = f2h(v[i]);
            vh[i] = f2h(val[i]);
            kc[4 * lane + i] = h2f(kh[i]);
            vc[4 * lane + i] = h2f(vh[i]);
        }
        if (sp == S - 1) {
            // append at pos: two lanes' 8-byte halves form one 16-byte agent-scope store
            const size_t at = (((size_t)a.block_table[pos / kBlk] * nkv + g) * kBlk + pos % kBlk) * kHeadDim;
            const uint32_t k01 = (uint32_t)kh[0] | ((uint32_t)kh[1] << 16), k23 = (uint32_t)kh[2] | ((uint32_t)kh[3] << 16);
            const uint32_t v01 = (uint32_t)vh[0] | ((uint32_t)vh[1] << 16), v23 = (uint32_t)vh[2] | ((uint32_t)vh[3] << 16);
            const uint32_t nk01 = __shfl_down(k01, 1, kWave), nk23 = __shfl_down(k23, 1, kWave);
            const uint32_t nv01 = __shfl_down(v01, 1, kWave), nv23 = __shfl_down(v23, 1, kWave);
            if ((lane & 1) == 0) {
                u32x4 kw, vw;
                kw.x = k01; kw.y = k23; kw.z = nk01; kw.w = nk23;
                vw.x = v01; vw.y = v23; vw.z = nv01; vw.w = nv23;
                st16_agent(kp + at, 8 * lane, kw);
                st16_agent(vp + at, 8 * lane, vw);
            }
        }
    }
    bar();
    mark(e, 2);
    // wave: positions p0 + 2*(wave + 8u) + half; 32 lanes per position, 8 dims per lane
    const int half = lane / 32, li = lane % 32;
    float qr[4][8], acc[4][8], m[4], l[4];
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
        m[gi] = -INFINITY;
        l[gi] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; d++) {
            qr[gi][d] = gi < G ? qs[gi * kHeadDim + 8 * li + d] : 0.0f;
            acc[gi][d] = 0.0f;
        }
    }
    wait_all();  // prefetched K/V rows
    mark(e, 3);
    for (int u = 0;; u++) {
        const int pp = p0 + 2 * (e.wave + kNW * u);
        if (pp >= p1) break;  // wave-uniform
        const int ps = pp + half;
        const bool valid = ps < p1;
        float kf[8], vf[8];
        if (ps == (int)pos) {
#pragma unroll
            for (int d = 0; d < 8; d++) { kf[d] = kc[8 * li + d]; vf[d] = vc[8 * li + d]; }
        } else if (valid) {
            u32x4 kw, vw;
            if (u < kAttnU) {
                kw = *(const u32x4*)(cur + u * 2048 + 16 * lane);
                vw = *(const u32x4*)(cur + u * 2048 + 1024 + 16 * lane);
            } else {
                const size_t at = (((size_t)a.block_table[ps / kBlk] * nkv + g) * kBlk + ps % kBlk) * kHeadDim + 8 * li;
                kw = *(const u32x4*)(kp + at);
                vw = *(const u32x4*)(vp + at);
            }
            kf[0] = lo_h(kw.x); kf[1] = hi_h(kw.x); kf[2] = lo_h(kw.y); kf[3] = hi_h(kw.y);
            kf[4] = lo_h(kw.z); kf[5] = hi_h(kw.z); kf[6] = lo_h(kw.w); kf[7] = hi_h(kw.w);
            vf[0] = lo_h(vw.x); vf[1] = hi_h(vw.x); vf[2] = lo_h(vw.y); vf[3] = hi_h(vw.y);
            vf[4] = lo_h(vw.z); vf[5] = hi_h(vw.z); vf[6] = lo_h(vw.w); vf[7] = hi_h(vw.w);
        } else {
#pragma unroll
            for (int d = 0; d < 8; d++) { kf[d] = 0.0f; vf[d] = 0.0f; }
        }
#pragma unroll
        for (int gi = 0; gi < 4; gi++) {
            if (gi < G) {
                float s = 0.0f;
#pragma unroll
                for (int d = 0; d < 8; d++) s = fmaf(qr[gi][d], kf[d], s);
                s = half_sum_dpp(s, lane);  // the position's 32 lanes
                if (valid) {
                    const float mn = fmaxf(m[gi], s);
                    const float corr = exp2_hw(m[gi] - mn), pw = exp2_hw(s - mn);
                    m[gi] = mn;
                    l[gi] = l[gi] * corr + pw;
#pragma unroll
                    for (int d = 0; d < 8; d++) acc[gi][d] = fmaf(pw, vf[d], acc[gi][d] * corr);
                }
            }
        }
    }
    mark(e, 4);
    // merge the two position halves of the wave, then write the wave's partial into its region
    float* wp = (float*)cur;  // [G][258]: m, l, acc[256]
#pragma unroll
    for (int gi = 0; gi < 4; gi++) {
        if (gi < G) {
            const float mo = __shfl_xor(m[gi], 32, kWave), lo = __shfl_xor(l[gi], 32, kWave);
            const float mn = fmaxf(m[gi], mo);
            const float ca = mn == -INFINITY ? 0.0f : exp2_hw(m[gi] - mn), cb = mn == -INFINITY ? 0.0f : exp2_hw(mo - mn);
#pragma unroll
            for (int d = 0; d < 8; d++) acc[gi][d] = acc[gi][d] * ca + __shfl_xor(acc[gi][d], 32, kWave) * cb;
            l[gi] = l[gi] * ca + lo * cb;
            m[gi] = mn;
            if (half == 0) {
#pragma unroll
                for (int d = 0; d < 8; d++) wp[gi * 258 + 2 + 8 * li + d] = acc[gi][d];
                if (li == 0) { wp[gi * 258] = m[gi]; wp[gi * 258 + 1] = l[gi]; }
            }
        }
    }
    bar();
    // merge the 8 waves: thread = (head gi, dims d0, d0 + 1)
    {
        const int gi = threadIdx.x >> 7, d0 = 2 * (threadIdx.x & 127);
        if (gi < G) {
            float mw[kNW], mn = -INFINITY;
#pragma unroll
            for (int w = 0; w < kNW; w++) {
                mw[w] = ((const float*)(e.regs + w * kWaveLds + rh * kHalf))[gi * 258];
                mn = fmaxf(mn, mw[w]);
            }
            float ls = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int w = 0; w < kNW; w++) {
                const float* pw = (const float*)(e.regs + w * kWaveLds + rh * kHalf) + gi * 258;
                const float cw = mw[w] == -INFINITY ? 0.0f : exp2_hw(mw[w] - mn);
                ls += pw[1] * cw;
                a0 += pw[2 + d0] * cw;
                a1 += pw[3 + d0] * cw;
            }
            const uint32_t base = (uint32_t)(((g * S + sp) * G + gi) * 258);
            put(out, base + 2 + d0, a0, tag);
            put(out, base + 3 + d0, a1, tag);
            if (d0 == 0) {
                put(out, base, mn, tag);
                put(out, base + 1, ls, tag);
            }
        }
    }
    bar();  // the regions are free again
    if (P.fold) {
        // the combine, folded in: workgroup (g, sp) with sp < 4 G merges q head g G + sp / 4, dims
        // 64 (sp % 4) .. + 63 over the group's S splits (an exchange among the group's workgroups)
        if (sp < 4 * G)
            comb_core(e, nq, G, S, g * G + sp / 4, sp % 4, out, P.part_stride, tag, in, P.in_cap, tin,
                      B.out + (size_t)(step & 1) * P.out_stride, tag, c);
    }
    mark(e, 5);
}

// The combine as a phase of its own (PH_COMB): workgroup = (q head h, 64 dims c).
__device__ __forceinline__ void comb_phase(const Env& e, CPhase& P, CBufs& B, int step, int p, const Ctl& c) {
    const DecodeArgs& a = *e.a;
    const int nq = P.heads, nkv = P.kv_heads, G = nq / nkv, S = P.splits;
    if (e.wg >= nq * 4) return;
    mark(e, 0);
    const uint32_t tin = tag_of(a, step, p - P.in_rel), tin2 = tag_of(a, step, p - P.in2_rel), tag = tag_of(a, step, p);
    const uint64_t* in = B.in + (size_t)(step & 1) * P.in_stride;
    const uint64_t* in2 = (const uint64_t*)B.aux + (size_t)(step & 1) * P.in2_stride;
    uint64_t* out = B.out + (size_t)(step & 1) * P.out_stride;
    mark(e, 1);
    comb_core(e, nq, G, S, e.wg / 4, e.wg % 4, in, P.in_cap, tin, in2, P.in2_cap, tin2, out, tag, c);
    mark(e, 2);
    mark(e, 3);
}

__device__ __forceinline__ float embed_val(const DecodeArgs& a, uint32_t tok, int c) {
    if (a.emb_kind == 0) return h2f(((const uint16_t*)a.emb_w)[(size_t)tok * a.hidden + c]);
    const uint32_t word = ((const uint32_t*)a.emb_w)[(size_t)tok * (a.hidden / 8) + c / 8];
    const uint32_t sz = a.emb_sz[(size_t)tok * (a.hidden / a.emb_group) + c / a.emb_group];
    return ((float)((word >> (4 * (c % 8))) & 15u) - hi_h(sz)) * lo_h(sz);
}

__device__ __forceinline__ void trace_done(const Env& e, int inst) {
    const DecodeArgs& a = *e.a;
    if (a.trace && inst < a.trace_cap) {
        bar();
        if (threadIdx.x == 0) a.trace[2 + 2 * ((size_t)inst * e.nwg + e.wg) + 1] = __builtin_amdgcn_s_memrealtime();
    }
}
__device__ __forceinline__ void trace_in(const Env& e, int inst) {
    const DecodeArgs& a = *e.a;
    if (a.trace && inst < a.trace_cap && threadIdx.x == 0)
        a.trace[2 + 2 * ((size_t)inst * e.nwg + e.wg)] = __builtin_amdgcn_s_memrealtime();
}

}  // namespace

// The program body; instantiated by the two kernels below so that profiles tell prompt-token runs
// from greedy decode windows.
__device__ __forceinline__ void decode_program(const DecodeArgs& a) {
    __shared__ __attribute__((aligned(16))) float xs[kXs];
    __shared__ __attribute__((aligned(16))) uint8_t regs[kNW * kWaveLds];
    __shared__ float red[2 * kNW];
    __shared__ uint32_t redi[kNW];
    __shared__ float rope[2 * 64];  // cos, sin of the step's RoPE angles
    __shared__ int bail;
    Env e;
    e.a = &a;
    e.wg = blockIdx.x;
    e.nwg = gridDim.x;
    // the same in every lane of a wave: readfirstlane lets the compiler keep it (and the row
    // ranges derived from it) in scalar registers, with scalar loop control
    e.wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    e.lane = threadIdx.x % kWave;
    e.gwm = e.wave * e.nwg + e.wg;
    e.nw = e.nwg * kNW;
    e.xs = xs;
    e.regs = regs;
    e.red = red;
    e.bail = &bail;
    // profiling: thread 0's sub-step timestamps of the running phase (LDS, so that no register
    // holds them for the whole launch)
    __shared__ unsigned long long tts[8];
    e.tt = tts;
    // profiling: the workgroup's place, (XCC_ID << 32 | HW_ID) + 1, kept in sub-step slot 6
    unsigned long long where = 0;
    if (a.sub) {
        unsigned xcc, hw;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
        where = (((unsigned long long)xcc << 32) | hw) + 1ull;
    }
    Ctl c{a.err, a.spin_limit, &bail};
    CBufs* prog = (CBufs*)a.prog;
    CPhase* shapes = (CPhase*)a.shapes;
    if (threadIdx.x == 0) bail = 0;
    if (a.trace && e.wg == 0 && threadIdx.x == 0) a.trace[0] = __builtin_amdgcn_s_memrealtime();
    WaveState ws;
    ws.hown[0] = ws.hown[1] = 0.0f;
    ws.best = -INFINITY;
    ws.best_i = 0xFFFFFFFFu;
    const Rows own = part(a.hidden, e.gwm, e.nw);  // residual rows of this wave (<= 2)
    auto region = [&](int half) { return regs + e.wave * kWaveLds + half * kHalf; };
    bar();

    uint32_t token = a.feed ? a.tok[0] : a.ids[0];
    // ids appended so far (tok[2]); only workgroup 0's thread 0 writes it during a launch, so it
    // is read once, here, before any prefetch: a load at the end of each step would complete only
    // behind that wave's prefetch of the next step, and the workgroup would start every step late
    uint32_t n_out = a.out_ids && e.wg == 0 && threadIdx.x == 0 ? a.tok[2] : 0u;
    int half = 0;  // half of the next region phase (region phases alternate between the halves)
    // the window's first two region phases (each region phase sends the one two ahead)
    prefetch(e, shapes[prog[a.reg0].shape], prog[a.reg0], 0, region(0), 0);
    prefetch(e, shapes[prog[a.reg1].shape], prog[a.reg1], 0, region(1), 1);
    for (int step = 0; step < a.n_steps; step++) {
        const uint32_t pos = a.pos0 + (uint32_t)step;
        const bool head = head_at(a, step);
        // embedding row (kernels/src/shaders.rs:405-434) times the first layer's input-norm gain,
        // in the layout the first in-projection reads; 1/rms in red[2 kNW - 1]
        {
            CPhase& P0 = shapes[prog[0].shape];
            const Step st0 = make_step(P0);
            if ((int)threadIdx.x < a.rope_dim / 2) {
                float sn, cs;
                sincosf((float)pos * a.inv_freq[threadIdx.x], &sn, &cs);
                rope[threadIdx.x] = cs;
                rope[64 + threadIdx.x] = sn;
            }
            float ss = 0.0f;
            for (int cc = threadIdx.x; cc < a.hidden; cc += kT) {
                const float v = embed_val(a, token, cc);
                xs[xs_slot(st0, cc)] = v * prog[0].gain[cc];
                ss += v * v;
            }
            ss = wave_sum_dpp(ss);
            if (e.lane == 0) red[e.wave] = ss;
            if (a.h_tiled) {
                // the residual rows this workgroup's tiled GEMVs own (their outputs of a hidden-wide phase)
                const int per = a.hidden / e.nwg, rem = a.hidden % e.nwg;
                const int r0 = e.wg * per + min(e.wg, rem), rn = per + (e.wg < rem ? 1 : 0);
                if ((int)threadIdx.x < rn) s_hres[threadIdx.x] = embed_val(a, token, r0 + (int)threadIdx.x);
            } else {
                if (own.n > 0) ws.hown[0] = embed_val(a, token, own.r0);
                if (own.n > 1) ws.hown[1] = embed_val(a, token, own.r0 + 1);
            }
            bar();
            if (threadIdx.x == 0) {
                float t = 0.0f;
                for (int w = 0; w < kNW; w++) t += red[w];
                red[2 * kNW - 1] = 1.0f / sqrtf(t / (float)a.hidden + a.eps);
            }
            bar();
        }
        ws.best = -INFINITY;
        ws.best_i = 0xFFFFFFFFu;
        for (int p = 0; p < a.nph; p++) {
            CBufs& B = prog[p];
            CPhase& P = shapes[B.shape];
            if (P.is_head && !head) continue;
            const int inst = step * a.nph + p;
            const int rh = half;
            if (a.sub) {
                if (threadIdx.x == 0) {
                    for (int k = 0; k < 8; k++) tts[k] = 0;
                    tts[6] = where;  // not a timestamp: where this workgroup runs
                }
            }
            switch (P.kind) {
                case PH_GEMV: {
                    const float inv = gemv_input(e, P, B, step, p, c);
                    if (bail) { wait_all(); return; }
                    trace_in(e, inst);
                    if (head_fast(P)) {
                        head_phase(e, P, B, ws, inv);
                    } else if (P.tiled) {
                        tiled_body(e, P, B, step, p, inv, region(rh));
                    } else {
                        gemv_body(e, P, B, step, p, ws, inv, region(rh), xs, rh);
                    }
                    break;
                }
                case PH_GDN:
                    mark(e, 0);
                    if (e.wg < P.heads * 16) gdn_input(e, P, B, step, p, e.wg, c);
                    mark(e, 1);
                    if (bail) { wait_all(); return; }
                    trace_in(e, inst);
                    gdn_body(e, P, B, step, p, c, region(rh), xs, red);
                    mark(e, 2);
                    break;
                case PH_GDNF: {
                    const float inv = gemv_input(e, P, B, step, p, c);
                    if (bail) { wait_all(); return; }
                    trace_in(e, inst);
                    gdnf_phase(e, P, B, step, p, inv, region(rh), c);
                    break;
                }
                case PH_ATTN:
                    trace_in(e, inst);
                    attn_phase(e, P, B, step, p, c, rh, rope);
                    break;
                default:
                    trace_in(e, inst);
                    comb_phase(e, P, B, step, p, c);
                    break;
            }
            if (bail) { wait_all(); return; }
            if (uses_region(P)) {
                // this phase's LDS reads are done: send the data of the region phase two ahead
                // into its half (the next region phase's data is in the other half)
                int ns = 0, np = 0;
                if (region_after(a, P, step, p, 2, ns, np)) prefetch(e, shapes[prog[np].shape], prog[np], ns, region(rh), rh);
                mark(e, 7);
                half ^= 1;
            }
            if (a.sub && threadIdx.x == 0 && inst < a.trace_cap) {
#pragma unroll
                for (int k = 0; k < 8; k++) a.sub[8 * ((size_t)inst * e.nwg + e.wg) + k] = tts[k];
            }
            // Every wave is done with xs and red before any wave stages the next phase's input
            // there: a wave can receive that input (published by other workgroups) while a slower
            // wave of its workgroup still reads this phase's.
            bar();
            trace_done(e, inst);
        }
        if (head && a.argmax) {
            // greedy pick over the LM head rows (argmax_partial / argmax_final,
            // kernels/src/shaders.rs:635-699): lanes -> waves -> workgroup -> every workgroup
#pragma unroll
            for (int mk = 32; mk >= 1; mk >>= 1) {
                const float ov = __shfl_xor(ws.best, mk, kWave);
                const uint32_t oi = (uint32_t)__shfl_xor((int)ws.best_i, mk, kWave);
                if (better(ov, oi, ws.best, ws.best_i)) { ws.best = ov; ws.best_i = oi; }
            }
            if (e.lane == 0) { red[e.wave] = ws.best; redi[e.wave] = ws.best_i; }
            bar();
            const uint32_t tag = tag_of(a, step, a.nph - 1);
            uint64_t* am = a.am + (size_t)(step & 1) * a.am_stride;
            if (threadIdx.x == 0) {
                float b = red[0];
                uint32_t bi = redi[0];
                for (int w = 1; w < kNW; w++)
                    if (better(red[w], redi[w], b, bi)) { b = red[w]; bi = redi[w]; }
                put(am, 2 * e.wg, b, tag);
                put(am, 2 * e.wg + 1, __uint_as_float(bi), tag);
            }
            float b = -INFINITY;
            uint32_t bi = 0xFFFFFFFFu;
            poll_pairs(am, 2 * e.nwg, e.nwg, tag, [](int q) { return 2 * q; },
                       [&](int q, float v0, float v1) {
                           const uint32_t i1 = __float_as_uint(v1);
                           if (better(v0, i1, b, bi)) { b = v0; bi = i1; }
                       },
                       c);
#pragma unroll
            for (int mk = 32; mk >= 1; mk >>= 1) {
                const float ov = __shfl_xor(b, mk, kWave);
                const uint32_t oi = (uint32_t)__shfl_xor((int)bi, mk, kWave);
                if (better(ov, oi, b, bi)) { b = ov; bi = oi; }
            }
            bar();
            if (e.lane == 0) { red[e.wave] = b; redi[e.wave] = bi; }
            bar();
            if (bail) { wait_all(); return; }
            float bb = red[0];
            uint32_t bbi = redi[0];
            for (int w = 1; w < kNW; w++)
                if (better(red[w], redi[w], bb, bbi)) { bb = red[w]; bbi = redi[w]; }
            const uint32_t pick = bbi == 0xFFFFFFFFu ? 0u : bbi;
            if (e.wg == 0 && threadIdx.x == 0) {
                a.tok[0] = pick;
                a.tok[1] = pos + 1;
                if (a.out_ids) {
                    if (n_out < a.out_cap) a.out_ids[n_out] = pick;
                    a.tok[2] = ++n_out;
                }
            }
            token = pick;
            bar();
        }
        if (step + 1 < a.n_steps && !a.feed) token = a.ids[step + 1];
    }
    wait_all();
    if (a.trace && e.wg == 0 && threadIdx.x == 0) a.trace[1] = __builtin_amdgcn_s_memrealtime();
}

// Greedy decode windows and single steps (feed 1).
__global__ __launch_bounds__(kT, 1) void k_decode(DecodeArgs a) { decode_program(a); }
// Prompt tokens taken from `ids` (feed 0): prefill and prefill_chunk.
__global__ __launch_bounds__(kT, 1) void k_prefill_tokens(DecodeArgs a) { decode_program(a); }

int decode_gemv_variant(int kind, int k) {
    if (k <= 0 || k % 512 != 0) return -1;
    if (kind == 1) return k <= 6144 ? 1 : -1;  // a q4 row of 6144 is 3456 bytes of LDS
    return k <= 4096 ? 0 : -1;                 // an f16 row of 4096 fills an 8 KiB half
}

void finalize_phase(Phase& P, int grid) {
    const int nw = grid * kNW;
    if (P.kind == PH_GEMV || P.kind == PH_GDNF) {
        P.fast_head = P.epi == EP_HEAD && (P.mkind == 0 || P.group == 64) && (P.k == 512 || P.k == 1024 || P.k == 2048);
        P.rper = P.rows / nw;
        P.rrem = P.rows % nw;
        P.rb = P.mkind ? P.k / 2 : P.k * 2;
        P.szb = P.mkind ? (P.k / P.group) * 4 : 0;
        P.stride = P.rb + P.szb;
        P.nm = P.epi == EP_SWIGLU ? 2 : 1;
        P.convb = P.epi == EP_CONV ? 32 : 0;  // in the wave's conv area, outside the half
        P.cap = kHalf / (P.stride * P.nm);
        if (P.epi == EP_CONV) P.cap = std::min(P.cap, kConvSlots);
        // one output past cap on wave 0 only: the workgroup's extra slot (the program pass that
        // keeps consecutive region phases from both using it may clear this)
        P.extra = P.kind == PH_GEMV && !P.tiled && !P.fast_head && !P.is_head && P.rrem > 0 && P.rper == P.cap &&
                  P.rrem <= grid && P.stride * P.nm <= kExtraBytes && (P.epi != EP_CONV || P.cap + 1 <= kConvSlots);
        P.dper = P.nm * ((P.rb + 1023) / 1024 + (P.szb + 1023) / 1024);
        int gs = 0;
        while (P.mkind && (1 << gs) < P.group) gs++;
        P.gshift = gs;
        P.n4 = P.k / 2048;
        P.n2 = (P.k % 2048) / 1024;
        P.n1 = (P.k % 1024) / 512;
        P.nsteps = P.mkind ? P.n4 + P.n2 + P.n1 : P.k / 512;
    }
    if ((P.kind == PH_ATTN || P.kind == PH_COMB) && P.kv_heads > 0) P.splits = std::min(grid / P.kv_heads, kMaxSplits);
    if (P.kind == PH_GEMV && P.tiled) {
        // outputs per workgroup, not per wave
        P.rper = P.rows / grid;
        P.rrem = P.rows % grid;
        const int n = P.rper + (P.rrem ? 1 : 0);
        P.ttiles = P.epi == EP_SWIGLU ? (n + 7) / 8 : (n + 15) / 16;
        P.tcw = P.k / 64 / kNW;
        P.nm = P.epi == EP_SWIGLU ? 2 : 1;
    }
    if (P.kind == PH_GDNF) {
        P.fast_head = 0;
        P.xcd = grid % 8 == 0 && P.heads % 8 == 0 && grid == 16 * P.heads;
    }
    P.region = (P.kind == PH_GEMV && !P.fast_head) || P.kind == PH_GDN || P.kind == PH_ATTN || P.kind == PH_GDNF;
}

bool gemv_tileable(const Phase& P, int grid) {
    if (P.kind != PH_GEMV || P.mkind != 1 || P.group % 64 != 0 || P.k % (64 * kNW) != 0 || P.xin != XI_EXCH) return false;
    if (P.epi != EP_STORE && P.epi != EP_RESID && P.epi != EP_SWIGLU) return false;
    const int n = (P.rows + grid - 1) / grid;
    const int T = P.epi == EP_SWIGLU ? (n + 7) / 8 : (n + 15) / 16;
    if (T < 1 || T > 4 || n > kT) return false;
    if (P.epi == EP_RESID && n > kTiledMaxRes) return false;
    if (P.xnorm == XN_GDN && P.k % kDK != 0) return false;
    const int Cw = P.k / 64 / kNW, NB = (Cw + 3) / 4;
    return T * NB * 2048 + T * Cw * 64 <= kHalf;  // nibble blocks, then pairs
}

bool gdn_fusable(int kind, int k, int group, int heads, int grid) {
    if (kind != 1 || k % 512 != 0 || k > 4096 || heads <= 0 || grid != 16 * heads) return false;
    const int rb = k / 2, szb = (k / group) * 4;
    if (szb % 16 != 0 || kGfSlots * (szb / 16) > kWave) return false;  // one transfer for every slot's pairs
    const int state = (kGfSlots * (rb + szb) + 96 + 127) & ~127;
    return state + 512 <= kHalf;
}

bool finalize_program(Phase* prog, int nph, DecodeArgs& a) {
    a.reg0 = a.reg1 = a.head_reg = -1;
    for (int p = 0; p < nph; p++) {
        if (!prog[p].region) continue;
        if (prog[p].is_head) a.head_reg = p;
        else if (a.reg0 < 0) a.reg0 = p;
        else if (a.reg1 < 0) a.reg1 = p;
    }
    for (int p = 0; p < nph; p++) {
        int c = 0;
        prog[p].nr[0] = prog[p].nr[1] = -1;
        for (int q = p + 1; q < nph && c < 2; q++)
            if (prog[q].region && !prog[q].is_head) prog[p].nr[c++] = q - p;
    }
    return a.reg1 >= 0 && (a.head_reg < 0 || a.head_reg == nph - 1);
}

void split_program(const Phase* prog, int nph, std::vector<PhaseBufs>& bufs, std::vector<Phase>& shapes,
                   std::vector<GdnExtra>& gdnx) {
    gdnx.clear();
    // the shape is every field before the buffers (all 4-byte fields: no padding inside)
    constexpr size_t kShapeBytes = offsetof(Phase, w);
    static_assert(kShapeBytes % 4 == 0, "shape fields are 4-byte");
    bufs.assign(nph, PhaseBufs());
    shapes.clear();
    for (int p = 0; p < nph; p++) {
        const Phase& P = prog[p];
        size_t s = 0;
        while (s < shapes.size() && std::memcmp(&shapes[s], &P, kShapeBytes) != 0) s++;
        if (s == shapes.size()) {
            Phase sh;
            std::memcpy((void*)&sh, (const void*)&P, kShapeBytes);
            shapes.push_back(sh);
        }
        PhaseBufs& b = bufs[p];
        b.shape = (uint32_t)s;
        b.gain = P.gain;
        b.in = P.in;
        b.out = P.out;
        if (P.kind == PH_GEMV || P.kind == PH_GDNF) {
            b.w = P.w;
            b.sz = P.sz;
            b.aux = P.conv_w;
            b.conv = P.conv;
            if (P.kind == PH_GDNF) {
                GdnExtra x;
                x.rec = P.rec;
                x.prm = P.prm;
                x.grp = P.grp;
                x.grp_stride = P.grp_stride;
                b.xi = (uint32_t)gdnx.size();
                gdnx.push_back(x);
            }
        } else if (P.kind == PH_GDN) {
            b.w = P.rec;
        } else if (P.kind == PH_ATTN) {
            b.w = P.kp;
            b.sz = P.vp;
            b.aux = P.part;
        } else {
            b.aux = P.in2;
        }
    }
}

hipError_t launch_decode(const DecodeArgs& a, int grid, hipStream_t st) {
    void* args[] = {(void*)&a};
    const void* fn = a.feed ? (const void*)k_decode : (const void*)k_prefill_tokens;
    return hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kT), args, 0, st);
}

int decode_max_grid() {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    for (const void* fn : {(const void*)k_decode, (const void*)k_prefill_tokens}) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, kT, 0) != hipSuccess || per < 1) return 0;
    }
    return cus;
}

}  // namespace qne
