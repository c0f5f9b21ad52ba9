// Host-visible description of the persistent decode kernel (kernels/decode.hip).
//
// A decode window runs as ONE cooperative launch. The per-token work is a fixed program of
// phases (built once at load, read by the kernel through the constant address space); each phase
// consumes a vector published by the previous phase and publishes its own. Vectors are handed over as tagged values: every f32
// is stored next to a 32-bit tag (the phase's sequence number) in one 8-byte agent-scope store,
// and a consumer polls until every tag it needs carries the expected number. No grid barrier and
// no cache-maintenance fence is needed: the tag proves the value next to it is the new one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

namespace qne {

// PH_GDNF: a GDN layer's in-projection and recurrent step in one phase (the workgroups of a head
// compute its projection rows, exchange q and k among themselves, then step the head's state).
enum PhaseKind { PH_GEMV = 0, PH_GDN = 1, PH_ATTN = 2, PH_COMB = 3, PH_GDNF = 4 };
// Input of a GEMV phase: the previous phase's published vector, or the step's embedding row.
enum { XI_EXCH = 0, XI_EMBED = 1 };
// Transform of that input: none, RMSNorm with `gain`, or the GDN output norm (per-head 1/rms from
// the published partial sums of squares).
enum { XN_PLAIN = 0, XN_NORM = 1, XN_GDN = 2 };
// Output of a GEMV phase: plain store, GDN causal conv + SiLU (first conv_ch rows), residual add
// into the rows of h the wave owns, SwiGLU of (gate, up) row pairs, LM head (logits + argmax).
enum { EP_STORE = 0, EP_CONV = 1, EP_RESID = 2, EP_SWIGLU = 3, EP_HEAD = 4 };

constexpr int kDecodeThreads = 512;
constexpr int kMaxPhases = 192;
constexpr int kHeadDim = 256;  // attention head size the kernel is written for
constexpr int kMaxSplits = 84;  // attention context splits per kv head (the combine stages 66 floats each, plus its reduction)

// One phase. `variant` selects the compiled GEMV shape (matrix kind and K). The integer fields
// come first: they are the phase's shape, which the kernel reads from a table of distinct shapes
// (every layer of a kind shares one). The buffers at the end are the host's; the kernel reads them
// from the phase's PhaseBufs record.
struct Phase {
    int kind = 0, variant = -1;
    int mkind = 0, k = 0, group = 64, rows = 0;  // GEMV matrix; rows = outputs (SwiGLU: pairs)
    int xin = XI_EXCH, xnorm = XN_PLAIN, epi = EP_STORE;
    int in_n = 0;       // values of the input vector (GEMV)
    int conv_ch = 0;    // EP_CONV: rows that go through the causal conv
    int heads = 0;      // GDN heads, or attention q heads
    int kv_heads = 0;   // attention
    int in_rel = 1;     // the input was published `in_rel` phases earlier in the same step
    int in2_rel = 0;    // second input (COMB: the gate in the in-projection output)
    int is_head = 0;    // phase runs only on steps that compute logits
    int xcd = 0;        // PH_GDNF: the 16 workgroups of a head share an XCD (workgroup w runs on XCD w % 8 + c)
    int tiled = 0;      // q4 GEMV on the matrix cores: rows owned by workgroups in tiles of 16, K split over waves
    int fold = 0;       // PH_ATTN: the combine of the partials runs in the same phase (no PH_COMB)
    uint32_t part_stride = 0;  // fold: entries of the partials buffer per step parity
    int ttiles = 0, tcw = 0;  // tiled: row tiles per workgroup, 64-column chunks per wave
    uint32_t in_stride = 0, in2_stride = 0, out_stride = 0;  // u64 entries
    uint32_t in_cap = 0, in2_cap = 0;  // entries readable from in / in2 (bounds of the polling loads)
    // Derived by finalize_phase from the fields above and the launch grid, so the kernel reads
    // constants instead of dividing:
    int region = 0;     // the phase reads data prefetched into an LDS half (LDS GEMV, GDN, attention)
    int fast_head = 0;  // LM head streamed through registers instead of an LDS half
    int rper = 0, rrem = 0;  // GEMV outputs per wave: rows / waves and rows % waves
    int rb = 0, szb = 0, stride = 0, nm = 1;  // GEMV row bytes, scale/zero bytes, their sum, rows per output
    int cap = 0, dper = 0, convb = 0;  // outputs per LDS half, DMA instructions per output, conv bytes per output
    int extra = 0;  // 1: a wave's one output past cap sits in the workgroup's extra slot (only wave 0
                    // has one: rrem <= workgroups); no two consecutive region phases use the slot
    int gshift = 6;     // log2(group)
    int n4 = 0, n2 = 0, n1 = 0, nsteps = 0;  // x steps: 2048/1024/512-column slabs (q4) or 512 (f16)
    int splits = 0;     // attention: context splits per kv head
    int nr[2] = {-1, -1};  // the next two region phases after this one in the same step (LM head
                           // excluded), as distances from this phase; -1: none
    // buffers
    const void* w = nullptr;
    const uint32_t* sz = nullptr;
    const float* gain = nullptr;    // XN_NORM gain; GDN: dt_bias, A_neg_exp, norm_w; ATTN: q_norm, k_norm
    const float* conv_w = nullptr;  // EP_CONV [conv_ch][4]
    float* conv = nullptr;          // EP_CONV state [conv_ch][4] (3 used)
    float* rec = nullptr;           // GDN state [heads][dv][dk] (value-major)
    uint16_t* kp = nullptr;         // attention pools [blocks][kv_heads][16][256]
    uint16_t* vp = nullptr;
    uint64_t* in = nullptr;         // input exchange buffer (step parity 0; parity 1 at + in_stride)
    uint64_t* in2 = nullptr;
    uint64_t* out = nullptr;        // output exchange buffer
    // PH_GDNF: the GDN parameters, and the head-group exchange of q, k, a, b ([heads][258] entries
    // per step parity, parity 1 at + grp_stride)
    const float* prm = nullptr;
    uint64_t* grp = nullptr;
    uint32_t grp_stride = 0;
    uint64_t* part = nullptr;  // PH_ATTN with fold: the partials buffer
};

// Per-phase buffers of a PH_GDNF phase beyond its PhaseBufs record (indexed by PhaseBufs::xi).
struct GdnExtra {
    float* rec = nullptr;          // recurrent state [heads][dv][dk]
    const float* prm = nullptr;    // dt_bias[heads], A_neg_exp[heads], norm_w[dv]
    uint64_t* grp = nullptr;       // head-group exchange
    uint32_t grp_stride = 0, pad = 0;
};
static_assert(sizeof(GdnExtra) == 32, "four 8-byte fields");

// The kernel's per-phase record: the phase's buffers and the index of its shape, in one 64-byte
// line. The program is read through the scalar data cache at every phase; with the shapes shared
// between layers, a 2B-sized token's program (about 150 of these plus ~16 shapes) stays resident
// there instead of missing to L2 on every phase. A slot holds what the phase's kind uses.
struct PhaseBufs {
    const void* w = nullptr;     // GEMV rows; GDN recurrent state; attention K pool
    const void* sz = nullptr;    // GEMV q4 (scale, zero) rows; attention V pool
    const float* gain = nullptr;
    const void* aux = nullptr;   // EP_CONV conv weights; combine: the second input; folded attention: its partials
    float* conv = nullptr;       // EP_CONV conv state
    uint64_t* in = nullptr;
    uint64_t* out = nullptr;
    uint32_t shape = 0;
    uint32_t xi = 0;  // PH_GDNF: index of its GdnExtra record
};
static_assert(sizeof(PhaseBufs) == 64, "one scalar-cache line per phase");

struct DecodeArgs {
    const PhaseBufs* prog = nullptr;  // per phase
    const Phase* shapes = nullptr;    // distinct shapes, indexed by PhaseBufs::shape
    const GdnExtra* gdnx = nullptr;   // PH_GDNF records, indexed by PhaseBufs::xi
    int nph = 0;  // phases per token
    // embedding (read by every workgroup at the start of a step)
    const void* emb_w = nullptr;
    const uint32_t* emb_sz = nullptr;
    int emb_kind = 0, emb_group = 64;
    int hidden = 0, vocab = 0;
    float eps = 1e-6f;
    int rope_dim = 64;
    const float* inv_freq = nullptr;
    const int32_t* block_table = nullptr;
    int max_blocks = 0;
    float* logits = nullptr;
    uint64_t* am = nullptr;  // argmax exchange: 2 entries per workgroup, parity stride am_stride
    uint32_t am_stride = 0;
    // tokens
    uint32_t* tok = nullptr;        // {token, pos, n_out, 0}
    const uint32_t* ids = nullptr;  // feed 0: token of step s is ids[s]
    uint32_t* out_ids = nullptr;    // greedy picks appended at tok[2]
    uint32_t out_cap = 0;
    int n_steps = 1;
    uint32_t pos0 = 0;
    int feed = 0;    // 0: tokens from ids, 1: greedy feedback
    int head = 0;    // 0: no LM head, 1: every step, 2: last step only
    int argmax = 0;  // greedy pick after the LM head
    uint32_t tag_base = 1;  // tag of phase p of step s = tag_base + s * nph + p
    // region phases (those that read prefetched data): the first two of a step (LM head excluded)
    // and the LM head when it is one (else -1); set by finalize_program
    int reg0 = -1, reg1 = -1, head_reg = -1;
    // 1: the residual stream's rows are owned by workgroups (the tiled GEMVs' output rows), kept in
    // LDS; 0: by waves (two rows at most per wave, in registers)
    int h_tiled = 0;
    unsigned* err = nullptr;  // [0] set on a polling timeout
    unsigned spin_limit = 1u << 20;
    // Optional device timeline (ticks of the constant-rate wall clock): trace[0] start, trace[1]
    // end (workgroup 0); for phase instance i = step * nph + p and workgroup w:
    // trace[2 + 2 (i * grid + w)] when w had its input, trace[3 + 2 (i * grid + w)] when w was
    // done. `trace_cap` phase instances are recorded.
    unsigned long long* trace = nullptr;
    int trace_cap = 0;
    // Optional finer timeline (profiling): for phase instance i and workgroup w, sub[8 (i * grid + w) + k]
    // holds timestamps of the phase's sub-steps (kept in registers, stored when the phase ends);
    // 0 = not reached. k = 0 entry. GEMV (entry = input staged): 1 x slice loaded, 2 first group's
    // rows done, 3 all rows published. GDN: 1 input staged, 2 state update published. Attention
    // partials: 1 input staged, 2 q/k normed and rotated, 3 context loop done, 4 partials
    // published. Combine: 1 partials staged, 2 gate staged, 3 published. Region phases: 7 the DMA
    // of the region phase two ahead issued. Slot 6 is not a timestamp: (XCC_ID << 32 | HW_ID) + 1
    // of the workgroup.
    unsigned long long* sub = nullptr;
};

// Fills the derived fields of P for a launch of `grid` workgroups (kDecodeThreads / 64 waves each).
void finalize_phase(Phase& P, int grid);
// Fills the region-phase links of a finalized program (Phase::nr, DecodeArgs::reg0 / reg1 / head_reg).
// Returns false if a step has fewer than two region phases besides the LM head.
bool finalize_program(Phase* prog, int nph, DecodeArgs& a);
// Splits a finalized program into the kernel's tables: one PhaseBufs per phase and the distinct
// shapes (phases equal in every field before the buffers share one).
void split_program(const Phase* prog, int nph, std::vector<PhaseBufs>& bufs, std::vector<Phase>& shapes,
                   std::vector<GdnExtra>& gdnx);
// Whether a GDN layer's in-projection (matrix kind, K, group) fits the fused PH_GDNF phase on a
// grid of `grid` workgroups with `heads` GDN heads of 128 channels.
bool gdn_fusable(int kind, int k, int group, int heads, int grid);
// Whether a GEMV phase (finalized fields not needed) can run tiled on the matrix cores.
bool gemv_tileable(const Phase& P, int grid);
constexpr int kTiledMaxRes = 16;  // residual rows a workgroup may own in the tiled layout
// GEMV shapes compiled into the kernel: variant id of (matrix kind, K), or -1.
int decode_gemv_variant(int kind, int k);
hipError_t launch_decode(const DecodeArgs& a, int grid, hipStream_t st);
// Largest cooperative grid for the decode kernel on the current device (one workgroup per CU).
int decode_max_grid();

}  // namespace qne
