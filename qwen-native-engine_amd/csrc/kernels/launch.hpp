// Host-side launchers of the standalone kernels, and the device helpers they share.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>


namespace qne {

constexpr int kArgmaxMaxBlocks = 1024;

enum { EPI_STORE = 0, EPI_ACCUMULATE = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };
enum { KIND_F16 = 0, KIND_Q4 = 1 };

// Where the greedy pick of the LM head goes. tok = {token, pos, n_out, 0}: the pick replaces
// tok[0], tok[1] advances by one (argmax_final, kernels/src/shaders.rs:692-695), and when `ids`
// is set the pick is also appended at ids[tok[2]++] (bounded by ids_cap).
struct ArgmaxOut {
    float* part_val = nullptr;
    uint32_t* part_idx = nullptr;
    unsigned* counter = nullptr;  // zero between launches; the last block resets it
    uint32_t* tok = nullptr;
    uint32_t* ids = nullptr;
    uint32_t ids_cap = 0;
};


bool launch_gemv(int kind, const void* W, const uint32_t* SZ, int rows, int k, int group, const float* x,
                 const float* gain, float eps, float* y, int epi, const ArgmaxOut& am, hipStream_t st);

// tok[0] = ids[i], tok[1] = pos.
void launch_set_tok(uint32_t* tok, const uint32_t* ids, int i, uint32_t pos, hipStream_t st);
// Measurement kernels: a streaming read of `bytes` (a multiple of 16) folded into sink
// [workgroups * 256], and a dispatch that does almost nothing.
void launch_stream_read(const void* data, size_t bytes, uint32_t* sink, int workgroups, hipStream_t st);
void launch_noop(float* y, hipStream_t st);
// The hand-over probe (k_exchange_probe): `workgroups` co-resident 512-thread workgroups exchange
// an n-value tagged vector `rounds` times through buf (2 n entries).
hipError_t launch_exchange_probe(uint64_t* buf, int n, int rounds, int workgroups, unsigned long long* ticks, unsigned* err,
                                 hipStream_t st);

// Pseudo-random uniform [-amp, amp) fill of n f16 or f32 values (benchmark state).
void launch_fill_uniform(void* p, size_t n, bool f16, uint64_t seed, float amp, hipStream_t st);

// Embedding row tok[0] -> h (f32). kind 0: f16 [V][H]; kind 1: q4.
void launch_embed(int kind, const void* W, const uint32_t* SZ, int group, int hidden, const uint32_t* tok,
                  float* h, hipStream_t st);

// Gated DeltaNet decode step, all heads (dk = dv = 128).
void launch_gdn_decode(const float* proj, float* conv_state, const float* conv_w, float* state, float* out,
                       const float* prm, int heads, hipStream_t st);
// The bare delta rule for batch x heads (q, k used as given).
void launch_delta_rule(const float* q, const float* k, const float* v, const float* beta, const float* g,
                       float* state, float* out, int batch, int heads, hipStream_t st);
// The delta rule over T tokens, token by token (value columns split over waves).
void launch_delta_rule_chunked(const float* q, const float* k, const float* v, const float* beta, const float* g,
                               float* state, float* out, int batch, int tokens, int heads, hipStream_t st);
// The delta rule over T tokens in the chunk-64 WY form on MFMA; ws holds wy_workspace_bytes.
size_t wy_workspace_bytes(int batch, int tokens, int heads);
// value_major: the state is the model's [B][H][dv][dk] instead of [B][H][dk][dv].
void launch_delta_rule_wy(const float* q, const float* k, const float* v, const float* beta, const float* g,
                          float* state, float* out, int batch, int tokens, int heads, float* ws, hipStream_t st,
                          int value_major = 0);

// Attention decode, model form: q/k RMSNorm + RoPE, f16 append at tok[1], split-context partials,
// combine with the sigmoid gate into `out`.
struct AttnModelArgs {
    const float* proj;      // [q(nq*hd) gate(nq*hd) k(nkv*hd) v(nkv*hd)]
    const float* norms;     // q_norm[hd], k_norm[hd]
    const float* inv_freq;  // [rope_dim/2]
    uint16_t* k_pool;       // [blocks][nkv][16][hd]
    uint16_t* v_pool;
    const int32_t* block_table;
    const uint32_t* tok;    // tok[1] = position
    float* qbuf;            // [nq][hd] normed, rotated queries
    float* part_ml;         // [nkv][splits][group][2]
    float* part_acc;        // [nkv][splits][group][hd]
    float* out;             // [nq][hd]
    int nq, nkv, rope_dim, splits;
    int max_blocks;         // entries of block_table
};
void launch_attention_model(const AttnModelArgs& a, hipStream_t st);
// Batched model form: row b (one sequence) has its projection at proj + b * proj_stride, position
// pos[b] and block table row b; outputs [rows][nq * hd].
struct AttnRowsArgs {
    const float* proj;
    size_t proj_stride;
    const float* norms;
    const float* inv_freq;
    uint16_t* k_pool;
    uint16_t* v_pool;
    const int32_t* block_table;  // [rows][max_blocks]
    const int32_t* pos;          // [rows]
    float* qbuf;                 // [rows][nq][hd]
    float* part_ml;              // [rows][nkv][splits][group][2]
    float* part_acc;             // [rows][nkv][splits][group][hd]
    float* out;                  // [rows][nq][hd]
    int nq, nkv, rope_dim, splits, max_blocks, rows;
    int bt_stride;               // entries between rows of block_table (0: one shared row)
    // With order, the partials' workgroups take the rows in that order (longest context first, so
    // the longest workgroups start first); the results do not depend on it.
    const int32_t* order = nullptr;
    // With `part`, the projection is the in-projection's split partials (splits x split_stride
    // floats, rows n apart) summed here in split order times the row's 1 / rms (from the sums of
    // x^2 of its operand x_in, K = k_in): the GEMM's reduce folded in. The gate, which the
    // combine reads from proj, is then written to gate_dst (rows proj_stride apart).
    const float* part = nullptr;
    int in_splits = 0, in_n = 0, k_in = 0;
    size_t split_stride = 0;
    const uint8_t* x_in = nullptr;
    float eps = 1e-6f;
    float* gate_dst = nullptr;
    // With frag_out, the output rows are also staged as the out-projection's operand (column
    // order order_out); out may then be null.
    uint8_t* frag_out = nullptr;
    int order_out = 0;
    // With split_len (a multiple of 32, at most 1024), the rows are consecutive tokens of one sequence
    // (bt_stride 0) and the partials come from the query-tile kernel: split s holds positions
    // [s * split_len, (s + 1) * split_len); splits * split_len must cover max_blocks * 16.
    int split_len = 0;
};
void launch_attention_rows(const AttnRowsArgs& a, hipStream_t st);
// Whether the query-tile prefill attention takes this head grouping (2 or 4 q heads per kv head).
bool prefill_attention_supported(int nq, int nkv);

// Per-row strides (in floats) of the batched GDN decode step.
struct GdnRowStrides {
    size_t proj = 0, conv = 0, state = 0, out = 0;
};
// Prefill of `tokens` consecutive tokens of one sequence: conv + norms + gates, the recurrence on
// the model's value-major state, the gated RMSNorm into mixed + n * mixed_stride (when set) and,
// with frag_out, into the out-projection's GEMM operand (column order order_out), the conv state
// shifted by the chunk. q, k, v, o: tokens * heads * 128 floats of scratch; g, beta: tokens * heads.
// With wy_ws (wy_workspace_bytes(1, tokens, heads)), the recurrence runs in the chunk-64 WY form
// over every complete block of 64 tokens that starts `lead` tokens in or 64 k after that, and
// sequentially over the tokens before and after them: with lead = the tokens up to the next
// multiple of 64 positions, the blocks are fixed by absolute position.
void launch_gdn_chunk(const float* proj, int proj_stride, float* conv_state, const float* conv_w, float* state,
                      const float* prm, int heads, int tokens, float* q, float* k, float* v, float* g, float* beta,
                      float* o, float* mixed, int mixed_stride, hipStream_t st, int lead = 0, float* wy_ws = nullptr,
                      uint8_t* frag_out = nullptr, int order_out = 0);
// Where the batched GDN step reads its projection and writes its output. With `part`, the
// projection is the in-projection's split partials (splits x split_stride floats, rows n apart)
// summed here in split order times the row's 1 / rms (from the sums of x^2 of its operand x_in,
// K = k_in): the GEMM's reduce folded in. With frag_out, the output rows are also staged as the
// out-projection's operand (column order order_out); out may then be null.
struct GdnRowsIO {
    const float* part = nullptr;
    int splits = 0, n = 0, k_in = 0;
    size_t split_stride = 0;
    const uint8_t* x_in = nullptr;
    float eps = 1e-6f;
    uint8_t* frag_out = nullptr;
    int order_out = 0;
};
void launch_gdn_decode_rows(const float* proj, float* conv_state, const float* conv_w, float* state, float* out,
                            const float* prm, int heads, int rows, const GdnRowStrides& rs, hipStream_t st,
                            const GdnRowsIO& io = GdnRowsIO());

// y = x W^T for up to kGemmRowsMax rows of x (batched decode: up to 64; chunked prefill: a pass of
// tokens), on MFMA, in tiles of 64 rows. The x operand is staged in `frag` (gemm_frag_bytes(K, m)):
// with x set, launch_gemm stages rows x + r * x_stride (times `gain`, the
// RMSNorm's 1 / rms then applied to the output: norm); with x null, `frag` already holds the
// operand and `norm` says whether its rows carry a deferred RMSNorm. Epilogues as the GEMV (store,
// residual add, SwiGLU with n_out = N / 2); y may be null when frag_out is set. With frag_out the
// result (times gain_out, column order order_out) is also staged as the next GEMM's x operand.
// `part` holds splits * mpad * N floats (mpad: m rounded up to 64) unless the GEMM applies the
// epilogue itself. The split count depends on the matrix only (gemm_splits), so a row's sums are
// added in the same order whatever the number of rows.
struct GemmArgs {
    const float* x = nullptr;
    int x_stride = 0;
    int m = 0;
    const float* gain = nullptr;
    float eps = 1e-6f;
    uint8_t* frag = nullptr;
    int norm = 0;
    int kind = KIND_Q4;
    const void* W = nullptr;
    const uint32_t* SZ = nullptr;
    const uint32_t* SZT = nullptr;  // q4: SZ tile-major ([row / 32][group][row % 32]), what k_gemm reads
    int N = 0, K = 0, group = 64;
    int splits = 1;
    int cps = 0;     // set by launch_gemm: chunks per split
    int mpad = 0;    // set by launch_gemm: m rounded up to a multiple of 64 (rows of the partials)
    int direct = 0;  // set by launch_gemm: the GEMM applies the epilogue itself
    int fuse = 0;    // set by launch_gemm: the GEMM applies the epilogue and stages its output itself
                     // (1: SwiGLU, 2: store or residual add); -1 from the caller: never
    float* part = nullptr;
    int epi = EPI_STORE;
    float* y = nullptr;
    int y_stride = 0;
    int n_out = 0;
    uint8_t* frag_out = nullptr;
    const float* gain_out = nullptr;
    int order_out = 0;  // 1: the column order of a q4 GEMM's operand
    int partials_only = 0;  // write the split partials (even with one split) and launch no reduce:
                            // the kernel that reads the output sums them
};
// One row of token sampling (the O(vocab) part of src/sampling.rs choose / try_sample).
struct SampleArgs {
    const float* logits = nullptr;  // vocab logits
    uint32_t V = 0;
    const uint32_t* seen = nullptr;  // bitset of generated tokens (presence penalty), or null
    float penalty = 0.0f;            // subtracted from a generated token's logit (0: none)
    const uint32_t* mask = nullptr;  // bitset of allowed tokens, or null (all allowed)
    uint32_t mask_len = 0;           // tokens the mask covers; tokens past it are not allowed
    uint32_t bias_token = 0xFFFFFFFFu;
    float bias = 0.0f;               // added to bias_token's logit first
    uint32_t k = 0;                  // 0: greedy; else top-k candidates (<= 1024)
    float* out_v = nullptr;          // k values, sorted by total order descending, ties by token
    uint32_t* out_i = nullptr;       // their tokens
    uint32_t* info = nullptr;        // [0] candidates written, [1] flags (1: NaN or +inf allowed,
                                     // 2: a finite token allowed), [2] the greedy pick
};
constexpr uint32_t kSampleMaxK = 1024;
// Device scratch one sampling call needs (counters, sampled keys, candidates).
size_t sample_scratch_bytes();
void launch_sample(const SampleArgs& a, void* scratch, hipStream_t st);

constexpr int kGemmRowsMax = 2048;
size_t gemm_frag_bytes(int K, int m);
// Split-K count of a GEMM on an N x K matrix: as many splits as keep a grid of N tiles x row_tiles
// x splits within one workgroup per CU (at least 2 chunks per split, at most 24). A caller passes a
// fixed row_tiles (not the rows of the call), so that a row's sums do not depend on the call.
int gemm_splits(int kind, int N, int K, int group, int row_tiles = 1);
bool gemm_shape_ok(int kind, int N, int K, int group, int m);
void launch_gemm(GemmArgs a, hipStream_t st);
// The tile-major copy of q4 (scale, zero) words the row-tiled GEMM reads (GemmArgs::SZT):
// tile_sz_words(rows, groups) words.
size_t tile_sz_words(int rows, int ngroups);
void launch_tile_sz(const uint32_t* sz, int rows, int ngroups, uint32_t* szt, hipStream_t st);
// The x operand of a GEMM from f32 rows (rows >= m zero), times gain when set.
void launch_stage_x(const float* x, int x_stride, int m, int K, const float* gain, int q4order, uint8_t* frag,
                    hipStream_t st);
// h[r] = embedding row tokens[r], r < m; with frag, h * gain is also staged as a GEMM's x operand.
// With order, order[0..m) = the rows 0..m-1 by decreasing pos (ties: lower row first), the order
// the attention partials run them in.
void launch_embed_rows(int kind, const void* W, const uint32_t* SZ, int group, int hidden, const uint32_t* tokens, int m,
                       float* h, uint8_t* frag, const float* gain, int q4order, hipStream_t st,
                       const int32_t* pos = nullptr, int32_t* order = nullptr);
// Greedy pick per row into out[r]; with `tokens`, also tokens[r] = pick and pos[r] += 1. `scratch`
// holds argmax_rows_scratch(m) bytes.
size_t argmax_rows_scratch(int m);
void launch_argmax_rows(const float* logits, int m, int V, uint32_t* out, uint32_t* tokens, int32_t* pos, void* scratch,
                        hipStream_t st);

// Scratch of the no-allocation paged decode entry point: a file-scope device array of
// kNoAllocScratchBytes in attention.hip. noalloc_scratch() returns its address on the current
// device, looked up (hipGetSymbolAddress) on the first call made with that device current and kept
// per device; it allocates nothing.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
float* noalloc_scratch();

// Raw paged decode for `batch` sequences: append k/v at ctx[b], attend over 0..ctx[b].
// With order (batch ints of scratch; used for batch <= 256), the append kernel ranks the sequences
// by decreasing context and the partials take them longest first.
void launch_paged_attn(const float* q, const float* k_new, const float* v_new, uint16_t* k_pool, uint16_t* v_pool,
                       const int32_t* block_table, int max_blocks, const int32_t* ctx, float* out, int batch, int nq,
                       int nkv, float* part_ml, float* part_acc, int splits, hipStream_t st, int32_t* order = nullptr);

}  // namespace qne
