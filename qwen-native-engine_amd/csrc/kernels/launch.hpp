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

// Embedding row tok[0] -> h (f32). kind 0: f16 [V][H]; kind 1: q4.
void launch_embed(int kind, const void* W, const uint32_t* SZ, int group, int hidden, const uint32_t* tok,
                  float* h, hipStream_t st);

// Gated DeltaNet decode step, all heads (dk = dv = 128).
void launch_gdn_decode(const float* proj, float* conv_state, const float* conv_w, float* state, float* out,
                       const float* prm, int heads, hipStream_t st);
// The bare delta rule for batch x heads (q, k used as given).
void launch_delta_rule(const float* q, const float* k, const float* v, const float* beta, const float* g,
                       float* state, float* out, int batch, int heads, hipStream_t st);
// The delta rule over T tokens in chunks of 64.
void launch_delta_rule_chunked(const float* q, const float* k, const float* v, const float* beta, const float* g,
                               float* state, float* out, int batch, int tokens, int heads, hipStream_t st);

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
// Raw paged decode for `batch` sequences: append k/v at ctx[b], attend over 0..ctx[b].
void launch_paged_attn(const float* q, const float* k_new, const float* v_new, uint16_t* k_pool, uint16_t* v_pool,
                       const int32_t* block_table, int max_blocks, const int32_t* ctx, float* out, int batch, int nq,
                       int nkv, float* part_ml, float* part_acc, int splits, hipStream_t st);

}  // namespace qne
