/* CPU oracle for the Qwen3.5 hybrid decoder path.
 *
 * TEST INFRASTRUCTURE ONLY. This restates the reference's math on the CPU so that the HIP engine
 * can be checked against it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and there only as the checker (or the timed CPU baseline), never as the product.
 *
 * Each function cites the reference file:line it restates (paths relative to the reference repo).
 * The shapes are config-driven instead of the reference's fixed constants, and three weight
 * encodings are supported: f16, the reference's MatMulNBits int4 (block 32, f16 scale, u4 zero
 * point) and the group-64 int4 with an f16 scale and an f16 zero.
 *
 * Precision: the same source is compiled twice. liboracle_f32.so accumulates in float (the
 * reference's CPU checks do the same, kernels/src/lib.rs:528-535), liboracle_f64.so accumulates
 * in double and evaluates exp/log/sqrt/sin/cos in double; use it to measure error.
 */
#ifndef QNE_ORACLE_H
#define QNE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OC_F16 = 0, OC_Q4G = 1, OC_Q4V1 = 2 };
enum { OC_STORE = 0, OC_ACCUMULATE = 1, OC_SWIGLU = 2 };

typedef struct {
    int32_t kind;  /* OC_F16 / OC_Q4G / OC_Q4V1 */
    int32_t rows;
    int32_t k;
    int32_t group; /* values per quantisation group (64 for OC_Q4G, 32 for OC_Q4V1) */
    const void* w; /* f16[rows*k] or u32[rows*k/8] nibbles, value c at bits 4*(c%8) of word c/8 */
    const void* s; /* f16 scales, [rows][k/group] */
    const void* z; /* OC_Q4G: f16 zeros [rows][k/group]; OC_Q4V1: u4 zero points, 2 per byte */
} oc_mat;

typedef struct {
    int32_t hidden, layers, full_attention_every, intermediate, vocab;
    int32_t n_q_heads, n_kv_heads, head_dim, rope_dim;
    int32_t gdn_heads, gdn_dk, gdn_dv, conv_kernel;
    int32_t max_context;
    float rope_theta;
    float eps;
} oc_config;

typedef struct {
    oc_mat mixer_in, mixer_out, gate_up, down;
    const float* input_norm;
    const float* post_norm;
    const float* attn_norms; /* q_norm[head_dim], k_norm[head_dim] */
    const float* conv_w;     /* [conv_channels][conv_kernel] */
    const float* gdn_params; /* dt_bias[H], A_neg_exp[H], norm_w[dv] */
} oc_layer;

typedef struct {
    oc_config c;
    oc_mat embed, lm_head;
    const float* final_norm;
    const oc_layer* layers;
} oc_model;

typedef struct oc_state oc_state;

/* ---- element kernels ---- */
float oc_f16_to_f32(uint16_t h);
uint16_t oc_f32_to_f16(float f); /* round to nearest even */
void oc_dequant_row(const oc_mat* m, int row, float* out);
void oc_gemv(const oc_mat* m, const float* x, float* y, int epilogue);
void oc_rmsnorm(const float* x, const float* g, float* y, int n, float eps);
void oc_embed(const oc_mat* m, uint32_t token, float* h);
void oc_argmax(const float* v, int n, uint32_t* idx, float* val);
void oc_rope_inv_freq(int rope_dim, float theta, float* inv_freq);
void oc_gdn_step(const oc_config* c, const float* proj, float* conv_state, const float* conv_w,
                 float* state, float* o, const float* prm);
void oc_attention_step(const oc_config* c, const float* proj, uint16_t* kc, uint16_t* vc,
                       uint32_t pos, float* o, const float* prm);
/* Raw recurrences for the kernel microbenches. */
void oc_delta_rule(int dk, int dv, const float* q, const float* k, const float* v, float beta,
                   float g, float* state, float* out);
void oc_attn_dense(int nq, int nkv, int hd, const float* q, const uint16_t* kc, const uint16_t* vc,
                   int len, float scale, float* out);

/* ---- sampling (src/sampling.rs), always in f32 as the reference ---- */
/* Sampler::new's state (src/sampling.rs:42-46) and one draw of its xorshift64 (:48-55). */
uint64_t oc_sampler_seed(uint64_t seed);
float oc_sampler_next_f32(uint64_t* state);
/* Sampler::try_sample (:58-67) with sample (:69-79) and choose (:81-134) over one row of V logits.
 * mask: NULL for none, else a bitset of mask_len tokens (bit i%32 of word i/32 allows token i);
 * seen: V bytes, the tokens this sampler generated (set when presence_penalty != 0). Equal values
 * are taken in increasing token order (the reference's unstable sorts leave that order open).
 * Returns 0 with *token set, or 1 for a distribution try_sample rejects (a NaN or +inf logit among
 * the allowed tokens, or no finite allowed logit). */
int oc_sample(const float* logits, uint32_t V, const uint32_t* mask, uint32_t mask_len, float temperature,
              uint32_t top_k, float top_p, float presence_penalty, uint64_t* state, uint8_t* seen,
              uint32_t* token);

/* ---- model ---- */
size_t oc_state_size_floats(const oc_model* m);
oc_state* oc_state_new(const oc_model* m);
void oc_state_free(oc_state* s);
void oc_reset(oc_state* s);
void oc_token(const oc_model* m, oc_state* s, uint32_t token, uint32_t pos, float* logits);
void oc_prefill_chunk(const oc_model* m, oc_state* s, const uint32_t* ids, int n, uint32_t start,
                      int finish_logits, float* logits);
void oc_copy_state(const oc_state* from, oc_state* to);
/* Dense views of the state for comparisons: recurrent state (f32), conv state (f32), KV (f16 as
 * [attn_layer][kv_head][max_context][head_dim]). */
float* oc_state_recurrent(oc_state* s, int gdn_layer);
float* oc_state_conv(oc_state* s, int gdn_layer);
uint16_t* oc_state_kcache(oc_state* s, int attn_layer);
uint16_t* oc_state_vcache(oc_state* s, int attn_layer);
int oc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
