/* CPU oracle: TEST INFRASTRUCTURE ONLY (see oracle.h). Compiled twice, with OC_REAL=float and
 * OC_REAL=double, into liboracle_f32.so and liboracle_f64.so. */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#ifndef OC_REAL
#define OC_REAL float
#endif
typedef OC_REAL real;

#define OC_IS_DOUBLE (sizeof(real) == sizeof(double))
static inline real r_exp(real x) { return OC_IS_DOUBLE ? (real)exp((double)x) : (real)expf((float)x); }
static inline real r_log(real x) { return OC_IS_DOUBLE ? (real)log((double)x) : (real)logf((float)x); }
static inline real r_sqrt(real x) { return OC_IS_DOUBLE ? (real)sqrt((double)x) : (real)sqrtf((float)x); }
static inline real r_sin(real x) { return OC_IS_DOUBLE ? (real)sin((double)x) : (real)sinf((float)x); }
static inline real r_cos(real x) { return OC_IS_DOUBLE ? (real)cos((double)x) : (real)cosf((float)x); }
static inline real r_silu(real x) { return x / ((real)1 + r_exp(-x)); } /* kernels/src/lib.rs:509-511 */

/* IEEE half -> float, including subnormals (kernels/src/lib.rs:473-482 restates the normal and
 * subnormal cases; it maps exponent 31 to NaN, here infinities stay infinite). */
float oc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1fu, frac = h & 0x3ffu, bits;
    if (exp == 0) {
        float v = (float)frac * 5.9604644775390625e-8f; /* 2^-24 */
        return (h & 0x8000u) ? -v : v;
    }
    if (exp == 31) bits = sign | 0x7f800000u | (frac << 13);
    else bits = sign | ((exp + 112u) << 23) | (frac << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t oc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) { /* subnormal half (|f| < 2^-14) */
        if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        int shift = 126 - (int)(ax >> 23); /* 14..24 */
        uint32_t v = mant >> shift, rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (v & 1u))) v++;
        return (uint16_t)(sign | v);
    }
    uint32_t v = ((ax >> 13) - (112u << 10)), rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) v++;
    return (uint16_t)(sign | v);
}

/* One dequantised row. OC_Q4V1 restates dequant_row (kernels/src/lib.rs:484-497):
 * q = (W[r*K/8 + c/8] >> 4*(c%8)) & 15, block b = c/32, scale = f16 S[r*K/32 + b],
 * zp = (Z[r*K/256 + b/8] >> 4*(b%8)) & 15, w = (q - zp) * scale. OC_Q4G keeps the nibble layout
 * with an f16 scale and f16 zero per `group` values: w = (q - z) * s. */
void oc_dequant_row(const oc_mat* m, int row, float* out) {
    const int k = m->k;
    if (m->kind == OC_F16) {
        const uint16_t* w = (const uint16_t*)m->w + (size_t)row * k;
        for (int c = 0; c < k; c++) out[c] = oc_f16_to_f32(w[c]);
        return;
    }
    const uint32_t* w = (const uint32_t*)m->w + (size_t)row * (k / 8);
    const uint16_t* s = (const uint16_t*)m->s;
    const int groups = k / m->group;
    /* the group's scale and zero are converted once and reused for its values */
    for (int b = 0; b < groups; b++) {
        float scale = oc_f16_to_f32(s[(size_t)row * groups + b]);
        float zp;
        if (m->kind == OC_Q4G) {
            zp = oc_f16_to_f32(((const uint16_t*)m->z)[(size_t)row * groups + b]);
        } else {
            const uint8_t* z = (const uint8_t*)m->z + (size_t)row * ((groups + 1) / 2);
            zp = (float)((z[b / 2] >> (4 * (b % 2))) & 15u);
        }
        for (int c = b * m->group; c < (b + 1) * m->group; c++) {
            uint32_t q = (w[c / 8] >> (4 * (c % 8))) & 15u;
            out[c] = ((float)q - zp) * scale;
        }
    }
}

static real dot_row(const oc_mat* m, int row, const float* x, float* scratch) {
    oc_dequant_row(m, row, scratch);
    real acc = 0;
    for (int c = 0; c < m->k; c++) acc += (real)scratch[c] * (real)x[c];
    return acc;
}

/* GEMV with the reference's three epilogues (kernels/src/shaders.rs:36-43, checked at
 * kernels/src/lib.rs:528-535): Store y = Wx, Accumulate y += Wx, SwiGlu y[r] = silu(g)*u with
 * g = row r, u = row r + rows/2. */
void oc_gemv(const oc_mat* m, const float* x, float* y, int epilogue) {
    const int out_rows = epilogue == OC_SWIGLU ? m->rows / 2 : m->rows;
#pragma omp parallel
    {
        float* scratch = (float*)malloc(sizeof(float) * (size_t)m->k);
#pragma omp for schedule(static)
        for (int r = 0; r < out_rows; r++) {
            real a = dot_row(m, r, x, scratch);
            if (epilogue == OC_STORE) y[r] = (float)a;
            else if (epilogue == OC_ACCUMULATE) y[r] = (float)((real)y[r] + a);
            else {
                real u = dot_row(m, r + out_rows, x, scratch);
                y[r] = (float)(r_silu(a) * u);
            }
        }
        free(scratch);
    }
}

/* y = x * rsqrt(sum(x^2)/n + eps) * g (kernels/src/shaders.rs:378-403). */
void oc_rmsnorm(const float* x, const float* g, float* y, int n, float eps) {
    real ss = 0;
    for (int i = 0; i < n; i++) ss += (real)x[i] * (real)x[i];
    real inv = (real)1 / r_sqrt(ss / (real)n + (real)eps);
    for (int i = 0; i < n; i++) y[i] = (float)((real)x[i] * inv * (real)g[i]);
}

/* Row `token` of the embedding, dequantised (kernels/src/shaders.rs:405-434). */
void oc_embed(const oc_mat* m, uint32_t token, float* h) { oc_dequant_row(m, (int)token, h); }

/* Greedy pick (kernels/src/shaders.rs:635-699): the largest value; ties go to the lowest index,
 * NaN never wins. */
void oc_argmax(const float* v, int n, uint32_t* idx, float* val) {
    float best = -INFINITY;
    uint32_t bi = 0;
    int found = 0;
    for (int i = 0; i < n; i++) {
        if (v[i] > best || (!found && v[i] == best)) { best = v[i]; bi = (uint32_t)i; found = 1; }
    }
    *idx = bi;
    *val = best;
}

/* inv_freq[i] = theta^(-2i/rope_dim), rounded to float (kernels/src/shaders.rs:587). The angle is
 * then float(pos) * inv_freq[i] in float arithmetic, as the shader computes it. */
void oc_rope_inv_freq(int rope_dim, float theta, float* inv_freq) {
    for (int i = 0; i < rope_dim / 2; i++)
        inv_freq[i] = (float)pow((double)theta, -(double)(2 * i) / (double)rope_dim);
}

/* Gated DeltaNet decode step for all heads (kernels/src/shaders.rs:436-520; CPU reference
 * kernels/src/lib.rs:578-628). proj = [q(H*dk) k(H*dk) v(H*dv) z(H*dv) a(H) b(H)],
 * prm = [dt_bias(H) A_neg_exp(H) norm_w(dv)], state S[h][j][t] with key j and value t. */
void oc_gdn_step(const oc_config* c, const float* proj, float* conv_state, const float* conv_w,
                 float* state, float* o, const float* prm) {
    const int H = c->gdn_heads, dk = c->gdn_dk, dv = c->gdn_dv, K = c->conv_kernel;
    const int channels = 2 * H * dk + H * dv;
    float* conv_out = (float*)malloc(sizeof(float) * (size_t)channels);
    /* causal conv over the q, k, v channels, then SiLU (shaders.rs:457-468) */
    for (int ch = 0; ch < channels; ch++) {
        float* st = conv_state + (size_t)ch * (K - 1);
        const float* w = conv_w + (size_t)ch * K;
        real y = 0;
        for (int i = 0; i < K - 1; i++) y += (real)st[i] * (real)w[i];
        y += (real)proj[ch] * (real)w[K - 1];
        for (int i = 0; i < K - 2; i++) st[i] = st[i + 1];
        st[K - 2] = proj[ch];
        conv_out[ch] = (float)r_silu(y);
    }
    const float* zs = proj + channels;
    const float* as = zs + H * dv;
    const float* bs = as + H;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < H; h++) {
        const float* q = conv_out + h * dk;
        const float* k = conv_out + H * dk + h * dk;
        const float* v = conv_out + 2 * H * dk + h * dv;
        real* qs = (real*)malloc(sizeof(real) * (size_t)dk);
        real* ks = (real*)malloc(sizeof(real) * (size_t)dk);
        real* out = (real*)malloc(sizeof(real) * (size_t)dv);
        real sq2 = 0, sk2 = 0;
        for (int j = 0; j < dk; j++) { sq2 += (real)q[j] * q[j]; sk2 += (real)k[j] * k[j]; }
        real nq = (real)1 / r_sqrt(sq2 + (real)1e-6), nk = (real)1 / r_sqrt(sk2 + (real)1e-6);
        real qscale = (real)1 / r_sqrt((real)dk);
        for (int j = 0; j < dk; j++) { qs[j] = (real)q[j] * nq * qscale; ks[j] = (real)k[j] * nk; }
        /* g = exp(A_neg_exp * ln(1 + e^(a + dt_bias))), beta = sigmoid(b) (shaders.rs:495-496) */
        real g = r_exp((real)prm[H + h] * r_log((real)1 + r_exp((real)as[h] + (real)prm[h])));
        real beta = (real)1 / ((real)1 + r_exp(-(real)bs[h]));
        real kq = 0;
        for (int j = 0; j < dk; j++) kq += ks[j] * qs[j];
        float* S = state + (size_t)h * dk * dv;
        for (int t = 0; t < dv; t++) {
            real sk = 0, sqv = 0;
            for (int j = 0; j < dk; j++) { real sv = S[(size_t)j * dv + t]; sk += sv * ks[j]; sqv += sv * qs[j]; }
            real dvv = beta * ((real)v[t] - g * sk);
            for (int j = 0; j < dk; j++) S[(size_t)j * dv + t] = (float)(g * (real)S[(size_t)j * dv + t] + dvv * ks[j]);
            out[t] = g * sqv + dvv * kq;
        }
        /* gated RMSNorm of the head output (shaders.rs:514-516) */
        real ss = 0;
        for (int t = 0; t < dv; t++) ss += out[t] * out[t];
        real inv = (real)1 / r_sqrt(ss / (real)dv + (real)1e-6);
        for (int t = 0; t < dv; t++)
            o[h * dv + t] = (float)(out[t] * inv * r_silu((real)zs[h * dv + t]) * (real)prm[2 * H + t]);
        free(qs); free(ks); free(out);
    }
    free(conv_out);
}

/* RMSNorm with weight, then rotate-half RoPE on the first rope_dim dims (shaders.rs:575-593). */
static void norm_rope(const oc_config* c, const float* x, const float* w, uint32_t pos, real* y) {
    const int hd = c->head_dim, half = c->rope_dim / 2;
    real ss = 0;
    for (int j = 0; j < hd; j++) ss += (real)x[j] * x[j];
    real inv = (real)1 / r_sqrt(ss / (real)hd + (real)1e-6);
    for (int j = 0; j < hd; j++) y[j] = (real)x[j] * inv * (real)w[j];
    float inv_freq[512];
    oc_rope_inv_freq(c->rope_dim, c->rope_theta, inv_freq);
    for (int i = 0; i < half; i++) {
        float angle = (float)pos * inv_freq[i];
        real cs = r_cos((real)angle), sn = r_sin((real)angle);
        real a = y[i], b = y[i + half];
        y[i] = a * cs - b * sn;
        y[i + half] = b * cs + a * sn;
    }
}

/* Gated GQA attention decode step (kernels/src/shaders.rs:522-633; CPU reference
 * kernels/src/lib.rs:630-677). proj = [q(nq*hd) gate(nq*hd) k(nkv*hd) v(nkv*hd)],
 * prm = [q_norm(hd) k_norm(hd)]. The normed, rotated key and the value are stored as f16 at `pos`
 * in kc/vc ([kv_head][max_context][hd]) before the scores are taken, so the current position is
 * read back rounded exactly as every later step reads it. */
void oc_attention_step(const oc_config* c, const float* proj, uint16_t* kc, uint16_t* vc,
                       uint32_t pos, float* o, const float* prm) {
    const int nq = c->n_q_heads, nkv = c->n_kv_heads, hd = c->head_dim, cap = c->max_context;
    const float* kp = proj + 2 * nq * hd;
    const float* vp = kp + nkv * hd;
    real* y = (real*)malloc(sizeof(real) * (size_t)hd);
    for (int g = 0; g < nkv; g++) {
        norm_rope(c, kp + g * hd, prm + hd, pos, y);
        for (int j = 0; j < hd; j++) {
            kc[((size_t)g * cap + pos) * hd + j] = oc_f32_to_f16((float)y[j]);
            vc[((size_t)g * cap + pos) * hd + j] = oc_f32_to_f16(vp[g * hd + j]);
        }
    }
    free(y);
    const int len = (int)pos + 1, group = nq / nkv;
    const real scale = (real)1 / r_sqrt((real)hd);
#pragma omp parallel for schedule(static)
    for (int h = 0; h < nq; h++) {
        const int g = h / group;
        real* q = (real*)malloc(sizeof(real) * (size_t)hd);
        real* sc = (real*)malloc(sizeof(real) * (size_t)len);
        real* acc = (real*)calloc((size_t)hd, sizeof(real));
        norm_rope(c, proj + h * hd, prm, pos, q);
        real m = -INFINITY;
        for (int l = 0; l < len; l++) {
            const uint16_t* kr = kc + ((size_t)g * cap + l) * hd;
            real d = 0;
            for (int j = 0; j < hd; j++) d += q[j] * (real)oc_f16_to_f32(kr[j]);
            sc[l] = d * scale;
            if (sc[l] > m) m = sc[l];
        }
        real total = 0;
        for (int l = 0; l < len; l++) { sc[l] = r_exp(sc[l] - m); total += sc[l]; }
        for (int l = 0; l < len; l++) {
            const uint16_t* vr = vc + ((size_t)g * cap + l) * hd;
            for (int j = 0; j < hd; j++) acc[j] += sc[l] * (real)oc_f16_to_f32(vr[j]);
        }
        const float* gate = proj + nq * hd + h * hd;
        for (int j = 0; j < hd; j++)
            o[h * hd + j] = (float)(acc[j] / total / ((real)1 + r_exp(-(real)gate[j])));
        free(q); free(sc); free(acc);
    }
}

/* The delta rule alone, one head, one token: sk = S^T k, dv = beta (v - g sk),
 * S' = g S + k dv^T, out = g S^T q + dv (k.q) = S'^T q (kernels/src/shaders.rs:498-512). */
void oc_delta_rule(int dk, int dv, const float* q, const float* k, const float* v, float beta,
                   float g, float* S, float* out) {
    real kq = 0;
    for (int j = 0; j < dk; j++) kq += (real)k[j] * q[j];
    for (int t = 0; t < dv; t++) {
        real sk = 0, sq = 0;
        for (int j = 0; j < dk; j++) { real s = S[(size_t)j * dv + t]; sk += s * k[j]; sq += s * q[j]; }
        real d = (real)beta * ((real)v[t] - (real)g * sk);
        for (int j = 0; j < dk; j++) S[(size_t)j * dv + t] = (float)((real)g * (real)S[(size_t)j * dv + t] + d * k[j]);
        out[t] = (float)((real)g * sq + d * kq);
    }
}

/* Dense GQA attention over an f16 cache [kv_head][len][hd] for q [nq][hd] (no gate): the dense
 * unpaged reference for the paged decode kernel. */
void oc_attn_dense(int nq, int nkv, int hd, const float* q, const uint16_t* kc, const uint16_t* vc,
                   int len, float scale, float* out) {
    const int group = nq / nkv;
    for (int h = 0; h < nq; h++) {
        const int g = h / group;
        real* sc = (real*)malloc(sizeof(real) * (size_t)len);
        real m = -INFINITY, total = 0;
        for (int l = 0; l < len; l++) {
            real d = 0;
            for (int j = 0; j < hd; j++) d += (real)q[h * hd + j] * (real)oc_f16_to_f32(kc[((size_t)g * len + l) * hd + j]);
            sc[l] = d * (real)scale;
            if (sc[l] > m) m = sc[l];
        }
        for (int l = 0; l < len; l++) { sc[l] = r_exp(sc[l] - m); total += sc[l]; }
        for (int j = 0; j < hd; j++) {
            real a = 0;
            for (int l = 0; l < len; l++) a += sc[l] * (real)oc_f16_to_f32(vc[((size_t)g * len + l) * hd + j]);
            out[h * hd + j] = (float)(a / total);
        }
        free(sc);
    }
}

/* ------------------------------------------------------------------------------------------ */
/* Sampling: src/sampling.rs, in f32 whatever OC_REAL is. */

uint64_t oc_sampler_seed(uint64_t seed) { return (seed * 0x9E3779B97F4A7C15ull) | 1ull; } /* :42-46 */

float oc_sampler_next_f32(uint64_t* state) { /* :48-55 */
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return (float)(x >> 40) / (float)(1ull << 24);
}

static int oc_allowed(const uint32_t* mask, uint32_t mask_len, uint32_t i) {
    return !mask || (i < mask_len && ((mask[i >> 5] >> (i & 31)) & 1u));
}

/* f32::total_cmp as an unsigned key: larger key = later in the total order. */
static uint32_t oc_total_key(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    return (u >> 31) ? ~u : (u | 0x80000000u);
}

typedef struct {
    float v;
    uint32_t i;
} oc_cand;

static int oc_cand_desc(const void* a, const void* b) {
    const oc_cand* x = (const oc_cand*)a;
    const oc_cand* y = (const oc_cand*)b;
    uint32_t kx = oc_total_key(x->v), ky = oc_total_key(y->v);
    if (kx != ky) return kx > ky ? -1 : 1;
    return x->i < y->i ? -1 : (x->i > y->i ? 1 : 0);
}

int oc_sample(const float* logits, uint32_t V, const uint32_t* mask, uint32_t mask_len, float temperature,
              uint32_t top_k, float top_p, float presence_penalty, uint64_t* state, uint8_t* seen,
              uint32_t* token) {
    /* try_sample: fail closed */
    int finite = 0;
    for (uint32_t i = 0; i < V; i++) {
        if (!oc_allowed(mask, mask_len, i)) continue;
        float l = logits[i];
        if (isnan(l) || l == INFINITY) return 1;
        finite |= isfinite(l);
    }
    if (!finite) return 1;
    /* choose */
    const float penalty = mask ? 0.0f : presence_penalty;
    uint32_t pick = 0;
    if (temperature <= 0.0f) {
        float best = -INFINITY;
        for (uint32_t i = 0; i < V; i++) {
            float l = logits[i];
            if (penalty != 0.0f && seen[i]) l = l - penalty;
            if (l > best && oc_allowed(mask, mask_len, i)) {
                best = l;
                pick = i;
            }
        }
    } else {
        oc_cand* c = (oc_cand*)malloc(sizeof(oc_cand) * (V ? V : 1));
        uint32_t n = 0;
        for (uint32_t i = 0; i < V; i++) {
            if (!oc_allowed(mask, mask_len, i)) continue;
            float l = logits[i];
            if (penalty != 0.0f && seen[i]) l = l - penalty;
            c[n].v = l;
            c[n].i = i;
            n++;
        }
        if (n > 0) {
            uint32_t k = top_k < 1 ? 1 : top_k;
            if (k > n) k = n;
            qsort(c, n, sizeof(oc_cand), oc_cand_desc);
            const float t = temperature, top = c[0].v;
            float* w = (float*)malloc(sizeof(float) * k);
            float total = 0.0f;
            for (uint32_t j = 0; j < k; j++) w[j] = expf((c[j].v - top) / t);
            for (uint32_t j = 0; j < k; j++) total += w[j];
            /* the smallest prefix reaching top_p of the mass */
            float kept = 0.0f;
            uint32_t m = 0;
            for (uint32_t j = 0; j < k; j++) {
                kept += w[j];
                m++;
                if (kept >= top_p * total) break;
            }
            float r = oc_sampler_next_f32(state) * kept;
            pick = c[m - 1].i;
            for (uint32_t j = 0; j < m; j++) {
                r -= w[j];
                if (r <= 0.0f) {
                    pick = c[j].i;
                    break;
                }
            }
            free(w);
        }
        free(c);
    }
    if (presence_penalty != 0.0f) seen[pick] = 1;
    *token = pick;
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Model: graph order of kernels/src/model.rs:220-269. Layer i is full attention iff
 * (i + 1) % full_attention_every == 0 (model.rs:230). */

struct oc_state {
    oc_config c;
    int n_gdn, n_attn;
    float* conv;      /* [n_gdn][channels][K-1] */
    float* rec;       /* [n_gdn][H][dk][dv] */
    uint16_t* kc;     /* [n_attn][nkv][cap][hd] */
    uint16_t* vc;
    float *h, *xn, *proj, *mixed, *act;
};

static int is_attn(const oc_config* c, int i) { return (i + 1) % c->full_attention_every == 0; }
static size_t conv_floats(const oc_config* c) { return (size_t)(2 * c->gdn_heads * c->gdn_dk + c->gdn_heads * c->gdn_dv) * (c->conv_kernel - 1); }
static size_t rec_floats(const oc_config* c) { return (size_t)c->gdn_heads * c->gdn_dk * c->gdn_dv; }
static size_t kv_halves(const oc_config* c) { return (size_t)c->n_kv_heads * c->max_context * c->head_dim; }

size_t oc_state_size_floats(const oc_model* m) {
    int na = 0;
    for (int i = 0; i < m->c.layers; i++) na += is_attn(&m->c, i);
    int ng = m->c.layers - na;
    return (size_t)ng * (conv_floats(&m->c) + rec_floats(&m->c)) + (size_t)na * kv_halves(&m->c);
}

oc_state* oc_state_new(const oc_model* m) {
    oc_state* s = (oc_state*)calloc(1, sizeof(oc_state));
    s->c = m->c;
    for (int i = 0; i < m->c.layers; i++) s->n_attn += is_attn(&m->c, i);
    s->n_gdn = m->c.layers - s->n_attn;
    const oc_config* c = &m->c;
    s->conv = (float*)calloc((size_t)s->n_gdn * conv_floats(c) + 1, sizeof(float));
    s->rec = (float*)calloc((size_t)s->n_gdn * rec_floats(c) + 1, sizeof(float));
    s->kc = (uint16_t*)calloc((size_t)s->n_attn * kv_halves(c) + 1, sizeof(uint16_t));
    s->vc = (uint16_t*)calloc((size_t)s->n_attn * kv_halves(c) + 1, sizeof(uint16_t));
    size_t attn_proj = (size_t)2 * c->n_q_heads * c->head_dim + (size_t)2 * c->n_kv_heads * c->head_dim;
    size_t gdn_proj = (size_t)2 * c->gdn_heads * c->gdn_dk + (size_t)2 * c->gdn_heads * c->gdn_dv + 2 * (size_t)c->gdn_heads;
    size_t proj = attn_proj > gdn_proj ? attn_proj : gdn_proj;
    size_t mixed = (size_t)c->n_q_heads * c->head_dim;
    if ((size_t)c->gdn_heads * c->gdn_dv > mixed) mixed = (size_t)c->gdn_heads * c->gdn_dv;
    s->h = (float*)calloc((size_t)c->hidden, sizeof(float));
    s->xn = (float*)calloc((size_t)c->hidden, sizeof(float));
    s->proj = (float*)calloc(proj, sizeof(float));
    s->mixed = (float*)calloc(mixed, sizeof(float));
    s->act = (float*)calloc((size_t)c->intermediate, sizeof(float));
    return s;
}

void oc_state_free(oc_state* s) {
    if (!s) return;
    free(s->conv); free(s->rec); free(s->kc); free(s->vc);
    free(s->h); free(s->xn); free(s->proj); free(s->mixed); free(s->act);
    free(s);
}

/* Model::reset (model.rs:313-320): clear recurrent, conv and KV state. */
void oc_reset(oc_state* s) {
    const oc_config* c = &s->c;
    memset(s->conv, 0, sizeof(float) * (size_t)s->n_gdn * conv_floats(c));
    memset(s->rec, 0, sizeof(float) * (size_t)s->n_gdn * rec_floats(c));
    memset(s->kc, 0, sizeof(uint16_t) * (size_t)s->n_attn * kv_halves(c));
    memset(s->vc, 0, sizeof(uint16_t) * (size_t)s->n_attn * kv_halves(c));
}

void oc_copy_state(const oc_state* from, oc_state* to) {
    const oc_config* c = &from->c;
    memcpy(to->conv, from->conv, sizeof(float) * (size_t)from->n_gdn * conv_floats(c));
    memcpy(to->rec, from->rec, sizeof(float) * (size_t)from->n_gdn * rec_floats(c));
    memcpy(to->kc, from->kc, sizeof(uint16_t) * (size_t)from->n_attn * kv_halves(c));
    memcpy(to->vc, from->vc, sizeof(uint16_t) * (size_t)from->n_attn * kv_halves(c));
}

float* oc_state_recurrent(oc_state* s, int i) { return s->rec + (size_t)i * rec_floats(&s->c); }
float* oc_state_conv(oc_state* s, int i) { return s->conv + (size_t)i * conv_floats(&s->c); }
uint16_t* oc_state_kcache(oc_state* s, int i) { return s->kc + (size_t)i * kv_halves(&s->c); }
uint16_t* oc_state_vcache(oc_state* s, int i) { return s->vc + (size_t)i * kv_halves(&s->c); }

/* The layers for one token at `pos`, leaving the residual stream in s->h. */
static void run_layers(const oc_model* m, oc_state* s, uint32_t token, uint32_t pos) {
    const oc_config* c = &m->c;
    oc_embed(&m->embed, token, s->h);
    int gi = 0, ai = 0;
    for (int i = 0; i < c->layers; i++) {
        const oc_layer* L = &m->layers[i];
        oc_rmsnorm(s->h, L->input_norm, s->xn, c->hidden, c->eps);
        oc_gemv(&L->mixer_in, s->xn, s->proj, OC_STORE);
        if (is_attn(c, i)) {
            oc_attention_step(c, s->proj, oc_state_kcache(s, ai), oc_state_vcache(s, ai), pos, s->mixed, L->attn_norms);
            ai++;
        } else {
            oc_gdn_step(c, s->proj, oc_state_conv(s, gi), L->conv_w, oc_state_recurrent(s, gi), s->mixed, L->gdn_params);
            gi++;
        }
        oc_gemv(&L->mixer_out, s->mixed, s->h, OC_ACCUMULATE);
        oc_rmsnorm(s->h, L->post_norm, s->xn, c->hidden, c->eps);
        oc_gemv(&L->gate_up, s->xn, s->act, OC_SWIGLU);
        oc_gemv(&L->down, s->act, s->h, OC_ACCUMULATE);
    }
}

static void head(const oc_model* m, oc_state* s, float* logits) {
    oc_rmsnorm(s->h, m->final_norm, s->xn, m->c.hidden, m->c.eps);
    oc_gemv(&m->lm_head, s->xn, logits, OC_STORE);
}

/* One token through the whole graph (Model::step, model.rs:380-392): logits for the next token. */
void oc_token(const oc_model* m, oc_state* s, uint32_t token, uint32_t pos, float* logits) {
    run_layers(m, s, token, pos);
    if (logits) head(m, s, logits);
}

/* oc_gemv for n tokens at once: y[t*ys + r] from x[t*xs ...] for t < n. Within one projection
 * the tokens of a prompt are independent, so each matrix row is dequantised once per block of
 * kTokBlock tokens and applied to all of them. Every (row, token) result is computed with the
 * operations of oc_gemv (dot_row's sum in column order, the same epilogue expression), so the
 * outputs are bitwise those of calling oc_gemv once per token. */
enum { kTokBlock = 32 };

static void dot_tokens(const oc_mat* m, int row, const float* xt, float* scratch, real* acc) {
    oc_dequant_row(m, row, scratch);
    for (int j = 0; j < kTokBlock; j++) acc[j] = 0;
    for (int c = 0; c < m->k; c++) {
        const real w = (real)scratch[c];
        const float* xc = xt + (size_t)c * kTokBlock;
        for (int j = 0; j < kTokBlock; j++) acc[j] += w * (real)xc[j];
    }
}

static void gemv_tokens(const oc_mat* m, const float* x, size_t xs, float* y, size_t ys, int n, int epilogue) {
    const int out_rows = epilogue == OC_SWIGLU ? m->rows / 2 : m->rows;
    const int k = m->k;
    float* xt = (float*)malloc(sizeof(float) * (size_t)k * kTokBlock);
    for (int t0 = 0; t0 < n; t0 += kTokBlock) {
        const int nt = n - t0 < kTokBlock ? n - t0 : kTokBlock;
        for (int c = 0; c < k; c++)
            for (int j = 0; j < kTokBlock; j++) xt[(size_t)c * kTokBlock + j] = j < nt ? x[(size_t)(t0 + j) * xs + c] : 0.0f;
#pragma omp parallel
        {
            float* scratch = (float*)malloc(sizeof(float) * (size_t)k);
            real a[kTokBlock], u[kTokBlock];
#pragma omp for schedule(static)
            for (int r = 0; r < out_rows; r++) {
                dot_tokens(m, r, xt, scratch, a);
                if (epilogue == OC_SWIGLU) dot_tokens(m, r + out_rows, xt, scratch, u);
                for (int j = 0; j < nt; j++) {
                    float* yr = y + (size_t)(t0 + j) * ys + r;
                    if (epilogue == OC_STORE) *yr = (float)a[j];
                    else if (epilogue == OC_ACCUMULATE) *yr = (float)((real)*yr + a[j]);
                    else *yr = (float)(r_silu(a[j]) * u[j]);
                }
            }
            free(scratch);
        }
    }
    free(xt);
}

/* The layers for tokens ids[0..n) at positions start.., layer by layer: every projection runs over
 * all n tokens at once (gemv_tokens), the mixers (conv + delta rule, attention) token by token in
 * order. Each token sees exactly the operations of run_layers, so the state and the last token's
 * residual stream (left in s->h) are bitwise those of n run_layers calls. */
static void run_layers_tokens(const oc_model* m, oc_state* s, const uint32_t* ids, int n, uint32_t start) {
    const oc_config* c = &m->c;
    const size_t H = (size_t)c->hidden;
    const size_t attn_proj = (size_t)2 * c->n_q_heads * c->head_dim + (size_t)2 * c->n_kv_heads * c->head_dim;
    const size_t gdn_proj = (size_t)2 * c->gdn_heads * c->gdn_dk + (size_t)2 * c->gdn_heads * c->gdn_dv + 2 * (size_t)c->gdn_heads;
    const size_t P = attn_proj > gdn_proj ? attn_proj : gdn_proj;
    size_t MX = (size_t)c->n_q_heads * c->head_dim;
    if ((size_t)c->gdn_heads * c->gdn_dv > MX) MX = (size_t)c->gdn_heads * c->gdn_dv;
    const size_t I = (size_t)c->intermediate;
    float* h = (float*)malloc(sizeof(float) * n * H);
    float* xn = (float*)malloc(sizeof(float) * n * H);
    float* proj = (float*)malloc(sizeof(float) * n * P);
    float* mixed = (float*)malloc(sizeof(float) * n * MX);
    float* act = (float*)malloc(sizeof(float) * n * I);
    for (int t = 0; t < n; t++) oc_embed(&m->embed, ids[t], h + t * H);
    int gi = 0, ai = 0;
    for (int i = 0; i < c->layers; i++) {
        const oc_layer* L = &m->layers[i];
        for (int t = 0; t < n; t++) oc_rmsnorm(h + t * H, L->input_norm, xn + t * H, c->hidden, c->eps);
        gemv_tokens(&L->mixer_in, xn, H, proj, P, n, OC_STORE);
        if (is_attn(c, i)) {
            for (int t = 0; t < n; t++)
                oc_attention_step(c, proj + t * P, oc_state_kcache(s, ai), oc_state_vcache(s, ai), start + (uint32_t)t,
                                  mixed + t * MX, L->attn_norms);
            ai++;
        } else {
            for (int t = 0; t < n; t++)
                oc_gdn_step(c, proj + t * P, oc_state_conv(s, gi), L->conv_w, oc_state_recurrent(s, gi), mixed + t * MX,
                            L->gdn_params);
            gi++;
        }
        gemv_tokens(&L->mixer_out, mixed, MX, h, H, n, OC_ACCUMULATE);
        for (int t = 0; t < n; t++) oc_rmsnorm(h + t * H, L->post_norm, xn + t * H, c->hidden, c->eps);
        gemv_tokens(&L->gate_up, xn, H, act, I, n, OC_SWIGLU);
        gemv_tokens(&L->down, act, I, h, H, n, OC_ACCUMULATE);
    }
    memcpy(s->h, h + (size_t)(n - 1) * H, sizeof(float) * H);
    free(h); free(xn); free(proj); free(mixed); free(act);
}

/* Model::prefill_chunk (model.rs:349-372): the tokens continue the state at `start`; with
 * finish_logits, the logits after the last one. It leaves the same state as feeding the tokens
 * one at a time (model.rs:337-338): the oracle runs them layer by layer in blocks of up to 512
 * tokens with exactly the arithmetic of oc_token (run_layers_tokens). */
void oc_prefill_chunk(const oc_model* m, oc_state* s, const uint32_t* ids, int n, uint32_t start,
                      int finish_logits, float* logits) {
    for (int i = 0; i < n; i += 512) {
        const int nb = n - i < 512 ? n - i : 512;
        run_layers_tokens(m, s, ids + i, nb, start + (uint32_t)i);
    }
    if (n > 0 && finish_logits && logits) head(m, s, logits);
}

int oc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
