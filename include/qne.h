/* qne: MI355X (gfx950) decode engine for the Qwen3.5 hybrid decoder.
 *
 * C ABI that replaces the `kernels` crate's `Model` (kernels/src/model.rs) of
 * arlinamid/qwen-native-engine. Plain pointers and sizes only. Every call returns 0 on success or a
 * negative QNE_E* code; qne_last_error() then holds a human-readable message (thread-local). No
 * exception and no allocation crosses the boundary except the opaque model handle, which only
 * qne_model_free releases. A model has a single owner: calls on one handle must not overlap.
 *
 * Every entry point cites the reference interface it replaces (file:line in the reference repo).
 */
#ifndef QNE_H
#define QNE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QNE_OK 0
#define QNE_EINVAL (-1)      /* bad argument (empty prompt, short buffer, ...) */
#define QNE_ECONTEXT (-2)    /* position or prompt beyond the KV-cache capacity */
#define QNE_ENOSNAPSHOT (-3) /* restore before snapshot */
#define QNE_EDEVICE (-4)     /* HIP error, no device, or device wait timeout */
#define QNE_EFORMAT (-5)     /* index.json / weights.bin rejected by validation */

typedef struct qne_model qne_model;

/* Message of the last failed call on this thread ("" if none). */
const char* qne_last_error(void);

/* Model::load(index_json, weights, tiles, allow_f16, dxc) -- kernels/src/model.rs:171.
 * Parses and validates index.json (format_version 1 or 2) against the weights blob before any
 * device work, then copies the tensors to HBM (tensors with the same (offset, bytes) are uploaded
 * once, model.rs:185-194). The caller may free `weights` after the call returns.
 * `options_json` (nullable) carries the reference's `tiles` argument and this library's flags;
 * recognised keys: "max_context" (default 4096, the reference's MAX_CONTEXT), "device" (HIP
 * ordinal, default 0), "engine" ("persistent" or "graph"), "prefill_graphs" (default true: each
 * qne_prefill_chunk pass replays a captured HIP graph; false launches the same kernels one by one,
 * for tools that trace kernel launches but not graph replays), "gdn_fusion" (default true: the
 * persistent decode kernel runs a GDN layer's in-projection and recurrent step as one phase where
 * the shapes allow; false keeps them two phases, with identical results), "mfma_gemv" (default
 * true: the persistent decode kernel's q4 GEMVs run on the int8 matrix cores, x as a 22-bit fixed
 * point per 64 columns; false runs them on the vector ALUs, the same results to f32 rounding),
 * "gemm_fusion" (default true: a qne_prefill_chunk GEMM with one split applies its SwiGLU or
 * residual add and stages the next GEMM's operand itself; false runs a separate reduce pass after
 * it, with identical results), "tiles" (a serialised ModelTiles, model.rs:90-98). A serialised ModelTiles may also be passed as the whole object. A tile profile
 * is validated like ModelTiles::validate (model.rs:101-109, called at model.rs:174, after the index
 * and before any device work): QNE_EINVAL "invalid kernel tile profile: Tile { ... }" for a tile the
 * reference rejects, or for a missing field. A valid profile changes nothing else: kernel shapes
 * here are chosen per matrix at load. `allow_f16` is accepted for signature parity. */
int qne_model_load(const char* index_json, size_t index_len, const void* weights, size_t weights_len,
                   const char* options_json, int allow_f16, qne_model** out);
/* drop(Model) */
int qne_model_free(qne_model* m);

/* Model::reset -- model.rs:314. Zeroes recurrent, conv and KV state. */
int qne_reset(qne_model* m);
/* Model::prefill -- model.rs:324. Token-by-token from position 0 with the full graph.
 * QNE_EINVAL if n == 0, QNE_ECONTEXT if n >= max_context. */
int qne_prefill(qne_model* m, const uint32_t* ids, size_t n);
/* Model::prefill_chunk -- model.rs:349 (prefill_batched / prefill_from are start = 0 /
 * finish_logits = 1 forms, model.rs:339-346). Continues the state at `start`. With
 * finish_logits, computes the logits after the last id and the greedy pick (last_token).
 * Like the reference's batched prefill (batch.rs), it runs the prompt in passes of up to 2048
 * tokens (fewer if max_context is smaller) through the batched MFMA GEMM, the GDN recurrence in the chunk-64 WY form over whole
 * 64-position blocks; the state equals qne_prefill's to f32 rounding. Calls cut at multiples of 64
 * positions give the same bits as one call; other cuts agree to f32 rounding. Models whose shapes
 * the batched kernels do not take run it token by token.
 * QNE_EINVAL if n == 0, QNE_ECONTEXT if start + n >= max_context. */
int qne_prefill_chunk(qne_model* m, const uint32_t* ids, size_t n, uint32_t start, int finish_logits);
/* Model::logits -- model.rs:374. Copies vocab floats; QNE_EINVAL if cap < vocab. */
int qne_logits(qne_model* m, float* out, size_t cap);
/* Model::step -- model.rs:380. Feeds `token` at `pos`, writes vocab logits; does not update the
 * greedy pick. QNE_ECONTEXT if pos >= max_context. */
int qne_step(qne_model* m, uint32_t token, uint32_t pos, float* out, size_t cap);
/* Model::step without the logits readback (the reference's step copies vocab floats to the host,
 * model.rs:388-391): the logits stay on the device, at qne_logits_device, for qne_sample. */
int qne_step_device(qne_model* m, uint32_t token, uint32_t pos);
/* The device address of the model's vocab logits (valid until qne_model_free; rewritten by
 * qne_step / qne_step_device / qne_prefill_chunk with finish_logits / qne_prefill). */
int qne_logits_device(qne_model* m, const float** out);
/* Model::snapshot / Model::restore -- model.rs:395, 406. restore: QNE_ENOSNAPSHOT before any
 * snapshot ("no snapshot taken"). */
int qne_snapshot(qne_model* m);
int qne_restore(qne_model* m);
/* Model::last_token -- model.rs:417: (greedy id, next position). */
int qne_last_token(qne_model* m, uint32_t* token, uint32_t* next_pos);
/* Model::decode -- model.rs:426-449. Greedy decode: out[0] = last_token().0, then submissions of
 * min(window, n - len) steps whose picks are fed back on the device. As in the reference, a
 * one-step submission appends its pick and a longer one appends that many u32::MAX (0xFFFFFFFF)
 * placeholders (model.rs:441-446); the loop continues while len < n and the LAST value appended is
 * not in `stop` (model.rs:433), so a stop id inside a window is not seen. *len = values written.
 * QNE_ECONTEXT ("context limit of ... tokens reached after ... generated tokens") if
 * next_pos + steps would exceed max_context. */
int qne_decode(qne_model* m, size_t n, uint32_t window, const uint32_t* stop, size_t nstop,
               uint32_t* out, size_t cap, size_t* len);
/* No counterpart in the reference (its decode reads back only the last pick of a window,
 * model.rs:439-446): the same loop with every step's pick appended on the device, so every id of
 * every window is returned, ending after the first id found in `stop` (with window > 1 the state
 * may have advanced past it, as in the reference). For callers that want a window's ids without a
 * host round trip per token. Same errors as qne_decode. */
int qne_decode_ids(qne_model* m, size_t n, uint32_t window, const uint32_t* stop, size_t nstop,
                   uint32_t* out, size_t cap, size_t* len);
/* Model::dispatches_per_token -- model.rs:309 (kernel launches per decode token). */
int qne_dispatches_per_token(qne_model* m, size_t* out);
/* Model.adapter -- model.rs:167: device name, written NUL-terminated into buf. */
int qne_adapter(qne_model* m, char* buf, size_t cap);
/* VOCAB / shaders::MAX_CONTEXT -- kernels/src/lib.rs:21, kernels/src/shaders.rs:34. */
int qne_vocab(qne_model* m, uint32_t* out);
int qne_max_context(qne_model* m, uint32_t* out);
/* Model::profile_token -- model.rs:305: device time of one decode token in ms (event-timed,
 * consumes one greedy token like the reference). */
int qne_profile_token(qne_model* m, double* ms);
/* Model::profile_token -- model.rs:305 (per-label sums of Gpu::profile, kernels/src/lib.rs:366-396):
 * consumes one greedy token with the device timeline of the persistent decode kernel on and writes
 * NUL-terminated JSON into buf: "total_ms", "tick_ms" (the timestamp unit); "labels" (label -> span
 * ms, summed over layers), "compute_median_ms", "handover_median_ms", and "phases" (per phase:
 * label, span, compute median / max, hand-over median / max); "sub_step_names" and
 * "sub_steps_median_ms" (per label, the medians of each phase kind's sub-steps); "chain" (per
 * phase: label, input-staged and published median / max, in ms after the previous phase's last
 * publish); and per phase and workgroup, in ticks after that same instant (-1: not recorded),
 * "publish_ticks", "input_ticks" and "sub_ticks" (the 8 sub-step timestamps; slot 6 is -1), and
 * "places" (per workgroup: [XCC_ID, the HW_ID register]). Labels are gdn.* /
 * attn.* per layer phase and lm_head. QNE_EINVAL if cap is too small (the message names the size)
 * or the model was loaded with the graph engine. Diagnostic only; about 2 MB for the 2B model. */
int qne_profile_token_json(qne_model* m, char* buf, size_t cap);
/* Device time (HIP events on the model's stream) of the windows of the last qne_decode call, in
 * ms, and the number of decode steps they ran; the counterpart of timing a submission with
 * Gpu::time (kernels/src/lib.rs:439-446) without host overhead. */
int qne_last_decode_timing(qne_model* m, double* ms, size_t* steps);

/* ---- kernel-level entry points (device pointers; the reference exposes these only through its
 * in-binary checks, kernels/src/lib.rs:513-712, and microbenches, lib.rs:714-963) ---- */

/* Matrix encodings of a device matrix. */
#define QNE_MAT_F16 0 /* w: f16 [rows][k] */
#define QNE_MAT_Q4 1  /* w: u32 [rows][k/8] nibbles; sz: f16 pairs (scale, zero) [rows][k/group] */
#define QNE_EPI_STORE 0
#define QNE_EPI_ACCUMULATE 1
#define QNE_EPI_SWIGLU 2

/* gemv / gemv_f16 / gemv_split_f16 + split_reduce -- kernels/src/shaders.rs:45-376, launched by
 * Gpu::gemv, lib.rs:311-338. y = W x with the Store / Accumulate / SwiGlu epilogue. If `norm` is
 * non-null, x is first replaced by rmsnorm(x) * norm (shaders.rs:378-403 fused as a prologue).
 * `rows` counts matrix rows (2 * outputs for SwiGlu). stream = 0 is the null stream. */
int qne_gemv(int kind, const void* w, const void* sz, int rows, int k, int group, const float* x,
             const float* norm, float eps, float* y, int epilogue, void* stream);
/* Repack host q4 data into the device layout used by qne_gemv: sz[r][g] = (scale, zero). */
int qne_pack_sz_q4g(const uint16_t* scales, const uint16_t* zeros, size_t n, uint16_t* sz);
/* The gated delta rule alone (kernels/src/shaders.rs:498-512) for `batch` sequences x `heads`
 * heads, dk = dv = 128: per (b,h) q,k [dk], v [dv], beta, g -> state [dk][dv] updated in place,
 * out [dv] = S'^T q. q and k are used as given (already normalised). */
int qne_gdn_step(const float* q, const float* k, const float* v, const float* beta, const float* g,
                 float* state, float* out, int batch, int heads, void* stream);
/* The same recurrence over T tokens per sequence in one call (batch.rs:166-255 semantics: the
 * state after the call is the state after T sequential steps): q,k [B][T][H][dk], v/out
 * [B][T][H][dv], beta/g [B][T][H]. From T = 64 on it runs in the chunk-64 WY form on f32 MFMA
 * (every chunk's intra-chunk solve at once, then the state chained over chunks); shorter calls run
 * token by token with the state in registers. g must be in (0, 1]. The WY operands' scratch is kept
 * per device (grown when a call needs more): calls that overlap on one device must not be issued. */
int qne_gdn_prefill_chunked(const float* q, const float* k, const float* v, const float* beta,
                            const float* g, float* state, float* out, int batch, int tokens,
                            int heads, void* stream);
/* Paged KV decode for `batch` sequences (kernels/src/shaders.rs:522-633 generalised): appends one
 * token's k,v (f16) per sequence at position ctx[b], then attends q over positions 0..ctx[b].
 * Pools are [num_blocks][nkv][16][hd] f16; block_table [batch][max_blocks] (int32);
 * q/out [batch][nq][hd] f32, k_new/v_new [batch][nkv][hd] f32. hd = 256. scale = 1/sqrt(hd).
 * On the null stream the call returns when the result is ready; on another stream it is enqueued
 * there. The partials' scratch is kept per device (allocated on first use, grown when a call needs
 * more): calls that overlap on one device must not be issued. */
int qne_paged_attn_decode(const float* q, const float* k_new, const float* v_new, void* k_pool,
                          void* v_pool, const int32_t* block_table, int max_blocks,
                          const int32_t* ctx, float* out, int batch, int nq, int nkv,
                          void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): qne_paged_attn_decode with
 * the same arguments, kernels and results, whose split partials live in a fixed device array of
 * 8 MiB (8388608 bytes) per GPU, held by each GPU the library runs on until the process ends. The
 * call allocates nothing. QNE_EINVAL, before any device work, if batch * nkv * splits * (nq/nkv)
 * * 1032 bytes exceed that (splits = min(max_blocks, ceil(1024 / (nkv * batch)))): up to 64
 * sequences of 16 q / 4 kv heads always fit. Every call on one GPU shares that GPU's array, so
 * calls that overlap on one GPU (from several threads or streams) race and must not be issued. */
int qne_paged_attn_decode_noalloc(const float* q, const float* k_new, const float* v_new, void* k_pool,
                                  void* v_pool, const int32_t* block_table, int max_blocks,
                                  const int32_t* ctx, float* out, int batch, int nq, int nkv,
                                  void* stream);

/* The batched form of gemv for m (1..2048) rows of x: y[r] = W x[r] for r < m, on f16 MFMA (x split
 * into two f16 halves, so the products keep about 22 bits), with the same norm prologue and
 * epilogues as qne_gemv. The reference's 16-token GEMM (kernels/src/batch.rs:12-99, Gpu::gemm
 * lib.rs:341-347) generalised to M up to 2048 (in tiles of 64 rows). x rows at x + r * x_stride (x_stride >= k, a multiple of 4), y
 * rows at y + r * y_stride. k must be a multiple of 64 and q4 groups a multiple of 64. On the null
 * stream the call returns when the result is ready. The split partials' scratch is kept per device
 * (grown when a call needs more): calls that overlap on one device must not be issued. */
int qne_gemm(int kind, const void* w, const void* sz, int rows, int k, int group, const float* x,
             int x_stride, int m, const float* norm, float eps, float* y, int y_stride, int epilogue,
             void* stream);

/* ---- measurement kernels (the reference's probes) ----
 * The streaming-read probe: `bandwidth` (kernels/src/shaders.rs:701-717), run by bandwidth_probe
 * (kernels/src/lib.rs:837-863). Reads every 16-byte word of data[0..bytes) once (non-temporal)
 * and xor-folds it into sink[workgroups * 256] (one word per thread); the read bandwidth a GEMV
 * with no unpacking work could reach. bytes: a positive multiple of 16. Enqueued on `stream`. */
int qne_stream_read(const void* data, size_t bytes, uint32_t* sink, uint32_t workgroups, void* stream);
/* The dispatch-cost probe: `noop` (kernels/src/shaders.rs:719-729) timed by dispatch_cost
 * (kernels/src/lib.rs:718-724). One 64-thread workgroup adds 1 to y[0]. Enqueued on `stream`. */
int qne_noop_dispatch(float* y, void* stream);
/* The hand-over probe. No counterpart in the reference: it measures the cost the persistent decode
 * kernel pays at each of its phases, for its callers' and maintainers' capacity planning. buf holds
 * 2 n uint64 entries (zeroed before the first call), ctl 2 (device memory). `workgroups`
 * 512-thread workgroups, all resident at once (cooperative launch on the null stream), exchange
 * an n-value vector `rounds` times: each publishes its share as (value, tag) pairs with
 * agent-scope stores and polls the whole vector until every tag is the round's, as the decode
 * kernel's phases do. Waits for the device; *us_per_round = the mean round over rounds 3..rounds
 * (workgroup 0's wall clock). QNE_EDEVICE if a poll timed out. n even, 2..6144. */
int qne_exchange_probe(uint64_t* buf, uint32_t n, uint32_t rounds, uint32_t workgroups, uint64_t* ctl, double* us_per_round);

/* ---- token sampling on the device ----
 * src/sampling.rs Sampler (the agent's temperature + top-k + top-p sampler with presence penalty
 * and grammar mask) over logits in device memory: the O(vocab) part (checks, penalty, mask, greedy
 * pick or the top-k candidates) runs on the GPU, and only the pick or the k best (value, token)
 * pairs cross to the host, where the softmax weights, top-p prefix and xorshift draw run in the
 * reference's f32 arithmetic. The same logits, options and seed give the reference's tokens
 * (equal logits are taken in increasing token order; the reference leaves that order open). */
typedef struct qne_sampler qne_sampler;
/* Sampler::new (src/sampling.rs:42-46) for a vocabulary of `vocab` tokens, on the current device.
 * temperature <= 0: greedy. top_k 0 is taken as 1 (as the reference does); QNE_EINVAL above 1024. */
int qne_sampler_create(float temperature, uint32_t top_k, float top_p, uint64_t seed, float presence_penalty,
                       uint32_t vocab, qne_sampler** out);
int qne_sampler_free(qne_sampler* s);
/* Sampler::try_sample (src/sampling.rs:58-79) over `vocab` logits at device address `logits`
 * (e.g. qne_logits_device). `bias` is added to token `bias_token` first (the agent's tool-call
 * bias, agent/src/session.rs:399-404; bias_token >= vocab for none). mask: host bitset (bit i%32
 * of word i/32 allows token i; tokens >= mask_len are not allowed) or NULL. The presence penalty
 * applies only without a mask; the picked token is remembered for it either way. QNE_EINVAL
 * ("non-finite model logits" / "no finite token is allowed by the sampling mask") where the
 * reference fails closed. Returns when the token is known. */
int qne_sample(qne_sampler* s, const float* logits, const uint32_t* mask, uint32_t mask_len, uint32_t bias_token,
               float bias, uint32_t* token, void* stream);

/* ---- batched continuous decode ----
 * Up to 64 sequences ("rows") advance one token per step through one loaded model's weights, each
 * row with its own paged KV cache and recurrent state. The reference decodes one sequence at a
 * time (Model::step / decode, kernels/src/model.rs:372-449); a row here follows exactly that step.
 * A batch holds the model's weights: free every batch before the model. */
typedef struct qne_batch qne_batch;
int qne_batch_create(qne_model* m, uint32_t max_rows, uint32_t max_context, qne_batch** out);
int qne_batch_free(qne_batch* b);
/* Row `row` takes over the model's current sequence (after qne_prefill / qne_decode): its KV cache,
 * recurrent state and next (token, position) as qne_last_token reports them. */
int qne_batch_admit(qne_batch* b, uint32_t row);
/* Row `row` of dst takes over row `src_row` of src (a batch over the same model, possibly dst
 * itself): its KV cache, recurrent state and next (token, position). No counterpart in the
 * reference (one sequence per Model); it moves a sequence between batches of different sizes. For
 * batches created with the same max_context, a row's results do not depend on the batch it runs in
 * (bit for bit): the attention split count follows from max_context alone. */
int qne_batch_copy_row(qne_batch* dst, uint32_t row, qne_batch* src, uint32_t src_row);
/* Row `row` becomes an empty sequence at position 0 whose next token is `token`. */
int qne_batch_reset_row(qne_batch* b, uint32_t row, uint32_t token);
/* The next token and position of rows 0..n-1 (either pointer may be null). */
int qne_batch_row_state(qne_batch* b, uint32_t n, uint32_t* tokens, uint32_t* pos);
/* One step of rows 0..n-1. `tokens` (n entries, may be null) replaces the rows' next tokens first.
 * `next` (n entries, may be null) receives each row's greedy pick; `logits` (may be null) the
 * rows' logits, n * vocab floats. Each row's next token becomes its pick, its position advances. */
int qne_batch_step(qne_batch* b, uint32_t n, const uint32_t* tokens, uint32_t* next, float* logits,
                   size_t logits_cap);
/* `steps` greedy steps of rows 0..n-1 chained on the device; out[s * n + r] = pick of row r at
 * step s (out may be null). */
int qne_batch_decode(qne_batch* b, uint32_t n, uint32_t steps, uint32_t* out, size_t cap);
/* Benchmark set-up: rows 0..n-1 get pseudo-random KV contents and recurrent state, random next
 * tokens and positions ctx[r]. */
int qne_batch_fill_synthetic(qne_batch* b, uint32_t n, const uint32_t* ctx, uint64_t seed);
/* Device time (ms) and step count of the last qne_batch_decode. */
int qne_batch_last_decode_timing(qne_batch* b, double* ms, size_t* steps);

/* ---- synthetic weights (seeded generator used by the benches and tests) ---- */
/* value[i] = std * N(0,1) from SplitMix64 + Box-Muller on a counter keyed by (seed, stream). */
int qne_synth_normal_f32(uint64_t seed, uint64_t stream, size_t n, float std, float* out);
int qne_synth_normal_f16(uint64_t seed, uint64_t stream, size_t n, float std, uint16_t* out);
/* Asymmetric min/max int4 quantisation with f16 scale and f16 zero per `group` values along each
 * row: w ~ (q - z) * s. Writes nibbles (u32 [rows][k/8]), scales and zeros ([rows][k/group]). */
int qne_quantize_q4g(const float* w, size_t rows, size_t k, size_t group, uint32_t* q,
                     uint16_t* scales, uint16_t* zeros);

#ifdef __cplusplus
}
#endif
#endif
