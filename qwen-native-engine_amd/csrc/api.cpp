// extern "C" boundary (include/qne.h): every call catches, maps the error to a return code and
// keeps the message for qne_last_error().
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <utility>
#include <vector>

#include "../../include/qne.h"
#include "batch.hpp"
#include "sample.hpp"
#include "error.hpp"
#include "hip_util.hpp"
#include "index.hpp"
#include "kernels/launch.hpp"
#include "model.hpp"

struct qne_model {
    qne::Model* m;
    int batches;  // live qne_batch objects that use this model's weights
};

struct qne_batch {
    qne::BatchDecoder* b;
    qne_model* owner;
};

namespace {
thread_local std::string g_last_error;

template <typename F>
int guard(F&& f) {
    try {
        f();
        g_last_error.clear();
        return QNE_OK;
    } catch (const qne::Error& e) {
        g_last_error = e.what();
        return e.code;
    } catch (const std::bad_alloc&) {
        g_last_error = "out of host memory";
        return QNE_EDEVICE;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return QNE_EINVAL;
    } catch (...) {
        g_last_error = "unknown error";
        return QNE_EINVAL;
    }
}

qne::Model& model(qne_model* m) {
    if (!m || !m->m) throw qne::Error(QNE_EINVAL, "null model handle");
    return *m->m;
}

void need(bool ok, const char* what) {
    if (!ok) throw qne::Error(QNE_EINVAL, what);
}

void check_launch() { qne::hip_check(hipGetLastError(), "kernel launch"); }

// Scratch of the kernel-level entry points (slot 0: paged-attention partials, slot 1: GEMM split
// partials, slot 2: the chunk operands of the WY delta rule), kept per device and grown on demand (held until the process ends), so that a call
// allocates only when it needs more than any call before it on that device. Calls of one entry
// point that overlap on one device share it.
enum { kWsAttention = 0, kWsGemm = 1, kWsGdn = 2, kWsSlots = 3 };
float* workspace(int slot, size_t bytes) {
    static std::mutex mu;
    static std::vector<std::pair<void*, size_t>> per_dev;
    int dev = 0;
    QNE_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    const size_t i = (size_t)dev * kWsSlots + slot;
    if (per_dev.size() <= i) per_dev.resize(i + 1, {nullptr, 0});
    auto& w = per_dev[i];
    if (w.second < bytes) {
        QNE_HIP(hipDeviceSynchronize());  // a smaller buffer may still be in use by an earlier call
        if (w.first) (void)hipFree(w.first);
        w.first = nullptr;
        w.second = 0;
        QNE_HIP(hipMalloc(&w.first, bytes));
        w.second = bytes;
    }
    return (float*)w.first;
}
}  // namespace

extern "C" {

const char* qne_last_error(void) { return g_last_error.c_str(); }

int qne_model_load(const char* index_json, size_t index_len, const void* weights, size_t weights_len,
                   const char* options_json, int allow_f16, qne_model** out) {
    (void)allow_f16;
    return guard([&] {
        need(index_json && out, "null argument");
        need(weights || weights_len == 0, "null weights");
        *out = nullptr;
        // Validate everything before any device work (model.rs:172-174).
        qne::ModelIndex ix = qne::parse_index(index_json, index_len, weights_len);
        qne::LoadOptions opt = qne::parse_options(options_json);
        qne::Model* m = new qne::Model(ix, (const uint8_t*)weights, weights_len, opt);
        *out = new qne_model{m, 0};
    });
}

int qne_model_free(qne_model* m) {
    return guard([&] {
        if (!m) return;
        need(m->batches == 0, "the model still has live batches (free them first)");
        delete m->m;
        delete m;
    });
}

int qne_reset(qne_model* m) { return guard([&] { model(m).reset(); }); }

int qne_prefill(qne_model* m, const uint32_t* ids, size_t n) {
    return guard([&] {
        need(ids || n == 0, "null ids");
        model(m).prefill(ids, n);
    });
}

int qne_prefill_chunk(qne_model* m, const uint32_t* ids, size_t n, uint32_t start, int finish_logits) {
    return guard([&] {
        need(ids || n == 0, "null ids");
        model(m).prefill_chunk(ids, n, start, finish_logits != 0);
    });
}

int qne_logits(qne_model* m, float* out, size_t cap) {
    return guard([&] {
        need(out != nullptr, "null output");
        model(m).logits(out, cap);
    });
}

int qne_step(qne_model* m, uint32_t token, uint32_t pos, float* out, size_t cap) {
    return guard([&] {
        need(out != nullptr, "null output");
        model(m).step(token, pos, out, cap);
    });
}

int qne_step_device(qne_model* m, uint32_t token, uint32_t pos) {
    return guard([&] { model(m).step_device(token, pos); });
}

int qne_logits_device(qne_model* m, const float** out) {
    return guard([&] {
        need(out != nullptr, "null output");
        *out = model(m).device_logits();
    });
}

int qne_snapshot(qne_model* m) { return guard([&] { model(m).snapshot(); }); }
int qne_restore(qne_model* m) { return guard([&] { model(m).restore(); }); }

int qne_last_token(qne_model* m, uint32_t* token, uint32_t* next_pos) {
    return guard([&] {
        need(token && next_pos, "null output");
        model(m).last_token(token, next_pos);
    });
}

int qne_decode(qne_model* m, size_t n, uint32_t window, const uint32_t* stop, size_t nstop, uint32_t* out, size_t cap,
               size_t* len) {
    return guard([&] {
        need(len != nullptr && (out || n == 0), "null output");
        need(stop || nstop == 0, "null stop list");
        *len = model(m).decode(n, window, stop, nstop, out, cap);
    });
}

int qne_decode_ids(qne_model* m, size_t n, uint32_t window, const uint32_t* stop, size_t nstop, uint32_t* out,
                   size_t cap, size_t* len) {
    return guard([&] {
        need(len != nullptr && (out || n == 0), "null output");
        need(stop || nstop == 0, "null stop list");
        *len = model(m).decode_ids(n, window, stop, nstop, out, cap);
    });
}

int qne_dispatches_per_token(qne_model* m, size_t* out) {
    return guard([&] {
        need(out != nullptr, "null output");
        *out = model(m).dispatches_per_token();
    });
}

int qne_adapter(qne_model* m, char* buf, size_t cap) {
    return guard([&] {
        need(buf && cap > 0, "null output");
        const std::string& a = model(m).adapter();
        need(cap > a.size(), "buffer too small");
        std::memcpy(buf, a.c_str(), a.size() + 1);
    });
}

int qne_vocab(qne_model* m, uint32_t* out) {
    return guard([&] {
        need(out != nullptr, "null output");
        *out = model(m).vocab();
    });
}

int qne_max_context(qne_model* m, uint32_t* out) {
    return guard([&] {
        need(out != nullptr, "null output");
        *out = model(m).max_context();
    });
}

int qne_profile_token(qne_model* m, double* ms) {
    return guard([&] {
        need(ms != nullptr, "null output");
        *ms = model(m).profile_token();
    });
}

int qne_profile_token_json(qne_model* m, char* buf, size_t cap) {
    return guard([&] {
        need(buf != nullptr, "null output");
        const std::string j = model(m).profile_token_json();
        if (j.size() + 1 > cap) throw qne::Error(QNE_EINVAL, "buffer too small: need " + std::to_string(j.size() + 1));
        std::memcpy(buf, j.c_str(), j.size() + 1);
    });
}

int qne_last_decode_timing(qne_model* m, double* ms, size_t* steps) {
    return guard([&] {
        need(ms && steps, "null output");
        model(m).last_decode_timing(ms, steps);
    });
}

// ---- kernel-level entry points ----

int qne_gemv(int kind, const void* w, const void* sz, int rows, int k, int group, const float* x, const float* norm,
             float eps, float* y, int epilogue, void* stream) {
    return guard([&] {
        need(kind == QNE_MAT_F16 || kind == QNE_MAT_Q4, "unknown matrix kind");
        need(w && x && y && rows > 0, "null or empty argument");
        need(kind == QNE_MAT_F16 || sz, "q4 needs sz");
        need(epilogue >= QNE_EPI_STORE && epilogue <= QNE_EPI_SWIGLU, "unknown epilogue");
        need(epilogue != QNE_EPI_SWIGLU || rows % 2 == 0, "SwiGlu needs an even row count");
        need(qne::gemv_k_supported(k), "unsupported k");
        need(kind == QNE_MAT_F16 || group == 32 || group == 64 || group == 128, "unsupported group");
        qne::ArgmaxOut none;
        if (!qne::launch_gemv(kind, w, (const uint32_t*)sz, rows, k, group, x, norm, eps, y, epilogue, none,
                              (hipStream_t)stream))
            throw qne::Error(QNE_EINVAL, "no kernel for this shape");
        check_launch();
    });
}

int qne_pack_sz_q4g(const uint16_t* scales, const uint16_t* zeros, size_t n, uint16_t* sz) {
    return guard([&] {
        need(scales && zeros && sz, "null argument");
        for (size_t i = 0; i < n; i++) {
            sz[2 * i] = scales[i];
            sz[2 * i + 1] = zeros[i];
        }
    });
}

int qne_gdn_step(const float* q, const float* k, const float* v, const float* beta, const float* g, float* state,
                 float* out, int batch, int heads, void* stream) {
    return guard([&] {
        need(q && k && v && beta && g && state && out, "null argument");
        need(batch > 0 && heads > 0 && batch <= 65535 && heads <= 65535, "bad batch or heads");
        qne::launch_delta_rule(q, k, v, beta, g, state, out, batch, heads, (hipStream_t)stream);
        check_launch();
    });
}

// From this many tokens on, qne_gdn_prefill_chunked runs the chunk-64 WY form; shorter calls run
// the token-by-token recurrence.
constexpr int kWyMinTokens = 64;

int qne_gdn_prefill_chunked(const float* q, const float* k, const float* v, const float* beta, const float* g,
                            float* state, float* out, int batch, int tokens, int heads, void* stream) {
    return guard([&] {
        need(q && k && v && beta && g && state && out, "null argument");
        need(batch > 0 && heads > 0 && tokens > 0 && batch <= 65535 && heads <= 65535, "bad sizes");
        if (tokens >= kWyMinTokens) {
            float* ws = workspace(kWsGdn, qne::wy_workspace_bytes(batch, tokens, heads));
            qne::launch_delta_rule_wy(q, k, v, beta, g, state, out, batch, tokens, heads, ws, (hipStream_t)stream);
        } else {
            qne::launch_delta_rule_chunked(q, k, v, beta, g, state, out, batch, tokens, heads, (hipStream_t)stream);
        }
        check_launch();
    });
}

int qne_paged_attn_decode(const float* q, const float* k_new, const float* v_new, void* k_pool, void* v_pool,
                          const int32_t* block_table, int max_blocks, const int32_t* ctx, float* out, int batch,
                          int nq, int nkv, void* stream) {
    return guard([&] {
        need(q && k_new && v_new && k_pool && v_pool && block_table && ctx && out, "null argument");
        need(batch > 0 && batch <= 65535 && nkv > 0 && nq % nkv == 0, "bad batch or heads");
        const int G = nq / nkv;
        need(G == 1 || G == 2 || G == 4, "nq/nkv must be 1, 2 or 4");
        need(max_blocks > 0, "max_blocks must be positive");
        // Split-context partials: about 1024 4-wave workgroups (4 per CU). Each wave keeps a whole
        // 16-position block (16 KB of K and V) in flight, so longer splits beat more workgroups
        // (measured for 64 sequences of mean context 2213: 4.75 / 4.66 / 4.40 / 3.82 TB/s at
        // 1024 / 2048 / 4096 / 8192 workgroups).
        int splits = (1024 + nkv * batch - 1) / (nkv * batch);
        if (splits < 1) splits = 1;
        if (splits > max_blocks) splits = max_blocks;
        const size_t parts = (size_t)batch * nkv * splits * G;
        hipStream_t st = (hipStream_t)stream;
        float* ws = workspace(kWsAttention, parts * 258 * 4 + (size_t)batch * 4);
        qne::launch_paged_attn(q, k_new, v_new, (uint16_t*)k_pool, (uint16_t*)v_pool, block_table, max_blocks, ctx,
                               out, batch, nq, nkv, ws, ws + parts * 2, splits, st, (int32_t*)(ws + parts * 258));
        check_launch();
        // the null stream keeps the call synchronous; on a caller's stream it is ordered like a kernel
        if (!stream) qne::hip_check(hipStreamSynchronize(st), "paged attention");
    });
}

int qne_paged_attn_decode_noalloc(const float* q, const float* k_new, const float* v_new, void* k_pool, void* v_pool,
                                  const int32_t* block_table, int max_blocks, const int32_t* ctx, float* out, int batch,
                                  int nq, int nkv, void* stream) {
    return guard([&] {
        need(q && k_new && v_new && k_pool && v_pool && block_table && ctx && out, "null argument");
        need(batch > 0 && batch <= 65535 && nkv > 0 && nq % nkv == 0, "bad batch or heads");
        const int G = nq / nkv;
        need(G == 1 || G == 2 || G == 4, "nq/nkv must be 1, 2 or 4");
        need(max_blocks > 0, "max_blocks must be positive");
        // the same split count as qne_paged_attn_decode, so both give the same results
        int splits = (1024 + nkv * batch - 1) / (nkv * batch);
        if (splits < 1) splits = 1;
        if (splits > max_blocks) splits = max_blocks;
        const size_t parts = (size_t)batch * nkv * splits * G;
        const size_t bytes = parts * 258 * 4 + (size_t)batch * 4;  // partials, then the sequences' order
        if (bytes > qne::kNoAllocScratchBytes)
            throw qne::Error(QNE_EINVAL, "qne_paged_attn_decode_noalloc: this call needs " + std::to_string(bytes) +
                                             " bytes of scratch (split partials and the sequences' order); its fixed scratch holds " +
                                             std::to_string(qne::kNoAllocScratchBytes) + " (use qne_paged_attn_decode)");
        float* ws = qne::noalloc_scratch();
        hipStream_t st = (hipStream_t)stream;
        qne::launch_paged_attn(q, k_new, v_new, (uint16_t*)k_pool, (uint16_t*)v_pool, block_table, max_blocks, ctx,
                               out, batch, nq, nkv, ws, ws + parts * 2, splits, st, (int32_t*)(ws + parts * 258));
        check_launch();
        if (!stream) qne::hip_check(hipStreamSynchronize(st), "paged attention");
    });
}

int qne_gemm(int kind, const void* w, const void* sz, int rows, int k, int group, const float* x, int x_stride, int m,
             const float* norm, float eps, float* y, int y_stride, int epilogue, void* stream) {
    return guard([&] {
        need(kind == QNE_MAT_F16 || kind == QNE_MAT_Q4, "unknown matrix kind");
        need(w && x && y && rows > 0, "null or empty argument");
        need(kind == QNE_MAT_F16 || sz, "q4 needs sz");
        need(epilogue >= QNE_EPI_STORE && epilogue <= QNE_EPI_SWIGLU, "unknown epilogue");
        need(epilogue != QNE_EPI_SWIGLU || rows % 2 == 0, "SwiGlu needs an even row count");
        need(qne::gemm_shape_ok(kind, rows, k, group, m), "unsupported shape (m 1..2048, k a multiple of 64, q4 group a multiple of 64)");
        const int n_out = epilogue == QNE_EPI_SWIGLU ? rows / 2 : rows;
        need(x_stride >= k && x_stride % 4 == 0, "x_stride must be >= k and a multiple of 4");
        need(y_stride >= n_out, "y_stride must be >= the output count");
        qne::GemmArgs a;
        a.x = x;
        a.x_stride = x_stride;
        a.m = m;
        a.gain = norm;
        a.eps = eps;
        a.kind = kind;
        a.W = w;
        a.SZ = (const uint32_t*)sz;
        a.N = rows;
        a.K = k;
        a.group = kind == QNE_MAT_Q4 ? group : 64;
        a.splits = qne::gemm_splits(kind, rows, k, a.group);
        a.epi = epilogue;
        a.y = y;
        a.y_stride = y_stride;
        a.n_out = n_out;
        const size_t part = (size_t)a.splits * ((m + 63) / 64 * 64) * rows;
        const size_t frag = (qne::gemm_frag_bytes(k, m) + 255) / 256 * 256;
        const size_t szt = kind == QNE_MAT_Q4 ? qne::tile_sz_words(rows, k / a.group) : 0;
        float* ws = workspace(kWsGemm, part * 4 + frag + szt * 4);
        a.part = ws;
        a.frag = (uint8_t*)(ws + part);
        hipStream_t st = (hipStream_t)stream;
        if (szt) {  // the GEMM reads the words tile-major
            uint32_t* d = (uint32_t*)(a.frag + frag);
            qne::launch_tile_sz((const uint32_t*)sz, rows, k / a.group, d, st);
            a.SZT = d;
        }
        qne::launch_gemm(a, st);
        check_launch();
        if (!stream) qne::hip_check(hipStreamSynchronize(st), "gemm");
    });
}

int qne_stream_read(const void* data, size_t bytes, uint32_t* sink, uint32_t workgroups, void* stream) {
    return guard([&] {
        need(data && sink, "null argument");
        need(bytes > 0 && bytes % 16 == 0, "bytes must be a positive multiple of 16");
        need(workgroups >= 1 && workgroups <= 65536, "workgroups must be 1..65536");
        qne::launch_stream_read(data, bytes, sink, (int)workgroups, (hipStream_t)stream);
        check_launch();
    });
}

int qne_exchange_probe(uint64_t* buf, uint32_t n, uint32_t rounds, uint32_t workgroups, uint64_t* ctl, double* us_per_round) {
    return guard([&] {
        need(buf && ctl && us_per_round, "null argument");
        need(n >= 2 && n <= 6144 && n % 2 == 0, "n must be even and in 2..6144");
        need(rounds >= 3 && rounds <= (1u << 30), "rounds must be 3..2^30");
        need(workgroups >= 1 && workgroups <= 65536, "workgroups must be 1..65536");
        qne::hip_check(hipMemset(ctl, 0, 16), "exchange probe");
        qne::hip_check(qne::launch_exchange_probe(buf, (int)n, (int)rounds, (int)workgroups, (unsigned long long*)ctl,
                                                   (unsigned*)(ctl + 1), nullptr),
                       "exchange probe (cooperative launch: the workgroups must fit on the device at once)");
        // the probe ran on the null stream: wait for it alone, not for every stream of the device
        qne::hip_check(hipStreamSynchronize(nullptr), "exchange probe");
        uint64_t h[2] = {0, 0};
        qne::hip_check(hipMemcpy(h, ctl, sizeof h, hipMemcpyDeviceToHost), "exchange probe");
        if (h[1] & 0xFFFFFFFFull) throw qne::Error(QNE_EDEVICE, "exchange probe: a poll timed out");
        int dev = 0, khz = 0;
        qne::hip_check(hipGetDevice(&dev), "exchange probe");
        // the wall clock the probe's timestamps count is the current device's
        qne::hip_check(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev), "exchange probe");
        *us_per_round = khz > 0 ? (double)h[0] * 1000.0 / khz / (double)(rounds - 2) : 0.0;
    });
}

int qne_noop_dispatch(float* y, void* stream) {
    return guard([&] {
        need(y != nullptr, "null argument");
        qne::launch_noop(y, (hipStream_t)stream);
        check_launch();
    });
}

struct qne_sampler {
    qne::DeviceSampler* s;
};

int qne_sampler_create(float temperature, uint32_t top_k, float top_p, uint64_t seed, float presence_penalty,
                       uint32_t vocab, qne_sampler** out) {
    return guard([&] {
        need(out != nullptr, "null argument");
        *out = nullptr;
        qne::SamplingOptions o;
        o.temperature = temperature;
        o.top_k = top_k;
        o.top_p = top_p;
        o.seed = seed;
        o.presence_penalty = presence_penalty;
        qne::DeviceSampler* d = new qne::DeviceSampler(o, vocab);
        *out = new qne_sampler{d};
    });
}

int qne_sampler_free(qne_sampler* s) {
    return guard([&] {
        if (!s) return;
        delete s->s;
        delete s;
    });
}

int qne_sample(qne_sampler* s, const float* logits, const uint32_t* mask, uint32_t mask_len, uint32_t bias_token,
               float bias, uint32_t* token, void* stream) {
    return guard([&] {
        need(s && s->s && logits && token, "null argument");
        *token = s->s->sample(logits, mask, mask_len, bias_token, bias, (hipStream_t)stream);
    });
}

namespace {
qne::BatchDecoder& batch(qne_batch* b) {
    if (!b || !b->b) throw qne::Error(QNE_EINVAL, "null batch handle");
    return *b->b;
}
}  // namespace

int qne_batch_create(qne_model* m, uint32_t max_rows, uint32_t max_context, qne_batch** out) {
    return guard([&] {
        need(out != nullptr, "null argument");
        *out = nullptr;
        qne::BatchDecoder* b = new qne::BatchDecoder(model(m), (int)max_rows, (int)max_context);
        *out = new qne_batch{b, m};
        m->batches++;
    });
}

int qne_batch_free(qne_batch* b) {
    return guard([&] {
        if (!b) return;
        delete b->b;
        if (b->owner) b->owner->batches--;
        delete b;
    });
}

int qne_batch_admit(qne_batch* b, uint32_t row) { return guard([&] { batch(b).admit((int)row); }); }

int qne_batch_copy_row(qne_batch* dst, uint32_t row, qne_batch* src, uint32_t src_row) {
    return guard([&] { batch(dst).copy_row((int)row, batch(src), (int)src_row); });
}

int qne_batch_reset_row(qne_batch* b, uint32_t row, uint32_t token) {
    return guard([&] { batch(b).reset_row((int)row, token); });
}

int qne_batch_row_state(qne_batch* b, uint32_t n, uint32_t* tokens, uint32_t* pos) {
    return guard([&] { batch(b).row_state((int)n, tokens, pos); });
}

int qne_batch_step(qne_batch* b, uint32_t n, const uint32_t* tokens, uint32_t* next, float* logits, size_t logits_cap) {
    return guard([&] { batch(b).step((int)n, tokens, next, logits, logits_cap); });
}

int qne_batch_decode(qne_batch* b, uint32_t n, uint32_t steps, uint32_t* out, size_t cap) {
    return guard([&] { batch(b).decode((int)n, (int)steps, out, cap); });
}

int qne_batch_fill_synthetic(qne_batch* b, uint32_t n, const uint32_t* ctx, uint64_t seed) {
    return guard([&] {
        need(ctx != nullptr, "null ctx");
        batch(b).fill_synthetic((int)n, ctx, seed);
    });
}

int qne_batch_last_decode_timing(qne_batch* b, double* ms, size_t* steps) {
    return guard([&] {
        need(ms && steps, "null argument");
        *ms = batch(b).last_ms();
        *steps = batch(b).last_steps();
    });
}

}  // extern "C"
