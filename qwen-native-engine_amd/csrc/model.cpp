// Model: load, state, per-token graph and the prefill / step / decode protocol of
// kernels/src/model.rs, on HIP.
#include "model.hpp"
#include "prefill.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <map>
#include <thread>

#include "error.hpp"
#include "hip_util.hpp"
#include "json.hpp"
#include "kernels/decode.hpp"
#include "kernels/launch.hpp"

namespace qne {

void wait_stream(hipStream_t st, double timeout_s) {
    using clk = std::chrono::steady_clock;
    const auto start = clk::now();
    int spins = 0;
    while (true) {
        hipError_t e = hipStreamQuery(st);
        if (e == hipSuccess) return;
        if (e != hipErrorNotReady) hip_check(e, "hipStreamQuery");
        if (++spins > 2000) std::this_thread::sleep_for(std::chrono::microseconds(50));
        if (std::chrono::duration<double>(clk::now() - start).count() > timeout_s)
            throw Error(QNE_EDEVICE, "GPU wait failed: timed out after " + std::to_string((long long)timeout_s) + " s");
    }
}

// ModelTiles::validate (kernels/src/model.rs:101-109) on a serialised tile profile: each of the six
// matrix kinds names a GEMV tile {f16, tpr, rpw, rpt, splits} (kernels/src/lib.rs:40-49), and a
// profile the reference would reject is rejected with its message. The kernels here choose their
// own shapes per matrix, so a valid profile changes nothing else.
static void validate_tiles(const Json& t) {
    static const char* kKinds[] = {"gdn_in", "attn_in", "out", "gate_up", "down", "lm_head"};
    if (t.type != Json::Object) throw Error(QNE_EINVAL, "tiles: expected a ModelTiles object");
    for (const char* kind : kKinds) {
        if (!t.has(kind)) throw Error(QNE_EINVAL, std::string("tiles: missing field `") + kind + "`");
        const Json& v = t.at(kind);
        if (v.type != Json::Object) throw Error(QNE_EINVAL, std::string("tiles: ") + kind + " is not a Tile object");
        if (!v.has("f16") || v.at("f16").type != Json::Bool)
            throw Error(QNE_EINVAL, std::string("tiles: ") + kind + ": missing or non-boolean field `f16`");
        const bool f16 = v.at("f16").b;
        uint32_t f[4];
        static const char* kFields[] = {"tpr", "rpw", "rpt", "splits"};
        for (int i = 0; i < 4; i++) {
            if (!v.has(kFields[i]))
                throw Error(QNE_EINVAL, std::string("tiles: ") + kind + ": missing field `" + kFields[i] + "`");
            const Json& x = v.at(kFields[i]);
            if (x.type != Json::Number || x.num < 0 || x.num > 4294967295.0 || x.num != (double)(uint32_t)x.num)
                throw Error(QNE_EINVAL, std::string("tiles: ") + kind + ": `" + kFields[i] + "` is not a u32");
            f[i] = (uint32_t)x.num;
        }
        const uint32_t tpr = f[0], rpw = f[1], rpt = f[2], splits = f[3];
        auto in = [](uint32_t v, std::initializer_list<uint32_t> set) {
            for (uint32_t s : set)
                if (v == s) return true;
            return false;
        };
        const bool ok = in(tpr, {1, 2, 4, 8, 16, 32, 64}) && in(rpw, {2, 4, 8, 16, 32}) && in(rpt, {1, 2, 4, 8}) &&
                        in(splits, {1, 2, 4, 8}) && (uint64_t)tpr * rpw <= 256 && (f16 || (rpt == 1 && splits == 1));
        if (!ok)
            throw Error(QNE_EINVAL, "invalid kernel tile profile: Tile { f16: " + std::string(f16 ? "true" : "false") +
                                        ", tpr: " + std::to_string(tpr) + ", rpw: " + std::to_string(rpw) +
                                        ", rpt: " + std::to_string(rpt) + ", splits: " + std::to_string(splits) + " }");
    }
}

LoadOptions parse_options(const char* json) {
    LoadOptions o;
    if (!json || !*json) return o;
    Json j = Json::parse(json, std::strlen(json));
    if (j.type != Json::Object) throw Error(QNE_EINVAL, "options must be a JSON object");
    // The reference's `tiles` argument: a serialised ModelTiles, either as the whole options object
    // or under "tiles".
    if (j.has("tiles")) validate_tiles(j.at("tiles"));
    else if (j.has("gdn_in") || j.has("attn_in") || j.has("out") || j.has("gate_up") || j.has("down") ||
             j.has("lm_head"))
        validate_tiles(j);
    if (j.has("max_context")) {
        uint64_t v = j.at("max_context").u64("max_context");
        if (v < 16 || v > (1u << 22)) throw Error(QNE_EINVAL, "max_context must be 16..4194304");
        o.max_context = (int)v;
    }
    if (j.has("device")) o.device = (int)j.at("device").u64("device");
    if (j.has("engine")) {
        const std::string& e = j.at("engine").string();
        if (e != "graph" && e != "persistent") throw Error(QNE_EINVAL, "engine must be \"persistent\" or \"graph\"");
        o.graph_engine = e == "graph";
    }
    if (j.has("mfma_gemv")) {
        const Json& v = j.at("mfma_gemv");
        if (v.type != Json::Bool) throw Error(QNE_EINVAL, "mfma_gemv must be true or false");
        o.mfma_gemv = v.b;
    }
    if (j.has("gemm_fusion")) {
        const Json& v = j.at("gemm_fusion");
        if (v.type != Json::Bool) throw Error(QNE_EINVAL, "gemm_fusion must be true or false");
        o.gemm_fusion = v.b;
    }
    if (j.has("gdn_fusion")) {
        const Json& v = j.at("gdn_fusion");
        if (v.type != Json::Bool) throw Error(QNE_EINVAL, "gdn_fusion must be true or false");
        o.gdn_fusion = v.b;
    }
    if (j.has("prefill_graphs")) {
        const Json& v = j.at("prefill_graphs");
        if (v.type != Json::Bool) throw Error(QNE_EINVAL, "prefill_graphs must be true or false");
        o.prefill_graphs = v.b;
    }
    return o;
}

static float f16_to_f32_host(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, f = h & 0x3ffu, bits;
    if (e == 0) {
        float v = (float)f * 5.9604644775390625e-8f;
        return (h & 0x8000u) ? -v : v;
    }
    bits = e == 31 ? (sign | 0x7f800000u | (f << 13)) : (sign | ((e + 112u) << 23) | (f << 13));
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

static uint16_t small_int_to_f16(unsigned v) {  // exact for 0..15
    if (v == 0) return 0;
    int e = 0;
    while ((v >> (e + 1)) != 0) e++;
    unsigned frac = (v << (10 - e)) & 0x3ffu;
    return (uint16_t)(((unsigned)(e + 15) << 10) | frac);
}

void* Model::dalloc(size_t bytes) {
    void* p = nullptr;
    QNE_HIP(hipMalloc(&p, bytes ? bytes : 16));
    allocations_.push_back(p);
    return p;
}

Model::Model(const ModelIndex& ix, const uint8_t* weights, uint64_t /*wlen*/, const LoadOptions& opt)
    : cfg_(ix.cfg), max_context_(opt.max_context), device_(opt.device) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) throw Error(QNE_EDEVICE, "no GPU adapter");
    if (device_ >= count) throw Error(QNE_EDEVICE, "device ordinal out of range");
    QNE_HIP(hipSetDevice(device_));
    hipDeviceProp_t prop;
    QNE_HIP(hipGetDeviceProperties(&prop, device_));
    adapter_ = std::string(prop.name[0] ? prop.name : "AMD GPU") + " (" + prop.gcnArchName + ", " +
               std::to_string(prop.multiProcessorCount) + " CUs) via HIP";
    QNE_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    QNE_HIP(hipEventCreate(&ev_start_));
    QNE_HIP(hipEventCreate(&ev_stop_));
    persistent_ = !opt.graph_engine;
    prefill_graphs_ = opt.prefill_graphs;
    gdn_fusion_ = opt.gdn_fusion;
    mfma_gemv_ = opt.mfma_gemv;
    gemm_fusion_ = opt.gemm_fusion;
    try {
        upload(ix, weights);
        alloc_state();
        if (persistent_) setup_engine();
        else build_graphs();
    } catch (...) {
        release();
        throw;
    }
}

Model::~Model() { release(); }

void Model::release() {
    if (device_ >= 0) (void)hipSetDevice(device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    delete chunk_;
    chunk_ = nullptr;
    for (hipGraphExec_t g : {g_layers_, g_head_logits_, g_head_greedy_})
        if (g) (void)hipGraphExecDestroy(g);
    g_layers_ = g_head_logits_ = g_head_greedy_ = nullptr;
    if (ev_start_) (void)hipEventDestroy(ev_start_);
    if (ev_stop_) (void)hipEventDestroy(ev_stop_);
    ev_start_ = ev_stop_ = nullptr;
    for (void* p : allocations_) (void)hipFree(p);
    allocations_.clear();
    if (host_tok_) (void)hipHostFree(host_tok_);
    if (host_logits_) (void)hipHostFree(host_logits_);
    if (host_ids_) (void)hipHostFree(host_ids_);
    if (host_err_) (void)hipHostFree(host_err_);
    host_tok_ = nullptr; host_logits_ = nullptr; host_ids_ = nullptr; host_err_ = nullptr;
    delete (DecodeArgs*)engine_args_;
    engine_args_ = nullptr;
    if (stream_) (void)hipStreamDestroy(stream_);
    stream_ = nullptr;
}

// Copies every tensor to HBM once. Tensors with the same (offset, bytes) share one upload, as in
// model.rs:185-194 (tied embedding / LM head). q4 scales and zeros are interleaved per group.
void Model::upload(const ModelIndex& ix, const uint8_t* weights) {
    std::map<std::pair<uint64_t, uint64_t>, void*> seen;
    auto raw = [&](const TensorRef& t) -> void* {
        auto key = std::make_pair(t.offset, t.bytes);
        auto it = seen.find(key);
        if (it != seen.end()) return it->second;
        void* d = dalloc(t.bytes);
        QNE_HIP(hipMemcpy(d, weights + t.offset, t.bytes, hipMemcpyHostToDevice));
        seen[key] = d;
        return d;
    };
    std::map<std::pair<uint64_t, uint64_t>, std::pair<uint32_t*, uint32_t*>> seen_sz;
    auto mat = [&](const std::string& name) -> DevMat {
        const MatInfo& m = ix.mat(name);
        DevMat d;
        d.kind = m.kind;
        d.rows = m.rows;
        d.k = m.k;
        d.group = m.group ? m.group : 64;
        d.w = raw(m.w);
        if (m.kind == MAT_Q4) {
            auto key = std::make_pair(m.s.offset, m.z.offset);
            auto it = seen_sz.find(key);
            if (it != seen_sz.end()) {
                d.sz = it->second.first;
                d.szt = it->second.second;
            } else {
                const size_t groups_per_row = (size_t)m.k / m.group, n = (size_t)m.rows * groups_per_row;
                std::vector<uint32_t> sz(n);
                const uint16_t* s = (const uint16_t*)(weights + m.s.offset);
                for (size_t r = 0; r < (size_t)m.rows; r++) {
                    for (size_t g = 0; g < groups_per_row; g++) {
                        const size_t i = r * groups_per_row + g;
                        uint16_t z16;
                        if (m.zero_u4) {
                            const uint8_t* z = weights + m.z.offset + r * ((groups_per_row + 1) / 2);
                            z16 = small_int_to_f16((z[g / 2] >> (4 * (g % 2))) & 15u);
                        } else {
                            z16 = ((const uint16_t*)(weights + m.z.offset))[i];
                        }
                        uint16_t s16;
                        std::memcpy(&s16, s + i, 2);
                        sz[i] = (uint32_t)s16 | ((uint32_t)z16 << 16);
                    }
                }
                uint32_t* dsz = (uint32_t*)dalloc(n * 4);
                QNE_HIP(hipMemcpy(dsz, sz.data(), n * 4, hipMemcpyHostToDevice));
                const size_t tiles = ((size_t)m.rows + 31) / 32, nt = tiles * groups_per_row * 32;
                std::vector<uint32_t> szt(nt, 0u);
                for (size_t r = 0; r < (size_t)m.rows; r++)
                    for (size_t g = 0; g < groups_per_row; g++)
                        szt[((r / 32) * groups_per_row + g) * 32 + r % 32] = sz[r * groups_per_row + g];
                uint32_t* dszt = (uint32_t*)dalloc(nt * 4);
                QNE_HIP(hipMemcpy(dszt, szt.data(), nt * 4, hipMemcpyHostToDevice));
                seen_sz[key] = {dsz, dszt};
                d.sz = dsz;
                d.szt = dszt;
            }
        }
        return d;
    };
    embed_ = mat("embed");
    lm_head_ = mat("lm_head");
    final_norm_ = (const float*)raw(ix.tensor("final_norm"));
    layers_.resize(cfg_.layers);
    for (int i = 0; i < cfg_.layers; i++) {
        const std::string p = "layer" + std::to_string(i) + ".";
        DevLayer& L = layers_[i];
        L.attn = cfg_.is_attn(i);
        L.input_norm = (const float*)raw(ix.tensor(p + "input_norm"));
        L.post_norm = (const float*)raw(ix.tensor(p + "post_norm"));
        L.in = mat(p + "mixer_in");
        L.out = mat(p + "mixer_out");
        L.gate_up = mat(p + "gate_up");
        L.down = mat(p + "down");
        if (L.attn) {
            L.norms = (const float*)raw(ix.tensor(p + "attn_norms"));
        } else {
            L.conv_w = (const float*)raw(ix.tensor(p + "conv_w"));
            L.gdn_params = (const float*)raw(ix.tensor(p + "gdn_params"));
        }
    }
    (void)f16_to_f32_host;
}

void Model::alloc_state() {
    const ModelConfig& c = cfg_;
    // conv state: 3 values per channel at a 4-float stride (16-byte rows the decode kernel DMAs)
    const size_t conv_b = (size_t)c.conv_channels() * 4 * 4;
    const size_t rec_b = (size_t)c.gdn_heads * c.gdn_dk * c.gdn_dv * 4;
    const int blocks = (max_context_ + 15) / 16;
    const size_t pool_b = (size_t)blocks * c.n_kv_heads * 16 * c.head_dim * 2;
    size_t total = 0;
    for (const DevLayer& L : layers_) total += L.attn ? 2 * pool_b : conv_b + rec_b;
    state_bytes_ = total;
    state_ = dalloc(total);
    uint8_t* p = (uint8_t*)state_;
    for (DevLayer& L : layers_) {
        if (L.attn) {
            L.k_pool = (uint16_t*)p; p += pool_b;
            L.v_pool = (uint16_t*)p; p += pool_b;
        } else {
            L.conv_state = (float*)p; p += conv_b;
            L.rec = (float*)p; p += rec_b;
        }
    }
    QNE_HIP(hipMemset(state_, 0, state_bytes_));

    // Block table of the single sequence: a fixed permutation of the pool, so the decode path
    // always goes through the same paged addressing as batched serving.
    std::vector<int32_t> bt(blocks);
    for (int i = 0; i < blocks; i++) bt[i] = i;
    uint64_t x = 0x9E3779B97F4A7C15ull;
    for (int i = blocks - 1; i > 0; i--) {
        x ^= x << 13; x ^= x >> 7; x ^= x << 17;
        std::swap(bt[i], bt[x % (uint64_t)(i + 1)]);
    }
    block_table_ = (int32_t*)dalloc(blocks * 4);
    QNE_HIP(hipMemcpy(block_table_, bt.data(), blocks * 4, hipMemcpyHostToDevice));
    bt_host_ = bt;

    size_t proj = (size_t)std::max(c.attn_proj(), c.gdn_proj());
    size_t mixed = (size_t)std::max(c.attn_out(), c.gdn_out());
    h_ = (float*)dalloc((size_t)c.hidden * 4);
    proj_ = (float*)dalloc(proj * 4);
    mixed_ = (float*)dalloc(mixed * 4);
    act_ = (float*)dalloc((size_t)c.intermediate * 4);
    logits_ = (float*)dalloc((size_t)c.vocab * 4);
    qbuf_ = (float*)dalloc((size_t)c.n_q_heads * c.head_dim * 4);
    // split-context partials: about 256 workgroups per attention layer
    attn_splits_ = std::max(1, std::min(256 / c.n_kv_heads, (max_context_ + 15) / 16));
    const size_t G = (size_t)(c.n_q_heads / c.n_kv_heads);
    part_ml_ = (float*)dalloc((size_t)c.n_kv_heads * attn_splits_ * G * 2 * 4);
    part_acc_ = (float*)dalloc((size_t)c.n_kv_heads * attn_splits_ * G * c.head_dim * 4);
    am_val_ = (float*)dalloc(kArgmaxMaxBlocks * 4);
    am_idx_ = (uint32_t*)dalloc(kArgmaxMaxBlocks * 4);
    am_counter_ = (unsigned*)dalloc(64);
    QNE_HIP(hipMemset(am_counter_, 0, 64));
    tok_ = (uint32_t*)dalloc(16);
    tok_backup_ = (uint32_t*)dalloc(16);
    QNE_HIP(hipMemset(tok_, 0, 16));
    ids_ = (uint32_t*)dalloc((size_t)max_context_ * 4);
    out_ids_ = (uint32_t*)dalloc((size_t)max_context_ * 4);
    std::vector<float> inv((size_t)c.rope_dim / 2);
    for (int i = 0; i < c.rope_dim / 2; i++) inv[i] = (float)std::pow(c.rope_theta, -(double)(2 * i) / (double)c.rope_dim);
    inv_freq_ = (float*)dalloc(inv.size() * 4);
    QNE_HIP(hipMemcpy(inv_freq_, inv.data(), inv.size() * 4, hipMemcpyHostToDevice));
    QNE_HIP(hipHostMalloc((void**)&host_tok_, 64, hipHostMallocDefault));
    QNE_HIP(hipHostMalloc((void**)&host_logits_, (size_t)c.vocab * 4, hipHostMallocDefault));
    QNE_HIP(hipHostMalloc((void**)&host_ids_, (size_t)max_context_ * 4, hipHostMallocDefault));
}

static void gemv_or_throw(const DevMat& m, const float* x, const float* gain, float eps, float* y, int epi,
                          const ArgmaxOut& am, hipStream_t st) {
    if (!launch_gemv(m.kind, m.w, m.sz, m.rows, m.k, m.group, x, gain, eps, y, epi, am, st))
        throw Error(QNE_EFORMAT, "no GEMV kernel for k=" + std::to_string(m.k));
}

// One token through the layers (model.rs:220-262): the embedding row of tok[0], then per layer
// RMSNorm -> mixer_in -> GDN | attention -> mixer_out (+=) -> RMSNorm -> gate_up (SwiGLU) ->
// down (+=). The RMSNorms are fused into the GEMV that consumes them.
void Model::enqueue_layers() {
    const ModelConfig& c = cfg_;
    ArgmaxOut none;
    launch_embed(embed_.kind, embed_.w, embed_.sz, embed_.group, c.hidden, tok_, h_, stream_);
    launches_++;
    for (const DevLayer& L : layers_) {
        gemv_or_throw(L.in, h_, L.input_norm, c.eps, proj_, EPI_STORE, none, stream_);
        launches_++;
        if (L.attn) {
            AttnModelArgs a;
            a.proj = proj_; a.norms = L.norms; a.inv_freq = inv_freq_;
            a.k_pool = L.k_pool; a.v_pool = L.v_pool; a.block_table = block_table_; a.tok = tok_;
            a.qbuf = qbuf_; a.part_ml = part_ml_; a.part_acc = part_acc_; a.out = mixed_;
            a.nq = c.n_q_heads; a.nkv = c.n_kv_heads; a.rope_dim = c.rope_dim; a.splits = attn_splits_;
            a.max_blocks = (max_context_ + 15) / 16;
            launch_attention_model(a, stream_);
            launches_ += 3;
        } else {
            launch_gdn_decode(proj_, L.conv_state, L.conv_w, L.rec, mixed_, L.gdn_params, c.gdn_heads, stream_);
            launches_++;
        }
        gemv_or_throw(L.out, mixed_, nullptr, c.eps, h_, EPI_ACCUMULATE, none, stream_);
        gemv_or_throw(L.gate_up, h_, L.post_norm, c.eps, act_, EPI_SWIGLU, none, stream_);
        gemv_or_throw(L.down, act_, nullptr, c.eps, h_, EPI_ACCUMULATE, none, stream_);
        launches_ += 3;
    }
}

// Final RMSNorm + LM head (model.rs:264-269); `greedy` adds the device argmax that feeds tok.
void Model::enqueue_head(bool greedy) {
    ArgmaxOut am;
    if (greedy) {
        am.part_val = am_val_; am.part_idx = am_idx_; am.counter = am_counter_; am.tok = tok_;
        am.ids = out_ids_; am.ids_cap = (uint32_t)max_context_;
    }
    gemv_or_throw(lm_head_, h_, final_norm_, cfg_.eps, logits_, greedy ? EPI_ARGMAX : EPI_STORE, am, stream_);
    launches_++;
}

void Model::build_graphs() {
    auto capture = [&](auto&& body) -> hipGraphExec_t {
        hipGraph_t g = nullptr;
        hipGraphExec_t e = nullptr;
        QNE_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
        try {
            body();
        } catch (...) {
            (void)hipStreamEndCapture(stream_, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        QNE_HIP(hipStreamEndCapture(stream_, &g));
        QNE_HIP(hipGraphInstantiate(&e, g, nullptr, nullptr, 0));
        (void)hipGraphDestroy(g);
        return e;
    };
    launches_ = 0;
    // QNE_NO_GRAPH=1 launches the same kernels directly on the stream (for tracing tools that do
    // not follow graph launches).
    const char* ng = std::getenv("QNE_NO_GRAPH");
    if (ng && *ng && *ng != '0') {
        use_graphs_ = false;
        enqueue_layers();
        const size_t before = launches_;
        enqueue_head(true);
        dispatches_ = (before - 1) + (launches_ - before);
        QNE_HIP(hipStreamSynchronize(stream_));
        return;
    }
    g_layers_ = capture([&] { enqueue_layers(); });
    g_head_logits_ = capture([&] { enqueue_head(false); });
    const size_t before = launches_;
    g_head_greedy_ = capture([&] { enqueue_head(true); });
    dispatches_ = (before - 1) + (launches_ - before);  // layers + greedy head
    QNE_HIP(hipStreamSynchronize(stream_));
}

// The persistent decode kernel's program: one Phase per piece of the token graph of
// model.rs:220-269, with its exchange buffers. Every (layer, phase) publishes into a buffer of its
// own, doubled by step parity, so a buffer is rewritten two steps after it was last read.
void Model::setup_engine() {
    const ModelConfig& c = cfg_;
    engine_grid_ = decode_max_grid();
    if (engine_grid_ <= 0) throw Error(QNE_EDEVICE, "the persistent decode kernel cannot be made co-resident");
    const int grid = engine_grid_, nw = grid * (kDecodeThreads / 64);
    auto unsupported = [](const std::string& why) {
        return Error(QNE_EFORMAT, "unsupported model architecture for the persistent decode kernel: " + why +
                                      " (load with {\"engine\": \"graph\"})");
    };
    if (c.hidden % 512 != 0 || c.hidden > 4096) throw unsupported("hidden must be a multiple of 512 and <= 4096");
    if (c.hidden > 2 * nw || c.hidden < grid) throw unsupported("hidden must lie in [workgroups, 2 * waves]");
    if (c.head_dim != kHeadDim) throw unsupported("head_dim must be 256");
    if (c.n_kv_heads <= 0 || c.n_q_heads % c.n_kv_heads != 0 || c.n_q_heads / c.n_kv_heads > 4)
        throw unsupported("n_q_heads / n_kv_heads must be 1..4");
    if (c.n_q_heads * 4 > grid) throw unsupported("too many attention heads for the grid");
    if (c.rope_dim % 8 != 0 || c.rope_dim > c.head_dim) throw unsupported("rope_dim must be a multiple of 8");
    if (c.gdn_dk != 128 || c.gdn_dv != 128) throw unsupported("GDN dk and dv must be 128");
    if (c.conv_kernel != 4) throw unsupported("the GDN conv kernel must be 4");
    const int S = std::min(grid / c.n_kv_heads, kMaxSplits), G = c.n_q_heads / c.n_kv_heads;
    if (S < 1) throw unsupported("too many kv heads");
    const int H = c.gdn_heads;
    if (H * 128 + H * 16 > 6144) throw unsupported("too many GDN heads");

    // exchange buffers: sizes per (layer, phase), allocated in one arena
    struct Buf {
        uint32_t n;
        size_t off;
    };
    std::vector<Buf> bufs;
    size_t total = 0;
    auto buf = [&](uint32_t n) {
        n = (n + 1) & ~1u;
        bufs.push_back({n, total});
        total += 2 * (size_t)n;
        return (int)bufs.size() - 1;
    };
    std::vector<Phase> prog;
    auto gemv = [&](const DevMat& m, int rows, int epi) {
        Phase P;
        P.kind = PH_GEMV;
        P.mkind = m.kind; P.k = m.k; P.group = m.group; P.rows = rows; P.epi = epi;
        P.w = m.w; P.sz = m.sz;
        if (decode_gemv_variant(m.kind, m.k) < 0) throw unsupported("matrix width " + std::to_string(m.k));
        const int rb = m.kind ? m.k / 2 : m.k * 2, szb = m.kind ? (m.k / m.group) * 4 : 0;
        if ((rb + szb) * (epi == EP_SWIGLU ? 2 : 1) + (epi == EP_CONV ? 32 : 0) > 8 * 1024)
            throw unsupported("rows too wide for the LDS region");
        if (m.kind == MAT_Q4 && m.group != 32 && m.group != 64 && m.group != 128)
            throw unsupported("q4 group size " + std::to_string(m.group));
        if (epi == EP_CONV && (rows + nw - 1) / nw > 64) throw unsupported("too many in-projection rows per wave");
        return P;
    };
    // input links: (phase index, buffer id) of each published vector
    std::vector<int> out_buf;
    std::vector<int> grp_buf;  // PH_GDNF: its head-group exchange buffer; PH_ATTN with fold: its partials (else -1)
    int h_prev = -1;  // buffer of the residual stream published by the previous layer's down
    auto push = [&](const Phase& P, int out, int grp, const char* label) {
        prog.push_back(P);
        out_buf.push_back(out);
        grp_buf.push_back(grp);
        phase_label_.push_back(label);
    };
    phase_label_.clear();
    for (int i = 0; i < c.layers; i++) {
        const DevLayer& L = layers_[i];
        const bool fuse = !L.attn && gdn_fusion_ && L.in.rows == c.gdn_proj() && c.gdn_dk == 128 &&
                          gdn_fusable(L.in.kind, L.in.k, L.in.group, H, grid);
        int b_mixed;
        if (fuse) {
            // in-projection, conv and the delta rule step in one phase (PH_GDNF)
            Phase f = gemv(L.in, L.in.rows, EP_CONV);
            f.kind = PH_GDNF;
            f.xin = i == 0 ? XI_EMBED : XI_EXCH;
            f.xnorm = XN_NORM;
            f.gain = L.input_norm;
            f.in_n = c.hidden;
            f.conv_ch = c.conv_channels();
            f.conv = L.conv_state;
            f.conv_w = L.conv_w;
            f.heads = H;
            f.rec = L.rec;
            f.prm = L.gdn_params;
            const int b_grp = buf((uint32_t)(H * 258));
            b_mixed = buf((uint32_t)(H * 128 + H * 16));
            push(f, b_mixed, b_grp, "gdn.mixer_in+gdn");
        }
        // mixer_in
        Phase in = gemv(L.in, L.in.rows, L.attn ? EP_STORE : EP_CONV);
        in.xin = i == 0 ? XI_EMBED : XI_EXCH;
        in.xnorm = XN_NORM;
        in.gain = L.input_norm;
        in.in_n = c.hidden;
        if (!L.attn) {
            in.conv_ch = c.conv_channels();
            in.conv = L.conv_state;
            in.conv_w = L.conv_w;
        }
        int in_rel_out = 1;
        if (fuse) {
        } else if (!L.attn) {
            const int b_proj = buf((uint32_t)L.in.rows);
            push(in, b_proj, -1, "gdn.mixer_in");
            Phase g;
            g.kind = PH_GDN;
            g.heads = H;
            g.gain = L.gdn_params;
            g.rec = L.rec;
            b_mixed = buf((uint32_t)(H * 128 + H * 16));
            push(g, b_mixed, -1, "gdn.gdn");
        } else {
            const int b_proj = buf((uint32_t)L.in.rows);
            push(in, b_proj, -1, "attn.mixer_in");
            Phase at;
            at.kind = PH_ATTN;
            at.heads = c.n_q_heads;
            at.kv_heads = c.n_kv_heads;
            at.gain = L.norms;
            at.kp = L.k_pool;
            at.vp = L.v_pool;
            const int b_part = buf((uint32_t)(c.n_kv_heads * S * G * 258));
            if (S >= 4 * G) {
                // the combine folded into the attention phase: the partials are the phase's own
                // exchange, the combined vector its output
                at.fold = 1;
                b_mixed = buf((uint32_t)(c.n_q_heads * 256));
                push(at, b_mixed, b_part, "attn.attention+combine");
            } else {
                push(at, b_part, -1, "attn.attention");
                Phase cb;
                cb.kind = PH_COMB;
                cb.heads = c.n_q_heads;
                cb.kv_heads = c.n_kv_heads;
                cb.in2_rel = 2;
                b_mixed = buf((uint32_t)(c.n_q_heads * 256));
                push(cb, b_mixed, -1, "attn.combine");
            }
        }
        const char* kind = L.attn ? "attn." : "gdn.";
        auto lab = [&](const char* n) { return (std::string(kind) + n); };
        Phase mo = gemv(L.out, c.hidden, EP_RESID);
        mo.xnorm = L.attn ? XN_PLAIN : XN_GDN;
        mo.heads = H;
        mo.in_n = L.attn ? c.attn_out() : H * 128 + H * 16;
        mo.in_rel = in_rel_out;
        const int b_h1 = buf((uint32_t)c.hidden);
        push(mo, b_h1, -1, lab("mixer_out").c_str());
        if (L.gate_up.rows != 2 * c.intermediate) throw unsupported("gate_up rows");
        Phase gu = gemv(L.gate_up, c.intermediate, EP_SWIGLU);
        gu.xnorm = XN_NORM;
        gu.gain = L.post_norm;
        gu.in_n = c.hidden;
        const int b_act = buf((uint32_t)c.intermediate);
        push(gu, b_act, -1, lab("gate_up").c_str());
        Phase dn = gemv(L.down, c.hidden, EP_RESID);
        dn.in_n = c.intermediate;
        h_prev = buf((uint32_t)c.hidden);
        push(dn, h_prev, -1, lab("down").c_str());
    }
    Phase hd = gemv(lm_head_, c.vocab, EP_HEAD);
    hd.xnorm = XN_NORM;
    hd.gain = final_norm_;
    hd.in_n = c.hidden;
    hd.is_head = 1;
    push(hd, -1, -1, "lm_head");
    if ((int)prog.size() > kMaxPhases) throw unsupported("too many layers");
    for (const Phase& P : prog)
        if (P.kind == PH_GEMV && (P.in_n > 6144 || P.in_n > P.k + 2048 * (P.xnorm == XN_GDN)))
            throw unsupported("input vector too long");

    exch_ = (uint64_t*)dalloc(total * 8);
    exch_bytes_ = total * 8;
    QNE_HIP(hipMemset(exch_, 0, exch_bytes_));
    auto base = [&](int b) { return exch_ + bufs[b].off; };
    for (size_t p = 0; p < prog.size(); p++) {
        Phase& P = prog[p];
        if (out_buf[p] >= 0) {
            P.out = base(out_buf[p]);
            P.out_stride = bufs[out_buf[p]].n;
        }
        if (grp_buf[p] >= 0 && P.kind == PH_GDNF) {
            P.grp = base(grp_buf[p]);
            P.grp_stride = bufs[grp_buf[p]].n;
        }
        if (grp_buf[p] >= 0 && P.kind == PH_ATTN) {
            P.part = base(grp_buf[p]);
            P.part_stride = bufs[grp_buf[p]].n;
        }
        if ((P.kind == PH_GEMV || P.kind == PH_GDNF) && P.xin == XI_EMBED) continue;
        const int src = (int)p - P.in_rel;
        if (src < 0 || out_buf[src] < 0) throw Error(QNE_EINVAL, "decode program: bad input link");
        P.in = base(out_buf[src]);
        P.in_stride = P.in_cap = bufs[out_buf[src]].n;
        if (P.in2_rel > 0) {
            const int s2 = (int)p - P.in2_rel;
            P.in2 = base(out_buf[s2]);
            P.in2_stride = P.in2_cap = bufs[out_buf[s2]].n;
        }
    }
    // q4 GEMVs on the matrix cores (tiled): all or none of the residual phases, since the tiled
    // phases keep the residual rows they own per workgroup
    bool tiled = mfma_gemv_ && (c.hidden + grid - 1) / grid <= kTiledMaxRes;
    for (const Phase& P : prog)
        if (P.kind == PH_GEMV && P.epi == EP_RESID && !gemv_tileable(P, grid)) tiled = false;
    if (tiled)
        for (Phase& P : prog) P.tiled = gemv_tileable(P, grid) ? 1 : 0;
    for (Phase& P : prog) finalize_phase(P, grid);
    {
        // the workgroup's extra GEMV slot is single, and a phase's data is sent two region phases
        // ahead: no two consecutive region phases (cyclically over steps; the LM head never uses
        // it, so skipping it changes nothing) may both use it
        std::vector<int> rp;
        for (int i = 0; i < (int)prog.size(); i++)
            if (prog[i].region && !prog[i].is_head) rp.push_back(i);
        for (bool changed = true; changed;) {
            changed = false;
            for (size_t j = 0; j < rp.size(); j++) {
                Phase& cur = prog[rp[j]];
                const Phase& prev = prog[rp[(j + rp.size() - 1) % rp.size()]];
                if (cur.extra && prev.extra) {
                    cur.extra = 0;
                    changed = true;
                }
            }
        }
    }
    DecodeArgs links;
    if (!finalize_program(prog.data(), (int)prog.size(), links)) throw unsupported("too few region phases per step");
    nph_ = (int)prog.size();
    phase_kind_.clear();
    for (const Phase& P : prog) phase_kind_.push_back(P.kind);
    std::vector<PhaseBufs> pbufs;
    std::vector<Phase> shapes;
    std::vector<GdnExtra> gdnx;
    split_program(prog.data(), (int)prog.size(), pbufs, shapes, gdnx);
    GdnExtra* d_gdnx = nullptr;
    if (!gdnx.empty()) {
        d_gdnx = (GdnExtra*)dalloc(gdnx.size() * sizeof(GdnExtra));
        QNE_HIP(hipMemcpy(d_gdnx, gdnx.data(), gdnx.size() * sizeof(GdnExtra), hipMemcpyHostToDevice));
    }
    PhaseBufs* d_prog = (PhaseBufs*)dalloc(pbufs.size() * sizeof(PhaseBufs));
    QNE_HIP(hipMemcpy(d_prog, pbufs.data(), pbufs.size() * sizeof(PhaseBufs), hipMemcpyHostToDevice));
    Phase* d_shapes = (Phase*)dalloc(shapes.size() * sizeof(Phase));
    QNE_HIP(hipMemcpy(d_shapes, shapes.data(), shapes.size() * sizeof(Phase), hipMemcpyHostToDevice));
    am_ = (uint64_t*)dalloc((size_t)4 * grid * 8);
    QNE_HIP(hipMemset(am_, 0, (size_t)4 * grid * 8));

    DecodeArgs* a = new DecodeArgs();
    engine_args_ = a;
    a->prog = d_prog;
    a->shapes = d_shapes;
    a->gdnx = d_gdnx;
    a->h_tiled = tiled ? 1 : 0;
    a->nph = nph_;
    a->reg0 = links.reg0; a->reg1 = links.reg1; a->head_reg = links.head_reg;
    a->emb_w = embed_.w; a->emb_sz = embed_.sz; a->emb_kind = embed_.kind; a->emb_group = embed_.group;
    a->hidden = c.hidden; a->vocab = c.vocab; a->eps = c.eps;
    a->rope_dim = c.rope_dim; a->inv_freq = inv_freq_;
    a->block_table = block_table_; a->max_blocks = (max_context_ + 15) / 16;
    a->logits = logits_;
    a->am = am_; a->am_stride = (uint32_t)(2 * grid);
    a->tok = tok_; a->ids = ids_; a->out_ids = out_ids_; a->out_cap = (uint32_t)max_context_;
    eng_bar_ = (unsigned*)dalloc(64);
    QNE_HIP(hipMemset(eng_bar_, 0, 64));
    a->err = eng_bar_;
    QNE_HIP(hipHostMalloc((void**)&host_err_, 64, hipHostMallocDefault));
    host_err_[0] = 0;
    tag_base_ = 1;
    dispatches_ = 1;  // one launch covers a whole decode window
    QNE_HIP(hipDeviceSynchronize());
}

void Model::run_engine(const EngineRun& r) {
    DecodeArgs a = *(const DecodeArgs*)engine_args_;
    const uint64_t tags = (uint64_t)r.n_steps * (uint64_t)nph_;
    if ((uint64_t)tag_base_ + tags >= 0xFFFF0000ull) {
        // tags would wrap: clear every exchange buffer and start again
        QNE_HIP(hipMemsetAsync(exch_, 0, exch_bytes_, stream_));
        QNE_HIP(hipMemsetAsync(am_, 0, (size_t)4 * engine_grid_ * 8, stream_));
        tag_base_ = 1;
    }
    a.feed = r.feed;
    a.head = r.head;
    a.argmax = r.argmax;
    a.n_steps = r.n_steps;
    a.pos0 = r.pos0;
    a.out_ids = r.record_ids ? out_ids_ : nullptr;
    a.trace = r.trace;
    a.sub = r.sub;
    a.trace_cap = r.trace_cap;
    a.tag_base = tag_base_;
    tag_base_ += (uint32_t)tags;
    pending_units_ += (double)tags;
    QNE_HIP(hipMemsetAsync(eng_bar_, 0, 8, stream_));
    QNE_HIP(launch_decode(a, engine_grid_, stream_));
    QNE_HIP(hipMemcpyAsync(host_err_, eng_bar_, 4, hipMemcpyDeviceToHost, stream_));
}

void Model::check_engine_error() {
    if (persistent_ && host_err_ && host_err_[0] != 0) {
        host_err_[0] = 0;
        throw Error(QNE_EDEVICE, "GPU wait failed: a phase of the decode kernel timed out waiting for its input");
    }
}

void Model::sync() {
    const double units = pending_units_;
    pending_units_ = 0.0;
    wait_stream(stream_, work_deadline_s(units));
    check_engine_error();
}

void Model::set_tok(uint32_t token, uint32_t pos) {
    host_tok_[0] = token;
    host_tok_[1] = pos;
    host_tok_[2] = 0;
    host_tok_[3] = 0;
    QNE_HIP(hipMemcpyAsync(tok_, host_tok_, 16, hipMemcpyHostToDevice, stream_));
}

static void check_ids(const uint32_t* ids, size_t n, int vocab) {
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= (uint32_t)vocab)
            throw Error(QNE_EINVAL, "token id " + std::to_string(ids[i]) + " outside the vocabulary");
}

void Model::run_layers_graph() {
    pending_units_ += 6.0 * (double)layers_.size();
    if (use_graphs_) QNE_HIP(hipGraphLaunch(g_layers_, stream_));
    else enqueue_layers();
}
void Model::run_head_graph(bool greedy) {
    if (use_graphs_) QNE_HIP(hipGraphLaunch(greedy ? g_head_greedy_ : g_head_logits_, stream_));
    else enqueue_head(greedy);
}

void Model::reset() {
    QNE_HIP(hipMemsetAsync(state_, 0, state_bytes_, stream_));
    sync();
}

// model.rs:324-334: every prompt token through the whole graph, positions from 0.
void Model::prefill(const uint32_t* ids, size_t n) {
    if (n == 0 || n >= (size_t)max_context_)
        throw Error(n == 0 ? QNE_EINVAL : QNE_ECONTEXT, "prompt length must be 1.." + std::to_string(max_context_));
    check_ids(ids, n, cfg_.vocab);
    std::memcpy(host_ids_, ids, n * 4);
    QNE_HIP(hipMemcpyAsync(ids_, host_ids_, n * 4, hipMemcpyHostToDevice, stream_));
    if (persistent_) {
        // Only the last token's LM head is observable (logits, greedy pick), so the others are
        // skipped: the state afterwards is the same.
        set_tok(ids[0], 0);
        EngineRun r;
        r.feed = 0; r.head = 2; r.argmax = 1; r.n_steps = (int)n; r.pos0 = 0;
        run_engine(r);
    } else {
        for (size_t i = 0; i < n; i++) {
            launch_set_tok(tok_, ids_, (int)i, (uint32_t)i, stream_);
            run_layers_graph();
            run_head_graph(true);
        }
    }
    sync();
}

// model.rs:349-372: continues the state at `start`; with finish_logits, the logits and greedy
// pick after the last token (tok = [pick, start + n]). Without it, tok is left as it was.
void Model::prefill_chunk(const uint32_t* ids, size_t n, uint32_t start, bool finish_logits) {
    if (n == 0 || (uint64_t)start + n >= (uint64_t)max_context_)
        throw Error(n == 0 ? QNE_EINVAL : QNE_ECONTEXT,
                    "context limit: " + std::to_string(start) + " + " + std::to_string(n) + " tokens does not fit in " +
                        std::to_string(max_context_));
    check_ids(ids, n, cfg_.vocab);
    std::memcpy(host_ids_, ids, n * 4);
    QNE_HIP(hipMemcpyAsync(ids_, host_ids_, n * 4, hipMemcpyHostToDevice, stream_));
    // The reference runs this path through its batched GEMM (batch.rs); so does this one, 64
    // tokens per pass, unless the shapes do not fit the batched GEMM.
    if (!chunk_tried_) {
        chunk_tried_ = true;
        try {
            chunk_ = new ChunkPrefill(*this);
        } catch (const Error& e) {
            if (e.code != QNE_EFORMAT) throw;
            chunk_ = nullptr;
        }
    }
    if (chunk_) {
        chunk_->run(ids_, n, start, finish_logits);
        sync();
        return;
    }
    if (persistent_) {
        // tok is only written by the greedy pick, so without finish_logits it stays as it was
        if (finish_logits) QNE_HIP(hipMemsetAsync(tok_ + 2, 0, 4, stream_));
        EngineRun r;
        r.feed = 0; r.head = finish_logits ? 2 : 0; r.argmax = finish_logits ? 1 : 0;
        r.n_steps = (int)n; r.pos0 = start;
        run_engine(r);
        sync();
        return;
    }
    if (!finish_logits) QNE_HIP(hipMemcpyAsync(tok_backup_, tok_, 16, hipMemcpyDeviceToDevice, stream_));
    for (size_t i = 0; i < n; i++) {
        launch_set_tok(tok_, ids_, (int)i, start + (uint32_t)i, stream_);
        run_layers_graph();
    }
    if (finish_logits) run_head_graph(true);
    else QNE_HIP(hipMemcpyAsync(tok_, tok_backup_, 16, hipMemcpyDeviceToDevice, stream_));
    sync();
}

void Model::logits(float* out, size_t cap) {
    if (cap < (size_t)cfg_.vocab) throw Error(QNE_EINVAL, "logits buffer smaller than the vocabulary");
    QNE_HIP(hipMemcpyAsync(host_logits_, logits_, (size_t)cfg_.vocab * 4, hipMemcpyDeviceToHost, stream_));
    sync();
    std::memcpy(out, host_logits_, (size_t)cfg_.vocab * 4);
}

// model.rs:380-392: host sampling owns the next token, so no device argmax.
void Model::step(uint32_t token, uint32_t pos, float* out, size_t cap) {
    if (pos >= (uint32_t)max_context_)
        throw Error(QNE_ECONTEXT, "context limit of " + std::to_string(max_context_) + " tokens reached");
    if (cap < (size_t)cfg_.vocab) throw Error(QNE_EINVAL, "logits buffer smaller than the vocabulary");
    step_device(token, pos);
    QNE_HIP(hipMemcpyAsync(host_logits_, logits_, (size_t)cfg_.vocab * 4, hipMemcpyDeviceToHost, stream_));
    sync();
    std::memcpy(out, host_logits_, (size_t)cfg_.vocab * 4);
}

void Model::step_device(uint32_t token, uint32_t pos) {
    if (pos >= (uint32_t)max_context_)
        throw Error(QNE_ECONTEXT, "context limit of " + std::to_string(max_context_) + " tokens reached");
    if (token >= (uint32_t)cfg_.vocab) throw Error(QNE_EINVAL, "token id outside the vocabulary");
    set_tok(token, pos);
    if (persistent_) {
        EngineRun r;
        r.feed = 1; r.head = 1; r.argmax = 0; r.n_steps = 1; r.pos0 = pos;
        run_engine(r);
    } else {
        run_layers_graph();
        run_head_graph(false);
    }
    sync();
}

// model.rs:395-414: device copies of all recurrent, conv and KV state.
void Model::snapshot() {
    if (!saved_) saved_ = dalloc(state_bytes_);
    QNE_HIP(hipMemcpyAsync(saved_, state_, state_bytes_, hipMemcpyDeviceToDevice, stream_));
    sync();
}

void Model::restore() {
    if (!saved_) throw Error(QNE_ENOSNAPSHOT, "no snapshot taken");
    QNE_HIP(hipMemcpyAsync(state_, saved_, state_bytes_, hipMemcpyDeviceToDevice, stream_));
    sync();
}

void Model::last_token(uint32_t* token, uint32_t* next_pos) {
    QNE_HIP(hipMemcpyAsync(host_tok_ + 4, tok_, 16, hipMemcpyDeviceToHost, stream_));
    sync();
    *token = host_tok_[4];
    *next_pos = host_tok_[5];
}

// model.rs:426-449, GPU-resident greedy loop: out[0] = last_token().0, then windows of up to
// `window` steps whose picks are fed back on the device. As in the reference, a window of one
// step yields its pick and a longer window yields u32::MAX placeholders (model.rs:441-446), and
// `stop` is checked against the last value pushed (model.rs:433), so it ends the loop only after a
// one-step window or on the first id.
size_t Model::decode(size_t n, uint32_t window, const uint32_t* stop, size_t nstop, uint32_t* out, size_t cap) {
    return decode_loop(n, window, stop, nstop, out, cap, false);
}

// The same loop with every step's pick appended on the device, so every window returns real ids;
// the loop ends after the first id found in `stop` (the state may have advanced past it inside a
// window, as the reference's does).
size_t Model::decode_ids(size_t n, uint32_t window, const uint32_t* stop, size_t nstop, uint32_t* out, size_t cap) {
    return decode_loop(n, window, stop, nstop, out, cap, true);
}

size_t Model::decode_loop(size_t n, uint32_t window, const uint32_t* stop, size_t nstop, uint32_t* out, size_t cap,
                          bool every_id) {
    if (window == 0) throw Error(QNE_EINVAL, "window must be >= 1");
    if (cap < 1 || (n > 0 && cap < n)) throw Error(QNE_EINVAL, "output buffer smaller than n");
    if (n == 0) return 0;
    uint32_t first, next_pos;
    last_token(&first, &next_pos);
    size_t len = 0;
    out[len++] = first;
    auto is_stop = [&](uint32_t id) {
        for (size_t i = 0; i < nstop; i++)
            if (stop[i] == id) return true;
        return false;
    };
    last_decode_ms_ = 0.0;
    last_decode_steps_ = 0;
    while (len < n && !is_stop(out[len - 1])) {
        const uint32_t steps = (uint32_t)std::min<size_t>(window, n - len);
        if ((uint64_t)next_pos + steps > (uint64_t)max_context_)
            throw Error(QNE_ECONTEXT, "context limit of " + std::to_string(max_context_) + " tokens reached after " +
                                          std::to_string(len) + " generated tokens");
        next_pos += steps;
        // tok[2] counts the ids appended on the device during this window
        QNE_HIP(hipMemsetAsync(tok_ + 2, 0, 4, stream_));
        QNE_HIP(hipEventRecord(ev_start_, stream_));
        if (persistent_) {
            EngineRun r;
            r.feed = 1; r.head = 1; r.argmax = 1; r.n_steps = (int)steps; r.pos0 = next_pos - steps;
            r.record_ids = true;
            run_engine(r);
        } else {
            for (uint32_t s = 0; s < steps; s++) {
                run_layers_graph();
                run_head_graph(true);
            }
        }
        QNE_HIP(hipEventRecord(ev_stop_, stream_));
        QNE_HIP(hipMemcpyAsync(host_ids_, out_ids_, (size_t)steps * 4, hipMemcpyDeviceToHost, stream_));
        sync();
        float ms = 0.0f;
        QNE_HIP(hipEventElapsedTime(&ms, ev_start_, ev_stop_));
        last_decode_ms_ += ms;
        last_decode_steps_ += steps;
        if (!every_id) {
            if (steps == 1) out[len++] = host_ids_[0];
            else
                for (uint32_t s = 0; s < steps; s++) out[len++] = 0xFFFFFFFFu;
            continue;
        }
        for (uint32_t s = 0; s < steps && len < n; s++) {
            out[len++] = host_ids_[s];
            if (is_stop(out[len - 1])) break;
        }
    }
    return len;
}

double Model::profile_token() {
    hipEvent_t a, b;
    QNE_HIP(hipEventCreate(&a));
    QNE_HIP(hipEventCreate(&b));
    QNE_HIP(hipEventRecord(a, stream_));
    if (persistent_) {
        uint32_t t, p;
        last_token(&t, &p);
        if (p >= (uint32_t)max_context_) throw Error(QNE_ECONTEXT, "context limit reached");
        EngineRun r;
        r.feed = 1; r.head = 1; r.argmax = 1; r.n_steps = 1; r.pos0 = p;
        QNE_HIP(hipEventRecord(a, stream_));
        run_engine(r);
    } else {
        run_layers_graph();
        run_head_graph(true);
    }
    QNE_HIP(hipEventRecord(b, stream_));
    sync();
    float ms = 0.0f;
    QNE_HIP(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return ms;
}

// Per-phase device times of one greedy decode token (the counterpart of Gpu::profile's
// per-label timestamp sums, kernels/src/lib.rs:366-396). For every phase and workgroup the
// timeline has the moment the workgroup had its input and the moment it was done. Reported per
// phase: the phase's span (latest done minus the previous phase's latest done), the median and
// maximum per-workgroup compute time (done - input), and the median and maximum hand-over latency
// (input - previous phase's latest done).
std::string Model::profile_token_json() {
    if (!persistent_) throw Error(QNE_EINVAL, "the phase profile needs the persistent engine");
    uint32_t t, p;
    last_token(&t, &p);
    if (p >= (uint32_t)max_context_) throw Error(QNE_ECONTEXT, "context limit reached");
    const int nph = nph_, grid = engine_grid_;
    const size_t n = 2 + 2 * (size_t)nph * grid;
    std::vector<unsigned long long> tr(n, 0ull);
    unsigned long long* d = (unsigned long long*)dalloc(n * 8);
    QNE_HIP(hipMemcpy(d, tr.data(), n * 8, hipMemcpyHostToDevice));
    EngineRun r;
    r.feed = 1; r.head = 1; r.argmax = 1; r.n_steps = 1; r.pos0 = p;
    r.trace = d;
    r.trace_cap = nph;
    const size_t nsub = 8 * (size_t)nph * grid;
    std::vector<unsigned long long> sub(nsub, 0ull);
    unsigned long long* dsub = (unsigned long long*)dalloc(nsub * 8);
    QNE_HIP(hipMemcpy(dsub, sub.data(), nsub * 8, hipMemcpyHostToDevice));
    r.sub = dsub;
    run_engine(r);
    sync();
    QNE_HIP(hipMemcpy(tr.data(), d, n * 8, hipMemcpyDeviceToHost));
    QNE_HIP(hipMemcpy(sub.data(), dsub, nsub * 8, hipMemcpyDeviceToHost));
    int khz = 0;
    QNE_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device_));
    const double tick_ms = khz > 0 ? 1.0 / (double)khz : 1e-5;
    auto ms = [&](unsigned long long a, unsigned long long b) { return b > a ? (double)(b - a) * tick_ms : 0.0; };
    auto med = [](std::vector<double> v) {
        if (v.empty()) return 0.0;
        std::sort(v.begin(), v.end());
        return v[v.size() / 2];
    };
    std::map<std::string, double> span_l, comp_l, exch_l;
    // critical chain: per phase, when each workgroup had its input staged and when it had
    // published, relative to the previous phase's last publish (sub-step slots per kind)
    std::string chain = "[";
    std::string pubs = "[", ins = "[", subt = "[";
    unsigned long long pub_prev = 0;
    std::map<std::string, std::vector<double>> sub_l;
    std::string phases = "[";
    unsigned long long prev = tr[0];
    for (int b = 0; b < nph; b++) {
        const std::string label = phase_label_[b];
        unsigned long long dmax = 0;
        std::vector<double> comp, exch;
        for (int w = 0; w < grid; w++) {
            const unsigned long long in = tr[2 + 2 * ((size_t)b * grid + w)], done = tr[3 + 2 * ((size_t)b * grid + w)];
            dmax = std::max(dmax, done);
            comp.push_back(ms(in, done));
            exch.push_back(ms(prev, in));
        }
        {
            // sub-steps: intervals between the consecutive stamped slots of each workgroup
            std::vector<std::vector<double>> parts;
            for (int w = 0; w < grid; w++) {
                const unsigned long long* q = sub.data() + 8 * ((size_t)b * grid + w);
                if (q[0] == 0) continue;
                int last = 0, n = 0;
                for (int k2 = 1; k2 < 8; k2++) {
                    if (q[k2] == 0 || k2 == 6) continue;  // slot 6: the workgroup's place
                    if ((int)parts.size() <= n) parts.resize(n + 1);
                    parts[n++].push_back(ms(q[last], q[k2]));
                    last = k2;
                }
            }
            if (!parts.empty()) {
                auto& v = sub_l[label];
                if (v.size() < parts.size()) v.resize(parts.size(), 0.0);
                for (size_t k2 = 0; k2 < parts.size(); k2++) v[k2] += med(parts[k2]);
            }
        }
        {
            const int kind = phase_kind_[b];  // 0 GEMV, 1 GDN, 2 attention, 3 combine, 4 fused GDN
            const int in_slot = kind == 0 || kind == 4 ? 0 : kind == 3 ? 2 : 1;
            const int pub_slot = kind == 0 || kind == 4 ? 3 : kind == 1 ? 2 : kind == 2 ? 5 : 3;
            std::vector<double> tin, tpub;
            unsigned long long pmax = 0;
            for (int w = 0; w < grid; w++) {
                const unsigned long long* q = sub.data() + 8 * ((size_t)b * grid + w);
                if (q[in_slot] == 0 || q[pub_slot] == 0) continue;
                pmax = std::max(pmax, q[pub_slot]);
                if (pub_prev) {
                    tin.push_back((double)((long long)q[in_slot] - (long long)pub_prev) * tick_ms);
                    tpub.push_back((double)((long long)q[pub_slot] - (long long)pub_prev) * tick_ms);
                }
            }
            {
                // every workgroup's publish time relative to the previous phase's last publish,
                // in ticks (-1: not recorded), for the analysis of which workgroups are late
                pubs += pubs.size() > 1 ? ",[" : "[";
                ins += ins.size() > 1 ? ",[" : "[";
                for (int w = 0; w < grid; w++) {
                    const unsigned long long* q = sub.data() + 8 * ((size_t)b * grid + w);
                    const long long d = pub_prev && q[pub_slot] ? (long long)q[pub_slot] - (long long)pub_prev : -1;
                    const long long di = pub_prev && q[in_slot] ? (long long)q[in_slot] - (long long)pub_prev : -1;
                    pubs += (w ? "," : "") + std::to_string(d);
                    ins += (w ? "," : "") + std::to_string(di);
                }
                pubs += "]";
                ins += "]";
                // and every workgroup's sub-step timestamps (slots 0..7, same origin; -1: none)
                subt += subt.size() > 1 ? ",[" : "[";
                for (int w = 0; w < grid; w++) {
                    const unsigned long long* q = sub.data() + 8 * ((size_t)b * grid + w);
                    subt += w ? ",[" : "[";
                    for (int k2 = 0; k2 < 8; k2++) {
                        const long long d = k2 == 6 ? -1 : pub_prev && q[k2] ? (long long)q[k2] - (long long)pub_prev : -1;
                        subt += (k2 ? "," : "") + std::to_string(d);
                    }
                    subt += "]";
                }
                subt += "]";
            }
            if (!tin.empty()) {
                char buf[224];
                std::snprintf(buf, sizeof buf, "%s[\"%s\",%.5f,%.5f,%.5f,%.5f]", chain.size() > 1 ? "," : "", label.c_str(),
                              med(tin), *std::max_element(tin.begin(), tin.end()), med(tpub),
                              *std::max_element(tpub.begin(), tpub.end()));
                chain += buf;
            }
            if (pmax) pub_prev = pmax;
        }
        const double span = ms(prev, dmax), cm = med(comp), em = med(exch);
        const double cx = *std::max_element(comp.begin(), comp.end()), ex = *std::max_element(exch.begin(), exch.end());
        span_l[label] += span;
        comp_l[label] += cm;
        exch_l[label] += em;
        char buf[224];
        std::snprintf(buf, sizeof buf, "%s[\"%s\",%.5f,%.5f,%.5f,%.5f,%.5f]", b ? "," : "", label.c_str(), span, cm, cx,
                      em, ex);
        phases += buf;
        prev = dmax;
    }
    phases += "]";
    auto obj = [](const std::map<std::string, double>& m) {
        std::string o = "{";
        for (auto& kv : m) {
            char buf[96];
            std::snprintf(buf, sizeof buf, "%s\"%s\":%.5f", o.size() > 1 ? "," : "", kv.first.c_str(), kv.second);
            o += buf;
        }
        return o + "}";
    };
    char head[200];
    std::snprintf(head, sizeof head, "{\"total_ms\":%.5f,\"tail_ms\":%.5f,\"tick_ms\":%.3g,", ms(tr[0], tr[1]),
                  ms(prev, tr[1]), tick_ms);
    // each workgroup's place: XCC_ID and the HW_ID register (CU, SIMD, shader array / engine bits)
    std::string places = "[";
    for (int w = 0; w < grid; w++) {
        const unsigned long long v = sub[8 * (size_t)w + 6];
        places += (w ? "," : "") + (v ? "[" + std::to_string((v - 1) >> 32) + "," + std::to_string((v - 1) & 0xFFFFFFFFull) + "]"
                                      : std::string("null"));
    }
    places += "]";
    std::string subs = "{";
    for (auto& kv : sub_l) {
        subs += (subs.size() > 1 ? ",\"" : "\"") + kv.first + "\":[";
        for (size_t k2 = 0; k2 < kv.second.size(); k2++) {
            char buf[32];
            std::snprintf(buf, sizeof buf, "%s%.5f", k2 ? "," : "", kv.second[k2]);
            subs += buf;
        }
        subs += "]";
    }
    subs += "}";
    return std::string(head) +
           "\"sub_step_names\":{\"gemv\":[\"x load\",\"first group\",\"other groups\",\"dma issue (two ahead)\"],"
           "\"gdn\":[\"input\",\"state update\",\"dma issue (two ahead)\"],"
           "\"gdn_fused\":[\"rows + q/k publish\",\"head q/k exchange\",\"state update\",\"dma issue (two ahead)\"],"
           "\"attention\":[\"input\",\"q/k prep\",\"K/V landed\",\"context loop\",\"merge + publish\",\"dma issue (two ahead)\"],"
           "\"combine\":[\"partials\",\"gate\",\"combine + publish\"]}," +
           "\"sub_steps_median_ms\":" + subs + ",\"labels\":" + obj(span_l) + ",\"compute_median_ms\":" + obj(comp_l) +
           ",\"handover_median_ms\":" + obj(exch_l) +
           ",\"phase_columns\":[\"label\",\"span\",\"compute_median\",\"compute_max\",\"handover_median\",\"handover_max\"]" +
           ",\"phases\":" + phases +
           ",\"chain_columns\":[\"label\",\"input_median\",\"input_max\",\"published_median\",\"published_max\"]" +
           ",\"chain\":" + chain + "]" + ",\"publish_ticks\":" + pubs + "],\"input_ticks\":" + ins + "],\"sub_ticks\":" + subt + "],\"places\":" + places + "}";
}

}  // namespace qne
