// BatchDecoder: the per-step graph of model.rs:220-269 over up to 64 rows, one HIP graph per row
// count. Weights are the Model's; every row has its own recurrent state and paged KV cache.
#include "batch.hpp"

#include <algorithm>
#include <cstring>
#include <random>
#include <string>

#include "error.hpp"
#include "hip_util.hpp"
#include "kernels/launch.hpp"

namespace qne {

namespace {
constexpr int kRowsMax = 64;

int attn_splits_for(int max_blocks) {
    // One context split per 512 positions of capacity, whatever the number of rows: a row's split
    // boundaries (and so the order its attention partials are merged in) depend only on its own
    // length, and a row's result is bitwise the same in a batch of any size. At 64 rows of 4096
    // positions that is 2048 workgroups per layer (64 sequences measured 15.9k / 15.9k / 15.7k
    // tok/s at 1024 / 2048 / 4096 workgroups: a wave keeps a whole 16-position block in flight).
    return std::max(1, std::min(max_blocks, (max_blocks + 31) / 32));
}
}  // namespace

int operand_order(const DevMat& W) { return W.kind == KIND_Q4 ? 1 : 0; }

void rows_gemm(const DevMat& W, int n, float eps, uint8_t* frag, int norm, float* part, float* y, int y_stride, int epi,
               uint8_t* frag_out, const float* gain_out, int order_out, hipStream_t st, int row_tiles, bool partials_only,
               bool fuse) {
    GemmArgs a;
    a.m = n;
    a.frag = frag;
    a.norm = norm;
    a.eps = eps;
    a.kind = W.kind;
    a.W = W.w;
    a.SZ = W.sz;
    a.SZT = W.szt;
    a.N = W.rows;
    a.K = W.k;
    a.group = W.group;
    a.splits = gemm_splits(W.kind, W.rows, W.k, W.group, row_tiles);
    a.part = part;
    a.epi = epi;
    a.y = y;
    a.y_stride = y_stride;
    a.n_out = epi == EPI_SWIGLU ? W.rows / 2 : W.rows;
    a.frag_out = frag_out;
    a.gain_out = gain_out;
    a.order_out = order_out;
    a.partials_only = partials_only ? 1 : 0;
    a.fuse = fuse ? 0 : -1;
    launch_gemm(a, st);
}

void rows_shapes_check(const ModelConfig& c) {
    const int G = c.n_kv_heads > 0 ? c.n_q_heads / c.n_kv_heads : 0;
    if (c.gdn_dk != 128 || c.gdn_dv != 128 || c.head_dim != 256 || c.n_kv_heads <= 0 ||
        c.n_q_heads % c.n_kv_heads != 0 || (G != 1 && G != 2 && G != 4) || c.hidden % 64 != 0 ||
        c.intermediate % 64 != 0)
        throw Error(QNE_EFORMAT, "unsupported shapes for the batched path (GDN 128 x 128, head_dim 256, "
                                 "1, 2 or 4 query heads per kv head, hidden and intermediate multiples of 64)");
}

void rows_workspace(const std::vector<DevLayer>& layers, const DevMat& head, int rows, int row_tiles, size_t* part_floats,
                    size_t* frag_bytes) {
    const size_t rpad = (size_t)(rows + 63) / 64 * 64;
    size_t part = 0, frag = 0;
    // layer GEMMs write partials even with one split (their reduce stages the next operand); the
    // LM head only when it has more than one
    auto need = [&](const DevMat& W, bool layer) {
        if (!gemm_shape_ok(W.kind, W.rows, W.k, W.group, 1) || W.k % 4 != 0)
            throw Error(QNE_EFORMAT, "unsupported matrix shape for the batched GEMM (k must be a multiple of 64, "
                                     "q4 groups a multiple of 64)");
        const int s = gemm_splits(W.kind, W.rows, W.k, W.group, row_tiles);
        if (layer || s > 1) part = std::max(part, (size_t)s * rpad * W.rows);
        frag = std::max(frag, gemm_frag_bytes(W.k, rows));
    };
    for (const DevLayer& L : layers)
        for (const DevMat* W : {&L.in, &L.out, &L.gate_up, &L.down}) need(*W, true);
    need(head, false);
    *part_floats = part;
    *frag_bytes = frag;
}

void* BatchDecoder::dalloc(size_t bytes) {
    void* p = nullptr;
    QNE_HIP(hipMalloc(&p, bytes ? bytes : 16));
    allocations_.push_back(p);
    return p;
}

void BatchDecoder::sync(double steps) {
    // a batched step is about 8 dependent launches per layer plus the LM head
    wait_stream(stream_, work_deadline_s(steps * (8.0 * (double)m_.layers_.size() + 4.0)));
}

BatchDecoder::BatchDecoder(Model& m, int max_rows, int max_context) : m_(m), max_rows_(max_rows), max_context_(max_context) {
    if (max_rows < 1 || max_rows > kRowsMax) throw Error(QNE_EINVAL, "rows must be 1..64");
    if (max_context < 1 || max_context > m.max_context_)
        throw Error(QNE_ECONTEXT, "batch context must be 1.." + std::to_string(m.max_context_));
    const ModelConfig& c = m.cfg_;
    rows_shapes_check(c);
    size_t part = 0, frag = 0;
    rows_workspace(m.layers_, m.lm_head_, kRowsMax, 1, &part, &frag);
    QNE_HIP(hipSetDevice(m.device_));
    QNE_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    QNE_HIP(hipEventCreate(&ev0_));
    QNE_HIP(hipEventCreate(&ev1_));
    try {
        max_blocks_ = (max_context + 15) / 16;
        conv_floats_ = (size_t)c.conv_channels() * 4;
        rec_floats_ = (size_t)c.gdn_heads * c.gdn_dk * c.gdn_dv;
        pool_block_elems_ = (size_t)c.n_kv_heads * 16 * c.head_dim;
        const size_t rows = (size_t)max_rows;
        for (const DevLayer& L : m.layers_) {
            if (L.attn) {
                kpool_.push_back((uint16_t*)dalloc(rows * max_blocks_ * pool_block_elems_ * 2));
                vpool_.push_back((uint16_t*)dalloc(rows * max_blocks_ * pool_block_elems_ * 2));
                conv_.push_back(nullptr);
                rec_.push_back(nullptr);
            } else {
                conv_.push_back((float*)dalloc(rows * conv_floats_ * 4));
                rec_.push_back((float*)dalloc(rows * rec_floats_ * 4));
                kpool_.push_back(nullptr);
                vpool_.push_back(nullptr);
                QNE_HIP(hipMemset(conv_.back(), 0, rows * conv_floats_ * 4));
                QNE_HIP(hipMemset(rec_.back(), 0, rows * rec_floats_ * 4));
            }
        }
        // Each row's logical blocks are a random permutation of the shared pool, so every read goes
        // through the paged addressing.
        bt_host_.resize(rows * max_blocks_);
        for (size_t i = 0; i < bt_host_.size(); i++) bt_host_[i] = (int32_t)i;
        std::mt19937_64 rng(0x5DEECE66Dull);
        std::shuffle(bt_host_.begin(), bt_host_.end(), rng);
        block_table_ = (int32_t*)dalloc(bt_host_.size() * 4);
        QNE_HIP(hipMemcpy(block_table_, bt_host_.data(), bt_host_.size() * 4, hipMemcpyHostToDevice));

        proj_w_ = std::max(c.attn_proj(), c.gdn_proj());
        mixed_w_ = std::max(c.attn_out(), c.gdn_out());
        h_ = (float*)dalloc((size_t)kRowsMax * c.hidden * 4);
        proj_ = (float*)dalloc((size_t)kRowsMax * proj_w_ * 4);
        mixed_ = (float*)dalloc((size_t)kRowsMax * mixed_w_ * 4);
        act_ = (float*)dalloc((size_t)kRowsMax * c.intermediate * 4);
        logits_ = (float*)dalloc((size_t)kRowsMax * c.vocab * 4);
        qbuf_ = (float*)dalloc((size_t)kRowsMax * c.n_q_heads * c.head_dim * 4);
        part_ = (float*)dalloc(part * 4);
        frag_a_ = (uint8_t*)dalloc(frag);
        frag_b_ = (uint8_t*)dalloc(frag);
        QNE_HIP(hipMemset(frag_a_, 0, frag));
        QNE_HIP(hipMemset(frag_b_, 0, frag));
        attn_part_rows_ = (size_t)max_rows * attn_splits_for(max_blocks_);
        const size_t G = (size_t)(c.n_q_heads / c.n_kv_heads);
        attn_ml_ = (float*)dalloc(attn_part_rows_ * c.n_kv_heads * G * 2 * 4);
        attn_acc_ = (float*)dalloc(attn_part_rows_ * c.n_kv_heads * G * c.head_dim * 4);
        tokens_ = (uint32_t*)dalloc(kRowsMax * 4);
        picks_ = (uint32_t*)dalloc(kRowsMax * 4);
        am_scratch_ = dalloc(argmax_rows_scratch(kRowsMax));
        pos_ = (int32_t*)dalloc(kRowsMax * 4);
        order_ = (int32_t*)dalloc(kRowsMax * 4);
        QNE_HIP(hipMemset(tokens_, 0, kRowsMax * 4));
        QNE_HIP(hipMemset(pos_, 0, kRowsMax * 4));
        QNE_HIP(hipHostMalloc((void**)&host_u32_, 2 * kRowsMax * 4, hipHostMallocDefault));
    } catch (...) {
        release();
        throw;
    }
}

BatchDecoder::~BatchDecoder() { release(); }

void BatchDecoder::release() {
    (void)hipSetDevice(m_.device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (auto& g : graphs_) (void)hipGraphExecDestroy(g.second);
    graphs_.clear();
    for (void* p : allocations_) (void)hipFree(p);
    allocations_.clear();
    if (host_u32_) (void)hipHostFree(host_u32_);
    host_u32_ = nullptr;
    if (ev0_) (void)hipEventDestroy(ev0_);
    if (ev1_) (void)hipEventDestroy(ev1_);
    ev0_ = ev1_ = nullptr;
    if (stream_) (void)hipStreamDestroy(stream_);
    stream_ = nullptr;
}

void BatchDecoder::check_row(int row) const {
    if (row < 0 || row >= max_rows_) throw Error(QNE_EINVAL, "row out of range");
}

// One decode step of rows 0..n-1: model.rs:220-269 with every GEMV a GEMM over the rows. The x
// operands alternate between two staging buffers: the kernel that produces an activation (the
// embedding, the reduce of the previous GEMM) stages it for the GEMM that reads it; the RMSNorm
// gains are folded in there and the 1 / rms factors applied by the consuming GEMM.
void BatchDecoder::enqueue_step(int n) {
    const ModelConfig& c = m_.cfg_;
    const auto order = operand_order;
    const DevLayer& first = m_.layers_.front();
    launch_embed_rows(m_.embed_.kind, m_.embed_.w, m_.embed_.sz, m_.embed_.group, c.hidden, tokens_, n, h_, frag_a_,
                      first.input_norm, order(first.in), stream_, pos_, order_);
    auto gemm = [&](const DevMat& W, uint8_t* frag, int norm, float* y, int y_stride, int epi, uint8_t* frag_out,
                    const float* gain_out, int order_out) {
        rows_gemm(W, n, c.eps, frag, norm, part_, y, y_stride, epi, frag_out, gain_out, order_out, stream_);
    };
    const int splits = attn_splits_for(max_blocks_);
    for (size_t li = 0; li < m_.layers_.size(); li++) {
        const DevLayer& L = m_.layers_[li];
        const bool last = li + 1 == m_.layers_.size();
        // in-projection of RMSNorm(h, input_norm), staged in frag_a: split partials only, summed
        // (times the rows' 1 / rms) by the GDN step or the attention prep that reads them
        rows_gemm(L.in, n, c.eps, frag_a_, 1, part_, nullptr, 0, EPI_STORE, nullptr, nullptr, 0, stream_, 1, true);
        const int in_splits = gemm_splits(L.in.kind, L.in.rows, L.in.k, L.in.group, 1);
        const size_t split_stride = (size_t)64 * L.in.rows;  // the partials of one split: 64 rows (n <= 64)
        if (L.attn) {
            AttnRowsArgs a;
            a.proj = proj_;
            a.proj_stride = (size_t)proj_w_;
            a.norms = L.norms;
            a.inv_freq = m_.inv_freq_;
            a.k_pool = kpool_[li];
            a.v_pool = vpool_[li];
            a.block_table = block_table_;
            a.pos = pos_;
            a.qbuf = qbuf_;
            a.part_ml = attn_ml_;
            a.part_acc = attn_acc_;
            a.out = mixed_;
            a.nq = c.n_q_heads;
            a.nkv = c.n_kv_heads;
            a.rope_dim = c.rope_dim;
            a.splits = splits;
            a.order = order_;
            a.max_blocks = max_blocks_;
            a.rows = n;
            a.bt_stride = max_blocks_;
            a.part = part_;
            a.in_splits = in_splits;
            a.in_n = L.in.rows;
            a.split_stride = split_stride;
            a.x_in = frag_a_;
            a.k_in = L.in.k;
            a.eps = c.eps;
            a.gate_dst = proj_;
            a.out = nullptr;
            a.frag_out = frag_b_;  // the out-projection's operand
            a.order_out = order(L.out);
            launch_attention_rows(a, stream_);
        } else {
            GdnRowStrides rs;
            rs.proj = (size_t)proj_w_;
            rs.conv = conv_floats_;
            rs.state = rec_floats_;
            rs.out = (size_t)L.out.k;
            GdnRowsIO io;
            io.part = part_;
            io.splits = in_splits;
            io.n = L.in.rows;
            io.split_stride = split_stride;
            io.x_in = frag_a_;
            io.k_in = L.in.k;
            io.eps = c.eps;
            io.frag_out = frag_b_;  // the out-projection's operand
            io.order_out = order(L.out);
            launch_gdn_decode_rows(nullptr, conv_[li], L.conv_w, rec_[li], nullptr, L.gdn_params, c.gdn_heads, n, rs,
                                   stream_, io);
        }
        // h += W_out mixed; stage RMSNorm(h, post_norm) for gate_up
        gemm(L.out, frag_b_, 0, h_, c.hidden, EPI_ACCUMULATE, frag_a_, L.post_norm, order(L.gate_up));
        // act = SwiGLU(W_gu RMSNorm(h)), staged for down
        gemm(L.gate_up, frag_a_, 1, nullptr, 0, EPI_SWIGLU, frag_b_, nullptr, order(L.down));
        // h += W_down act; stage RMSNorm(h, next gain) for the next layer or the LM head
        const float* next_gain = last ? m_.final_norm_ : m_.layers_[li + 1].input_norm;
        const int next_order = last ? order(m_.lm_head_) : order(m_.layers_[li + 1].in);
        gemm(L.down, frag_b_, 0, h_, c.hidden, EPI_ACCUMULATE, frag_a_, next_gain, next_order);
    }
    gemm(m_.lm_head_, frag_a_, 1, logits_, c.vocab, EPI_STORE, nullptr, nullptr, 0);
    launch_argmax_rows(logits_, n, c.vocab, picks_, tokens_, pos_, am_scratch_, stream_);
}

hipGraphExec_t BatchDecoder::graph_for(int n) {
    auto it = graphs_.find(n);
    if (it != graphs_.end()) return it->second;
    hipGraph_t g = nullptr;
    hipGraphExec_t e = nullptr;
    QNE_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    try {
        enqueue_step(n);
    } catch (...) {
        (void)hipStreamEndCapture(stream_, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    QNE_HIP(hipStreamEndCapture(stream_, &g));
    QNE_HIP(hipGraphInstantiate(&e, g, nullptr, nullptr, 0));
    (void)hipGraphDestroy(g);
    graphs_[n] = e;
    return e;
}

void BatchDecoder::admit(int row) {
    check_row(row);
    uint32_t token = 0, next = 0;
    m_.last_token(&token, &next);
    if ((int)next >= max_context_) throw Error(QNE_ECONTEXT, "the model's sequence does not fit the batch context");
    const size_t nblk = (next + 15) / 16;
    size_t ai = 0;
    for (size_t li = 0; li < m_.layers_.size(); li++) {
        const DevLayer& L = m_.layers_[li];
        if (L.attn) {
            const size_t bytes = pool_block_elems_ * 2;
            for (size_t i = 0; i < nblk; i++) {
                const size_t src = (size_t)m_.bt_host_[i] * pool_block_elems_;
                const size_t dst = (size_t)bt_host_[(size_t)row * max_blocks_ + i] * pool_block_elems_;
                QNE_HIP(hipMemcpyAsync(kpool_[li] + dst, L.k_pool + src, bytes, hipMemcpyDeviceToDevice, stream_));
                QNE_HIP(hipMemcpyAsync(vpool_[li] + dst, L.v_pool + src, bytes, hipMemcpyDeviceToDevice, stream_));
            }
            ai++;
        } else {
            QNE_HIP(hipMemcpyAsync(conv_[li] + (size_t)row * conv_floats_, L.conv_state, conv_floats_ * 4,
                                   hipMemcpyDeviceToDevice, stream_));
            QNE_HIP(hipMemcpyAsync(rec_[li] + (size_t)row * rec_floats_, L.rec, rec_floats_ * 4, hipMemcpyDeviceToDevice,
                                   stream_));
        }
    }
    host_u32_[0] = token;
    host_u32_[1] = next;
    QNE_HIP(hipMemcpyAsync(tokens_ + row, host_u32_, 4, hipMemcpyHostToDevice, stream_));
    QNE_HIP(hipMemcpyAsync(pos_ + row, host_u32_ + 1, 4, hipMemcpyHostToDevice, stream_));
    sync();
}

void BatchDecoder::copy_row(int row, BatchDecoder& src, int src_row) {
    check_row(row);
    src.check_row(src_row);
    if (&src.m_ != &m_) throw Error(QNE_EINVAL, "the batches decode different models");
    uint32_t token = 0, next = 0;
    {
        uint32_t t[kRowsMax], p[kRowsMax];
        src.row_state(src_row + 1, t, p);
        token = t[src_row];
        next = p[src_row];
    }
    if ((int)next >= max_context_) throw Error(QNE_ECONTEXT, "the row's sequence does not fit the batch context");
    if (&src == this && src_row == row) return;
    const size_t nblk = (next + 15) / 16;
    for (size_t li = 0; li < m_.layers_.size(); li++) {
        if (m_.layers_[li].attn) {
            const size_t bytes = pool_block_elems_ * 2;
            for (size_t i = 0; i < nblk; i++) {
                const size_t from = (size_t)src.bt_host_[(size_t)src_row * src.max_blocks_ + i] * pool_block_elems_;
                const size_t to = (size_t)bt_host_[(size_t)row * max_blocks_ + i] * pool_block_elems_;
                QNE_HIP(hipMemcpyAsync(kpool_[li] + to, src.kpool_[li] + from, bytes, hipMemcpyDeviceToDevice, stream_));
                QNE_HIP(hipMemcpyAsync(vpool_[li] + to, src.vpool_[li] + from, bytes, hipMemcpyDeviceToDevice, stream_));
            }
        } else {
            QNE_HIP(hipMemcpyAsync(conv_[li] + (size_t)row * conv_floats_, src.conv_[li] + (size_t)src_row * conv_floats_,
                                   conv_floats_ * 4, hipMemcpyDeviceToDevice, stream_));
            QNE_HIP(hipMemcpyAsync(rec_[li] + (size_t)row * rec_floats_, src.rec_[li] + (size_t)src_row * rec_floats_,
                                   rec_floats_ * 4, hipMemcpyDeviceToDevice, stream_));
        }
    }
    host_u32_[0] = token;
    host_u32_[1] = next;
    QNE_HIP(hipMemcpyAsync(tokens_ + row, host_u32_, 4, hipMemcpyHostToDevice, stream_));
    QNE_HIP(hipMemcpyAsync(pos_ + row, host_u32_ + 1, 4, hipMemcpyHostToDevice, stream_));
    sync();
}

void BatchDecoder::reset_row(int row, uint32_t token) {
    check_row(row);
    if (token >= (uint32_t)m_.cfg_.vocab) throw Error(QNE_EINVAL, "token id out of range");
    for (size_t li = 0; li < m_.layers_.size(); li++) {
        if (m_.layers_[li].attn) continue;
        QNE_HIP(hipMemsetAsync(conv_[li] + (size_t)row * conv_floats_, 0, conv_floats_ * 4, stream_));
        QNE_HIP(hipMemsetAsync(rec_[li] + (size_t)row * rec_floats_, 0, rec_floats_ * 4, stream_));
    }
    host_u32_[0] = token;
    host_u32_[1] = 0;
    QNE_HIP(hipMemcpyAsync(tokens_ + row, host_u32_, 4, hipMemcpyHostToDevice, stream_));
    QNE_HIP(hipMemcpyAsync(pos_ + row, host_u32_ + 1, 4, hipMemcpyHostToDevice, stream_));
    sync();
}

void BatchDecoder::row_state(int n, uint32_t* tokens, uint32_t* pos) {
    if (n < 1 || n > max_rows_) throw Error(QNE_EINVAL, "rows must be 1..max_rows");
    QNE_HIP(hipMemcpyAsync(host_u32_, tokens_, n * 4, hipMemcpyDeviceToHost, stream_));
    QNE_HIP(hipMemcpyAsync(host_u32_ + kRowsMax, pos_, n * 4, hipMemcpyDeviceToHost, stream_));
    sync();
    if (tokens) std::memcpy(tokens, host_u32_, n * 4);
    if (pos) std::memcpy(pos, host_u32_ + kRowsMax, n * 4);
}

void BatchDecoder::step(int n, const uint32_t* tokens, uint32_t* next, float* logits, size_t logits_cap) {
    if (n < 1 || n > max_rows_) throw Error(QNE_EINVAL, "rows must be 1..max_rows");
    const ModelConfig& c = m_.cfg_;
    if (logits && logits_cap < (size_t)n * c.vocab) throw Error(QNE_EINVAL, "logits buffer smaller than rows * vocab");
    uint32_t pos[kRowsMax];
    row_state(n, nullptr, pos);
    for (int r = 0; r < n; r++)
        if ((int)pos[r] >= max_context_) throw Error(QNE_ECONTEXT, "a row is at the end of its context");
    if (tokens) {
        for (int r = 0; r < n; r++)
            if (tokens[r] >= (uint32_t)c.vocab) throw Error(QNE_EINVAL, "token id out of range");
        std::memcpy(host_u32_, tokens, n * 4);
        QNE_HIP(hipMemcpyAsync(tokens_, host_u32_, n * 4, hipMemcpyHostToDevice, stream_));
    }
    QNE_HIP(hipGraphLaunch(graph_for(n), stream_));
    QNE_HIP(hipMemcpyAsync(host_u32_, picks_, n * 4, hipMemcpyDeviceToHost, stream_));
    if (logits) QNE_HIP(hipMemcpyAsync(logits, logits_, (size_t)n * c.vocab * 4, hipMemcpyDeviceToHost, stream_));
    sync();
    if (next) std::memcpy(next, host_u32_, n * 4);
}

void BatchDecoder::decode(int n, int steps, uint32_t* out, size_t cap) {
    if (n < 1 || n > max_rows_) throw Error(QNE_EINVAL, "rows must be 1..max_rows");
    if (steps < 0) throw Error(QNE_EINVAL, "steps must be >= 0");
    if (out && cap < (size_t)n * steps) throw Error(QNE_EINVAL, "output buffer smaller than rows * steps");
    uint32_t pos[kRowsMax];
    row_state(n, nullptr, pos);
    for (int r = 0; r < n; r++)
        if ((int)pos[r] + steps > max_context_) throw Error(QNE_ECONTEXT, "a row would run past its context");
    if (steps == 0) return;
    hipGraphExec_t g = graph_for(n);
    uint32_t* ids = nullptr;
    if (out) ids = (uint32_t*)dalloc((size_t)n * steps * 4);
    QNE_HIP(hipEventRecord(ev0_, stream_));
    for (int s = 0; s < steps; s++) {
        QNE_HIP(hipGraphLaunch(g, stream_));
        if (ids) QNE_HIP(hipMemcpyAsync(ids + (size_t)s * n, picks_, n * 4, hipMemcpyDeviceToDevice, stream_));
    }
    QNE_HIP(hipEventRecord(ev1_, stream_));
    if (ids) QNE_HIP(hipMemcpyAsync(out, ids, (size_t)n * steps * 4, hipMemcpyDeviceToHost, stream_));
    sync((double)steps);
    float ms = 0.0f;
    QNE_HIP(hipEventElapsedTime(&ms, ev0_, ev1_));
    last_ms_ = ms;
    last_steps_ = (size_t)steps;
    if (ids) {
        QNE_HIP(hipFree(ids));
        allocations_.pop_back();
    }
}

void BatchDecoder::fill_synthetic(int n, const uint32_t* ctx, uint64_t seed) {
    if (n < 1 || n > max_rows_) throw Error(QNE_EINVAL, "rows must be 1..max_rows");
    const ModelConfig& c = m_.cfg_;
    for (int r = 0; r < n; r++)
        if ((int)ctx[r] >= max_context_) throw Error(QNE_ECONTEXT, "context length past the batch context");
    uint64_t stream = 0;
    for (size_t li = 0; li < m_.layers_.size(); li++) {
        if (m_.layers_[li].attn) {
            const size_t e = (size_t)max_rows_ * max_blocks_ * pool_block_elems_;
            launch_fill_uniform(kpool_[li], e, true, seed + 1000003ull * ++stream, 1.7320508f, stream_);  // variance 1
            launch_fill_uniform(vpool_[li], e, true, seed + 1000003ull * ++stream, 1.7320508f, stream_);
        } else {
            launch_fill_uniform(conv_[li], (size_t)n * conv_floats_, false, seed + 1000003ull * ++stream, 0.05f, stream_);
            launch_fill_uniform(rec_[li], (size_t)n * rec_floats_, false, seed + 1000003ull * ++stream, 0.05f, stream_);
        }
    }
    std::mt19937_64 rng(seed);
    for (int r = 0; r < n; r++) {
        host_u32_[r] = (uint32_t)(rng() % (uint64_t)c.vocab);
        host_u32_[kRowsMax + r] = ctx[r];
    }
    QNE_HIP(hipMemcpyAsync(tokens_, host_u32_, n * 4, hipMemcpyHostToDevice, stream_));
    QNE_HIP(hipMemcpyAsync(pos_, host_u32_ + kRowsMax, n * 4, hipMemcpyHostToDevice, stream_));
    QNE_HIP(hipGetLastError());
    sync();
}

}  // namespace qne
