// ChunkPrefill: model.rs:220-269 over the tokens of a prompt chunk, one HIP graph per chunk length.
#include "prefill.hpp"

#include <algorithm>
#include <cstring>

#include "batch.hpp"
#include "error.hpp"
#include "hip_util.hpp"
#include "kernels/launch.hpp"

namespace qne {

void* ChunkPrefill::dalloc(size_t bytes) {
    void* p = nullptr;
    QNE_HIP(hipMalloc(&p, bytes ? bytes : 16));
    allocations_.push_back(p);
    return p;
}

ChunkPrefill::ChunkPrefill(Model& m) : m_(m), st_(m.stream_) {
    const ModelConfig& c = m.cfg_;
    rows_shapes_check(c);
    size_t part = 0, frag = 0;
    pass_ = std::min(kPassMax, (m.max_context_ + 63) / 64 * 64);
    row_tiles_ = pass_ / 64;
    rows_workspace(m.layers_, m.lm_head_, pass_, row_tiles_, &part, &frag);
    try {
        const size_t T = pass_;
        proj_w_ = std::max(c.attn_proj(), c.gdn_proj());
        // Attention partials over fixed position ranges (kPrefillSplitLen positions each, cut at the
        // row's own position), so that a token's result does not depend on how the prompt was
        // chunked; head groupings the query-tile kernel does not take use per-row partials over
        // a fixed split count.
        const int max_blocks = (m.max_context_ + 15) / 16;
        if (prefill_attention_supported(c.n_q_heads, c.n_kv_heads)) {
            split_len_ = kPrefillSplitLen;
            splits_ = (max_blocks * 16 + split_len_ - 1) / split_len_;
        } else {
            splits_ = std::max(1, std::min(16, max_blocks));
        }
        ids_ = (uint32_t*)dalloc(T * 4);
        pos_ = (int32_t*)dalloc(T * 4);
        h_ = (float*)dalloc(T * c.hidden * 4);
        proj_ = (float*)dalloc(T * proj_w_ * 4);
        qbuf_ = (float*)dalloc(T * c.n_q_heads * c.head_dim * 4);
        part_ = (float*)dalloc(part * 4);
        const size_t G = (size_t)(c.n_q_heads / c.n_kv_heads);
        attn_ml_ = (float*)dalloc(T * c.n_kv_heads * splits_ * G * 2 * 4);
        attn_acc_ = (float*)dalloc(T * c.n_kv_heads * splits_ * G * c.head_dim * 4);
        const size_t hk = T * c.gdn_heads * c.gdn_dk;
        gq_ = (float*)dalloc(hk * 4);
        gk_ = (float*)dalloc(hk * 4);
        gv_ = (float*)dalloc(hk * 4);
        go_ = (float*)dalloc(hk * 4);
        gg_ = (float*)dalloc(T * c.gdn_heads * 4);
        gb_ = (float*)dalloc(T * c.gdn_heads * 4);
        wy_ws_ = (float*)dalloc(wy_workspace_bytes(1, (int)T, c.gdn_heads));
        frag_a_ = (uint8_t*)dalloc(frag);
        frag_b_ = (uint8_t*)dalloc(frag);
        frag_c_ = (uint8_t*)dalloc(frag);
        QNE_HIP(hipMemset(frag_a_, 0, frag));
        QNE_HIP(hipMemset(frag_b_, 0, frag));
        // Only the attention combine and the GDN output write frag_c_ (rows < the pass's tokens), so
        // the rows of a last row tile past them hold zeros or earlier rows' staged values, always
        // finite; the out-projection's rows are independent and those rows are never stored.
        QNE_HIP(hipMemset(frag_c_, 0, frag));
        QNE_HIP(hipHostMalloc((void**)&host_pos_, T * 4, hipHostMallocDefault));
    } catch (...) {
        release();
        throw;
    }
}

ChunkPrefill::~ChunkPrefill() { release(); }

void ChunkPrefill::release() {
    if (st_) (void)hipStreamSynchronize(st_);
    for (auto& g : lru_) (void)hipGraphExecDestroy(g.second);
    lru_.clear();
    graphs_.clear();
    for (void* p : allocations_) (void)hipFree(p);
    allocations_.clear();
    if (host_pos_) (void)hipHostFree(host_pos_);
    host_pos_ = nullptr;
}

// The tokens of one chunk (ids_, positions pos_) through every layer: the same graph as a batched
// decode step (BatchDecoder::enqueue_step) with the rows being consecutive tokens of one sequence.
void ChunkPrefill::enqueue_chunk(int n, int lead) {
    const ModelConfig& c = m_.cfg_;
    const DevLayer& first = m_.layers_.front();
    launch_embed_rows(m_.embed_.kind, m_.embed_.w, m_.embed_.sz, m_.embed_.group, c.hidden, ids_, n, h_, frag_a_,
                      first.input_norm, operand_order(first.in), st_);
    auto gemm = [&](const DevMat& W, uint8_t* frag, int norm, float* y, int y_stride, int epi, uint8_t* frag_out,
                    const float* gain_out, int order_out) {
        rows_gemm(W, n, c.eps, frag, norm, part_, y, y_stride, epi, frag_out, gain_out, order_out, st_, row_tiles_, false,
                  m_.gemm_fusion_);
    };
    const int max_blocks = (m_.max_context_ + 15) / 16;
    for (size_t li = 0; li < m_.layers_.size(); li++) {
        const DevLayer& L = m_.layers_[li];
        const bool last = li + 1 == m_.layers_.size();
        gemm(L.in, frag_a_, 1, proj_, proj_w_, EPI_STORE, nullptr, nullptr, 0);
        if (L.attn) {
            AttnRowsArgs a;
            a.proj = proj_;
            a.proj_stride = (size_t)proj_w_;
            a.norms = L.norms;
            a.inv_freq = m_.inv_freq_;
            a.k_pool = L.k_pool;
            a.v_pool = L.v_pool;
            a.block_table = m_.block_table_;
            a.bt_stride = 0;  // every row is the same sequence
            a.pos = pos_;
            a.qbuf = qbuf_;
            a.part_ml = attn_ml_;
            a.part_acc = attn_acc_;
            a.out = nullptr;  // the combine stages the out-projection's operand itself
            a.frag_out = frag_c_;
            a.order_out = operand_order(L.out);
            a.nq = c.n_q_heads;
            a.nkv = c.n_kv_heads;
            a.rope_dim = c.rope_dim;
            a.splits = splits_;
            a.split_len = split_len_;
            a.max_blocks = max_blocks;
            a.rows = n;
            launch_attention_rows(a, st_);
        } else {
            launch_gdn_chunk(proj_, proj_w_, L.conv_state, L.conv_w, L.rec, L.gdn_params, c.gdn_heads, n, gq_, gk_, gv_,
                             gg_, gb_, go_, nullptr, L.out.k, st_, lead, wy_ws_, frag_c_, operand_order(L.out));
        }
        gemm(L.out, frag_c_, 0, h_, c.hidden, EPI_ACCUMULATE, frag_a_, L.post_norm, operand_order(L.gate_up));
        gemm(L.gate_up, frag_a_, 1, nullptr, 0, EPI_SWIGLU, frag_b_, nullptr, operand_order(L.down));
        // the last layer's h is read by the LM head of the model (one token), not by a GEMM
        const float* next_gain = last ? nullptr : m_.layers_[li + 1].input_norm;
        gemm(L.down, frag_b_, 0, h_, c.hidden, EPI_ACCUMULATE, last ? nullptr : frag_a_, next_gain,
             last ? 0 : operand_order(m_.layers_[li + 1].in));
    }
}

hipGraphExec_t ChunkPrefill::graph_for(int n, int lead) {
    const int key = graph_key(n, lead);
    auto it = graphs_.find(key);
    if (it != graphs_.end()) {
        lru_.splice(lru_.begin(), lru_, it->second);  // now the most recently used
        return it->second->second;
    }
    if (lru_.size() >= kGraphCap) {
        // drop the least recently used graph; the stream is idle (run() synchronizes before every
        // pass), so no launch of it is pending
        QNE_HIP(hipStreamSynchronize(st_));
        (void)hipGraphExecDestroy(lru_.back().second);
        graphs_.erase(lru_.back().first);
        lru_.pop_back();
    }
    hipGraph_t g = nullptr;
    hipGraphExec_t e = nullptr;
    QNE_HIP(hipStreamBeginCapture(st_, hipStreamCaptureModeThreadLocal));
    try {
        enqueue_chunk(n, lead);
    } catch (...) {
        (void)hipStreamEndCapture(st_, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    QNE_HIP(hipStreamEndCapture(st_, &g));
    QNE_HIP(hipGraphInstantiate(&e, g, nullptr, nullptr, 0));
    (void)hipGraphDestroy(g);
    lru_.emplace_front(key, e);
    graphs_[key] = lru_.begin();
    return e;
}

void ChunkPrefill::run(const uint32_t* ids_dev, size_t n, uint32_t start, bool finish_logits) {
    const ModelConfig& c = m_.cfg_;
    int last = 0;
    for (size_t off = 0; off < n; off += (size_t)pass_) {
        const int t = (int)std::min<size_t>((size_t)pass_, n - off);
        // the previous chunk's graph has read pos_ before these copies run (same stream)
        QNE_HIP(hipStreamSynchronize(st_));
        for (int i = 0; i < t; i++) host_pos_[i] = (int32_t)(start + off + i);
        QNE_HIP(hipMemcpyAsync(pos_, host_pos_, t * 4, hipMemcpyHostToDevice, st_));
        QNE_HIP(hipMemcpyAsync(ids_, ids_dev + off, t * 4, hipMemcpyDeviceToDevice, st_));
        // tokens until the next multiple of 64 positions: the GDN blocks after them are fixed by
        // absolute position, so calls cut at multiples of 64 give the same bits
        const int lead = (int)((64 - (start + off) % 64) % 64);
        if (m_.prefill_graphs_) QNE_HIP(hipGraphLaunch(graph_for(t, lead), st_));
        else enqueue_chunk(t, lead);  // the same kernels, launched one by one
        last = t;
    }
    if (finish_logits) {
        // model.rs:361-367: tok = [0, start + n - 1], the last token's h, the LM head and the pick
        // (which advances tok[1] to start + n)
        QNE_HIP(hipMemcpyAsync(m_.h_, h_ + (size_t)(last - 1) * c.hidden, (size_t)c.hidden * 4, hipMemcpyDeviceToDevice,
                               st_));
        m_.host_tok_[8] = 0;
        m_.host_tok_[9] = start + (uint32_t)n - 1;
        m_.host_tok_[10] = 0;
        m_.host_tok_[11] = 0;
        QNE_HIP(hipMemcpyAsync(m_.tok_, m_.host_tok_ + 8, 16, hipMemcpyHostToDevice, st_));
        m_.enqueue_head(true);
    }
    QNE_HIP(hipGetLastError());
}

}  // namespace qne
