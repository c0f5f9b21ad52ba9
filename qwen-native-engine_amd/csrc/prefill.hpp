// Chunked prefill on the batched GEMM: Model::prefill_chunk (kernels/src/model.rs:349-372) runs
// the prompt up to 512 tokens per pass, as the reference's prefill_batched runs 16
// (kernels/src/batch.rs). A pass's tokens are the rows of one pass through the layers: every
// projection is one MFMA GEMM over the pass (in tiles of 64 rows, so the weights stream once per
// pass), attention appends the pass's K/V and each token attends positions up to its own (causal by
// construction), and the GDN recurrence runs over the pass's tokens in order on the model's state.
// The LM head runs on the last token only. The GEMMs' split counts are fixed for the model (those
// of a full pass), so a token's result does not depend on how the prompt is cut into calls.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <list>
#include <map>
#include <utility>
#include <vector>

#include "model.hpp"

namespace qne {

class ChunkPrefill {
  public:
    // Tokens per pass: 2048, or the context rounded up to 64 if smaller (fixed per model, so the
    // GEMMs' split counts, chosen for a full pass, are too). Longer passes stream each weight matrix
    // over more rows: a 4000-id prompt took 0.079 s in 512-token passes, 0.067 s in 1024, 0.061 s
    // in 2048 and 0.060 s in one pass.
    static constexpr int kPassMax = 2048;
    static constexpr size_t kGraphCap = 48;  // instantiated pass graphs kept (least recently used dropped)
    explicit ChunkPrefill(Model& m);
    ~ChunkPrefill();
    ChunkPrefill(const ChunkPrefill&) = delete;
    ChunkPrefill& operator=(const ChunkPrefill&) = delete;

    // Tokens ids_dev[0..n) (device) at positions start..start+n-1 on the model's state; with
    // finish_logits, the LM head and greedy pick of the last one (tok = [pick, start + n]).
    void run(const uint32_t* ids_dev, size_t n, uint32_t start, bool finish_logits);

  private:
    void release();
    void* dalloc(size_t bytes);
    // one pass of n tokens whose first `lead` tokens end at a multiple of 64 positions (the GDN
    // recurrence runs the whole 64-position blocks after them in the WY form)
    void enqueue_chunk(int n, int lead);
    hipGraphExec_t graph_for(int n, int lead);

  public:
    // The launch sequence of a pass depends on n and on the sequential head min(lead, n) only (the
    // WY block count and the sequential tail follow from them): the graph cache key.
    static int graph_key(int n, int lead) { return n * 64 + std::min(std::max(lead, 0), n); }
    size_t graphs_cached() const { return lru_.size(); }

  private:

    Model& m_;
    hipStream_t st_;
    std::vector<void*> allocations_;
    // instantiated pass graphs by graph_key, most recently used first (at most kGraphCap)
    std::list<std::pair<int, hipGraphExec_t>> lru_;
    std::map<int, std::list<std::pair<int, hipGraphExec_t>>::iterator> graphs_;
    static constexpr int kPrefillSplitLen = 1024;  // positions per attention split of the query-tile kernel
    int pass_ = 0, row_tiles_ = 0;  // tokens per pass, its 64-row tiles
    int proj_w_ = 0, splits_ = 1, split_len_ = 0;
    uint32_t* ids_ = nullptr;  // the chunk's token ids
    int32_t* pos_ = nullptr;   // the chunk's positions
    int32_t* host_pos_ = nullptr;  // pinned
    float *h_ = nullptr, *proj_ = nullptr, *qbuf_ = nullptr, *part_ = nullptr;
    float *attn_ml_ = nullptr, *attn_acc_ = nullptr;
    float *gq_ = nullptr, *gk_ = nullptr, *gv_ = nullptr, *go_ = nullptr, *gg_ = nullptr, *gb_ = nullptr;
    float* wy_ws_ = nullptr;  // the WY form's per-chunk operands
    // GEMM operands: the in-projection and gate_up input (a), the down input (b), the
    // out-projection input, staged by the attention combine and the GDN output (c)
    uint8_t *frag_a_ = nullptr, *frag_b_ = nullptr, *frag_c_ = nullptr;
};

}  // namespace qne
