// Batched continuous decode: up to 64 sequences ("rows") advance one token per step through the
// weights of a loaded Model, each row with its own paged KV cache and recurrent state.
//
// The reference decodes one sequence at a time (kernels/src/model.rs:372-449) and batches only the
// 16-token prefill GEMM (kernels/src/batch.rs:12-99); this object applies that GEMM form across
// sequences so the weights are read once per step for every row.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <vector>

#include "model.hpp"

namespace qne {

// One GEMM of a pass over up to 512 rows (a batched decode step of up to 64, or a prefill pass),
// with its reduce, the split count chosen for row_tiles tiles of 64 rows: W applied to the x
// operand staged in `frag` (norm: its rows carry a deferred RMSNorm), epilogue into y, and with
// frag_out the result staged for the next GEMM (times gain_out). partials_only: only the split
// partials are written (into part); the kernel that reads the output sums them. fuse: a GEMM with
// one split may apply its epilogue and staging itself (false: always the reduce pass; the same
// results).
void rows_gemm(const DevMat& W, int n, float eps, uint8_t* frag, int norm, float* part, float* y, int y_stride,
               int epi, uint8_t* frag_out, const float* gain_out, int order_out, hipStream_t st, int row_tiles = 1,
               bool partials_only = false, bool fuse = true);
// 1 when a GEMM on W takes its x operand in the q4 column order.
int operand_order(const DevMat& W);
// Throws QNE_EFORMAT unless the model's shapes fit the batched kernels.
void rows_shapes_check(const ModelConfig& c);
// Scratch of the GEMMs of a pass of up to `rows` rows over the layers, with the split counts of
// gemm_splits(..., row_tiles): split partials (floats) and one staged x operand (bytes). Throws
// when a matrix shape is not supported by the batched GEMM.
void rows_workspace(const std::vector<DevLayer>& layers, const DevMat& head, int rows, int row_tiles, size_t* part_floats,
                    size_t* frag_bytes);

class BatchDecoder {
  public:
    BatchDecoder(Model& m, int max_rows, int max_context);
    ~BatchDecoder();
    BatchDecoder(const BatchDecoder&) = delete;
    BatchDecoder& operator=(const BatchDecoder&) = delete;

    int max_rows() const { return max_rows_; }
    int max_context() const { return max_context_; }
    // Row `row` takes over the model's current sequence: its KV cache and recurrent state, and its
    // next (token, position) as reported by Model::last_token.
    void admit(int row);
    // Row `row` takes over row `src_row` of `src` (a batch over the same model; `src` may be this
    // batch): its KV cache, recurrent state, next token and position.
    void copy_row(int row, BatchDecoder& src, int src_row);
    // Row `row` becomes an empty sequence (position 0, zero state) whose next token is `token`.
    void reset_row(int row, uint32_t token);
    // The next (token, position) of rows 0..n-1.
    void row_state(int n, uint32_t* tokens, uint32_t* pos);
    // One step of rows 0..n-1. With `tokens` set, those tokens replace the rows' next tokens first.
    // Writes each row's greedy pick to `next` (n entries) and, when `logits` is set, the rows'
    // logits (n * vocab floats). Every row's next token becomes its pick and its position advances.
    void step(int n, const uint32_t* tokens, uint32_t* next, float* logits, size_t logits_cap);
    // `steps` greedy steps of rows 0..n-1 chained on the device; out[s * n + r] = pick of row r at
    // step s.
    void decode(int n, int steps, uint32_t* out, size_t cap);
    // Benchmark set-up: rows 0..n-1 get pseudo-random KV contents and recurrent state, random next
    // tokens, and positions ctx[r].
    void fill_synthetic(int n, const uint32_t* ctx, uint64_t seed);
    double last_ms() const { return last_ms_; }
    size_t last_steps() const { return last_steps_; }

  private:
    void release();
    void* dalloc(size_t bytes);
    void enqueue_step(int n);
    hipGraphExec_t graph_for(int n);
    void check_row(int row) const;
    void sync(double steps = 1.0);  // waits with a deadline for `steps` batched steps

    Model& m_;
    int max_rows_, max_context_, max_blocks_;
    hipStream_t stream_ = nullptr;
    std::vector<void*> allocations_;
    std::map<int, hipGraphExec_t> graphs_;
    hipEvent_t ev0_ = nullptr, ev1_ = nullptr;

    // per layer: rows x state
    std::vector<float*> conv_, rec_;
    std::vector<uint16_t*> kpool_, vpool_;
    size_t conv_floats_ = 0, rec_floats_ = 0, pool_block_elems_ = 0;
    int32_t* block_table_ = nullptr;  // [max_rows][max_blocks]
    std::vector<int32_t> bt_host_;

    // activations [64][...]
    int proj_w_ = 0, mixed_w_ = 0;
    float *h_ = nullptr, *proj_ = nullptr, *mixed_ = nullptr, *act_ = nullptr, *logits_ = nullptr, *qbuf_ = nullptr;
    float *part_ = nullptr, *attn_ml_ = nullptr, *attn_acc_ = nullptr;
    uint8_t *frag_a_ = nullptr, *frag_b_ = nullptr;  // staged x operands of the GEMMs
    size_t attn_part_rows_ = 0;  // rows * splits the attention partials hold
    uint32_t *tokens_ = nullptr, *picks_ = nullptr, *ids_ = nullptr;
    int32_t* pos_ = nullptr;
    int32_t* order_ = nullptr;  // the step's rows by decreasing position (attention partials' order)
    void* am_scratch_ = nullptr;  // per-row argmax partials
    uint32_t* host_u32_ = nullptr;  // pinned, 2 * 64 entries
    double last_ms_ = 0.0;
    size_t last_steps_ = 0;
};

}  // namespace qne
