// The decoder behind the C ABI: the `Model` of kernels/src/model.rs rebuilt on HIP for MI355X.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "index.hpp"

namespace qne {

struct DevMat {
    int kind = 0;  // 0 f16, 1 q4
    int rows = 0, k = 0, group = 64;
    const void* w = nullptr;
    const uint32_t* sz = nullptr;  // q4: (scale, zero) f16 pairs per group, [row][group]
    // q4: the same words tile-major, [row / 32][group][row % 32] (rows padded to 32 with zeros), so
    // that the row-tiled GEMM reads a tile's 32 words of a group from one 128-byte line
    const uint32_t* szt = nullptr;
};

struct DevLayer {
    bool attn = false;
    DevMat in, out, gate_up, down;
    const float* input_norm = nullptr;
    const float* post_norm = nullptr;
    const float* norms = nullptr;       // attention: q_norm, k_norm
    const float* conv_w = nullptr;      // GDN
    const float* gdn_params = nullptr;  // GDN
    float* conv_state = nullptr;
    float* rec = nullptr;
    uint16_t* k_pool = nullptr;
    uint16_t* v_pool = nullptr;
};

struct LoadOptions {
    int max_context = 4096;
    int device = 0;
    bool graph_engine = false;  // per-kernel hipGraph path instead of the persistent kernel
    bool prefill_graphs = true;  // prefill_chunk passes replay captured graphs (false: direct launches)
    bool gdn_fusion = true;      // persistent kernel: GDN in-projection and step in one phase where the shapes allow
    bool mfma_gemv = true;       // persistent kernel: q4 GEMVs on the int8 matrix cores where the shapes allow
    bool gemm_fusion = true;     // prefill GEMMs with one split apply their epilogue and staging themselves
};

struct EngineRun {
    int feed = 0;          // 0: ids, 1: greedy feedback from tok[0]
    int head = 0;          // 0 none, 1 every step, 2 last step
    int argmax = 0;
    int n_steps = 1;
    uint32_t pos0 = 0;
    bool record_ids = false;
    unsigned long long* trace = nullptr;
    unsigned long long* sub = nullptr;
    int trace_cap = 0;
};

LoadOptions parse_options(const char* json);

class ChunkPrefill;

class Model {
  public:
    Model(const ModelIndex& ix, const uint8_t* weights, uint64_t wlen, const LoadOptions& opt);
    ~Model();
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    void reset();
    void prefill(const uint32_t* ids, size_t n);
    void prefill_chunk(const uint32_t* ids, size_t n, uint32_t start, bool finish_logits);
    void logits(float* out, size_t cap);
    void step(uint32_t token, uint32_t pos, float* out, size_t cap);
    // step without the logits readback: they stay in device_logits() (for DeviceSampler).
    void step_device(uint32_t token, uint32_t pos);
    const float* device_logits() const { return logits_; }
    void snapshot();
    void restore();
    void last_token(uint32_t* token, uint32_t* next_pos);
    // Model::decode (model.rs:426-449): a window of more than one step yields u32::MAX placeholders.
    size_t decode(size_t n, uint32_t window, const uint32_t* stop, size_t nstop, uint32_t* out, size_t cap);
    // The same loop returning every id of every window and stopping after the first stop id.
    size_t decode_ids(size_t n, uint32_t window, const uint32_t* stop, size_t nstop, uint32_t* out, size_t cap);
    double profile_token();
    // One greedy decode token with the device timeline on; JSON of per-phase times (persistent
    // engine only).
    std::string profile_token_json();
    void last_decode_timing(double* ms, size_t* steps) const {
        *ms = last_decode_ms_;
        *steps = last_decode_steps_;
    }

    size_t dispatches_per_token() const { return dispatches_; }
    const std::string& adapter() const { return adapter_; }
    uint32_t vocab() const { return (uint32_t)cfg_.vocab; }
    uint32_t max_context() const { return (uint32_t)max_context_; }

  private:
    friend class BatchDecoder;
    friend class ChunkPrefill;
    void release();
    void upload(const ModelIndex& ix, const uint8_t* weights);
    void alloc_state();
    void build_graphs();
    void enqueue_layers();
    void enqueue_head(bool greedy);
    void set_tok(uint32_t token, uint32_t pos);
    void run_layers_graph();
    void run_head_graph(bool greedy);
    void setup_engine();
    void run_engine(const EngineRun& r);
    void check_engine_error();
    void sync();
    size_t decode_loop(size_t n, uint32_t window, const uint32_t* stop, size_t nstop, uint32_t* out, size_t cap,
                       bool every_id);
    void* dalloc(size_t bytes);

    ModelConfig cfg_;
    int max_context_ = 4096;
    int device_ = 0;
    hipStream_t stream_ = nullptr;
    std::string adapter_;
    std::vector<void*> allocations_;

    DevMat embed_, lm_head_;
    const float* final_norm_ = nullptr;
    std::vector<DevLayer> layers_;

    // state (cleared by reset, copied by snapshot)
    void* state_ = nullptr;
    size_t state_bytes_ = 0;
    void* saved_ = nullptr;

    // activations and bookkeeping
    float *h_ = nullptr, *proj_ = nullptr, *mixed_ = nullptr, *act_ = nullptr, *logits_ = nullptr, *qbuf_ = nullptr;
    float *part_ml_ = nullptr, *part_acc_ = nullptr, *am_val_ = nullptr, *inv_freq_ = nullptr;
    uint32_t *am_idx_ = nullptr, *tok_ = nullptr, *tok_backup_ = nullptr, *ids_ = nullptr, *out_ids_ = nullptr;
    unsigned* am_counter_ = nullptr;
    int32_t* block_table_ = nullptr;
    std::vector<int32_t> bt_host_;  // host copy of block_table_
    int attn_splits_ = 1;
    uint32_t* host_tok_ = nullptr;  // pinned
    float* host_logits_ = nullptr;  // pinned
    uint32_t* host_ids_ = nullptr;  // pinned

    hipGraphExec_t g_layers_ = nullptr, g_head_logits_ = nullptr, g_head_greedy_ = nullptr;
    hipEvent_t ev_start_ = nullptr, ev_stop_ = nullptr;
    bool use_graphs_ = true;
    // persistent engine
    bool persistent_ = true;
    bool prefill_graphs_ = true;  // ChunkPrefill replays captured graphs (else launches directly)
    bool gdn_fusion_ = true;      // the decode program fuses each GDN layer's in-projection and step
    bool gemm_fusion_ = true;     // prefill GEMMs with one split apply their epilogue (no reduce pass)
    bool mfma_gemv_ = true;       // the decode program runs q4 GEMVs tiled on the matrix cores
    std::vector<std::string> phase_label_;  // per decode-program phase, for the profile
    int engine_grid_ = 0;
    void* engine_args_ = nullptr;  // host copy of DecodeArgs (opaque here)
    unsigned* eng_bar_ = nullptr;  // [0] error flag of the decode kernel
    uint64_t* exch_ = nullptr;     // tagged exchange buffers of the decode program
    size_t exch_bytes_ = 0;
    uint64_t* am_ = nullptr;       // argmax exchange
    int nph_ = 0;                  // phases per token
    std::vector<int> phase_kind_;  // PhaseKind of each phase (profile labels)
    uint32_t tag_base_ = 1;
    unsigned* host_err_ = nullptr;  // pinned
    double last_decode_ms_ = 0.0;
    size_t last_decode_steps_ = 0;
    size_t dispatches_ = 0;
    size_t launches_ = 0;  // kernel launches counted while recording
    double pending_units_ = 0.0;  // dependent device steps enqueued since the last sync (its deadline)
    // prefill_chunk on the batched GEMM (created on first use; null when the shapes do not fit it)
    ChunkPrefill* chunk_ = nullptr;
    bool chunk_tried_ = false;
};

}  // namespace qne
