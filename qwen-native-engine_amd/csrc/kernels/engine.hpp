// Host-visible description of the persistent decode engine (kernels/engine.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qne {

// A weight matrix in HBM: f16 [rows][k], or q4 nibbles [rows][k/8] with (scale, zero) f16 pairs
// [rows][k/group].
struct EMat {
    const void* w = nullptr;
    const uint32_t* sz = nullptr;
    int kind = 0;  // 0 f16, 1 q4
    int rows = 0, k = 0, group = 64;
};

struct ELayer {
    EMat in, out, gu, down;
    const float* in_norm = nullptr;
    const float* post_norm = nullptr;
    const float* norms = nullptr;   // attention: q_norm, k_norm
    const float* conv_w = nullptr;  // GDN [channels][4]
    const float* prm = nullptr;     // GDN dt_bias[H], A_neg_exp[H], norm_w[dv]
    float* conv = nullptr;          // GDN conv state [channels][3]
    float* rec = nullptr;           // GDN state, value-major [H][dv][dk]
    uint16_t* k_pool = nullptr;     // attention [blocks][nkv][16][hd]
    uint16_t* v_pool = nullptr;
    int attn = 0;
};

struct EngineArgs {
    const ELayer* layers = nullptr;
    int n_layers = 0;
    EMat embed, lm;
    const float* final_norm = nullptr;
    int hidden = 0, inter = 0, vocab = 0;
    int nq = 0, nkv = 0, rope_dim = 64, gdn_heads = 0;
    int max_blocks = 0, splits = 1;
    float eps = 1e-6f;
    const float* inv_freq = nullptr;
    const int32_t* block_table = nullptr;
    // activations
    float* h = nullptr;
    float* proj = nullptr;
    float* mixed = nullptr;
    float* gdn_sq = nullptr;  // per (head, column block) sums of squares of the GDN outputs
    float* act = nullptr;
    float* logits = nullptr;
    float* att_ml = nullptr;   // [nkv][splits][G][2]
    float* att_acc = nullptr;  // [nkv][splits][G][hd]
    unsigned* att_cnt = nullptr;  // [nkv] arrival counters (zero between uses)
    float* am_val = nullptr;
    uint32_t* am_idx = nullptr;
    // tokens
    uint32_t* tok = nullptr;        // {token, pos, n_out, 0}
    const uint32_t* ids = nullptr;  // feed 0: token of step s is ids[s]
    uint32_t* out_ids = nullptr;    // greedy picks appended at tok[2]
    uint32_t out_cap = 0;
    int n_steps = 1;
    uint32_t pos0 = 0;
    int feed = 0;       // 0: tokens from ids, 1: greedy feedback from the previous step's argmax
    int head = 0;       // 0: no LM head, 1: every step, 2: last step only
    int argmax = 0;     // run the greedy pick after the LM head
    // grid barrier
    unsigned* bar = nullptr;
    unsigned* err = nullptr;
    unsigned spin_limit = 1u << 22;
};

constexpr int kEngineThreads = 512;

// Launches the persistent kernel cooperatively (one workgroup per CU). Returns the HIP status.
hipError_t launch_engine(const EngineArgs& a, int grid, hipStream_t st);
// Largest cooperative grid the engine can use on the current device.
int engine_max_grid();

}  // namespace qne
