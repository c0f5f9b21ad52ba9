// Small kernels: embedding row gather (kernels/src/shaders.rs:405-434 reads the row index on the
// device so a GPU-resident decode loop never needs the host), token-slot updates.
#include "gemv.hpp"
#include "launch.hpp"

namespace qne {

// h[c] = W[tok[0]][c] for an f16 table, or the dequantised q4 row (value (q - z) * s).
__global__ void k_embed(int kind, const void* __restrict__ W, const uint32_t* __restrict__ SZ, int group, int hidden,
                        const uint32_t* __restrict__ tok, float* __restrict__ h) {
    const size_t row = tok[0];
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < hidden; c += gridDim.x * blockDim.x) {
        if (kind == KIND_F16) {
            h[c] = h2f(((const uint16_t*)W)[row * hidden + c]);
        } else {
            const uint32_t word = ((const uint32_t*)W)[row * (hidden / 8) + c / 8];
            const float q = (float)((word >> (4 * (c % 8))) & 15u);
            const uint32_t sz = SZ[row * (hidden / group) + c / group];
            h[c] = (q - hi_h(sz)) * lo_h(sz);
        }
    }
}

// tok = {ids[i], pos, tok[2], tok[3]}: the host writes of tok in Model::prefill (model.rs:329),
// done on the device so a whole prompt is one upload.
__global__ void k_set_tok(uint32_t* __restrict__ tok, const uint32_t* __restrict__ ids, int i, uint32_t pos) {
    tok[0] = ids[i];
    tok[1] = pos;
}

void launch_set_tok(uint32_t* tok, const uint32_t* ids, int i, uint32_t pos, hipStream_t st) {
    hipLaunchKernelGGL(k_set_tok, dim3(1), dim3(1), 0, st, tok, ids, i, pos);
}

void launch_embed(int kind, const void* W, const uint32_t* SZ, int group, int hidden, const uint32_t* tok, float* h,
                  hipStream_t st) {
    const int blocks = (hidden + 255) / 256;
    hipLaunchKernelGGL(k_embed, dim3(blocks), dim3(256), 0, st, kind, W, SZ, group, hidden, tok, h);
}

}  // namespace qne
