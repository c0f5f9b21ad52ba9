// Chunked gated delta rule in the WY (UT) form on f32 MFMA, for multi-token calls
// (qne_gdn_prefill_chunked). Same math as the sequential recurrence of kernels/src/batch.rs:166-255
// (gdn_b) and kernels/src/shaders.rs:436-520 (gdn), per token t and value column:
//     d_t = beta_t (v_t - g_t S^T k_t),  S <- g_t S + k_t d_t^T,  o_t = S^T q_t.
//
// Over a chunk of C = 64 positions with L_i = sum_{j<=i} log g_j, gamma_i = exp(L_i) and the state
// S0 on entry, unrolling the recurrence gives (rows = positions):
//     (I + A) D = diag(beta) V - diag(beta gamma) K S0,   A_ij = beta_i e^{L_i - L_j} k_i.k_j (j < i)
//     D = U - W S0,   T = (I + A)^-1,  U = T diag(beta) V,  W = T diag(beta gamma) K
//     O = diag(gamma) Q S0 + P D,      P_ij = e^{L_i - L_j} q_i.k_j (j <= i)
//     S_C = gamma_{C-1} S0 + sum_j e^{L_{C-1} - L_j} k_j d_j^T.
// Only the last two lines depend on S0, so the chunk-parallel part (A, T, U, W, P) runs for every
// chunk at once and the chain over chunks is four small GEMMs per chunk.
//
// Design for gfx950:
//  - k_wy_prep: one 256-thread workgroup per (sequence, head, chunk). K and Q of the chunk sit in
//    LDS (A and T then take Q's place), V in registers, 66 KiB of LDS: two workgroups per CU;
//    K K^T and K Q^T run on v_mfma_f32_16x16x4f32 (only the lower-triangle tiles: each wave
//    gets five), T is inverted in 16 x 16 blocks (forward substitution on the diagonal blocks, MFMA
//    for the rest), and U, W^T are again MFMA over the triangular T. The results are written
//    in the exact register-fragment order in which the chain kernel feeds them to the MFMA.
//  - k_wy_chain: one wave per (sequence, head, 16 value columns), the 128 x 16 state slice in 32
//    VGPRs for the whole sequence. The contraction index of every chain GEMM is ordered so that the
//    accumulator of one MFMA is the B operand of the next with no data movement: state register r
//    of key tile kt is the B operand of the step that contracts keys 16kt + 4g + r (g = lane / 16),
//    and D likewise over positions. A workgroup is four column waves of one (sequence, head); the
//    chunk's operands (W, U, P, q, the decayed K^T, L: 128 KiB) are staged once per workgroup in
//    LDS by global_load_lds, each buffer refilled for the next chunk as soon as its phase of the
//    current chunk (D, output, state) is done, so the copies overlap two phases of MFMA work. The
//    two workgroups of a (sequence, head) run on one XCD (workgroups are dealt to XCDs round robin),
//    so they share the chunk operands in its L2.
// Positions past the sequence end are padding: k = q = v = 0, beta = 0, g = 1, which leaves the
// state and every real output unchanged.
#include "common.hpp"
#include "launch.hpp"
#include "lds_dma.hpp"

namespace qne {

namespace {

using namespace lds_dma;

constexpr int kC = 64;     // positions per chunk
constexpr int kD = 128;    // dk = dv
constexpr int kKS = 132;   // LDS row stride (floats) of K and Q: rows 16 apart x 4 columns on distinct banks
constexpr int kAS = 68;    // LDS row stride of the A / T matrix
// Per (sequence, head, chunk) workspace, in floats:
//  Wf [pt 4][kt 8][lane 64][4]: -W[16pt + lane%16][16kt + 4(lane/16) + r]
//  Uf [pt 4][cg 8][lane 64][4]:  U[16pt + 4(lane/16) + r][16cg + lane%16]
//  Pf [it 4][pt 4][lane 64][4]:  P[16it + lane%16][16pt + 4(lane/16) + r]
//  Kf [kt 8][pt 4][lane 64][4]:  e^{L_63 - L_p} K[p][16kt + lane%16], p = 16pt + 4(lane/16) + r
//  Lf [64]: L_i / ln 2 (padding repeats the last real position's value)
constexpr int kWfOff = 0, kUfOff = 8192, kPfOff = 16384, kKfOff = 20480, kLfOff = 28672, kWyFloats = 28736;

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Sum over the four lanes of a quad.
__device__ __forceinline__ float quad_sum(float v) {
    v += QNE_DPP(v, 0xB1);  // quad_perm [1, 0, 3, 2]
    v += QNE_DPP(v, 0x4E);  // quad_perm [2, 3, 0, 1]
    return v;
}

__global__ __launch_bounds__(256) void k_wy_prep(const float* __restrict__ q, const float* __restrict__ k,
                                                 const float* __restrict__ v, const float* __restrict__ beta,
                                                 const float* __restrict__ g, float* __restrict__ ws, int T, int H) {
    __shared__ __attribute__((aligned(16))) float Ks[kC * kKS];
    // q, then A and T (stride kAS) once every wave has read q: 66 KiB in all, so two workgroups
    // share a CU. V goes to registers instead (each lane's 32 values of its wave's U columns).
    __shared__ __attribute__((aligned(16))) float Qs[kC * kKS];
    float* const As = Qs;
    static_assert(kAS <= kKS, "A / T fit the q buffer");
    __shared__ float Ls[kC], Bs[kC], BGs[kC], Ds[kC];
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z, NC = gridDim.x;
    const int t0 = c * kC, n = min(kC, T - t0);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    float* out = ws + ((size_t)(b * H + h) * NC + c) * kWyFloats;
    const size_t row0 = ((size_t)b * T + t0) * H + h;  // (position t0, head h) of sequence b

    // K and Q rows by LDS DMA (one row per instruction, 32 lanes); padding rows zeroed by stores
#pragma unroll
    for (int u = 0; u < kC / 4; u++) {
        const int t = w * (kC / 4) + u;
        if (lane < 32) {
            if (t < n) {
                dma16(k + (row0 + (size_t)t * H) * kD + 4 * lane, Ks + t * kKS);
                dma16(q + (row0 + (size_t)t * H) * kD + 4 * lane, Qs + t * kKS);
            } else {
                *(f4*)(Ks + t * kKS + 4 * lane) = f4{0.0f, 0.0f, 0.0f, 0.0f};
                *(f4*)(Qs + t * kKS + 4 * lane) = f4{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    }
    if (w == 0) {
        // L in log2 units: every decay product below is one hardware exp2
        const int t = lane;
        float lgv = 0.0f, bt = 0.0f;
        if (t < n) {
            // a decay below 2^-115 is taken as 2^-115 (its products vanish either way)
            lgv = fmaxf(__log2f(g[row0 + (size_t)t * H]), -115.0f);
            bt = beta[row0 + (size_t)t * H];
        }
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float u = __shfl_up(lgv, o, 64);
            if (lane >= o) lgv += u;
        }
        Ls[t] = lgv;
        Bs[t] = bt;
        BGs[t] = bt * __builtin_amdgcn_exp2f(lgv);
        Ds[t] = __builtin_amdgcn_exp2f(__shfl(lgv, kC - 1, 64) - lgv);
        out[kLfOff + t] = lgv;
    }
    wait_vm<0>();  // this wave's K, Q rows
    __syncthreads();
    // V for U (below): lane (lr, lg) of wave w takes V[4 s + lg][32 w + lr] and V[4 s + lg][32 w + 16 + lr],
    // s = 0..15, loaded now and used after T is inverted
    float vr0[16], vr1[16];
#pragma unroll
    for (int s = 0; s < 16; s++) {
        const int p = 4 * s + lg;
        const float* vp = v + (row0 + (size_t)min(p, n - 1) * H) * kD + 32 * w + lr;
        vr0[s] = p < n ? vp[0] : 0.0f;
        vr1[s] = p < n ? vp[16] : 0.0f;
    }

    // K K^T tiles (w, t <= w) -> A;  K Q^T tiles (w, t >= w) -> P. Five tiles per wave.
    {
        f4 acc[5];
        const float* bsrc[5];
        int bt[5];
#pragma unroll
        for (int x = 0; x < 5; x++) {
            acc[x] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            const bool kk = x <= w;
            bt[x] = kk ? x : x - 1;
            bsrc[x] = (kk ? Ks : Qs) + (16 * bt[x] + lr) * kKS + 4 * lg;
        }
        // the contraction over keys runs in the order key = 16 sp + 4 (lane / 16) + j, so that each lane
        // reads its four steps' operands as one 16-byte word
        const float* asrc = Ks + (16 * w + lr) * kKS + 4 * lg;
#pragma unroll 2
        for (int sp = 0; sp < kD / 16; sp++) {
            const f4 a = *(const f4*)(asrc + 16 * sp);
            f4 bb[5];
#pragma unroll
            for (int x = 0; x < 5; x++) bb[x] = *(const f4*)(bsrc[x] + 16 * sp);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int x = 0; x < 5; x++) acc[x] = mfma4(a[j], bb[x][j], acc[x]);
        }
        __syncthreads();  // every wave has read q: A overwrites it
#pragma unroll
        for (int x = 0; x < 5; x++) {
            const int t = bt[x];
            if (x <= w) {
                // A[i][j], i = 16w + 4lg + r, j = 16t + lr; zero on and above the diagonal
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int i = 16 * w + 4 * lg + r, j = 16 * t + lr;
                    As[i * kAS + j] = j < i ? Bs[i] * __builtin_amdgcn_exp2f(Ls[i] - Ls[j]) * acc[x][r] : 0.0f;
                }
            } else {
                // (K Q^T)[j][i] with j = 16w + 4lg + r, i = 16t + lr: P[i][j], zero above the diagonal
                f4 p;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int j = 16 * w + 4 * lg + r, i = 16 * t + lr;
                    p[r] = j <= i ? __builtin_amdgcn_exp2f(Ls[i] - Ls[j]) * acc[x][r] : 0.0f;
                }
                *(f4*)(out + kPfOff + ((t * 4 + w) * 64 + lane) * 4) = p;
            }
        }
    }
    __syncthreads();  // A is complete

    // T = (I + A)^-1 in 16 x 16 blocks (A_ij, T_ij: block row i, block column j).
    //  (1) T_ww = (I + A_ww)^-1 by forward substitution, wave w on diagonal block w: lane = (column
    //      c = lane/4 of the block, residue s = lane%4) holds T_ww[4m + s][c] in tv[m]; a row's sum is
    //      split over the quad's residues and combined with two DPP steps. A_ww is zero on and above
    //      its diagonal and tv starts at zero, so reading past the diagonal adds nothing.
    //  (2) Block rows i = 1..3 in turn: T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj on MFMA, wave j on
    //      block (i, j); T_ij overwrites A_ij once block row i no longer reads A.
    {
        const int cT = lane >> 2, sres = lane & 3;
        const float* ab = As + 16 * w * kAS + 16 * w + sres;
        float tv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float p = 0.0f;
#pragma unroll
            for (int m = 0; m < (i + 3) / 4; m++) p = fmaf(ab[i * kAS + 4 * m], tv[m], p);
            const float val = (i == cT ? 1.0f : 0.0f) - quad_sum(p);
            if (sres == (i & 3)) tv[i >> 2] = val;
        }
#pragma unroll
        for (int m = 0; m < 4; m++) As[(16 * w + 4 * m + sres) * kAS + 16 * w + cT] = tv[m];
    }
    __syncthreads();
#pragma unroll
    for (int i = 1; i < 4; i++) {
        f4 tij = {0.0f, 0.0f, 0.0f, 0.0f};
        if (w < i) {
            f4 x = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int kb = w; kb < i; kb++) {
                // X += A_ik T_kj: A operand A_ik[lr][4s + lg], B operand T_kj[4s + lg][lr]
#pragma unroll
                for (int st = 0; st < 4; st++)
                    x = mfma4(As[(16 * i + lr) * kAS + 16 * kb + 4 * st + lg], As[(16 * kb + 4 * st + lg) * kAS + 16 * w + lr], x);
            }
            // T_ii X, contracting over the rows of X in the order of its registers (step st <-> row 4lg + st)
#pragma unroll
            for (int st = 0; st < 4; st++) tij = mfma4(As[(16 * i + lr) * kAS + 16 * i + 4 * lg + st], x[st], tij);
        }
        __syncthreads();  // block row i no longer reads A
        if (w < i) {
#pragma unroll
            for (int r = 0; r < 4; r++) As[(16 * i + 4 * lg + r) * kAS + 16 * w + lr] = -tij[r];
        }
        __syncthreads();
    }

    wait_vm<0>();  // this wave's V values (and its P stores)
    // U (row tiles pt, column tiles cg = 2w, 2w + 1) and W^T (key tiles kt = 2w, 2w + 1, position
    // tiles pt) over the lower-triangular T: tile pt contracts positions < 16 (pt + 1).
#pragma unroll
    for (int pt = 0; pt < 4; pt++) {
        f4 u0 = {0.0f, 0.0f, 0.0f, 0.0f}, u1 = u0, w0 = u0, w1 = u0;
        const float* ta = As + (16 * pt + lr) * kAS + lg;  // T[16pt + lr][4s + lg]
#pragma unroll
        for (int s = 0; s < 4 * (pt + 1); s++) {
            const int p = 4 * s + lg;
            const float tval = ta[4 * s];
            const float bv = Bs[p], bg = BGs[p];
            u0 = mfma4(tval, bv * vr0[s], u0);
            u1 = mfma4(tval, bv * vr1[s], u1);
            // W^T[key][pos] = sum_p (beta gamma K)[p][key] T[pos][p]: A = (beta gamma K)^T, B = T^T
            w0 = mfma4(bg * Ks[p * kKS + 16 * (2 * w) + lr], tval, w0);
            w1 = mfma4(bg * Ks[p * kKS + 16 * (2 * w + 1) + lr], tval, w1);
        }
        *(f4*)(out + kUfOff + ((pt * 8 + 2 * w) * 64 + lane) * 4) = u0;
        *(f4*)(out + kUfOff + ((pt * 8 + 2 * w + 1) * 64 + lane) * 4) = u1;
        *(f4*)(out + kWfOff + ((pt * 8 + 2 * w) * 64 + lane) * 4) = -w0;
        *(f4*)(out + kWfOff + ((pt * 8 + 2 * w + 1) * 64 + lane) * 4) = -w1;
    }
    // the decayed K^T as the A operand of the state update: thread -> (kt, pt) blocks, lane slot
    for (int i = tid; i < 32 * 64; i += 256) {
        const int blk = i >> 6, l = i & 63, kt = blk >> 2, pt = blk & 3;
        f4 kv;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int p = 16 * pt + 4 * (l >> 4) + r;
            kv[r] = Ds[p] * Ks[p * kKS + 16 * kt + (l & 15)];
        }
        *(f4*)(out + kKfOff + i * 4) = kv;
    }
}

// LDS staging of one chunk in a chain workgroup of CGW column groups, in floats: W (all tiles), U
// (the workgroup's column groups), P, q in A-fragment order, the decayed K^T, L; then the waves'
// partial sums ([wave][tile 4][lane 64][4]: D, later the rows of Q S).
template <int CGW>
struct ChainLds {
    static constexpr int kSW = 0, kSU = 8192, kSP = kSU + CGW * 1024, kSQ = kSP + 4096, kSK = kSQ + 8192,
                         kSL = kSK + 8192, kSX = kSL + 64, kFloats = kSX + 4 * CGW * 1024;
};

// The chain over chunks: workgroup = (sequence, head, CGW column groups of 16 value columns),
// 4 CGW waves = CGW column groups (cgl = wave / 4) x 4 key quarters (kq = wave % 4, key tiles
// 2 kq, 2 kq + 1, the wave's 32 keys of the state slice in 8 VGPRs). Per chunk:
//  - D = U - W S: each key quarter contracts its 32 keys, the four partials meet in LDS and every
//    wave of the column group adds them in quarter order (so all four hold the same D);
//  - O = diag(gamma) Q S + P D: the rows of Q S likewise by key quarter; wave kq then owns output
//    row tile kq, adds the four partial rows in quarter order and its P D terms (row tile kq needs
//    position tiles 0..kq of D), and stores them;
//  - S = gamma_63 S + Kf D on the wave's own key tiles.
// A chain's MFMA work is split four ways (about 100-112 MFMAs per wave and chunk instead of 424),
// and a (sequence, head) runs as 8 / CGW workgroups, all on one XCD (workgroups are dealt to XCDs
// round robin), which share its chunk operands in that XCD's L2. CGW = 1 puts one wave on each
// SIMD of a CU and twice as many CUs to work (for few sequences); CGW = 2 halves the workgroups
// (for grids that already fill the chip). Both add the same partials in the same order.
template <int CGW>
__global__ __launch_bounds__(256 * CGW) void k_wy_chain(const float* __restrict__ q, const float* __restrict__ ws,
                                                        float* __restrict__ state, float* __restrict__ out, int T,
                                                        int H, int BH, int value_major) {
    using Lds = ChainLds<CGW>;
    constexpr int kSW = Lds::kSW, kSU = Lds::kSU, kSP = Lds::kSP, kSQ = Lds::kSQ, kSK = Lds::kSK, kSL = Lds::kSL,
                  kSX = Lds::kSX;
    constexpr int NW = 4 * CGW, PER = 8 / CGW;  // waves; workgroups per (sequence, head)
    // vector-memory instructions per wave: W + U + L, P + q, K copies; the output stores
    constexpr int kNWul = 32 / NW + 2, kNQp = 48 / NW, kNK = 32 / NW, kNSt = 4;
    __shared__ __attribute__((aligned(16))) float sm[Lds::kFloats];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, lr = lane & 15, lg = lane >> 4;
    const int cgl = wv >> 2, kq = wv & 3;
    const int id = blockIdx.x, xcd = id & 7, slot = id >> 3;
    const int bh = (slot / PER) * 8 + xcd, part = slot % PER, cg = CGW * part + cgl;
    if (bh >= BH) return;  // the whole workgroup
    const int b = bh / H, h = bh % H, NC = (T + kC - 1) / kC;
    const int col = 16 * cg + lr;

    // Copies of chunk c's operands; the NW waves copy 1 / NW of every buffer each (1 KiB blocks).
    auto issue_wul = [&](int c) {
        const float* wc = ws + ((size_t)bh * NC + c) * kWyFloats;
#pragma unroll
        for (int u = 0; u < 32 / NW; u++) {
            const int blk = wv + NW * u;
            dma16(wc + kWfOff + blk * 256 + lane * 4, sm + kSW + blk * 256);
        }
        {  // U block (column group wv / 4, position tile wv % 4)
            const int ucg = wv >> 2, upt = wv & 3;
            dma16(wc + kUfOff + ((upt * 8 + CGW * part + ucg) * 64 + lane) * 4, sm + kSU + (ucg * 4 + upt) * 256);
        }
        constexpr int kL = 64 / NW;  // L values per wave
        if (lane < kL) dma4(wc + kLfOff + kL * wv + lane, sm + kSL + kL * wv);
    };
    auto issue_qp = [&](int c) {
        const float* wc = ws + ((size_t)bh * NC + c) * kWyFloats;
        const int t0 = c * kC, n = min(kC, T - t0);
#pragma unroll
        for (int u = 0; u < 16 / NW; u++) {
            const int blk = wv + NW * u;
            dma16(wc + kPfOff + blk * 256 + lane * 4, sm + kSP + blk * 256);
        }
        // q block (pt, kt): lane i <- q[16pt + i%16][16kt + 4(i/16) .. +3]; padding rows repeat a real row
#pragma unroll
        for (int u = 0; u < 32 / NW; u++) {
            const int blk = wv + NW * u, pt = blk >> 3, kt = blk & 7;
            const int p = min(16 * pt + lr, n - 1);
            dma16(q + (((size_t)b * T + t0 + p) * H + h) * kD + 16 * kt + 4 * lg, sm + kSQ + blk * 256);
        }
    };
    auto issue_k = [&](int c) {
        const float* wc = ws + ((size_t)bh * NC + c) * kWyFloats;
#pragma unroll
        for (int u = 0; u < 32 / NW; u++) {
            const int blk = wv + NW * u;
            dma16(wc + kKfOff + blk * 256 + lane * 4, sm + kSK + blk * 256);
        }
    };

    // state entry (key j, value column col): [dk][dv], or the model's value-major [dv][dk]
    float* S0 = state + (size_t)bh * kD * kD;
    auto sidx = [&](int j) { return value_major ? (size_t)col * kD + j : (size_t)j * kD + col; };
    f4 S[2];  // key tiles 2 kq + j
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) S[j][r] = S0[sidx(16 * (2 * kq + j) + 4 * lg + r)];
    // the state loads complete before the first copies are counted
    wait_vm<0>();
    issue_wul(0);
    issue_qp(0);
    issue_k(0);
    f4* X = (f4*)(sm + kSX);  // [wave][tile][lane]
    const int x0 = 4 * cgl;   // the column group's first wave

    for (int c = 0; c < NC; c++) {
        const bool more = c + 1 < NC;
        const int t0 = c * kC, n = min(kC, T - t0);
        const size_t row0 = ((size_t)b * T + t0) * H + h;

        // after W, U, L of c: the stores of chunk c - 1 (issued before the q, P copies), q, P, K
        wait_vm<kNQp + kNK>();
        __syncthreads();
        f4 D[4];
#pragma unroll
        for (int pt = 0; pt < 4; pt++)
            D[pt] = kq == 0 ? *(const f4*)(sm + kSU + ((cgl * 4 + pt) * 64 + lane) * 4) : f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int kt = 2 * kq + j;
            f4 a[4];
#pragma unroll
            for (int pt = 0; pt < 4; pt++) a[pt] = *(const f4*)(sm + kSW + ((pt * 8 + kt) * 64 + lane) * 4);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int pt = 0; pt < 4; pt++) D[pt] = mfma4(a[pt][r], S[j][r], D[pt]);
        }
#pragma unroll
        for (int pt = 0; pt < 4; pt++) X[(wv * 4 + pt) * 64 + lane] = D[pt];
        float gqa[16];  // gamma of the rows this lane holds in every row tile: 16 pt + 4lg + r
#pragma unroll
        for (int pt = 0; pt < 4; pt++)
#pragma unroll
            for (int r = 0; r < 4; r++) gqa[pt * 4 + r] = __builtin_amdgcn_exp2f(sm[kSL + 16 * pt + 4 * lg + r]);
        const float gl = __builtin_amdgcn_exp2f(sm[kSL + kC - 1]);
        __syncthreads();  // W, U, L are no longer read; the D partials are in
        if (more) issue_wul(c + 1);
#pragma unroll
        for (int pt = 0; pt < 4; pt++) {
            f4 d = X[((x0 + 0) * 4 + pt) * 64 + lane];
#pragma unroll
            for (int w = 1; w < 4; w++) d += X[((x0 + w) * 4 + pt) * 64 + lane];
            D[pt] = d;
        }

        // after q, P of c: K of c, W, U, L of c + 1
        if (more) wait_vm<kNK + kNWul>();
        else wait_vm<kNK>();
        __syncthreads();  // also: every wave has read the D partials
        f4 O[4];
#pragma unroll
        for (int pt = 0; pt < 4; pt++) O[pt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int kt = 2 * kq + j;
            f4 a[4];
#pragma unroll
            for (int pt = 0; pt < 4; pt++) a[pt] = *(const f4*)(sm + kSQ + ((pt * 8 + kt) * 64 + lane) * 4);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int pt = 0; pt < 4; pt++) O[pt] = mfma4(a[pt][r], S[j][r], O[pt]);
        }
        // diag(gamma) on the rows of Q S0: row 16pt + 4lg + r of register r
#pragma unroll
        for (int pt = 0; pt < 4; pt++)
#pragma unroll
            for (int r = 0; r < 4; r++) O[pt][r] *= gqa[pt * 4 + r];
#pragma unroll
        for (int pt = 0; pt < 4; pt++) X[(wv * 4 + pt) * 64 + lane] = O[pt];
        __syncthreads();
        // output row tile kq: the four quarters' rows of Q S, then + P D over position tiles 0..kq
        f4 o = X[((x0 + 0) * 4 + kq) * 64 + lane];
#pragma unroll
        for (int w = 1; w < 4; w++) o += X[((x0 + w) * 4 + kq) * 64 + lane];
        for (int pt = 0; pt <= kq; pt++) {  // wave-uniform
            const f4 a = *(const f4*)(sm + kSP + ((kq * 4 + pt) * 64 + lane) * 4);
#pragma unroll
            for (int r = 0; r < 4; r++) o = mfma4(a[r], D[pt][r], o);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int p = 16 * kq + 4 * lg + r;
            if (p < n) out[(row0 + (size_t)p * H) * kD + col] = o[r];
        }
        __syncthreads();  // q, P and the partial rows are no longer read
        if (more) issue_qp(c + 1);

        // after K of c: W, U, L of c + 1, this chunk's stores, q, P of c + 1; on the last chunk
        // everything
        if (more) wait_vm<kNWul + kNSt + kNQp>();
        else wait_vm<0>();
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 2; j++) S[j] *= gl;
#pragma unroll
        for (int pt = 0; pt < 4; pt++) {
            f4 a[2];
#pragma unroll
            for (int j = 0; j < 2; j++) a[j] = *(const f4*)(sm + kSK + (((2 * kq + j) * 4 + pt) * 64 + lane) * 4);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < 2; j++) S[j] = mfma4(a[j][r], D[pt][r], S[j]);
        }
        __syncthreads();  // K is no longer read
        if (more) issue_k(c + 1);
    }
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) S0[sidx(16 * (2 * kq + j) + 4 * lg + r)] = S[j][r];
}

}  // namespace

size_t wy_workspace_bytes(int batch, int tokens, int heads) {
    return (size_t)batch * heads * ((tokens + kC - 1) / kC) * kWyFloats * sizeof(float);
}

void launch_delta_rule_wy(const float* q, const float* k, const float* v, const float* beta, const float* g,
                          float* state, float* out, int batch, int tokens, int heads, float* ws, hipStream_t st,
                          int value_major) {
    const int NC = (tokens + kC - 1) / kC, BH = batch * heads;
    hipLaunchKernelGGL(k_wy_prep, dim3(NC, heads, batch), dim3(256), 0, st, q, k, v, beta, g, ws, tokens, heads);
    // one column group per workgroup while that leaves a CU per workgroup (256 CUs), else two
    if (BH <= 32)
        hipLaunchKernelGGL((k_wy_chain<1>), dim3(64 * ((BH + 7) / 8)), dim3(256), 0, st, q, ws, state, out, tokens,
                           heads, BH, value_major);
    else
        hipLaunchKernelGGL((k_wy_chain<2>), dim3(32 * ((BH + 7) / 8)), dim3(512), 0, st, q, ws, state, out, tokens,
                           heads, BH, value_major);
}

}  // namespace qne
