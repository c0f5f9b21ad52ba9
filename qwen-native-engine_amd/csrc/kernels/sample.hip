// Token sampling over one row of logits on the device: the O(vocab) part of src/sampling.rs
// Sampler::try_sample / choose (:58-134) -- the fail-closed checks, the presence penalty and grammar
// mask, the greedy pick, and for temperature sampling the top-k candidates in the order the
// reference sorts them (f32 total order, descending). The O(k) tail (softmax weights, top-p prefix,
// the xorshift draw) runs on the host in the reference's exact f32 arithmetic.
//
// Design for gfx950. Keys are the f32 total order as u32. The row (0.6 MB) is read by 128
// workgroups, since one CU cannot keep enough loads in flight to stream it quickly:
//  1. k_sample_part: per slice of the row -- the checks, the allowed count, the greedy best, and the
//     keys of 32 evenly spaced tokens;
//  2. k_sample_plan (one workgroup): merges the slices (flags, count, greedy pick: the lowest token
//     among the equal maxima), then picks from the 4096 sampled keys (radix select, LDS histograms)
//     a threshold with, by a wide margin, at least k allowed tokens at or above it (all allowed tokens
//     when there are at most 4096);
//  3. k_sample_collect: per slice, the tokens at or above the threshold into a candidate buffer
//     (slots from a global counter: a few hundred to a few thousand candidates);
//  4. k_sample_final (one workgroup): sorts the candidates by (key descending, token ascending), so
//     the first k are exactly the reference's top k. When the threshold left fewer than k or more than
//     4096 candidates (rows with thousands of equal logits), an exact radix select over the whole row
//     runs instead: three LDS histogram passes (11 + 11 + 10 bits) find the k-th largest key, and one
//     pass in token order collects the keys above it and the lowest token ids among those equal to it.
#include "common.hpp"
#include "launch.hpp"

namespace qne {

namespace {

constexpr int kST = 1024;             // threads of the single-workgroup kernels
constexpr int kSW = kST / kWave;
constexpr int kPT = 256;              // threads of the per-slice kernels
constexpr int kParts = 128;           // slices
constexpr int kPerPart = 32;          // sampled keys per slice
constexpr int kCap = 4096;            // candidate slots (= kParts * kPerPart)
static_assert(kParts * kPerPart == kCap, "one sampled key per candidate slot");

// Scratch of one sampling call (device memory, sample_scratch_bytes()).
struct Scratch {
    uint32_t flags[kParts], n[kParts], bi[kParts];
    float bv[kParts];
    uint32_t samples[kCap];
    uint32_t ctl[4];  // [0] 1: nothing more to do, [1] threshold key, [2] k, [3] candidate count
    uint32_t ckey[kCap], cidx[kCap];
    float cval[kCap];
};

// f32 total order (f32::total_cmp) as an unsigned key: larger key = later in the order.
__device__ __forceinline__ uint32_t total_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u >> 31) ? ~u : (u | 0x80000000u);
}

struct Tok {
    float raw;  // logit (+ bias): what try_sample checks
    float v;    // raw - penalty for a generated token: what choose compares
    bool ok;    // allowed by the mask
};

__device__ __forceinline__ Tok token_at(const SampleArgs& a, uint32_t i) {
    Tok t;
    float l = a.logits[i];
    if (i == a.bias_token) l = l + a.bias;
    t.raw = l;
    t.v = (a.penalty != 0.0f && a.seen && ((a.seen[i >> 5] >> (i & 31)) & 1u)) ? l - a.penalty : l;
    t.ok = !a.mask || (i < a.mask_len && ((a.mask[i >> 5] >> (i & 31)) & 1u));
    return t;
}

// f(i, token) over the tokens [lo, hi) (lo a multiple of 4) by NT threads, each taking groups of 4
// consecutive tokens (one seen word and one mask word each) with 16 tokens' loads in flight; a thread
// visits its tokens in increasing order.
template <int NT, typename F>
__device__ __forceinline__ void scan_tokens(const SampleArgs& a, uint32_t lo, uint32_t hi, F&& f) {
    const uint32_t G = (hi - lo + 3) / 4;
    for (uint32_t g0 = threadIdx.x; g0 < G; g0 += 4 * NT) {
        float l[4][4];
        uint32_t sw[4], mw[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t g = g0 + u * NT, i = lo + 4 * g;
#pragma unroll
            for (int e = 0; e < 4; e++) l[u][e] = (g < G && i + e < hi) ? a.logits[i + e] : 0.0f;
            sw[u] = (g < G && a.seen) ? a.seen[i >> 5] : 0u;
            mw[u] = (g < G && a.mask && i < a.mask_len) ? a.mask[i >> 5] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t g = g0 + u * NT;
            if (g >= G) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t i = lo + 4 * g + e;
                if (i >= hi) continue;
                Tok x;
                float v = l[u][e];
                if (i == a.bias_token) v = v + a.bias;
                x.raw = v;
                x.v = (a.penalty != 0.0f && a.seen && ((sw[u] >> (i & 31)) & 1u)) ? v - a.penalty : v;
                x.ok = !a.mask || (i < a.mask_len && ((mw[u] >> (i & 31)) & 1u));
                f(i, x);
            }
        }
    }
}

// The slice [lo, hi) of part p (lo a multiple of 4).
__device__ __forceinline__ void part_range(uint32_t V, int p, uint32_t& lo, uint32_t& hi) {
    const uint32_t per = ((V + kParts - 1) / kParts + 3) & ~3u;
    lo = min(V, per * (uint32_t)p);
    hi = min(V, lo + per);
}

// (value, token) a beats b for the greedy pick: larger value, then lower token; a missing
// candidate (token ~0) never wins.
__device__ __forceinline__ bool greedy_better(float av, uint32_t ai, float bv, uint32_t bi) {
    return ai != 0xFFFFFFFFu && (bi == 0xFFFFFFFFu || av > bv || (av == bv && ai < bi));
}

// Exclusive prefix sum over a 1024-thread block in thread order; *total gets the sum. Ends with a
// barrier.
__device__ uint32_t block_scan(uint32_t x, uint32_t* red, uint32_t* total) {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    uint32_t incl = x;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t y = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += y;
    }
    if (lane == kWave - 1) red[w] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (int j = 0; j < kSW; j++) {
            const uint32_t c = red[j];
            red[j] = s;
            s += c;
        }
        red[kSW] = s;
    }
    __syncthreads();
    const uint32_t r = red[w] + incl - x;
    *total = red[kSW];
    __syncthreads();
    return r;
}

// In a histogram of nb bins (bin b counts the keys whose digit is b), the bin holding the need-th
// largest key: *bin, and *above = the count in the bins above it. Thread t owns bins
// [per t, per t + per); the counts above each thread come from a suffix scan in thread order.
// Every thread gets the result.
__device__ void select_bin(const uint32_t* hist, int nb, uint32_t need, uint32_t* red, uint32_t* res, int* bin,
                           uint32_t* above) {
    const int per = nb / kST, t = threadIdx.x, lane = t & (kWave - 1), w = t / kWave;
    uint32_t s = 0;
    for (int j = 0; j < per; j++) s += hist[per * t + j];
    uint32_t incl = s;  // sum over this wave's lanes >= lane
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t y = __shfl_down(incl, o, kWave);
        if (lane + o < kWave) incl += y;
    }
    if (lane == 0) red[w] = incl;
    __syncthreads();
    if (t == 0) {
        uint32_t acc = 0;
        for (int j = kSW - 1; j >= 0; j--) {
            const uint32_t c = red[j];
            red[j] = acc;  // the waves above wave j
            acc += c;
        }
    }
    __syncthreads();
    const uint32_t ab = red[w] + incl - s;  // keys in the bins of the threads above
    if (ab < need && need <= ab + s) {
        uint32_t acc = ab;
        for (int j = per - 1; j >= 0; j--) {
            const uint32_t c = hist[per * t + j];
            if (acc + c >= need) {
                res[0] = (uint32_t)(per * t + j);
                res[1] = acc;
                break;
            }
            acc += c;
        }
    }
    __syncthreads();
    *bin = (int)res[0];
    *above = res[1];
    __syncthreads();
}

// Bitonic sort of slots [0, N) (N a power of two <= kCap) into key-descending, token-ascending
// order by a 1024-thread block; every thread takes its share of the N/2 pairs of each stage.
template <bool kVal>
__device__ void bitonic(uint32_t* key, uint32_t* idx, float* val, int N) {
    for (int size = 2; size <= N; size <<= 1) {
        for (int ls = __builtin_ctz((unsigned)size) - 1; ls >= 0; ls--) {
            const int stride = 1 << ls;
            for (int p = threadIdx.x; p < N / 2; p += kST) {
                const int i = ((p >> ls) << (ls + 1)) | (p & (stride - 1)), j = i + stride;
                const uint32_t ka = key[i], kb = key[j], ia = idx[i], ib = idx[j];
                const bool a_first = ka > kb || (ka == kb && ia < ib);  // i before j in the final order
                const bool up = (i & size) == 0;                         // this block sorts in the final order
                if (up ? !a_first : a_first) {
                    key[i] = kb;
                    key[j] = ka;
                    idx[i] = ib;
                    idx[j] = ia;
                    if (kVal) {
                        const float vi = val[i];
                        val[i] = val[j];
                        val[j] = vi;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// 1. Per slice: checks, allowed count, greedy best, 32 sampled keys.
__global__ __launch_bounds__(kPT) void k_sample_part(const SampleArgs a, Scratch* ws) {
    __shared__ float sv[kPT / kWave];
    __shared__ uint32_t si[kPT / kWave], sf[kPT / kWave], sn[kPT / kWave];
    const int p = blockIdx.x, t = threadIdx.x, lane = t & (kWave - 1), w = t / kWave;
    uint32_t lo, hi;
    part_range(a.V, p, lo, hi);
    uint32_t flags = 0, n = 0, besti = 0xFFFFFFFFu;
    float best = -INFINITY;
    scan_tokens<kPT>(a, lo, hi, [&](uint32_t i, const Tok& x) {
        if (!x.ok) return;
        if (isnan(x.raw) || x.raw == INFINITY) flags |= 1u;
        if (isfinite(x.raw)) flags |= 2u;
        n++;
        // the reference's greedy scan: strictly greater replaces, so the lowest token wins a tie
        if (x.v > best) {
            best = x.v;
            besti = i;
        }
    });
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        flags |= __shfl_xor(flags, o, kWave);
        n += __shfl_xor(n, o, kWave);
        const float ov = __shfl_xor(best, o, kWave);
        const uint32_t oi = __shfl_xor(besti, o, kWave);
        if (greedy_better(ov, oi, best, besti)) {
            best = ov;
            besti = oi;
        }
    }
    if (lane == 0) {
        sv[w] = best;
        si[w] = besti;
        sf[w] = flags;
        sn[w] = n;
    }
    if (t < kPerPart) {
        // evenly spaced tokens of the slice; 0 (below every allowed key) where none or not allowed
        uint32_t key = 0u;
        if (hi > lo) {
            const uint32_t i = lo + (uint32_t)(((uint64_t)t * (hi - lo)) / kPerPart);
            const Tok x = token_at(a, i);
            if (x.ok) key = total_key(x.v);
        }
        ws->samples[p * kPerPart + t] = key;
    }
    __syncthreads();
    if (t == 0) {
        float b = -INFINITY;
        uint32_t ib = 0xFFFFFFFFu, f = 0, nn = 0;
        for (int j = 0; j < kPT / kWave; j++) {
            f |= sf[j];
            nn += sn[j];
            if (greedy_better(sv[j], si[j], b, ib)) {
                b = sv[j];
                ib = si[j];
            }
        }
        ws->flags[p] = f;
        ws->n[p] = nn;
        ws->bv[p] = b;
        ws->bi[p] = ib;
    }
}

// 2. Merge the slices; the candidate threshold (a radix select over the sampled keys).
__global__ __launch_bounds__(kST) void k_sample_plan(const SampleArgs a, Scratch* ws) {
    __shared__ uint32_t hist[2048];
    __shared__ uint32_t red[kSW + 1];
    __shared__ uint32_t res[2];
    __shared__ float wv[kSW];
    __shared__ uint32_t wi[kSW], wf[kSW], wn[kSW];
    __shared__ uint32_t plan[3];
    const int t = threadIdx.x, lane = t & (kWave - 1), w = t / kWave;
    // the slices' flags, counts and greedy candidates, reduced over the block
    uint32_t f = 0, nn = 0, ib = 0xFFFFFFFFu;
    float b = -INFINITY;
    if (t < kParts) {
        f = ws->flags[t];
        nn = ws->n[t];
        b = ws->bv[t];
        ib = ws->bi[t];
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
        f |= __shfl_xor(f, o, kWave);
        nn += __shfl_xor(nn, o, kWave);
        const float ov = __shfl_xor(b, o, kWave);
        const uint32_t oi = __shfl_xor(ib, o, kWave);
        if (greedy_better(ov, oi, b, ib)) {
            b = ov;
            ib = oi;
        }
    }
    if (lane == 0) {
        wv[w] = b;
        wi[w] = ib;
        wf[w] = f;
        wn[w] = nn;
    }
    __syncthreads();
    if (t == 0) {
        for (int j = 1; j < kSW; j++) {
            f |= wf[j];
            nn += wn[j];
            if (greedy_better(wv[j], wi[j], b, ib)) {
                b = wv[j];
                ib = wi[j];
            }
        }
        a.info[0] = 0;
        a.info[1] = f;
        a.info[2] = ib == 0xFFFFFFFFu ? 0u : ib;
        const uint32_t k = min(a.k, nn);
        plan[0] = nn;
        plan[1] = k;
        // greedy, nothing allowed, or a row the host rejects (a NaN or +inf allowed): no candidates
        plan[2] = (a.k == 0 || k == 0 || (f & 1u)) ? 1u : 0u;
    }
    __syncthreads();
    const uint32_t n = plan[0], k = plan[1], done = plan[2];
    if (done) {
        if (t == 0) ws->ctl[0] = 1u;
        return;  // the whole block
    }
    uint32_t Ts = 0;  // all allowed tokens when they fit the candidate slots
    if (n > (uint32_t)kCap) {
        constexpr int kPer = kCap / kST;  // sampled keys per thread
        uint32_t key[kPer];
        uint32_t cnt = 0;
#pragma unroll
        for (int e = 0; e < kPer; e++) {
            key[e] = ws->samples[kPer * t + e];
            cnt += key[e] != 0u;
        }
        uint32_t as;
        (void)block_scan(cnt, red, &as);  // allowed tokens among the samples (key 0: not allowed)
        // about kp = k as / n of the allowed samples lie at or above the k-th largest key, with a
        // spread of ~sqrt(kp) in that rank: the j-th largest allowed sample, j = kp + 5 sqrt(kp) + 3,
        // leaves at least k allowed tokens above it all but ~1e-6 of the time (and about
        // j n / as candidates). With no allowed sample the threshold admits everything and the final
        // kernel falls back to the exact select.
        if (as > 0) {
            const float kp = (float)k * (float)as / (float)n;
            uint32_t need = min(as, max(1u, (uint32_t)ceilf(kp + 5.0f * sqrtf(kp) + 3.0f)));
            uint32_t prefix = 0;
#pragma unroll
            for (int p = 0; p < 3; p++) {
                const int sh = p == 0 ? 21 : (p == 1 ? 10 : 0), wd = p == 2 ? 10 : 11;
                const int nb = 1 << wd, hi = sh + wd;
                for (int bb = t; bb < nb; bb += kST) hist[bb] = 0;
                __syncthreads();
#pragma unroll
                for (int e = 0; e < kPer; e++) {
                    if (key[e] == 0u || (hi < 32 && (key[e] >> hi) != prefix)) continue;
                    atomicAdd(&hist[(key[e] >> sh) & (nb - 1)], 1u);
                }
                __syncthreads();
                int bin;
                uint32_t above;
                select_bin(hist, nb, need, red, res, &bin, &above);
                prefix = (prefix << wd) | (uint32_t)bin;
                need -= above;
            }
            Ts = prefix;
        }
    }
    if (t == 0) {
        ws->ctl[0] = 0u;
        ws->ctl[1] = Ts;
        ws->ctl[2] = k;
        ws->ctl[3] = 0u;
    }
}

// 3. Per slice: the candidates at or above the threshold.
__global__ __launch_bounds__(kPT) void k_sample_collect(const SampleArgs a, Scratch* ws) {
    if (ws->ctl[0]) return;  // the whole grid
    const uint32_t Ts = ws->ctl[1];
    uint32_t lo, hi;
    part_range(a.V, blockIdx.x, lo, hi);
    scan_tokens<kPT>(a, lo, hi, [&](uint32_t i, const Tok& x) {
        if (!x.ok) return;
        const uint32_t key = total_key(x.v);
        if (key < Ts) return;
        const uint32_t pos = atomicAdd(&ws->ctl[3], 1u);
        if (pos < (uint32_t)kCap) {
            ws->ckey[pos] = key;
            ws->cidx[pos] = i;
            ws->cval[pos] = x.v;
        }
    });
}

// 4. The top k in order (or the exact select over the row).
__global__ __launch_bounds__(kST) void k_sample_final(const SampleArgs a, Scratch* ws) {
    __shared__ uint32_t hist[2048];
    __shared__ uint32_t red[kSW + 1];
    __shared__ uint32_t res[2];
    __shared__ uint32_t ckey[kCap], cidx[kCap];
    __shared__ float cval[kCap];
    const int t = threadIdx.x;
    if (ws->ctl[0]) return;  // the whole block
    const uint32_t k = ws->ctl[2];
    uint32_t c = ws->ctl[3];
    const bool exact = c < k || c > (uint32_t)kCap;
    if (!exact) {
        for (uint32_t j = t; j < c; j += kST) {
            ckey[j] = ws->ckey[j];
            cidx[j] = ws->cidx[j];
            cval[j] = ws->cval[j];
        }
    } else {
        // the k-th largest key T by its digits (bits 31..21, 20..10, 9..0), LDS histograms
        uint32_t prefix = 0, above_all = 0, need = k;
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const int sh = p == 0 ? 21 : (p == 1 ? 10 : 0), wd = p == 2 ? 10 : 11;
            const int nb = 1 << wd;
            for (int b = t; b < nb; b += kST) hist[b] = 0;
            __syncthreads();
            const int hi = sh + wd;
            scan_tokens<kST>(a, 0u, a.V, [&](uint32_t, const Tok& x) {
                if (!x.ok) return;
                const uint32_t key = total_key(x.v);
                if (hi < 32 && (key >> hi) != prefix) return;
                atomicAdd(&hist[(key >> sh) & (nb - 1)], 1u);
            });
            __syncthreads();
            int bin;
            uint32_t above;
            select_bin(hist, nb, need, red, res, &bin, &above);
            prefix = (prefix << wd) | (uint32_t)bin;
            need -= above;
            above_all += above;
        }
        const uint32_t T = prefix;            // the k-th largest key
        const uint32_t n_gt = above_all;      // keys above T (< k)
        const uint32_t n_eq_take = k - n_gt;  // keys equal to T taken, lowest token ids first
        // collection in token order: thread t owns [t * C, t * C + C)
        const uint32_t V = a.V, C = (V + kST - 1) / kST;
        const uint32_t i0 = min(V, (uint32_t)t * C), i1 = min(V, i0 + C);
        uint32_t g = 0, e = 0;
        for (uint32_t i = i0; i < i1; i++) {
            const Tok x = token_at(a, i);
            if (!x.ok) continue;
            const uint32_t key = total_key(x.v);
            g += key > T;
            e += key == T;
        }
        uint32_t tot;
        uint32_t gpos = block_scan(g, red, &tot);
        uint32_t epos = block_scan(e, red, &tot);
        for (uint32_t i = i0; i < i1; i++) {
            const Tok x = token_at(a, i);
            if (!x.ok) continue;
            const uint32_t key = total_key(x.v);
            if (key > T) {
                ckey[gpos] = key;
                cidx[gpos] = i;
                cval[gpos] = x.v;
                gpos++;
            } else if (key == T) {
                if (epos < n_eq_take) {
                    ckey[n_gt + epos] = key;
                    cidx[n_gt + epos] = i;
                    cval[n_gt + epos] = x.v;
                }
                epos++;
            }
        }
        c = k;
    }
    // sort the c candidates (padded to a power of two with keys that sort last): key descending,
    // token ascending; the first k are the reference's scratch after its select and sort
    int N = 2;
    while ((uint32_t)N < c) N <<= 1;
    for (int j = t; j < N; j += kST) {
        if ((uint32_t)j >= c) {
            ckey[j] = 0u;
            cidx[j] = 0xFFFFFFFFu;
            cval[j] = 0.0f;
        }
    }
    __syncthreads();
    bitonic<true>(ckey, cidx, cval, N);
    if ((uint32_t)t < k) {
        a.out_v[t] = cval[t];
        a.out_i[t] = cidx[t];
    }
    if (t == 0) a.info[0] = k;
}

}  // namespace

size_t sample_scratch_bytes() { return sizeof(Scratch); }

void launch_sample(const SampleArgs& a, void* scratch, hipStream_t st) {
    Scratch* ws = (Scratch*)scratch;
    hipLaunchKernelGGL(k_sample_part, dim3(kParts), dim3(kPT), 0, st, a, ws);
    hipLaunchKernelGGL(k_sample_plan, dim3(1), dim3(kST), 0, st, a, ws);
    hipLaunchKernelGGL(k_sample_collect, dim3(kParts), dim3(kPT), 0, st, a, ws);
    hipLaunchKernelGGL(k_sample_final, dim3(1), dim3(kST), 0, st, a, ws);
}

}  // namespace qne
