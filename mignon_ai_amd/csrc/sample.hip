// Token sampling on the device: generate.SampleRawLogitsAdvanced (internal/generate/sample.go:31-171) and
// the per-step rules of sampleContinuation (sample.go:196-247: trigram blocking, repetition window), one
// workgroup per row.
//
// Every quantity the reference computes in float64 is computed in float64 here, in the reference's order:
// the softmax denominators and every cumulative sum are sequential sums in the order the reference adds
// (index order, or descending probability after the sort), so the chosen token is the one the reference
// picks for the same logits and the same uniform draw. The candidate sort orders equal probabilities by
// token index (Go's pdqsort leaves their order unspecified).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "sample.hpp"

namespace mg {

namespace {

constexpr int kThreads = 256;

// SplitMix64's output function (Vigna): the uniform of draw k from seed s is the top 53 bits of
// mix64(s + k * golden), k = step + 1, i.e. the k-th output of a SplitMix64 generator seeded with s.
__device__ __forceinline__ double uniform_draw(uint64_t seed, int step) {
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (uint64_t)(step + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) * 0x1.0p-53;
}

// (value, index) ordering of the candidate sort: larger value first, then smaller index
__device__ __forceinline__ bool before(double va, int ia, double vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

__device__ void bitonic_desc(double* key, int* idx, int n2) {
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n2; i += blockDim.x) {
                const int l = i ^ j;
                if (l > i) {
                    const bool up = (i & k) == 0;  // this block of k ends up in descending order
                    const double a = key[i], b = key[l];
                    const int ia = idx[i], ib = idx[l];
                    const bool swap = up ? before(b, ib, a, ia) : before(a, ia, b, ib);
                    if (swap) {
                        key[i] = b; key[l] = a;
                        idx[i] = ib; idx[l] = ia;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// One step of a wave-wide (value, index) argmax through DPP lane moves (VALU latency, no LDS round
// trip): lanes outside row_mask keep their own pair.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void argmax_dpp(double& v, int& i) {
    const int lo = __double2loint(v), hi = __double2hiint(v);
    const int olo = __builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, 0xF, false);
    const int ohi = __builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, 0xF, false);
    const int oi = __builtin_amdgcn_update_dpp(i, i, CTRL, ROW_MASK, 0xF, false);
    const double ov = __hiloint2double(ohi, olo);
    if (before(ov, oi, v, i)) { v = ov; i = oi; }
}

// The wave's first maximum (larger value, then smaller index), in every lane: quad swaps, half-row and
// row mirrors, then the row broadcasts carry each row's result upwards so that lane 63 holds the wave's.
__device__ __forceinline__ void wave_argmax(double& v, int& i) {
    argmax_dpp<0xB1, 0xF>(v, i);   // quad_perm [1,0,3,2]
    argmax_dpp<0x4E, 0xF>(v, i);   // quad_perm [2,3,0,1]
    argmax_dpp<0x141, 0xF>(v, i);  // row_half_mirror
    argmax_dpp<0x140, 0xF>(v, i);  // row_mirror
    argmax_dpp<0x142, 0xA>(v, i);  // row_bcast:15 into rows 1 and 3
    argmax_dpp<0x143, 0xC>(v, i);  // row_bcast:31 into rows 2 and 3
    const int lo = __builtin_amdgcn_readlane(__double2loint(v), 63);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(v), 63);
    i = __builtin_amdgcn_readlane(i, 63);
    v = __hiloint2double(hi, lo);
}

__device__ __forceinline__ void block_argmax(double v, int i, double* red_v, int* red_i, double& best_v, int& best_i) {
    // first maximum: larger value, then smaller index
    for (int o = 32; o > 0; o >>= 1) {
        const double ov = __shfl_xor(v, o);
        const int oi = __shfl_xor(i, o);
        if (before(ov, oi, v, i)) { v = ov; i = oi; }
    }
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) { red_v[w] = v; red_i[w] = i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        double bv = red_v[0];
        int bi = red_i[0];
        for (int k = 1; k < nw; k++)
            if (before(red_v[k], red_i[k], bv, bi)) { bv = red_v[k]; bi = red_i[k]; }
        red_v[0] = bv; red_i[0] = bi;
    }
    __syncthreads();
    best_v = red_v[0];
    best_i = red_i[0];
    __syncthreads();
}

// Sequential float64 sum x[0] + x[1] + ... in that order (the reference's loop); with prefix, x[i] is
// replaced by the running sum through i. One lane, in batches of 16 values held in two register sets that
// alternate: each batch's LDS reads are issued before the previous batch's additions (scheduling barriers
// keep them there), so the chain of dependent additions does not wait for LDS.
template <int B>
__device__ __forceinline__ void seq_batch(double* x, int i, const double2 (&v)[B / 2], double& s, bool prefix) {
    double2 o[B / 2];
#pragma unroll
    for (int k = 0; k < B / 2; k++) {
        s += v[k].x;
        o[k].x = s;
        s += v[k].y;
        o[k].y = s;
    }
    if (prefix) {
#pragma unroll
        for (int k = 0; k < B / 2; k++) *(double2*)(x + i + 2 * k) = o[k];
    }
}

__device__ double seq_sum(double* x, int n, bool prefix) {
    constexpr int B = 16;
    double s = 0.0;
    const int nb = ((uintptr_t)x & 15) == 0 ? n / (2 * B) * (2 * B) : 0;
    if (nb) {
        double2 v0[B / 2], v1[B / 2];
#pragma unroll
        for (int k = 0; k < B / 2; k++) v0[k] = *(const double2*)(x + 2 * k);
        for (int i = 0; i < nb; i += 2 * B) {
#pragma unroll
            for (int k = 0; k < B / 2; k++) v1[k] = *(const double2*)(x + i + B + 2 * k);
            __builtin_amdgcn_sched_barrier(0);
            seq_batch<B>(x, i, v0, s, prefix);
            __builtin_amdgcn_sched_barrier(0);
            const int j = min(i + 2 * B, nb - B);  // the next pair's first batch (past the end: a batch again)
#pragma unroll
            for (int k = 0; k < B / 2; k++) v0[k] = *(const double2*)(x + j + 2 * k);
            __builtin_amdgcn_sched_barrier(0);
            seq_batch<B>(x, i + B, v1, s, prefix);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    for (int i = nb; i < n; i++) {
        s += x[i];
        if (prefix) x[i] = s;
    }
    return s;
}

// The first k with r <= x[0] + ... + x[k] (summed in order), or dflt: the sequential scan of the
// reference, for short candidate lists.
__device__ int seq_find(const double* x, int n, double r, int dflt) {
    double cum = 0.0;
    for (int i = 0; i < n; i++) {
        cum += x[i];
        if (r <= cum) return i;
    }
    return dflt;
}

constexpr int kExtract = 64;  // candidates taken one by one before falling back to a full sort

// PHASE: 0 the whole draw; 2 from the exponentials in a.scratch (sample_exp_kernel) and their sums in
// a.sums (sample_sum_kernel) on, truncated sampling only.
template <int PHASE>
__global__ __launch_bounds__(kThreads) void sample_rows_kernel(SampleArgs a) {
    __shared__ double cand_v[kExtract];
    __shared__ int cand_i[kExtract];
    extern __shared__ __align__(16) double smp_smem[];
    __shared__ double red_v[kThreads / 64];
    __shared__ int red_i[kThreads / 64];
    __shared__ int chosen_sh;
    __shared__ int32_t win_sh[kRepWindow];
    const int row = blockIdx.x;
    const int V = a.V, n2 = a.n2;
    double* key = smp_smem;           // [n2] logits, then probabilities
    int* idx = (int*)(smp_smem + n2);  // [n2] token ids once sorted
    const long long base = (long long)row * a.ld;
    if constexpr (PHASE == 2) {
        if (a.flags && a.flags[row] == 0) return;  // drawn by sample_pick_kernel
        for (int i = threadIdx.x; i < V; i += blockDim.x) key[i] = a.scratch[(long long)row * V + i];
    } else {
        for (int i = threadIdx.x; i < V; i += blockDim.x)
            key[i] = a.logits32 ? (double)a.logits32[base + i] : a.logits64[base + i];
    }
    __syncthreads();

    if constexpr (PHASE != 2) {
        const int col = a.hist ? a.col : 0;
        const int32_t* g = a.hist ? a.hist + (long long)row * a.hist_ld : nullptr;
        // trigram blocking over the generated tokens (sample.go:211-224): every earlier occurrence of the
        // last two tokens bans the token that followed it (one thread per position; a token banned twice
        // is written the same value twice)
        if (a.trigram && col >= 2) {
            const int32_t w1 = g[col - 2], w2 = g[col - 1];
            for (int i = threadIdx.x; i + 2 < col; i += blockDim.x)
                if (g[i] == w1 && g[i + 1] == w2) {
                    const int32_t b = g[i + 2];
                    if (b >= 0 && b < V) key[b] = -DBL_MAX;
                }
        }
        // the repetition window: the last kRepWindow tokens of prefix + generated (sample.go:206-209),
        // gathered by one thread each
        const int from_hist = min(col, kRepWindow);
        const int plen = a.prefix_len ? a.prefix_len[row] : 0;
        const int from_pre = min(plen, kRepWindow - from_hist);
        const int nwin = from_pre + from_hist;
        if (a.p.rep_penalty > 1.0 && threadIdx.x < nwin) {
            const int k = threadIdx.x;
            win_sh[k] = k < from_pre ? a.prefix[(long long)row * a.prefix_ld + plen - from_pre + k]
                                     : g[col - from_hist + (k - from_pre)];
        }
        __syncthreads();
        // repetition penalty over the window, each distinct token once, after the bans
        // (sample.go:47-66)
        if (a.p.rep_penalty > 1.0 && threadIdx.x == 0) {
            for (int i = 0; i < nwin; i++) {
                const int32_t t = win_sh[i];
                if (t < 0 || t >= V) continue;
                bool seen = false;
                for (int j = 0; j < i; j++) seen |= win_sh[j] == t;
                if (!seen) key[t] = key[t] > 0 ? key[t] / a.p.rep_penalty : key[t] * a.p.rep_penalty;
            }
        }
    }
    __syncthreads();

    int chosen = 0;
    if (a.p.temperature <= 0.001) {
        double v = -INFINITY;  // the first maximum, as the reference's scan from index 0
        int bi = 0x7fffffff;
        for (int i = threadIdx.x; i < V; i += blockDim.x)
            if (before(key[i], i, v, bi)) { v = key[i]; bi = i; }
        double bv;
        block_argmax(v, bi, red_v, red_i, bv, chosen);
    } else {
        if constexpr (PHASE != 2) {
            const double invT = 1.0 / a.p.temperature;
            double v = -DBL_MAX;
            for (int i = threadIdx.x; i < V; i += blockDim.x) {
                const double sc = key[i] * invT;
                key[i] = sc;
                v = fmax(v, sc);
            }
            double mx;
            int dummy;
            block_argmax(v, 0, red_v, red_i, mx, dummy);
            for (int i = threadIdx.x; i < V; i += blockDim.x) key[i] = exp(key[i] - mx);
            __syncthreads();
        }
        const double u = a.u ? a.u[row] : uniform_draw(a.seeds[row], a.step);
        if (a.p.top_k <= 0 && a.p.top_p >= 0.9999) {
            // pure temperature sampling (sample.go:91-109): the running sums never decrease (every term
            // is >= 0), so the first index whose running sum reaches r is the count of those below it
            if (threadIdx.x == 0) red_v[0] = u * seq_sum(key, V, true);
            __syncthreads();
            const double r = red_v[0];
            int below = 0;
            for (int i = threadIdx.x; i < V; i += blockDim.x) below += key[i] < r;
            for (int o = 32; o > 0; o >>= 1) below += __shfl_xor(below, o);
            __syncthreads();
            if ((threadIdx.x & 63) == 0) red_i[threadIdx.x >> 6] = below;
            __syncthreads();
            if (threadIdx.x == 0) {
                int t = 0;
                for (int w = 0; w < (int)(blockDim.x >> 6); w++) t += red_i[w];
                chosen_sh = t < V ? t : 0;
            }
            __syncthreads();
            chosen = chosen_sh;
        } else {
            // truncated sampling (sample.go:111-171): probabilities p / sum(p), then the candidates in
            // descending order (equal probabilities by token id), cut by top-k and top-p
            if (threadIdx.x == 0) red_v[0] = 1.0 / (PHASE == 2 ? a.sums[row] : seq_sum(key, V, false));
            __syncthreads();
            const double inv = red_v[0];
            for (int i = threadIdx.x; i < V; i += blockDim.x) key[i] *= inv;
            __syncthreads();
            const int kcap = (a.p.top_k > 0 && a.p.top_k < V) ? a.p.top_k : V;
            const bool use_p = a.p.top_p > 0.0 && a.p.top_p < 1.0;
            int active = 0;
            const double* cv = cand_v;
            const int* ci = cand_i;
            if (kcap <= kExtract || use_p) {
                // The candidates one at a time, most probable first, until top-k or top-p is met, by the
                // first wave alone (no barriers). Lane L owns tokens L, L + 64, ... and keeps the four best
                // of them sorted in registers; a round is one wave argmax over the lanes' heads (DPP), then
                // the winning lane pops its head. A lane rescans its tokens (the taken ones marked below
                // every probability) only when all four of its cached ones are taken.
                const int rounds = min(kcap, kExtract);
                if (threadIdx.x < 64) {
                    const int lane = threadIdx.x;
                    double cv4[4];
                    int ci4[4];
                    auto refill = [&]() {
#pragma unroll
                        for (int q = 0; q < 4; q++) { cv4[q] = -INFINITY; ci4[q] = 0x7fffffff; }
                        for (int i0 = lane; i0 < V; i0 += 8 * 64) {
                            double kv[8];
#pragma unroll
                            for (int k = 0; k < 8; k++) kv[k] = key[min(i0 + 64 * k, V - 1)];
#pragma unroll
                            for (int k = 0; k < 8; k++) {
                                const int i = i0 + 64 * k;
                                double v = kv[k];
                                int vi = i;
                                if (i >= V || !before(v, vi, cv4[3], ci4[3])) continue;
                                // insertion into the sorted four
#pragma unroll
                                for (int q = 0; q < 4; q++) {
                                    if (before(v, vi, cv4[q], ci4[q])) {
                                        const double tv = cv4[q];
                                        const int ti = ci4[q];
                                        cv4[q] = v; ci4[q] = vi;
                                        v = tv; vi = ti;
                                    }
                                }
                            }
                        }
                    };
                    refill();
                    int taken = 0;  // this lane's tokens taken since its last refill
                    double cp = 0.0;
                    int act = 0;
                    for (int r = 0; r < rounds; r++) {
                        double bv = cv4[0];
                        int bi = ci4[0];
                        wave_argmax(bv, bi);
                        if (lane == 0) { cand_v[r] = bv; cand_i[r] = bi; }
                        cp += bv;
                        if ((use_p && cp >= a.p.top_p) || r + 1 == kcap) {
                            act = r + 1;
                            break;
                        }
                        if ((bi & 63) == lane) {
                            key[bi] = -2.0;  // taken: below every probability
                            cv4[0] = cv4[1]; ci4[0] = ci4[1];
                            cv4[1] = cv4[2]; ci4[1] = ci4[2];
                            cv4[2] = cv4[3]; ci4[2] = ci4[3];
                            cv4[3] = -INFINITY; ci4[3] = 0x7fffffff;
                            if (++taken == 4) {
                                refill();
                                taken = 0;
                            }
                        }
                    }
                    if (lane == 0) chosen_sh = act;
                }
                __syncthreads();
                active = chosen_sh;
                if (active == 0) {  // top-p not reached within kExtract candidates: sort them all
                    __syncthreads();
                    if (threadIdx.x == 0)
                        for (int r = 0; r < rounds; r++) key[cand_i[r]] = cand_v[r];
                    __syncthreads();
                }
            }
            if (active == 0) {
                for (int i = threadIdx.x; i < n2; i += blockDim.x) {
                    if (i < V) {
                        idx[i] = i;
                    } else {
                        key[i] = -1.0;  // padding sorts last
                        idx[i] = 0x7fffffff;
                    }
                }
                __syncthreads();
                bitonic_desc(key, idx, n2);
                if (threadIdx.x == 0) {
                    int act = kcap;
                    if (use_p) {
                        double cp = 0.0;
                        int cut = 0;
                        for (int i = 0; i < act; i++) {
                            cp += key[i];
                            cut = i + 1;
                            if (cp >= a.p.top_p) break;
                        }
                        act = cut;
                    }
                    chosen_sh = act;
                }
                __syncthreads();
                active = chosen_sh;
                cv = key;
                ci = idx;
                __syncthreads();
            }
            if (threadIdx.x == 0) {
                int c;
                if (active == 1) {
                    c = ci[0];
                } else {  // sampleFromCDF (sample.go:173-190)
                    double sp = 0.0;
                    for (int i = 0; i < active; i++) sp += cv[i];
                    const double r = u * sp;
                    c = ci[active - 1];
                    const int k = seq_find(cv, active, r, -1);
                    if (k >= 0) c = ci[k];
                }
                chosen_sh = c;
            }
            __syncthreads();
            chosen = chosen_sh;
        }
    }
    if (threadIdx.x == 0) {
        a.out[(long long)row * a.out_ld + a.out_col] = chosen;
        if (a.next_ids) a.next_ids[row] = chosen;
    }
}

// The penalised, tempered exponentials of one row per workgroup, the first launch of a sampled draw:
// e[i] = exp(x[i] / T - max_j x[j] / T) into a.scratch, x the logits after the trigram bans and the
// repetition penalty (sample.go:47-109 up to the exponentials, the same operations in float64 as
// sample_rows_kernel). The row stays in registers, KP values per thread; the bans are a bit per token
// in LDS and the window's penalised values a short list beside them, read by the threads that own those
// tokens. Without a row in LDS many rows run per CU.
template <int KP>
__global__ __launch_bounds__(kThreads) void sample_exp_kernel(SampleArgs a) {
    __shared__ uint32_t ban[kMaxSampleVocab / 32];
    __shared__ int32_t win_sh[kRepWindow];
    __shared__ int32_t ovr_t[kRepWindow];
    __shared__ double ovr_v[kRepWindow];
    __shared__ int novr_sh;
    __shared__ double red_v[kThreads / 64];
    __shared__ int red_i[kThreads / 64];
    const int row = blockIdx.x, V = a.V, tid = threadIdx.x;
    const long long base = (long long)row * a.ld;
    auto logit = [&](int i) { return a.logits32 ? (double)a.logits32[base + i] : a.logits64[base + i]; };
    // every load unconditional (columns clamped into the row), so that all KP are in flight at once
    double x[KP];
    if (a.logits32) {
        float xf[KP];
#pragma unroll
        for (int k = 0; k < KP; k++) xf[k] = a.logits32[base + min(tid + k * kThreads, V - 1)];
#pragma unroll
        for (int k = 0; k < KP; k++) x[k] = xf[k];
    } else {
#pragma unroll
        for (int k = 0; k < KP; k++) x[k] = a.logits64[base + min(tid + k * kThreads, V - 1)];
    }
    for (int w = tid; w < (V + 31) / 32; w += kThreads) ban[w] = 0;
    const int col = a.hist ? a.col : 0;
    const int32_t* g = a.hist ? a.hist + (long long)row * a.hist_ld : nullptr;
    const int from_hist = min(col, kRepWindow);
    const int plen = a.prefix_len ? a.prefix_len[row] : 0;
    const int from_pre = min(plen, kRepWindow - from_hist);
    const int nwin = from_pre + from_hist;
    const bool rep = a.p.rep_penalty > 1.0;
    if (rep && tid < nwin)  // the window: the last kRepWindow tokens of prefix + generated (sample.go:206-209)
        win_sh[tid] = tid < from_pre ? a.prefix[(long long)row * a.prefix_ld + plen - from_pre + tid]
                                     : g[col - from_hist + (tid - from_pre)];
    __syncthreads();
    // trigram blocking over the generated tokens (sample.go:211-224): every earlier occurrence of the
    // last two tokens bans the token that followed it
    if (a.trigram && col >= 2) {
        const int32_t w1 = g[col - 2], w2 = g[col - 1];
        for (int i = tid; i + 2 < col; i += kThreads)
            if (g[i] == w1 && g[i + 1] == w2) {
                const int32_t b = g[i + 2];
                if (b >= 0 && b < V) atomicOr(&ban[b >> 5], 1u << (b & 31));
            }
    }
    __syncthreads();
    // repetition penalty, each distinct window token once, on its value after the bans (sample.go:47-66)
    if (tid == 0) {
        int no = 0;
        if (rep)
            for (int i = 0; i < nwin; i++) {
                const int32_t t = win_sh[i];
                if (t < 0 || t >= V) continue;
                bool seen = false;
                for (int j = 0; j < i; j++) seen |= win_sh[j] == t;
                if (seen) continue;
                const double k0 = (ban[t >> 5] >> (t & 31)) & 1 ? -DBL_MAX : logit(t);
                ovr_t[no] = t;
                ovr_v[no] = k0 > 0 ? k0 / a.p.rep_penalty : k0 * a.p.rep_penalty;
                no++;
            }
        novr_sh = no;
    }
    __syncthreads();
    const int novr = novr_sh;
    const double invT = 1.0 / a.p.temperature;
    double v = -DBL_MAX;
#pragma unroll
    for (int k = 0; k < KP; k++) {
        const int i = tid + k * kThreads;
        if (i >= V) continue;
        double key = (ban[i >> 5] >> (i & 31)) & 1 ? -DBL_MAX : x[k];
        for (int j = 0; j < novr; j++)
            if (ovr_t[j] == i) key = ovr_v[j];
        x[k] = key * invT;
        v = fmax(v, x[k]);
    }
    double mx;
    int dummy;
    block_argmax(v, 0, red_v, red_i, mx, dummy);
    // The exponentials (8 bytes per token: 134 MB for 4096 rows of 4096) are stored and read back
    // (sample_sum_kernel, sample_pick_kernel) non-temporally, so that they do not displace the decode
    // step's weights and code from the caches.
    double* e = a.scratch + (long long)row * V;
#pragma unroll
    for (int k = 0; k < KP; k++) {
        const int i = tid + k * kThreads;
        if (i < V) __builtin_nontemporal_store(exp(x[k] - mx), e + i);
    }
}

// Truncated draw of one row by one wave, from the exponentials in a.scratch and the row sums in
// a.sums (top-k of at most kExtract, or top-p): p = e * (1 / sum), then the candidates in descending
// order (equal probabilities by token id) until top-k or top-p is met, and the draw over them
// (sample.go:111-190). The wave reads its row once, in batches of 8 values per lane. Every candidate
// lies at or above t, the rounds-th largest of the lanes' largest probabilities (at least rounds values
// do), and t only grows as the batches come in, so a batch's values at or above the current t are kept
// (compacted into LDS) and the rest can never be candidates. The kept values are then sorted in LDS. A row
// whose top-p mass is not reached within kExtract candidates, or whose kept values outgrow kPickCap, is
// flagged for sample_rows_kernel<2>, which sorts the whole row.
constexpr int kPickCap = 512;

// The k-th largest (1 <= k <= 64) of the wave's 64 values, in every lane: a bitonic sort across the
// lanes into descending order, then lane k - 1's value.
__device__ __forceinline__ double wave_kth_largest(double x, int k, int lane) {
#pragma unroll
    for (int s = 2; s <= 64; s <<= 1) {
#pragma unroll
        for (int j = s >> 1; j > 0; j >>= 1) {
            const double y = __shfl_xor(x, j);
            const bool keep_max = ((lane & j) == 0) == ((lane & s) == 0);
            x = keep_max ? fmax(x, y) : fmin(x, y);
        }
    }
    return __shfl(x, k - 1);
}

// Drops the kept values below t, keeping the others' order; returns how many remain.
__device__ __forceinline__ int pick_refilter(double* cv, int* ci, int count, double t, int lane) {
    int kept = 0;
    for (int q = 0; q < count; q += 64) {
        const int i = q + lane;
        const double v = i < count ? cv[i] : -1.0;
        const int id = i < count ? ci[i] : 0;
        const bool keep = i < count && v >= t;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(keep);
        // every slot written lies below every slot still to be read
        if (keep) {
            const int pos = kept + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
            cv[pos] = v;
            ci[pos] = id;
        }
        kept += __popcll(bal);
    }
    return kept;
}

__global__ __launch_bounds__(64) void sample_pick_kernel(SampleArgs a) {
    __shared__ double cand_v[kPickCap];
    __shared__ int cand_i[kPickCap];
    const int row = blockIdx.x, lane = threadIdx.x, V = a.V;
    const double* e = a.scratch + (long long)row * V;
    const double inv = 1.0 / a.sums[row];
    const int kcap = (a.p.top_k > 0 && a.p.top_k < V) ? a.p.top_k : V;
    const bool use_p = a.p.top_p > 0.0 && a.p.top_p < 1.0;
    const int rounds = min(kcap, kExtract);
    double m = -1.0;  // this lane's largest probability so far (probabilities are >= 0)
    double t = -1.0;
    int count = 0;
    bool over = false;
    for (int b = 0; b < V; b += 8 * 64) {
        double kv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) kv[k] = __builtin_nontemporal_load(e + min(b + 64 * k + lane, V - 1)) * inv;
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (b + 64 * k + lane < V) m = fmax(m, kv[k]);
        t = wave_kth_largest(m, rounds, lane);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (count + 64 > kPickCap) {
                count = pick_refilter(cand_v, cand_i, count, t, lane);
                if (count + 64 > kPickCap) {
                    over = true;
                    break;
                }
            }
            const int i = b + 64 * k + lane;
            const bool keep = i < V && kv[k] >= t;
            const uint64_t bal = __builtin_amdgcn_ballot_w64(keep);
            if (keep) {
                const int pos = count + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
                cand_v[pos] = kv[k];
                cand_i[pos] = i;
            }
            count += __popcll(bal);
        }
        if (over) break;
    }
    int act = 0;
    if (!over) {
        count = pick_refilter(cand_v, cand_i, count, t, lane);
        int n2 = 64;
        while (n2 < count) n2 <<= 1;
        for (int i = count + lane; i < n2; i += 64) {
            cand_v[i] = -1.0;  // padding sorts last
            cand_i[i] = 0x7fffffff;
        }
        __syncthreads();
        bitonic_desc(cand_v, cand_i, n2);
        if (lane == 0) {
            double cp = 0.0;
            for (int r = 0; r < rounds; r++) {
                cp += cand_v[r];
                if ((use_p && cp >= a.p.top_p) || r + 1 == kcap) {
                    act = r + 1;
                    break;
                }
            }
        }
    }
    if (lane != 0) return;
    a.flags[row] = act == 0;
    if (act == 0) return;
    int c = cand_i[0];
    if (act > 1) {  // sampleFromCDF (sample.go:173-190)
        const double u = a.u ? a.u[row] : uniform_draw(a.seeds[row], a.step);
        double sp = 0.0;
        for (int i = 0; i < act; i++) sp += cand_v[i];
        const double r = u * sp;
        c = cand_i[act - 1];
        const int k = seq_find(cand_v, act, r, -1);
        if (k >= 0) c = cand_i[k];
    }
    a.out[(long long)row * a.out_ld + a.out_col] = c;
    if (a.next_ids) a.next_ids[row] = c;
}

// The rows' sequential float64 sums, one lane per row: sums[row] = e[0] + e[1] + ... in index order (the
// reference's loop). Each row is one chain of V dependent additions, so the kernel is bound by how fast a
// lane can be fed: kSumRows rows per wave (the remaining lanes idle), one wave per CU, and the rows stream
// through an LDS ring of kSumRing blocks of kSumCols columns, filled by direct global-to-LDS loads (no
// registers held), so that about kSumRing blocks are in flight while the lanes add. For pure temperature
// sampling (pure != 0) the lane also draws: the first index whose running sum reaches u * sum (the same
// sums again), or 0 when none does.
//
// A block holds row j's 16-byte column pair p at slot j * kSumPairs + (p ^ j): the lanes reading one pair
// of their rows at once touch 16 different slots, so the reads do not conflict in the LDS banks.
constexpr int kSumRows = 16;
constexpr int kSumCols = 32;
constexpr int kSumPairs = kSumCols / 2;
constexpr int kSumBlockLoads = kSumRows * kSumPairs / 64;  // 1 KiB direct-to-LDS loads per block
constexpr int kSumBlock = kSumRows * kSumCols;             // doubles per ring slot
constexpr int kSumRing = 16;
static_assert(kSumPairs == kSumRows, "the slot swizzle pairs every row with every column pair");
static_assert(kSumBlockLoads * (kSumRing - 2) == 56, "the ring's waits below count 56 loads in flight");

// One 16-byte load per lane from global memory straight into LDS, non-temporal (the exponentials are
// read once more, by sample_pick_kernel, and never again): lane L's bytes land at LDS offset lds + 16 L. Issued through inline assembly, with the waits for it written out below, because the
// compiler, which cannot tell which LDS bytes such a load writes, waits for every one of them before any
// LDS read, and the ring would then hold one block in flight instead of kSumRing. The load takes its LDS
// address from M0, which the compiler reserves (it cannot be listed as clobbered): nothing else in this
// file's device code uses M0, so no value of the compiler's lives there. An LDS-DMA load may not read M0
// in the instruction right after the SALU write of it (one wait state, which the compiler cannot add
// inside an asm statement): the s_nop.
__device__ __forceinline__ void lds_load16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(lds) : "memory");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Loads block cb of rows r0.. into ring slot dst: load u of lane L fills slot u * 64 + L, i.e. row
// (u * 64 + L) / kSumPairs and pair ((u * 64 + L) % kSumPairs) ^ row; rows and columns clamped into the
// array (clamped loads fetch valid memory that nobody reads).
__device__ __forceinline__ void sum_block_issue(const double* e, int n, int V, int r0, int cb, int lane,
                                                uint32_t dst) {
#pragma unroll
    for (int u = 0; u < kSumBlockLoads; u++) {
        const int s = u * 64 + lane, j = s / kSumPairs, p = (s % kSumPairs) ^ j;
        const int r = min(r0 + j, n - 1);
        const int c = min(cb * kSumCols + 2 * p, V - 2);
        lds_load16(e + (long long)r * V + c, dst + u * 1024);
    }
}

// Visits e[row][0], e[row][1], ... in order for the wave's rows (lane L < kSumRows: row r0 + L), f(index,
// value) per element; stops after the block in which every lane's f has returned true.
template <class F>
__device__ __forceinline__ void sum_rows_scan(const double* e, int n, int V, int r0, int lane, double* ring, F&& f) {
    const bool mine_row = lane < kSumRows;
    if (V & 1) {  // rows not 16-byte aligned: each lane reads its own row
        if (!mine_row) return;
        const double* rowp = e + (long long)min(r0 + lane, n - 1) * V;
        for (int c = 0; c < V; c++)
            if (f(c, rowp[c])) break;
        return;
    }
    const int nb = (V + kSumCols - 1) / kSumCols;
    const uint32_t ring0 = lds_offset(ring);
    constexpr uint32_t kSlotBytes = kSumBlock * sizeof(double);
    // only vector memory operations of this scan may be outstanding when its waits count them
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int pre = min(nb, kSumRing - 1);
    // each lane's source of load u of a whole block, column 0: block cb adds cb * kSumCols (the clamped
    // addresses of sum_block_issue are needed only for the last, partial block)
    const double* src[kSumBlockLoads];
#pragma unroll
    for (int u = 0; u < kSumBlockLoads; u++) {
        const int s = u * 64 + lane, j = s / kSumPairs, p = (s % kSumPairs) ^ j;
        src[u] = e + (long long)min(r0 + j, n - 1) * V + 2 * p;
    }
    auto issue = [&](int cb, uint32_t dst) {
        if ((cb + 1) * kSumCols <= V) {
#pragma unroll
            for (int u = 0; u < kSumBlockLoads; u++) lds_load16(src[u] + cb * kSumCols, dst + u * 1024);
        } else {
            sum_block_issue(e, n, V, r0, cb, lane, dst);
        }
    };
    for (int b = 0; b < pre; b++) issue(b, ring0 + b * kSlotBytes);
    bool done = !mine_row;
    const int jl = lane & (kSumRows - 1);
    auto full = [&](int cb) { return (cb + 1) * kSumCols <= V; };
    // a block's values into registers; read by every lane whatever it needs (a ring slot is always valid
    // LDS), so that no branch hides from the compiler how many LDS reads are outstanding, and the wait for
    // one block's values does not also wait for the next block's
    auto rd = [&](double2(&v)[kSumPairs], int cb) {
        const double2* m = (const double2*)(ring + (cb % kSumRing) * kSumBlock) + jl * kSumPairs;
#pragma unroll
        for (int p = 0; p < kSumPairs; p++) v[p] = m[p ^ jl];
    };
    // Block cb from registers cur, while block cb + 1 is read into nxt: the LDS reads of the next block
    // overlap the chain of additions. True once every lane is done.
    auto step = [&](int cb, double2(&cur)[kSumPairs], double2(&nxt)[kSumPairs]) {
        // cur has arrived, and the slot refilled now (block cb - 1's) was read before it (the builtin, not
        // inline assembly: the compiler counts this wait, so it adds no wait of its own for cur below)
        __builtin_amdgcn_s_waitcnt(0xc07f);
        asm volatile("" ::: "memory");
        if (cb + kSumRing - 1 < nb) {
            issue(cb + kSumRing - 1, ring0 + ((cb + kSumRing - 1) % kSumRing) * kSlotBytes);
            asm volatile("s_waitcnt vmcnt(56)" ::: "memory");  // block cb + 1 is in LDS
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        rd(nxt, cb + 1);
        const int c0 = cb * kSumCols;
        if (!done) {
            if (full(cb)) {
#pragma unroll
                for (int p = 0; p < kSumPairs; p++) {
                    if (!done && f(c0 + 2 * p, cur[p].x)) done = true;
                    if (!done && f(c0 + 2 * p + 1, cur[p].y)) done = true;
                }
            } else {
                // the last block of a vocabulary that is not a multiple of kSumCols was loaded from
                // clamped columns: its values are read from their true columns
                const double* rowp = e + (long long)min(r0 + lane, n - 1) * V;
                for (int c = c0; c < V; c++)
                    if (!done && f(c, rowp[c])) done = true;
            }
        }
        return __builtin_amdgcn_ballot_w64(!done) == 0;
    };
    double2 va[kSumPairs], vb[kSumPairs];
    if (pre == kSumRing - 1) asm volatile("s_waitcnt vmcnt(56)" ::: "memory");  // block 0 is in LDS
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    rd(va, 0);
    for (int cb = 0; cb < nb; cb += 2) {
        if (step(cb, va, vb)) break;
        if (cb + 1 < nb && step(cb + 1, vb, va)) break;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the scan
}

__global__ __launch_bounds__(64) void sample_sum_kernel(SampleArgs a, int pure) {
    __shared__ __align__(16) double ring[kSumRing * kSumBlock];
    const int lane = threadIdx.x, r0 = blockIdx.x * kSumRows, row = r0 + lane;
    const int V = a.V, n = a.n;
    double s = 0.0;
    sum_rows_scan(a.scratch, n, V, r0, lane, ring, [&](int, double v) {
        s += v;
        return false;
    });
    if (!pure) {
        if (lane < kSumRows && row < n) a.sums[row] = s;
        return;
    }
    // every lane stays for the second pass: each lane loads its share of every block
    const int rc = min(row, n - 1);
    const double u = a.u ? a.u[rc] : uniform_draw(a.seeds[rc], a.step);
    const double r = u * s;
    double c = 0.0;
    int t = V;
    sum_rows_scan(a.scratch, n, V, r0, lane, ring, [&](int i, double v) {
        c += v;
        if (c >= r) {
            t = i;
            return true;
        }
        return false;
    });
    if (lane >= kSumRows || row >= n) return;
    const int chosen = t < V ? t : 0;
    a.out[(long long)row * a.out_ld + a.out_col] = chosen;
    if (a.next_ids) a.next_ids[row] = chosen;
}

}  // namespace

size_t sample_scratch_bytes(int n, int V) {
    return ((size_t)n * V + (size_t)n) * sizeof(double) + ((size_t)n * sizeof(int32_t) + 7) / 8 * 8;
}

int sample_n2(int V) {
    int n2 = 1;
    while (n2 < V) n2 <<= 1;
    return n2;
}

size_t sample_lds_bytes(int V) { return (size_t)sample_n2(V) * (sizeof(double) + sizeof(int)); }

hipError_t launch_sample(const SampleArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    // the candidate sort (and its index array) is only reachable when top-k leaves more than kExtract
    // candidates or top-p is on; otherwise the row of float64 values is all the kernel keeps in LDS
    const bool truncated = a.p.temperature > 0.001 && !(a.p.top_k <= 0 && a.p.top_p >= 0.9999);
    const int kcap = (a.p.top_k > 0 && a.p.top_k < a.V) ? a.p.top_k : a.V;
    const bool use_p = a.p.top_p > 0.0 && a.p.top_p < 1.0;
    const bool may_sort = truncated && (kcap > kExtract || use_p);
    const size_t lds = may_sort ? sample_lds_bytes(a.V) : (size_t)a.V * sizeof(double);
    static const hipError_t attr0 = hipFuncSetAttribute((const void*)sample_rows_kernel<0>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                                        (int)sample_lds_bytes(kMaxSampleVocab));
    static const hipError_t attr2 = hipFuncSetAttribute((const void*)sample_rows_kernel<2>,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                                        (int)sample_lds_bytes(kMaxSampleVocab));
    if (attr0 != hipSuccess) return attr0;
    if (attr2 != hipSuccess) return attr2;
    const bool sampled = a.p.temperature > 0.001;
    if (!sampled || !a.scratch || !a.sums) {
        hipLaunchKernelGGL(sample_rows_kernel<0>, dim3(a.n), dim3(kThreads), lds, s, a);
        return hipGetLastError();
    }
    // three passes: exponentials per row, the rows' sums one lane per row, then the truncated draw (one
    // wave per row; the rows it flags, and every row when top-k exceeds kExtract without top-p, sorted)
    if (a.V <= 4 * kThreads) hipLaunchKernelGGL(sample_exp_kernel<4>, dim3(a.n), dim3(kThreads), 0, s, a);
    else if (a.V <= 8 * kThreads) hipLaunchKernelGGL(sample_exp_kernel<8>, dim3(a.n), dim3(kThreads), 0, s, a);
    else if (a.V <= 16 * kThreads) hipLaunchKernelGGL(sample_exp_kernel<16>, dim3(a.n), dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL(sample_exp_kernel<kMaxSampleVocab / kThreads>, dim3(a.n), dim3(kThreads), 0, s, a);
    hipLaunchKernelGGL(sample_sum_kernel, dim3((a.n + kSumRows - 1) / kSumRows), dim3(64), 0, s, a, truncated ? 0 : 1);
    if (truncated) {
        SampleArgs b = a;
        b.flags = nullptr;
        if ((kcap <= kExtract || use_p) && a.flags) {
            hipLaunchKernelGGL(sample_pick_kernel, dim3(a.n), dim3(64), 0, s, a);
            b.flags = a.flags;
        }
        hipLaunchKernelGGL(sample_rows_kernel<2>, dim3(a.n), dim3(kThreads), lds, s, b);
    }
    return hipGetLastError();
}

}  // namespace mg
