// Non-GEMM kernels of the INT8 engine for gfx950: per-row embedding / residual / RMSNorm / limb
// expansion, the selective-latch scan, windowed attention, head statistics and the quantiser.
//
// Arithmetic follows the reference INT8 engine (internal/quant/stream.go, internal/quant/attention.go,
// internal/nn) with the same rounding points; the reduction orders of the reference's AVX2 kernels are
// reproduced where a result depends on them (RMSNorm's sum of squares, attention dot products, softmax
// sums, the P.V accumulation), so these stages are bit-identical to the reference given equal inputs.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "common.hpp"
#include "gemm.hpp"
#include "kernels.hpp"
#include "options.hpp"

namespace mg {

namespace {

// ------------------------------------------------------------------------------------------------
// Row kernel: one workgroup (4 waves) per 16-token tile, i.e. one row block of the GEMM operand layout.
// Wave w owns rows 4w..4w+3 and processes RB of them at a time with all their loads in flight; lane L
// holds float4 chunks c = L + 64i (elements 4c..4c+3). RMSNorm's sum of squares follows DotF32's AVX2
// order: 16 sequential partial sums over 16-element chunks, computed for RB rows at once by 16-lane
// groups. Limb bytes go to a padded LDS copy of the tile's fragments (one dword per chunk and limb),
// which is then written out with 16-byte stores.
// ------------------------------------------------------------------------------------------------
constexpr int ROW_TILE = 16;
// The row and scan kernels' outputs (normalised rows, limb fragments) are far larger than the caches at
// the sizes that matter and are read back by the next kernel from memory in any case: non-temporal
// stores (c5: latch scan 11.59 -> 11.32 ms per step, row kernels 31.1 -> 30.9).
__device__ __forceinline__ void nt_store4(float* dst, float4 v) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, (f4*)dst);
}
// LDS staging of one 16-row tile in the fragment layout: each 1 KiB fragment padded to 1088 bytes and
// each 256-byte column group inside it to 272, so that a wave's dword writes of one row spread over
// the banks.
__device__ __forceinline__ int stage_off(int o) { return (o >> 10) * 1088 + ((o >> 8) & 3) * 272 + (o & 255); }

// Rows per wave pass: enough loads in flight for narrow rows, few enough registers for wide ones (the
// 1024-column rows of the GLU output: one row per pass holds 162 registers, three waves per SIMD, against
// 213 and two for two rows: c5 row kernels 28.0 -> 27.0 ms per step; 384-column rows lose 5 ms with two
// per pass instead of four).
template <int NS4>
constexpr int row_batch() { return NS4 <= 2 ? 4 : (NS4 <= 3 ? 2 : 1); }

template <int NS4>
__global__ __launch_bounds__(256) void row_kernel(RowArgs a) {
    constexpr int RB = row_batch<NS4>();
    extern __shared__ __align__(16) int8_t row_smem[];
    int8_t* smem = row_smem;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int D = a.D, Dp = a.Dp, C4 = Dp >> 2;
    const int m_base = blockIdx.x * ROW_TILE;
    int8_t* stage = smem;
    const int stage_bytes = a.limbs ? (Dp >> 6) * 3 * 1088 : 0;
    const int xstride = Dp + 16;
    float* xs = (float*)(smem + stage_bytes) + w * RB * xstride;

    for (int j0 = 0; j0 < 4; j0 += RB) {
        float4 x[RB][NS4];
        int rows[RB];
        // ---- loads (and the embedding / residual writes) for RB rows. Loads are unconditional, from a
        // row and column clamped into the arrays, all issued before any is used, and masked afterwards
        // (a guarded load becomes a branch that waits for it on the spot); stores stay guarded. The mode
        // is tested once, outside the unrolled loops, so that each mode's loads share one basic block.
        int mcl[RB];
        bool okr[RB][NS4];
#pragma unroll
        for (int j = 0; j < RB; j++) {
            const int m = m_base + 4 * w + j0 + j;
            rows[j] = m;
            mcl[j] = min(m, a.M - 1);
#pragma unroll
            for (int i = 0; i < NS4; i++) okr[j][i] = m < a.M && lane + 64 * i < C4;
        }
        auto coff = [&](int j, int i) { return (long long)mcl[j] * Dp + 4 * min(lane + 64 * i, C4 - 1); };
        if (a.mode == ROW_RESID) {
            // inter-block residual: blockIn += cur; cur = blockIn (stream.go:157-163)
            float4 bi[RB][NS4], cu[RB][NS4];
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    bi[j][i] = *(const float4*)(a.block_in + coff(j, i));
                    cu[j][i] = *(const float4*)(a.cur + coff(j, i));
                }
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    const float4 v = make_float4(bi[j][i].x + cu[j][i].x, bi[j][i].y + cu[j][i].y,
                                                 bi[j][i].z + cu[j][i].z, bi[j][i].w + cu[j][i].w);
                    if (okr[j][i]) {
                        *(float4*)(a.block_in + coff(j, i)) = v;
                        *(float4*)(a.cur + coff(j, i)) = v;
                    }
                    x[j][i] = okr[j][i] ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
        } else if (a.mode == ROW_EMBED) {
            // quant.Model.appendPosition: clamp the id, dequantise (stream.go:144-152)
            int id[RB];
#pragma unroll
            for (int j = 0; j < RB; j++) {
                int v = a.ids[mcl[j]];
                id[j] = (v < 0 || v >= a.V) ? 0 : v;
            }
            int8_t eb[RB][NS4][4];
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++)
#pragma unroll
                    for (int k = 0; k < 4; k++)
                        eb[j][i][k] = a.emb[(long long)id[j] * D + min(4 * min(lane + 64 * i, C4 - 1) + k, D - 1)];
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    const int c = lane + 64 * i;
                    float t[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) t[k] = (okr[j][i] && 4 * c + k < D) ? (float)eb[j][i][k] * a.emb_scale : 0.0f;
                    const float4 v = make_float4(t[0], t[1], t[2], t[3]);
                    if (okr[j][i]) {
                        *(float4*)(a.cur + coff(j, i)) = v;
                        *(float4*)(a.block_in + coff(j, i)) = v;
                    }
                    x[j][i] = v;
                }
        } else if (a.mode == ROW_RULE) {
            // rule input [n | left | g] (stream.go:180-184, ca.AssembleNeighborhood): chunk c lies in
            // segment c / (seg/4) (segments are multiples of 4 columns wide)
            const int seg = a.seg, s4 = seg >> 2;
            float4 raw[RB][NS4];
            bool segok[RB][NS4];
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    const int cc = min(lane + 64 * i, C4 - 1);
                    const int sg = cc / s4, col = 4 * (cc - sg * s4);
                    const int mm = mcl[j];
                    const int t = mm % a.T;
                    const bool has_left = t >= a.dil;
                    const long long row = sg == 1 ? (has_left ? mm - a.dil : mm) : mm;
                    const float* base = sg == 2 ? a.src2 : a.src;
                    raw[j][i] = *(const float4*)(base + row * seg + col);
                    segok[j][i] = sg != 1 || has_left;
                }
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    const int c = lane + 64 * i;
                    const int cc = min(c, C4 - 1);
                    const int col = 4 * (cc - (cc / s4) * s4);
                    const bool ok = okr[j][i] && segok[j][i];
                    float4 v = raw[j][i];
                    v.x = (ok && col + 0 < D) ? v.x : 0.0f;
                    v.y = (ok && col + 1 < D) ? v.y : 0.0f;
                    v.z = (ok && col + 2 < D) ? v.z : 0.0f;
                    v.w = (ok && col + 3 < D) ? v.w : 0.0f;
                    x[j][i] = v;
                }
        } else {
            const float* sp = a.src ? a.src : a.cur;
            const int lds = a.src ? a.lds : Dp;
            long long r[RB];
#pragma unroll
            for (int j = 0; j < RB; j++) r[j] = a.row_map ? a.row_map[mcl[j]] : mcl[j];
            float4 raw[RB][NS4];
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++) raw[j][i] = *(const float4*)(sp + r[j] * lds + 4 * min(lane + 64 * i, C4 - 1));
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    // columns past D (and rows or chunks out of range) read as zero
                    const int c = lane + 64 * i;
                    const bool ok = okr[j][i];
                    float4 v = raw[j][i];
                    v.x = (ok && 4 * c + 0 < D) ? v.x : 0.0f;
                    v.y = (ok && 4 * c + 1 < D) ? v.y : 0.0f;
                    v.z = (ok && 4 * c + 2 < D) ? v.z : 0.0f;
                    v.w = (ok && 4 * c + 3 < D) ? v.w : 0.0f;
                    x[j][i] = v;
                }
        }

        // ---- RMSNorm (nn.RMSNormForwardF32, internal/nn/rmsnorm.go:14-32)
        if (a.gamma) {
#pragma unroll
            for (int j = 0; j < RB; j++)
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    const int c = lane + 64 * i;
                    if (c < C4) *(float4*)(xs + j * xstride + 4 * c) = x[j][i];
                }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes have landed
            __builtin_amdgcn_wave_barrier();
            // lane 16j + p: partial sum p of row j, sequential over the 16-element chunks
            const int jr = lane >> 4, p = lane & 15;
            const float* xr = xs + (jr < RB ? jr : 0) * xstride;
            float part = 0.0f;
            if (jr < RB) {
                const int c16 = D >> 4;
#pragma unroll 8
                for (int c = 0; c < c16; c++) {
                    const float v = xr[16 * c + p];
                    part = fmaf(v, v, part);
                }
                if (p < 8 && D - 16 * c16 >= 8) {
                    const float v = xr[16 * c16 + p];
                    part = fmaf(v, v, part);
                }
            }
            float v8[8];
            const int base = lane & 48;
#pragma unroll
            for (int q = 0; q < 8; q++) v8[q] = __shfl(part, base + q, 64) + __shfl(part, base + q + 8, 64);
            float ss = hreduce8(v8);
            for (int e = (D >> 3) << 3; e < D; e++) {
                const float t = xr[e];
                const float pp = t * t;
                ss = ss + pp;
            }
            const float rms = (float)sqrt((double)(ss / (float)D + 1e-5f));
            const float inv = 1.0f / rms;
#pragma unroll
            for (int j = 0; j < RB; j++) {
                const float inv_j = __shfl(inv, 16 * j, 64);
                if (a.rinv && lane == 0 && rows[j] < a.M) a.rinv[rows[j]] = inv_j;
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    const int c = lane + 64 * i;
                    const float4 gm = *(const float4*)(a.gamma + 4 * min(c, C4 - 1));
                    if (c < C4) {
                        float4 v = x[j][i];
                        v.x = (v.x * inv_j) * gm.x;
                        v.y = (v.y * inv_j) * gm.y;
                        v.z = (v.z * inv_j) * gm.z;
                        v.w = (v.w * inv_j) * gm.w;
                        x[j][i] = v;
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();  // xs is rewritten by this wave's next rows
        }

        // ---- outputs: normalised rows, limb expansion into the staged tile
#pragma unroll
        for (int j = 0; j < RB; j++) {
            const int m = rows[j];
            const bool valid = m < a.M;
            if (a.nout && valid) {
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    const int c = lane + 64 * i;
                    if (c < C4) nt_store4(a.nout + (long long)m * Dp + 4 * c, x[j][i]);
                }
            }
            if (a.limbs) {
                float mx = 0.0f;
#pragma unroll
                for (int i = 0; i < NS4; i++)
                    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x[j][i].x), fabsf(x[j][i].y)), fmaxf(fabsf(x[j][i].z), fabsf(x[j][i].w))));
                mx = wave_max(mx);
                float sc, inv;
                limb_scale(mx, sc, inv);
                const int rr = 4 * w + j0 + j;
#pragma unroll
                for (int i = 0; i < NS4; i++) {
                    const int c = lane + 64 * i;
                    if (c < C4) {
                        uint32_t w0, w1, w2;
                        split4_pack(x[j][i], inv, w0, w1, w2);
                        // elements 4c..4c+3: K step c>>4, byte 4(c&3) of column group (c>>2)&3, row rr
                        const int o = (c >> 4) * 3072 + (rr + 16 * ((c >> 2) & 3)) * 16 + 4 * (c & 3);
                        *(uint32_t*)(stage + stage_off(o)) = w0;
                        *(uint32_t*)(stage + stage_off(o + 1024)) = w1;
                        *(uint32_t*)(stage + stage_off(o + 2048)) = w2;
                    }
                }
                if (lane == 0 && valid) a.lscale[m] = sc;
            }
        }
    }
    if (a.limbs) {
        __syncthreads();
        const int bytes = 3 * Dp * ROW_TILE;  // Dp/64 K steps x 3 limbs x 1 KiB
        int8_t* dst = a.limbs + (long long)blockIdx.x * bytes;
        for (int o = threadIdx.x * 16; o < bytes; o += 256 * 16)
            __builtin_nontemporal_store(*(const v4i*)(stage + stage_off(o)), (v4i*)(dst + o));
    }
}

// Rule input [n | left | g] of token m, channel d, limb-expanded with row scale 1/inv into the GEMM
// fragment layout (K = 3*Dp; segment s occupies columns [s*Dp, (s+1)*Dp)).
__device__ __forceinline__ void store_x_limbs(int8_t* xl, int m, int d, int Dp, int kc, float n, float left, float g,
                                              float inv) {
    const float v[3] = {n, left, g};
#pragma unroll
    for (int sg = 0; sg < 3; sg++) {
        Limbs L = split_limbs(v[sg], inv);
        const int k = sg * Dp + d;
        xl[frag_off_a(m, k, 0, kc)] = L.q0;
        xl[frag_off_a(m, k, 1, kc)] = L.q1;
        xl[frag_off_a(m, k, 2, kc)] = L.q2;
    }
}

// ------------------------------------------------------------------------------------------------
// Latch scan: one workgroup per sequence, one thread per channel, sequential over positions.
// quant.Model.updateLatch (stream.go:195-205): g = lam*g + (1-lam)*n, written for every position (the
// rule input [n | left | g] is then limb-expanded by the row kernel in ROW_RULE mode). Rounds of 16
// positions: every load of the round is issued first (none depends on the latch), from clamped rows.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void scan_kernel(ScanArgs a) {
    const int b = blockIdx.x;
    const int d = threadIdx.x;
    const int D = a.D, Dp = a.Dp, T = a.T;
    const int last = a.lens ? a.lens[b] - 1 : -1;
    const bool on = d < D;
    const int dc = min(d, D - 1);
    const long long seq0 = (long long)b * T;
    float g = 0.0f;
    for (int t0 = 0; t0 < T; t0 += 16) {
        const int nt = min(16, T - t0);
        float nv[16], lm[16];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const long long m = seq0 + min(t0 + k, T - 1);
            nv[k] = a.nf[m * Dp + dc];
            lm[k] = a.lam[m * Dp + dc];
        }
#pragma unroll
        for (int k = 0; k < 16; k++) {
            if (k < nt) {
                if (on) {
                    const float p1 = lm[k] * g;
                    const float p2 = (1.0f - lm[k]) * nv[k];
                    g = p1 + p2;
                }
                a.g[(seq0 + t0 + k) * Dp + d] = on ? g : 0.0f;
                if (t0 + k == last && a.g_out) a.g_out[(long long)b * Dp + d] = on ? g : 0.0f;
            }
        }
    }
}

// Row maxima of 16 positions across a wave: v[k] is this lane's value for position k. Each exchange
// halves the set a lane keeps (the half its lane bit selects) and folds in the partner's maxima of that
// half; afterwards lane L holds the wave's maximum for position 8*b5 + 4*b4 + 2*b3 + b2 (bK = bit K
// of L), in all four lanes that share bits 2..5.
// (The empty asm makes each pair's values opaque, so that the compiler selects between the two values
// and does not turn the choice into a lane-dependent index into the array.)
__device__ __forceinline__ float opaque(float x) {
    asm("" : "+v"(x));
    return x;
}

__device__ __forceinline__ float wave_max16(float (&v)[16], int lane) {
#pragma unroll
    for (int h = 8, o = 32; h >= 1; h >>= 1, o >>= 1) {
        const bool hi = (lane & o) != 0;
#pragma unroll
        for (int i = 0; i < h; i++) {
            const float lo = opaque(v[i]), up = opaque(v[i + h]);
            const float keep = hi ? up : lo;
            const float send = hi ? lo : up;
            v[i] = fmaxf(keep, __shfl_xor(send, o, 64));
        }
    }
    float r = v[0];
    r = fmaxf(r, __shfl_xor(r, 2, 64));
    r = fmaxf(r, __shfl_xor(r, 1, 64));
    return r;
}

// ------------------------------------------------------------------------------------------------
// Latch scan fused with the rule input. One workgroup per sequence; thread j owns channels 2j, 2j+1
// and runs the recurrence over the positions in rounds of one 16-token tile (T is a multiple of 16, so
// a tile never spans two sequences). Per round:
//   - loads of n and lambda for the 16 positions, all issued first;
//   - g = lam*g + (1-lam)*n with scan_kernel's rounding (stream.go:195-205);
//   - the absmax of each row [n | left | g] (stream.go:180-184): the wave maxima of |n| and |g|
//     (wave_max16) are combined through LDS, and the left segment's maximum is the max|n| of row
//     t - dil, kept in a 64-row ring (dilations are at most 48, so the ring never overwrites a row
//     still needed);
//   - the three segments, limb-expanded into LDS in the fragment layout, one at a time, each stored as
//     whole 1 KiB fragments; the left neighbours n[t - dil] are loaded again (from cache) only then.
// The output is byte-identical to scan_kernel followed by row_kernel in ROW_RULE mode, without writing
// g and reading it back. g is stored only as a session's exported state.
// RN: n is not read from a normalised copy but recomputed from the norm's source rows and the row
// kernel's 1/rms per row, with the row kernel's operations, (x * rinv) * gamma: the same bits, and the
// normalised rows never have to be written.
// ------------------------------------------------------------------------------------------------
template <bool RN>
__global__ __launch_bounds__(512) void scan_rule_kernel(ScanArgs a) {
    extern __shared__ __align__(16) int8_t sr_smem[];
    const int b = blockIdx.x, j = threadIdx.x, lane = j & 63, w = j >> 6, nw = blockDim.x >> 6;
    const int D = a.D, Dp = a.Dp, T = a.T, C2 = Dp >> 1, dil = a.dil;
    const int jc = min(j, C2 - 1);
    const int seg_bytes = (Dp >> 6) * 3072;  // one segment of a tile: Dp/64 K steps x 3 limbs x 1 KiB
    int8_t* stage = sr_smem;
    float* red = (float*)(sr_smem + (seg_bytes >> 10) * 1088);  // [2][nw][16] wave maxima of |n|, |g|
    float* nring = red + 32 * nw;                                // [64] max|n| of row t at t & 63
    float* part = nring + 64;                                    // [16] max(|n|, |g|) of the round's rows
    float* invs = part + 16;                                     // [16] 127 / row absmax
    const long long seq0 = (long long)b * T;
    const int last = a.lens ? a.lens[b] - 1 : -1;
    const bool on = j < C2;
    const bool c0 = on && 2 * j < D, c1 = on && 2 * j + 1 < D;  // columns past D are zero
    // elements 2j, 2j+1 of a row: chunk cc of four, K step cc>>4, byte 4(cc&3) + 2(j&1) of column group
    // (cc>>2)&3
    const int cc = j >> 1;
    const int o0 = (cc >> 4) * 3072 + 256 * ((cc >> 2) & 3) + 4 * (cc & 3) + 2 * (j & 1);
    const int p = 8 * ((lane >> 5) & 1) + 4 * ((lane >> 4) & 1) + 2 * ((lane >> 3) & 1) + ((lane >> 2) & 1);
    float g0 = 0.0f, g1 = 0.0f;
    const float* nsrc = RN ? a.xn : a.nf;
    const float2 gm = RN ? *(const float2*)(a.gamma + 2 * jc) : make_float2(1.0f, 1.0f);
    // n of a row from its loaded value (RN: the source value and the row's 1/rms)
    auto nrm = [&](float2 v, float r) { return RN ? make_float2((v.x * r) * gm.x, (v.y * r) * gm.y) : v; };
    // 1/rms of the round's row k: lane k of a vector load (each lane loads row lane & 15), read out with
    // readlane (scalar loads would share the LDS traffic's completion counter)
    auto lane_k = [](float v, int k) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), k)); };
    // n (RN: its source and 1/rms) and lambda of the round, loaded while the previous round is packed
    // and stored
    float2 nv[16], gv[16];
    float rn = RN ? a.rinv[seq0 + (lane & 15)] : 1.0f;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        nv[k] = *(const float2*)(nsrc + (seq0 + k) * Dp + 2 * jc);
        gv[k] = *(const float2*)(a.lam + (seq0 + k) * Dp + 2 * jc);
    }
    for (int t0 = 0; t0 < T; t0 += 16) {
        float mn[16], mg[16];
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const float2 nk = nrm(nv[k], lane_k(rn, k));
            const float n0 = c0 ? nk.x : 0.0f, n1 = c1 ? nk.y : 0.0f;
            if (c0) {
                const float p1 = gv[k].x * g0;
                const float p2 = (1.0f - gv[k].x) * n0;
                g0 = p1 + p2;
            }
            if (c1) {
                const float p1 = gv[k].y * g1;
                const float p2 = (1.0f - gv[k].y) * n1;
                g1 = p1 + p2;
            }
            nv[k] = make_float2(n0, n1);
            gv[k] = make_float2(g0, g1);
            mn[k] = fmaxf(fabsf(n0), fabsf(n1));
            mg[k] = fmaxf(fabsf(g0), fabsf(g1));
            if (t0 + k == last && a.g_out && on) *(float2*)(a.g_out + (long long)b * Dp + 2 * j) = gv[k];
        }
        const float wn = wave_max16(mn, lane);
        const float wg = wave_max16(mg, lane);
        if ((lane & 3) == 0) {
            red[w * 16 + p] = wn;
            red[(nw + w) * 16 + p] = wg;
        }
        __syncthreads();
        if (j < 16) {
            float nr = red[j], gr = red[nw * 16 + j];
            for (int v = 1; v < nw; v++) {
                nr = fmaxf(nr, red[v * 16 + j]);
                gr = fmaxf(gr, red[(nw + v) * 16 + j]);
            }
            nring[(t0 + j) & 63] = nr;
            part[j] = fmaxf(nr, gr);
        }
        __syncthreads();
        if (j < 16) {
            const int t = t0 + j;
            const float mx = fmaxf(part[j], t >= dil ? nring[(t - dil) & 63] : 0.0f);
            float sc, inv;
            limb_scale(mx, sc, inv);
            a.xs[seq0 + t] = sc;
            invs[j] = inv;
        }
        __syncthreads();
        // the left neighbours (recently loaded rows: from cache), staged second
        float2 lv[16];
        const float rl = RN ? a.rinv[seq0 + max(t0 + (lane & 15) - dil, 0)] : 1.0f;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int t = t0 + k;
            const long long ml = seq0 + max(t - dil, 0);
            const float2 v = nrm(*(const float2*)(nsrc + ml * Dp + 2 * jc), lane_k(rl, k));
            const bool hl = t >= dil;
            lv[k] = make_float2((hl && c0) ? v.x : 0.0f, (hl && c1) ? v.y : 0.0f);
        }
        // the next round's n and lambda (this round's again after the last: in bounds, unused)
        const int tn = t0 + 16 < T ? t0 + 16 : t0;
        float2 nvn[16], gvn[16];
        const float rnn = RN ? a.rinv[seq0 + tn + (lane & 15)] : 1.0f;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            nvn[k] = *(const float2*)(nsrc + (seq0 + tn + k) * Dp + 2 * jc);
            gvn[k] = *(const float2*)(a.lam + (seq0 + tn + k) * Dp + 2 * jc);
        }
        float inv[16];
#pragma unroll
        for (int k = 0; k < 16; k++) inv[k] = invs[k];
        int8_t* dst = a.xl + (seq0 + t0) / 16 * (3LL * seg_bytes);  // this tile's rule-input fragments
        auto segment = [&](const float2 (&x)[16], int sg) {
            if (on) {
                // o0 + 16k stays inside o0's 256-byte column group (o0 & 255 <= 14), so every digit's LDS
                // address is sb plus a constant
                int8_t* sb = stage + stage_off(o0);
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    uint32_t w0, w1, w2;
                    split2_pack(x[k], inv[k], w0, w1, w2);
                    *(uint16_t*)(sb + 16 * k) = (uint16_t)w0;
                    *(uint16_t*)(sb + 16 * k + 1088) = (uint16_t)w1;
                    *(uint16_t*)(sb + 16 * k + 2176) = (uint16_t)w2;
                }
            }
            __syncthreads();
            for (int o = j * 16; o < seg_bytes; o += blockDim.x * 16)
                __builtin_nontemporal_store(*(const v4i*)(stage + stage_off(o)), (v4i*)(dst + sg * seg_bytes + o));
            __syncthreads();
        };
        segment(nv, 0);
        segment(lv, 1);
        segment(gv, 2);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            nv[k] = nvn[k];
            gv[k] = gvn[k];
        }
        rn = rnn;
    }
}


__global__ __launch_bounds__(1024) void latch_step_kernel(LatchStepArgs a) {
    __shared__ float red[16];
    const int s_ = blockIdx.x;
    const int d = threadIdx.x;
    const int lane = d & 63, w = d >> 6, nw = blockDim.x >> 6;
    const int D = a.D, Dp = a.Dp;
    const int pos = a.pos[s_];
    float n = 0.0f, left = 0.0f, g = 0.0f;
    if (d < D) {
        n = a.nf[(long long)s_ * Dp + d];
        float lam = a.lam[(long long)s_ * Dp + d];
        g = a.g[(long long)s_ * Dp + d];
        float p1 = lam * g;
        float p2 = (1.0f - lam) * n;
        g = p1 + p2;
        a.g[(long long)s_ * Dp + d] = g;
        float* ring = a.norm_ring + (long long)s_ * a.ring * Dp;
        ring[(long long)(pos % a.ring) * Dp + d] = n;
        if (pos >= a.dil) left = ring[(long long)((pos - a.dil) % a.ring) * Dp + d];
    }
    float mx = fmaxf(fabsf(n), fmaxf(fabsf(left), fabsf(g)));
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < nw; i++) mx = fmaxf(mx, red[i]);
    float sc, inv;
    limb_scale(mx, sc, inv);
    store_x_limbs(a.xl, s_, d, Dp, 3 * Dp / 64, n, left, g, inv);
    if (d == 0) a.xs[s_] = sc;
}

// ------------------------------------------------------------------------------------------------
// Attention (quant.Model.attendPosition, internal/quant/attention.go:69-104)
// ------------------------------------------------------------------------------------------------

// nn.WindowStart (internal/nn/attention.go:54-60)
__device__ __forceinline__ int window_start(int i, int window) {
    return (window > 0 && i - window + 1 > 0) ? i - window + 1 : 0;
}

// AddScaledF32 on AVX2 (vec_amd64.s:65-123): element i is fused when it lies in a 16- or 8-chunk,
// the last DH % 8 elements take an unfused multiply and add.
template <int DH>
__device__ __forceinline__ float axpy_ref(int i, float alpha, float x, float y) {
    constexpr int fused = (DH / 8) * 8;
    if (i < fused) return fmaf(alpha, x, y);
    float p = x * alpha;
    return p + y;
}

constexpr int ATT_QT = 64;  // queries per workgroup (one per lane)

// Copies `rows` rows of DH floats (global row stride ld) into LDS rows of stride DS, 16 bytes per lane
// per step when the width allows it, with several loads in flight.
template <int DH, int DS>
__device__ __forceinline__ void stage_rows(float* kv, const float* src, int ld, int rows, int lane) {
    if constexpr (DH % 4 == 0) {
        constexpr int C4 = DH / 4;
        const int n4 = rows * C4;
#pragma unroll 4
        for (int e = lane; e < n4; e += 64) {
            const int r = e / C4, c = e % C4;
            *(float4*)(kv + r * DS + 4 * c) = *(const float4*)(src + (long long)r * ld + 4 * c);
        }
    } else {
        for (int e = lane; e < rows * DH; e += 64) {
            const int r = e / DH, i = e % DH;
            kv[r * DS + i] = src[(long long)r * ld + i];
        }
    }
}

// LDS row stride of the staged keys/values. Lanes read consecutive rows (consecutive queries look at
// consecutive keys). Widths that are a multiple of 4 take 16-byte rows padded by 4 floats, read with
// 128-bit loads (consecutive rows land 4 banks apart); other widths take an odd stride and scalar reads.
template <int DH>
constexpr bool att_vec() { return DH % 4 == 0; }
template <int DH>
constexpr int att_stride() { return att_vec<DH>() ? DH + 4 : DH + 1; }

// DotF32 (dotProductASM_F32 order, see dot_f32_ref) of a register vector with an LDS row, the row
// read 16 bytes at a time.
template <int DH>
__device__ __forceinline__ float dot_ref_lds4(const float (&q)[DH], const float* row) {
    const float4* r4 = (const float4*)row;
    float a0[8], a1[8];
#pragma unroll
    for (int j = 0; j < 8; j++) { a0[j] = 0.0f; a1[j] = 0.0f; }
    int i = 0;
#pragma unroll
    for (; i + 16 <= DH; i += 16) {
        float4 k0 = r4[i / 4], k1 = r4[i / 4 + 1], k2 = r4[i / 4 + 2], k3 = r4[i / 4 + 3];
        a0[0] = fmaf(q[i + 0], k0.x, a0[0]); a0[1] = fmaf(q[i + 1], k0.y, a0[1]);
        a0[2] = fmaf(q[i + 2], k0.z, a0[2]); a0[3] = fmaf(q[i + 3], k0.w, a0[3]);
        a0[4] = fmaf(q[i + 4], k1.x, a0[4]); a0[5] = fmaf(q[i + 5], k1.y, a0[5]);
        a0[6] = fmaf(q[i + 6], k1.z, a0[6]); a0[7] = fmaf(q[i + 7], k1.w, a0[7]);
        a1[0] = fmaf(q[i + 8], k2.x, a1[0]); a1[1] = fmaf(q[i + 9], k2.y, a1[1]);
        a1[2] = fmaf(q[i + 10], k2.z, a1[2]); a1[3] = fmaf(q[i + 11], k2.w, a1[3]);
        a1[4] = fmaf(q[i + 12], k3.x, a1[4]); a1[5] = fmaf(q[i + 13], k3.y, a1[5]);
        a1[6] = fmaf(q[i + 14], k3.z, a1[6]); a1[7] = fmaf(q[i + 15], k3.w, a1[7]);
    }
    if (i + 8 <= DH) {
        float4 k0 = r4[i / 4], k1 = r4[i / 4 + 1];
        a0[0] = fmaf(q[i + 0], k0.x, a0[0]); a0[1] = fmaf(q[i + 1], k0.y, a0[1]);
        a0[2] = fmaf(q[i + 2], k0.z, a0[2]); a0[3] = fmaf(q[i + 3], k0.w, a0[3]);
        a0[4] = fmaf(q[i + 4], k1.x, a0[4]); a0[5] = fmaf(q[i + 5], k1.y, a0[5]);
        a0[6] = fmaf(q[i + 6], k1.z, a0[6]); a0[7] = fmaf(q[i + 7], k1.w, a0[7]);
        i += 8;
    }
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = a0[j] + a1[j];
    float s = hreduce8(v);
#pragma unroll
    for (; i < DH; i++) {
        float p = q[i] * row[i];
        s = s + p;
    }
    return s;
}

// One workgroup per (sequence, 64-query tile, head). Keys of the tile's whole window are staged in LDS,
// each lane scores its query against them (DotF32 order), runs the reference softmax, then the values
// replace the keys in LDS for the P.V accumulation.
// dot_ref_lds4 with the row in registers (DH a multiple of 4): the same products and additions in the
// same order.
template <int DH>
__device__ __forceinline__ float dot_ref_reg4(const float (&q)[DH], const float4 (&r4)[DH / 4]) {
    float a0[8], a1[8];
#pragma unroll
    for (int j = 0; j < 8; j++) { a0[j] = 0.0f; a1[j] = 0.0f; }
    int i = 0;
#pragma unroll
    for (; i + 16 <= DH; i += 16) {
        const float4 k0 = r4[i / 4], k1 = r4[i / 4 + 1], k2 = r4[i / 4 + 2], k3 = r4[i / 4 + 3];
        a0[0] = fmaf(q[i + 0], k0.x, a0[0]); a0[1] = fmaf(q[i + 1], k0.y, a0[1]);
        a0[2] = fmaf(q[i + 2], k0.z, a0[2]); a0[3] = fmaf(q[i + 3], k0.w, a0[3]);
        a0[4] = fmaf(q[i + 4], k1.x, a0[4]); a0[5] = fmaf(q[i + 5], k1.y, a0[5]);
        a0[6] = fmaf(q[i + 6], k1.z, a0[6]); a0[7] = fmaf(q[i + 7], k1.w, a0[7]);
        a1[0] = fmaf(q[i + 8], k2.x, a1[0]); a1[1] = fmaf(q[i + 9], k2.y, a1[1]);
        a1[2] = fmaf(q[i + 10], k2.z, a1[2]); a1[3] = fmaf(q[i + 11], k2.w, a1[3]);
        a1[4] = fmaf(q[i + 12], k3.x, a1[4]); a1[5] = fmaf(q[i + 13], k3.y, a1[5]);
        a1[6] = fmaf(q[i + 14], k3.z, a1[6]); a1[7] = fmaf(q[i + 15], k3.w, a1[7]);
    }
    if (i + 8 <= DH) {
        const float4 k0 = r4[i / 4], k1 = r4[i / 4 + 1];
        a0[0] = fmaf(q[i + 0], k0.x, a0[0]); a0[1] = fmaf(q[i + 1], k0.y, a0[1]);
        a0[2] = fmaf(q[i + 2], k0.z, a0[2]); a0[3] = fmaf(q[i + 3], k0.w, a0[3]);
        a0[4] = fmaf(q[i + 4], k1.x, a0[4]); a0[5] = fmaf(q[i + 5], k1.y, a0[5]);
        a0[6] = fmaf(q[i + 6], k1.z, a0[6]); a0[7] = fmaf(q[i + 7], k1.w, a0[7]);
        i += 8;
    }
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = a0[j] + a1[j];
    float s = hreduce8(v);
    if (i < DH) {  // DH % 8 == 4: the last four, unfused
        const float4 k = r4[i / 4];
        const float t[4] = {k.x, k.y, k.z, k.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float p = q[i + e] * t[e];
            s = s + p;
        }
    }
    return s;
}

template <int DH>
__global__ __launch_bounds__(64) void attention_kernel(AttnArgs a) {
    constexpr int DS = att_stride<DH>();
    extern __shared__ __align__(16) float smem[];
    const int nqt = (a.T + ATT_QT - 1) / ATT_QT;
    const int b = blockIdx.x / nqt, qt = blockIdx.x % nqt;
    const int h = blockIdx.y;
    const int lane = threadIdx.x;
    const int T = a.T, D = a.D, cap = a.cap;
    const int t0 = qt * ATT_QT;
    const int t1 = min(t0 + ATT_QT, T);
    const int r0 = max(window_start(t0, a.window), max(t0 - cap + 1, 0));
    const int rows = t1 - r0;
    float* kv = smem;                            // [rows][DS]
    float* sc = smem + (ATT_QT + cap - 1) * DS;  // [cap][64]
    const long long base = (long long)b * T;
    const int ld = 3 * D;

    stage_rows<DH, DS>(kv, a.qkv + (base + r0) * ld + D + h * DH, ld, rows, lane);
    __syncthreads();

    const int t = t0 + lane;
    const bool active = t < t1;
    float q[DH];
    int lo = 0, span = 0;
    float inv = 0.0f;
    if (active) {
        const float* qp = a.qkv + (base + t) * ld + h * DH;
        if constexpr (att_vec<DH>()) {
#pragma unroll
            for (int i = 0; i < DH; i += 4) {
                float4 v = *(const float4*)(qp + i);
                q[i] = v.x; q[i + 1] = v.y; q[i + 2] = v.z; q[i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < DH; i++) q[i] = qp[i];
        }
        lo = max(window_start(t, a.window), t - cap + 1);
        span = t - lo + 1;
        const float scale = (float)(1.0 / sqrt((double)DH));
        float mx = -3.40282347e38f;
        for (int jj = 0; jj < span; jj++) {
            const float* k = kv + (lo + jj - r0) * DS;
            float s;
            if constexpr (att_vec<DH>()) s = dot_ref_lds4<DH>(q, k) * scale;
            else s = dot_f32_ref<DH>(q, k) * scale;
            sc[jj * 64 + lane] = s;
            if (s > mx) mx = s;
        }
        // nn.SoftmaxInPlaceF32 (internal/nn/head.go:151-172)
        float sum = 0.0f;
        for (int jj = 0; jj < span; jj++) {
            float e = fast_exp_ref(sc[jj * 64 + lane] - mx);
            sc[jj * 64 + lane] = e;
            sum += e;
        }
        inv = 1.0f / sum;
    }
    __syncthreads();
    stage_rows<DH, DS>(kv, a.qkv + (base + r0) * ld + 2 * D + h * DH, ld, rows, lane);
    __syncthreads();
    if (!active) return;
    float o[DH];
#pragma unroll
    for (int i = 0; i < DH; i++) o[i] = 0.0f;
    for (int jj = 0; jj < span; jj++) {
        float p = sc[jj * 64 + lane] * inv;
        const float* v = kv + (lo + jj - r0) * DS;
        if constexpr (att_vec<DH>()) {
            const float4* v4 = (const float4*)v;
#pragma unroll
            for (int i = 0; i < DH; i += 4) {
                float4 vv = v4[i / 4];
                o[i] = axpy_ref<DH>(i, p, vv.x, o[i]);
                o[i + 1] = axpy_ref<DH>(i + 1, p, vv.y, o[i + 1]);
                o[i + 2] = axpy_ref<DH>(i + 2, p, vv.z, o[i + 2]);
                o[i + 3] = axpy_ref<DH>(i + 3, p, vv.w, o[i + 3]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < DH; i++) o[i] = axpy_ref<DH>(i, p, v[i], o[i]);
        }
    }
    float* dst = a.att + (base + t) * a.Dp + h * DH;
    if constexpr (att_vec<DH>()) {
#pragma unroll
        for (int i = 0; i < DH; i += 4) *(float4*)(dst + i) = make_float4(o[i], o[i + 1], o[i + 2], o[i + 3]);
    } else {
#pragma unroll
        for (int i = 0; i < DH; i++) dst[i] = o[i];
    }
}

// ------------------------------------------------------------------------------------------------
// Windowed attention on the matrix cores (v_mfma_f32_16x16x4f32). One wave per 16-query tile of one
// (sequence, head); G consecutive tiles per workgroup share keys and values staged in LDS.
//
// Scores are computed transposed, S^T = K Q^T, so that afterwards lane L holds the scores of query
// t0 + (L & 15) against keys jb + 4(L >> 4) + r of each 16-key block: exactly the A operand that P.V
// needs (the K dimension of each P.V step is the four keys {jb + 4g + r}), so P never leaves registers.
// The head dimension is consumed in the order 16g + 4(L >> 4) + s, which makes every Q and K operand one
// float4 load; dimensions past dh are zero. Masking, the scale (float32(1/sqrt(dh))), the max-shifted
// exponentials (the reference's FastExp), 1/sum and p = e*inv follow nn.SoftmaxInPlaceF32; only the
// summation order of the dot products and of the softmax sum differ from the sequential reference.
// ------------------------------------------------------------------------------------------------
typedef float v4f __attribute__((ext_vector_type(4)));

// Column swizzle of the transposed values in LDS: row r (a head dimension) stores key k at column
// k ^ vswz(r). The swizzle flips bits 2-3 of the key, so groups of four keys stay contiguous and
// 16-byte aligned (every P.V operand is still one 16-byte read, conflict-free) and a key never leaves its
// block of 16. The transposing writes, where 16 lanes write one key's 16 dimension-quads, then spread
// over all banks instead of two.
__device__ __forceinline__ int vswz(int r) { return 4 * ((r >> 3) & 3); }

// S^T for key blocks SKIP..NKB-1 of one wave; the SKIP leading blocks hold only keys before the
// sequence start (masked in the softmax), so their scores stay zero and no MFMA is spent on them.
// Each block's sum runs over (g, e) in order; the blocks' chains are independent and interleaved, so
// consecutive MFMAs never wait on each other's results.
template <int ND, int NKB, int KS, int SKIP>
__device__ __forceinline__ void attn_scores(v4f (&s)[NKB], const float* att_lds, int w, int qi, int kg,
                                            const v4f (&qv)[ND]) {
#pragma unroll
    for (int kb = 0; kb < NKB; kb++) s[kb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < ND; g++) {
        v4f kv[NKB];
#pragma unroll
        for (int kb = SKIP; kb < NKB; kb++) kv[kb] = *(const v4f*)(att_lds + (16 * (w + kb) + qi) * KS + 16 * g + 4 * kg);
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int kb = SKIP; kb < NKB; kb++) s[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kb][e], qv[g][e], s[kb], 0, 0, 0);
    }
}

// The softmax exponential of the matrix-core attention kernels: the hardware 2^x of x*log2(e), within a
// few ulp of e^x over the scores' range (x <= 0), where the reference-order kernels evaluate the
// reference's FastExp polynomial bit for bit. These kernels already differ from the reference order in
// their fp32 summation order, and this takes ~13 of the ~15 VALU instructions per score.
__device__ __forceinline__ float attn_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// out = P V over key blocks SKIP..NKB-1 (the skipped blocks' probabilities are zero: leaving them out
// adds nothing, bit for bit).
// Each output group's sum runs over (kb, r) in order; the groups' chains are interleaved.
template <int ND, int NKB, int VS, int SKIP>
__device__ __forceinline__ void attn_pv(v4f (&o)[ND], const v4f (&s)[NKB], float inv, const float* att_lds, int w,
                                        int qi, int kg) {
#pragma unroll
    for (int g = 0; g < ND; g++) o[g] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = SKIP; kb < NKB; kb++) {
        v4f vv[ND];
#pragma unroll
        for (int g = 0; g < ND; g++)
            vv[g] = *(const v4f*)(att_lds + (16 * g + qi) * VS + ((16 * (w + kb) + 4 * kg) ^ vswz(16 * g + qi)));
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = s[kb][r] * inv;
#pragma unroll
            for (int g = 0; g < ND; g++) o[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(p, vv[g][r], o[g], 0, 0, 0);
        }
    }
}

// Windowed causal attention on the fp32 matrix cores. A workgroup is G waves; wave w takes the 16
// queries of tile G*grp + w for head blockIdx.y. The 16*(NKB+G-1) keys the G tiles attend are staged in
// LDS once: keys first (row-major), then, over the same buffer, values transposed, so that every matrix
// operand is one 16-byte LDS read. Per wave: S^T = K Q^T over NKB blocks of 16 keys (dims 16g + 4kg + e),
// the reference's softmax in registers, then out = P V. More tiles per workgroup read each key and value
// from memory fewer times (G = 8 covers a 128-token sequence with every key loaded once).
template <int ND, int NKB, int G>
__global__ __launch_bounds__(64 * G) void attention_mfma_kernel(AttnArgs a, int dh) {
    constexpr int NT = 64 * G;            // threads
    constexpr int KEYS = 16 * (NKB + G - 1);  // keys of the workgroup's G query tiles
    constexpr int DP = 16 * ND;           // head width padded to the MFMA's 16
    constexpr int KS = DP + 4;            // LDS row stride of K (floats)
    constexpr int VS = KEYS + 4;          // LDS row stride of V^T (floats)
    constexpr int CH = DP / 4;            // 16-byte chunks per key row
    constexpr int NCH = KEYS * CH;
    constexpr int PER = (NCH + NT - 1) / NT;
    extern __shared__ __align__(16) float att_lds[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, tid = threadIdx.x;
    const int T = a.T, D = a.D, cap = a.cap, ld = 3 * D;
    const int qtiles = (T + 15) >> 4;
    const int groups = (qtiles + G - 1) / G;
    const int b = blockIdx.x / groups;
    const int grp = blockIdx.x % groups;
    const int tile = grp * G + w;
    const int h = blockIdx.y;
    const int t0 = tile * 16;
    const int qi = lane & 15, kg = lane >> 4;
    const float* seq = a.qkv + (long long)b * T * ld;
    const float* qb = seq + h * dh;
    const float* kb_ = seq + D + h * dh;
    const float* vb = seq + 2 * D + h * dh;
    const float scale = (float)(1.0 / sqrt((double)dh));
    const int kbase = grp * 16 * G + 16 - 16 * NKB;  // key of LDS row 0

    // Every global load is unconditional, from an address clamped into the sequence and the head, and
    // masked afterwards (a guarded load becomes a branch that waits for it on the spot). Keys outside
    // [0, T) and dims past dh are zero.
    const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f kreg[PER], vreg[PER];
#pragma unroll
    for (int p = 0; p < PER; p++) {
        const int e = min(tid + NT * p, NCH - 1);
        const int key = e / CH, d = 4 * (e - key * CH);
        const int j = kbase + key;
        const long long off = (long long)min(max(j, 0), T - 1) * ld + min(d, dh - 4);
        const float mask = (j >= 0 && j < T && d < dh) ? 1.0f : 0.0f;
        kreg[p] = *(const v4f*)(kb_ + off) * mask;
        vreg[p] = *(const v4f*)(vb + off) * mask;
    }
    // Q^T operand: query t0 + qi, dims 16g + 4kg .. +3
    v4f qv[ND];
    {
        const int t = min(t0 + qi, T - 1);
#pragma unroll
        for (int g = 0; g < ND; g++) {
            const int d = 16 * g + 4 * kg;
            qv[g] = *(const v4f*)(qb + (long long)t * ld + min(d, dh - 4)) * (d < dh ? 1.0f : 0.0f);
        }
    }
#pragma unroll
    for (int p = 0; p < PER; p++) {
        const int e = tid + NT * p;
        if (e < NCH) {
            const int key = e / CH, c = e - key * CH;
            *(v4f*)(att_lds + key * KS + 4 * c) = kreg[p];
        }
    }
    __syncthreads();
    // s[kb][r] = q.k for query t0 + qi and key kbase + 16(w + kb) + 4kg + r. The leading blocks whose keys
    // all lie before the sequence start (the first tiles of a sequence) are skipped; the count is
    // uniform per wave and selects one of a few unrolled variants (more than 4 such blocks: 4 skipped).
    int skip = 0;
#pragma unroll
    for (int kb = 0; kb < NKB - 1; kb++)
        if (kbase + 16 * (w + kb) + 15 < 0) skip = kb + 1;
    skip = min(skip, 4);
    v4f s[NKB];
    switch (skip) {
        case 0: attn_scores<ND, NKB, KS, 0>(s, att_lds, w, qi, kg, qv); break;
        case 1: attn_scores<ND, NKB, KS, 1>(s, att_lds, w, qi, kg, qv); break;
        case 2: attn_scores<ND, NKB, KS, 2>(s, att_lds, w, qi, kg, qv); break;
        case 3: attn_scores<ND, NKB, KS, 3>(s, att_lds, w, qi, kg, qv); break;
        default: attn_scores<ND, NKB, KS, 4>(s, att_lds, w, qi, kg, qv); break;
    }
    __syncthreads();  // every wave's keys are read: the buffer takes the values
#pragma unroll
    for (int p = 0; p < PER; p++) {
        const int e = tid + NT * p;
        if (e < NCH) {
            const int key = e / CH, c = e - key * CH;
#pragma unroll
            for (int i = 0; i < 4; i++) att_lds[(4 * c + i) * VS + (key ^ vswz(4 * c + i))] = vreg[p][i];
        }
    }
    const int t = t0 + qi;
    const int jstart = kbase + 16 * w;
    const int lo = max(window_start(t, a.window), t - cap + 1);
    float mx = -3.40282347e38f;
#pragma unroll
    for (int kb = 0; kb < NKB; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int j = jstart + 16 * kb + 4 * kg + r;
            const float v = s[kb][r] * scale;
            s[kb][r] = v;
            if (j >= lo && j <= t && v > mx) mx = v;
        }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float sum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < NKB; kb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int j = jstart + 16 * kb + 4 * kg + r;
            const float e = (j >= lo && j <= t) ? attn_exp(s[kb][r] - mx) : 0.0f;
            s[kb][r] = e;
            sum += e;
        }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    const float inv = 1.0f / sum;
    __syncthreads();
    // out = P V: A = P (query qi, key jb + 4kg + r), B = V (key jb + 4kg + r, dim 16g + qi)
    v4f o[ND];
    switch (skip) {
        case 0: attn_pv<ND, NKB, VS, 0>(o, s, inv, att_lds, w, qi, kg); break;
        case 1: attn_pv<ND, NKB, VS, 1>(o, s, inv, att_lds, w, qi, kg); break;
        case 2: attn_pv<ND, NKB, VS, 2>(o, s, inv, att_lds, w, qi, kg); break;
        case 3: attn_pv<ND, NKB, VS, 3>(o, s, inv, att_lds, w, qi, kg); break;
        default: attn_pv<ND, NKB, VS, 4>(o, s, inv, att_lds, w, qi, kg); break;
    }
    if (tile >= qtiles) return;
    // o[g][r] = out[query t0 + 4kg + r][dim 16g + qi]
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int tq = t0 + 4 * kg + r;
        if (tq >= T) continue;
        float* dst = a.att + ((long long)b * T + tq) * a.Dp + h * dh;
#pragma unroll
        for (int g = 0; g < ND; g++) {
            const int d = 16 * g + qi;
            if (d < dh) dst[d] = o[g][r];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Attention projection fused with windowed attention (teacher-forced forward, 128-token sequences)
// ------------------------------------------------------------------------------------------------
// A workgroup of 8 waves holds head h's slab of the QKV weights in LDS (per K step: the head's q, k and v
// fragments, 3*ND KiB) and streams a run of sequences through it. Per sequence, wave w takes tokens
// 16w..16w+15: its limb fragments (all K steps, fetched while the previous sequence's attention runs)
// meet the slab on v_mfma_i32_16x16x64_i8 once for k, once for v, once for q. The epilogue is the QKV
// GEMM's (EPI_F32: three digit sums combined, times row scale and weight scale), and its layout (lane L:
// token L & 15, channels 16i + 4(L >> 4) + r) is already the Q^T operand of attention_mfma_kernel, whose
// key layout the k rows are written in (LDS row = key - kbase) and whose value transpose the v registers
// are written in after the scores. Scores, softmax and P.V then run exactly as in attention_mfma_kernel
// with one group of G = 8 tiles, so the output is the same bit for bit, without the fp32 q/k/v round trip
// through memory.
// Waves per SIMD the compiler allocates registers for: two (up to 256 registers) in general; four (at most
// 128, so that two 8-wave workgroups share a CU) for narrow heads with short windows over small models,
// whose LDS (about 47 KiB at D = 128) leaves room for the second workgroup.
constexpr int qkv_attn_waves(int ND, int NKB, int KC) { return ND == 2 && NKB <= 5 && KC == 2 ? 4 : 2; }

template <int ND, int NKB, int KC>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(qkv_attn_waves(ND, NKB, KC),
                                                                     qkv_attn_waves(ND, NKB, KC)))) void qkv_attention_kernel(
    QkvAttnArgs a, int run_seqs, int n_runs) {
    constexpr int G = 8;
    constexpr int DP = 16 * ND;               // head width
    constexpr int KEYS = 16 * (NKB + G - 1);  // key rows of attention_mfma_kernel: keys kbase .. kbase + KEYS - 1
    constexpr int ZROWS = 16 * (NKB - 1);     // its leading rows: keys before the sequence start, never read
                                              // (every key block holding them is skipped)
    constexpr int KS = DP + 4;                // K row stride (floats), as attention_mfma_kernel
    constexpr int VS = KEYS - ZROWS + 4;      // V^T row stride: the allocated keys, +4 as there
    constexpr int NF = 3 * ND;                // weight fragments per K step
    constexpr int SLAB = KC * NF * 1024;
    constexpr int KBYTES = (KEYS - ZROWS) * KS * 4;
    extern __shared__ __align__(16) int8_t qa_smem[];
    int8_t* slab = qa_smem;
    // K rows and V^T columns of keys 0..127 only, addressed as attention_mfma_kernel addresses its buffer
    // (key row / column key - kbase, never below ZROWS), so that its score and P.V routines run unchanged
    float* klds = (float*)(qa_smem + SLAB) - ZROWS * KS;
    float* vlds = (float*)(qa_smem + SLAB + KBYTES) - ZROWS;
    const int slot = blockIdx.x >> 3;
    const int h = slot % a.heads;
    const int run = (slot / a.heads) * 8 + (blockIdx.x & 7);  // all heads of a run on one XCD
    if (run >= n_runs) return;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qi = lane & 15, kg = lane >> 4;
    const int D = a.D, T = 16 * G;
    {
        // slab[ks][f][1 KiB], f = part*ND + i: fragment (part*D + h*DP)/16 + i of K step ks (part 0 q, 1 k, 2 v)
        const long long np16 = a.Np3 >> 4;
        for (int c = tid; c < KC * NF * 64; c += 512) {
            const int ks = c / (NF * 64), f = (c >> 6) % NF, o = (c & 63) << 4;
            const int part = f / ND, i = f - part * ND;
            const long long frag = ((part * D + h * DP) >> 4) + i;
            *(v4i*)(slab + ((long long)c << 4)) = *(const v4i*)(a.W + (ks * np16 + frag) * 1024 + o);
        }
    }
    const float scale = (float)(1.0 / sqrt((double)DP));
    const int kbase = 16 - 16 * NKB;
    int skip = 0;  // leading key blocks of this wave wholly before the sequence start (as attention_mfma_kernel)
#pragma unroll
    for (int kb = 0; kb < NKB - 1; kb++)
        if (kbase + 16 * (w + kb) + 15 < 0) skip = kb + 1;
    skip = min(skip, 4);
    const int t = 16 * w + qi;
    const int lo = max(window_start(t, a.window), t - a.cap + 1);
    const int jstart = kbase + 16 * w;
    const int key = t - kbase;  // this lane's token as a key row
    const int s_begin = run * run_seqs, s_end = min(s_begin + run_seqs, a.B);
    v4i af[KC][3];
    auto load_a = [&](int b) {
        const int8_t* ap = a.A + ((long long)b * (T / 16) + w) * (KC * 3 * 1024) + lane * 16;
#pragma unroll
        for (int ks = 0; ks < KC; ks++)
#pragma unroll
            for (int l = 0; l < 3; l++) af[ks][l] = *(const v4i*)(ap + (ks * 3 + l) * 1024);
    };
    load_a(s_begin);
    __syncthreads();
    const int8_t* wl = slab + lane * 16;
    for (int b = s_begin; b < s_end; b++) {
        const long long m0 = (long long)b * T + 16 * w;
        const float sw = a.As[m0 + qi] * a.wscale;
        v4f qv[ND];
        // parts in the order k, v (both to LDS), q (kept in registers)
#pragma unroll
        for (int pi = 0; pi < 3; pi++) {
            const int part = pi == 0 ? 1 : pi == 1 ? 2 : 0;
            v4i acc[3][ND];
#pragma unroll
            for (int ks = 0; ks < KC; ks++) {
                v4i wf[ND];
#pragma unroll
                for (int i = 0; i < ND; i++) wf[i] = *(const v4i*)(wl + ((ks * NF + part * ND + i) << 10));
#pragma unroll
                for (int i = 0; i < ND; i++)
#pragma unroll
                    for (int l = 0; l < 3; l++)
                        acc[l][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[i], af[ks][l],
                                                                          ks == 0 ? v4i{0, 0, 0, 0} : acc[l][i], 0, 0, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, ND, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 3 * ND, 0);
            }
#pragma unroll
            for (int i = 0; i < ND; i++) {
                v4f v;
#pragma unroll
                for (int r = 0; r < 4; r++)
                    v[r] = fmaf((float)acc[2][i][r], kInvLimb2, fmaf((float)acc[1][i][r], kInvLimb1, (float)acc[0][i][r])) * sw;
                if (pi == 0) {
                    *(v4f*)(klds + key * KS + 16 * i + 4 * kg) = v;
                } else if (pi == 1) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int d = 16 * i + 4 * kg + r;
                        vlds[d * VS + (key ^ vswz(d))] = v[r];
                    }
                } else {
                    qv[i] = v;
                }
            }
        }
        // the next sequence's fragments load during this one's attention
        if (b + 1 < s_end) load_a(b + 1);
        __syncthreads();  // every key row and value column is written
        v4f s[NKB];
        switch (skip) {
            case 0: attn_scores<ND, NKB, KS, 0>(s, klds, w, qi, kg, qv); break;
            case 1: attn_scores<ND, NKB, KS, 1>(s, klds, w, qi, kg, qv); break;
            case 2: attn_scores<ND, NKB, KS, 2>(s, klds, w, qi, kg, qv); break;
            case 3: attn_scores<ND, NKB, KS, 3>(s, klds, w, qi, kg, qv); break;
            default: attn_scores<ND, NKB, KS, 4>(s, klds, w, qi, kg, qv); break;
        }
        float mx = -3.40282347e38f;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int j = jstart + 16 * kb + 4 * kg + r;
                const float v = s[kb][r] * scale;
                s[kb][r] = v;
                if (j >= lo && j <= t && v > mx) mx = v;
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        float sum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int j = jstart + 16 * kb + 4 * kg + r;
                const float e = (j >= lo && j <= t) ? attn_exp(s[kb][r] - mx) : 0.0f;
                s[kb][r] = e;
                sum += e;
            }
        sum += __shfl_xor(sum, 16, 64);
        sum += __shfl_xor(sum, 32, 64);
        const float inv = 1.0f / sum;
        v4f o[ND];
        switch (skip) {
            case 0: attn_pv<ND, NKB, VS, 0>(o, s, inv, vlds, w, qi, kg); break;
            case 1: attn_pv<ND, NKB, VS, 1>(o, s, inv, vlds, w, qi, kg); break;
            case 2: attn_pv<ND, NKB, VS, 2>(o, s, inv, vlds, w, qi, kg); break;
            case 3: attn_pv<ND, NKB, VS, 3>(o, s, inv, vlds, w, qi, kg); break;
            default: attn_pv<ND, NKB, VS, 4>(o, s, inv, vlds, w, qi, kg); break;
        }
        // o[g][r] = out[query 16w + 4kg + r][dim 16g + qi]: in rows, or in the fp32-operand GEMM's fragment
        // order when that GEMM reads it (with the per-head maxima below)
        if (a.amax) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int g = 0; g < ND; g++) a.att[frag_off_f32(m0 + 4 * kg + r, h * DP + 16 * g + qi, a.Dp >> 6)] = o[g][r];
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float* dst = a.att + (m0 + 4 * kg + r) * a.Dp + h * DP;
#pragma unroll
                for (int g = 0; g < ND; g++) dst[16 * g + qi] = o[g][r];
            }
        }
        if (a.amax) {
            // the head's largest |value| of each query row, for the output projection's operand scale:
            // query 16w + 4kg + r is held by the 16 lanes qi of row kg (a DPP row), ND values each
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float v = fabsf(o[0][r]);
#pragma unroll
                for (int g = 1; g < ND; g++) v = fmaxf(v, fabsf(o[g][r]));
                v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1, 0, 3, 2]
                v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2, 3, 0, 1]
                v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
                v = fmaxf(v, dpp_move<0x140>(v));  // row_mirror
                if (qi == r) a.amax[(m0 + 4 * kg + r) * a.amax_ld + h] = v;
            }
        }
        __syncthreads();  // every wave's keys and values are read before the next sequence's are written
    }
}

// One wavefront per (session, head): lane j scores key j of the ring, lane i accumulates output i.
template <int DH>
__global__ __launch_bounds__(64) void attention_step_kernel(AttnStepArgs a) {
    __shared__ float es[256];
    __shared__ float qs[DH];
    __shared__ float inv_sh;
    const int s_ = blockIdx.x / a.heads, h = blockIdx.x % a.heads;
    const int lane = threadIdx.x;
    const int D = a.D, cap = a.cap;
    const int pos = a.pos[s_];
    const int lo = max(window_start(pos, a.window), pos - cap + 1);
    const int span = pos - lo + 1;
    const float* qkv = a.qkv + (long long)s_ * 3 * D;
    const float* kr = a.kring + ((long long)s_ * a.heads + h) * cap * DH;
    const float* vr = a.vring + ((long long)s_ * a.heads + h) * cap * DH;
    for (int i = lane; i < DH; i += 64) qs[i] = qkv[h * DH + i];
    __syncthreads();
    float q[DH];
#pragma unroll
    for (int i = 0; i < DH; i++) q[i] = qs[i];
    const float scale = (float)(1.0 / sqrt((double)DH));
    float mx = -3.40282347e38f;
    for (int jj = lane; jj < span; jj += 64) {
        int j = lo + jj;
        const float* k = (j == pos) ? qkv + D + h * DH : kr + (long long)(j % cap) * DH;
        float s = dot_f32_ref<DH>(q, k) * scale;
        es[jj] = s;
        mx = fmaxf(mx, s);
    }
    mx = wave_max(mx);
    for (int jj = lane; jj < span; jj += 64) es[jj] = fast_exp_ref(es[jj] - mx);
    __syncthreads();
    if (lane == 0) {
        float sum = 0.0f;
        for (int jj = 0; jj < span; jj++) sum += es[jj];
        inv_sh = 1.0f / sum;
    }
    __syncthreads();
    const float inv = inv_sh;
    for (int i = lane; i < DH; i += 64) {
        float o = 0.0f;
        for (int jj = 0; jj < span; jj++) {
            int j = lo + jj;
            float p = es[jj] * inv;
            float v = (j == pos) ? qkv[2 * D + h * DH + i] : vr[(long long)(j % cap) * DH + i];
            o = axpy_ref<DH>(i, p, v, o);
        }
        a.att[(long long)s_ * a.Dp + h * DH + i] = o;
    }
    // record this position's key and value (slot pos % cap; the evicted key is outside the window)
    float* kw = a.kring + (((long long)s_ * a.heads + h) * cap + pos % cap) * DH;
    float* vw = a.vring + (((long long)s_ * a.heads + h) * cap + pos % cap) * DH;
    for (int i = lane; i < DH; i += 64) {
        kw[i] = qkv[D + h * DH + i];
        vw[i] = qkv[2 * D + h * DH + i];
    }
}

// Makes this wave's LDS writes visible to its own later reads (LDS operations of one wave complete in
// order): a workgroup-wide barrier is not needed where every LDS region is private to one wave.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
}

// ------------------------------------------------------------------------------------------------
// Packed K/V rings. A ring row (one head's key or value at one position) is held as dh/4 groups of
// three 32-bit words, each group four 24-bit two's-complement mantissas m, with one power-of-two scale
// s = 2^e per row: the element is m * s, exactly. e = E - 23 for the row's largest magnitude
// amax = f * 2^E (f in [0.5, 1)), so the largest element keeps 23 significant bits and every element
// lies within 2^-24 * amax of its fp32 value, the precision the limb planes give every matrix operand
// relative to its row. Three bytes per element instead of four: decode attention, which streams the
// rings, reads 3/4 of the bytes. Decoding is exact (a 24-bit integer times a power of two), so every
// kernel that reads a packed ring sees the same fp32 values and the decode kernels stay bit-identical
// to each other.
// ------------------------------------------------------------------------------------------------
struct Pk3 {
    uint32_t x, y, z;
};

// The exponent e of a row whose largest magnitude is amax (amax * 2^-e < 2^23; e >= -120 keeps 2^e a
// normal float, rows below 2^-97 lose their low bits).
__device__ __forceinline__ int kv_exp(float amax) {
    int E;
    (void)frexpf(amax, &E);
    return max(E - 23, -120);
}

__device__ __forceinline__ uint32_t kv_mant(float v, int e) {
    const float r = fminf(fmaxf(rintf(ldexpf(v, -e)), -8388607.0f), 8388607.0f);
    return (uint32_t)(int)r & 0xffffffu;
}

__device__ __forceinline__ Pk3 kv_pack(float4 v, int e) {
    const uint32_t u0 = kv_mant(v.x, e), u1 = kv_mant(v.y, e), u2 = kv_mant(v.z, e), u3 = kv_mant(v.w, e);
    return Pk3{u0 | (u1 << 24), (u1 >> 8) | (u2 << 16), (u2 >> 16) | (u3 << 8)};
}

// Global loads and stores of one group, as three dword accesses the compiler joins into one.
__device__ __forceinline__ Pk3 ldg_pk3(const Pk3* p) {
    const __attribute__((address_space(1))) uint32_t* q = (const __attribute__((address_space(1))) uint32_t*)p;
    return Pk3{q[0], q[1], q[2]};
}
__device__ __forceinline__ Pk3 ldg_pk3_nt(const Pk3* p) {
    typedef uint32_t u3 __attribute__((ext_vector_type(3)));
    const u3 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u3*)p);
    return Pk3{v.x, v.y, v.z};
}

__device__ __forceinline__ void stg_pk3(Pk3* p, Pk3 v) {
    __attribute__((address_space(1))) uint32_t* q = (__attribute__((address_space(1))) uint32_t*)p;
    q[0] = v.x;
    q[1] = v.y;
    q[2] = v.z;
}

__device__ __forceinline__ float4 kv_unpack(Pk3 w, float s) {
    const int m0 = (int)(w.x << 8) >> 8;
    const int m1 = (int)(__builtin_amdgcn_alignbit(w.y, w.x, 24) << 8) >> 8;
    const int m2 = (int)(__builtin_amdgcn_alignbit(w.z, w.y, 16) << 8) >> 8;
    const int m3 = (int)w.z >> 8;
    return float4{(float)m0 * s, (float)m1 * s, (float)m2 * s, (float)m3 * s};
}

// LDS floats of one head in rk_head, a multiple of four (16-byte aligned regions side by side): the
// values [cap][DH + 4], the query [DH], with packed rings read from global memory (PK, not QL) the
// current position's key [DH], the scores [cap].
__host__ __device__ constexpr int rk_lds_floats(int cap, int dh, bool kcur = false) {
    return (cap * (dh + 4) + dh + (kcur ? dh : 0) + cap + 3) & ~3;
}

// One (session, head) of decode attention for caches of at most 64 positions, by one wave, with each
// lane's key row in registers: lane jj loads key lo + jj itself and scores it, so only the values (and
// the scores) go through LDS, about half the LDS of the staged kernel and twice the waves per CU.
// Bit-identical to it: the same reference-order dot product, softmax and P.V. Every global load (the
// query, this position's key and value, the key rows, the value rows) is issued before the first wait,
// so a wave makes one memory round trip. `sm` (rk_lds_floats) and `inv_sh` are private to the wave.
// Returns output element `lane` of the head (lanes < DH) and records this position's key and value in
// the ring. PK: the rings are packed (kpack/kscale, vpack/vscale); the ring rows are decoded as they
// are loaded, and the current position's key and value, which are not yet in the ring, come in fp32
// (through LDS without QL: lanes C4..2C4-1 hold the key, 2C4..3C4-1 the value, as their `mine`).
// ST (packed rings without QL, heads of at most 32): the rings are streamed, for sets whose rings are
// larger than the caches. Key rows are then read like the value rows, consecutive lanes on consecutive
// groups, with non-temporal loads, and reach their lanes through LDS: the loads no longer displace the
// decode step's weights and code from the caches. With a row per lane, each cache line of the keys is
// read by C4 loads and has to stay cached between them, which non-temporal loads do not allow.
template <int DH, bool QL = false, bool PK = false, bool ST = false>
__device__ __forceinline__ float rk_head(const AttnStepArgs& a, int s_, int h, int lane, float* sm, float& inv_sh) {
    constexpr int DS = DH + 4;
    constexpr int C4 = DH / 4;
    static_assert(3 * C4 <= 64, "one float4 of q, k or v per lane");
    const int cap = a.cap;
    constexpr bool CUR_LANES = PK && !QL;  // the current key and value from the lanes holding them
    float* vs = sm;                           // [cap][DS]
    float* qs = vs + cap * DS;                // [DH]
    float* kc = qs + DH;                      // [DH] (CUR_LANES)
    float* es = kc + (CUR_LANES ? DH : 0);    // [cap]
    const int D = a.D;
    const int pos = a.pos[s_];
    const int lo = max(window_start(pos, a.window), pos - cap + 1);
    const int span = pos - lo + 1;  // at most cap <= 64
    const float* qkv = a.qkv + (long long)s_ * 3 * D;
    const long long row0 = ((long long)s_ * a.heads + h) * cap;  // ring row of slot 0
    const float* kr = a.kring + row0 * DH;
    const float* vr = a.vring + row0 * DH;
    // q, k, v of this position: in LDS (QL) or global memory; the rings in global memory. Typed loads, so
    // that the compiler need not treat them as generic (flat) accesses, which it serialises.
    auto qkv4 = [&](const float* p) -> float4 {
        if constexpr (QL) {
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 v = *(const __attribute__((address_space(3))) f4*)p;
            return float4{v.x, v.y, v.z, v.w};
        } else {
            return ldg((const float4*)p);
        }
    };
    // group c of packed ring row `sl` (kpack or vpack) and that row's scale
    // (the head's ring base is uniform over the wave; only 32-bit offsets vary over the lanes)
    auto pk4 = [&](const uint32_t* ring, const float* scl, int sl, int c) -> float4 {
        const Pk3 w = ldg_pk3(((const Pk3*)ring + row0 * C4) + (sl * C4 + c));
        return kv_unpack(w, ldg((scl + row0) + sl));
    };
    constexpr bool KST = ST && CUR_LANES && C4 <= 8;
    // lanes 0..3*C4-1: one float4 each of this position's q, k and v (part lane / C4, chunk lane % C4)
    const int qpart = min(lane / C4, 2), qc = lane % C4;
    const float4 mine = qkv4(qkv + qpart * D + h * DH + 4 * qc);
    // ring slot of key lo + jj (jj < span <= cap): one wrap, no division per key
    const int lo_slot = lo % cap;
    auto slot = [&](int jj) { const int r = lo_slot + jj; return r >= cap ? r - cap : r; };
    // this lane's key row (key lo + lane; the current position's from qkv, not yet in the ring)
    float4 krow[C4];
    if constexpr (KST) {
        // key and value rows 0..span-2 with coalesced streaming loads (consecutive lanes on consecutive
        // groups), every load issued before the first store; the keys pass through the value region of LDS
        // to the lanes that score them, then the values take their place. The current position's key and
        // value come from the lanes holding them.
        const int nr = (span - 1) * C4;
        // the row scales, lane r holding row r's, handed to the lanes of each row's groups by shuffles
        const int jr = min(lane, max(span - 2, 0));
        const float ksr = __builtin_nontemporal_load((const __attribute__((address_space(1))) float*)((a.kscale + row0) + slot(jr)));
        const float vsr = __builtin_nontemporal_load((const __attribute__((address_space(1))) float*)((a.vscale + row0) + slot(jr)));
        Pk3 kw8[8], vw8[8];
        int off[8], rowu[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int e = min(u * 64 + lane, max(nr - 1, 0));
            const int jj = e / C4, c = e - jj * C4;
            off[u] = jj * DS + 4 * c;
            rowu[u] = jj;
            kw8[u] = ldg_pk3_nt(((const Pk3*)a.kpack + row0 * C4) + (slot(jj) * C4 + c));
            vw8[u] = ldg_pk3_nt(((const Pk3*)a.vpack + row0 * C4) + (slot(jj) * C4 + c));
        }
        float4 kb[8], vb[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            kb[u] = kv_unpack(kw8[u], __shfl(ksr, rowu[u], 64));
            vb[u] = kv_unpack(vw8[u], __shfl(vsr, rowu[u], 64));
        }
#pragma unroll
        for (int u = 0; u < 8; u++) *(float4*)(vs + off[u]) = kb[u];
        if (qpart == 1 && lane < 2 * C4) *(float4*)(vs + (span - 1) * DS + 4 * qc) = mine;
        wave_lds_sync();
        {
            const int jj = min(lane, span - 1);
#pragma unroll
            for (int c = 0; c < C4; c++) krow[c] = *(const float4*)(vs + jj * DS + 4 * c);
        }
        wave_lds_sync();
#pragma unroll
        for (int u = 0; u < 8; u++) *(float4*)(vs + off[u]) = vb[u];
        if (qpart == 2 && lane < 3 * C4) *(float4*)(vs + (span - 1) * DS + 4 * qc) = mine;
    } else {
        const int jj = min(lane, span - 1);
        if constexpr (PK) {
            // the ring row (the current position's slot is read too, in bounds, and its value replaced)
#pragma unroll
            for (int c = 0; c < C4; c++) krow[c] = pk4(a.kpack, a.kscale, slot(jj), c);
            if constexpr (QL) {
                if (jj == span - 1) {
#pragma unroll
                    for (int c = 0; c < C4; c++) krow[c] = qkv4(qkv + D + h * DH + 4 * c);
                }
            }
        } else if constexpr (QL) {
            // q, k, v in LDS: the ring row and the LDS row are separate loads (the current position's
            // ring slot is read too, in bounds, and its value discarded)
            const float* kp = kr + (long long)slot(jj) * DH;
#pragma unroll
            for (int c = 0; c < C4; c++) krow[c] = ldg((const float4*)(kp + 4 * c));
            if (jj == span - 1) {
#pragma unroll
                for (int c = 0; c < C4; c++) krow[c] = qkv4(qkv + D + h * DH + 4 * c);
            }
        } else {
            const float* kp = jj == span - 1 ? qkv + D + h * DH : kr + (long long)slot(jj) * DH;
#pragma unroll
            for (int c = 0; c < C4; c++) krow[c] = ldg((const float4*)(kp + 4 * c));
        }
    }
    // values: rows jj = 0..span-1 into LDS, every load issued before the first store. Lanes past the
    // end repeat the last element (the same bytes to the same address), so no store is conditional and
    // no load can be moved next to its store. Packed rings without QL: rows 0..span-2 from the ring, the
    // current position's row from the lanes holding it.
    const int n4 = KST ? 0 : (CUR_LANES ? span - 1 : span) * C4;
    for (int e0 = 0; e0 < n4; e0 += 8 * 64) {
        float4 vb[8];
        int off[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int e = min(e0 + u * 64 + lane, n4 - 1);
            const int jj = e / C4, c = e - jj * C4;
            if constexpr (PK) {
                vb[u] = pk4(a.vpack, a.vscale, slot(jj), c);
                if constexpr (QL) {
                    if (jj == span - 1) vb[u] = qkv4(qkv + 2 * D + h * DH + 4 * c);
                }
            } else if constexpr (QL) {
                vb[u] = ldg((const float4*)(vr + (long long)slot(jj) * DH + 4 * c));
                if (jj == span - 1) vb[u] = qkv4(qkv + 2 * D + h * DH + 4 * c);
            } else {
                const float* vp = jj == span - 1 ? qkv + 2 * D + h * DH : vr + (long long)slot(jj) * DH;
                vb[u] = ldg((const float4*)(vp + 4 * c));
            }
            off[u] = jj * DS + 4 * c;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) *(float4*)(vs + off[u]) = vb[u];
    }
    if constexpr (CUR_LANES && !KST) {
        if (qpart == 1 && lane < 2 * C4) *(float4*)(kc + 4 * qc) = mine;
        if (qpart == 2 && lane < 3 * C4) *(float4*)(vs + (span - 1) * DS + 4 * qc) = mine;
    }
    if (lane < C4) *(float4*)(qs + 4 * lane) = mine;
    wave_lds_sync();
    if constexpr (CUR_LANES && !KST) {
        if (lane == span - 1) {
#pragma unroll
            for (int c = 0; c < C4; c++) krow[c] = *(const float4*)(kc + 4 * c);
        }
    }
    float q[DH];
#pragma unroll
    for (int i = 0; i < DH; i += 4) {
        const float4 t = *(const float4*)(qs + i);
        q[i] = t.x; q[i + 1] = t.y; q[i + 2] = t.z; q[i + 3] = t.w;
    }
    const float scale = (float)(1.0 / sqrt((double)DH));
    const float sc = dot_ref_reg4<DH>(q, krow) * scale;
    const float mx = wave_max(lane < span ? sc : -3.40282347e38f);
    const float ex = lane < span ? fast_exp_ref(sc - mx) : 0.0f;
    if (lane < span) es[lane] = ex;
    wave_lds_sync();
    if (lane == 0) {
        float sum = 0.0f;  // nn.SoftmaxInPlaceF32's sequential sum
#pragma unroll 8
        for (int jj = 0; jj < span; jj++) sum += es[jj];
        inv_sh = 1.0f / sum;
    }
    wave_lds_sync();
    // p = e * (1 / sum), as SoftmaxInPlaceF32 leaves it: each lane its own key's, once
    if (lane < span) es[lane] = ex * inv_sh;
    wave_lds_sync();
    float o = 0.0f;
    if (lane < DH) {
#pragma unroll 8
        for (int jj = 0; jj < span; jj++) o = axpy_ref<DH>(lane, es[jj], vs[jj * DS + lane], o);
    }
    // record this position's key and value (slot pos % cap; the evicted key is outside the window)
    if constexpr (PK) {
        // the row's largest magnitude over the C4 lanes holding it (every lane takes part): for C4 a power
        // of two the groups are aligned quads, half-rows and rows, reduced by DPP moves; else by shuffles
        const float am = fmaxf(fmaxf(fabsf(mine.x), fabsf(mine.y)), fmaxf(fabsf(mine.z), fabsf(mine.w)));
        float rm = am;
        if constexpr ((C4 & (C4 - 1)) == 0) {
            if constexpr (C4 >= 2) rm = fmaxf(rm, dpp_move<0xB1>(rm));   // quad_perm [1, 0, 3, 2]
            if constexpr (C4 >= 4) rm = fmaxf(rm, dpp_move<0x4E>(rm));   // quad_perm [2, 3, 0, 1]
            if constexpr (C4 >= 8) rm = fmaxf(rm, dpp_move<0x141>(rm));  // row_half_mirror
            if constexpr (C4 >= 16) rm = fmaxf(rm, dpp_move<0x140>(rm)); // row_mirror
        } else {
            rm = 0.0f;
#pragma unroll
            for (int i = 0; i < C4; i++) rm = fmaxf(rm, __shfl(am, qpart * C4 + i, 64));
        }
        if (lane >= C4 && lane < 3 * C4) {
            const int e = kv_exp(rm);
            const long long r = row0 + pos % cap;
            uint32_t* ring = lane < 2 * C4 ? a.kpack : a.vpack;
            stg_pk3((Pk3*)ring + r * C4 + qc, kv_pack(mine, e));
            if (qc == 0) stg((lane < 2 * C4 ? a.kscale : a.vscale) + r, ldexpf(1.0f, e));
        }
    } else {
        if (lane >= C4 && lane < 3 * C4) {
            float* ring = lane < 2 * C4 ? a.kring : a.vring;
            stg((float4*)(ring + (row0 + pos % cap) * DH + 4 * qc), mine);
        }
    }
    return o;
}

// Decode attention, one wave per (session, head), key rows in registers (rk_head); PK: packed rings.
template <int DH, bool PK>
__global__ __launch_bounds__(64) void attention_step_rk_kernel(AttnStepArgs a) {
    extern __shared__ __align__(16) float rk_smem[];
    __shared__ float rk_inv;
    const int s_ = blockIdx.x / a.heads, h = blockIdx.x % a.heads;
    const int lane = threadIdx.x;
    const float o = rk_head<DH, false, PK>(a, s_, h, lane, rk_smem, rk_inv);
    if (lane < DH) a.att[(long long)s_ * a.Dp + h * DH + lane] = o;
}

// Decode attention of one session per workgroup, one wave per head (rk_head), fused with the limb
// expansion of the attention output that the out projection reads: the row's absolute maximum over
// all heads gives its scale, and each lane writes its element's three limbs (row_kernel's ROW_SRC
// digits and scale, from the same values), so the output never goes through memory as fp32.
// PK: packed rings; ST: streamed (rk_head).
template <int DH, bool PK, bool ST = false>
__global__ __launch_bounds__(1024) void attention_step_rows_kernel(AttnStepArgs a) {
    extern __shared__ __align__(16) float rows_smem[];
    __shared__ float inv_sh[16], red[16];
    const int s_ = blockIdx.x, h = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (a.done && a.done[s_] >= 0) return;  // a finished session of a batched decode (the whole workgroup)
    const float o = rk_head<DH, false, PK, ST>(a, s_, h, lane, rows_smem + h * rk_lds_floats(a.cap, DH, PK), inv_sh[h]);
    const float mx = wave_max(lane < DH ? fabsf(o) : 0.0f);
    if (lane == 0) red[h] = mx;
    __syncthreads();
    float amax = red[0];
    for (int i = 1; i < a.heads; i++) amax = fmaxf(amax, red[i]);
    float sc, inv;
    limb_scale(amax, sc, inv);
    const int kc = a.Dp >> 6;
    if (lane < DH) {
        const Limbs L = split_limbs(o, inv);
        const int k = h * DH + lane;
        a.xl[frag_off_a(s_, k, 0, kc)] = L.q0;
        a.xl[frag_off_a(s_, k, 1, kc)] = L.q1;
        a.xl[frag_off_a(s_, k, 2, kc)] = L.q2;
    }
    for (int k = a.D + (int)threadIdx.x; k < a.Dp; k += blockDim.x)  // padding channels read as zero
#pragma unroll
        for (int l = 0; l < 3; l++) a.xl[frag_off_a(s_, k, l, kc)] = 0;
    if (threadIdx.x == 0) a.xs[s_] = sc;
}

// Decode attention, staged: the span's key and value head slices go to LDS with 16-byte loads (eight
// lanes per 128 bytes, a batch of loads in flight before any is stored), then the same reference-order
// scores, softmax and P.V as attention_step_kernel, read from LDS: bit-identical results, one memory
// round trip per batch instead of one per key.
template <int DH>
__global__ __launch_bounds__(64) void attention_step_lds_kernel(AttnStepArgs a) {
    constexpr int DS = DH + 4;  // LDS row stride (16-byte rows, consecutive rows 4 banks apart)
    constexpr int C4 = DH / 4;
    extern __shared__ __align__(16) float step_smem[];
    const int cap = a.cap;
    float* ks = step_smem;          // [cap][DS]
    float* vs = ks + cap * DS;      // [cap][DS]
    float* es = vs + cap * DS;      // [cap]
    __shared__ float inv_sh;
    const int s_ = blockIdx.x / a.heads, h = blockIdx.x % a.heads;
    const int lane = threadIdx.x;
    const int D = a.D;
    const int pos = a.pos[s_];
    const int lo = max(window_start(pos, a.window), pos - cap + 1);
    const int span = pos - lo + 1;
    const float* qkv = a.qkv + (long long)s_ * 3 * D;
    const float* kr = a.kring + ((long long)s_ * a.heads + h) * cap * DH;
    const float* vr = a.vring + ((long long)s_ * a.heads + h) * cap * DH;
    // rows jj = 0..span-1 hold key/value j = lo + jj (the current position's from qkv, not yet in the ring)
    const int n4 = span * C4;
    for (int e0 = 0; e0 < n4; e0 += 8 * 64) {
        float4 kb[8], vb[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int e = min(e0 + u * 64 + lane, n4 - 1);
            const int jj = e / C4, c = e - jj * C4;
            const int j = lo + jj;
            const float* kp = j == pos ? qkv + D + h * DH : kr + (long long)(j % cap) * DH;
            const float* vp = j == pos ? qkv + 2 * D + h * DH : vr + (long long)(j % cap) * DH;
            kb[u] = *(const float4*)(kp + 4 * c);
            vb[u] = *(const float4*)(vp + 4 * c);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int e = e0 + u * 64 + lane;
            if (e < n4) {
                const int jj = e / C4, c = e - jj * C4;
                *(float4*)(ks + jj * DS + 4 * c) = kb[u];
                *(float4*)(vs + jj * DS + 4 * c) = vb[u];
            }
        }
    }
    float q[DH];
#pragma unroll
    for (int i = 0; i < DH; i += 4) {
        const float4 t = *(const float4*)(qkv + h * DH + i);
        q[i] = t.x; q[i + 1] = t.y; q[i + 2] = t.z; q[i + 3] = t.w;
    }
    __syncthreads();
    const float scale = (float)(1.0 / sqrt((double)DH));
    float mx = -3.40282347e38f;
    for (int jj = lane; jj < span; jj += 64) {
        const float sc = dot_ref_lds4<DH>(q, ks + jj * DS) * scale;
        es[jj] = sc;
        mx = fmaxf(mx, sc);
    }
    mx = wave_max(mx);
    for (int jj = lane; jj < span; jj += 64) es[jj] = fast_exp_ref(es[jj] - mx);
    __syncthreads();
    if (lane == 0) {
        float sum = 0.0f;  // nn.SoftmaxInPlaceF32's sequential sum
#pragma unroll 8
        for (int jj = 0; jj < span; jj++) sum += es[jj];
        inv_sh = 1.0f / sum;
    }
    __syncthreads();
    const float inv = inv_sh;
    for (int i = lane; i < DH; i += 64) {
        float o = 0.0f;
#pragma unroll 8
        for (int jj = 0; jj < span; jj++) o = axpy_ref<DH>(i, es[jj] * inv, vs[jj * DS + i], o);
        a.att[(long long)s_ * a.Dp + h * DH + i] = o;
    }
    // record this position's key and value (slot pos % cap; the evicted key is outside the window)
    float* kw = a.kring + (((long long)s_ * a.heads + h) * cap + pos % cap) * DH;
    float* vw = a.vring + (((long long)s_ * a.heads + h) * cap + pos % cap) * DH;
    for (int i = lane; i < DH; i += 64) {
        kw[i] = qkv[D + h * DH + i];
        vw[i] = qkv[2 * D + h * DH + i];
    }
}

// ------------------------------------------------------------------------------------------------
// Attention of any head width and any span (the fallback where no kernel above applies): one wave
// per (row, head), batched rows reading their keys and values from the QKV rows of their sequence,
// decode rows from their ring. Bit-identical to the reference order, like the kernels above:
//   - Scores. DotF32's sixteen accumulator chains (vec_amd64.s:4-63) run on the sixteen lanes of a
//     group, one key per group and four keys per wave step: lane u takes elements 16c + u of every
//     16-chunk (u < 8 accumulator 0, u >= 8 accumulator 1) and, for u < 8, the trailing 8-chunk.
//     The fold (a0 + a1, the high half onto the low, then the two shuffles) is the same additions
//     through shuffles, and lane 0 of the group adds the unfused tail products in element order.
//   - Softmax. Scores in LDS; max over the wave, FastExp, the sum in index order by one lane.
//   - P.V. Lane i accumulates output elements i, i + 64, ... over the keys in order (AddScaledF32:
//     fused inside the 16- and 8-chunks, unfused in the tail).
// Keys and values pass through LDS in chunks of at most kWaveStage floats, all of a chunk's loads
// issued before its first store.
// ------------------------------------------------------------------------------------------------
constexpr int kWaveStage = 4096;  // floats of one staged chunk of key or value rows

__host__ __device__ inline int wave_chunk_keys(int dh) {
    const int k = kWaveStage / dh / 4 * 4;
    return k < 4 ? 4 : (k > 256 ? 256 : k);
}

// Copies rows j0 .. j0+nk-1 (dh floats each, rowp(j) gives row j) to stage[(j - j0)*dh ..]. nk*dh
// is at most kWaveStage, so a lane moves at most 64 floats.
template <class RowFn>
__device__ __forceinline__ void wave_stage(float* stage, const RowFn& rowp, int j0, int nk, int dh, int lane) {
    const int n = nk * dh;
    const float inv_dh = 1.0f / (float)dh;
    for (int e0 = 0; e0 < n; e0 += 16 * 64) {
        float buf[16];
        int off[16];
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const int e = min(e0 + t * 64 + lane, n - 1);  // lanes past the end repeat the last element
            int key = (int)(((float)e + 0.5f) * inv_dh);   // e < 4096: one correction step suffices
            if (key * dh > e) key--;
            else if ((key + 1) * dh <= e) key++;
            buf[t] = rowp(j0 + key)[e - key * dh];
            off[t] = e;
        }
#pragma unroll
        for (int t = 0; t < 16; t++) stage[off[t]] = buf[t];
    }
}

// LDS floats of attention_wave_kernel for spans of at most `span` keys.
__host__ __device__ inline int wave_lds_floats(int span) { return kWaveStage + span; }

// NC = 16-element chunk slots per lane: dh <= 16*NC.
template <int NC>
__global__ __launch_bounds__(64) void attention_wave_kernel(AttnWaveArgs a) {
    constexpr int NO = (NC + 3) / 4;  // output elements per lane
    extern __shared__ __align__(16) float wv_smem[];
    float* stage = wv_smem;            // [kWaveStage]
    float* sc = wv_smem + kWaveStage;  // [span]
    const int row = blockIdx.x, h = blockIdx.y;
    const int lane = threadIdx.x, u = lane & 15, grp = lane >> 4;
    const int dh = a.dh, D = a.D, cap = a.cap;
    int pos;
    long long seq0 = 0;  // batched: first row of the sequence
    if (a.step) {
        pos = a.pos[row];
    } else {
        const int b = row / a.T;
        pos = row - b * a.T;
        seq0 = (long long)b * a.T;
    }
    const int lo = max(window_start(pos, a.window), pos - cap + 1);
    const int span = pos - lo + 1;
    const float* qrow = a.qkv + (long long)row * 3 * D + h * dh;
    const long long ring0 = ((long long)row * a.heads + h) * cap;
    auto krow = [&](int j) -> const float* {
        if (a.step) return j == pos ? qrow + D : a.kring + (ring0 + j % cap) * dh;
        return a.qkv + (seq0 + j) * 3 * D + D + h * dh;
    };
    auto vrow = [&](int j) -> const float* {
        if (a.step) return j == pos ? qrow + 2 * D : a.vring + (ring0 + j % cap) * dh;
        return a.qkv + (seq0 + j) * 3 * D + 2 * D + h * dh;
    };
    const int n16 = dh >> 4;
    const bool has8 = (dh & 15) >= 8;
    const int t0 = (has8 ? 8 : 0), ntail = dh - 16 * n16 - t0;  // tail lanes t0 .. t0+ntail-1 of slot n16
    float qr[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) qr[c] = (16 * c + u < dh) ? qrow[16 * c + u] : 0.0f;
    const float scale = (float)(1.0 / sqrt((double)dh));
    const int KC = wave_chunk_keys(dh);

    float mx = -3.40282347e38f;
    for (int c0 = 0; c0 < span; c0 += KC) {
        const int nk = min(KC, span - c0);
        wave_stage(stage, krow, lo + c0, nk, dh, lane);
        wave_lds_sync();
        for (int k4 = 0; k4 < nk; k4 += 4) {
            const int kk = min(k4 + grp, nk - 1);
            const float* kr = stage + kk * dh;
            float acc = 0.0f, tailp = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                if (c < n16) acc = fmaf(qr[c], kr[16 * c + u], acc);
                if (c == n16) {
                    const float kv = kr[min(16 * c + u, dh - 1)];
                    if (has8 && u < 8) acc = fmaf(qr[c], kv, acc);
                    tailp = qr[c] * kv;
                }
            }
            float v = acc + __shfl_xor(acc, 8, 16);
            v = v + __shfl_xor(v, 4, 16);
            v = v + __shfl_xor(v, 2, 16);
            float s = v + __shfl_xor(v, 1, 16);
            for (int t = 0; t < ntail; t++) {
                const float p = __shfl(tailp, t0 + t, 16);
                s = s + p;
            }
            s = s * scale;
            if (u == 0 && k4 + grp < nk) {
                sc[c0 + k4 + grp] = s;
                mx = fmaxf(mx, s);
            }
        }
        wave_lds_sync();  // the stage is rewritten by the next chunk
    }
    // nn.SoftmaxInPlaceF32 (internal/nn/head.go:91-112)
    mx = wave_max(mx);
    for (int jj = lane; jj < span; jj += 64) sc[jj] = fast_exp_ref(sc[jj] - mx);
    wave_lds_sync();
    float inv = 0.0f;
    if (lane == 0) {
        float sum = 0.0f;
#pragma unroll 8
        for (int jj = 0; jj < span; jj++) sum += sc[jj];
        inv = 1.0f / sum;
    }
    inv = __shfl(inv, 0, 64);

    const int fused = dh / 8 * 8;
    float o[NO];
#pragma unroll
    for (int r = 0; r < NO; r++) o[r] = 0.0f;
    for (int c0 = 0; c0 < span; c0 += KC) {
        const int nk = min(KC, span - c0);
        wave_stage(stage, vrow, lo + c0, nk, dh, lane);
        wave_lds_sync();
        for (int kk = 0; kk < nk; kk++) {
            const float p = sc[c0 + kk] * inv;
            const float* vr = stage + kk * dh;
#pragma unroll
            for (int r = 0; r < NO; r++) {
                const int i = lane + 64 * r;
                if (i < dh) {
                    const float x = vr[i];
                    if (i < fused) {
                        o[r] = fmaf(p, x, o[r]);
                    } else {
                        const float t = x * p;
                        o[r] = t + o[r];
                    }
                }
            }
        }
        wave_lds_sync();
    }
    float* dst = a.att + (long long)row * a.Dp + h * dh;
#pragma unroll
    for (int r = 0; r < NO; r++) {
        const int i = lane + 64 * r;
        if (i < dh) dst[i] = o[r];
    }
    if (a.step) {  // record this position's key and value (slot pos % cap lies outside the window)
        float* kw = a.kring + (ring0 + pos % cap) * dh;
        float* vw = a.vring + (ring0 + pos % cap) * dh;
        for (int i = lane; i < dh; i += 64) {
            kw[i] = qrow[D + i];
            vw[i] = qrow[2 * D + i];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Head statistics, log-probs, bits
// ------------------------------------------------------------------------------------------------
// Per-row softmax statistics from the logits GEMM's per-tile (max, sum exp(l - max), first argmax).
// Sixteen lanes per row read the row's tiles coalesced (lane l takes tiles l, l+16, ...), then merge
// across the group with xor shuffles: the larger max wins and rescales the other sum, equal maxima keep
// the smaller index (the reference's first maximum, internal/generate/greedy.go:89-102).
__device__ __forceinline__ void merge_stats(float& bm, float& bs, int& bi, float om, float os, int oi) {
    if (om == -INFINITY) return;
    const float nm = fmaxf(bm, om);
    const float ns = (bm == -INFINITY ? 0.0f : bs * __expf(bm - nm)) + os * __expf(om - nm);
    const int ni = (om > bm) ? oi : (bm > om) ? bi : min(bi, oi);
    bm = nm; bs = ns; bi = ni;
}

// Workgroup barrier over LDS only, for the one-workgroup decode steps: their waves exchange data through
// LDS alone (what they store to global memory is read by later kernels, or by the storing lane), so
// outstanding global loads and stores need not drain at each phase boundary.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ------------------------------------------------------------------------------------------------
// One session's decode step in one workgroup (step1_kernel)
// ------------------------------------------------------------------------------------------------
constexpr int S1_THREADS = 512;

// The row kernel's RMSNorm scale (1/rms) of one row x[0..D), by one wave: 16 partial sums in DotF32's
// order, their fold, the unfused tail, then float32(sqrt(float64(ss/D + 1e-5))) (row_kernel).
__device__ __forceinline__ float s1_rms_inv(const float* x, int D, int lane) {
    const int p = lane & 15;
    float part = 0.0f;
    const int c16 = D >> 4;
#pragma unroll 8
    for (int c = 0; c < c16; c++) {
        const float v = x[16 * c + p];
        part = fmaf(v, v, part);
    }
    if (p < 8 && D - 16 * c16 >= 8) {
        const float v = x[16 * c16 + p];
        part = fmaf(v, v, part);
    }
    float v8[8];
#pragma unroll
    for (int q = 0; q < 8; q++) v8[q] = lane_value(part, q) + lane_value(part, q + 8);
    float ss = hreduce8(v8);
    for (int e = (D >> 3) << 3; e < D; e++) {
        const float t = x[e];
        const float pp = t * t;
        ss = ss + pp;
    }
    const float rms = (float)sqrt((double)(ss / (float)D + 1e-5f));
    return 1.0f / rms;
}

// Workgroup maximum of per-thread values (every thread gets it). red: 8 floats of LDS, read after the one
// barrier here; consecutive reductions alternate between two such buffers, so that a reduction's writes
// never meet the previous one's reads (the barrier of the reduction between them orders the two).
__device__ __forceinline__ float s1_block_max(float v, float* red, int lane, int w) {
    v = wave_max(v);
    if (lane == 0) red[w] = v;
    lds_barrier();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < S1_THREADS / 64; i++) m = fmaxf(m, red[i]);
    return m;
}

// Limb planes of one row (values x[d] for d < Dvalid, zero up to Kp) in the single-row operand layout
// xl[k >> 6][limb][k & 63]; returns the row scale. The digits and scale are the row kernel's.
__device__ __forceinline__ float s1_limbs(const float* x, int Dvalid, int Kp, int8_t* xl, float* red, int tid,
                                          int lane, int w) {
    float m = 0.0f;
    for (int d = tid; d < Dvalid; d += S1_THREADS) m = fmaxf(m, fabsf(x[d]));
    const float amax = s1_block_max(m, red, lane, w);
    float sc, inv;
    limb_scale(amax, sc, inv);
    for (int k = tid; k < Kp; k += S1_THREADS) {
        const Limbs L = split_limbs(k < Dvalid ? x[k] : 0.0f, inv);
        int8_t* o = xl + (k >> 6) * 3072 + ((16 * ((k >> 4) & 3)) << 4) + (k & 15);
        o[0] = L.q0;
        o[1024] = L.q1;
        o[2048] = L.q2;
    }
    return sc;
}

__device__ __forceinline__ float s1_dot(const v4i (&acc)[3], int r) {
    return fmaf((float)acc[2][r], kInvLimb2, fmaf((float)acc[1][r], kInvLimb1, (float)acc[0][r]));
}

// Matrix phases of the one-workgroup decode steps (8 waves; the limb operand xl holds the rows of up to
// 16 sessions in the MFMA's token columns). Wave w takes units w, w + 8, ... of the phase: with TS_FRAG one
// 16-channel fragment (GF units per group), with TS_PAIR the fragment pair 2q (value), 2q + 1 (gate)
// (GF/2 per group), with TS_TILE the GF consecutive fragments GF*u .. GF*u + GF - 1 (one per group).
// A group's weights are requested KB K steps at a time (GF * KB loads in flight; loads past the wave's
// units or past the last K step repeat a valid address and go unused), with the group's bias values
// (`bias`, indexed by output row, or null), then multiplied by the tile's limb planes (all 16 token
// columns). After a group's last K step `epi` gets, for each unit, the combined dot products of token
// lane & 15, channels c0 .. c0 + 3 with c0 = 16 f + 4 (lane >> 4), and the bias of those rows:
// epi(f, v[4], b) (TS_FRAG), epi(q, vv[4], vg[4], bv, bg) (TS_PAIR), or epi(u, acc, b[GF]) (TS_TILE).
// K512 (TS_FRAG, the head): the digit planes combined as the head GEMMs combine them (limb_sum_k512).
enum { TS_FRAG = 0, TS_PAIR = 1, TS_TILE = 2 };
template <int MODE, int GF, int KB, bool K512 = false, class Epi>
__device__ __forceinline__ void ts_matvec(const int8_t* W, const float* bias, int np16, int kc, int nunits,
                                          const int8_t* xl, int lane, int w, Epi&& epi) {
    constexpr int UPG = MODE == TS_FRAG ? GF : MODE == TS_PAIR ? GF / 2 : 1;  // units per group
    const int mine = nunits > w ? (nunits - 1 - w) / 8 + 1 : 0;
    const int8_t* wl = W + lane * 16;
    const int8_t* xp = xl + lane * 16;
    for (int gi = 0; gi * UPG < mine; gi++) {
        int fr[GF];
        bool ok[GF];
#pragma unroll
        for (int g = 0; g < GF; g++) {
            const int u0 = UPG * gi + (MODE == TS_FRAG ? g : MODE == TS_PAIR ? g / 2 : 0);
            ok[g] = u0 < mine;
            const int un = w + 8 * min(u0, mine - 1);
            fr[g] = MODE == TS_FRAG ? un : MODE == TS_PAIR ? 2 * un + (g & 1) : GF * un + g;
        }
        // the bias with the weights (after the MFMAs for whole tiles, whose accumulators fill the registers)
        float4 b4[GF];
        auto load_bias = [&] {
#pragma unroll
            for (int g = 0; g < GF; g++)
                b4[g] = bias ? ldg((const float4*)(bias + 16 * fr[g] + 4 * (lane >> 4))) : float4{0.0f, 0.0f, 0.0f, 0.0f};
        };
        if constexpr (MODE != TS_TILE) load_bias();
        v4i acc[GF][3];
#pragma unroll
        for (int g = 0; g < GF; g++) acc[g][0] = acc[g][1] = acc[g][2] = v4i{0, 0, 0, 0};
        for (int k0 = 0; k0 < kc; k0 += KB) {
            v4i wv[GF][KB];
#pragma unroll
            for (int g = 0; g < GF; g++)
#pragma unroll
                for (int j = 0; j < KB; j++)
                    wv[g][j] = ldg((const v4i*)(wl + (((long long)min(k0 + j, kc - 1) * np16 + fr[g]) << 10)));
            // keep the batch together: the scheduler would otherwise sink each load to its first MFMA
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < KB; j++) {
                if (k0 + j >= kc) break;
                v4i xv[3];
#pragma unroll
                for (int l = 0; l < 3; l++) xv[l] = *(const v4i*)(xp + (k0 + j) * 3072 + l * 1024);
#pragma unroll
                for (int g = 0; g < GF; g++)
                    if (ok[g])
#pragma unroll
                        for (int l = 0; l < 3; l++)
                            acc[g][l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[g][j], xv[l], acc[g][l], 0, 0, 0);
            }
        }
        if constexpr (MODE == TS_TILE) {
            load_bias();
            epi(w + 8 * gi, acc, b4);
        } else if constexpr (MODE == TS_PAIR) {
#pragma unroll
            for (int p = 0; p < GF / 2; p++)
                if (ok[2 * p]) {
                    float vv[4], vg[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        vv[r] = s1_dot(acc[2 * p], r);
                        vg[r] = s1_dot(acc[2 * p + 1], r);
                    }
                    epi(fr[2 * p] >> 1, vv, vg, b4[2 * p], b4[2 * p + 1]);
                }
        } else {
#pragma unroll
            for (int g = 0; g < GF; g++)
                if (ok[g]) {
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        v[r] = K512 ? limb_sum_k512(acc[g][0][r], acc[g][1][r], acc[g][2][r]) : s1_dot(acc[g], r);
                    epi(fr[g], v, b4[g]);
                }
        }
    }
}

// PK: the set's K/V rings are packed (a separate instantiation, so that the fp32-ring kernel, which the
// latency-bound small sets take, carries none of the packed path's code).
template <int DH, bool PK>
__global__ __launch_bounds__(S1_THREADS) void step1_kernel(Step1Args a) {
    extern __shared__ __align__(16) float s1_smem[];
    __shared__ float red[16];
    __shared__ float rk_inv[8];
    __shared__ float bcast[4];
    const int s_ = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int D = a.D, Dp = a.Dp, H = a.H, Hp = a.Hp, V = a.V, Vp = a.Vp;
    const int ntiles = Vp / LX_BN;
    float* cur = s1_smem;
    float* bin = cur + Dp;
    float* nrm = bin + Dp;
    float* lam = nrm + Dp;
    float* hbuf = lam + Dp;
    float* qkv = hbuf + Hp;
    float* att = qkv + 3 * Dp;
    float* logit = att + Dp;
    float* tstats = logit + Vp;
    float* rk = tstats + 4 * ntiles;
    const int rkf = (rk_lds_floats(a.cap, DH) + 3) & ~3;  // per head, 16-byte aligned
    int8_t* xl = (int8_t*)(rk + a.heads * rkf);
    if (a.done && a.done[s_] >= 0) return;  // a finished session of a batched decode
    // the two halves of red, alternating between consecutive workgroup reductions (s1_block_max)
    int red_half = 0;
    auto next_red = [&]() {
        red_half ^= 1;
        return red + 8 * red_half;
    };
    const int pos = a.pos[s_];
    {
        int id = a.ids[s_];
        id = (id < 0 || id >= V) ? 0 : id;  // quant.Model.appendPosition clamps (stream.go:144-146)
        for (int d = tid; d < Dp; d += S1_THREADS) {
            const float v = d < D ? (float)a.emb[(long long)id * D + d] * a.emb_scale : 0.0f;
            cur[d] = v;
            bin[d] = v;
        }
    }
    lds_barrier();
    int bs = 0, ab = 0;
    for (int b = 0; b < a.nblocks; b++) {
        const Step1Block& B = a.blocks[b];
        if (b > 0) {
            // blockIn += cur; cur = blockIn (stream.go:157-163)
            for (int d = tid; d < Dp; d += S1_THREADS) {
                const float v = bin[d] + cur[d];
                bin[d] = v;
                cur[d] = v;
            }
            lds_barrier();
        }
        for (int st = 0; st < B.steps; st++, bs++) {
            int dil = B.init_dil;
            for (int q = 0; q < st && dil < 32; q++) dil *= B.dil_base;
            dil = min(dil, 32);
            // n = RMSNorm(cur; gamma) (stream.go:166-171)
            if (B.gamma) {
                if (w == 0) {
                    const float inv = s1_rms_inv(cur, D, lane);
                    if (lane == 0) bcast[0] = inv;
                }
                lds_barrier();
                const float inv = bcast[0];
                for (int d = tid; d < Dp; d += S1_THREADS) nrm[d] = d < D ? (cur[d] * inv) * ldg(B.gamma + d) : 0.0f;
            } else {
                for (int d = tid; d < Dp; d += S1_THREADS) nrm[d] = d < D ? cur[d] : 0.0f;
            }
            // (no barrier: s1_limbs reads element d of nrm in the thread that wrote it)
            const float sn = s1_limbs(nrm, D, Dp, xl, next_red(), tid, lane, w);
            lds_barrier();
            // lambda = sigmoid_clamped(n.W_sel*s + base) (stream.go:195-205)
            {
                const float sw = sn * B.ssel;
                ts_matvec<TS_FRAG, 4, 2>(B.wsel, a.latch_base, a.NpD / 16, Dp / 64, a.NpD / 16, xl, lane, w,
                                         [&](int f, const float (&v)[4], float4 b) {
                    if (lane & 15) return;
                    const int c0 = 16 * f + 4 * (lane >> 4);
                    const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (c0 + r < D) lam[c0 + r] = sigmoid_epi(fmaf(v[r], sw, bb[r]));
                });
            }
            lds_barrier();
            // latch update, norm ring and the rule input [n | left | g] (latch_step_kernel)
            float nv = 0.0f, lv = 0.0f, gv = 0.0f;
            const int d = tid;
            if (d < D) {
                nv = nrm[d];
                const float l = lam[d];
                float* gp = a.g + ((long long)bs * a.S + s_) * Dp + d;
                gv = *gp;
                const float p1 = l * gv;
                const float p2 = (1.0f - l) * nv;
                gv = p1 + p2;
                *gp = gv;
                float* ring = a.norm_ring + ((long long)bs * a.S + s_) * a.ring * Dp;
                ring[(long long)(pos % a.ring) * Dp + d] = nv;
                if (pos >= dil) lv = ring[(long long)((pos - dil) % a.ring) * Dp + d];
            }
            const float amax = s1_block_max(fmaxf(fabsf(nv), fmaxf(fabsf(lv), fabsf(gv))), next_red(), lane, w);
            float sx, ix;
            limb_scale(amax, sx, ix);
            {
                const float v3[3] = {nv, lv, gv};
                if (d < Dp) {
#pragma unroll
                    for (int sg = 0; sg < 3; sg++) {
                        const Limbs L = split_limbs(v3[sg], ix);
                        const int k = sg * Dp + d;
                        int8_t* o = xl + (k >> 6) * 3072 + ((16 * ((k >> 4) & 3)) << 4) + (k & 15);
                        o[0] = L.q0;
                        o[1024] = L.q1;
                        o[2048] = L.q2;
                    }
                }
            }
            lds_barrier();
            // h = GLU(x) (stream.go:214-220): fragment pairs (value 2q, gate 2q + 1)
            {
                const float sw = sx * B.s1;
                ts_matvec<TS_PAIR, 4, 2>(B.w1, B.b1, 2 * Hp / 16, 3 * Dp / 64, Hp / 16, xl, lane, w,
                                         [&](int q, const float (&vv)[4], const float (&vg)[4], float4 bv, float4 bg) {
                    if (lane & 15) return;
                    const int c0 = 16 * q + 4 * (lane >> 4);
                    const float bvv[4] = {bv.x, bv.y, bv.z, bv.w}, bgg[4] = {bg.x, bg.y, bg.z, bg.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float ov = fmaf(vv[r], sw, bvv[r]);
                        const float gt = sigmoid_epi(fmaf(vg[r], sw, bgg[r]));
                        hbuf[c0 + r] = c0 + r < H ? ov * gt : 0.0f;
                    }
                });
            }
            lds_barrier();
            const float sh = s1_limbs(hbuf, H, Hp, xl, next_red(), tid, lane, w);
            lds_barrier();
            // cur = highway(cur, W2 h) (stream.go:222-229)
            {
                const float sw = sh * B.s2;
                ts_matvec<TS_PAIR, 4, 2>(B.w2, B.b2, 2 * Dp / 16, Hp / 64, Dp / 16, xl, lane, w,
                                         [&](int q, const float (&vv)[4], const float (&vg)[4], float4 bv, float4 bg) {
                    if (lane & 15) return;
                    const int c0 = 16 * q + 4 * (lane >> 4);
                    const float bvv[4] = {bv.x, bv.y, bv.z, bv.w}, bgg[4] = {bg.x, bg.y, bg.z, bg.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int c = c0 + r;
                        if (c < D) {
                            const float ov = fmaf(vv[r], sw, bvv[r]);
                            const float gt = sigmoid_epi(fmaf(vg[r], sw, bgg[r]));
                            const float x1 = (1.0f - gt) * cur[c];
                            const float x2 = gt * ov;
                            cur[c] = x1 + x2;
                        }
                    }
                });
            }
            lds_barrier();
        }
        if (B.attn) {
            // attendPosition (internal/quant/attention.go:69-104)
            if (w == 0) {
                const float inv = s1_rms_inv(cur, D, lane);
                if (lane == 0) bcast[0] = inv;
            }
            lds_barrier();
            {
                const float inv = bcast[0];
                for (int d = tid; d < Dp; d += S1_THREADS) nrm[d] = d < D ? (cur[d] * inv) * ldg(B.anorm + d) : 0.0f;
            }
            const float sa = s1_limbs(nrm, D, Dp, xl, next_red(), tid, lane, w);
            lds_barrier();
            {
                const float sw = sa * B.sqkv;
                ts_matvec<TS_FRAG, 4, 2>(B.qkv, nullptr, a.Np3 / 16, Dp / 64, a.Np3 / 16, xl, lane, w,
                                         [&](int f, const float (&v)[4], float4) {
                    if (lane & 15) return;
                    const int c0 = 16 * f + 4 * (lane >> 4);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (c0 + r < 3 * D) qkv[c0 + r] = v[r] * sw;
                });
            }
            lds_barrier();
            if (w < a.heads) {
                AttnStepArgs sa_;
                sa_.S = 1; sa_.D = D; sa_.Dp = Dp; sa_.heads = a.heads; sa_.window = a.window; sa_.cap = a.cap;
                sa_.pos = a.pos + s_;
                sa_.qkv = qkv;
                const long long rows0 = ((long long)ab * a.S + s_) * a.heads * a.cap;  // ring rows before this one's
                float o;
                if constexpr (PK) {
                    sa_.kpack = a.kpack + rows0 * kv_row_words(DH);
                    sa_.vpack = a.vpack + rows0 * kv_row_words(DH);
                    sa_.kscale = a.kscale + rows0;
                    sa_.vscale = a.vscale + rows0;
                    o = rk_head<DH, true, true>(sa_, 0, w, lane, rk + w * rkf, rk_inv[w]);
                } else {
                    sa_.kring = a.kring + rows0 * DH;
                    sa_.vring = a.vring + rows0 * DH;
                    o = rk_head<DH, true>(sa_, 0, w, lane, rk + w * rkf, rk_inv[w]);
                }
                if (lane < DH) att[w * DH + lane] = o;
            }
            lds_barrier();
            const float so_ = s1_limbs(att, D, Dp, xl, next_red(), tid, lane, w);
            lds_barrier();
            {
                const float sw = so_ * B.so;
                ts_matvec<TS_FRAG, 4, 2>(B.wo, nullptr, a.NpD / 16, Dp / 64, a.NpD / 16, xl, lane, w,
                                         [&](int f, const float (&v)[4], float4) {
                    if (lane & 15) return;
                    const int c0 = 16 * f + 4 * (lane >> 4);
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (c0 + r < D) cur[c0 + r] = cur[c0 + r] + v[r] * sw;
                });
            }
            lds_barrier();
            ab++;
        }
    }
    // headLogits (internal/quant/stream.go:232-248)
    if (a.final_norm) {
        if (w == 0) {
            const float inv = s1_rms_inv(cur, D, lane);
            if (lane == 0) bcast[0] = inv;
        }
        lds_barrier();
        const float inv = bcast[0];
        for (int d = tid; d < Dp; d += S1_THREADS) nrm[d] = d < D ? (cur[d] * inv) * a.final_norm[d] : 0.0f;
    } else {
        for (int d = tid; d < Dp; d += S1_THREADS) nrm[d] = d < D ? cur[d] : 0.0f;
    }
    const float sf = s1_limbs(nrm, D, Dp, xl, next_red(), tid, lane, w);
    lds_barrier();
    {
        const float sw = sf * a.head_scale;
        ts_matvec<TS_FRAG, 4, 2, true>(a.headw, a.headb, Vp / 16, Dp / 64, Vp / 16, xl, lane, w,
                                       [&](int f, const float (&v)[4], float4 b) {
            if (lane & 15) return;
            const int c0 = 16 * f + 4 * (lane >> 4);
            *(float4*)(logit + c0) = float4{fmaf(v[0], sw, b.x), fmaf(v[1], sw, b.y), fmaf(v[2], sw, b.z), fmaf(v[3], sw, b.w)};
        });
    }
    lds_barrier();
    if (a.logits) {  // coalesced: the row may live in host memory
        float* lo = a.logits + (long long)s_ * V;
        for (int c = tid; c < V; c += S1_THREADS) lo[c] = logit[c];
    }
    // (a step asked for the logits alone, as Append is, needs none of the statistics below)
    if (!(a.argmax || a.prob || a.next_ids || a.out_ids || a.out_probs)) {
        if (tid == 0) a.pos[s_] = pos + 1;
        return;
    }
    // per 128-channel tile: the logits epilogue's statistics (max, sum exp(l - max), first argmax), with
    // its lane structure (lane group g4 = lane >> 4 holds channels 4g4 + 16ti + r)
    const bool want_argmax = a.argmax || a.next_ids || a.out_ids;
    for (int t = w; t < ntiles; t += S1_THREADS / 64) {
        const float l2e = 1.4426950408889634f;
        const int nb = t * LX_BN + 4 * (lane >> 4);
        float y[8][4];
#pragma unroll
        for (int ti = 0; ti < 8; ti++) {
            const float4 v = *(const float4*)(logit + nb + 16 * ti);
            y[ti][0] = v.x; y[ti][1] = v.y; y[ti][2] = v.z; y[ti][3] = v.w;
        }
        float mx = y[0][0];
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int r = 0; r < 4; r++) mx = fmaxf(mx, y[ti][r]);
        const float ml = mx == -INFINITY ? 0.0f : mx * l2e;
        float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int r = 0; r < 4; r++) s4[r] += __builtin_amdgcn_exp2f(fmaf(y[ti][r], l2e, -ml));
        float bmax = mx, bsum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        int bidx = 0x7fffffff;
        if (want_argmax && mx > -INFINITY) {
            int off = 0;
#pragma unroll
            for (int ti = 7; ti >= 0; ti--)
#pragma unroll
                for (int r = 3; r >= 0; r--) off = y[ti][r] == mx ? ti * 16 + r : off;
            bidx = nb + off;
        }
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {
            float om = __shfl_xor(bmax, o, 64), os = __shfl_xor(bsum, o, 64);
            int oi = __shfl_xor(bidx, o, 64);
            float nm = fmaxf(bmax, om);
            float ns = (bmax == -INFINITY ? 0.0f : bsum * __expf(bmax - nm)) +
                       (om == -INFINITY ? 0.0f : os * __expf(om - nm));
            int ni = (om > bmax) ? oi : (bmax > om) ? bidx : min(bidx, oi);
            bmax = nm; bsum = ns; bidx = ni;
        }
        if (lane == 0) {
            tstats[3 * t] = bmax;
            tstats[3 * t + 1] = bsum;
            tstats[3 * t + 2] = __int_as_float(bidx);
        }
    }
    lds_barrier();
    // their combination (head_combine_kernel), 16 lanes of wave 0
    if (w == 0 && lane < 16) {
        const int l = lane;
        float bm = -INFINITY, bsm = 0.0f;
        int bi = 0x7fffffff;
        for (int t = l; t < ntiles; t += 16) merge_stats(bm, bsm, bi, tstats[3 * t], tstats[3 * t + 1], __float_as_int(tstats[3 * t + 2]));
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) {
            const float om = __shfl_xor(bm, o, 16), os = __shfl_xor(bsm, o, 16);
            const int oi = __shfl_xor(bi, o, 16);
            merge_stats(bm, bsm, bi, om, os, oi);
        }
        if (l == 0) {
            const double p = 1.0 / (double)bsm;
            if (a.argmax) a.argmax[s_] = bi;
            if (a.prob) a.prob[s_] = p;
            if (a.next_ids) a.next_ids[s_] = bi;
            const int oc = a.col ? *a.col : a.out_col;
            if (a.out_ids) a.out_ids[(long long)s_ * a.out_ld + oc] = bi;
            if (a.out_probs) a.out_probs[(long long)s_ * a.out_ld + oc] = p;
            a.pos[s_] = pos + 1;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Decode step of a tile of 16 sessions per workgroup (tile_step_kernel)
// ------------------------------------------------------------------------------------------------
// The 16 sessions of a tile are the 16 token columns of v_mfma_i32_16x16x64_i8, so every weight
// fragment, loaded once per workgroup, serves all of them. The step runs in segments: a segment ends
// once an attention block's projection q, k, v is written; that block's attention (with the limb
// expansion of its output, attention_step_rows_kernel) runs between segments, and the next segment
// starts with the block's out projection. cur and blockIn go through memory between segments. In the
// row phases (residual, norms, limb planes, the latch update) wave w owns rows w and w + 8, lane L
// channels 4L + 256i .. +3. Every operation is the layered step's, in its order: results are
// bit-identical.
constexpr int TS_NS = 16;
constexpr int TS_THREADS = 512;
constexpr int TS_NI = 2;  // float4 chunks of a state row per lane (state size up to 512)

// LDS of tile_step_kernel (offsets in floats, the limb operand's in bytes): cur and blockIn [16][Dp + 4];
// one region reused by n and lambda [2][16][Dp + 4], h [16][Hp + 4] and the head's tile statistics
// [16][Vp/128][3]; then the limb operand xl [K/64][3 planes][1 KiB] for K up to max(3 Dp, Hp).
struct TsLds {
    int ld, hld, cur, bin, nrm, lam, h, ts, xl_off, bytes;
};
__host__ __device__ inline TsLds ts_lds(int Dp, int Hp, int Vp) {
    TsLds L;
    L.ld = Dp + 4;
    L.hld = Hp + 4;
    L.cur = 0;
    L.bin = TS_NS * L.ld;
    const int u = 2 * TS_NS * L.ld;
    L.nrm = u;
    L.lam = u + TS_NS * L.ld;
    L.h = u;
    L.ts = u;
    int usz = 2 * TS_NS * L.ld;
    usz = usz > TS_NS * L.hld ? usz : TS_NS * L.hld;
    usz = usz > TS_NS * (Vp / 128) * 3 ? usz : TS_NS * (Vp / 128) * 3;
    L.xl_off = ((u + usz) * 4 + 15) & ~15;
    const int kmax = 3 * Dp > Hp ? 3 * Dp : Hp;
    L.bytes = L.xl_off + (kmax / 64) * 3072;
    return L;
}

// Byte offset in xl of channel k (a multiple of 4) of token column t: fragment (K step k/64, plane 0),
// lane t + 16*((k >> 4) & 3), byte k & 15.
__device__ __forceinline__ int ts_xoff(int k, int t) { return (k >> 6) * 3072 + ((t + 16 * ((k >> 4) & 3)) << 4) + (k & 15); }

// The three limb planes of chunk v (channels k .. k + 3 of token column t) into xl.
__device__ __forceinline__ void ts_put_limbs(int8_t* xl, int k, int t, float4 v, float inv) {
    uint32_t w0, w1, w2;
    split4_pack(v, inv, w0, w1, w2);
    int8_t* o = xl + ts_xoff(k, t);
    *(uint32_t*)o = w0;
    *(uint32_t*)(o + 1024) = w1;
    *(uint32_t*)(o + 2048) = w2;
}

__device__ __forceinline__ float ts_amax4(float m, float4 v) {
    return fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
}

// Limb planes of one row (chunks v[i] = channels 4*lane + 256*i .. +3, zero at and past the row's valid
// channels) into column t of xl, for channels below Kp; returns the row scale. One wave: the row
// kernel's scale (the row's absolute maximum) and digits.
template <int NI>
__device__ __forceinline__ float ts_row_limbs(const float4 (&v)[NI], int Kp, int t, int8_t* xl, int lane) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; i++) m = ts_amax4(m, v[i]);
    float sc, inv;
    limb_scale(wave_max(m), sc, inv);
#pragma unroll
    for (int i = 0; i < NI; i++)
        if (4 * lane + 256 * i < Kp) ts_put_limbs(xl, 4 * lane + 256 * i, t, v[i], inv);
    return sc;
}

__device__ __forceinline__ float4 ts_ld4(const float* p, int k, int valid) {
    if (k + 4 <= valid) return *(const float4*)(p + k);
    float4 r = {0.0f, 0.0f, 0.0f, 0.0f};
    if (k < valid) r.x = p[k];
    if (k + 1 < valid) r.y = p[k + 1];
    if (k + 2 < valid) r.z = p[k + 2];
    return r;
}

// s1_rms_inv of two rows by one wave, their chains interleaved (the same operations per row).
__device__ __forceinline__ void ts_rms_inv2(const float* x0, const float* x1, int D, int lane, float (&inv)[2]) {
    const int p = lane & 15;
    float part0 = 0.0f, part1 = 0.0f;
    const int c16 = D >> 4;
#pragma unroll 8
    for (int c = 0; c < c16; c++) {
        const float v0 = x0[16 * c + p], v1 = x1[16 * c + p];
        part0 = fmaf(v0, v0, part0);
        part1 = fmaf(v1, v1, part1);
    }
    if (p < 8 && D - 16 * c16 >= 8) {
        const float v0 = x0[16 * c16 + p], v1 = x1[16 * c16 + p];
        part0 = fmaf(v0, v0, part0);
        part1 = fmaf(v1, v1, part1);
    }
    float a8[8], b8[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        a8[q] = lane_value(part0, q) + lane_value(part0, q + 8);
        b8[q] = lane_value(part1, q) + lane_value(part1, q + 8);
    }
    float ss0 = hreduce8(a8), ss1 = hreduce8(b8);
    for (int e = (D >> 3) << 3; e < D; e++) {
        const float t0 = x0[e], t1 = x1[e];
        const float p0 = t0 * t0, p1 = t1 * t1;
        ss0 = ss0 + p0;
        ss1 = ss1 + p1;
    }
    inv[0] = 1.0f / (float)sqrt((double)(ss0 / (float)D + 1e-5f));
    inv[1] = 1.0f / (float)sqrt((double)(ss1 / (float)D + 1e-5f));
}

// Rows w and w + 8 by wave w: with `resid`, first blockIn += cur; cur = blockIn (stream.go:157-163);
// then n = RMSNorm(cur; gamma) (cur itself without gamma; s1_rms_inv, the row kernel's order), kept when
// `keep` is given, and its limb planes (K = Dp). gamma is loaded once for both rows, and the two rows'
// dependent chains are interleaved. keep: the
// n rows' base (row stride ld) or null. sc: the two row scales.
__device__ __forceinline__ void ts_norm_rows(float* cur, float* bin, int ld, bool resid, const float* gamma, int D,
                                             int Dp, float* keep, int8_t* xl, int w, int lane, float (&sc)[2]) {
    float4 gm[TS_NI];
#pragma unroll
    for (int i = 0; i < TS_NI; i++) {
        const int k = 4 * lane + 256 * i;
        gm[i] = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (gamma) {
            if (k + 4 <= D) {
                gm[i] = ldg((const float4*)(gamma + k));
            } else {
#pragma unroll
                for (int u = 0; u < 3; u++)
                    if (k + u < D) (&gm[i].x)[u] = ldg(gamma + k + u);
            }
        }
    }
    const int tr[2] = {w, w + 8};
    if (resid) {
#pragma unroll
        for (int i = 0; i < TS_NI; i++) {
            const int k = 4 * lane + 256 * i;
            if (k < Dp) {
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    float* x = cur + tr[r] * ld + k;
                    float* b = bin + tr[r] * ld + k;
                    const float4 c = *(const float4*)x, bb = *(const float4*)b;
                    const float4 v = {bb.x + c.x, bb.y + c.y, bb.z + c.z, bb.w + c.w};
                    *(float4*)x = v;
                    *(float4*)b = v;
                }
            }
        }
        wave_lds_sync();
    }
    float inv[2] = {1.0f, 1.0f};
    if (gamma) ts_rms_inv2(cur + tr[0] * ld, cur + tr[1] * ld, D, lane, inv);
    float4 v[2][TS_NI];
    float m[2] = {0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int i = 0; i < TS_NI; i++) {
            const int k = 4 * lane + 256 * i;
            float4 u = ts_ld4(cur + tr[r] * ld, k, D);
            if (gamma) {
                u.x = (u.x * inv[r]) * gm[i].x;
                u.y = (u.y * inv[r]) * gm[i].y;
                u.z = (u.z * inv[r]) * gm[i].z;
                u.w = (u.w * inv[r]) * gm[i].w;
            }
            v[r][i] = u;
            if (keep && k < Dp) *(float4*)(keep + tr[r] * ld + k) = u;
            m[r] = ts_amax4(m[r], u);
        }
    const float a0 = wave_max(m[0]), a1 = wave_max(m[1]);
    float ix[2];
    limb_scale(a0, sc[0], ix[0]);
    limb_scale(a1, sc[1], ix[1]);
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
        for (int i = 0; i < TS_NI; i++)
            if (4 * lane + 256 * i < Dp) ts_put_limbs(xl, 4 * lane + 256 * i, tr[r], v[r][i], ix[r]);
}

__global__ __launch_bounds__(TS_THREADS) void tile_step_kernel(TileStepArgs a) {
    extern __shared__ __align__(16) float ts_smem[];
    __shared__ float rsc[TS_NS];  // row scales of the current limb operand
    const int s0 = blockIdx.x * TS_NS, ns = min(TS_NS, a.S - s0);
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (a.done) {
        // a tile whose sessions have all finished (a batched decode's stop tokens) is skipped
        const bool run = lane < ns && a.done[s0 + lane] < 0;
        if (!__any(run)) return;
    }
    const int D = a.D, Dp = a.Dp, H = a.H, Hp = a.Hp, V = a.V, Vp = a.Vp;
    const TsLds L = ts_lds(Dp, Hp, Vp);
    const int ld = L.ld, hld = L.hld;
    float* cur = ts_smem + L.cur;
    float* bin = ts_smem + L.bin;
    float* nrm = ts_smem + L.nrm;
    float* lam = ts_smem + L.lam;
    float* hb = ts_smem + L.h;
    float* tst = ts_smem + L.ts;
    int8_t* xl = (int8_t*)ts_smem + L.xl_off;
    const int kcD = Dp >> 6;

    // A segment that starts with an out projection reads that projection's limb operand and row scales;
    // every row's position (the ring slots of the latch updates, constant through the step) is read here
    // too. These loads are all issued before the state rows' below, and nothing is stored before the
    // last of them has been issued, so the segment's start costs one memory round trip.
    constexpr int TS_AX = 3;  // 16-byte chunks of the limb operand per thread: kcD * 192 <= 1536 (Dp <= 512)
    v4i ax[TS_AX];
    float axs = 0.0f;
    if (a.seg_out) {
        const int8_t* src = a.att_xl + (long long)blockIdx.x * kcD * 3072;
#pragma unroll
        for (int u = 0; u < TS_AX; u++) {
            const int c = tid + TS_THREADS * u;
            ax[u] = c < kcD * 192 ? *(const v4i*)(src + c * 16) : v4i{0, 0, 0, 0};
        }
        if (tid < ns) axs = a.att_xs[s0 + tid];
    }
    int rpos[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = w + 8 * i;
        rpos[i] = __builtin_amdgcn_readfirstlane(a.pos[s0 + (t < ns ? t : 0)]);
    }
    // state rows (each wave its own): the embedding (quant.Model.appendPosition, ids clamped as
    // stream.go:144-146), or the previous segment's cur and blockIn; rows past the set are zero
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = w + 8 * i;
        const bool ok = t < ns;
        int id = 0;
        if (ok && a.seg_block == 0 && !a.seg_out) {
            id = a.ids[s0 + t];
            id = (id < 0 || id >= V) ? 0 : id;
        }
#pragma unroll
        for (int ii = 0; ii < TS_NI; ii++) {
            const int k = 4 * lane + 256 * ii;
            if (k >= Dp) continue;
            float4 c = {0.0f, 0.0f, 0.0f, 0.0f}, bi = c;
            if (ok) {
                if (a.seg_block == 0 && !a.seg_out) {
                    const int8_t* e = a.emb + (long long)id * D;
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        if (k + u < D) (&c.x)[u] = (float)e[k + u] * a.emb_scale;
                    bi = c;
                } else {
                    const long long row = (long long)(s0 + t) * Dp;
                    c = *(const float4*)(a.cur + row + k);
                    bi = *(const float4*)(a.bin + row + k);
                }
            }
            *(float4*)(cur + t * ld + k) = c;
            *(float4*)(bin + t * ld + k) = bi;
        }
    }
    int b = a.seg_block;
    if (a.seg_out) {
        // the out projection of block b, whose attention has run: cur += att.W_o * s (attention.go:100-103)
#pragma unroll
        for (int u = 0; u < TS_AX; u++) {
            const int c = tid + TS_THREADS * u;
            if (c < kcD * 192) *(v4i*)(xl + c * 16) = ax[u];
        }
        if (tid < TS_NS) rsc[tid] = axs;  // zero past the set
        lds_barrier();
        const Step1Block& B = a.blocks[b];
        ts_matvec<TS_FRAG, 4, 2>(B.wo, nullptr, a.NpD / 16, kcD, a.NpD / 16, xl, lane, w, [&](int f, const float (&v)[4], float4) {
            const int c0 = 16 * f + 4 * (lane >> 4), t = lane & 15;
            const float sw = rsc[t] * B.so;
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (c0 + r < D) cur[t * ld + c0 + r] = cur[t * ld + c0 + r] + v[r] * sw;
        });
        b++;
    }
    lds_barrier();
    int bs = 0;  // block steps before block b: the index of its latch state and norm ring
    for (int q = 0; q < b; q++) bs += a.blocks[q].steps;
    for (; b < a.nblocks; b++) {
        const Step1Block& B = a.blocks[b];
        bool resid = b > 0;  // blockIn += cur; cur = blockIn at the block's start, by each row's wave
        if (B.steps == 0 && resid) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int t = w + 8 * i;
#pragma unroll
                for (int ii = 0; ii < TS_NI; ii++) {
                    const int k = 4 * lane + 256 * ii;
                    if (k < Dp) {
                        float* x = cur + t * ld + k;
                        float* bb = bin + t * ld + k;
                        const float4 c = *(const float4*)x, bv = *(const float4*)bb;
                        const float4 v = {bv.x + c.x, bv.y + c.y, bv.z + c.z, bv.w + c.w};
                        *(float4*)x = v;
                        *(float4*)bb = v;
                    }
                }
            }
            resid = false;
            lds_barrier();
        }
        for (int st = 0; st < B.steps; st++, bs++) {
            int dil = B.init_dil;
            for (int q = 0; q < st && dil < 32; q++) dil *= B.dil_base;
            dil = min(dil, 32);
            // n = RMSNorm(cur; gamma) (stream.go:166-171) and its limbs
            {
                float sc[2];
                ts_norm_rows(cur, bin, ld, resid && st == 0, B.gamma, D, Dp, nrm, xl, w, lane, sc);
                if (lane == 0) {
                    rsc[w] = sc[0];
                    rsc[w + 8] = sc[1];
                }
            }
            lds_barrier();
            // lambda = sigmoid_clamped(n.W_sel*s + base) (stream.go:195-205)
            ts_matvec<TS_FRAG, 4, 2>(B.wsel, a.latch_base, a.NpD / 16, kcD, a.NpD / 16, xl, lane, w,
                                     [&](int f, const float (&v)[4], float4 b) {
                const int c0 = 16 * f + 4 * (lane >> 4), t = lane & 15;
                const float sw = rsc[t] * B.ssel;
                const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (c0 + r < D) lam[t * ld + c0 + r] = sigmoid_epi(fmaf(v[r], sw, bb[r]));
            });
            lds_barrier();
            // latch update, norm ring and the rule input [n | left | g] (latch_step_kernel): both rows'
            // memory reads are issued before either row is computed
            {
                float4 gq[2][TS_NI], lq[2][TS_NI];
                int posr[2];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int t = w + 8 * i;
                    const bool ok = t < ns;
                    const int s = s0 + (ok ? t : 0);
                    posr[i] = rpos[i];
                    const float* gbase = a.g + ((long long)bs * a.S + s) * Dp;
                    const float* ring = a.norm_ring + ((long long)bs * a.S + s) * a.ring * Dp;
                    const int p = posr[i];
                    const float* lslot = ring + (long long)((p >= dil ? p - dil : 0) % a.ring) * Dp;
#pragma unroll
                    for (int ii = 0; ii < TS_NI; ii++) {
                        const int k = min(4 * lane + 256 * ii, Dp - 4);
                        gq[i][ii] = ok ? ldg((const float4*)(gbase + k)) : float4{0.0f, 0.0f, 0.0f, 0.0f};
                        lq[i][ii] = ok && p >= dil ? ldg((const float4*)(lslot + k)) : float4{0.0f, 0.0f, 0.0f, 0.0f};
                    }
                }
                float4 nv2[2][TS_NI], lv2[2][TS_NI], gv2[2][TS_NI];
                float m2[2] = {0.0f, 0.0f};
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int t = w + 8 * i;
                    const bool ok = t < ns;
                    const int s = s0 + (ok ? t : 0);
                    const int p = posr[i];
                    float* gbase = a.g + ((long long)bs * a.S + s) * Dp;
                    float* ring = a.norm_ring + ((long long)bs * a.S + s) * a.ring * Dp;
                    float* wslot = ring + (long long)(p % a.ring) * Dp;
                    float4 (&nv)[TS_NI] = nv2[i], (&lv)[TS_NI] = lv2[i], (&gv)[TS_NI] = gv2[i];
                    float& m = m2[i];
#pragma unroll
                    for (int ii = 0; ii < TS_NI; ii++) {
                        const int k = 4 * lane + 256 * ii;
                        float ne[4] = {0.0f, 0.0f, 0.0f, 0.0f}, le[4] = {0.0f, 0.0f, 0.0f, 0.0f},
                              ge[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                        if (ok && k < Dp) {
                            const float4 n4 = *(const float4*)(nrm + t * ld + k), l4 = *(const float4*)(lam + t * ld + k);
                            const float nn[4] = {n4.x, n4.y, n4.z, n4.w}, ll[4] = {l4.x, l4.y, l4.z, l4.w};
                            const float gg[4] = {gq[i][ii].x, gq[i][ii].y, gq[i][ii].z, gq[i][ii].w};
                            const float lf[4] = {lq[i][ii].x, lq[i][ii].y, lq[i][ii].z, lq[i][ii].w};
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                if (k + e < D) {
                                    ne[e] = nn[e];
                                    const float p1 = ll[e] * gg[e];
                                    const float p2 = (1.0f - ll[e]) * nn[e];
                                    ge[e] = p1 + p2;
                                    le[e] = lf[e];
                                }
                            }
                            if (k + 4 <= D) {
                                stg((float4*)(gbase + k), float4{ge[0], ge[1], ge[2], ge[3]});
                                stg((float4*)(wslot + k), float4{ne[0], ne[1], ne[2], ne[3]});
                            } else {
#pragma unroll
                                for (int e = 0; e < 4; e++)
                                    if (k + e < D) {
                                        stg(gbase + k + e, ge[e]);
                                        stg(wslot + k + e, ne[e]);
                                    }
                            }
                        }
                        nv[ii] = float4{ne[0], ne[1], ne[2], ne[3]};
                        lv[ii] = float4{le[0], le[1], le[2], le[3]};
                        gv[ii] = float4{ge[0], ge[1], ge[2], ge[3]};
                        m = ts_amax4(ts_amax4(ts_amax4(m, nv[ii]), lv[ii]), gv[ii]);
                    }
                }
                // both rows' maxima, then their digits
                const float a0 = wave_max(m2[0]), a1 = wave_max(m2[1]);
                float sx[2], ix[2];
                limb_scale(a0, sx[0], ix[0]);
                limb_scale(a1, sx[1], ix[1]);
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int t = w + 8 * i;
#pragma unroll
                    for (int ii = 0; ii < TS_NI; ii++) {
                        const int k = 4 * lane + 256 * ii;
                        if (k < Dp) {
                            ts_put_limbs(xl, k, t, nv2[i][ii], ix[i]);
                            ts_put_limbs(xl, Dp + k, t, lv2[i][ii], ix[i]);
                            ts_put_limbs(xl, 2 * Dp + k, t, gv2[i][ii], ix[i]);
                        }
                    }
                    if (lane == 0) rsc[t] = sx[i];
                }
            }
            lds_barrier();
            // h = GLU(x) (stream.go:214-220): fragment pairs (value 2q, gate 2q + 1)
            ts_matvec<TS_PAIR, 4, 3>(B.w1, B.b1, 2 * Hp / 16, 3 * kcD, Hp / 16, xl, lane, w,
                                     [&](int q, const float (&vv)[4], const float (&vg)[4], float4 bv, float4 bg) {
                const int c0 = 16 * q + 4 * (lane >> 4), t = lane & 15;
                const float sw = rsc[t] * B.s1;
                const float bvv[4] = {bv.x, bv.y, bv.z, bv.w}, bgg[4] = {bg.x, bg.y, bg.z, bg.w};
                float h[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float ov = fmaf(vv[r], sw, bvv[r]);
                    const float gt = sigmoid_epi(fmaf(vg[r], sw, bgg[r]));
                    h[r] = c0 + r < H ? ov * gt : 0.0f;
                }
                *(float4*)(hb + t * hld + c0) = float4{h[0], h[1], h[2], h[3]};
            });
            lds_barrier();
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int t = w + 8 * i;
                float4 v[4];
#pragma unroll
                for (int ii = 0; ii < 4; ii++) v[ii] = ts_ld4(hb + t * hld, 4 * lane + 256 * ii, H);
                const float sc = ts_row_limbs<4>(v, Hp, t, xl, lane);
                if (lane == 0) rsc[t] = sc;
            }
            lds_barrier();
            // cur = highway(cur, W2 h) (stream.go:222-229)
            ts_matvec<TS_PAIR, 4, 2>(B.w2, B.b2, 2 * Dp / 16, Hp / 64, Dp / 16, xl, lane, w,
                                     [&](int q, const float (&vv)[4], const float (&vg)[4], float4 bv, float4 bg) {
                const int c0 = 16 * q + 4 * (lane >> 4), t = lane & 15;
                const float sw = rsc[t] * B.s2;
                const float bvv[4] = {bv.x, bv.y, bv.z, bv.w}, bgg[4] = {bg.x, bg.y, bg.z, bg.w};
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int c = c0 + r;
                    if (c < D) {
                        const float ov = fmaf(vv[r], sw, bvv[r]);
                        const float gt = sigmoid_epi(fmaf(vg[r], sw, bgg[r]));
                        const float x1 = (1.0f - gt) * cur[t * ld + c];
                        const float x2 = gt * ov;
                        cur[t * ld + c] = x1 + x2;
                    }
                }
            });
            lds_barrier();
        }
        if (B.attn) {
            // attendPosition's projection (internal/quant/attention.go:69-80): q, k, v of every session to
            // memory for the attention kernel; cur and blockIn for the next segment
            {
                float sc[2];
                ts_norm_rows(cur, bin, ld, resid && B.steps == 0, B.anorm, D, Dp, nullptr, xl, w, lane, sc);
                if (lane == 0) {
                    rsc[w] = sc[0];
                    rsc[w + 8] = sc[1];
                }
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int t = w + 8 * i;
                if (t < ns) {
                    const long long row = (long long)(s0 + t) * Dp;
#pragma unroll
                    for (int ii = 0; ii < TS_NI; ii++) {
                        const int k = 4 * lane + 256 * ii;
                        if (k < Dp) {
                            *(float4*)(a.cur + row + k) = *(const float4*)(cur + t * ld + k);
                            *(float4*)(a.bin + row + k) = *(const float4*)(bin + t * ld + k);
                        }
                    }
                }
            }
            lds_barrier();
            ts_matvec<TS_FRAG, 6, 2>(B.qkv, nullptr, a.Np3 / 16, kcD, a.Np3 / 16, xl, lane, w,
                                     [&](int f, const float (&v)[4], float4) {
                const int c0 = 16 * f + 4 * (lane >> 4), t = lane & 15;
                const float sw = rsc[t] * B.sqkv;
                if (t < ns) {
                    float* o = a.qkv + (long long)(s0 + t) * 3 * D + c0;
                    if (c0 + 4 <= 3 * D && (D & 3) == 0) {
                        stg((float4*)o, float4{v[0] * sw, v[1] * sw, v[2] * sw, v[3] * sw});
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++)
                            if (c0 + r < 3 * D) o[r] = v[r] * sw;
                    }
                }
            });
            return;
        }
    }
    // headLogits (internal/quant/stream.go:232-248)
    {
        float sc[2];
        ts_norm_rows(cur, bin, ld, false, a.final_norm, D, Dp, nullptr, xl, w, lane, sc);
        if (lane == 0) {
            rsc[w] = sc[0];
            rsc[w + 8] = sc[1];
        }
    }
    lds_barrier();
    // 128-channel tiles of the vocabulary, wave w taking tiles w, w + 8, ...: the logits epilogue's
    // statistics per token (max, sum exp(l - max), first argmax) with its lane structure
    const int ntiles = Vp / LX_BN;
    const bool want_argmax = a.argmax || a.next_ids || a.out_ids;
    const int t = lane & 15, g4 = lane >> 4;
    const float sw = rsc[t] * a.head_scale;
    // K = Dp <= 512 (tile_step_fits; its LDS takes Dp <= 320): within limb_sum_k512's bound
    ts_matvec<TS_TILE, 8, 1>(a.headw, a.headb, Vp / 16, kcD, ntiles, xl, lane, w,
                             [&](int tt, const v4i (&acc)[8][3], const float4 (&b4)[8]) {
        float y[8][4];
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const float bb[4] = {b4[g].x, b4[g].y, b4[g].z, b4[g].w};
#pragma unroll
            for (int r = 0; r < 4; r++) y[g][r] = fmaf(limb_sum_k512(acc[g][0][r], acc[g][1][r], acc[g][2][r]), sw, bb[r]);
        }
        const int nb = tt * LX_BN + 4 * g4;
        if (a.logits && t < ns) {
            float* lo = a.logits + (long long)(s0 + t) * V;
#pragma unroll
            for (int ti = 0; ti < 8; ti++) {
                const int c = nb + 16 * ti;
                if ((V & 3) == 0 && c + 4 <= V) {
                    *(float4*)(lo + c) = float4{y[ti][0], y[ti][1], y[ti][2], y[ti][3]};
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (c + r < V) lo[c + r] = y[ti][r];
                }
            }
        }
        const float l2e = 1.4426950408889634f;
        float mx = y[0][0];
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int r = 0; r < 4; r++) mx = fmaxf(mx, y[ti][r]);
        const float ml = mx == -INFINITY ? 0.0f : mx * l2e;
        float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int r = 0; r < 4; r++) s4[r] += __builtin_amdgcn_exp2f(fmaf(y[ti][r], l2e, -ml));
        float bmax = mx, bsum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        int bidx = 0x7fffffff;
        if (want_argmax && mx > -INFINITY) {
            int off = 0;
#pragma unroll
            for (int ti = 7; ti >= 0; ti--)
#pragma unroll
                for (int r = 3; r >= 0; r--) off = y[ti][r] == mx ? ti * 16 + r : off;
            bidx = nb + off;
        }
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {
            float om = __shfl_xor(bmax, o, 64), os = __shfl_xor(bsum, o, 64);
            int oi = __shfl_xor(bidx, o, 64);
            float nm = fmaxf(bmax, om);
            float ns_ = (bmax == -INFINITY ? 0.0f : bsum * __expf(bmax - nm)) +
                        (om == -INFINITY ? 0.0f : os * __expf(om - nm));
            int ni = (om > bmax) ? oi : (bmax > om) ? bidx : min(bidx, oi);
            bmax = nm; bsum = ns_; bidx = ni;
        }
        if (g4 == 0) {
            float* d = tst + (t * ntiles + tt) * 3;
            d[0] = bmax;
            d[1] = bsum;
            d[2] = __int_as_float(bidx);
        }
    });
    lds_barrier();
    // their combination (head_combine_kernel): 16 lanes per session, waves 0..3
    if (w < 4) {
        const int tk = 4 * w + (lane >> 4), l = lane & 15;
        const float* st = tst + tk * ntiles * 3;
        float bm = -INFINITY, bsm = 0.0f;
        int bi = 0x7fffffff;
        for (int u = l; u < ntiles; u += 16) merge_stats(bm, bsm, bi, st[3 * u], st[3 * u + 1], __float_as_int(st[3 * u + 2]));
#pragma unroll
        for (int o = 8; o >= 1; o >>= 1) {
            const float om = __shfl_xor(bm, o, 16), os = __shfl_xor(bsm, o, 16);
            const int oi = __shfl_xor(bi, o, 16);
            merge_stats(bm, bsm, bi, om, os, oi);
        }
        if (l == 0 && tk < ns) {
            const int s = s0 + tk;
            const double p = 1.0 / (double)bsm;
            if (a.argmax) a.argmax[s] = bi;
            if (a.prob) a.prob[s] = p;
            if (a.next_ids) a.next_ids[s] = bi;
            const int oc = a.col ? *a.col : a.out_col;
            if (a.out_ids) a.out_ids[(long long)s * a.out_ld + oc] = bi;
            if (a.out_probs) a.out_probs[(long long)s * a.out_ld + oc] = p;
            a.pos[s] = a.pos[s] + 1;
        }
    }
}

__global__ __launch_bounds__(256) void head_combine_kernel(HeadCombineArgs a) {
    const int l = threadIdx.x & 15;
    const int m = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int mc = min(m, a.M - 1);
    const float* st = a.stats + (long long)mc * a.ntiles * 3;
    float bm = -INFINITY, bs = 0.0f;
    int bi = 0x7fffffff;
    for (int t = l; t < a.ntiles; t += 16) merge_stats(bm, bs, bi, st[3 * t], st[3 * t + 1], __float_as_int(st[3 * t + 2]));
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) {
        const float om = __shfl_xor(bm, o, 16), os = __shfl_xor(bs, o, 16);
        const int oi = __shfl_xor(bi, o, 16);
        merge_stats(bm, bs, bi, om, os, oi);
    }
    if (l != 0 || m >= a.M) return;
    float lse = bm + logf(bs);
    if (a.lse) a.lse[m] = lse;
    if (a.argmax) a.argmax[m] = bi;
    double p = 1.0 / (double)bs;
    if (a.prob) a.prob[m] = p;
    if (a.logprob) {
        int tg = a.tgt ? a.tgt[m] : -1;
        a.logprob[m] = (tg >= 0 && tg < a.V) ? a.tlog[m] - lse : __int_as_float(0x7fc00000);
    }
    if (a.next_ids) a.next_ids[m] = bi;
    const int oc = a.col ? *a.col : a.out_col;
    if (a.out_ids) a.out_ids[(long long)m * a.out_ld + oc] = bi;
    if (a.out_probs) a.out_probs[(long long)m * a.out_ld + oc] = p;
}

// eval's nll.score accumulates nats in float64 target by target (internal/eval/eval.go:25-48);
// tokenizer.BitsPerByte divides by ln 2 and the count (internal/tokenizer/bytes.go:5-11), with the
// token count in place of bytes. Position t's logits predict ids[t+1].
__global__ void bits_kernel(int B, int T, const float* logprob, const int32_t* ids, int V, float* bits) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    double nats = 0.0;
    int n = 0;
    for (int t = 0; t + 1 < T; t++) {
        int tg = ids[(long long)b * T + t + 1];
        if (tg < 0 || tg >= V) continue;
        nats -= (double)logprob[(long long)b * T + t];
        n++;
    }
    bits[b] = n ? (float)(nats / (0.6931471805599453 * n)) : 0.0f;
}

// ------------------------------------------------------------------------------------------------
// quant.NewTensorF32 (internal/quant/tensor.go:12-42)
// ------------------------------------------------------------------------------------------------
__global__ void absmax_kernel(const float* w, long long n, unsigned* out) {
    float m = 0.0f;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        m = fmaxf(m, fabsf(w[i]));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(m));
}

__global__ void quantize_kernel(const float* w, long long n, int8_t* q, const unsigned* amax_bits, float* scale_out) {
    const float maxAbs = __uint_as_float(*amax_bits);
    const float s = maxAbs / 127.0f;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
        float v = 0.0f;
        if (maxAbs != 0.0f) {
            v = roundf(w[i] / s);  // round half away from zero, like math.Round
            v = fminf(fmaxf(v, -127.0f), 127.0f);
        }
        q[i] = (int8_t)v;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale_out = maxAbs == 0.0f ? 1.0f : s;
}

// ------------------------------------------------------------------------------------------------
// session state export and small helpers
// ------------------------------------------------------------------------------------------------
__global__ void export_ring_kernel(int B, int T, int Dp, int ring, const int32_t* lens, const float* nf, float* nr) {
    const int b = blockIdx.x;
    const int len = lens[b];
    const int p0 = max(0, len - ring);
    for (int p = p0; p < len; p++)
        for (int d = threadIdx.x; d < Dp; d += blockDim.x)
            nr[((long long)b * ring + p % ring) * Dp + d] = nf[((long long)b * T + p) * Dp + d];
}

// The rings are head-major, [session][head][slot][dh], so that a decode step's key and value rows of one
// head are one contiguous block.
__global__ void export_kv_kernel(int B, int T, int D, int heads, int cap, const int32_t* lens, const float* qkv,
                                 float* kr, float* vr) {
    const int b = blockIdx.x;
    const int len = min(max(lens[b], 0), T);
    const int p0 = max(0, len - cap);
    const int dh = D / heads;
    for (int p = p0; p < len; p++)
        for (int d = threadIdx.x; d < D; d += blockDim.x) {
            const float* row = qkv + ((long long)b * T + p) * 3 * D;
            const int h = d / dh;
            const long long o = (((long long)b * heads + h) * cap + p % cap) * dh + (d - h * dh);
            kr[o] = row[D + d];
            vr[o] = row[2 * D + d];
        }
}

// export_kv_kernel into packed rings: one wave per position at a time (four per workgroup, one workgroup
// per sequence). The wave stages the position's key and value rows [k | v] in LDS with coalesced 16-byte
// loads, finds each (head, key or value) row's exponent (kv_exp of its largest magnitude), and packs one
// group of four per lane (kv_pack, as rk_head packs a decode step's row).
__host__ __device__ inline int export_kv_wave_floats(int D, int heads) { return 2 * D + ((2 * heads + 3) & ~3); }

__global__ __launch_bounds__(256) void export_kv_packed_kernel(int B, int T, int D, int heads, int cap,
                                                               const int32_t* lens, const float* qkv, uint32_t* kpack,
                                                               uint32_t* vpack, float* kscale, float* vscale) {
    extern __shared__ __align__(16) float ex_smem[];
    const int b = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int len = min(max(lens[b], 0), T);
    const int p0 = max(0, len - cap);
    const int dh = D / heads, c4 = dh / 4, nc = D / 2;  // float4 chunks of [k | v]
    float* xw = ex_smem + w * export_kv_wave_floats(D, heads);
    int* ew = (int*)(xw + 2 * D);  // [2 heads] row exponents: rows 0..heads-1 keys, heads..2heads-1 values
    for (int p = p0 + w; p < len; p += 4) {
        const float* src = qkv + ((long long)b * T + p) * 3 * D + D;  // k then v, 2D floats
        for (int c = lane; c < nc; c += 64) *(float4*)(xw + 4 * c) = ldg((const float4*)(src + 4 * c));
        wave_lds_sync();
        for (int r = lane; r < 2 * heads; r += 64) {
            float am = 0.0f;
            for (int d = 0; d < dh; d++) am = fmaxf(am, fabsf(xw[r * dh + d]));
            ew[r] = kv_exp(am);
        }
        wave_lds_sync();
        for (int c = lane; c < nc; c += 64) {
            const int r = c / c4, g = c - r * c4;
            const int part = r >= heads, h = r - part * heads, e = ew[r];
            const long long row = ((long long)b * heads + h) * cap + p % cap;
            stg_pk3((Pk3*)(part ? vpack : kpack) + row * c4 + g, kv_pack(*(const float4*)(xw + 4 * c), e));
            if (g == 0) stg((part ? vscale : kscale) + row, ldexpf(1.0f, e));
        }
        wave_lds_sync();  // the wave's buffer takes the next position
    }
}

// The same where a row's C4 = dh/4 groups (a power of two up to 16) sit on an aligned quad, half-row or
// row of lanes: one lane per group of [k | v] (a wave takes 64 groups at a time, whole rows), the row's
// largest magnitude by DPP moves, no LDS. Same rows and bytes as export_kv_packed_kernel.
template <int C4>
__global__ __launch_bounds__(256) void export_kv_packed_dpp_kernel(int B, int T, int D, int heads, int cap,
                                                                   const int32_t* lens, const float* qkv,
                                                                   uint32_t* kpack, uint32_t* vpack, float* kscale,
                                                                   float* vscale) {
    const int b = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int len = min(max(lens[b], 0), T);
    const int p0 = max(0, len - cap);
    const int nc = D / 2;                        // groups of [k | v] per position
    const int per = (nc + 63) / 64;              // 64-lane passes per position
    for (int it = w; it < (len - p0) * per; it += 4) {
        const int p = p0 + it / per, c = (it % per) * 64 + lane;
        const bool ok = c < nc;
        const float4 x = ldg((const float4*)(qkv + ((long long)b * T + p) * 3 * D + D + 4 * min(c, nc - 1)));
        float m = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
        if constexpr (C4 >= 2) m = fmaxf(m, dpp_move<0xB1>(m));   // quad_perm [1, 0, 3, 2]
        if constexpr (C4 >= 4) m = fmaxf(m, dpp_move<0x4E>(m));   // quad_perm [2, 3, 0, 1]
        if constexpr (C4 >= 8) m = fmaxf(m, dpp_move<0x141>(m));  // row_half_mirror
        if constexpr (C4 >= 16) m = fmaxf(m, dpp_move<0x140>(m)); // row_mirror
        if (ok) {
            const int r = c / C4, g = c % C4;  // row r: keys 0..heads-1, then values
            const int part = r >= heads, h = r - part * heads, e = kv_exp(m);
            const long long row = ((long long)b * heads + h) * cap + p % cap;
            stg_pk3((Pk3*)(part ? vpack : kpack) + row * C4 + g, kv_pack(x, e));
            if (g == 0) stg((part ? vscale : kscale) + row, ldexpf(1.0f, e));
        }
    }
}

__global__ void set_pos_kernel(int S, const int32_t* lens, int32_t* pos, int add, int32_t* col) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < S) pos[i] = (lens ? lens[i] : pos[i]) + add;
    if (i == 0 && col) *col += 1;
}

__global__ void fill_i32_kernel(int32_t* p, int n, int v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void fill_f32_kernel(float* p, long long n, float v) {
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
        p[i] = v;
}

// LDS bytes of attention_kernel: the staged rows of a 64-query tile's window and the scores.
size_t attn_exact_lds(const AttnArgs& a, int dh) {
    const int stride = dh % 4 == 0 ? dh + 4 : dh + 1;
    return (size_t)((ATT_QT + a.cap - 1) * stride + a.cap * 64) * sizeof(float);
}

template <int DH>
hipError_t attn_t(const AttnArgs& a, hipStream_t s) {
    const int nqt = (a.T + ATT_QT - 1) / ATT_QT;
    const size_t lds = attn_exact_lds(a, DH);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    static const hipError_t attr = hipFuncSetAttribute((const void*)attention_kernel<DH>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(attention_kernel<DH>, dim3(a.B * nqt, a.heads), dim3(64), lds, s, a);
    return hipGetLastError();
}

template <int ND, int NKB, int G>
hipError_t attn_mfma_g(const AttnArgs& a, int dh, hipStream_t s) {
    const int qtiles = (a.T + 15) / 16;
    const int groups = (qtiles + G - 1) / G;
    constexpr int KEYS = 16 * (NKB + G - 1), DP = 16 * ND;
    constexpr size_t lds = sizeof(float) * std::max(KEYS * (DP + 4), DP * (KEYS + 4));
    static const hipError_t attr = hipFuncSetAttribute((const void*)attention_mfma_kernel<ND, NKB, G>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((attention_mfma_kernel<ND, NKB, G>), dim3(a.B * groups, a.heads), dim3(64 * G), lds, s, a,
                       dh);
    return hipGetLastError();
}

// Eight query tiles per workgroup where sequences have at least six, four from three, two for sequences of
// one or two tiles (a wave past the sequence's last tile computes a tile that is never stored: with four
// per workgroup, half of a 32-token prefill's waves did).
template <int ND, int NKB>
hipError_t attn_mfma_t(const AttnArgs& a, int dh, hipStream_t s) {
    const int qtiles = (a.T + 15) / 16;
    if (qtiles >= 6) return attn_mfma_g<ND, NKB, 8>(a, dh, s);
    return qtiles >= 3 ? attn_mfma_g<ND, NKB, 4>(a, dh, s) : attn_mfma_g<ND, NKB, 2>(a, dh, s);
}

// Key blocks per 16-query tile: the widest span any query attends is W = min(window, cap) keys, so the
// tile's keys fit in 1 + ceil((W - 1)/16) blocks of 16 (at most 17 variants' worth: spans up to 257
// keys). The kernel keeps every block's scores in registers, so it runs where ND*NKB <= 20 (head width up
// to 64 with spans up to 64 keys, narrower heads with longer spans) and for widths 68..128 with spans up
// to 64 keys; other shapes take the reference-order kernels.
int attn_mfma_blocks(const AttnArgs& a) {
    const int W = a.window > 0 ? std::min(a.window, a.cap) : a.cap;
    const int nkb = 1 + (W - 1 + 15) / 16;
    return nkb <= 3 ? 3 : nkb <= 5 ? 5 : nkb <= 9 ? 9 : nkb <= 17 ? 17 : 0;  // 0: longer than any variant
}
int attn_mfma_nd(int dh) { return dh <= 16 ? 1 : dh <= 32 ? 2 : dh <= 64 ? 4 : dh <= 80 ? 5 : dh <= 96 ? 6 : 8; }
bool attn_mfma_fits(const AttnArgs& a, int dh) {
    if (dh % 4 || dh > 128) return false;
    const int nd = attn_mfma_nd(dh), nkb = attn_mfma_blocks(a);
    if (nkb == 0) return false;
    return nd <= 4 ? nd * nkb <= 20 : nkb <= 5;  // widths past 64: windows of up to 64 keys
}

hipError_t attn_mfma(const AttnArgs& a, int dh, hipStream_t s) {
    switch (attn_mfma_nd(dh) * 100 + attn_mfma_blocks(a)) {
        case 103: return attn_mfma_t<1, 3>(a, dh, s);
        case 105: return attn_mfma_t<1, 5>(a, dh, s);
        case 109: return attn_mfma_t<1, 9>(a, dh, s);
        case 117: return attn_mfma_t<1, 17>(a, dh, s);
        case 203: return attn_mfma_t<2, 3>(a, dh, s);
        case 205: return attn_mfma_t<2, 5>(a, dh, s);
        case 209: return attn_mfma_t<2, 9>(a, dh, s);
        case 403: return attn_mfma_t<4, 3>(a, dh, s);
        case 405: return attn_mfma_t<4, 5>(a, dh, s);
        case 503: return attn_mfma_t<5, 3>(a, dh, s);
        case 505: return attn_mfma_t<5, 5>(a, dh, s);
        case 603: return attn_mfma_t<6, 3>(a, dh, s);
        case 605: return attn_mfma_t<6, 5>(a, dh, s);
        case 803: return attn_mfma_t<8, 3>(a, dh, s);
        case 805: return attn_mfma_t<8, 5>(a, dh, s);
        default: return hipErrorInvalidValue;
    }
}

// Compute units of the current device (cached per device).
int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus[dev] = 256;
    return cus[dev];
}

// Sequences per workgroup of the fused attention (one workgroup per CU at a time: 139 KiB of LDS).
// Around B*heads/2048 runs (long enough to amortise the slab copy, several workgroups per CU), chosen so
// that the workgroups fill whole rounds of the CUs: a last round that occupies a few CUs keeps the rest
// idle for a whole run (c5's 8192-sequence passes: 24 sequences per run made 8.02 rounds, 32 make 6;
// 21.6 -> 18.0 ms per step). Ties go to the length nearest the target, then the longer one.
int qkv_run_length(int B, int heads) {
    const int cus = device_cus();
    const int r0 = std::max(1, std::min(32, B * heads / 2048));
    int best = r0;
    double best_eff = -1.0;
    for (int R = std::max(1, r0 / 2); R <= std::min(64, 2 * r0); R++) {
        const double rounds = (double)heads * ((B + R - 1) / R) / cus;
        const double eff = rounds / std::ceil(rounds);
        const bool better = eff > best_eff + 1e-9 ||
                            (eff > best_eff - 1e-9 && (std::abs(R - r0) < std::abs(best - r0) ||
                                                       (std::abs(R - r0) == std::abs(best - r0) && R > best)));
        if (better) {
            best = R;
            best_eff = std::max(best_eff, eff);
        }
    }
    return best;
}

template <int ND, int NKB, int KC>
hipError_t qkv_attn_t(const QkvAttnArgs& a, hipStream_t s) {
    constexpr int G = 8, DP = 16 * ND, KEYS = 16 * (NKB + G - 1), ZROWS = 16 * (NKB - 1);
    constexpr size_t lds = (size_t)KC * 3 * ND * 1024 + sizeof(float) * ((KEYS - ZROWS) * (DP + 4) + DP * (KEYS + 4 - ZROWS));
    static const hipError_t attr = hipFuncSetAttribute((const void*)qkv_attention_kernel<ND, NKB, KC>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    const int R = qkv_run_length(a.B, a.heads);
    const int n_runs = (a.B + R - 1) / R;
    const int grid = 8 * a.heads * ((n_runs + 7) / 8);
    hipLaunchKernelGGL((qkv_attention_kernel<ND, NKB, KC>), dim3(grid), dim3(512), lds, s, a, R, n_runs);
    return hipGetLastError();
}

template <int ND, int NKB>
hipError_t qkv_attn_k(const QkvAttnArgs& a, hipStream_t s) {
    switch (a.Dp / 64) {
        case 2: return qkv_attn_t<ND, NKB, 2>(a, s);
        case 4: return qkv_attn_t<ND, NKB, 4>(a, s);
        default: return qkv_attn_t<ND, NKB, 6>(a, s);
    }
}

template <int DH>
hipError_t attn_step_t(const AttnStepArgs& a, hipStream_t s) {
    if constexpr (DH % 4 == 0 && DH <= 64) {
        if (a.cap <= 64) {
            const bool pk = a.kpack != nullptr;
            const size_t lds = (size_t)rk_lds_floats(a.cap, DH, pk) * sizeof(float);
            if (pk) hipLaunchKernelGGL((attention_step_rk_kernel<DH, true>), dim3(a.S * a.heads), dim3(64), lds, s, a);
            else hipLaunchKernelGGL((attention_step_rk_kernel<DH, false>), dim3(a.S * a.heads), dim3(64), lds, s, a);
            return hipGetLastError();
        }
    }
    if (a.kpack) return hipErrorInvalidValue;  // packed rings: the kernels above only
    if constexpr (DH % 4 == 0) {
        const size_t lds = ((size_t)2 * a.cap * (DH + 4) + a.cap) * sizeof(float);
        if (lds <= 64 * 1024) {
            hipLaunchKernelGGL(attention_step_lds_kernel<DH>, dim3(a.S * a.heads), dim3(64), lds, s, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL(attention_step_kernel<DH>, dim3(a.S * a.heads), dim3(64), 0, s, a);
    return hipGetLastError();
}

// One attention block's packed K/V rings (words and scales) in bytes: decode attention streams them,
// without keeping them cached, from this size on, which is the Infinity Cache's (256 MiB). Below it the
// rings of a step can stay cached until the next step reads them again (a chat set's rings, 157 MB:
// 9.3 ms per batch with cached loads against 9.7 streamed, A/B on one box; c4's, 419 MB: 30.86 ms against
// 29.79).
constexpr double kStreamRingBytes = 256.0 * 1024 * 1024;
inline double kv_ring_bytes(const AttnStepArgs& a) {
    return 2.0 * a.S * a.heads * a.cap * (3.0 * (a.D / a.heads) + 4.0);
}

template <int DH>
hipError_t attn_step_rows_t(const AttnStepArgs& a, hipStream_t s) {
    if constexpr (DH % 4 == 0 && DH <= 64) {
        const bool pk = a.kpack != nullptr;
        const size_t lds = (size_t)a.heads * rk_lds_floats(a.cap, DH, pk) * sizeof(float);
        static const hipError_t attr = hipFuncSetAttribute((const void*)attention_step_rows_kernel<DH, false>,
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                                           (int)kStepRowsMaxLds);
        static const hipError_t attr_pk = hipFuncSetAttribute((const void*)attention_step_rows_kernel<DH, true>,
                                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                                              (int)kStepRowsMaxLds);
        if (attr != hipSuccess) return attr;
        if (attr_pk != hipSuccess) return attr_pk;
        const bool st = a.stream_rings > 0 || (a.stream_rings < 0 && kv_ring_bytes(a) >= kStreamRingBytes);
        if (pk && DH <= 32 && st) {
            static const hipError_t attr_st = hipFuncSetAttribute(
                (const void*)attention_step_rows_kernel<DH, true, true>, hipFuncAttributeMaxDynamicSharedMemorySize,
                (int)kStepRowsMaxLds);
            if (attr_st != hipSuccess) return attr_st;
            hipLaunchKernelGGL((attention_step_rows_kernel<DH, true, true>), dim3(a.S), dim3(64 * a.heads), lds, s, a);
        } else if (pk) {
            hipLaunchKernelGGL((attention_step_rows_kernel<DH, true>), dim3(a.S), dim3(64 * a.heads), lds, s, a);
        } else {
            hipLaunchKernelGGL((attention_step_rows_kernel<DH, false>), dim3(a.S), dim3(64 * a.heads), lds, s, a);
        }
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

template <int NS4>
hipError_t row_t(const RowArgs& a, hipStream_t s) {
    const int tiles = (a.M + ROW_TILE - 1) / ROW_TILE;
    const size_t lds = (a.limbs ? (size_t)(a.Dp / 64) * 3 * 1088 : 0) +
                       (a.gamma ? (size_t)4 * row_batch<NS4>() * (a.Dp + 16) * sizeof(float) : 0);
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)row_kernel<NS4>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(row_kernel<NS4>, dim3(tiles), dim3(256), lds, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_row(const RowArgs& a, hipStream_t s) {
    if (a.M <= 0) return hipSuccess;
    if (a.Dp % 64 || a.Dp < 64 || a.Dp > 3072) return hipErrorInvalidValue;
    if (a.mode == ROW_RULE && (a.seg % 64 || 3 * a.seg != a.Dp || a.gamma || a.nout || a.T < 1 || a.dil < 0))
        return hipErrorInvalidValue;
    switch ((a.Dp + 255) / 256) {
        case 1: return row_t<1>(a, s);
        case 2: return row_t<2>(a, s);
        case 3: return row_t<3>(a, s);
        case 4: return row_t<4>(a, s);
        case 5: return row_t<5>(a, s);
        case 6: return row_t<6>(a, s);
        case 7: return row_t<7>(a, s);
        case 8: return row_t<8>(a, s);
        case 9: return row_t<9>(a, s);
        case 10: return row_t<10>(a, s);
        case 11: return row_t<11>(a, s);
        default: return row_t<12>(a, s);
    }
}

hipError_t launch_scan(const ScanArgs& a, hipStream_t s) {
    if (a.B <= 0) return hipSuccess;
    if (a.Dp % 64 || a.Dp > 1024 || a.D < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(scan_kernel, dim3(a.B), dim3(a.Dp), 0, s, a);
    return hipGetLastError();
}

bool scan_rule_fits(int T, int Dp, int dil) { return T % 16 == 0 && Dp % 64 == 0 && Dp <= 1024 && dil >= 1 && dil <= 48; }

hipError_t launch_scan_rule(const ScanArgs& a, hipStream_t s) {
    if (!scan_rule_fits(a.T, a.Dp, a.dil) || a.D > a.Dp) return hipErrorInvalidValue;
    if (a.B == 0 || a.T == 0) return hipSuccess;
    const int threads = ((a.Dp / 2 + 63) / 64) * 64;
    const size_t lds = (size_t)(a.Dp / 64) * 3 * 1088 + (2 * (threads / 64) * 16 + 64 + 16 + 16) * sizeof(float);
    if ((a.xn != nullptr) != (a.rinv != nullptr) || (a.xn != nullptr) != (a.gamma != nullptr) || (!a.xn && !a.nf))
        return hipErrorInvalidValue;
    if (a.xn) hipLaunchKernelGGL(scan_rule_kernel<true>, dim3(a.B), dim3(threads), lds, s, a);
    else hipLaunchKernelGGL(scan_rule_kernel<false>, dim3(a.B), dim3(threads), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_latch_step(const LatchStepArgs& a, hipStream_t s) {
    if (a.S <= 0) return hipSuccess;
    if (a.Dp % 64 || a.Dp > 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(latch_step_kernel, dim3(a.S), dim3(a.Dp), 0, s, a);
    return hipGetLastError();
}

#define DH_SWITCH(dh, FN, ...)                \
    switch (dh) {                             \
        case 1: return FN<1>(__VA_ARGS__);     \
        case 2: return FN<2>(__VA_ARGS__);     \
        case 4: return FN<4>(__VA_ARGS__);     \
        case 8: return FN<8>(__VA_ARGS__);     \
        case 12: return FN<12>(__VA_ARGS__);   \
        case 20: return FN<20>(__VA_ARGS__);   \
        case 40: return FN<40>(__VA_ARGS__);   \
        case 80: return FN<80>(__VA_ARGS__);   \
        case 16: return FN<16>(__VA_ARGS__);   \
        case 24: return FN<24>(__VA_ARGS__);   \
        case 32: return FN<32>(__VA_ARGS__);   \
        case 48: return FN<48>(__VA_ARGS__);   \
        case 64: return FN<64>(__VA_ARGS__);   \
        case 96: return FN<96>(__VA_ARGS__);   \
        case 128: return FN<128>(__VA_ARGS__); \
        default: return hipErrorInvalidValue; \
    }

// Head widths with instantiated width-specific kernels (DH_SWITCH).
bool dh_compiled(int dh) {
    switch (dh) {
        case 1: case 2: case 4: case 8: case 12: case 16: case 20: case 24: case 32: case 40: case 48: case 64:
        case 80: case 96: case 128: return true;
        default: return false;
    }
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
    if (a.B <= 0 || a.T <= 0) return hipSuccess;
    if (a.heads <= 0 || a.D % a.heads || a.cap <= 0) return hipErrorInvalidValue;
    const int dh = a.D / a.heads;
    const int mode = option(OPT_ATTENTION_KERNEL);
    if (mode != ATTN_EXACT && attn_mfma_fits(a, dh)) return attn_mfma(a, dh, s);
    if (dh_compiled(dh) && attn_exact_lds(a, dh) <= 160 * 1024) DH_SWITCH(dh, attn_t, a, s)
    AttnWaveArgs w;
    w.rows = a.B * a.T; w.T = a.T; w.D = a.D; w.Dp = a.Dp; w.heads = a.heads; w.dh = dh;
    w.window = a.window; w.cap = a.cap; w.qkv = a.qkv; w.att = a.att;
    return launch_attention_wave(w, s);
}

bool qkv_attention_fits(const QkvAttnArgs& a) {
    if (a.heads <= 0 || a.D % a.heads || a.T != 128 || a.cap <= 0) return false;
    const int dh = a.D / a.heads;
    if ((dh != 32 && dh != 64) || (a.Dp != 128 && a.Dp != 256 && a.Dp != 384) || a.Np3 % 16) return false;
    AttnArgs t;
    t.T = a.T; t.window = a.window; t.cap = a.cap;
    const int nkb = attn_mfma_blocks(t);
    return dh == 32 ? (nkb == 3 || nkb == 5 || nkb == 9) : (nkb == 3 || nkb == 5);
}

hipError_t launch_qkv_attention(const QkvAttnArgs& a, hipStream_t s) {
    if (a.B <= 0) return hipSuccess;
    if (!qkv_attention_fits(a)) return hipErrorInvalidValue;
    AttnArgs t;
    t.T = a.T; t.window = a.window; t.cap = a.cap;
    const int nkb = attn_mfma_blocks(t), dh = a.D / a.heads;
    switch ((dh / 16) * 100 + nkb) {
        case 203: return qkv_attn_k<2, 3>(a, s);
        case 205: return qkv_attn_k<2, 5>(a, s);
        case 209: return qkv_attn_k<2, 9>(a, s);
        case 403: return qkv_attn_k<4, 3>(a, s);
        default: return qkv_attn_k<4, 5>(a, s);
    }
}

bool attention_step_rows_fits(const AttnStepArgs& a) {
    if (a.heads <= 0 || a.heads > 16 || a.D % a.heads) return false;
    const int dh = a.D / a.heads;
    if (dh % 4 || dh > 64 || a.cap > 64 || a.Dp % 64) return false;
    switch (dh) {  // the widths DH_SWITCH instantiates
        case 4: case 8: case 12: case 16: case 20: case 24: case 32: case 40: case 48: case 64: break;
        default: return false;
    }
    // sized for packed rings (the larger of the two layouts), so that a set's ring format, chosen by this
    // fit, never depends on it
    return (size_t)a.heads * rk_lds_floats(a.cap, dh, true) * sizeof(float) <= kStepRowsMaxLds;
}

hipError_t launch_attention_step_rows(const AttnStepArgs& a, hipStream_t s) {
    if (a.S <= 0) return hipSuccess;
    if (!attention_step_rows_fits(a) || !a.xl || !a.xs) return hipErrorInvalidValue;
    if (a.kpack && (!a.vpack || !a.kscale || !a.vscale)) return hipErrorInvalidValue;
    DH_SWITCH(a.D / a.heads, attn_step_rows_t, a, s)
}

hipError_t launch_attention_step(const AttnStepArgs& a, hipStream_t s) {
    if (a.S <= 0) return hipSuccess;
    if (a.heads <= 0 || a.D % a.heads || a.cap <= 0) return hipErrorInvalidValue;
    const int dh = a.D / a.heads;
    if (a.kpack && (!a.vpack || !a.kscale || !a.vscale)) return hipErrorInvalidValue;
    if (dh_compiled(dh) && a.cap <= 256) DH_SWITCH(dh, attn_step_t, a, s)
    if (a.kpack) return hipErrorInvalidValue;  // packed rings: attention_step_rk_kernel's shapes only
    AttnWaveArgs w;
    w.rows = a.S; w.D = a.D; w.Dp = a.Dp; w.heads = a.heads; w.dh = dh; w.window = a.window; w.cap = a.cap;
    w.step = true; w.qkv = a.qkv; w.pos = a.pos; w.kring = a.kring; w.vring = a.vring; w.att = a.att;
    return launch_attention_wave(w, s);
}

template <int NC>
hipError_t attn_wave_t(const AttnWaveArgs& a, int span_max, hipStream_t s) {
    const size_t lds = (size_t)wave_lds_floats(span_max) * sizeof(float);
    static const hipError_t attr = hipFuncSetAttribute((const void*)attention_wave_kernel<NC>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(attention_wave_kernel<NC>, dim3(a.rows, a.heads), dim3(64), lds, s, a);
    return hipGetLastError();
}

hipError_t launch_attention_wave(const AttnWaveArgs& a, hipStream_t s) {
    if (a.rows <= 0) return hipSuccess;
    if (a.heads <= 0 || a.dh <= 0 || a.dh > kMaxHeadWidth || a.D != a.heads * a.dh || a.cap <= 0 || a.T <= 0)
        return hipErrorInvalidValue;
    if (a.step ? (!a.pos || !a.kring || !a.vring) : a.rows % a.T) return hipErrorInvalidValue;
    // the widest span a query attends: min(window, cap) keys, and at most T in a batch
    int span_max = a.window > 0 ? std::min(a.window, a.cap) : a.cap;
    if (!a.step) span_max = std::min(span_max, a.T);
    if (span_max > kMaxAttnSpan) return hipErrorInvalidValue;
    const int nc = (a.dh + 15) / 16;
    if (nc <= 1) return attn_wave_t<1>(a, span_max, s);
    if (nc <= 2) return attn_wave_t<2>(a, span_max, s);
    if (nc <= 4) return attn_wave_t<4>(a, span_max, s);
    if (nc <= 8) return attn_wave_t<8>(a, span_max, s);
    if (nc <= 16) return attn_wave_t<16>(a, span_max, s);
    if (nc <= 32) return attn_wave_t<32>(a, span_max, s);
    return attn_wave_t<64>(a, span_max, s);
}

size_t step1_lds_bytes(const Step1Args& a, int dh) {
    const size_t floats = (size_t)8 * a.Dp + a.Hp + a.Vp + 4 * (a.Vp / LX_BN) +
                          (size_t)a.heads * ((rk_lds_floats(a.cap, dh) + 3) & ~3);
    const size_t xl = (size_t)(std::max(3 * a.Dp, a.Hp) / 64) * 3072;  // limb operand, MFMA fragment layout
    return floats * sizeof(float) + xl;
}

bool step1_fits(const Step1Args& a) {
    if (a.S <= 0 || a.D > 512 || a.Dp > 512 || a.Hp > 1024 || a.Vp > 16384 || a.nblocks <= 0) return false;
    const int dh = a.heads > 0 ? a.D / a.heads : 16;
    if (a.heads > 0 && (a.heads > S1_THREADS / 64 || a.D % a.heads || (dh != 16 && dh != 32 && dh != 64) ||
                        a.cap > 64 || a.cap <= 0))
        return false;
    return step1_lds_bytes(a, dh) <= 150 * 1024;
}

template <int DH, bool PK>
hipError_t step1_pk_t(const Step1Args& a, hipStream_t s) {
    const size_t lds = step1_lds_bytes(a, DH);
    static const hipError_t attr = hipFuncSetAttribute((const void*)step1_kernel<DH, PK>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((step1_kernel<DH, PK>), dim3(a.S), dim3(S1_THREADS), lds, s, a);
    return hipGetLastError();
}

template <int DH>
hipError_t step1_t(const Step1Args& a, hipStream_t s) {
    return a.kpack ? step1_pk_t<DH, true>(a, s) : step1_pk_t<DH, false>(a, s);
}

bool tile_step_fits(const TileStepArgs& a) {
    if (a.S <= 0 || a.nblocks <= 0 || a.D > 512 || a.Dp > 512 || a.Hp > 1024 || a.Dp % 64 || a.Hp % 64 || a.Vp % LX_BN)
        return false;
    return (size_t)ts_lds(a.Dp, a.Hp, a.Vp).bytes <= kTileStepMaxLds;
}

hipError_t launch_tile_step(const TileStepArgs& a, hipStream_t s) {
    if (!tile_step_fits(a)) return hipErrorInvalidValue;
    static const hipError_t attr = hipFuncSetAttribute((const void*)tile_step_kernel,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kTileStepMaxLds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(tile_step_kernel, dim3((a.S + TS_NS - 1) / TS_NS), dim3(TS_THREADS),
                       (size_t)ts_lds(a.Dp, a.Hp, a.Vp).bytes, s, a);
    return hipGetLastError();
}

hipError_t launch_step1(const Step1Args& a, hipStream_t s) {
    if (!step1_fits(a)) return hipErrorInvalidValue;
    switch (a.heads > 0 ? a.D / a.heads : 16) {
        case 16: return step1_t<16>(a, s);
        case 32: return step1_t<32>(a, s);
        default: return step1_t<64>(a, s);
    }
}

hipError_t launch_head_combine(const HeadCombineArgs& a, hipStream_t s) {
    if (a.M <= 0) return hipSuccess;
    hipLaunchKernelGGL(head_combine_kernel, dim3((a.M + 15) / 16), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_bits(int B, int T, const float* logprob, const int32_t* ids, int V, float* bits, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    hipLaunchKernelGGL(bits_kernel, dim3((B + 255) / 256), dim3(256), 0, s, B, T, logprob, ids, V, bits);
    return hipGetLastError();
}

hipError_t launch_quantize(const float* w, long long n, int8_t* q, float* scale, float* amax_tmp, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    unsigned* am = (unsigned*)amax_tmp;
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, s, (int32_t*)am, 1, 0);
    long long blocks = (n + 255) / 256;
    int g = (int)(blocks < 4096 ? blocks : 4096);
    hipLaunchKernelGGL(absmax_kernel, dim3(g), dim3(256), 0, s, w, n, am);
    hipLaunchKernelGGL(quantize_kernel, dim3(g), dim3(256), 0, s, w, n, q, am, scale);
    return hipGetLastError();
}

hipError_t launch_export_ring(int B, int T, int Dp, int ring, const int32_t* lens, const float* nf, float* norm_ring,
                              hipStream_t s) {
    if (B <= 0) return hipSuccess;
    hipLaunchKernelGGL(export_ring_kernel, dim3(B), dim3(256), 0, s, B, T, Dp, ring, lens, nf, norm_ring);
    return hipGetLastError();
}

hipError_t launch_export_kv(int B, int T, int D, int heads, int cap, const int32_t* lens, const float* qkv,
                            float* kring, float* vring, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    if (heads <= 0 || D % heads != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(export_kv_kernel, dim3(B), dim3(256), 0, s, B, T, D, heads, cap, lens, qkv, kring, vring);
    return hipGetLastError();
}

hipError_t launch_export_kv_packed(int B, int T, int D, int heads, int cap, const int32_t* lens, const float* qkv,
                                   uint32_t* kpack, uint32_t* vpack, float* kscale, float* vscale, hipStream_t s) {
    if (B <= 0) return hipSuccess;
    if (heads <= 0 || D % heads != 0 || (D / heads) % 4) return hipErrorInvalidValue;
    if (D > 1024) return hipErrorInvalidValue;
    switch (D / heads / 4) {
#define MG_EXPORT_DPP(C)                                                                                        \
    case C:                                                                                                     \
        hipLaunchKernelGGL(export_kv_packed_dpp_kernel<C>, dim3(B), dim3(256), 0, s, B, T, D, heads, cap, lens, qkv, \
                           kpack, vpack, kscale, vscale);                                                       \
        return hipGetLastError();
        MG_EXPORT_DPP(1)
        MG_EXPORT_DPP(2)
        MG_EXPORT_DPP(4)
        MG_EXPORT_DPP(8)
        MG_EXPORT_DPP(16)
#undef MG_EXPORT_DPP
        default: break;
    }
    const size_t lds = (size_t)4 * export_kv_wave_floats(D, heads) * sizeof(float);
    hipLaunchKernelGGL(export_kv_packed_kernel, dim3(B), dim3(256), lds, s, B, T, D, heads, cap, lens, qkv, kpack,
                       vpack, kscale, vscale);
    return hipGetLastError();
}

hipError_t launch_set_pos(int S, const int32_t* lens, int32_t* pos, int add, hipStream_t s, int32_t* col) {
    if (S <= 0) return hipSuccess;
    hipLaunchKernelGGL(set_pos_kernel, dim3((S + 255) / 256), dim3(256), 0, s, S, lens, pos, add, col);
    return hipGetLastError();
}

__global__ void advance_kernel(int32_t* p) { *p += 1; }

hipError_t launch_advance(int32_t* p, hipStream_t s) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_fill_i32(int32_t* p, int n, int v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_i32_kernel, dim3((n + 255) / 256), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

hipError_t launch_fill_f32(float* p, long long n, float v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    long long blocks = (n + 255) / 256;
    int g = (int)(blocks < 8192 ? blocks : 8192);
    hipLaunchKernelGGL(fill_f32_kernel, dim3(g), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

}  // namespace mg
