// Int8 MFMA GEMMs for gfx950 (v_mfma_i32_16x16x64_i8) with the engine's fused epilogues.
//
// Orientation: the MFMA row operand is the weight matrix (output channels) and the column operand the
// activations (tokens), so lane L of a 16x16 accumulator tile holds token (L & 15) and four consecutive
// channels 4*(L >> 4) + r. Each lane therefore owns whole per-token quantities (one activation scale,
// one output row), and its four results are contiguous in the token-major output.
//
// Limb-expanded GEMM (gemm_lx_kernel): fp32 activations arrive as three int8 digit planes with one scale
// per token (x ~= s*(q0 + q1/254 + q2/254^2)); each plane has its own exact int32 accumulator and the
// three are combined in fp32 once, in the epilogue. Workgroup = 4 waves = 128 channels x 64 tokens;
// each wave owns 16 tokens and all 128 channels (8 MFMA tiles x 3 planes), two workgroups per CU. The
// weight tile of a K step (8 KiB) is shared through double-buffered LDS; activation fragments, three
// times the bytes, go straight from global memory (L2) into registers one K step ahead, so LDS carries
// only weights.
//
// Plain int8 GEMM (gemm_c2_kernel, config 2): row-major operands, 4 waves in a 2 x 2 grid, both
// operands staged through LDS with an 80-byte row stride (conflict-free 16-byte fragment reads).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "gemm.hpp"
#include "options.hpp"

namespace mg {

namespace {

typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store4(float* dst, const float v[4], int nvalid_here, bool aligned) {
    if (nvalid_here >= 4 && aligned) {
        *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        for (int r = 0; r < 4 && r < nvalid_here; r++) dst[r] = v[r];
    }
}

// Epilogue of one wave's 16-token x 128-channel tile (first token mt0, channel tile n_tile).
//
// The three digit-plane sums of tile ti, register r combine into the fp32 dot product
// x.w = s*(P0 + P1/254 + P2/254^2) times the weight scale; s*wscale is one factor per token, and a
// bias is added with the same FMA. Token of this lane: mt0 + (L & 15); channel of (ti, r):
// n0 + 16ti + 4*(L >> 4) + r. Kept lean: for K = 384 the epilogue's VALU work is comparable to the
// MFMA work of the whole tile.
// B256: the digits are base 256 (an fp32 operand expanded as it is loaded, digits256_4).
// K512: K is at most 512 (the head GEMMs): limb_sum_k512.
template <bool B256 = false, bool K512 = false>
__device__ __forceinline__ float limb_dot(const v4i (&acc)[3][8], int ti, int r) {
    if constexpr (K512) return limb_sum_k512(acc[0][ti][r], acc[1][ti][r], acc[2][ti][r]);
    if constexpr (B256)
        return fmaf((float)acc[2][ti][r], kInvLimb256_2, fmaf((float)acc[1][ti][r], kInvLimb256_1, (float)acc[0][ti][r]));
    return fmaf((float)acc[2][ti][r], kInvLimb2, fmaf((float)acc[1][ti][r], kInvLimb1, (float)acc[0][ti][r]));
}

// Per-token values the epilogue needs, loaded when the tile starts so that their latency hides behind
// the tile's MFMAs.
// (Only loads here: any arithmetic on a loaded value would make the compiler wait for it at once.)
struct EpiRow {
    float s = 0.0f;   // activation scale (times the weight scale in the epilogue)
    int tgt = -1;     // EPI_LOGITS: target id
    float lse = 0.0f; // EPI_PROBS: log-sum-exp
};

template <int EPI>
__device__ __forceinline__ EpiRow epi_row(const GemmArgs& g, int m) {
    EpiRow e;
    const int mm = min(m, g.M - 1);  // rows past M are never stored; their values are not used
    e.s = g.As[mm];
    if constexpr (EPI == EPI_LOGITS) {
        if (g.tgt) e.tgt = g.tgt[mm];
    }
    if constexpr (EPI == EPI_PROBS) e.lse = g.lse[mm];
    return e;
}

// Staged output (STG): a wave's 16 x 128 fp32 output tile is written to its LDS region (row stride
// STG_LD floats: rows start 4 banks apart, so the 16 rows of one column group hit distinct banks) and
// then stored as rows, two 512-byte row segments per store instruction, instead of sixteen 64-byte
// pieces: far fewer cache lines per instruction for the address unit.
constexpr int STG_LD = 132;
constexpr int STG_BYTES = 8 * 16 * STG_LD * 4;  // eight waves

__device__ __forceinline__ void stg_put(float* stg, int lane, int ti, const float v[4]) {
    *(float4*)(stg + (lane & 15) * STG_LD + 16 * ti + 4 * (lane >> 4)) = make_float4(v[0], v[1], v[2], v[3]);
}

// Rows mt0..mt0+15, channels n0 + [0, 128) of `out` (row stride ldo) from the staged tile, as whole
// 512-byte row segments. Store kinds: ST_PLAIN; ST_NT non-temporal, for outputs far larger than the L2
// that the next kernel reads back from memory in any case; ST_STREAM non-temporal with both coherence
// scope bits set (sc0 sc1 nt). Chosen per output by measurement: the probabilities take ST_STREAM (21.0 ms
// per c5 step against 22.0 with ST_NT and 23.7 with ST_PLAIN); the logits (0.291 ms per c3 launch
// against 0.308 with ST_STREAM) and the config-2 GEMM take ST_NT.
enum StoreKind : int { ST_PLAIN = 0, ST_NT = 1, ST_STREAM = 2 };

template <int SK = ST_PLAIN>
__device__ __forceinline__ void stg_flush(const GemmArgs& g, const float* stg, int lane, int mt0, int n0, float* out,
                                          long long ldo) {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes have landed
    __builtin_amdgcn_wave_barrier();
    const int c = 4 * (lane & 31);
    const int nv = g.nvalid - n0 - c;  // valid channels from this lane's column on
    const bool vec = nv >= 4 && (ldo & 3) == 0;
    // row mt0 + (L >> 5) + 2k: a wave-uniform base plus a per-lane offset that is the same for every
    // tile (no per-row 64-bit multiplies)
    float* const base = out + (long long)mt0 * ldo + n0;
    const long long loff = (long long)(lane >> 5) * ldo + c;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int row = (lane >> 5) + 2 * k;
        const int m = mt0 + row;
        const float4 v = *(const float4*)(stg + row * STG_LD + c);
        if (m < g.M && nv > 0) {
            float* dst = base + 2 * k * ldo + loff;
            if (vec) {
                if constexpr (SK == ST_STREAM) {
                    // The compiler does not see what an asm statement is, so it does not add the wait state
                    // a store of more than 8 bytes needs before a VALU instruction may overwrite its data
                    // registers: the s_nop is that wait (a schedule that reused the data registers for the
                    // next row's address right after the store wrote address bits into the output).
                    const f4v t = {v.x, v.y, v.z, v.w};
                    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1 nt\n\ts_nop 1" ::"v"(dst), "v"(t) : "memory");
                } else if constexpr (SK == ST_NT) {
                    const f4v t = {v.x, v.y, v.z, v.w};
                    __builtin_nontemporal_store(t, (f4v*)dst);
                } else {
                    *(float4*)dst = v;
                }
            } else {
                const float t[4] = {v.x, v.y, v.z, v.w};
                for (int r = 0; r < 4 && r < nv; r++) dst[r] = t[r];
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
}

// The next block's RMSNorm statistics of four new blockIn values at channels ch.. (nv of them valid): their
// sum of squares and their largest |v * gamma_next|, accumulated per lane.
__device__ __forceinline__ void block_stats(const GemmArgs& g, int ch, const float v[4], int nv, float& ssq,
                                            float& mxg) {
    const float4 gm = *(const float4*)(g.gamma_next + ch);  // gamma is padded to a multiple of 64 columns
    const float gg[4] = {gm.x, gm.y, gm.z, gm.w};
#pragma unroll
    for (int r = 0; r < 4; r++) {
        if (r < nv) {
            ssq = fmaf(v[r], v[r], ssq);
            mxg = fmaxf(mxg, fabsf(v[r] * gg[r]));
        }
    }
}
// A row's statistics over the tile: the four lane groups of a token combine, the first writes.
__device__ __forceinline__ void stats_out(const GemmArgs& g, int m, int n_tile, int lane, float ssq, float mxg) {
    ssq += __shfl_xor(ssq, 16, 64);
    ssq += __shfl_xor(ssq, 32, 64);
    mxg = fmaxf(mxg, __shfl_xor(mxg, 16, 64));
    mxg = fmaxf(mxg, __shfl_xor(mxg, 32, 64));
    if (lane < 16) {
        g.ssq_out[(long long)m * g.stat_ld + n_tile] = ssq;
        g.mxg_out[(long long)m * g.stat_ld + n_tile] = mxg;
    }
}

// bias_t: the bias of this tile's 128 channels (global memory, or the workgroup's LDS copy).
// STG: outputs of EPI_F32, EPI_LATCH, EPI_PROBS and EPI_LOGITS go through the wave's LDS region `stg`.
template <int EPI, bool STG = false, bool B256 = false, bool K512 = false>
__device__ __forceinline__ void lx_epilogue(const GemmArgs& g, const v4i (&acc)[3][8], int mt0, int n0, int n_tile,
                                            int lane, const EpiRow& row, const float* bias_t, float* stg = nullptr) {
    const int g4 = lane >> 4;
    const int m = mt0 + (lane & 15);
    const bool mok = m < g.M;
    const float sw = row.s * g.wscale;
    const int nb = n0 + 4 * g4;
    const bool vec = (g.ldo & 3) == 0;

    if constexpr (EPI == EPI_F32 || EPI == EPI_LATCH) {
        if (!STG && !mok) return;
        float* orow = g.out + (long long)m * g.ldo;
#pragma unroll
        for (int ti = 0; ti < 8; ti++) {
            const int n = nb + ti * 16;
            const int nv = g.nvalid - n;
            if (!STG && nv <= 0) continue;
            float v[4];
            if constexpr (EPI == EPI_LATCH) {
                const float4 b = *(const float4*)(bias_t + 4 * g4 + ti * 16);
                const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = sigmoid_epi(fmaf(limb_dot<B256>(acc, ti, r), sw, bb[r]));
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = limb_dot<B256>(acc, ti, r) * sw;
            }
            if constexpr (STG) stg_put(stg, lane, ti, v);
            else store4(orow + n, v, nv, vec);
        }
        if constexpr (STG) stg_flush<ST_NT>(g, stg, lane, mt0, n0, g.out, g.ldo);
    } else if constexpr (EPI == EPI_RESID) {
        // cur += x.w: all eight row segments are loaded before any is needed (one memory latency). With
        // resid, the new state is added into resid instead (blockIn += cur) and cur is left as it was.
        if (!mok) return;
        const long long ro = (long long)m * g.ldcur;
        const float* crow = (g.cur_in ? g.cur_in : g.cur) + ro;
        float* orow = g.resid ? g.resid + ro : g.cur + ro;
        const bool cvec = (g.ldcur & 3) == 0;
        float c[8][4], rs[8][4];
#pragma unroll
        for (int ti = 0; ti < 8; ti++) {
            const int n = nb + ti * 16;
            const int nv = g.nvalid - n;
            if (nv >= 4 && cvec) {
                const float4 t = *(const float4*)(crow + n);
                c[ti][0] = t.x; c[ti][1] = t.y; c[ti][2] = t.z; c[ti][3] = t.w;
                if (g.resid) {
                    const float4 u = *(const float4*)(orow + n);
                    rs[ti][0] = u.x; rs[ti][1] = u.y; rs[ti][2] = u.z; rs[ti][3] = u.w;
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    c[ti][r] = r < nv ? crow[n + r] : 0.0f;
                    if (g.resid) rs[ti][r] = r < nv ? orow[n + r] : 0.0f;
                }
            }
        }
        float ssq = 0.0f, mxg = 0.0f;  // the next block's RMSNorm statistics of the new blockIn values
#pragma unroll
        for (int ti = 0; ti < 8; ti++) {
            const int n = nb + ti * 16;
            const int nv = g.nvalid - n;
            if (nv <= 0) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = c[ti][r] + limb_dot<B256>(acc, ti, r) * sw;
            if (g.resid) {
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = rs[ti][r] + v[r];  // blockIn += cur (stream.go:157-163)
            }
            store4(orow + n, v, nv, cvec);
            if (g.ssq_out) block_stats(g, n, v, nv, ssq, mxg);
        }
        if (g.ssq_out) stats_out(g, m, n_tile, lane, ssq, mxg);
    } else if constexpr (EPI == EPI_PROBS) {
        // p = exp(l - lse) = 2^(x.w*log2e + (b - lse)*log2e)
        if (!STG && !mok) return;
        const float l2e = 1.4426950408889634f;
        const float swl = sw * l2e, lsel = row.lse * l2e;
        float* orow = g.out + (long long)m * g.ldo;
#pragma unroll
        for (int ti = 0; ti < 8; ti++) {
            const int n = nb + ti * 16;
            const int nv = g.nvalid - n;
            if (!STG && nv <= 0) continue;
            const float4 b = *(const float4*)(bias_t + 4 * g4 + ti * 16);
            const float bb[4] = {b.x, b.y, b.z, b.w};
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = __builtin_amdgcn_exp2f(fmaf(limb_dot<B256, K512>(acc, ti, r), swl, fmaf(bb[r], l2e, -lsel)));
            if constexpr (STG) stg_put(stg, lane, ti, v);
            else store4(orow + n, v, nv, vec);
        }
        if constexpr (STG) stg_flush<ST_STREAM>(g, stg, lane, mt0, n0, g.out, g.ldo);
    } else if constexpr (EPI == EPI_GLU || EPI == EPI_HIGHWAY) {
        // W rows are reordered in blocks of 32: 16 value rows then the 16 matching gate rows, so tile
        // pair (2p, 2p+1) holds value and gate of output channel n0/2 + 16p + 4*(L >> 4) + r.
        if (!mok) return;
        float c[4][4], rs[4][4];
        const float* crow = nullptr;
        float* wrow = nullptr;
        const bool cvec = (g.ldcur & 3) == 0;
        if constexpr (EPI == EPI_HIGHWAY) {
            // the four cur segments this lane updates (and, with resid, the four it adds into), loaded
            // together
            const long long ro = (long long)m * g.ldcur;
            crow = (g.cur_in ? g.cur_in : g.cur) + ro;
            wrow = g.resid ? g.resid + ro : g.cur + ro;
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int ch = n0 / 2 + p * 16 + 4 * g4;
                const int nv = g.nvalid - ch;
                if (nv >= 4 && cvec) {
                    const float4 t = *(const float4*)(crow + ch);
                    c[p][0] = t.x; c[p][1] = t.y; c[p][2] = t.z; c[p][3] = t.w;
                    if (g.resid) {
                        const float4 u = *(const float4*)(wrow + ch);
                        rs[p][0] = u.x; rs[p][1] = u.y; rs[p][2] = u.z; rs[p][3] = u.w;
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        c[p][r] = r < nv ? crow[ch + r] : 0.0f;
                        if (g.resid) rs[p][r] = r < nv ? wrow[ch + r] : 0.0f;
                    }
                }
            }
        }
        float* orow = g.out + (long long)m * g.ldo;
        float hm = 0.0f;  // EPI_GLU: the largest |h| of this lane's outputs
        float ssq = 0.0f, mxg = 0.0f;  // EPI_HIGHWAY into blockIn: the next block's RMSNorm statistics
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int ch = n0 / 2 + p * 16 + 4 * g4;
            const int nv = g.nvalid - ch;
            if (nv <= 0) continue;
            const int rv = 32 * p + 4 * g4;  // value rows rv..rv+3, gate rows rv+16.. within the tile
            const float4 bv = *(const float4*)(bias_t + rv), bg = *(const float4*)(bias_t + rv + 16);
            const float bvv[4] = {bv.x, bv.y, bv.z, bv.w}, bgg[4] = {bg.x, bg.y, bg.z, bg.w};
            float ov[4], gt[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                ov[r] = fmaf(limb_dot<B256>(acc, 2 * p, r), sw, bvv[r]);
                gt[r] = sigmoid_epi(fmaf(limb_dot<B256>(acc, 2 * p + 1, r), sw, bgg[r]));
            }
            float v[4];
            if constexpr (EPI == EPI_GLU) {
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = ov[r] * gt[r];  // mlpHidden *= sigmoid(gate) (stream.go:218-220)
                if (g.amax_out) {
                    // fragment order: the four channels are consecutive there too (one 16-byte store;
                    // padding channels hold the zeros their zero weights and bias give)
                    *(float4*)(g.out + frag_off_f32(m, ch, g.Np >> 7)) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
                    store4(orow + ch, v, nv, vec);
                }
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (r < nv) hm = fmaxf(hm, fabsf(v[r]));
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float a = (1.0f - gt[r]) * c[p][r];  // highway (stream.go:226-229)
                    const float b = gt[r] * ov[r];
                    v[r] = a + b;
                }
                if (g.resid) {
#pragma unroll
                    for (int r = 0; r < 4; r++) v[r] = rs[p][r] + v[r];  // blockIn += cur (stream.go:157-163)
                }
                store4(wrow + ch, v, nv, cvec);
                if (g.ssq_out) block_stats(g, ch, v, nv, ssq, mxg);
            }
        }
        if constexpr (EPI == EPI_HIGHWAY) {
            if (g.ssq_out) stats_out(g, m, n_tile, lane, ssq, mxg);
        }
        if constexpr (EPI == EPI_GLU) {
            // the row's partial maximum over this tile's 64 outputs: the four lane groups of a token combine
            if (g.amax_out) {
                hm = fmaxf(hm, __shfl_xor(hm, 16, 64));
                hm = fmaxf(hm, __shfl_xor(hm, 32, 64));
                if (g4 == 0) g.amax_out[(long long)m * g.amax_out_ld + n_tile] = hm;
            }
        }
    } else if constexpr (EPI == EPI_LOGITS) {
        // Logits of this lane's 32 channels (vocabulary padding has bias -inf and zero weights, so its
        // logits are -inf): their max, then the sum of exp(l - max) and the first channel holding the max.
        // Two passes over registers: no running rescale, and the argmax only when it is wanted.
        const float l2e = 1.4426950408889634f;
        float* orow = g.out ? g.out + (long long)m * g.ldo : nullptr;
        float y[8][4];
#pragma unroll
        for (int ti = 0; ti < 8; ti++) {
            const int n = nb + ti * 16;
            const float4 b = *(const float4*)(bias_t + 4 * g4 + ti * 16);
            const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int r = 0; r < 4; r++) y[ti][r] = fmaf(limb_dot<B256, K512>(acc, ti, r), sw, bb[r]);
            if constexpr (STG) {
                if (orow) stg_put(stg, lane, ti, y[ti]);
            } else if (orow && mok) {
                const int nv = g.nvalid - n;
                if (nv > 0) store4(orow + n, y[ti], nv, vec);
            }
        }
        // the target logit of each token row: from the staged tile, one lane per row, when the logits are
        // staged for their stores; otherwise the lane holding it selects it without branches (cheaper than
        // staging the tile for one value per row: c5's statistics pass 17.2 -> 16.9 ms)
        if (g.tgt) {
            if (STG && orow) {
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the staged tile has landed
                __builtin_amdgcn_wave_barrier();
                const int t0 = row.tgt - n0;
                if (lane < 16 && mok && t0 >= 0 && t0 < LX_BN) g.tlog[m] = stg[lane * STG_LD + t0];
            } else {
                const int t = row.tgt - nb;  // the target's position among this lane's channels
                float tv = 0.0f;
#pragma unroll
                for (int ti = 0; ti < 8; ti++)
#pragma unroll
                    for (int r = 0; r < 4; r++) tv = t == ti * 16 + r ? y[ti][r] : tv;
                if (mok && t >= 0 && t < LX_BN && (t & 12) == 0) g.tlog[m] = tv;
            }
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
        if (g.want_argmax && mx > -INFINITY) {
            // channels rise with (ti, r): scanning downwards, the last hit is the first index (kept as the
            // offset 16ti + r, a literal, and turned into a channel once)
            int off = 0;
#pragma unroll
            for (int ti = 7; ti >= 0; ti--)
#pragma unroll
                for (int r = 3; r >= 0; r--) off = y[ti][r] == mx ? ti * 16 + r : off;
            bidx = nb + off;
        }
        // the four lane groups interleave channels: combine, the smaller index wins ties
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
        if (mok && g4 == 0) {
            float* dst = g.stats + ((long long)m * g.stats_ld + n_tile) * 3;
            dst[0] = bmax; dst[1] = bsum; dst[2] = __int_as_float(bidx);
        }
        if constexpr (STG) {
            if (orow) stg_flush<ST_NT>(g, stg, lane, mt0, n0, g.out, g.ldo);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Limb-expanded GEMM
// ------------------------------------------------------------------------------------------------
// Two waves per SIMD (96 accumulator registers each): while one wave runs its epilogue or waits on a
// barrier or a load, the other's MFMAs keep the matrix unit busy.
template <int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_lx_kernel(GemmArgs g) {
    __shared__ __align__(16) int8_t Ws[2][8 * 1024];

    const int nt = g.Np / LX_BN;
    const int mt = (g.M + LX_BM - 1) / LX_BM;
    const int total = nt * mt;
    const int t = xcd_tile(blockIdx.x, total);
    if (t >= total) return;
    const int m0 = (t / nt) * LX_BM;
    const int n_tile = t % nt;
    const int n0 = n_tile * LX_BN;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int kc = g.Kp >> 6;

    // weight tile of K step ks: 8 KiB contiguous at wbase + ks*wstep
    const int8_t* wbase = g.W + (long long)(n0 >> 4) * 1024 + tid * 16;
    const long long wstep = (long long)(g.Np >> 4) * 1024;
    // activation fragments of this wave's 16-token tile: limb l of K step ks at abase + (ks*3 + l) KiB
    const int mtile = (m0 + w * 16) >> 4;
    const int8_t* abase = g.A + ((long long)mtile * kc * 3) * 1024 + lane * 16;

    v4i acc[3][8];
#pragma unroll
    for (int l = 0; l < 3; l++)
#pragma unroll
        for (int ti = 0; ti < 8; ti++) acc[l][ti] = v4i{0, 0, 0, 0};
    const EpiRow row = epi_row<EPI>(g, m0 + w * 16 + (lane & 15));

    v4i wreg0, wreg1, acur[3], anext[3];
    wreg0 = *(const v4i*)(wbase);
    wreg1 = *(const v4i*)(wbase + 4096);
#pragma unroll
    for (int l = 0; l < 3; l++) acur[l] = *(const v4i*)(abase + l * 1024);
    *(v4i*)(&Ws[0][tid * 16]) = wreg0;
    *(v4i*)(&Ws[0][4096 + tid * 16]) = wreg1;
    // Drain the prologue loads here: otherwise the in-order vmcnt bookkeeping carried into the loop
    // makes the first MFMA of every K step wait for that step's own prefetches.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int ks = 0; ks < kc; ks++) {
        const int buf = ks & 1;
        const bool more = ks + 1 < kc;
        if (more) {
            const int8_t* wp = wbase + (ks + 1) * wstep;
            wreg0 = *(const v4i*)(wp);
            wreg1 = *(const v4i*)(wp + 4096);
            const long long ao = (long long)(ks + 1) * 3 * 1024;
#pragma unroll
            for (int l = 0; l < 3; l++) anext[l] = *(const v4i*)(abase + ao + l * 1024);
        }
        // all eight weight fragments of the step are requested at once; the MFMAs of fragment ti then
        // only wait for the first ti+1 reads
        v4i wf[8];
#pragma unroll
        for (int ti = 0; ti < 8; ti++) wf[ti] = *(const v4i*)(&Ws[buf][ti * 1024 + lane * 16]);
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int l = 0; l < 3; l++)
                acc[l][ti] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ti], acur[l], acc[l][ti], 0, 0, 0);
        // keep the eight LDS reads ahead of the MFMAs (the default schedule funnels them through one
        // register quad with a full LDS wait before every few MFMAs)
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 24, 0);
        if (more) {
            *(v4i*)(&Ws[buf ^ 1][tid * 16]) = wreg0;
            *(v4i*)(&Ws[buf ^ 1][4096 + tid * 16]) = wreg1;
#pragma unroll
            for (int l = 0; l < 3; l++) acur[l] = anext[l];
        }
        __syncthreads();
    }

    // the head's GEMMs (logits, probabilities) over K <= 512 combine the digit planes with limb_sum_k512,
    // in this kernel and the weight-stationary one alike
    if constexpr (EPI == EPI_LOGITS || EPI == EPI_PROBS) {
        if (kc <= 8) {
            lx_epilogue<EPI, false, false, true>(g, acc, m0 + w * 16, n0, n_tile, lane, row, g.bias ? g.bias + n0 : nullptr);
            return;
        }
    }
    lx_epilogue<EPI>(g, acc, m0 + w * 16, n0, n_tile, lane, row, g.bias ? g.bias + n0 : nullptr);
}

// ------------------------------------------------------------------------------------------------
// Weight-stationary limb-expanded GEMM
// ------------------------------------------------------------------------------------------------
// A workgroup of 8 waves copies one 128-channel weight slab (all K steps, kc*8 KiB) and its bias into
// LDS once, then streams a run of token tiles through it: wave w takes 16-token tiles t_begin + w,
// + 8, ... of the run. After the slab load there is no barrier: each wave reads weight fragments from
// the read-only slab and its own activation fragments straight from global memory, two K steps ahead
// (three register sets, rotated by unrolling the K loop by three). The prefetch runs across tiles: the
// last two K steps of a tile fetch the first two steps of the wave's next tile, before the epilogue's
// stores. REM = kc % 3 (3 for kc == 2) fixes at compile time where those land. Two waves per SIMD: one wave's epilogue
// overlaps the other's MFMAs.
//
// Block b -> (XCD b % 8, slot b / 8); slot -> (channel slab slot % nt, run (slot / nt)*8 + XCD), so all
// slabs of a run execute on one XCD and its activations are fetched from HBM into that XCD's L2 once.
template <int EPI, int REM, bool STG, int KCF = 0>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_slab_kernel(GemmArgs g,
                                                                                                   int run_tiles,
                                                                                                   int n_runs) {
    extern __shared__ __align__(16) int8_t slab[];
    const int nt = g.Np / LX_BN;
    const int slot = blockIdx.x >> 3;
    const int n_tile = slot % nt;
    const int run = (slot / nt) * 8 + (blockIdx.x & 7);
    if (run >= n_runs) return;
    const int n0 = n_tile * LX_BN;
    // the wave index, in a scalar register: tile indices and every address derived from them stay scalar
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kc = g.Kp >> 6;
    float* bias_s = (float*)(slab + kc * 8192);
    float* stg = STG ? (float*)(slab + kc * 8192 + LX_BN * 4) + w * 16 * STG_LD : nullptr;

    {
        // slab[ks][ti][1 KiB] <- W fragments (ks, n0/16 + ti): 8 KiB contiguous per K step
        const int8_t* src = g.W + (long long)(n0 >> 4) * 1024;
        const long long wstep = (long long)(g.Np >> 4) * 1024;
        const int chunks = kc * 512;  // 16-byte chunks, 512 per K step
#pragma unroll 4
        for (int c = tid; c < chunks; c += 512)
            *(v4i*)(slab + ((long long)c << 4)) = *(const v4i*)(src + (c >> 9) * wstep + ((c & 511) << 4));
        if (tid < LX_BN) bias_s[tid] = g.bias ? g.bias[n0 + tid] : 0.0f;
    }
    __syncthreads();

    const int mtiles = (g.M + 15) >> 4;
    const int t_begin = run * run_tiles;
    const int t_end = min(t_begin + run_tiles, mtiles);
    int tile = t_begin + w;
    if (tile >= t_end) return;
    const int8_t* wlane = slab + lane * 16;
    const long long astep = 3 * 1024;  // one K step of one tile: three limb fragments
    const long long tstep = (long long)kc * astep;

    const int8_t* ap = g.A + (long long)tile * tstep + lane * 16;
    if constexpr (KCF > 0) {
        // Short K (kc == KCF): the whole next tile's A fragments are loaded right after this tile's
        // MFMAs, before its outputs are stored. Loads and stores share one in-order completion counter,
        // so no load the MFMAs wait for is ever queued behind a tile's stores.
        v4i a[KCF][3];
#pragma unroll
        for (int ks = 0; ks < KCF; ks++)
#pragma unroll
            for (int l = 0; l < 3; l++) a[ks][l] = *(const v4i*)(ap + ks * astep + l * 1024);
        for (;;) {
            const EpiRow row = epi_row<EPI>(g, tile * 16 + (lane & 15));
            const int next = tile + 8;
            const int8_t* np = next < t_end ? ap + 8 * tstep : ap;
            v4i acc[3][8];
#pragma unroll
            for (int ks = 0; ks < KCF; ks++) {
                v4i wf[8];
                const int8_t* wp = wlane + ks * 8192;
#pragma unroll
                for (int ti = 0; ti < 8; ti++) wf[ti] = *(const v4i*)(wp + ti * 1024);
#pragma unroll
                for (int ti = 0; ti < 8; ti++)
#pragma unroll
                    for (int l = 0; l < 3; l++)
                        acc[l][ti] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ti], a[ks][l],
                                                                           ks == 0 ? v4i{0, 0, 0, 0} : acc[l][ti], 0, 0, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 24, 0);
            }
#pragma unroll
            for (int ks = 0; ks < KCF; ks++)
#pragma unroll
                for (int l = 0; l < 3; l++) a[ks][l] = *(const v4i*)(np + ks * astep + l * 1024);
            lx_epilogue<EPI, STG, false, EPI == EPI_LOGITS || EPI == EPI_PROBS>(g, acc, tile * 16, n0, n_tile, lane,
                                                                                row, bias_s, stg);  // K <= 384
            if (next >= t_end) break;
            tile = next;
            ap = np;
        }
        return;
    }
    v4i a0[3], a1[3], a2[3];
#pragma unroll
    for (int l = 0; l < 3; l++) a0[l] = *(const v4i*)(ap + l * 1024);
#pragma unroll
    for (int l = 0; l < 3; l++) a1[l] = *(const v4i*)(ap + astep + l * 1024);  // kc >= 2

    for (;;) {
        const EpiRow row = epi_row<EPI>(g, tile * 16 + (lane & 15));
        // the next tile's fragments (this tile's again when there is none: harmless, in bounds)
        const int next = tile + 8;
        const int8_t* np = next < t_end ? ap + 8 * tstep : ap;
        v4i acc[3][8];
        // One K step: multiply step ks held in `cur` (the first step of a tile starts from zero); with
        // PF, first prefetch step ks+2 (of this tile, or of the next) into `nxt`. Every path issues the
        // same loads in the same order, so the compiler's in-order load counting lets each step wait
        // only for the loads two steps back.
        auto step = [&](int ks, v4i (&cur)[3], v4i (&nxt)[3], auto pf, auto first) {
            if constexpr (decltype(pf)::value) {
                const int8_t* src = ks + 2 < kc ? ap + (ks + 2) * astep : np + (ks + 2 - kc) * astep;
#pragma unroll
                for (int l = 0; l < 3; l++) nxt[l] = *(const v4i*)(src + l * 1024);
            }
            v4i wf[8];
            const int8_t* wp = wlane + ks * 8192;
#pragma unroll
            for (int ti = 0; ti < 8; ti++) wf[ti] = *(const v4i*)(wp + ti * 1024);
#pragma unroll
            for (int ti = 0; ti < 8; ti++)
#pragma unroll
                for (int l = 0; l < 3; l++)
                    acc[l][ti] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        wf[ti], cur[l], decltype(first)::value ? v4i{0, 0, 0, 0} : acc[l][ti], 0, 0, 0);
            // order: the step's global prefetches, its eight LDS reads, then the MFMAs
            if constexpr (decltype(pf)::value) __builtin_amdgcn_sched_group_barrier(0x020, 3, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 24, 0);
        };
        constexpr std::true_type YES{};
        constexpr std::false_type NO{};
        if constexpr (REM == 3) {
            // kc == 2: a2 is free, and a0 once step 0 is done
            step(0, a0, a2, NO, YES);
#pragma unroll
            for (int l = 0; l < 3; l++) a0[l] = *(const v4i*)(np + l * 1024);
#pragma unroll
            for (int l = 0; l < 3; l++) a2[l] = *(const v4i*)(np + astep + l * 1024);
            step(1, a1, a0, NO, NO);
        } else {
            step(0, a0, a2, YES, YES);  // kc >= 3
            step(1, a1, a0, YES, NO);
            step(2, a2, a1, YES, NO);
            int ks = 3;
            for (; ks + 3 <= kc; ks += 3) {
                step(ks, a0, a2, YES, NO);
                step(ks + 1, a1, a0, YES, NO);
                step(ks + 2, a2, a1, YES, NO);
            }
            if constexpr (REM == 1) step(ks, a0, a2, YES, NO);
            if constexpr (REM == 2) {
                // a0 (after this step) and a2 are free for the next tile's first two steps
                step(ks, a0, a2, NO, NO);
#pragma unroll
                for (int l = 0; l < 3; l++) a0[l] = *(const v4i*)(np + l * 1024);
#pragma unroll
                for (int l = 0; l < 3; l++) a2[l] = *(const v4i*)(np + astep + l * 1024);
                step(ks + 1, a1, a0, NO, NO);
            }
        }
        constexpr bool HEAD = EPI == EPI_LOGITS || EPI == EPI_PROBS;
        if (HEAD && kc <= 8)
            lx_epilogue<EPI, STG, false, HEAD>(g, acc, tile * 16, n0, n_tile, lane, row, bias_s, stg);
        else
            lx_epilogue<EPI, STG>(g, acc, tile * 16, n0, n_tile, lane, row, bias_s, stg);
        if (next >= t_end) break;
        tile = next;
        ap = np;
        // where the next tile's steps 0 and 1 arrived: (a0, a1), (a1, a2) or (a0, a2) for REM 0, 1, 2 (3)
        if constexpr (REM == 1) {
#pragma unroll
            for (int l = 0; l < 3; l++) { a0[l] = a1[l]; a1[l] = a2[l]; }
        } else if constexpr (REM >= 2) {
#pragma unroll
            for (int l = 0; l < 3; l++) a1[l] = a2[l];
        }
    }
}

// Epilogues whose outputs go through the wave's LDS staging region
template <int EPI>
constexpr bool can_stage() { return EPI == EPI_F32 || EPI == EPI_LATCH || EPI == EPI_PROBS || EPI == EPI_LOGITS; }

// ------------------------------------------------------------------------------------------------
// Weight-stationary GEMM on an fp32 operand
// ------------------------------------------------------------------------------------------------
// gemm_slab_kernel's structure (the channel slab in LDS, runs of tiles per workgroup, 8 waves, two per
// SIMD, the same block-to-XCD mapping) with the activations read as fp32, so that no separate pass writes
// their limb planes. Lane L loads the 16 consecutive values of its token (L & 15) that make up its part of
// a K step's fragment (columns 64k + 16(L >> 4) .. +15: four 16-byte loads, each 1 KiB contiguous over the
// wave in the operand's fragment order; or, for ROWS, from the row itself) and expands them to the three
// base-256 digit planes (digits256_4) with the row's scale:
//   fragment order (EPI_HIGHWAY, EPI_RESID): the scale from the producer's partial maxima (GemmArgs::amax);
//   ROWS (EPI_LATCH): the values are first normalised as RMSNorm does, (x * (1/rms)) * gamma, 1/rms and the
//     scale from the previous block's partial statistics (GemmArgs::ssq, mxg), gamma from LDS.
// Lane group g loads four of the partials, the next tile's while the current one runs.
//
// Software pipeline over the K steps k of a tile: step k issues the loads of step k+2 (of this tile, or
// the next tile's first two), expands step k+1's values, loaded one step earlier, and runs step k's MFMAs
// on the digits expanded during step k-1; the expansion's VALU instructions are interleaved with those
// MFMAs (they do not feed them). The last step of a tile expands the next tile's first step with that
// tile's scale. Two buffers each of values (raw) and digits (dg) alternate with the parity of k: the K loop
// is unrolled by two.
template <int EPI, bool ODD, bool ROWS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_slab_fa_kernel(GemmArgs g,
                                                                                                      int run_tiles,
                                                                                                      int n_runs) {
    constexpr bool STG = can_stage<EPI>();
    extern __shared__ __align__(16) int8_t slab[];
    const int nt = g.Np / LX_BN;
    const int slot = blockIdx.x >> 3;
    const int n_tile = slot % nt;
    const int run = (slot / nt) * 8 + (blockIdx.x & 7);
    if (run >= n_runs) return;
    const int n0 = n_tile * LX_BN;
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kc = g.Kp >> 6;  // >= 2; odd exactly when ODD
    float* bias_s = (float*)(slab + kc * 8192);
    float* stg = STG ? (float*)(slab + kc * 8192 + LX_BN * 4) + w * 16 * STG_LD : nullptr;
    float* gam_s = (float*)(slab + kc * 8192 + LX_BN * 4 + (STG ? STG_BYTES : 0));  // ROWS: gamma, Kp floats
    {
        const int8_t* src = g.W + (long long)(n0 >> 4) * 1024;
        const long long wstep = (long long)(g.Np >> 4) * 1024;
#pragma unroll 4
        for (int c = tid; c < kc * 512; c += 512)
            *(v4i*)(slab + ((long long)c << 4)) = *(const v4i*)(src + (c >> 9) * wstep + ((c & 511) << 4));
        if (tid < LX_BN) bias_s[tid] = g.bias ? g.bias[n0 + tid] : 0.0f;
        if constexpr (ROWS)
            for (int c = tid; c < g.Kp; c += 512) gam_s[c] = g.gamma[c];
    }
    __syncthreads();

    const int mtiles = (g.M + 15) >> 4;
    const int t_begin = run * run_tiles;
    const int t_end = min(t_begin + run_tiles, mtiles);
    int tile = t_begin + w;
    if (tile >= t_end) return;
    const int8_t* wlane = slab + lane * 16;
    const int lg = lane >> 4;
    // ROWS: rows past M read row M - 1 (loaded, never stored). Fragment order: rows of the last tile past M
    // hold whatever the buffer held (loaded, never stored).
    constexpr int KSTEP = ROWS ? 64 : 1024;  // floats from one K step of this lane's values to the next
    constexpr int ISTEP = ROWS ? 4 : 256;    // and from one of its four loads to the next
    auto arow = [&](int t) -> const float* {
        if constexpr (ROWS) return g.Af + (long long)min(t * 16 + (lane & 15), g.M - 1) * g.lda + 16 * lg;
        return g.Af + ((long long)t * kc * 4 << 8) + lane * 4;
    };
    // four partial values j = 4*lg .. 4*lg + 3 of a tile's row from p (clamped into the row's ld >= 4
    // entries; entries from n on are masked when reduced)
    auto part4 = [&](const float* p, int ld, int t) -> float4 {
        return *(const float4*)(p + (long long)min(t * 16 + (lane & 15), g.M - 1) * ld + min(4 * lg, ld - 4));
    };
    struct Parts {
        float4 a, b;
    };
    auto parts = [&](int t) -> Parts {
        if constexpr (ROWS) return Parts{part4(g.ssq, g.stat_ld, t), part4(g.mxg, g.stat_ld, t)};
        return Parts{part4(g.amax, g.amax_ld, t), float4{}};
    };
    struct Scale {
        float s, inv, rinv;
    };
    // the row's scale (and 1/rms for ROWS) from its partials; every lane of the token gets the same values
    auto row_scale = [&](const Parts& pv) -> Scale {
        const int j = 4 * lg, n = ROWS ? g.stat_n : g.amax_n;
        const float4 a = pv.a;
        float m = fmaxf(fmaxf(j < n ? a.x : 0.0f, j + 1 < n ? a.y : 0.0f), fmaxf(j + 2 < n ? a.z : 0.0f, j + 3 < n ? a.w : 0.0f));
        Scale r;
        r.rinv = 1.0f;
        if constexpr (ROWS) {
            // sum of squares: the partials in a fixed order (each lane group's four, then the groups)
            float ss = ((j < n ? a.x : 0.0f) + (j + 1 < n ? a.y : 0.0f)) + ((j + 2 < n ? a.z : 0.0f) + (j + 3 < n ? a.w : 0.0f));
            ss += __shfl_xor(ss, 16, 64);
            ss += __shfl_xor(ss, 32, 64);
            const float4 b = pv.b;
            m = fmaxf(fmaxf(j < n ? b.x : 0.0f, j + 1 < n ? b.y : 0.0f), fmaxf(j + 2 < n ? b.z : 0.0f, j + 3 < n ? b.w : 0.0f));
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            // nn.RMSNormForwardF32 (internal/nn/rmsnorm.go:14-32), as the row kernel computes it
            const float rms = (float)sqrt((double)(ss / (float)g.D + 1e-5f));
            r.rinv = 1.0f / rms;
            // |(x * rinv) * gamma| <= rinv * |x * gamma| up to three roundings: a bound of the largest digit
            m = r.rinv * m * 1.000001f;
        } else {
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
        }
        limb256_scale(m, r.s, r.inv);
        return r;
    };
    auto load_step = [&](f4v (&r)[4], const float* p) {
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = *(const f4v*)(p + ISTEP * i);
    };
    // digits of one K step's values (k: the step, for gamma)
    auto expand = [&](const f4v (&r)[4], int k, const Scale& sc, v4i (&d)[3]) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 x = float4{r[i].x, r[i].y, r[i].z, r[i].w};
            if constexpr (ROWS) {
                const float4 gm = *(const float4*)(gam_s + 64 * k + 16 * lg + 4 * i);
                x = float4{(x.x * sc.rinv) * gm.x, (x.y * sc.rinv) * gm.y, (x.z * sc.rinv) * gm.z, (x.w * sc.rinv) * gm.w};
            }
            uint32_t w0, w1, w2;
            digits256_4(x, sc.inv, w0, w1, w2);
            d[0][i] = (int)w0;
            d[1][i] = (int)w1;
            d[2][i] = (int)w2;
        }
    };
    // ROWS: 1/rms of each row of a tile, from the first channel tile's workgroups
    auto put_rinv = [&](int t, const Scale& sc) {
        if constexpr (ROWS) {
            const int m = t * 16 + (lane & 15);
            if (n_tile == 0 && lane < 16 && m < g.M) g.rinv[m] = sc.rinv;
        }
    };

    // Entering a tile: step 0's digits in dg[0], step 1's values in raw[1].
    f4v raw[2][4];
    v4i dg[2][3];
    const float* ap = arow(tile);
    Scale cur = row_scale(parts(tile));
    put_rinv(tile, cur);
    load_step(raw[0], ap);
    load_step(raw[1], ap + KSTEP);
    expand(raw[0], 0, cur, dg[0]);

    for (;;) {
        const int next = tile + 8;
        const bool more = next < t_end;
        const float* np = more ? arow(next) : ap;
        const Parts pn = parts(more ? next : tile);
        Scale nxt = cur;
        v4i acc[3][8];
        // Step k: raw[P] held step k's values (expanded at step k-1) and takes step k+2's; raw[P^1] holds
        // step k+1's, expanded into dg[P^1] (the next tile's step 0 at the last step); MFMAs on dg[P].
        auto step = [&](int k, auto par, auto first, auto last) {
            constexpr int P = decltype(par)::value, Q = P ^ 1;
            // loads of step k + 2: this tile's, or the next tile's step 0 or 1 (this tile's own again when
            // there is no next tile: harmless, in bounds)
            load_step(raw[P], k + 2 < kc ? ap + (k + 2) * KSTEP : np + (k + 2 - kc) * KSTEP);
            Scale sc = cur;
            int kx = k + 1;
            if constexpr (decltype(last)::value) {
                nxt = row_scale(pn);
                sc = nxt;
                kx = 0;
            }
            v4i wf[4];
            const int8_t* wp = wlane + k * 8192;
#pragma unroll
            for (int h = 0; h < 2; h++) {
#pragma unroll
                for (int ti = 0; ti < 4; ti++) wf[ti] = *(const v4i*)(wp + (4 * h + ti) * 1024);
                // half of the expansion of step k + 1 (two of its four 16-byte groups)
#pragma unroll
                for (int i = 2 * h; i < 2 * h + 2; i++) {
                    float4 x = float4{raw[Q][i].x, raw[Q][i].y, raw[Q][i].z, raw[Q][i].w};
                    if constexpr (ROWS) {
                        const float4 gm = *(const float4*)(gam_s + 64 * kx + 16 * lg + 4 * i);
                        x = float4{(x.x * sc.rinv) * gm.x, (x.y * sc.rinv) * gm.y, (x.z * sc.rinv) * gm.z,
                                   (x.w * sc.rinv) * gm.w};
                    }
                    uint32_t w0, w1, w2;
                    digits256_4(x, sc.inv, w0, w1, w2);
                    dg[Q][0][i] = (int)w0;
                    dg[Q][1][i] = (int)w1;
                    dg[Q][2][i] = (int)w2;
                }
#pragma unroll
                for (int ti = 0; ti < 4; ti++)
#pragma unroll
                    for (int l = 0; l < 3; l++)
                        acc[l][4 * h + ti] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                            wf[ti], dg[P][l], decltype(first)::value ? v4i{0, 0, 0, 0} : acc[l][4 * h + ti], 0, 0, 0);
                if (h == 0) __builtin_amdgcn_sched_group_barrier(0x020, 4, 0);  // the step's four global loads
                __builtin_amdgcn_sched_group_barrier(0x100, ROWS ? 6 : 4, 0);   // LDS weight (and gamma) reads
#pragma unroll
                for (int i = 0; i < 12; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // up to three VALU instructions
                }
            }
        };
        constexpr std::integral_constant<int, 0> P0{};
        constexpr std::integral_constant<int, 1> P1{};
        constexpr std::true_type YES{};
        constexpr std::false_type NO{};
        step(0, P0, YES, NO);
        if constexpr (ODD) {
            // kc = 2j + 1 >= 3: the last step is even
            for (int k = 1; k < kc - 2; k += 2) {
                step(k, P1, NO, NO);
                step(k + 1, P0, NO, NO);
            }
            step(kc - 2, P1, NO, NO);
            step(kc - 1, P0, NO, YES);
        } else {
            // kc = 2j >= 2: the last step is odd
            for (int k = 1; k < kc - 1; k += 2) {
                step(k, P1, NO, NO);
                step(k + 1, P0, NO, NO);
            }
            step(kc - 1, P1, NO, YES);
        }
        EpiRow row;
        row.s = cur.s;
        lx_epilogue<EPI, STG, true>(g, acc, tile * 16, n0, n_tile, lane, row, bias_s, stg);
        if (!more) break;
        tile = next;
        ap = np;
        cur = nxt;
        put_rinv(tile, cur);
        if constexpr (ODD) {
            // the last (even) step expanded the next tile's step 0 into dg[1] and loaded its step 1 into raw[0]
#pragma unroll
            for (int l = 0; l < 3; l++) dg[0][l] = dg[1][l];
#pragma unroll
            for (int i = 0; i < 4; i++) raw[1][i] = raw[0][i];
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Plain int8 GEMM (config 2)
// ------------------------------------------------------------------------------------------------
constexpr int LDSR = 80;  // LDS row stride in bytes (64 data + 16 pad)

__global__ __launch_bounds__(256) void gemm_c2_kernel(GemmArgs g) {
    __shared__ __align__(16) int8_t Ws[2][GEMM_BN * LDSR];
    __shared__ __align__(16) int8_t As[2][GEMM_BM * LDSR];

    const int nt = g.Np / GEMM_BN;
    const int mt = (g.M + GEMM_BM - 1) / GEMM_BM;
    const int total = nt * mt;
    const int t = xcd_tile(blockIdx.x, total);
    if (t >= total) return;
    const int m0 = (t / nt) * GEMM_BM;
    const int n0 = (t % nt) * GEMM_BN;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wn = w & 1, wm = w >> 1;
    const int lrow = lane & 15, lgrp = lane >> 4;

    v4i wreg[2], areg;
    const int a_row_l = tid >> 2, a_col = (tid & 3) * 16;
    const int a_m = m0 + a_row_l;
    const bool a_ok = a_m < g.M;
    const int8_t* a_base = g.A + (long long)(a_ok ? a_m : 0) * g.a_row + a_col;
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int c = tid + i * 256;
            wreg[i] = *(const v4i*)(g.W + (long long)(n0 + (c >> 2)) * g.ldw + k0 + (c & 3) * 16);
        }
        areg = a_ok ? *(const v4i*)(a_base + k0) : v4i{0, 0, 0, 0};
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int c = tid + i * 256;
            *(v4i*)(&Ws[buf][(c >> 2) * LDSR + (c & 3) * 16]) = wreg[i];
        }
        *(v4i*)(&As[buf][a_row_l * LDSR + a_col]) = areg;
    };

    v4i acc[4][2];
#pragma unroll
    for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++) acc[ti][tj] = v4i{0, 0, 0, 0};

    const int ksteps = g.Kp / GEMM_BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int ks = 0; ks < ksteps; ks++) {
        const int buf = ks & 1;
        if (ks + 1 < ksteps) gload((ks + 1) * GEMM_BK);
        v4i wf[4], af[2];
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
            wf[ti] = *(const v4i*)(&Ws[buf][(wn * 64 + ti * 16 + lrow) * LDSR + lgrp * 16]);
#pragma unroll
        for (int tj = 0; tj < 2; tj++)
            af[tj] = *(const v4i*)(&As[buf][(wm * 32 + tj * 16 + lrow) * LDSR + lgrp * 16]);
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
#pragma unroll
            for (int tj = 0; tj < 2; tj++)
                acc[ti][tj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ti], af[tj], acc[ti][tj], 0, 0, 0);
        if (ks + 1 < ksteps) sstore(buf ^ 1);
        __syncthreads();
    }

    const int nb = n0 + wn * 64 + 4 * lgrp;
    if (m0 + GEMM_BM <= g.M && n0 + GEMM_BN <= g.nvalid && (g.ldo & 3) == 0 && !g.out_i32) {
        // A whole tile: each half (tj) of the 64 x 128 fp32 result goes through LDS (the operand buffers
        // are free once the loop's last barrier has passed) and out as 512-byte row segments with
        // non-temporal stores, instead of 64-byte pieces of 16 rows per store (measured at c2: 0.127 ms,
        // against 0.146 with both coherence scope bits set as well and 0.210 with plain stores).
        constexpr int OLD = GEMM_BN + 4;  // staged row stride (floats)
        float* ot = (float*)&Ws[0][0];    // 32 rows: 16.9 KB of the 20 KB buffer
        float* const out0 = g.out + (long long)m0 * g.ldo + n0;
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
                const int n = nb + ti * 16;
                float4 v;
                v.x = (float)acc[ti][tj][0] * g.wscale_n[n];
                v.y = (float)acc[ti][tj][1] * g.wscale_n[n + 1];
                v.z = (float)acc[ti][tj][2] * g.wscale_n[n + 2];
                v.w = (float)acc[ti][tj][3] * g.wscale_n[n + 3];
                *(float4*)(ot + (wm * 16 + lrow) * OLD + wn * 64 + ti * 16 + 4 * lgrp) = v;
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = tid + 256 * i;
                const int row = c >> 5, col = 4 * (c & 31);  // staged row = wm * 16 + lrow
                const float4 v = *(const float4*)(ot + row * OLD + col);
                const f4v t = {v.x, v.y, v.z, v.w};
                float* dst = out0 + (long long)((row >> 4) * 32 + tj * 16 + (row & 15)) * g.ldo + col;
                __builtin_nontemporal_store(t, (f4v*)dst);
            }
            __syncthreads();  // the staged half is read before the next one is written
        }
        return;
    }
#pragma unroll
    for (int tj = 0; tj < 2; tj++) {
        const int m = m0 + wm * 32 + tj * 16 + lrow;
        if (m >= g.M) continue;
#pragma unroll
        for (int ti = 0; ti < 4; ti++) {
            const int n = nb + ti * 16;
            const int nv = g.nvalid - n;
            if (nv <= 0) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = (float)acc[ti][tj][r] * g.wscale_n[min(n + r, g.nvalid - 1)];
            store4(g.out + (long long)m * g.ldo + n, v, nv, (g.ldo & 3) == 0);
            if (g.out_i32) {
                int32_t* dst = g.out_i32 + (long long)m * g.ldo + n;
                if (nv >= 4 && (g.ldo & 3) == 0) *(v4i*)dst = acc[ti][tj];
                else for (int r = 0; r < 4 && r < nv; r++) dst[r] = acc[ti][tj][r];
            }
        }
    }
}

template <int EPI>
hipError_t launch_lx_t(const GemmArgs& a, hipStream_t stream) {
    const int total = (a.Np / LX_BN) * ((a.M + LX_BM - 1) / LX_BM);
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_lx_kernel<EPI>), dim3(xcd_grid(total)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

template <int EPI, int REM, bool STG, int KCF = 0>
hipError_t slab_launch(const GemmArgs& a, int grid, int lds, int run_tiles, int n_runs, hipStream_t stream) {
    // dynamic LDS above the default limit must be allowed once per kernel
    static const hipError_t attr = hipFuncSetAttribute((const void*)gemm_slab_kernel<EPI, REM, STG, KCF>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, slab_lds_limit());
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((gemm_slab_kernel<EPI, REM, STG, KCF>), dim3(grid), dim3(512), lds, stream, a, run_tiles, n_runs);
    return hipGetLastError();
}

// whole-tile prefetch for kc in {2, 4, 6}; 0 when the pipelined loop is used
template <int EPI, bool STG>
hipError_t slab_launch_full(int kc, const GemmArgs& a, int grid, int lds, int run_tiles, int n_runs, hipStream_t stream) {
    if (kc == 2) return slab_launch<EPI, 0, STG, 2>(a, grid, lds, run_tiles, n_runs, stream);
    if (kc == 4) return slab_launch<EPI, 0, STG, 4>(a, grid, lds, run_tiles, n_runs, stream);
    return slab_launch<EPI, 0, STG, 6>(a, grid, lds, run_tiles, n_runs, stream);
}


template <int EPI>
hipError_t launch_slab_t(const GemmArgs& a, hipStream_t stream) {
    const int nt = a.Np / LX_BN;
    const int mtiles = (a.M + 15) / 16;
    if (mtiles == 0) return hipSuccess;
    const int kc = a.Kp / 64;
    int lds = kc * 8192 + LX_BN * 4;
    const bool stg = can_stage<EPI>() && lds + STG_BYTES <= slab_lds_limit();
    if (stg) lds += STG_BYTES;
    // runs of R groups of 8 tiles: long enough to amortise the slab copy, short enough to fill the chip
    // (wide GEMMs have workgroups to spare and take longer runs)
    const int groups = (mtiles + 7) / 8;
    const int R = std::max(1, std::min(nt >= 8 ? 32 : 16, groups * nt / 512));
    const int run_tiles = 8 * R;
    const int n_runs = (mtiles + run_tiles - 1) / run_tiles;
    const int grid = 8 * nt * ((n_runs + 7) / 8);
    // REM = kc % 3 for kc >= 3; 3 marks kc == 2
    const int rem = kc == 2 ? 3 : kc % 3;
    // The whole-tile prefetch holds 18-24 more registers per K step; the residual epilogue's loads (state
    // and blockIn rows) do not fit beside it without spilling.
    const bool full = (kc == 2 || kc == 4 || kc == 6) && EPI != EPI_RESID;
    if constexpr (can_stage<EPI>()) {
        if (stg && full) return slab_launch_full<EPI, true>(kc, a, grid, lds, run_tiles, n_runs, stream);
        if (stg) {
            switch (rem) {
                case 0: return slab_launch<EPI, 0, true>(a, grid, lds, run_tiles, n_runs, stream);
                case 1: return slab_launch<EPI, 1, true>(a, grid, lds, run_tiles, n_runs, stream);
                case 2: return slab_launch<EPI, 2, true>(a, grid, lds, run_tiles, n_runs, stream);
                default: return slab_launch<EPI, 3, true>(a, grid, lds, run_tiles, n_runs, stream);
            }
        }
    }
    if (full) return slab_launch_full<EPI, false>(kc, a, grid, lds, run_tiles, n_runs, stream);
    switch (rem) {
        case 0: return slab_launch<EPI, 0, false>(a, grid, lds, run_tiles, n_runs, stream);
        case 1: return slab_launch<EPI, 1, false>(a, grid, lds, run_tiles, n_runs, stream);
        case 2: return slab_launch<EPI, 2, false>(a, grid, lds, run_tiles, n_runs, stream);
        default: return slab_launch<EPI, 3, false>(a, grid, lds, run_tiles, n_runs, stream);
    }
}

template <int EPI>
hipError_t launch_any_t(const GemmArgs& a, hipStream_t stream) {
    // automatic: the weight-stationary kernel whenever its slab fits in LDS and the batch is large
    const int mode = option(OPT_GEMM_KERNEL);
    const bool fits = a.Kp >= 128 && (long long)(a.Kp / 64) * 8192 + LX_BN * 4 <= slab_lds_limit();
    const bool many = a.M >= kSlabMinRows || (a.M >= kSlabMinRowsWideK && a.Kp >= 256);
    if (fits && (mode == GEMM_SLAB || (mode == GEMM_AUTO && many))) return launch_slab_t<EPI>(a, stream);
    return launch_lx_t<EPI>(a, stream);
}

template <int EPI, bool ODD, bool ROWS>
hipError_t fa_launch(const GemmArgs& a, int grid, int lds, int run_tiles, int n_runs, hipStream_t stream) {
    static const hipError_t attr = hipFuncSetAttribute((const void*)gemm_slab_fa_kernel<EPI, ODD, ROWS>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, slab_lds_limit());
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((gemm_slab_fa_kernel<EPI, ODD, ROWS>), dim3(grid), dim3(512), lds, stream, a, run_tiles, n_runs);
    return hipGetLastError();
}

// LDS of the fp32-operand kernel: the slab, its bias, the output staging (epilogues that stage) and gamma
// (normalised rows)
int fa_lds(int epi, const GemmArgs& a) {
    const bool stg = epi == EPI_F32 || epi == EPI_LATCH || epi == EPI_PROBS || epi == EPI_LOGITS;
    return (a.Kp / 64) * 8192 + LX_BN * 4 + (stg ? STG_BYTES : 0) + (epi == EPI_LATCH ? a.Kp * 4 : 0);
}

template <int EPI, bool ROWS>
hipError_t launch_fa_t(const GemmArgs& a, hipStream_t stream) {
    const int nt = a.Np / LX_BN;
    const int mtiles = (a.M + 15) / 16;
    if (mtiles == 0) return hipSuccess;
    const int kc = a.Kp / 64;
    const int lds = fa_lds(EPI, a);
    // the runs of launch_slab_t
    const int groups = (mtiles + 7) / 8;
    const int R = std::max(1, std::min(nt >= 8 ? 32 : 16, groups * nt / 512));
    const int run_tiles = 8 * R;
    const int n_runs = (mtiles + run_tiles - 1) / run_tiles;
    const int grid = 8 * nt * ((n_runs + 7) / 8);
    if (kc & 1) return fa_launch<EPI, true, ROWS>(a, grid, lds, run_tiles, n_runs, stream);
    return fa_launch<EPI, false, ROWS>(a, grid, lds, run_tiles, n_runs, stream);
}

}  // namespace

int slab_lds_limit() {
    static const int limit = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) return 0;
        return v;
    }();
    return limit;
}

hipError_t launch_gemm_lx(int epi, const GemmArgs& a, hipStream_t stream) {
    if (a.Np % LX_BN || a.Kp % 64 || a.Kp <= 0 || a.M < 0) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_F32: return launch_any_t<EPI_F32>(a, stream);
        case EPI_LATCH: return launch_any_t<EPI_LATCH>(a, stream);
        case EPI_GLU: return launch_any_t<EPI_GLU>(a, stream);
        case EPI_HIGHWAY: return launch_any_t<EPI_HIGHWAY>(a, stream);
        case EPI_RESID: return launch_any_t<EPI_RESID>(a, stream);
        case EPI_LOGITS: return launch_any_t<EPI_LOGITS>(a, stream);
        case EPI_PROBS: return launch_any_t<EPI_PROBS>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

bool gemm_fa_fits(int epi, const GemmArgs& a) {
    if (epi != EPI_HIGHWAY && epi != EPI_RESID && epi != EPI_LATCH) return false;
    if (a.Np % LX_BN || a.Kp % 64 || a.Kp < 128 || a.M <= 0 || !a.Af || ((uintptr_t)a.Af & 15)) return false;
    if (epi == EPI_LATCH) {
        if (!a.ssq || !a.mxg || !a.gamma || !a.rinv || a.D <= 0 || a.lda < a.Kp || (a.lda & 3)) return false;
        if (a.stat_n < 1 || a.stat_n > 16 || a.stat_ld < 4 || a.stat_ld < a.stat_n || (a.stat_ld & 3)) return false;
    } else if (!a.amax || a.amax_n < 1 || a.amax_n > 16 || a.amax_ld < 4 || a.amax_ld < a.amax_n || (a.amax_ld & 3)) {
        return false;
    }
    if (fa_lds(epi, a) > slab_lds_limit()) return false;
    const int mode = option(OPT_GEMM_KERNEL);
    const bool many = a.M >= kSlabMinRows || (a.M >= kSlabMinRowsWideK && a.Kp >= 256);
    return mode == GEMM_SLAB || (mode == GEMM_AUTO && many);
}

hipError_t launch_gemm_fa(int epi, const GemmArgs& a, hipStream_t stream) {
    if (!gemm_fa_fits(epi, a)) return hipErrorInvalidValue;
    if (epi == EPI_HIGHWAY) return launch_fa_t<EPI_HIGHWAY, false>(a, stream);
    if (epi == EPI_LATCH) return launch_fa_t<EPI_LATCH, true>(a, stream);
    return launch_fa_t<EPI_RESID, false>(a, stream);
}

hipError_t launch_gemm_c2(const GemmArgs& a, hipStream_t stream) {
    if (a.Np % GEMM_BN || a.Kp % GEMM_BK || a.Kp <= 0 || a.M < 0) return hipErrorInvalidValue;
    const int total = (a.Np / GEMM_BN) * ((a.M + GEMM_BM - 1) / GEMM_BM);
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(gemm_c2_kernel, dim3(xcd_grid(total)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mg
