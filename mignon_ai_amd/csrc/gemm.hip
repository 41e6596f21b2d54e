// Int8 MFMA GEMM for gfx950 (v_mfma_i32_16x16x64_i8) with the engine's fused epilogues.
//
// Orientation: the MFMA row operand is the weight matrix (output channels) and the column operand the
// activations (tokens), so lane l of a 16x16 accumulator tile holds token (l & 15) and four consecutive
// channels 4*(l >> 4) + r. Each lane therefore owns whole per-token quantities (one activation scale,
// one output row), and its four results are contiguous in the token-major output.
//
// Workgroup: 256 threads = 4 waves in a 2 (channels) x 2 (tokens) grid; workgroup tile 128 channels x
// 64 tokens, wave tile 64 x 32 = 4 x 2 MFMA tiles. K advances 64 bytes per step through a double-
// buffered LDS stage (row stride 80 B: conflict-free 16-byte fragment reads).
//
// Limb-expanded activations (nl = 3) accumulate each digit plane in its own exact int32 accumulator;
// at every scale-chunk boundary the three are combined in fp32 and scaled by the per-token chunk scale.
#include "common.hpp"
#include "gemm.hpp"

namespace mg {

namespace {

constexpr int LDSR = 80;  // LDS row stride in bytes (64 data + 16 pad)

template <int NL>
struct Acc {
    v4i p[NL][4][2];
    float f[4][2][4];
};

__device__ __forceinline__ void store4(float* dst, const float v[4], int nvalid_here, bool aligned) {
    if (nvalid_here >= 4 && aligned) {
        *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        for (int r = 0; r < 4 && r < nvalid_here; r++) dst[r] = v[r];
    }
}

template <int NL, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
    __shared__ __align__(16) int8_t Ws[2][GEMM_BN * LDSR];
    __shared__ __align__(16) int8_t As[2][NL][GEMM_BM * LDSR];

    const int nt = g.Np / GEMM_BN;
    const int mt = (g.M + GEMM_BM - 1) / GEMM_BM;
    const int total = nt * mt;
    const int t = xcd_tile(blockIdx.x, total);
    if (t >= total) return;
    const int m0 = (t / nt) * GEMM_BM;
    const int n_tile = t % nt;
    const int n0 = n_tile * GEMM_BN;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wn = w & 1, wm = w >> 1;
    const int lrow = lane & 15, lgrp = lane >> 4;

    // Global -> register staging: W tile 128 x 64 B (2 x 16 B per thread), A tile 64 x 64 B per limb.
    v4i wreg[2], areg[NL];
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
#pragma unroll
        for (int l = 0; l < NL; l++) {
            if (a_ok) areg[l] = *(const v4i*)(a_base + l * g.a_limb + k0);
            else areg[l] = v4i{0, 0, 0, 0};
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int c = tid + i * 256;
            *(v4i*)(&Ws[buf][(c >> 2) * LDSR + (c & 3) * 16]) = wreg[i];
        }
#pragma unroll
        for (int l = 0; l < NL; l++) *(v4i*)(&As[buf][l][a_row_l * LDSR + a_col]) = areg[l];
    };

    Acc<NL> acc;
#pragma unroll
    for (int l = 0; l < NL; l++)
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
#pragma unroll
            for (int tj = 0; tj < 2; tj++) acc.p[l][ti][tj] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int ti = 0; ti < 4; ti++)
#pragma unroll
        for (int tj = 0; tj < 2; tj++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc.f[ti][tj][r] = 0.0f;

    // Per-token chunk scales (limb-expanded A): token of this lane in each token tile.
    int tok[2];
#pragma unroll
    for (int tj = 0; tj < 2; tj++) tok[tj] = m0 + wm * 32 + tj * 16 + lrow;

    const int ksteps = g.Kp / GEMM_BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int ks = 0; ks < ksteps; ks++) {
        const int buf = ks & 1;
        if (ks + 1 < ksteps) gload((ks + 1) * GEMM_BK);
        v4i wf[4], af[NL][2];
#pragma unroll
        for (int ti = 0; ti < 4; ti++)
            wf[ti] = *(const v4i*)(&Ws[buf][(wn * 64 + ti * 16 + lrow) * LDSR + lgrp * 16]);
#pragma unroll
        for (int l = 0; l < NL; l++)
#pragma unroll
            for (int tj = 0; tj < 2; tj++)
                af[l][tj] = *(const v4i*)(&As[buf][l][(wm * 32 + tj * 16 + lrow) * LDSR + lgrp * 16]);
#pragma unroll
        for (int l = 0; l < NL; l++)
#pragma unroll
            for (int ti = 0; ti < 4; ti++)
#pragma unroll
                for (int tj = 0; tj < 2; tj++)
                    acc.p[l][ti][tj] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wf[ti], af[l][tj], acc.p[l][ti][tj], 0, 0, 0);
        if (NL == 3 && (ks + 1) % g.kc_steps == 0) {
            const int c = ks / g.kc_steps;
#pragma unroll
            for (int tj = 0; tj < 2; tj++) {
                float s = tok[tj] < g.M ? g.As[(long long)tok[tj] * g.as_ld + c] : 0.0f;
#pragma unroll
                for (int ti = 0; ti < 4; ti++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        float v = fmaf((float)acc.p[NL - 1][ti][tj][r], kInvLimb2,
                                       fmaf((float)acc.p[NL > 1 ? 1 : 0][ti][tj][r], kInvLimb1, (float)acc.p[0][ti][tj][r]));
                        acc.f[ti][tj][r] = fmaf(s, v, acc.f[ti][tj][r]);
                    }
#pragma unroll
                for (int l = 0; l < NL; l++)
#pragma unroll
                    for (int ti = 0; ti < 4; ti++) acc.p[l][ti][tj] = v4i{0, 0, 0, 0};
            }
        }
        if (ks + 1 < ksteps) sstore(buf ^ 1);
        __syncthreads();
    }

    // ------------------------------------------------------------------------------------------
    // Epilogues. Channel of (ti, r) for this lane: n0 + wn*64 + ti*16 + 4*lgrp + r.
    // ------------------------------------------------------------------------------------------
    const int nb = n0 + wn * 64 + 4 * lgrp;

    if constexpr (EPI == EPI_C2) {
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            const int m = tok[tj];
            if (m >= g.M) continue;
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
                const int n = nb + ti * 16;
                const int nv = g.nvalid - n;
                if (nv <= 0) continue;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; r++) v[r] = (float)acc.p[0][ti][tj][r] * g.wscale_n[min(n + r, g.nvalid - 1)];
                store4(g.out + (long long)m * g.ldo + n, v, nv, (g.ldo & 3) == 0);
                if (g.out_i32) {
                    int32_t* dst = g.out_i32 + (long long)m * g.ldo + n;
                    if (nv >= 4 && (g.ldo & 3) == 0) *(v4i*)dst = acc.p[0][ti][tj];
                    else for (int r = 0; r < 4 && r < nv; r++) dst[r] = acc.p[0][ti][tj][r];
                }
            }
        }
    } else if constexpr (EPI == EPI_F32 || EPI == EPI_LATCH || EPI == EPI_RESID || EPI == EPI_PROBS) {
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            const int m = tok[tj];
            if (m >= g.M) continue;
            float lse_m = 0.0f;
            if constexpr (EPI == EPI_PROBS) lse_m = g.lse[m];
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
                const int n = nb + ti * 16;
                const int nv = g.nvalid - n;
                if (nv <= 0) continue;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float y = acc.f[ti][tj][r] * g.wscale;
                    if constexpr (EPI == EPI_LATCH) y = sigmoid_clamped(y + g.bias[n + r]);
                    if constexpr (EPI == EPI_PROBS) {
                        y = y + g.bias[n + r];
                        y = __expf(y - lse_m);
                    }
                    v[r] = y;
                }
                if constexpr (EPI == EPI_RESID) {
                    float* dst = g.cur + (long long)m * g.ldcur + n;
                    for (int r = 0; r < 4 && r < nv; r++) dst[r] = dst[r] + v[r];
                } else {
                    store4(g.out + (long long)m * g.ldo + n, v, nv, (g.ldo & 3) == 0);
                }
            }
        }
    } else if constexpr (EPI == EPI_HIGHWAY) {
        // W rows are reordered in blocks of 32: 16 value rows then the 16 matching gate rows, so tile
        // pair (2p, 2p+1) holds value and gate of the same output channel in the same registers.
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            const int m = tok[tj];
            if (m >= g.M) continue;
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                const int ch = (n0 + wn * 64) / 2 + pp * 16 + 4 * lgrp;
                const int row_v = nb + (2 * pp) * 16, row_g = row_v + 16;
                float* dst = g.cur + (long long)m * g.ldcur + ch;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if (ch + r >= g.nvalid) continue;
                    float ov = acc.f[2 * pp][tj][r] * g.wscale;
                    ov = ov + g.bias[row_v + r];
                    float og = acc.f[2 * pp + 1][tj][r] * g.wscale;
                    og = og + g.bias[row_g + r];
                    float gate = sigmoid_clamped(og);
                    float c = dst[r];
                    float a = (1.0f - gate) * c;
                    float b = gate * ov;
                    dst[r] = a + b;
                }
            }
        }
    } else if constexpr (EPI == EPI_GLU) {
        // Same pairing as EPI_HIGHWAY (value rows, then gate rows). The workgroup produces 64 hidden
        // units [n0/2, n0/2 + 64) of each token: one limb-scale chunk.
        float* red = (float*)&Ws[0][0];  // [2 wm][2 tj][16 tok][2 wn]
        float h[2][2][4];
        float amax[2];
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            float mx = 0.0f;
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                const int row_v = nb + (2 * pp) * 16, row_g = row_v + 16;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float hv = acc.f[2 * pp][tj][r] * g.wscale;
                    hv = hv + g.bias[row_v + r];
                    float hg = acc.f[2 * pp + 1][tj][r] * g.wscale;
                    hg = hg + g.bias[row_g + r];
                    float y = hv * sigmoid_clamped(hg);
                    h[tj][pp][r] = y;
                    mx = fmaxf(mx, fabsf(y));
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            amax[tj] = mx;
        }
        if (lgrp == 0) {
#pragma unroll
            for (int tj = 0; tj < 2; tj++) red[((wm * 2 + tj) * 16 + lrow) * 2 + wn] = amax[tj];
        }
        __syncthreads();
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            const int m = tok[tj];
            float mx = fmaxf(red[((wm * 2 + tj) * 16 + lrow) * 2 + 0], red[((wm * 2 + tj) * 16 + lrow) * 2 + 1]);
            if (m >= g.M) continue;
            float s, inv;
            limb_scale(mx, s, inv);
            int8_t* row = g.hl + (long long)m * g.hl_row;
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                const int ch = (n0 + wn * 64) / 2 + pp * 16 + 4 * lgrp;
                uint32_t q0 = 0, q1 = 0, q2 = 0;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    Limbs L = split_limbs(h[tj][pp][r], inv);
                    q0 |= (uint32_t)(uint8_t)L.q0 << (8 * r);
                    q1 |= (uint32_t)(uint8_t)L.q1 << (8 * r);
                    q2 |= (uint32_t)(uint8_t)L.q2 << (8 * r);
                }
                *(uint32_t*)(row + ch) = q0;
                *(uint32_t*)(row + g.hl_limb + ch) = q1;
                *(uint32_t*)(row + 2 * g.hl_limb + ch) = q2;
            }
            if (wn == 0 && lgrp == 0) g.hs[(long long)m * g.hs_ld + n_tile] = s;
        }
    } else if constexpr (EPI == EPI_LOGITS) {
        float* red = (float*)&Ws[0][0];  // [2 wm][2 tj][16 tok][2 wn][3]
#pragma unroll
        for (int tj = 0; tj < 2; tj++) {
            const int m = tok[tj];
            const bool mok = m < g.M;
            const int target = (mok && g.tgt) ? g.tgt[m] : -1;
            float bmax = -INFINITY, bsum = 0.0f;
            int bidx = 0x7fffffff;
#pragma unroll
            for (int ti = 0; ti < 4; ti++) {
                const int n = nb + ti * 16;
                const int nv = g.nvalid - n;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float y = acc.f[ti][tj][r] * g.wscale;
                    y = y + g.bias[min(n + r, g.Np - 1)];
                    v[r] = y;
                    if (r < nv) {
                        if (y > bmax) {
                            bsum = bsum * __expf(bmax - y) + 1.0f;
                            bmax = y;
                            bidx = n + r;
                        } else {
                            bsum += __expf(y - bmax);
                        }
                        if (n + r == target) g.tlog[m] = y;
                    }
                }
                if (mok && g.out && nv > 0) store4(g.out + (long long)m * g.ldo + n, v, nv, (g.ldo & 3) == 0);
            }
            // combine the four lane groups (channels interleave by group; the smaller index wins ties)
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
            if (lgrp == 0) {
                float* rr = red + (((wm * 2 + tj) * 16 + lrow) * 2 + wn) * 3;
                rr[0] = bmax; rr[1] = bsum; rr[2] = __int_as_float(bidx);
            }
        }
        __syncthreads();
        if (wn == 0 && lgrp == 0) {
#pragma unroll
            for (int tj = 0; tj < 2; tj++) {
                const int m = tok[tj];
                if (m >= g.M) continue;
                const float* r0 = red + (((wm * 2 + tj) * 16 + lrow) * 2 + 0) * 3;
                const float* r1 = r0 + 3;
                float m0v = r0[0], m1v = r1[0];
                int i0 = __float_as_int(r0[2]), i1 = __float_as_int(r1[2]);
                float nm = fmaxf(m0v, m1v);
                float ns = (m0v == -INFINITY ? 0.0f : r0[1] * __expf(m0v - nm)) +
                           (m1v == -INFINITY ? 0.0f : r1[1] * __expf(m1v - nm));
                int ni = (m1v > m0v) ? i1 : (m0v > m1v) ? i0 : min(i0, i1);
                float* dst = g.stats + ((long long)m * g.stats_ld + n_tile) * 3;
                dst[0] = nm; dst[1] = ns; dst[2] = __int_as_float(ni);
            }
        }
    }
}

template <int NL, int EPI>
hipError_t launch_t(const GemmArgs& a, hipStream_t stream) {
    const int nt = a.Np / GEMM_BN;
    const int mt = (a.M + GEMM_BM - 1) / GEMM_BM;
    const int total = nt * mt;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL((gemm_kernel<NL, EPI>), dim3(xcd_grid(total)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm(int nl, int epi, const GemmArgs& a, hipStream_t stream) {
    if (a.Np % GEMM_BN || a.Kp % GEMM_BK || a.Kp <= 0 || a.M < 0) return hipErrorInvalidValue;
    if (nl == 1) {
        if (epi == EPI_C2) return launch_t<1, EPI_C2>(a, stream);
        return hipErrorInvalidValue;
    }
    if (nl != 3 || a.kc_steps <= 0 || (a.Kp / GEMM_BK) % a.kc_steps) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_F32: return launch_t<3, EPI_F32>(a, stream);
        case EPI_LATCH: return launch_t<3, EPI_LATCH>(a, stream);
        case EPI_GLU: return launch_t<3, EPI_GLU>(a, stream);
        case EPI_HIGHWAY: return launch_t<3, EPI_HIGHWAY>(a, stream);
        case EPI_RESID: return launch_t<3, EPI_RESID>(a, stream);
        case EPI_LOGITS: return launch_t<3, EPI_LOGITS>(a, stream);
        case EPI_PROBS: return launch_t<3, EPI_PROBS>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mg
