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
#include "common.hpp"
#include "gemm.hpp"

namespace mg {

namespace {

__device__ __forceinline__ void store4(float* dst, const float v[4], int nvalid_here, bool aligned) {
    if (nvalid_here >= 4 && aligned) {
        *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
    } else {
        for (int r = 0; r < 4 && r < nvalid_here; r++) dst[r] = v[r];
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
    const int g4 = lane >> 4;
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

    // ------------------------------------------------------------------------------------------
    // Epilogue: combine the three digit planes of tile ti, register r, into the fp32 dot product
    // (x.w = s*(P0 + P1/254 + P2/254^2)) times the weight scale.
    // Token of this lane: m0 + 16w + (L & 15); channel of (ti, r): n0 + 16ti + 4*(L >> 4) + r.
    // ------------------------------------------------------------------------------------------
    const int m = m0 + w * 16 + (lane & 15);
    const bool mok = m < g.M;
    float y[8][4];
    {
        const float s = mok ? g.As[m] : 0.0f;
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float v = fmaf((float)acc[2][ti][r], kInvLimb2, fmaf((float)acc[1][ti][r], kInvLimb1, (float)acc[0][ti][r]));
                y[ti][r] = (s * v) * g.wscale;
            }
    }
    const int nb = n0 + 4 * g4;

    if constexpr (EPI == EPI_F32 || EPI == EPI_LATCH || EPI == EPI_RESID || EPI == EPI_PROBS) {
        if (!mok) return;
        float lse_m = 0.0f;
        if constexpr (EPI == EPI_PROBS) lse_m = g.lse[m];
#pragma unroll
        for (int ti = 0; ti < 8; ti++) {
            const int n = nb + ti * 16;
            const int nv = g.nvalid - n;
            if (nv <= 0) continue;
            float v[4];
            float4 b = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if constexpr (EPI == EPI_LATCH || EPI == EPI_PROBS) b = *(const float4*)(g.bias + n);
            const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float yy = y[ti][r];
                if constexpr (EPI == EPI_LATCH) yy = sigmoid_clamped_f32(yy + bb[r]);
                if constexpr (EPI == EPI_PROBS) {
                    yy = yy + bb[r];
                    yy = __expf(yy - lse_m);
                }
                v[r] = yy;
            }
            if constexpr (EPI == EPI_RESID) {
                float* dst = g.cur + (long long)m * g.ldcur + n;
                for (int r = 0; r < 4 && r < nv; r++) dst[r] = dst[r] + v[r];
            } else {
                store4(g.out + (long long)m * g.ldo + n, v, nv, (g.ldo & 3) == 0);
            }
        }
    } else if constexpr (EPI == EPI_GLU || EPI == EPI_HIGHWAY) {
        // W rows are reordered in blocks of 32: 16 value rows then the 16 matching gate rows, so tile
        // pair (2p, 2p+1) holds value and gate of output channel n0/2 + 16p + 4*(L >> 4) + r.
        if (!mok) return;
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const int ch = n0 / 2 + p * 16 + 4 * g4;
            const int row_v = n0 + 32 * p + 4 * g4, row_g = row_v + 16;
            if (ch >= g.nvalid) continue;
            const float4 bv = *(const float4*)(g.bias + row_v), bg = *(const float4*)(g.bias + row_g);
            const float bvv[4] = {bv.x, bv.y, bv.z, bv.w}, bgg[4] = {bg.x, bg.y, bg.z, bg.w};
            float v[4];
            if constexpr (EPI == EPI_GLU) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float ov = y[2 * p][r] + bvv[r];
                    float og = y[2 * p + 1][r] + bgg[r];
                    v[r] = ov * sigmoid_clamped_f32(og);  // mlpHidden *= sigmoid(gate) (stream.go:218-220)
                }
                store4(g.out + (long long)m * g.ldo + ch, v, g.nvalid - ch, (g.ldo & 3) == 0);
            } else {
                float* dst = g.cur + (long long)m * g.ldcur + ch;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if (ch + r >= g.nvalid) continue;
                    float ov = y[2 * p][r] + bvv[r];
                    float gate = sigmoid_clamped_f32(y[2 * p + 1][r] + bgg[r]);
                    float c = dst[r];
                    float a = (1.0f - gate) * c;  // highway (stream.go:226-229)
                    float b = gate * ov;
                    dst[r] = a + b;
                }
            }
        }
    } else if constexpr (EPI == EPI_LOGITS) {
        const int target = (mok && g.tgt) ? g.tgt[m] : -1;
        // logits of this lane's 32 channels, then (max, first argmax, sum exp) in two passes
        float bmax = -INFINITY;
        int bidx = 0x7fffffff;
#pragma unroll
        for (int ti = 0; ti < 8; ti++) {
            const int n = nb + ti * 16;
            const int nv = g.nvalid - n;
            const float4 b = *(const float4*)(g.bias + n);
            const float bb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float yy = y[ti][r] + bb[r];
                if (r >= nv) yy = -INFINITY;
                y[ti][r] = yy;
                if (yy > bmax) {  // channels rise with (ti, r): ties keep the first index
                    bmax = yy;
                    bidx = n + r;
                }
                if (n + r == target) g.tlog[m] = yy;
            }
            if (mok && g.out && nv > 0) store4(g.out + (long long)m * g.ldo + n, y[ti], nv, (g.ldo & 3) == 0);
        }
        float bsum = 0.0f;
#pragma unroll
        for (int ti = 0; ti < 8; ti++)
#pragma unroll
            for (int r = 0; r < 4; r++) bsum += __expf(y[ti][r] - bmax);
        if (bmax == -INFINITY) bsum = 0.0f;  // every channel of this lane is vocabulary padding
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

}  // namespace

hipError_t launch_gemm_lx(int epi, const GemmArgs& a, hipStream_t stream) {
    if (a.Np % LX_BN || a.Kp % 64 || a.Kp <= 0 || a.M < 0) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_F32: return launch_lx_t<EPI_F32>(a, stream);
        case EPI_LATCH: return launch_lx_t<EPI_LATCH>(a, stream);
        case EPI_GLU: return launch_lx_t<EPI_GLU>(a, stream);
        case EPI_HIGHWAY: return launch_lx_t<EPI_HIGHWAY>(a, stream);
        case EPI_RESID: return launch_lx_t<EPI_RESID>(a, stream);
        case EPI_LOGITS: return launch_lx_t<EPI_LOGITS>(a, stream);
        case EPI_PROBS: return launch_lx_t<EPI_PROBS>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_c2(const GemmArgs& a, hipStream_t stream) {
    if (a.Np % GEMM_BN || a.Kp % GEMM_BK || a.Kp <= 0 || a.M < 0) return hipErrorInvalidValue;
    const int total = (a.Np / GEMM_BN) * ((a.M + GEMM_BM - 1) / GEMM_BM);
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(gemm_c2_kernel, dim3(xcd_grid(total)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace mg
