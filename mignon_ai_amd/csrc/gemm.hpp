// Int8 MFMA GEMM of the engine: C[m][n] = sum_k A[m][k] * W[n][k], A token-major, W in the reference
// layout (one row per output channel, K contiguous: kernels.MatVecInt8, internal/kernels/int8.go:31-41).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mg {

enum Epi : int {
    EPI_C2 = 0,       // standalone int8 GEMM: C = float(acc)*scale[n], optional int32 acc
    EPI_F32 = 1,      // y = acc*s                                  (attention QKV)
    EPI_LATCH = 2,    // lambda = sigmoid_clamped(acc*s + base[n])  (latch selector)
    EPI_GLU = 3,      // h = (acc_v*s + b_v) * sigmoid_clamped(acc_g*s + b_g) -> limb-expanded h
    EPI_HIGHWAY = 4,  // cur = (1-g)*cur + g*(acc_v*s + b_v), g = sigmoid_clamped(acc_g*s + b_g)
    EPI_RESID = 5,    // cur += acc*s                               (attention output projection)
    EPI_LOGITS = 6,   // l = acc*s + b: optional store, per-tile (max, sum exp, first argmax), target logit
    EPI_PROBS = 7,    // p = exp(acc*s + b - lse[m])
};

// Tile shape: 128 output channels x 64 tokens per workgroup, K in steps of 64.
constexpr int GEMM_BN = 128;
constexpr int GEMM_BM = 64;
constexpr int GEMM_BK = 64;

struct GemmArgs {
    // A (tokens): row m, limb l at A + m*a_row + l*a_limb; int8, Kp bytes valid per limb row.
    const int8_t* A = nullptr;
    long long a_row = 0;
    long long a_limb = 0;
    // Limb scales: As[m*as_ld + c] for K chunk c of kc_steps*64 columns (limb-expanded A only).
    const float* As = nullptr;
    int as_ld = 1;
    int kc_steps = 1;
    // W (channels): row n at W + n*ldw, Np rows (multiple of 128), Kp columns (multiple of 64).
    const int8_t* W = nullptr;
    int ldw = 0;
    int M = 0, Np = 0, Kp = 0;
    int nvalid = 0;  // output channels that exist (the rest are padding)
    float wscale = 1.0f;
    const float* wscale_n = nullptr;  // per-channel scale (EPI_C2)
    const float* bias = nullptr;      // per W row (after any reordering)
    float* out = nullptr;             // fp32 output, row stride ldo
    long long ldo = 0;
    int32_t* out_i32 = nullptr;       // EPI_C2 raw accumulators (row stride ldo)
    float* cur = nullptr;             // EPI_HIGHWAY / EPI_RESID state, row stride ldcur
    int ldcur = 0;
    int8_t* hl = nullptr;             // EPI_GLU limb output: row m, limb l at hl + m*hl_row + l*hl_limb
    long long hl_row = 0;
    long long hl_limb = 0;
    float* hs = nullptr;              // EPI_GLU limb scales [m][hs_ld], one per 64 outputs
    int hs_ld = 0;
    float* stats = nullptr;           // EPI_LOGITS: [m][stats_ld][3] = max, sum exp(l - max), argmax
    int stats_ld = 0;
    const int32_t* tgt = nullptr;     // EPI_LOGITS: target id per row (or null)
    float* tlog = nullptr;            // EPI_LOGITS: target logit per row
    const float* lse = nullptr;       // EPI_PROBS: log-sum-exp per row
};

// nl = number of A limbs (1: plain int8 A; 3: limb-expanded fp32 activations).
hipError_t launch_gemm(int nl, int epi, const GemmArgs& a, hipStream_t stream);

}  // namespace mg
