// Int8 MFMA GEMMs of the engine: C[m][n] = sum_k A[m][k] * W[n][k], A token-major, W one row per output
// channel with K contiguous (kernels.MatVecInt8's layout, internal/kernels/int8.go:31-41).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mg {

enum Epi : int {
    EPI_C2 = 0,       // standalone int8 GEMM: C = float(acc)*scale[n], optional int32 acc
    EPI_F32 = 1,      // y = acc*s                                  (attention QKV)
    EPI_LATCH = 2,    // lambda = sigmoid_clamped(acc*s + base[n])  (latch selector)
    EPI_GLU = 3,      // h = (acc_v*s + b_v) * sigmoid_clamped(acc_g*s + b_g), fp32
    EPI_HIGHWAY = 4,  // cur = (1-g)*cur + g*(acc_v*s + b_v), g = sigmoid_clamped(acc_g*s + b_g)
    EPI_RESID = 5,    // cur += acc*s                               (attention output projection)
    EPI_LOGITS = 6,   // l = acc*s + b: optional store, per-tile (max, sum exp, first argmax), target logit
    EPI_PROBS = 7,    // p = exp(acc*s + b - lse[m])
};

// ------------------------------------------------------------------------------------------------
// Fragment layout. Operands of v_mfma_i32_16x16x64_i8 are 16 rows x 64 bytes, lane L holding row
// (L & 15) and bytes [16*(L >> 4), +16). Both GEMM operands are stored as such 1 KiB fragments so that
// every fragment is one coalesced 16-byte-per-lane load:
//   weights      [K/64][Np/16][1 KiB]          (all channel tiles of one K step are contiguous)
//   activations  [Mp/16][K/64][3 limbs][1 KiB]  (Mp = M rounded up to LX_ROWS)
// ------------------------------------------------------------------------------------------------
__host__ __device__ inline long long frag_off_a(int m, int k, int limb, int kc) {
    return ((((long long)(m >> 4) * kc + (k >> 6)) * 3 + limb) << 10) + (((m & 15) + 16 * ((k >> 4) & 3)) << 4) + (k & 15);
}
__host__ __device__ inline long long frag_off_w(int n, int k, int np) {
    return ((((long long)(k >> 6) * (np >> 4)) + (n >> 4)) << 10) + (((n & 15) + 16 * ((k >> 4) & 3)) << 4) + (k & 15);
}
// fp32 operand in fragment order (launch_gemm_fa), [Mp/16][K/64][4][64 lanes][4 floats]: element (m, k) sits
// where lane (m & 15) + 16*((k >> 4) & 3) reads it with its (k >> 2) & 3'th 16-byte load of K step k >> 6,
// so each of a K step's four loads is 1 KiB contiguous over the wave. Offset in floats.
__host__ __device__ inline long long frag_off_f32(long long m, int k, int kc) {
    return ((((m >> 4) * kc + (k >> 6)) * 4 + ((k >> 2) & 3)) << 8) + (((m & 15) + 16 * ((k >> 4) & 3)) << 2) + (k & 3);
}

// Tile of the limb-expanded GEMM: 128 channels x 64 tokens per workgroup (4 waves x 16 tokens).
constexpr int LX_BN = 128;
constexpr int LX_BM = 64;
// Activation buffers in the fragment layout are allocated in whole 128-row blocks.
constexpr int LX_ROWS = 128;
// Tile of the plain int8 GEMM (config 2): 128 channels x 64 tokens.
constexpr int GEMM_BN = 128;
constexpr int GEMM_BM = 64;
constexpr int GEMM_BK = 64;

struct GemmArgs {
    // Limb-expanded A (fragment layout) with one scale per token row; or plain row-major int8 A (c2).
    const int8_t* A = nullptr;
    long long a_row = 0;              // c2: row stride
    const float* As = nullptr;        // per-row limb scale
    // W: fragment layout (limb-expanded path) or row-major [Np][ldw] (c2).
    const int8_t* W = nullptr;
    int ldw = 0;
    int M = 0, Np = 0, Kp = 0;
    int nvalid = 0;                   // output channels that exist (the rest are padding)
    float wscale = 1.0f;
    const float* wscale_n = nullptr;  // per-channel scale (EPI_C2)
    const float* bias = nullptr;      // per W row (after any reordering), Np entries
    float* out = nullptr;             // fp32 output, row stride ldo
    long long ldo = 0;
    int32_t* out_i32 = nullptr;       // EPI_C2 raw accumulators (row stride ldo)
    float* cur = nullptr;             // EPI_HIGHWAY / EPI_RESID state, row stride ldcur
    int ldcur = 0;
    const float* cur_in = nullptr;    // EPI_HIGHWAY / EPI_RESID: read the state from here (null: from cur)
    float* resid = nullptr;           // EPI_HIGHWAY / EPI_RESID: when set, the new state v is added into
                                      // it (resid += v, the inter-block residual) instead of stored to cur
    float* stats = nullptr;           // EPI_LOGITS: [m][stats_ld][3] = max, sum exp(l - max), argmax
    int stats_ld = 0;
    int want_argmax = 1;              // EPI_LOGITS: 0 leaves the argmax entry of the statistics unset
    const int32_t* tgt = nullptr;     // EPI_LOGITS: target id per row (or null)
    float* tlog = nullptr;            // EPI_LOGITS: target logit per row
    const float* lse = nullptr;       // EPI_PROBS: log-sum-exp per row
    // fp32 operand (launch_gemm_fa): A is given as fp32 values Af in fragment order (frag_off_f32 with
    // kc = Kp/64, whole 16-row tiles; padding columns meet zero weights) and expanded to digits as it is
    // loaded, with one scale per row from the largest of the row's partial maxima amax[m * amax_ld + j],
    // j < amax_n (each the largest |x| over a part of the row, written by the kernel that produced the row).
    const float* Af = nullptr;
    const float* amax = nullptr;
    int amax_ld = 0, amax_n = 0;
    // EPI_GLU: when set, h goes to `out` in fragment order (frag_off_f32, kc = Np/128) instead of rows, and the
    // largest |h| of each row's 64 outputs of every channel tile to amax_out[m * amax_out_ld + tile] (the
    // operand of a GEMM reading h as fp32)
    float* amax_out = nullptr;
    int amax_out_ld = 0;
    // RMSNorm statistics between blocks, [m * stat_ld + tile] per row and channel tile. Producer (EPI_HIGHWAY
    // or EPI_RESID with resid, when ssq_out is set): the sum of squares of the row's new blockIn values in
    // the tile (ssq_out) and their largest |v * gamma_next[channel]| (mxg_out). Consumer (launch_gemm_fa with
    // EPI_LATCH on rows): A = RMSNorm(Af rows; gamma) is formed as the rows are loaded (row stride lda
    // floats), 1/rms from the sum of the row's stat_n partial sums of squares over D channels, the digits'
    // scale from 1/rms times the largest partial maximum; 1/rms of each row is written to rinv.
    float* ssq_out = nullptr;
    float* mxg_out = nullptr;
    const float* gamma_next = nullptr;
    const float* ssq = nullptr;
    const float* mxg = nullptr;
    const float* gamma = nullptr;
    int stat_ld = 0, stat_n = 0, D = 0;
    long long lda = 0;
    float* rinv = nullptr;
};

// Values of OPT_GEMM_KERNEL.
enum GemmKernel : int { GEMM_AUTO = 0, GEMM_STREAM = 1, GEMM_SLAB = 2 };
// Token rows from which the weight-stationary kernel is used when its slab fits in LDS: from 8192 rows
// always, from 2048 rows when K is at least 256 (c4's decode steps of 4096 rows: 41.2 ms per step with
// it against 43.3 with the streaming kernel; the chat model's K = 128 GEMMs stay faster streaming).
constexpr int kSlabMinRows = 8192;
constexpr int kSlabMinRowsWideK = 2048;
// Largest dynamic LDS allocation of one workgroup on the current device (bytes).
int slab_lds_limit();

// Limb-expanded GEMM (epilogues EPI_F32 .. EPI_PROBS).
hipError_t launch_gemm_lx(int epi, const GemmArgs& a, hipStream_t stream);
// Plain int8 GEMM of config 2 (EPI_C2).
hipError_t launch_gemm_c2(const GemmArgs& a, hipStream_t stream);

// The weight-stationary GEMM on an fp32 operand for epilogues EPI_HIGHWAY and EPI_RESID (Af in fragment
// order, amax: see GemmArgs) and EPI_LATCH (Af rows normalised as loaded: ssq, mxg, gamma, rinv): each row
// is expanded to three base-256 digit planes as it is loaded,
// x ~= (amax/64)*(q0 + q1/256 + q2/65536) with x*2^22/amax rounded to an integer q below 2^22 in
// magnitude (representation error below 1.8e-7*amax), so no separate pass writes the limb planes.
// gemm_fa_fits: whether the shapes and the batch take it (the same batch sizes as the weight-stationary
// kernel of launch_gemm_lx).
bool gemm_fa_fits(int epi, const GemmArgs& a);
hipError_t launch_gemm_fa(int epi, const GemmArgs& a, hipStream_t stream);

}  // namespace mg
