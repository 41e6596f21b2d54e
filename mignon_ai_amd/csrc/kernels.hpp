// Launchers for the engine's non-GEMM kernels (see kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mg {

enum RowMode : int { ROW_SRC = 0, ROW_EMBED = 1, ROW_RESID = 2, ROW_RULE = 3 };

// Values of OPT_ATTENTION_KERNEL.
enum AttnKernel : int { ATTN_AUTO = 0, ATTN_EXACT = 1, ATTN_MFMA = 2, ATTN_FUSED = 3 };

struct RowArgs {
    int M = 0, D = 0, Dp = 0;
    int mode = ROW_SRC;
    const int32_t* ids = nullptr;      // ROW_EMBED
    const int8_t* emb = nullptr;       // [V][D]
    float emb_scale = 0;
    int V = 0;
    float* cur = nullptr;              // [M][Dp] (ROW_EMBED, ROW_RESID, and ROW_SRC when src is null)
    float* block_in = nullptr;         // [M][Dp]
    const float* src = nullptr;        // ROW_SRC source rows (row stride lds), or null for cur
    int lds = 0;
    const int32_t* row_map = nullptr;  // ROW_SRC: output row m reads source row row_map[m]
    const float* gamma = nullptr;      // RMSNorm scales, or null (copy)
    float* nout = nullptr;             // normalised rows [M][Dp], or null
    float* rinv = nullptr;             // with gamma: each row's 1/rms [M], or null
    int8_t* limbs = nullptr;           // limb-expanded rows in the GEMM fragment layout (K = Dp)
    float* lscale = nullptr;           // [M]
    // ROW_RULE: the rule input [n | left | g] of each position, three segments of `seg` columns (Dp =
    // 3*seg, D = valid columns per segment): n = src[m], left = src[m - dil] (zero for t < dil, t = m % T),
    // g = src2[m], all with row stride seg.
    const float* src2 = nullptr;
    int seg = 0, dil = 1, T = 1;
};
hipError_t launch_row(const RowArgs& a, hipStream_t s);

// Selective latch over whole sequences (teacher-forced forward): g[m] for every position.
struct ScanArgs {
    int B = 0, T = 0, D = 0, Dp = 0;
    const float* lam = nullptr;  // [B*T][Dp]
    const float* nf = nullptr;   // [B*T][Dp]
    // scan_rule only, in place of nf: n recomputed as (x * rinv) * gamma from the norm's source rows x
    // [B*T][Dp] and the row kernel's 1/rms per row, the row kernel's own operations (bit-identical)
    const float* xn = nullptr;
    const float* rinv = nullptr;
    const float* gamma = nullptr;
    float* g = nullptr;          // [B*T][Dp] latch state after each position (may be lam itself)
    const int32_t* lens = nullptr;  // per-sequence length (export position lens[b]-1) or null
    float* g_out = nullptr;         // exported latch state [B][Dp] or null
    // scan_rule only: the rule input [n | left | g] limb-expanded (K = 3*Dp) with one scale per row
    int dil = 1;
    int8_t* xl = nullptr;
    float* xs = nullptr;
};
hipError_t launch_scan(const ScanArgs& a, hipStream_t s);
// Whether launch_scan_rule takes these sizes (T a multiple of 16, Dp <= 1024, dilation at most 48).
bool scan_rule_fits(int T, int Dp, int dil);
hipError_t launch_scan_rule(const ScanArgs& a, hipStream_t s);

// One streaming position per session: latch update, norm ring write and the rule input.
struct LatchStepArgs {
    int S = 0, D = 0, Dp = 0, dil = 1, ring = 1;
    const int32_t* pos = nullptr;  // [S]
    const float* lam = nullptr;    // [S][Dp]
    const float* nf = nullptr;     // [S][Dp]
    float* g = nullptr;            // latch state [S][Dp]
    float* norm_ring = nullptr;    // [S][ring][Dp]
    int8_t* xl = nullptr;          // fragment layout, K = 3*Dp
    float* xs = nullptr;           // [S]
};
hipError_t launch_latch_step(const LatchStepArgs& a, hipStream_t s);

// Windowed causal attention over whole sequences (teacher-forced forward).
struct AttnArgs {
    int B = 0, T = 0, D = 0, Dp = 0, heads = 0, window = 0, cap = 0;
    const float* qkv = nullptr;  // [B*T][3D]
    float* att = nullptr;        // [B*T][Dp]
};
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);

// The attention projection fused with windowed attention (teacher-forced forward): per sequence and head,
// the head's q, k and v come from the limb-expanded normalised rows and the QKV weights on the int8 matrix
// cores and stay on chip (k and v in LDS, q in registers); only the attention output is written. The
// q, k, v values and the attention arithmetic are those of the separate QKV GEMM (EPI_F32) followed by
// attention_mfma_kernel, so the output is bit-identical to that pair.
struct QkvAttnArgs {
    int B = 0, T = 0, D = 0, Dp = 0, heads = 0, window = 0, cap = 0;
    const int8_t* A = nullptr;   // limb-expanded rows, GEMM fragment layout (K = Dp)
    const float* As = nullptr;   // [B*T] row scales
    const int8_t* W = nullptr;   // QKV weights, fragment layout [Dp/64][Np3/16][1 KiB], rows q | k | v
    int Np3 = 0;
    float wscale = 1.0f;
    float* att = nullptr;        // [B*T][Dp], or with amax in the fp32-operand fragment order (frag_off_f32)
    float* amax = nullptr;       // when set: [B*T][amax_ld], entry h = the largest |att| of the row's head h
    int amax_ld = 0;
};
// Whether the fused kernel takes these shapes: 128-token sequences, head width 32 or 64, Dp of 128, 256
// or 384, and attended spans the matrix-core attention kernel covers.
bool qkv_attention_fits(const QkvAttnArgs& a);
hipError_t launch_qkv_attention(const QkvAttnArgs& a, hipStream_t s);

// Attention for one streaming position per session over its key/value ring.
struct AttnStepArgs {
    int S = 0, D = 0, Dp = 0, heads = 0, window = 0, cap = 0;
    const int32_t* pos = nullptr;  // [S]
    const float* qkv = nullptr;    // [S][3D]
    float* kring = nullptr;        // [S][heads][cap][D / heads]
    float* vring = nullptr;        // [S][heads][cap][D / heads]
    float* att = nullptr;          // [S][Dp]
    int8_t* xl = nullptr;          // attention_step_rows: limbs of the output, fragment layout, K = Dp
    float* xs = nullptr;           // attention_step_rows: [S] row scales
    const int32_t* done = nullptr; // attention_step_rows: [S] or null: sessions with done[i] >= 0 are skipped
    // Packed rings (set: kring and vring are not used). Each row (one head, one slot) is dh/4 groups of
    // three words holding four 24-bit mantissas, with a power-of-two scale per row. Read by the kernels
    // built on rk_head only (attention_step_rows, and attention_step_rk where launch_attention_step
    // selects it); launch_attention_step rejects them elsewhere.
    uint32_t* kpack = nullptr;     // [S][heads][cap][3 * dh / 4]
    uint32_t* vpack = nullptr;     // [S][heads][cap][3 * dh / 4]
    float* kscale = nullptr;       // [S][heads][cap]
    float* vscale = nullptr;       // [S][heads][cap]
    // attention_step_rows on packed rings: stream them (non-temporal loads, heads of at most 32) from a
    // ring size on (-1), never (0) or always (1)
    int stream_rings = -1;
};
// Words of one packed ring row of head width dh (a multiple of 4).
constexpr int kv_row_words(int dh) { return 3 * dh / 4; }
hipError_t launch_attention_step(const AttnStepArgs& a, hipStream_t s);
// Decode attention fused with the limb expansion of its output (one workgroup per session, one wave per
// head): writes xl/xs, as the row kernel would from att, instead of att. For head widths that are a
// multiple of 4 up to 64, caches of at most 64 positions and at most 16 heads.
constexpr size_t kStepRowsMaxLds = 156 * 1024;  // dynamic LDS; the static part and the 160 KiB total
bool attention_step_rows_fits(const AttnStepArgs& a);
hipError_t launch_attention_step_rows(const AttnStepArgs& a, hipStream_t s);

// Attention of any head width and span, one wave per (row, head): the fallback of launch_attention and
// launch_attention_step where no specialised kernel applies (same results, reference order).
struct AttnWaveArgs {
    int rows = 0;   // batched: B*T; decode: sessions
    int T = 1;      // batched: positions per sequence
    int D = 0, Dp = 0, heads = 0, dh = 0, window = 0, cap = 0;
    bool step = false;             // decode: keys and values from the rings, position pos[row]
    const float* qkv = nullptr;    // [rows][3D]
    const int32_t* pos = nullptr;  // decode [S]
    float* kring = nullptr;        // decode [S][heads][cap][dh]
    float* vring = nullptr;
    float* att = nullptr;          // [rows][Dp]
};
// Longest span (keys per query) the fallback kernel takes: its scores live in LDS.
constexpr int kMaxAttnSpan = 32768;
// Largest head width of any attention kernel.
constexpr int kMaxHeadWidth = 1024;
hipError_t launch_attention_wave(const AttnWaveArgs& a, hipStream_t s);

// One decode step of a few sessions, each session's whole model step (norms, latch, rule, attention,
// head) in one workgroup: for small sets, where the batched step's ~10 launches per block, each a few
// microseconds at one row, dominate. Same arithmetic as the batched step (limb-expanded int8 MFMA with
// the GEMM epilogues' formulas, the row kernels' and latch step's reductions, rk_head's attention, the
// head's per-tile statistics and their combination), so its outputs equal the batched step's bit for bit.
struct Step1Block {
    int steps = 0, dil_base = 2, init_dil = 1, attn = 0;
    const int8_t* w1 = nullptr; const float* b1 = nullptr; float s1 = 0;   // fragment layout, rows paired
    const int8_t* w2 = nullptr; const float* b2 = nullptr; float s2 = 0;
    const int8_t* wsel = nullptr; float ssel = 0;
    const float* gamma = nullptr;                                          // or null: no normalisation
    const float* anorm = nullptr;
    const int8_t* qkv = nullptr; float sqkv = 0;
    const int8_t* wo = nullptr; float so = 0;
};
struct Step1Args {
    int S = 0, D = 0, Dp = 0, H = 0, Hp = 0, V = 0, Vp = 0, NpD = 0, Np3 = 0;
    int heads = 0, window = 0, cap = 0, ring = 1, nblocks = 0;
    const Step1Block* blocks = nullptr;  // device array [nblocks]
    const int8_t* emb = nullptr; float emb_scale = 0;
    const int8_t* headw = nullptr; const float* headb = nullptr; float head_scale = 0;
    const float* final_norm = nullptr; const float* latch_base = nullptr;
    // session state (the engine's layouts): pos [S]; g [nbs][S][Dp]; norm ring [nbs][S][ring][Dp];
    // K/V rings [nattn][S][heads][cap][dh], or packed (kpack set, AttnStepArgs' layout per attention
    // block: words [nattn][S][heads][cap][3 dh / 4], scales [nattn][S][heads][cap])
    int32_t* pos = nullptr; float* g = nullptr; float* norm_ring = nullptr; float* kring = nullptr; float* vring = nullptr;
    uint32_t* kpack = nullptr; uint32_t* vpack = nullptr; float* kscale = nullptr; float* vscale = nullptr;
    const int32_t* ids = nullptr;        // [S]
    float* logits = nullptr;             // [S][V] or null
    int32_t* argmax = nullptr;           // [S] or null
    double* prob = nullptr;              // [S] or null
    int32_t* next_ids = nullptr;         // [S] or null
    int32_t* out_ids = nullptr;          // [S][out_ld] at column *col (or out_col)
    double* out_probs = nullptr;
    int out_ld = 0, out_col = 0;
    const int32_t* col = nullptr;
    const int32_t* done = nullptr;       // [S] or null: sessions with done[i] >= 0 are skipped (finished)
};
// Whether the one-workgroup step takes this model (state size up to 512, hidden size up to 1024, at most
// 8 attention heads of width 16, 32 or 64 over caches of at most 64 positions, vocabulary up to 16384).
bool step1_fits(const Step1Args& a);
hipError_t launch_step1(const Step1Args& a, hipStream_t s);

// A decode step for tiles of 16 sessions, one workgroup each (the 16 token columns of the matrix cores),
// in segments: segment 0 runs from the embedding to the first attention block's projection q, k, v;
// segment k > 0 starts with the out projection of the block whose attention just ran
// (attention_step_rows_kernel, which writes the out projection's operand) and runs to the next
// attention block's projection or through the head. Same session state and outputs as Step1Args.
struct TileStepArgs : Step1Args {
    int seg_block = 0;               // first block of the segment
    int seg_out = 0;                 // 1: the segment starts with that block's out projection
    float* cur = nullptr;            // [S][Dp] cur and blockIn between segments
    float* bin = nullptr;
    float* qkv = nullptr;            // [S][3D]: the projection that ends a segment
    const int8_t* att_xl = nullptr;  // the attention output's limb planes (fragment layout, K = Dp)
    const float* att_xs = nullptr;   // and their row scales [S]
};
constexpr size_t kTileStepMaxLds = 150 * 1024;
// Whether the tiled step takes this model (state size up to 512, hidden size up to 1024, and its LDS).
bool tile_step_fits(const TileStepArgs& a);
hipError_t launch_tile_step(const TileStepArgs& a, hipStream_t s);

// Per-row combination of the head GEMM's per-tile statistics.
struct HeadCombineArgs {
    int M = 0, ntiles = 0;
    const float* stats = nullptr;  // [M][ntiles][3]
    float* lse = nullptr;          // [M] or null
    int32_t* argmax = nullptr;     // [M] or null
    double* prob = nullptr;        // [M] or null: 1 / sum exp(l - max)
    const float* tlog = nullptr;   // [M] target logits (with tgt)
    const int32_t* tgt = nullptr;  // [M] target ids (invalid: < 0 or >= V)
    int V = 0;
    float* logprob = nullptr;      // [M] or null
    // greedy decode bookkeeping (optional)
    int32_t* next_ids = nullptr;   // [M]
    int32_t* out_ids = nullptr;    // [M][out_ld] at column out_col
    double* out_probs = nullptr;
    int out_ld = 0, out_col = 0;
    const int32_t* col = nullptr;  // when set, the output column is *col instead of out_col (one captured
                                   // decode step serves every column)
    const int32_t* done = nullptr; // [M] or null: sessions with done[i] >= 0 have finished (a batched decode's
                                   // stop token); the one-workgroup steps may skip them
};
hipError_t launch_head_combine(const HeadCombineArgs& a, hipStream_t s);

// Per-sequence bits per token from per-position log-probs (targets t = 1..T-1).
hipError_t launch_bits(int B, int T, const float* logprob, const int32_t* ids, int V, float* bits, hipStream_t s);

// Per-tensor symmetric quantiser (quant.NewTensorF32).
hipError_t launch_quantize(const float* w, long long n, int8_t* q, float* scale, float* amax_tmp, hipStream_t s);

// Session state export after a batched prefill.
hipError_t launch_export_ring(int B, int T, int Dp, int ring, const int32_t* lens, const float* nf, float* norm_ring,
                              hipStream_t s);
hipError_t launch_export_kv(int B, int T, int D, int heads, int cap, const int32_t* lens, const float* qkv,
                            float* kring, float* vring, hipStream_t s);
// The same into packed rings (AttnStepArgs::kpack's layout; head width a multiple of 4).
hipError_t launch_export_kv_packed(int B, int T, int D, int heads, int cap, const int32_t* lens, const float* qkv,
                                   uint32_t* kpack, uint32_t* vpack, float* kscale, float* vscale, hipStream_t s);
// pos[i] = (lens ? lens[i] : pos[i]) + add; with col set, also advances the decode column *col by one.
hipError_t launch_set_pos(int S, const int32_t* lens, int32_t* pos, int add, hipStream_t s, int32_t* col = nullptr);
hipError_t launch_fill_i32(int32_t* p, int n, int v, hipStream_t s);
// *p += 1 (one thread).
hipError_t launch_advance(int32_t* p, hipStream_t s);
hipError_t launch_fill_f32(float* p, long long n, float v, hipStream_t s);

}  // namespace mg
