// CPU restatement of the reference INT8 engine (mignon-ai internal/quant over internal/kernels).
//
// TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP engine in mignon_ai_amd/.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only as the
// checker or the timed CPU baseline -- never as a code path of the product.
//
// It restates the reference's arithmetic step by step, with the same fp32 rounding points:
//   - Go on amd64 (GOAMD64=v1) emits no implicit FMA, so this file is built with -ffp-contract=off and
//     uses fmaf() exactly where the AVX2 assembly uses VFMADD.
//   - The AVX2 kernels' accumulator layouts and reduction trees are reproduced lane by lane.
// Every function cites the reference file:line it follows (paths relative to the reference root).
//
// Parity pins (what checks this file): tests/test_oracle_*.py.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <cfloat>
#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include <immintrin.h>

namespace {

// ---------------------------------------------------------------------------------------------
// internal/kernels
// ---------------------------------------------------------------------------------------------

// Horizontal reduction shared by dotProductASM_F32 and dotInt8ASM_F32 after the accumulators have
// been summed into one 8-lane register v: VEXTRACTF128/VADDPS folds lanes i and i+4, VSHUFPS 0x4E
// adds the pairs (0,2),(1,3) and VSHUFPS 0x01 adds the two results
// (internal/kernels/vec_amd64.s:38-44, :655-661).
inline float hreduce8(const float v[8]) {
    float f0 = v[0] + v[4], f1 = v[1] + v[5], f2 = v[2] + v[6], f3 = v[3] + v[7];
    float g0 = f0 + f2, g1 = f1 + f3;
    return g0 + g1;
}

// kernels.DotF32 on an AVX2 machine: dotProductASM_F32 (internal/kernels/vec_amd64.s:4-63).
// Two 8-lane FMA accumulators over 16-element chunks, one more 8-chunk into acc0, the reduction
// tree, then the scalar tail with an unfused multiply and add.
float dot_f32_scalar(const float* x, const float* y, int n) {
    float a0[8] = {0}, a1[8] = {0};
    int i = 0;
    for (; n - i >= 16; i += 16) {
        for (int j = 0; j < 8; j++) {
            a0[j] = fmaf(x[i + j], y[i + j], a0[j]);
            a1[j] = fmaf(x[i + 8 + j], y[i + 8 + j], a1[j]);
        }
    }
    if (n - i >= 8) {
        for (int j = 0; j < 8; j++) a0[j] = fmaf(x[i + j], y[i + j], a0[j]);
        i += 8;
    }
    float v[8];
    for (int j = 0; j < 8; j++) v[j] = a0[j] + a1[j];
    float s = hreduce8(v);
    for (; i < n; i++) {
        float p = x[i] * y[i];
        s = s + p;
    }
    return s;
}

// kernels.DotInt8F32 on an AVX2 machine: dotInt8ASM_F32 (internal/kernels/vec_amd64.s:603-679).
// Four 8-lane accumulators (Y0, Y1, Y4, Y5) over 32-element chunks, 8-chunks into Y0, then
// (Y0+Y1)+(Y4+Y5), the reduction tree and the unfused scalar tail.
float dot_i8_f32_scalar(const float* x, const int8_t* w, int n) {
    float a0[8] = {0}, a1[8] = {0}, a4[8] = {0}, a5[8] = {0};
    int i = 0;
    for (; n - i >= 32; i += 32) {
        for (int j = 0; j < 8; j++) {
            a0[j] = fmaf((float)w[i + j], x[i + j], a0[j]);
            a1[j] = fmaf((float)w[i + 8 + j], x[i + 8 + j], a1[j]);
            a4[j] = fmaf((float)w[i + 16 + j], x[i + 16 + j], a4[j]);
            a5[j] = fmaf((float)w[i + 24 + j], x[i + 24 + j], a5[j]);
        }
    }
    for (; n - i >= 8; i += 8) {
        for (int j = 0; j < 8; j++) a0[j] = fmaf((float)w[i + j], x[i + j], a0[j]);
    }
    float v[8];
    for (int j = 0; j < 8; j++) {
        float s01 = a0[j] + a1[j];
        float s45 = a4[j] + a5[j];
        v[j] = s01 + s45;
    }
    float s = hreduce8(v);
    for (; i < n; i++) {
        float p = (float)w[i] * x[i];
        s = s + p;
    }
    return s;
}

// The same two kernels with AVX2/FMA intrinsics, issued as the reference's assembly issues them
// (VPMOVSXBD/VCVTDQ2PS/VFMADD231PS per 8 lanes, VADDPS between accumulators). Each lane runs the same
// FMA chain as the scalar restatement above, so the bits are identical; this path exists so that the
// CPU baseline runs at the reference's vector width. Chosen at run time when the CPU has AVX2 and FMA.
__attribute__((target("avx2,fma"))) float dot_f32_avx2(const float* x, const float* y, int n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    int i = 0;
    for (; n - i >= 16; i += 16) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), _mm256_loadu_ps(y + i), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 8), _mm256_loadu_ps(y + i + 8), a1);
    }
    if (n - i >= 8) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), _mm256_loadu_ps(y + i), a0);
        i += 8;
    }
    float v[8];
    _mm256_storeu_ps(v, _mm256_add_ps(a0, a1));
    float s = hreduce8(v);
    for (; i < n; i++) {
        float p = x[i] * y[i];
        s = s + p;
    }
    return s;
}

__attribute__((target("avx2,fma"))) inline __m256 widen8(const int8_t* w) {
    return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)w)));
}

__attribute__((target("avx2,fma"))) float dot_i8_f32_avx2(const float* x, const int8_t* w, int n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a4 = _mm256_setzero_ps(), a5 = _mm256_setzero_ps();
    int i = 0;
    for (; n - i >= 32; i += 32) {
        a0 = _mm256_fmadd_ps(widen8(w + i), _mm256_loadu_ps(x + i), a0);
        a1 = _mm256_fmadd_ps(widen8(w + i + 8), _mm256_loadu_ps(x + i + 8), a1);
        a4 = _mm256_fmadd_ps(widen8(w + i + 16), _mm256_loadu_ps(x + i + 16), a4);
        a5 = _mm256_fmadd_ps(widen8(w + i + 24), _mm256_loadu_ps(x + i + 24), a5);
    }
    for (; n - i >= 8; i += 8) a0 = _mm256_fmadd_ps(widen8(w + i), _mm256_loadu_ps(x + i), a0);
    float v[8];
    _mm256_storeu_ps(v, _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a4, a5)));
    float s = hreduce8(v);
    for (; i < n; i++) {
        float p = (float)w[i] * x[i];
        s = s + p;
    }
    return s;
}

const bool g_avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
int g_force_scalar = 0;

inline float dot_f32(const float* x, const float* y, int n) {
    return (g_avx2 && !g_force_scalar) ? dot_f32_avx2(x, y, n) : dot_f32_scalar(x, y, n);
}
inline float dot_i8_f32(const float* x, const int8_t* w, int n) {
    return (g_avx2 && !g_force_scalar) ? dot_i8_f32_avx2(x, w, n) : dot_i8_f32_scalar(x, w, n);
}

// kernels.MatVecInt8 (internal/kernels/int8.go:31-41): y[r] = Dot(x, W[r])*scale, then += bias[r]
// as a separately rounded add.
void matvec_i8(float* y, int rows, const int8_t* w, int stride, float scale, const float* x, int cols,
               const float* bias) {
    for (int r = 0; r < rows; r++) {
        float v = dot_i8_f32(x, w + (size_t)r * stride, cols) * scale;
        if (bias) v = v + bias[r];
        y[r] = v;
    }
}

// One element of vecExpASM_F32 (internal/kernels/vec_amd64.s:281-430): clamp to [-88, 88],
// k = round-to-nearest-even(x*log2e), two-constant ln2 reduction with FMA, the degree-5 polynomial
// as an FMA chain, and 2^k built from exponent bits. The 8-wide loop and the scalar tail compute the
// same function.
float fast_exp(float x) {
    auto bits = [](uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; };
    const float invLn2 = bits(0x3fb8aa3bu), ln2Hi = bits(0x3f317200u), ln2Lo = bits(0x35bfbe8eu);
    const float c2 = bits(0x3f000000u), c3 = bits(0x3e2aaaabu), c4 = bits(0x3d2aaaabu), c5 = bits(0x3c088889u);
    x = (x < 88.0f) ? x : 88.0f;    // VMINPS
    x = (x > -88.0f) ? x : -88.0f;  // VMAXPS
    float k = nearbyintf(x * invLn2);  // VROUNDPS $0 (default MXCSR: nearest even)
    float r = fmaf(-k, ln2Hi, x);
    r = fmaf(-k, ln2Lo, r);
    float p = fmaf(r, c5, c4);
    p = fmaf(r, p, c3);
    p = fmaf(r, p, c2);
    p = fmaf(r, p, 1.0f);
    p = fmaf(r, p, 1.0f);
    int32_t ki = (int32_t)k + 127;
    uint32_t e = (uint32_t)ki << 23;
    return p * bits(e);
}

// nn.SoftmaxInPlaceF32 (internal/nn/head.go:151-172) with kernels.VecExpF32 (AVX2 path).
void softmax_inplace(float* logits, float* scratch, int n) {
    float maxLogit = -FLT_MAX;
    for (int i = 0; i < n; i++)
        if (logits[i] > maxLogit) maxLogit = logits[i];
    for (int i = 0; i < n; i++) scratch[i] = logits[i] - maxLogit;
    for (int i = 0; i < n; i++) logits[i] = fast_exp(scratch[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += logits[i];
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) logits[i] *= inv;
}

// kernels.AddScaledF32 on AVX2 (vecAddScaledASM_F32, internal/kernels/vec_amd64.s:65-123):
// y = fma(alpha, x, y) over 16- and 8-element chunks, unfused multiply then add in the tail.
void add_scaled(float* y, const float* x, float alpha, int n) {
    int i = 0;
    for (; n - i >= 16; i += 16)
        for (int j = 0; j < 16; j++) y[i + j] = fmaf(alpha, x[i + j], y[i + j]);
    if (n - i >= 8) {
        for (int j = 0; j < 8; j++) y[i + j] = fmaf(alpha, x[i + j], y[i + j]);
        i += 8;
    }
    for (; i < n; i++) {
        float p = x[i] * alpha;
        y[i] = p + y[i];
    }
}

// nn.RMSNormForwardF32 (internal/nn/rmsnorm.go:14-32), eps = nn.RMSNormEpsilonF32 = 1e-5.
void rmsnorm(const float* x, const float* gamma, float* out, int D) {
    const float eps = 1e-5f;
    float sumSq = dot_f32(x, x, D);
    float rms = (float)std::sqrt((double)(sumSq / (float)D + eps));
    float inv = 1.0f / rms;
    for (int d = 0; d < D; d++) {
        float hat = x[d] * inv;
        out[d] = hat * gamma[d];
    }
}

// quant.sigmoidClamped (internal/quant/stream.go:127-136), bound ca.SigmoidClampBoundF32 = 15.
inline float sigmoid_clamped(float x) {
    if (x > 15.0f) return 1.0f;
    if (x < -15.0f) return 0.0f;
    return 1.0f / (1.0f + (float)std::exp((double)(-x)));
}

// ca.StepDilation (internal/ca/layout.go:22-30), MaxCADilation = 32 (internal/ca/config.go:58-59).
int step_dilation(int initial, int base, int step) {
    int d = initial;
    for (int s = 0; s < step && d < 32; s++) d *= base;
    return std::min(d, 32);
}

// ---------------------------------------------------------------------------------------------
// Model (internal/quant/model.go, internal/quant/attention.go)
// ---------------------------------------------------------------------------------------------

struct Block {
    int steps = 1, dil_base = 2, init_dil = 1;
    std::vector<int8_t> w1, w2, wsel;  // [2H][3D], [2D][H], [D][D]
    float s1 = 1, s2 = 1, ssel = 1;
    std::vector<float> b1, b2, gamma;   // gamma empty: no normalisation (stream.go:167-171)
    bool has_attn = false;
    std::vector<float> attn_norm;
    std::vector<int8_t> qkv, wo;        // [3D][D], [D][D]
    float sqkv = 1, so = 1;
    int dilation(int step) const { return step_dilation(init_dil, dil_base, step); }
};

}  // namespace

struct OrModel {
    int V, D, H, heads, window, max_context;
    bool tied;
    std::vector<int8_t> embed;  // [V][D]
    float embed_scale = 1;
    std::vector<Block> blocks;
    std::vector<float> final_norm;  // empty: no final normalisation
    std::vector<int8_t> head_w;     // untied head [V][D]
    float head_scale = 1;
    std::vector<float> head_b;      // [V] (empty: no bias)
    std::vector<float> latch_base;  // ca.ComputeSelectiveLatchBaseLogits

    const int8_t* headW() const { return tied ? embed.data() : head_w.data(); }
    float headScale() const { return tied ? embed_scale : head_scale; }
    // quant.Model.normRing (internal/quant/stream.go:37-47)
    int norm_ring() const {
        int longest = 0;
        for (auto& b : blocks)
            for (int s = 0; s < b.steps; s++) longest = std::max(longest, b.dilation(s));
        return longest + 1;
    }
    // quant.Model.attnCache (internal/quant/attention.go:46-52)
    int attn_cache() const { return window > 0 ? window : max_context; }
};

namespace {

// ca.ComputeDecayLatchConstants (internal/ca/layout.go:60-85) and
// ca.ComputeSelectiveLatchBaseLogits (internal/ca/latch.go:9-25).
std::vector<float> latch_base_logits(int D) {
    std::vector<float> base(D);
    const double minT = 1.5, maxT = 64.0;
    for (int d = 0; d < D; d++) {
        double td;
        if (D == 1) {
            td = minT;
        } else {
            double ratio = std::pow(maxT / minT, 1.0 / (double)(D - 1));
            td = minT * std::pow(ratio, (double)d);
        }
        float decay = (float)std::pow(2.0, -1.0 / td);
        double lam = (double)decay;
        if (lam <= 0.0) base[d] = -15.0f;
        else if (lam >= 1.0) base[d] = 15.0f;
        else base[d] = (float)std::log(lam / (1.0 - lam));
    }
    return base;
}

// quantSeqState (internal/quant/stream.go:19-35) plus the per-model scratch vectors, kept per
// state here so a model can be shared by worker threads (the reference serialises on q.mu instead).
struct SeqState {
    int n = 0;
    std::vector<int> step_offset;
    int ring = 1;
    std::vector<std::vector<std::vector<float>>> norm;  // [blockStep][ring][D]
    std::vector<std::vector<float>> latch;              // [blockStep][D]
    int attn_cap = 0;
    std::vector<std::vector<float>> attnK, attnV;       // [block][cap*D]
    std::vector<float> attn_scores, attn_scratch;
    std::vector<float> cur, next, block_in;
    // scratch (quant.Model buffers, model.go:56-66 and attention.go:56-60)
    std::vector<float> mlp_input, mlp_hidden, mlp_gate, mlp_output, latch_logit, norm_scratch, logits;
    std::vector<float> a_norm, a_qkv, a_att, a_proj;

    explicit SeqState(const OrModel& q) {
        int D = q.D;
        ring = q.norm_ring();
        step_offset.resize(q.blocks.size());
        cur.assign(D, 0); next.assign(D, 0); block_in.assign(D, 0);
        int total = 0;
        for (size_t b = 0; b < q.blocks.size(); b++) { step_offset[b] = total; total += q.blocks[b].steps; }
        attn_cap = q.attn_cache();
        attnK.resize(q.blocks.size()); attnV.resize(q.blocks.size());
        for (size_t b = 0; b < q.blocks.size(); b++) {
            if (q.blocks[b].has_attn) {
                attnK[b].assign((size_t)attn_cap * D, 0);
                attnV[b].assign((size_t)attn_cap * D, 0);
                attn_scores.assign(attn_cap, 0);
                attn_scratch.assign(attn_cap, 0);
            }
        }
        norm.assign(total, std::vector<std::vector<float>>(ring, std::vector<float>(D, 0)));
        latch.assign(total, std::vector<float>(D, 0));
        mlp_input.assign(3 * D, 0); mlp_hidden.assign(q.H, 0); mlp_gate.assign(q.H, 0);
        mlp_output.assign(2 * D, 0); latch_logit.assign(D, 0); norm_scratch.assign(D, 0);
        logits.assign(q.V, 0);
        a_norm.assign(D, 0); a_qkv.assign(3 * D, 0); a_att.assign(D, 0); a_proj.assign(D, 0);
    }
    // quantSeqState.bytes (internal/quant/stream.go:87-101): CA caches counted at 8 B per element.
    long long bytes() const {
        long long n = (long long)cur.size() + next.size() + block_in.size();
        for (size_t s = 0; s < norm.size(); s++) {
            for (auto& row : norm[s]) n += row.size();
            n += latch[s].size();
        }
        long long n32 = (long long)attn_scores.size() + attn_scratch.size();
        for (size_t b = 0; b < attnK.size(); b++) n32 += attnK[b].size() + attnV[b].size();
        return n * 8 + n32 * 4;
    }
    // quantSeqState.reset (internal/quant/stream.go:115-121)
    void reset() {
        n = 0;
        for (auto& l : latch) std::fill(l.begin(), l.end(), 0.0f);
    }
};

// The latch update of one channel (internal/quant/stream.go:202): lambda*g + (1 - lambda)*n, each
// product rounded separately.
inline float latch_combine(float lam, float g, float n) {
    float a = lam * g;
    float b = (1.0f - lam) * n;
    return a + b;
}

// quant.Model.updateLatch (internal/quant/stream.go:195-205)
float* update_latch(const OrModel& q, SeqState& st, float* gl, const Block& blk, const float* normCell) {
    int D = q.D;
    matvec_i8(st.latch_logit.data(), D, blk.wsel.data(), D, blk.ssel, normCell, D, q.latch_base.data());
    for (int d = 0; d < D; d++) gl[d] = latch_combine(sigmoid_clamped(st.latch_logit[d]), gl[d], normCell[d]);
    return gl;
}

// quant.Model.applyRule (internal/quant/stream.go:207-230) with ca.AssembleNeighborhood
// (internal/ca/neighborhood.go:13-25).
void apply_rule(const OrModel& q, SeqState& st, const Block& blk, const float* normCell, const float* left,
                const float* latch, const float* self, float* next) {
    int D = q.D, H = q.H, inDim = 3 * D;
    float* x = st.mlp_input.data();
    std::memcpy(x, normCell, D * sizeof(float));
    if (left) std::memcpy(x + D, left, D * sizeof(float));
    else std::fill(x + D, x + 2 * D, 0.0f);
    std::memcpy(x + 2 * D, latch, D * sizeof(float));
    matvec_i8(st.mlp_hidden.data(), H, blk.w1.data(), inDim, blk.s1, x, inDim, blk.b1.data());
    matvec_i8(st.mlp_gate.data(), H, blk.w1.data() + (size_t)H * inDim, inDim, blk.s1, x, inDim, blk.b1.data() + H);
    for (int h = 0; h < H; h++) st.mlp_hidden[h] *= sigmoid_clamped(st.mlp_gate[h]);
    matvec_i8(st.mlp_output.data(), 2 * D, blk.w2.data(), H, blk.s2, st.mlp_hidden.data(), H, blk.b2.data());
    for (int s = 0; s < D; s++) {
        float gate = sigmoid_clamped(st.mlp_output[D + s]);
        float a = (1.0f - gate) * self[s];
        float b = gate * st.mlp_output[s];
        next[s] = a + b;
    }
}

// nn.WindowStart (internal/nn/attention.go:54-60)
inline int window_start(int i, int window) {
    if (window > 0 && i - window + 1 > 0) return i - window + 1;
    return 0;
}

// The attention of one position over keys and values lo..pos (internal/quant/attention.go:82-101): per
// head, scores q.k * (1/sqrt(dh)) in DotF32 order, SoftmaxInPlaceF32, then out += p_j * v_j with
// AddScaledF32. Key and value row j sit at keys/values + (j % ring) * stride; out is [D] and zeroed first.
void attend_heads(const float* query_row, const float* keys, const float* values, size_t stride, int ring, int lo,
                  int pos, int D, int heads, float* scores, float* scratch, float* out) {
    int dh = D / heads, span = pos - lo + 1;
    float scale = (float)(1.0 / std::sqrt((double)dh));
    std::fill(out, out + D, 0.0f);
    for (int h = 0; h < heads; h++) {
        const float* query = query_row + h * dh;
        for (int j = lo; j <= pos; j++) {
            size_t k = (size_t)(j % ring) * stride;
            scores[j - lo] = dot_f32(query, keys + k + h * dh, dh) * scale;
        }
        softmax_inplace(scores, scratch, span);
        float* o = out + h * dh;
        for (int j = lo; j <= pos; j++) {
            size_t v = (size_t)(j % ring) * stride;
            add_scaled(o, values + v + h * dh, scores[j - lo], dh);
        }
    }
}

// quant.Model.attendPosition (internal/quant/attention.go:69-104)
void attend_position(const OrModel& q, SeqState& st, int b, const Block& blk, int pos) {
    int D = q.D, heads = q.heads;
    rmsnorm(st.cur.data(), blk.attn_norm.data(), st.a_norm.data(), D);
    matvec_i8(st.a_qkv.data(), 3 * D, blk.qkv.data(), D, blk.sqkv, st.a_norm.data(), D, nullptr);
    float* keys = st.attnK[b].data();
    float* values = st.attnV[b].data();
    int ring = st.attn_cap;
    int slot = pos % ring;
    std::memcpy(keys + (size_t)slot * D, st.a_qkv.data() + D, D * sizeof(float));
    std::memcpy(values + (size_t)slot * D, st.a_qkv.data() + 2 * D, D * sizeof(float));
    int lo = std::max(window_start(pos, q.window), pos - ring + 1);
    attend_heads(st.a_qkv.data(), keys, values, D, ring, lo, pos, D, heads, st.attn_scores.data(),
                 st.attn_scratch.data(), st.a_att.data());
    matvec_i8(st.a_proj.data(), D, blk.wo.data(), D, blk.so, st.a_att.data(), D, nullptr);
    for (int d = 0; d < D; d++) st.cur[d] += st.a_proj[d];
}

// quant.Model.appendPosition (internal/quant/stream.go:138-193)
void append_position(const OrModel& q, SeqState& st, int token, bool needOutput) {
    int D = q.D;
    int pos = st.n;
    if (token < 0 || token >= q.V) token = 0;
    size_t offset = (size_t)token * D;
    for (int d = 0; d < D; d++) {
        float v = (float)q.embed[offset + d] * q.embed_scale;
        st.cur[d] = v;
        st.block_in[d] = v;
    }
    int numBlocks = (int)q.blocks.size();
    for (int b = 0; b < numBlocks; b++) {
        const Block& blk = q.blocks[b];
        if (b > 0) {
            for (int d = 0; d < D; d++) {
                st.block_in[d] += st.cur[d];
                st.cur[d] = st.block_in[d];
            }
        }
        for (int step = 0; step < blk.steps; step++) {
            int bs = st.step_offset[b] + step;
            float* normCell = st.norm[bs][pos % st.ring].data();
            if ((int)blk.gamma.size() == D) rmsnorm(st.cur.data(), blk.gamma.data(), normCell, D);
            else std::memcpy(normCell, st.cur.data(), D * sizeof(float));
            float* latch = update_latch(q, st, st.latch[bs].data(), blk, normCell);
            if (!needOutput && b == numBlocks - 1 && step == blk.steps - 1 && !blk.has_attn) break;
            const float* left = nullptr;
            int leftIdx = pos - blk.dilation(step);
            if (leftIdx >= 0) left = st.norm[bs][leftIdx % st.ring].data();
            apply_rule(q, st, blk, normCell, left, latch, st.cur.data(), st.next.data());
            std::swap(st.cur, st.next);
        }
        if (blk.has_attn) attend_position(q, st, b, blk, pos);
    }
    st.n++;
}

// quant.Model.headLogits (internal/quant/stream.go:232-248); logits stay fp32 here, the caller
// widens them to float64 exactly as the reference does.
const float* head_logits(const OrModel& q, SeqState& st, const float* cell) {
    int D = q.D;
    if ((int)q.final_norm.size() == D) {
        rmsnorm(cell, q.final_norm.data(), st.norm_scratch.data(), D);
        cell = st.norm_scratch.data();
    }
    matvec_i8(st.logits.data(), q.V, q.headW(), D, q.headScale(), cell, D,
              q.head_b.empty() ? nullptr : q.head_b.data());
    return st.logits.data();
}

// quant.Model.prefill (internal/quant/stream.go:250-261)
const float* prefill(const OrModel& q, SeqState& st, const int* tokens, int n) {
    if (n > q.max_context) {
        tokens += n - q.max_context;
        n = q.max_context;
    }
    st.reset();
    for (int i = 0; i < n; i++) append_position(q, st, tokens[i], i == n - 1);
    return head_logits(q, st, st.cur.data());
}

template <class F>
void parallel_for(int n, int nthreads, F&& f) {
    if (nthreads <= 1 || n <= 1) {
        for (int i = 0; i < n; i++) f(0, i);
        return;
    }
    nthreads = std::min(nthreads, n);
    std::atomic<int> next{0};
    std::vector<std::thread> ts;
    for (int t = 0; t < nthreads; t++)
        ts.emplace_back([&, t] {
            for (int i; (i = next.fetch_add(1)) < n;) f(t, i);
        });
    for (auto& t : ts) t.join();
}

}  // namespace

// quantSession (internal/quant/session.go:11-68)
struct OrSession {
    OrModel* q;
    SeqState st;
    int window;
    std::vector<int> tokens;
    int fed = 0;
    OrSession(OrModel* m, int ctx) : q(m), st(*m) {
        window = m->max_context;
        if (ctx > 0 && ctx < window) window = ctx;
    }
};

extern "C" {

// quant.NewModel (internal/quant/model.go:90-118): maxContext < ca.DefaultMinContextSize (64) is
// replaced by defaultContext = 128 (model.go:11-12).
OrModel* or_model_new(int V, int D, int H, int nblocks, int tied, int heads, int window, int max_context) {
    OrModel* m = new OrModel();
    m->V = V; m->D = D; m->H = H; m->tied = tied != 0; m->heads = heads; m->window = window;
    m->max_context = max_context < 64 ? 128 : max_context;
    m->blocks.resize(nblocks);
    m->latch_base = latch_base_logits(D);
    return m;
}

void or_model_free(OrModel* m) { delete m; }

int or_model_max_context(const OrModel* m) { return m->max_context; }

void or_model_set_embed(OrModel* m, const int8_t* q, float scale) {
    m->embed.assign(q, q + (size_t)m->V * m->D);
    m->embed_scale = scale;
}

void or_model_set_block(OrModel* m, int b, int steps, int dil_base, int init_dil, const int8_t* w1, float s1,
                        const float* b1, const int8_t* w2, float s2, const float* b2, const float* gamma,
                        int gamma_len, const int8_t* wsel, float ssel) {
    Block& k = m->blocks[b];
    int D = m->D, H = m->H;
    k.steps = steps; k.dil_base = dil_base; k.init_dil = init_dil;
    k.w1.assign(w1, w1 + (size_t)2 * H * 3 * D); k.s1 = s1; k.b1.assign(b1, b1 + 2 * H);
    k.w2.assign(w2, w2 + (size_t)2 * D * H); k.s2 = s2; k.b2.assign(b2, b2 + 2 * D);
    k.gamma.assign(gamma, gamma + gamma_len);
    k.wsel.assign(wsel, wsel + (size_t)D * D); k.ssel = ssel;
}

void or_model_set_attn(OrModel* m, int b, const float* norm, const int8_t* qkv, float sqkv, const int8_t* wo,
                       float so) {
    Block& k = m->blocks[b];
    int D = m->D;
    k.has_attn = true;
    k.attn_norm.assign(norm, norm + D);
    k.qkv.assign(qkv, qkv + (size_t)3 * D * D); k.sqkv = sqkv;
    k.wo.assign(wo, wo + (size_t)D * D); k.so = so;
}

void or_model_set_head(OrModel* m, const float* final_norm, int fn_len, const int8_t* head_w, float head_scale,
                       const float* head_b, int hb_len) {
    m->final_norm.assign(final_norm, final_norm + fn_len);
    if (!m->tied && head_w) {
        m->head_w.assign(head_w, head_w + (size_t)m->V * m->D);
        m->head_scale = head_scale;
    }
    m->head_b.assign(head_b, head_b + hb_len);
}

// quant.Model.Call (internal/quant/model.go:120-133). Returns 0 (and writes nothing) for an empty
// input, like the reference's nil.
int or_call(OrModel* m, const int* ids, int n, double* logits) {
    if (n <= 0) return 0;
    SeqState st(*m);
    const float* l = prefill(*m, st, ids, n);
    for (int v = 0; v < m->V; v++) logits[v] = (double)l[v];
    return m->V;
}

OrSession* or_session_new(OrModel* m, int ctx) { return new OrSession(m, ctx); }
void or_session_free(OrSession* s) { delete s; }

// quantSession.Prefill (internal/quant/session.go:30-39, :58-63)
int or_session_prefill(OrSession* s, const int* ids, int n, double* logits) {
    if (n > s->window) {
        ids += n - s->window;
        n = s->window;
    }
    s->tokens.assign(ids, ids + n);
    if (s->tokens.empty()) return 0;
    s->fed = (int)s->tokens.size();
    const float* l = prefill(*s->q, s->st, s->tokens.data(), (int)s->tokens.size());
    for (int v = 0; v < s->q->V; v++) logits[v] = (double)l[v];
    return s->q->V;
}

// quantSession.Append (internal/quant/session.go:41-56)
int or_session_append(OrSession* s, int token, double* logits) {
    s->tokens.push_back(token);
    if ((int)s->tokens.size() > s->window) s->tokens.erase(s->tokens.begin());
    const float* l;
    if (s->fed == 0 || s->st.n != s->fed) {
        s->fed = (int)s->tokens.size();
        l = prefill(*s->q, s->st, s->tokens.data(), (int)s->tokens.size());
    } else {
        append_position(*s->q, s->st, token, true);
        s->fed++;
        l = head_logits(*s->q, s->st, s->st.cur.data());
    }
    for (int v = 0; v < s->q->V; v++) logits[v] = (double)l[v];
    return s->q->V;
}

// quantSession.StateBytes (internal/quant/session.go:65-68)
long long or_session_state_bytes(OrSession* s) { return s->st.bytes(); }

// Teacher-forced logits of every position of B independent sequences of length T: the route the
// reference's genbench times (Prefill(ids[:1]) then Append(ids[t])), which is bit-identical to Call
// over each prefix (internal/quant/session_test.go:18-52). The streaming session is used directly so
// that T may exceed the window, as a session streams past it. logits: [B][T][V] fp32.
int or_forward_all(OrModel* m, const int* ids, int B, int T, float* logits, int nthreads) {
    parallel_for(B, nthreads, [&](int, int b) {
        SeqState st(*m);
        const int* seq = ids + (size_t)b * T;
        for (int t = 0; t < T; t++) {
            append_position(*m, st, seq[t], true);
            const float* l = head_logits(*m, st, st.cur.data());
            std::memcpy(logits + ((size_t)b * T + t) * m->V, l, m->V * sizeof(float));
        }
    });
    return 0;
}

// Greedy decode of B sessions (internal/generate/greedy.go:63-102): Prefill(prompt), then argmax with
// the first maximum, probability 1/sum(exp(l - max)) in float64, and Append(best) while fewer than
// max_tokens tokens were produced. No stop tokens. out_ids/out_probs: [B][max_tokens].
// ctx is the session window (NewSession(ctx)).
int or_greedy(OrModel* m, const int* prompts, int B, int P, int max_tokens, int ctx, int* out_ids,
              double* out_probs, int nthreads) {
    parallel_for(B, nthreads, [&](int, int b) {
        OrSession s(m, ctx);
        std::vector<double> logits(m->V);
        int got = or_session_prefill(&s, prompts + (size_t)b * P, P, logits.data());
        int produced = 0;
        while (produced < max_tokens && got > 0) {
            int best = 0;
            for (int i = 0; i < m->V; i++)
                if (logits[i] > logits[best]) best = i;
            double sum = 0.0;
            for (int i = 0; i < m->V; i++) sum += std::exp(logits[i] - logits[best]);
            out_ids[(size_t)b * max_tokens + produced] = best;
            out_probs[(size_t)b * max_tokens + produced] = 1.0 / sum;
            produced++;
            if (produced < max_tokens) got = or_session_append(&s, best, logits.data());
        }
    });
    return 0;
}

// 1 selects the scalar restatement of the dot kernels even on AVX2 machines (tests compare both).
void or_force_scalar(int on) { g_force_scalar = on; }
int or_has_avx2(void) { return g_avx2 ? 1 : 0; }

// Single-kernel entry points for the kernel-level pins.
float or_dot_f32(const float* x, const float* y, int n) { return dot_f32(x, y, n); }
float or_dot_i8_f32(const float* x, const int8_t* w, int n) { return dot_i8_f32(x, w, n); }
float or_fast_exp(float x) { return fast_exp(x); }
float or_sigmoid_clamped(float x) { return sigmoid_clamped(x); }
void or_rmsnorm(const float* x, const float* gamma, float* out, int D) { rmsnorm(x, gamma, out, D); }
void or_softmax(float* logits, int n) {
    std::vector<float> scratch(n);
    softmax_inplace(logits, scratch.data(), n);
}
void or_add_scaled(float* y, const float* x, float alpha, int n) { add_scaled(y, x, alpha, n); }
void or_matvec_i8(float* y, int rows, const int8_t* w, int stride, float scale, const float* x, int cols,
                  const float* bias) {
    matvec_i8(y, rows, w, stride, scale, x, cols, bias);
}
// Stage-level pins for the engine's batched kernels. The latch recurrence of updateLatch
// (internal/quant/stream.go:195-205) over B sequences of T positions given lambda (the sigmoid of the
// latch logits) and the normalised cells, the latch starting from zero (quantSeqState.reset,
// stream.go:115-121): g[b][t] = lambda*g[b][t-1] + (1 - lambda)*n. Rows of D values, stride ld.
void or_latch_seq(const float* lam, const float* nf, int B, int T, int D, int ld, float* g) {
    for (int b = 0; b < B; b++) {
        std::vector<float> gl(D, 0.0f);
        for (int t = 0; t < T; t++) {
            size_t r = ((size_t)b * T + t) * ld;
            for (int d = 0; d < D; d++) {
                gl[d] = latch_combine(lam[r + d], gl[d], nf[r + d]);
                g[r + d] = gl[d];
            }
        }
    }
}

// attendPosition's attention (internal/quant/attention.go:82-101, without the norm and projections)
// for every position of B sequences of T positions whose q, k, v rows are given ([B*T][3D]: q | k | v):
// position t attends to lo..t with lo = max(WindowStart(t, window), t - cap + 1), as a session whose
// ring holds cap positions. att: [B*T][ld].
void or_attend_seq(const float* qkv, int B, int T, int D, int heads, int window, int cap, float* att, int ld) {
    std::vector<float> scores(T), scratch(T);
    for (int b = 0; b < B; b++) {
        const float* rows = qkv + (size_t)b * T * 3 * D;
        for (int t = 0; t < T; t++) {
            int lo = std::max(window_start(t, window), t - cap + 1);
            attend_heads(rows + (size_t)t * 3 * D, rows + D, rows + 2 * D, (size_t)3 * D, T, lo, t, D, heads,
                         scores.data(), scratch.data(), att + ((size_t)b * T + t) * ld);
        }
    }
}

void or_latch_base(int D, float* out) {
    auto b = latch_base_logits(D);
    std::memcpy(out, b.data(), D * sizeof(float));
}

// quant.NewTensorF32 (internal/quant/tensor.go:12-42): scale = max|w|/127 in fp32, q = clamp(round
// half away from zero of the fp32 quotient w/scale, +-127); an all-zero tensor gets scale 1.
void or_quantize(const float* w, long long n, int8_t* q, float* scale) {
    if (n <= 0) { *scale = 0; return; }
    float maxAbs = 0.0f;
    for (long long i = 0; i < n; i++) {
        float a = (float)std::fabs((double)w[i]);
        if (a > maxAbs) maxAbs = a;
    }
    if (maxAbs == 0) {
        std::memset(q, 0, (size_t)n);
        *scale = 1.0f;
        return;
    }
    float s = maxAbs / 127.0f;
    for (long long i = 0; i < n; i++) {
        double v = std::round((double)(w[i] / s));
        if (v > 127) v = 127;
        else if (v < -127) v = -127;
        q[i] = (int8_t)v;
    }
    *scale = s;
}

// Config-2 GEMM by exact integer arithmetic: acc[m][n] = sum_k A[m][k]*W[n][k] in int64 (checked to
// fit int32), C[m][n] = float(acc)*s[n]. kernels.DotInt8F32 on integer-valued inputs returns the same
// float whenever sum|a*w| < 2^24 (every partial sum is then an exactly representable integer), and
// MatVecInt8 then multiplies once by the scale (internal/kernels/int8.go:8-41).
int or_gemm_i8_exact(const int8_t* A, int M, int K, const int8_t* W, int N, const float* s, float* C,
                     int32_t* acc, int nthreads) {
    std::atomic<int> overflow{0};
    parallel_for(M, nthreads, [&](int, int m) {
        const int8_t* a = A + (size_t)m * K;
        for (int n = 0; n < N; n++) {
            const int8_t* w = W + (size_t)n * K;
            long long sum = 0;
            for (int k = 0; k < K; k++) sum += (int)a[k] * (int)w[k];
            if (sum > INT32_MAX || sum < INT32_MIN) overflow = 1;
            if (acc) acc[(size_t)m * N + n] = (int32_t)sum;
            if (C) C[(size_t)m * N + n] = (float)sum * s[n];
        }
    });
    return overflow.load() ? -1 : 0;
}

// Config-2 GEMM the way the reference computes it: kernels.MatVecInt8 per activation row, the int8
// activations converted to float32 first (DotInt8F32 then one multiply by the channel scale). Used as
// the timed CPU baseline of the standalone GEMM.
int or_gemm_i8_ref(const int8_t* A, int M, int K, const int8_t* W, int N, const float* s, float* C, int nthreads) {
    parallel_for(M, nthreads, [&](int, int m) {
        std::vector<float> x(K);
        for (int k = 0; k < K; k++) x[k] = (float)A[(size_t)m * K + k];
        for (int n = 0; n < N; n++) C[(size_t)m * N + n] = dot_i8_f32(x.data(), W + (size_t)n * K, K) * s[n];
    });
    return 0;
}

}  // extern "C"
