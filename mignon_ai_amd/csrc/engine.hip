// Host side of the engine: device model layout, the batched teacher-forced forward, streaming sessions
// and the C ABI (include/mignon_hip.h).
//
// Execution is step-major: every token in flight advances through one rule step together (the float
// engine's order, internal/ca/forward.go:99-142), which the reference states is equivalent to its
// position-major streaming order (internal/quant/stream.go:11-17). Per block step:
//   row kernel      RMSNorm(cur; gamma) -> n (fp32) and limb-expanded n
//   GEMM LATCH      lambda = sigmoid_clamped(n . W_select^T * s + base)
//   scan            g_t = lambda*g_{t-1} + (1-lambda)*n_t; x = [n_t | n_{t-dil} | g_t] limb-expanded
//   GEMM GLU        h = (x.W1v*s + b1v) * sigmoid_clamped(x.W1g*s + b1g), limb-expanded per 64 units
//   GEMM HIGHWAY    cur = (1-g)*cur + g*o, o = h.W2^T*s + b2
// then the attention sublayer (row kernel, QKV GEMM, windowed attention, Out GEMM into cur) and the
// tied head (row kernel, logits GEMM with fused softmax statistics).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/mignon_hip.h"
#include "common.hpp"
#include "gemm.hpp"
#include "kernels.hpp"
#include "model_file.hpp"
#include "options.hpp"
#include "sample.hpp"
#include "text_abi.hpp"

namespace mg {

std::atomic<int> g_options[OPT_COUNT];

int option(int opt) { return (opt >= 0 && opt < OPT_COUNT) ? g_options[opt].load(std::memory_order_relaxed) : 0; }

int options_key() {
    int k = 0;
    for (int o = 0; o < OPT_COUNT; o++) k = k * 4 + g_options[o].load(std::memory_order_relaxed);
    return k;
}

int set_option(int opt, int value) {
    if (opt < 0 || opt >= OPT_COUNT) return -1;
    if (value < 0) return g_options[opt].load();
    if (value > (opt == OPT_ATTENTION_KERNEL || opt == OPT_STEP_KERNEL ? 3 : 2)) return -1;
    return g_options[opt].exchange(value);
}

namespace {

thread_local std::string g_last_error;

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory) throw Error(MG_ERR_NOMEM, std::string(what) + ": out of device memory");
    if (e == hipErrorInvalidValue) throw Error(MG_ERR_INVALID, std::string(what) + ": invalid launch arguments");
    throw Error(MG_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPCHECK(x) hip_check((x), #x)

void require(bool ok, const std::string& msg) {
    if (!ok) throw Error(MG_ERR_INVALID, msg);
}

struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
    bool borrowed = false;  // points into memory the buffer does not own (never freed or grown)
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { release(); }
    void release() {
        if (p && !borrowed) (void)hipFree(p);
        p = nullptr;
        n = 0;
        borrowed = false;
    }
    void ensure(size_t bytes) {
        if (bytes <= n) return;
        if (borrowed) throw Error(MG_ERR_INVALID, "internal: a borrowed buffer cannot grow");
        release();
        if (bytes == 0) return;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            p = nullptr;
            (void)hipGetLastError();
            throw Error(MG_ERR_NOMEM, "device allocation of " + std::to_string(bytes) + " bytes failed");
        }
        n = bytes;
    }
    template <class T>
    T* as() const { return (T*)p; }
};

struct DevBlock {
    int steps = 1, dil_base = 2, init_dil = 1;
    int8_t* w1 = nullptr; float* b1 = nullptr; float s1 = 0;  // [2Hp][3Dp] value/gate rows paired by 16
    int8_t* w2 = nullptr; float* b2 = nullptr; float s2 = 0;  // [2Dp][Hp] value/gate rows paired by 16
    int8_t* wsel = nullptr; float ssel = 0;                   // [NpD][Dp]
    float* gamma = nullptr;                                   // [Dp] or null (no normalisation)
    bool attn = false;
    float* anorm = nullptr;
    int8_t* qkv = nullptr; float sqkv = 0;                    // [Np3][Dp]
    int8_t* wo = nullptr; float so = 0;                       // [NpD][Dp]
    // ca.StepDilation (internal/ca/layout.go:22-30)
    int dilation(int step) const {
        int d = init_dil;
        for (int s = 0; s < step && d < 32; s++) d *= dil_base;
        return std::min(d, 32);
    }
};

// Kernel classes timed by the optional profiler (HIP events around every launch on the launch stream).
enum KClass : int {
    K_ROW = 0, K_GEMM_LATCH, K_SCAN, K_LATCH_STEP, K_GEMM_GLU, K_GEMM_HIGHWAY, K_GEMM_QKV, K_ATTN, K_ATTN_STEP,
    K_GEMM_OUT, K_GEMM_LOGITS, K_HEAD_COMBINE, K_GEMM_PROBS, K_BITS, K_EXPORT, K_GEMM_I8, K_SAMPLE, K_QKV_ATTN,
    K_STEP1, K_TILE_STEP, K_NCLASS
};
const char* const kClassNames[K_NCLASS] = {
    "row_norm_pack", "gemm_latch", "latch_scan", "latch_step", "gemm_glu", "gemm_highway", "gemm_qkv",
    "attention", "attention_step", "gemm_out", "gemm_logits", "head_combine", "gemm_probs", "bits",
    "state_export", "gemm_i8", "sample", "qkv_attention", "session_step", "tile_step"};

struct Profile {
    bool on = false;
    std::vector<hipEvent_t> pool;
    size_t used = 0;
    struct Rec {
        int cls;
        size_t start;        // index of the start event (end = start + 1)
        double bytes, ops;   // algorithmic HBM bytes and int8 ops of the launch (0: not stated)
    };
    std::vector<Rec> recs;
    ~Profile() {
        for (hipEvent_t e : pool) (void)hipEventDestroy(e);
    }
    hipEvent_t next() {
        if (used == pool.size()) {
            hipEvent_t e;
            if (hipEventCreate(&e) != hipSuccess) throw Error(MG_ERR_DEVICE, "hipEventCreate failed");
            pool.push_back(e);
        }
        return pool[used++];
    }
};

// Records start/end events around the launches in its scope when the model's profiler is on, with the
// algorithmic work the caller states for them: the HBM bytes the launches must move (operands read once,
// results written once) and their int8 multiply-accumulates x 2.
struct ProfScope {
    Profile* p;
    hipStream_t s;
    int cls;
    size_t start = 0;
    double bytes = 0, ops = 0;
    ProfScope(Profile& pr, int c, hipStream_t st, double b = 0, double o = 0)
        : p(pr.on ? &pr : nullptr), s(st), cls(c), bytes(b), ops(o) {
        if (p) {
            start = p->used;
            (void)hipEventRecord(p->next(), s);
        }
    }
    ~ProfScope() {
        if (p) {
            (void)hipEventRecord(p->next(), s);
            p->recs.push_back({cls, start, bytes, ops});
        }
    }
};

// Workspace for a batch of tokens in flight.
struct Workspace {
    int cap_tokens = 0;
    long long gen = 0;  // bumped whenever the buffers below are reallocated (captured graphs hold their addresses)
    DevBuf cur, bin, nf, rinv, lam, nl, ns, xl, xs, h, hl, hs, qkv, att, stats, lse, tlog, logprob, argmax, prob, ids,
        tgt, rowmap, lens, tmp;
    // partial row maxima of the GEMM operands read as fp32: the GLU output's per channel tile, the attention
    // output's per head
    DevBuf hmx, amx;
    // the next block's RMSNorm statistics per row and channel tile of the GEMM that wrote blockIn
    DevBuf ssq, mxg;
};

// Row strides (floats) of the partial-maxima buffers: at least 4 and a multiple of 4 (the fp32-operand
// GEMM reads them as float4s).
int hmx_ld(int Hp) { return round_up(std::max(Hp / 64, 4), 4); }
int amx_ld(int heads) { return round_up(std::max(heads, 4), 4); }
// ... and of the RMSNorm statistics: one entry per channel tile of the highway (2*Dp/128) or out
// projection (NpD/128) GEMM
int stat_ld(const mg_model* m);

}  // namespace
}  // namespace mg

struct mg_model {
    int device = 0;
    int V = 0, D = 0, H = 0, Dp = 0, Hp = 0, heads = 0, window = 0, max_context = 0, ring = 1, cap = 0;
    int NpD = 0, Np3 = 0, Vp = 0, nattn = 0, nbs = 0;
    bool tied = true;
    long long num_params = 0;
    std::vector<std::unique_ptr<mg::DevBuf>> bufs;
    int8_t* emb = nullptr;
    float emb_scale = 0;
    std::vector<mg::DevBlock> blocks;
    int8_t* headw = nullptr;
    float head_scale = 0;
    float* headb = nullptr;
    float* final_norm = nullptr;
    float* latch_base = nullptr;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // caller-owned cancellation flag polled by batched decodes (mg_model_set_cancel); set without the lock
    std::atomic<const volatile int32_t*> cancel{nullptr};
    mg::Step1Block* s1blocks = nullptr;  // device copy of the blocks for step1_kernel
    mg::Workspace ws;
    mg::Workspace* wsp = nullptr;  // while set (an allocation-free call), the workspace in use instead of ws
    mg::Profile prof;
    std::mutex mu;
    // the session set of the last mg_generate_* call, kept for the next call of the same size and window
    // (taken out while a call uses it, so concurrent calls never share it)
    std::atomic<mg_sessions*> gen_cache{nullptr};
};

struct mg_sessions {
    mg_model* m = nullptr;
    int n = 0, window = 0;
    mg::DevBuf norm_ring, g, kring, vring, pos, next_ids, out_ids, out_probs, logits, argmax, prob;
    // K/V ring format, fixed at creation (OPT_KV_RINGS): packed rows in kring/vring with their scales in
    // kscale/vscale, or fp32 rows
    bool kv_packed = false;
    mg::DevBuf kscale, vscale;
    mg::DevBuf sample_ws;  // the sampler's exponentials and row sums
    // stop-token bookkeeping of mg_sessions_decode_greedy_until: per-session reply length, the stopped
    // count, and a ring of pinned host slots the count is copied to after each step (one event each)
    static constexpr int kStopRing = 8;
    mg::DevBuf stop_count, stopped;
    int32_t* stop_host = nullptr;
    hipEvent_t stop_ev[kStopRing] = {};
    // mg_sessions_step with host pointers: device buffers for its ids and outputs and a pinned host
    // mirror (coherent, mapped: io_host_dev is its device address), kept for the life of the set (no
    // allocation per step)
    mg::DevBuf io;
    uint8_t* io_host = nullptr;
    uint8_t* io_host_dev = nullptr;
    // The last step captured as a HIP graph, replayed while what its launches captured is unchanged:
    // the workspace's buffers, the engine options and the output pointers.
    mg::DevBuf col;  // decode column of the graph-replayed steps (advanced by each step on the device)
    struct StepGraph {
        hipGraphExec_t exec = nullptr;
        long long ws_gen = -1;
        int opts = -1;
        static constexpr int kKey = 12;
        const void* ptrs[kKey] = {};
        bool failed = false;  // capture is not possible here: launch one kernel at a time
        void reset() {
            if (exec) (void)hipGraphExecDestroy(exec);
            exec = nullptr;
            ws_gen = -1;
        }
    } graph;
    // kStepsPerGraph consecutive steps of a batched greedy decode captured as one graph (fewer graph
    // boundaries, each of which leaves the device idle for several microseconds)
    StepGraph graph_multi;
    ~mg_sessions() {
        graph.reset();
        graph_multi.reset();
        for (hipEvent_t& e : stop_ev)
            if (e) (void)hipEventDestroy(e);
        if (stop_host) (void)hipHostFree(stop_host);
        if (io_host) (void)hipHostFree(io_host);
    }
};

namespace mg {
namespace {

// Sets of up to this many sessions take the one-workgroup-per-session step automatically.
constexpr int kStep1MaxSessions = 256;

// Whether a new session set of n sessions of this model keeps packed K/V rings: the decode attention of
// every step kernel that can run on the set (attention_step_rows, step1's rk_head) reads them where the
// rows kernel fits the model. Automatic for sets larger than the one-workgroup step takes: there decode
// attention streams the rings of thousands of sessions and reads a quarter fewer bytes; a small set's step
// is a chain of dependent phases, where decoding the rows only lengthens it (one session's Append 58 ->
// 61 us with packed rings).
bool kv_rings_packed(const mg_model* m, int n) {
    const int opt = option(OPT_KV_RINGS);
    if (m->nattn <= 0 || opt == 1 || (opt == 0 && n <= kStep1MaxSessions)) return false;
    AttnStepArgs a;
    a.S = 1; a.D = m->D; a.Dp = m->Dp; a.heads = m->heads; a.window = m->window; a.cap = m->cap;
    return attention_step_rows_fits(a);
}

// The K/V rings of attention block ab of a set: packed words and scales, or fp32 rows.
void ring_args(mg_sessions* s, int ab, AttnStepArgs& a) {
    const mg_model* m = s->m;
    const size_t rows = (size_t)ab * s->n * m->heads * m->cap;  // ring rows of the earlier blocks
    if (s->kv_packed) {
        const size_t words = rows * kv_row_words(m->D / m->heads);
        a.kpack = s->kring.as<uint32_t>() + words; a.vpack = s->vring.as<uint32_t>() + words;
        a.kscale = s->kscale.as<float>() + rows; a.vscale = s->vscale.as<float>() + rows;
    } else {
        const size_t floats = rows * (m->D / m->heads);
        a.kring = s->kring.as<float>() + floats; a.vring = s->vring.as<float>() + floats;
    }
}

template <class T>
T* upload(mg_model* m, const std::vector<T>& h) {
    m->bufs.emplace_back(new DevBuf());
    DevBuf& b = *m->bufs.back();
    b.ensure(std::max<size_t>(h.size() * sizeof(T), 16));
    if (!h.empty()) HIPCHECK(hipMemcpy(b.p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return b.as<T>();
}

// Row-major [Np][Kp] int8 weights -> the GEMM's fragment layout (gemm.hpp).
std::vector<int8_t> frag_pack(const std::vector<int8_t>& w, int Np, int Kp) {
    std::vector<int8_t> out((size_t)Np * Kp);
    for (int n = 0; n < Np; n++)
        for (int k = 0; k < Kp; k++) out[frag_off_w(n, k, Np)] = w[(size_t)n * Kp + k];
    return out;
}

// quant.Model.normRing (internal/quant/stream.go:37-47)
int norm_ring_of(const std::vector<DevBlock>& blocks) {
    int longest = 0;
    for (auto& b : blocks)
        for (int s = 0; s < b.steps; s++) longest = std::max(longest, b.dilation(s));
    return longest + 1;
}

std::vector<float> latch_base_logits(int D) {
    // ca.ComputeDecayLatchConstants + ca.ComputeSelectiveLatchBaseLogits (internal/ca/layout.go:60-85,
    // internal/ca/latch.go:9-25): sigmoid(base_d) = 2^(-1/T_d), T_d geometric from 1.5 to 64 tokens.
    std::vector<float> base(D);
    for (int d = 0; d < D; d++) {
        double td = D == 1 ? 1.5 : 1.5 * std::pow(std::pow(64.0 / 1.5, 1.0 / (double)(D - 1)), (double)d);
        float decay = (float)std::pow(2.0, -1.0 / td);
        double lam = (double)decay;
        base[d] = lam <= 0.0 ? -15.0f : lam >= 1.0 ? 15.0f : (float)std::log(lam / (1.0 - lam));
    }
    return base;
}

void build_device_model(mg_model* m, const HostModel& hm, int max_context) {
    const int V = hm.V, D = hm.D, H = hm.H;
    m->V = V; m->D = D; m->H = H;
    m->Dp = round_up(D, 64);
    m->Hp = round_up(H, 64);
    m->NpD = round_up(m->Dp, LX_BN);
    m->Np3 = round_up(3 * D, LX_BN);
    m->Vp = round_up(V, LX_BN);
    m->tied = hm.tied;
    m->heads = hm.attn_heads;
    m->window = hm.attn_window;
    int ctx = max_context > 0 ? max_context : hm.context_size;
    m->max_context = ctx < 64 ? 128 : ctx;  // quant.NewModel (internal/quant/model.go:91-95)
    m->cap = m->window > 0 ? m->window : m->max_context;
    m->num_params = hm.num_params;
    const int Dp = m->Dp, Hp = m->Hp;

    m->emb = upload(m, hm.embed);
    m->emb_scale = hm.embed_scale;
    m->latch_base = nullptr;
    {
        std::vector<float> base = latch_base_logits(D);
        base.resize(m->NpD, 0.0f);
        m->latch_base = upload(m, base);
    }
    m->blocks.resize(hm.blocks.size());
    m->nattn = 0;
    m->nbs = 0;
    for (size_t b = 0; b < hm.blocks.size(); b++) {
        const HostBlock& hb = hm.blocks[b];
        DevBlock& db = m->blocks[b];
        db.steps = hb.steps;
        db.dil_base = hb.dilation_base;
        db.init_dil = hb.initial_dilation;
        m->nbs += hb.steps;
        // W1: rows regrouped in blocks of 32 = 16 value rows + the 16 matching gate rows; each input
        // segment (n, left, g) padded from D to Dp columns.
        std::vector<int8_t> w1((size_t)2 * Hp * 3 * Dp, 0);
        std::vector<float> b1((size_t)2 * Hp, 0.0f);
        for (int r = 0; r < 2 * Hp; r++) {
            int blk = r / 32, i = r % 32, j = 16 * blk + (i % 16);
            if (j >= H) continue;
            int src = i < 16 ? j : H + j;
            for (int seg = 0; seg < 3; seg++)
                std::memcpy(&w1[(size_t)r * 3 * Dp + seg * Dp], &hb.w1[(size_t)src * 3 * D + seg * D], D);
            b1[r] = hb.b1[src];
        }
        db.w1 = upload(m, frag_pack(w1, 2 * Hp, 3 * Dp)); db.b1 = upload(m, b1); db.s1 = hb.s1;
        // W2: same pairing (16 delta rows + 16 highway-gate rows), hidden columns padded to Hp.
        std::vector<int8_t> w2((size_t)2 * Dp * Hp, 0);
        std::vector<float> b2((size_t)2 * Dp, 0.0f);
        for (int r = 0; r < 2 * Dp; r++) {
            int blk = r / 32, i = r % 32, c = 16 * blk + (i % 16);
            if (c >= D) continue;
            int src = i < 16 ? c : D + c;
            std::memcpy(&w2[(size_t)r * Hp], &hb.w2[(size_t)src * H], H);
            b2[r] = hb.b2[src];
        }
        db.w2 = upload(m, frag_pack(w2, 2 * Dp, Hp)); db.b2 = upload(m, b2); db.s2 = hb.s2;
        std::vector<int8_t> ws((size_t)m->NpD * Dp, 0);
        for (int r = 0; r < D; r++) std::memcpy(&ws[(size_t)r * Dp], &hb.wsel[(size_t)r * D], D);
        db.wsel = upload(m, frag_pack(ws, m->NpD, Dp)); db.ssel = hb.ssel;
        if ((int)hb.gamma.size() == D) {
            std::vector<float> g(hb.gamma);
            g.resize(Dp, 0.0f);
            db.gamma = upload(m, g);
        }
        db.attn = hb.has_attn;
        if (hb.has_attn) {
            m->nattn++;
            std::vector<float> an(hb.attn_norm);
            an.resize(Dp, 0.0f);
            db.anorm = upload(m, an);
            std::vector<int8_t> q((size_t)m->Np3 * Dp, 0);
            for (int r = 0; r < 3 * D; r++) std::memcpy(&q[(size_t)r * Dp], &hb.qkv[(size_t)r * D], D);
            db.qkv = upload(m, frag_pack(q, m->Np3, Dp)); db.sqkv = hb.sqkv;
            std::vector<int8_t> o((size_t)m->NpD * Dp, 0);
            for (int r = 0; r < D; r++) std::memcpy(&o[(size_t)r * Dp], &hb.wo[(size_t)r * D], D);
            db.wo = upload(m, frag_pack(o, m->NpD, Dp)); db.so = hb.so;
        }
    }
    m->ring = norm_ring_of(m->blocks);
    const std::vector<int8_t>& hw = hm.tied ? hm.embed : hm.head_w;
    std::vector<int8_t> head((size_t)m->Vp * Dp, 0);
    for (int r = 0; r < V; r++) std::memcpy(&head[(size_t)r * Dp], &hw[(size_t)r * D], D);
    m->headw = upload(m, frag_pack(head, m->Vp, Dp));
    m->head_scale = hm.tied ? hm.embed_scale : hm.head_scale;
    // vocabulary padding: bias -inf (with zero weight rows) makes its logits -inf, so the head's
    // epilogues need no per-channel validity test
    std::vector<float> hb(m->Vp, -INFINITY);
    for (int v = 0; v < V; v++) hb[v] = (size_t)v < hm.head_b.size() ? hm.head_b[v] : 0.0f;
    m->headb = upload(m, hb);
    if ((int)hm.final_norm.size() == D) {
        std::vector<float> fn(hm.final_norm);
        fn.resize(Dp, 0.0f);
        m->final_norm = upload(m, fn);
    }
    {
        std::vector<Step1Block> sb(m->blocks.size());
        for (size_t b = 0; b < m->blocks.size(); b++) {
            const DevBlock& db = m->blocks[b];
            Step1Block& x = sb[b];
            x.steps = db.steps; x.dil_base = db.dil_base; x.init_dil = db.init_dil; x.attn = db.attn ? 1 : 0;
            x.w1 = db.w1; x.b1 = db.b1; x.s1 = db.s1; x.w2 = db.w2; x.b2 = db.b2; x.s2 = db.s2;
            x.wsel = db.wsel; x.ssel = db.ssel; x.gamma = db.gamma; x.anorm = db.anorm;
            x.qkv = db.qkv; x.sqkv = db.sqkv; x.wo = db.wo; x.so = db.so;
        }
        if (!sb.empty()) m->s1blocks = upload(m, sb);
    }
    if (m->nattn > 0) {
        if (m->heads <= 0 || D % m->heads) throw Error(MG_ERR_FORMAT, "model file: attention heads must divide the state size");
        // every head width up to kMaxHeadWidth runs (the state size is at most 1024); the fallback attention
        // kernel keeps a query's scores in LDS, which bounds the cache
        if (m->cap > kMaxAttnSpan)
            throw Error(MG_ERR_UNSUPPORTED, "attention cache of " + std::to_string(m->cap) + " positions is above the " +
                                                std::to_string(kMaxAttnSpan) + " supported");
    }
}

// ------------------------------------------------------------------------------------------------
// Workspace sizing: every per-token buffer for up to `tokens` rows.
// ------------------------------------------------------------------------------------------------
// The workspace in use: the model's own, or the view of the static scratch an allocation-free call
// installs for its duration.
Workspace& ws_of(mg_model* m) { return m->wsp ? *m->wsp : m->ws; }

int stat_ld(const mg_model* m) { return round_up(std::max(std::max(2 * m->Dp, m->NpD) / LX_BN, 4), 4); }

// Calls f(buffer, bytes) for every workspace buffer that `tokens` rows need.
template <class F>
void ws_sizes(const mg_model* m, Workspace& w, int tokens, F&& f) {
    size_t M = (size_t)tokens;
    const size_t Mp = (size_t)round_up(tokens, LX_ROWS);  // limb operands are read in whole row tiles
    const size_t Dp = m->Dp, Hp = m->Hp, D = m->D;
    f(w.cur, M * Dp * 4);
    f(w.bin, M * Dp * 4);
    f(w.nf, M * Dp * 4);
    f(w.rinv, M * 4);
    f(w.lam, M * Dp * 4);
    f(w.nl, Mp * 3 * Dp);
    f(w.ns, Mp * 4);
    f(w.xl, Mp * 9 * Dp);
    f(w.xs, Mp * 4);
    f(w.h, Mp * Hp * 4);  // rows, or whole 16-row tiles in the fp32-operand fragment order
    f(w.hl, Mp * 3 * Hp);
    f(w.hs, Mp * 4);
    f(w.hmx, M * hmx_ld(m->Hp) * 4);
    f(w.ssq, M * stat_ld(m) * 4);
    f(w.mxg, M * stat_ld(m) * 4);
    if (m->nattn) {
        f(w.qkv, M * 3 * D * 4);
        f(w.att, Mp * Dp * 4);
        f(w.amx, M * amx_ld(m->heads) * 4);
    }
    f(w.stats, M * (m->Vp / LX_BN) * 12);
    f(w.lse, M * 4);
    f(w.tlog, M * 4);
    f(w.logprob, M * 4);
    f(w.argmax, M * 4);
    f(w.prob, M * 8);
    f(w.ids, M * 4);
    f(w.tgt, M * 4);
    f(w.rowmap, M * 4);
    f(w.lens, M * 4);
}

void ensure_ws(mg_model* m, int tokens) {
    Workspace& w = ws_of(m);
    if (tokens <= w.cap_tokens) return;
    w.gen++;
    ws_sizes(m, w, tokens, [](DevBuf& b, size_t bytes) { b.ensure(bytes); });
    w.cap_tokens = tokens;
}

// Lays the buffers `tokens` rows need out in one region, each at a 256-byte boundary: returns the region's
// size, and with base set makes every buffer of w a borrowed view into [base, base + size).
size_t carve_ws(const mg_model* m, Workspace& w, int tokens, uint8_t* base) {
    size_t off = 0;
    ws_sizes(m, w, tokens, [&](DevBuf& b, size_t bytes) {
        off = (off + 255) / 256 * 256;
        if (base) {
            b.release();
            b.p = base + off;
            b.n = bytes;
            b.borrowed = true;
        }
        off += bytes;
    });
    if (base) w.cap_tokens = tokens;
    return off;
}

GemmArgs lx_args(const int8_t* A, const float* As, const int8_t* W, int Np, int Kp, int M, int nvalid, float wscale) {
    GemmArgs g;
    g.A = A; g.As = As;
    g.W = W; g.Np = Np; g.Kp = Kp; g.M = M; g.nvalid = nvalid; g.wscale = wscale;
    return g;
}

int gemm_class(int epi) {
    switch (epi) {
        case EPI_LATCH: return K_GEMM_LATCH;
        case EPI_GLU: return K_GEMM_GLU;
        case EPI_HIGHWAY: return K_GEMM_HIGHWAY;
        case EPI_F32: return K_GEMM_QKV;
        case EPI_RESID: return K_GEMM_OUT;
        case EPI_LOGITS: return K_GEMM_LOGITS;
        case EPI_PROBS: return K_GEMM_PROBS;
        default: return K_GEMM_I8;
    }
}

// Algorithmic work of one limb-expanded GEMM launch over g.M token rows: int8 MACs x 2 at the model's
// unpadded shape (one pass of the weight matrix), and the bytes it must move: the three limb planes and
// row scales of A, the weights and bias once, and what its epilogue reads and writes.
void gemm_work(const mg_model* m, int epi, const GemmArgs& g, double& bytes, double& ops) {
    const double M = g.M, D = m->D, H = m->H, V = m->V;
    double k = 0, rows = 0;
    switch (epi) {
        case EPI_LATCH: k = D; rows = D; break;
        case EPI_GLU: k = 3 * D; rows = 2 * H; break;
        case EPI_HIGHWAY: k = H; rows = 2 * D; break;
        case EPI_F32: k = D; rows = 3 * D; break;
        case EPI_RESID: k = D; rows = D; break;
        default: k = D; rows = V; break;  // EPI_LOGITS, EPI_PROBS
    }
    ops = 2.0 * M * k * rows;
    bytes = M * (3.0 * g.Kp + 4) + (double)g.Kp * g.Np + (g.bias ? 4.0 * g.Np : 0);
    const double nv = g.nvalid;
    switch (epi) {
        case EPI_HIGHWAY:
        case EPI_RESID: bytes += (g.resid ? 12.0 : 8.0) * M * nv; break;  // state read, (blockIn read,) write
        case EPI_LOGITS: bytes += (g.out ? 4.0 * M * nv : 0) + 12.0 * M * g.stats_ld + (g.tgt ? 8.0 * M : 0); break;
        case EPI_PROBS: bytes += 4.0 * M * nv + 4.0 * M; break;
        default: bytes += 4.0 * M * nv; break;
    }
}

void gemm(mg_model* m, int epi, const GemmArgs& g, hipStream_t s) {
    double bytes = 0, ops = 0;
    if (m->prof.on) gemm_work(m, epi, g, bytes, ops);
    ProfScope ps(m->prof, gemm_class(epi), s, bytes, ops);
    HIPCHECK(launch_gemm_lx(epi, g, s));
}

// The GEMM on an fp32 operand (launch_gemm_fa): its algorithmic bytes count the fp32 rows and their
// partial maxima (or RMSNorm statistics, and the 1/rms written) instead of limb planes.
void gemm_fa(mg_model* m, int epi, const GemmArgs& g, hipStream_t s) {
    double bytes = 0, ops = 0;
    if (m->prof.on) {
        gemm_work(m, epi, g, bytes, ops);
        const double per_row = epi == EPI_LATCH ? 8.0 * g.stat_n + 4.0 : 4.0 * g.amax_n;
        bytes += (double)g.M * (4.0 * g.Kp + per_row - (3.0 * g.Kp + 4));
    }
    ProfScope ps(m->prof, gemm_class(epi), s, bytes, ops);
    HIPCHECK(launch_gemm_fa(epi, g, s));
}

// Bytes a row-kernel launch must move: its source rows (the embedding's int8 rows and ids; cur and
// blockIn for the residual; two fp32 rows per position for the rule input, whose left neighbour is a
// re-read of a row already fetched), then its fp32 outputs and the limb planes with their row scales.
double row_bytes(const RowArgs& r) {
    const double M = r.M, D = r.D;
    double b = 0;
    switch (r.mode) {
        case ROW_EMBED: b = M * (4 + D + 8 * D); break;
        case ROW_RESID: b = M * 16 * D; break;
        case ROW_RULE: b = M * 8 * D; break;
        default: b = M * 4 * D + (r.row_map ? 4 * M : 0); break;
    }
    if (r.nout) b += M * 4 * D;
    if (r.rinv) b += M * 4;
    if (r.limbs) b += M * (3.0 * r.Dp + 4);
    return b;
}

// Row kernel helper: mode + optional norm, writes n (fp32) and the limb-expanded copy into ws.nl/ns.
void row_call(mg_model* m, int M, int mode, const int32_t* ids, const float* src, int lds, const int32_t* row_map,
              const float* gamma, float* nout, bool limbs, hipStream_t s, float* rinv = nullptr) {
    Workspace& w = ws_of(m);
    RowArgs r;
    r.M = M; r.D = m->D; r.Dp = m->Dp; r.mode = mode;
    r.ids = ids; r.emb = m->emb; r.emb_scale = m->emb_scale; r.V = m->V;
    r.cur = w.cur.as<float>(); r.block_in = w.bin.as<float>();
    r.src = src; r.lds = lds; r.row_map = row_map; r.gamma = gamma; r.nout = nout; r.rinv = rinv;
    if (limbs) {
        r.limbs = w.nl.as<int8_t>(); r.lscale = w.ns.as<float>();
    }
    ProfScope ps(m->prof, K_ROW, s, row_bytes(r));
    HIPCHECK(launch_row(r, s));
}

__global__ void targets_kernel(int M, int T, const int32_t* ids, int32_t* tgt) {
    int m = blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= M) return;
    tgt[m] = (m % T) < T - 1 ? ids[m + 1] : -1;
}

__global__ void last_rows_kernel(int B, int T, const int32_t* lens, int32_t* rowmap) {
    int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) rowmap[b] = b * T + lens[b] - 1;
}

// Prompt windowing (quantSession.Prefill keeps the last `window` tokens, internal/quant/session.go:30-39)
// into a [S][Tw] token matrix padded with id 0; lengths are clamped to 1..max_len.
__global__ void window_ids_kernel(int S, int max_len, int window, int Tw, const int32_t* in, const int32_t* lens_in,
                                  int32_t* out, int32_t* lens_out) {
    int s = blockIdx.x;
    int len = min(max(lens_in[s], 1), max_len);
    int L = min(len, window), off = len - L;
    for (int t = threadIdx.x; t < Tw; t += blockDim.x) out[(long long)s * Tw + t] = t < L ? in[(long long)s * max_len + off + t] : 0;
    if (threadIdx.x == 0) lens_out[s] = L;
}

// Stop tokens of a batched greedy decode: count[i] is -1 while session i runs, then the column of its first
// stop token (its reply length); *stopped counts sessions that have stopped.
constexpr int kMaxStops = 8;
struct StopSet {
    int32_t id[kMaxStops];
    int n;
};

__global__ void stop_init_kernel(int S, int32_t* count, int32_t* stopped) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < S) count[i] = -1;
    if (i == 0) *stopped = 0;
}

__global__ void stop_scan_kernel(int S, int col, const int32_t* ids, int ld, StopSet stops, int32_t* count,
                                 int32_t* stopped) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= S || count[i] >= 0) return;
    const int32_t t = ids[(long long)i * ld + col];
    bool hit = false;
    for (int k = 0; k < stops.n; k++) hit |= t == stops.id[k];
    if (hit) {
        count[i] = col;
        atomicAdd(stopped, 1);
    }
}

// Sessions without a stop token among the produced columns 0..cut-1 get reply length cut (max_tokens, or
// the column before which a cancellation stopped the decode).
__global__ void stop_finish_kernel(int S, int cut, int32_t* count) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < S && (count[i] < 0 || count[i] > cut)) count[i] = cut;
}

// Scoring windows: row r of a [B][T] token matrix is tokens[start[r] .. start[r] + len[r]), padded with id 0
// (positions past len[r] are never scored, and no position depends on a later one).
__global__ void gather_rows_kernel(int B, int T, const int32_t* tokens, const long long* start, const int32_t* len,
                                   int32_t* out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)B * T) return;
    const int r = (int)(i / T), t = (int)(i - (long long)r * T);
    out[i] = t < len[r] ? tokens[start[r] + t] : 0;
}

// ------------------------------------------------------------------------------------------------
// The model body over M rows. Batched mode (sess == null): rows are B sequences of T positions.
// Prefill export (sess != null, step == false): also writes the session state at each sequence's last
// position. Step mode (step == true): one position per session against its device-resident state.
// On return ws.cur holds the final cell state of every row.
// ------------------------------------------------------------------------------------------------
struct BodyCtx {
    int B = 0, T = 1;
    const int32_t* ids = nullptr;
    mg_sessions* sess = nullptr;
    bool step = false;
    const int32_t* lens = nullptr;  // prefill export lengths (device)
};

void run_body(mg_model* m, const BodyCtx& c, hipStream_t s) {
    Workspace& w = ws_of(m);
    const int M = c.B * c.T;
    const int Dp = m->Dp, Hp = m->Hp, D = m->D;
    int bs = 0, ab = 0;
    // The inter-block residual (blockIn += cur; cur = blockIn, stream.go:157-163) is done by the last GEMM
    // of a block when the next block has steps: it adds its new state into blockIn instead of storing
    // cur. The next block then reads its input from blockIn (norm and first highway), and cur is only
    // written again by that highway.
    bool in_bin = false;  // this block's input is in blockIn, and cur is stale
    // GEMMs that read the GLU output or the attention output as fp32 rows (batched passes; decode steps
    // keep one operand path, so that their kernels stay bit-identical to each other)
    const bool fp32_ops = !c.step && option(OPT_OPERANDS) != 1;
    const int sk = option(OPT_SCAN_KERNEL);
    const bool many = (long long)c.B * ((Dp / 2 + 63) / 64) >= 1024;
    auto fused_scan_at = [&](const DevBlock& blk, int st) {
        return !c.step && scan_rule_fits(c.T, Dp, blk.dilation(st)) && (sk == 2 || (sk == 0 && many));
    };
    // The latch GEMM of a block whose input is in blockIn (added there by the previous block's last GEMM)
    // reads those rows itself and normalises them as it loads them, from RMSNorm statistics that last GEMM
    // writes, where the fp32 operands are on, the fused scan recomputes n (so n itself is never needed) and
    // the kernel takes the shapes. Decided for every block first: the previous block's GEMM must know.
    std::vector<char> norm_fused(m->blocks.size(), 0);
    for (size_t b = 1; b < m->blocks.size(); b++) {
        const DevBlock& pb = m->blocks[b - 1];
        const DevBlock& blk = m->blocks[b];
        const bool prev_into_bin = blk.steps > 0 && (pb.attn || pb.steps > 0);
        if (!fp32_ops || c.sess || !prev_into_bin || !blk.gamma || !fused_scan_at(blk, 0)) continue;
        GemmArgs t;
        t.W = blk.wsel; t.Np = m->NpD; t.Kp = Dp; t.M = M;
        t.Af = w.bin.as<float>(); t.lda = Dp; t.ssq = w.ssq.as<float>(); t.mxg = w.mxg.as<float>();
        t.gamma = blk.gamma; t.rinv = w.rinv.as<float>(); t.D = D; t.stat_ld = stat_ld(m);
        t.stat_n = (pb.attn ? m->NpD : 2 * Dp) / LX_BN;
        norm_fused[b] = gemm_fa_fits(EPI_LATCH, t);
    }
    // the RMSNorm statistics a GEMM writing block b's new blockIn adds, where block b + 1 takes them
    auto stats_for_next = [&](size_t b, GemmArgs& g) {
        if (b + 1 < m->blocks.size() && norm_fused[b + 1]) {
            g.ssq_out = w.ssq.as<float>(); g.mxg_out = w.mxg.as<float>();
            g.gamma_next = m->blocks[b + 1].gamma; g.stat_ld = stat_ld(m);
        }
    };
    for (size_t b = 0; b < m->blocks.size(); b++) {
        const DevBlock& blk = m->blocks[b];
        const int mode = b == 0 ? ROW_EMBED : ROW_RESID;
        const bool fuse_next = b + 1 < m->blocks.size() && m->blocks[b + 1].steps > 0 && (blk.attn || blk.steps > 0);
        if (blk.steps == 0) row_call(m, M, mode, c.ids, nullptr, 0, nullptr, nullptr, nullptr, false, s);
        for (int st = 0; st < blk.steps; st++, bs++) {
            const int dil = blk.dilation(st);
            // The rule input's latch scan: fused with the rule-input packing when it fits and there are
            // enough sequences (one workgroup each; at least 1024 waves: c3's 1024 sequences run faster
            // fused, c1's 64 separate) to cover the latency of its sequential rounds. Without a session
            // export (and with a norm) it recomputes n from the norm's source rows and 1/rms, so n is
            // never stored.
            const bool fused_scan = fused_scan_at(blk, st);
            const bool keep_n = c.step || c.sess || !fused_scan || !blk.gamma;
            float* nout = keep_n ? w.nf.as<float>() : nullptr;
            float* rinv = keep_n ? nullptr : w.rinv.as<float>();
            // the rows the norm reads: blockIn when the previous block added its state there, else cur
            // (the embedding and the residual write both)
            const float* nsrc = (st == 0 && in_bin) ? w.bin.as<float>() : w.cur.as<float>();
            // lambda = sigmoid_clamped(n.W_sel*s + base) (stream.go:195-205) on n = RMSNorm(cur; gamma)
            // (stream.go:166-171): the norm in a row pass (fused with the embedding / residual at step 0) that
            // writes n's limb planes, or, at a block's first step, inside the latch GEMM
            GemmArgs g = lx_args(w.nl.as<int8_t>(), w.ns.as<float>(), blk.wsel, m->NpD, Dp, M, D, blk.ssel);
            g.bias = m->latch_base; g.out = w.lam.as<float>(); g.ldo = Dp;
            if (st == 0 && norm_fused[b]) {
                const DevBlock& pb = m->blocks[b - 1];
                g.Af = w.bin.as<float>(); g.lda = Dp; g.ssq = w.ssq.as<float>(); g.mxg = w.mxg.as<float>();
                g.gamma = blk.gamma; g.rinv = w.rinv.as<float>(); g.D = D; g.stat_ld = stat_ld(m);
                g.stat_n = (pb.attn ? m->NpD : 2 * Dp) / LX_BN;
                gemm_fa(m, EPI_LATCH, g, s);
            } else {
                if (st == 0 && in_bin)
                    row_call(m, M, ROW_SRC, nullptr, w.bin.as<float>(), Dp, nullptr, blk.gamma, nout, true, s, rinv);
                else
                    row_call(m, M, st == 0 ? mode : ROW_SRC, c.ids, nullptr, 0, nullptr, blk.gamma, nout, true, s, rinv);
                gemm(m, EPI_LATCH, g, s);
            }
            if (c.step) {
                LatchStepArgs la;
                la.S = M; la.D = D; la.Dp = Dp; la.dil = dil; la.ring = m->ring;
                la.pos = c.sess->pos.as<int32_t>(); la.lam = w.lam.as<float>(); la.nf = w.nf.as<float>();
                la.g = c.sess->g.as<float>() + (size_t)bs * c.B * Dp;
                la.norm_ring = c.sess->norm_ring.as<float>() + (size_t)bs * c.B * m->ring * Dp;
                la.xl = w.xl.as<int8_t>(); la.xs = w.xs.as<float>();
                // per session: lambda, n, g and the ring's left row in; g, the ring slot and the rule
                // input's limbs out
                ProfScope ps(m->prof, K_LATCH_STEP, s, (double)M * (24.0 * D + 9.0 * Dp + 8));
                HIPCHECK(launch_latch_step(la, s));
            } else {
                // g for every position, written over lambda (each element is read before it is replaced)
                ScanArgs sa;
                sa.B = c.B; sa.T = c.T; sa.D = D; sa.Dp = Dp;
                sa.lam = w.lam.as<float>(); sa.nf = w.nf.as<float>(); sa.g = w.lam.as<float>();
                if (c.sess) {
                    sa.lens = c.lens;
                    sa.g_out = c.sess->g.as<float>() + (size_t)bs * c.B * Dp;
                    ProfScope ps(m->prof, K_EXPORT, s);
                    HIPCHECK(launch_export_ring(c.B, c.T, Dp, m->ring, c.lens, w.nf.as<float>(),
                                                c.sess->norm_ring.as<float>() + (size_t)bs * c.B * m->ring * Dp, s));
                }
                // rule input [n | left | g] (stream.go:180-184), limb-expanded with one scale per row
                if (fused_scan) {
                    sa.dil = dil; sa.xl = w.xl.as<int8_t>(); sa.xs = w.xs.as<float>();
                    if (!keep_n) {
                        sa.nf = nullptr; sa.xn = nsrc; sa.rinv = rinv; sa.gamma = blk.gamma;
                    }
                    // lambda and n in (the left neighbour is a re-read), the rule input's limbs out
                    ProfScope ps(m->prof, K_SCAN, s, (double)M * (8.0 * D + 9.0 * Dp + 4));
                    HIPCHECK(launch_scan_rule(sa, s));
                } else {
                    {
                        ProfScope ps(m->prof, K_SCAN, s, (double)M * 12.0 * D);
                        HIPCHECK(launch_scan(sa, s));
                    }
                    RowArgs r;
                    r.M = M; r.mode = ROW_RULE; r.D = D; r.Dp = 3 * Dp; r.seg = Dp; r.dil = dil; r.T = c.T;
                    r.src = w.nf.as<float>(); r.src2 = w.lam.as<float>();
                    r.limbs = w.xl.as<int8_t>(); r.lscale = w.xs.as<float>();
                    ProfScope ps(m->prof, K_SCAN, s, row_bytes(r));
                    HIPCHECK(launch_row(r, s));
                }
            }
            // cur = highway(cur, W2 h) (stream.go:222-229): on h as fp32 rows where the fp32-operand GEMM
            // takes it (the GLU then also writes each row's partial maxima), else on h's limb planes
            GemmArgs gh = lx_args(w.hl.as<int8_t>(), w.hs.as<float>(), blk.w2, 2 * Dp, Hp, M, D, blk.s2);
            gh.bias = blk.b2; gh.cur = w.cur.as<float>(); gh.ldcur = Dp;
            if (st == 0 && in_bin) gh.cur_in = w.bin.as<float>();
            if (st + 1 == blk.steps && !blk.attn && fuse_next) {
                gh.resid = w.bin.as<float>();
                stats_for_next(b, gh);
            }
            gh.Af = w.h.as<float>();
            gh.amax = w.hmx.as<float>(); gh.amax_ld = hmx_ld(Hp); gh.amax_n = Hp / 64;
            const bool h_fp32 = fp32_ops && gemm_fa_fits(EPI_HIGHWAY, gh);
            // h = GLU(x) (stream.go:214-220) in fp32
            g = lx_args(w.xl.as<int8_t>(), w.xs.as<float>(), blk.w1, 2 * Hp, 3 * Dp, M, m->H, blk.s1);
            g.bias = blk.b1; g.out = w.h.as<float>(); g.ldo = Hp;
            if (h_fp32) {
                g.amax_out = w.hmx.as<float>(); g.amax_out_ld = hmx_ld(Hp);
            }
            gemm(m, EPI_GLU, g, s);
            if (h_fp32) {
                gemm_fa(m, EPI_HIGHWAY, gh, s);
            } else {
                // h limb-expanded with one scale per row
                RowArgs r;
                r.M = M; r.D = m->H; r.Dp = Hp; r.mode = ROW_SRC; r.src = w.h.as<float>(); r.lds = Hp;
                r.limbs = w.hl.as<int8_t>(); r.lscale = w.hs.as<float>();
                {
                    ProfScope ps(m->prof, K_ROW, s, row_bytes(r));
                    HIPCHECK(launch_row(r, s));
                }
                gemm(m, EPI_HIGHWAY, gh, s);
            }
        }
        if (blk.attn) {
            // attendPosition (internal/quant/attention.go:69-104)
            bool att_limbs = false;  // the attention kernel wrote the out projection's operand itself
            row_call(m, M, ROW_SRC, nullptr, nullptr, 0, nullptr, blk.anorm, nullptr, true, s);
            // teacher-forced batches without a session export: the projection fused with attention, when
            // the shapes fit (q, k and v never go through memory)
            QkvAttnArgs qa;
            qa.B = c.B; qa.T = c.T; qa.D = D; qa.Dp = Dp; qa.heads = m->heads; qa.window = m->window; qa.cap = m->cap;
            qa.A = w.nl.as<int8_t>(); qa.As = w.ns.as<float>(); qa.W = blk.qkv; qa.Np3 = m->Np3; qa.wscale = blk.sqkv;
            qa.att = w.att.as<float>();
            const int am = option(OPT_ATTENTION_KERNEL);
            const bool fused = !c.step && !c.sess && (am == ATTN_AUTO || am == ATTN_FUSED) && qkv_attention_fits(qa);
            // cur += W_o att (attention.go:100-103): on att as fp32 rows where the fp32-operand GEMM takes it
            // (the fused attention then also writes each row's per-head maxima)
            GemmArgs go = lx_args(w.nl.as<int8_t>(), w.ns.as<float>(), blk.wo, m->NpD, Dp, M, D, blk.so);
            go.cur = w.cur.as<float>(); go.ldcur = Dp;
            if (fuse_next) {
                go.resid = w.bin.as<float>();
                stats_for_next(b, go);
            }
            go.Af = w.att.as<float>();
            go.amax = w.amx.as<float>(); go.amax_ld = amx_ld(m->heads); go.amax_n = m->heads;
            const bool att_fp32 = fused && fp32_ops && gemm_fa_fits(EPI_RESID, go);
            if (att_fp32) {
                qa.amax = w.amx.as<float>(); qa.amax_ld = amx_ld(m->heads);
            }
            GemmArgs g = lx_args(w.nl.as<int8_t>(), w.ns.as<float>(), blk.qkv, m->Np3, Dp, M, 3 * D, blk.sqkv);
            g.out = w.qkv.as<float>(); g.ldo = 3 * D;
            if (fused) {
                double bytes = 0, ops = 0;
                if (m->prof.on) {
                    gemm_work(m, EPI_F32, g, bytes, ops);
                    bytes += (double)M * (4.0 * D - 4.0 * 3 * D);  // the attention output instead of q, k, v
                }
                ProfScope ps(m->prof, K_QKV_ATTN, s, bytes, ops);
                HIPCHECK(launch_qkv_attention(qa, s));
            } else {
                gemm(m, EPI_F32, g, s);
            }
            if (!fused && c.step) {
                AttnStepArgs aa;
                aa.S = M; aa.D = D; aa.Dp = Dp; aa.heads = m->heads; aa.window = m->window; aa.cap = m->cap;
                aa.pos = c.sess->pos.as<int32_t>(); aa.qkv = w.qkv.as<float>();
                ring_args(c.sess, ab, aa);
                aa.att = w.att.as<float>();
                ProfScope ps(m->prof, K_ATTN_STEP, s);
                if (attention_step_rows_fits(aa)) {
                    // the output goes straight to the out projection's limbs
                    aa.xl = w.nl.as<int8_t>(); aa.xs = w.ns.as<float>();
                    HIPCHECK(launch_attention_step_rows(aa, s));
                    att_limbs = true;
                } else {
                    HIPCHECK(launch_attention_step(aa, s));
                }
            } else if (!fused) {
                if (c.sess) {
                    ProfScope ps(m->prof, K_EXPORT, s);
                    AttnStepArgs r;
                    ring_args(c.sess, ab, r);
                    if (c.sess->kv_packed)
                        HIPCHECK(launch_export_kv_packed(c.B, c.T, D, m->heads, m->cap, c.lens, w.qkv.as<float>(),
                                                         r.kpack, r.vpack, r.kscale, r.vscale, s));
                    else
                        HIPCHECK(launch_export_kv(c.B, c.T, D, m->heads, m->cap, c.lens, w.qkv.as<float>(), r.kring,
                                                  r.vring, s));
                }
                AttnArgs aa;
                aa.B = c.B; aa.T = c.T; aa.D = D; aa.Dp = Dp; aa.heads = m->heads; aa.window = m->window; aa.cap = m->cap;
                aa.qkv = w.qkv.as<float>(); aa.att = w.att.as<float>();
                // q, k and v of every position in, the output row out
                ProfScope ps(m->prof, K_ATTN, s, (double)M * 16.0 * D);
                HIPCHECK(launch_attention(aa, s));
            }
            if (att_fp32) {
                gemm_fa(m, EPI_RESID, go, s);
            } else {
                if (!att_limbs) row_call(m, M, ROW_SRC, nullptr, w.att.as<float>(), Dp, nullptr, nullptr, nullptr, true, s);
                gemm(m, EPI_RESID, go, s);
            }
            ab++;
        }
        in_bin = fuse_next;
    }
    if (m->blocks.empty()) row_call(m, M, ROW_EMBED, c.ids, nullptr, 0, nullptr, nullptr, nullptr, false, s);
}

// Head over M rows of ws.cur (optionally gathered through row_map): final RMSNorm, logits GEMM with
// per-tile softmax statistics, then the per-row combination.
void run_head(mg_model* m, int M, const int32_t* row_map, const int32_t* tgt, float* logits_out, HeadCombineArgs hc,
              hipStream_t s) {
    Workspace& w = ws_of(m);
    // headLogits (internal/quant/stream.go:232-248)
    row_call(m, M, ROW_SRC, nullptr, nullptr, 0, row_map, m->final_norm, nullptr, true, s);
    GemmArgs g = lx_args(w.nl.as<int8_t>(), w.ns.as<float>(), m->headw, m->Vp, m->Dp, M, m->V, m->head_scale);
    g.bias = m->headb; g.out = logits_out; g.ldo = m->V;
    g.stats = w.stats.as<float>(); g.stats_ld = m->Vp / LX_BN;
    g.want_argmax = hc.argmax || hc.next_ids || hc.out_ids;
    g.tgt = tgt; g.tlog = w.tlog.as<float>();
    gemm(m, EPI_LOGITS, g, s);
    hc.M = M; hc.ntiles = m->Vp / LX_BN; hc.stats = w.stats.as<float>(); hc.V = m->V;
    hc.tgt = tgt; hc.tlog = w.tlog.as<float>();
    // the per-tile statistics (and target logits) in; per-row results out
    const double outs = 4.0 * (!!hc.lse + !!hc.argmax + !!hc.logprob + !!hc.next_ids + !!hc.out_ids) +
                        8.0 * (!!hc.prob + !!hc.out_probs);
    ProfScope ps(m->prof, K_HEAD_COMBINE, s, (double)M * (12.0 * hc.ntiles + (tgt ? 8.0 : 0) + outs));
    HIPCHECK(launch_head_combine(hc, s));
}

struct Guard {
    mg_model* m;
    std::lock_guard<std::mutex> lk;
    explicit Guard(mg_model* mm) : m(mm), lk(mm->mu) { HIPCHECK(hipSetDevice(mm->device)); }
};

// Host<->device staging for calls given host pointers.
struct Staging {
    std::vector<std::unique_ptr<DevBuf>> bufs;
    template <class T>
    T* in(const T* host, size_t n, hipStream_t s) {
        bufs.emplace_back(new DevBuf());
        bufs.back()->ensure(std::max<size_t>(n * sizeof(T), 16));
        if (n) HIPCHECK(hipMemcpyAsync(bufs.back()->p, host, n * sizeof(T), hipMemcpyHostToDevice, s));
        return bufs.back()->as<T>();
    }
    template <class T>
    T* out(size_t n) {
        bufs.emplace_back(new DevBuf());
        bufs.back()->ensure(std::max<size_t>(n * sizeof(T), 16));
        return bufs.back()->as<T>();
    }
};

template <class F>
int guarded(F&& f) {
    try {
        return f();
    } catch (const Error& e) {
        g_last_error = e.what();
        return e.code;
    } catch (const FormatError& e) {
        g_last_error = e.what();
        return MG_ERR_FORMAT;
    } catch (const std::bad_alloc&) {
        g_last_error = "host allocation failed";
        return MG_ERR_NOMEM;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return MG_ERR_FORMAT;
    }
}

// Tokens per workspace pass of a teacher-forced batch, at most. c5's 2^21 tokens in one pass: 170.9 ms per
// step against 172.1 in two passes of 2^20 (each kernel's ramp and tail once instead of twice), for ~44 GB
// of workspace instead of ~22.
constexpr long long kMaxChunkTokens = 1 << 21;

// Tokens per pass for this model: kMaxChunkTokens, or fewer where the device's free memory (plus what the
// workspace already holds, which a larger one replaces) would not hold that workspace with a quarter of
// the free memory to spare. At least 1 (a pass that cannot be allocated then fails with MG_ERR_NOMEM).
long long pass_tokens(mg_model* m) {
    Workspace& w = ws_of(m);
    if (w.cap_tokens >= kMaxChunkTokens) return kMaxChunkTokens;
    if (m->wsp) return std::max(1, w.cap_tokens);  // a borrowed workspace cannot grow
    Workspace probe;
    const int sample = 1 << 16;
    const double per_token = (double)carve_ws(m, probe, sample, nullptr) / sample;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) {
        (void)hipGetLastError();
        return kMaxChunkTokens;
    }
    double held = 0;
    ws_sizes(m, w, std::max(w.cap_tokens, 1), [&](DevBuf& b, size_t) { held += (double)b.n; });
    const double budget = 0.75 * (double)free_b + held;
    return std::max<long long>(1, std::min<long long>(kMaxChunkTokens, (long long)(budget / per_token)));
}

// Stop tokens of a batched decode: after each column is written, scan() marks the sessions whose token is
// a stop token and copies the stopped count into a pinned host slot behind an event; keep_going(k) holds
// the host at most kLag steps ahead of the device and says whether step k is still needed: not when every
// session has stopped, nor when the model's cancellation flag is set (generate's Cancel, checked before each
// token: internal/generate/greedy.go:68-70, internal/generate/sample.go:204-206), which cuts every reply
// before column k.
struct StopTracker {
    static constexpr int kLag = 2;
    mg_sessions* s;
    int S, max_tokens;
    int cut;  // columns produced: max_tokens unless cancelled
    StopSet set;
    const int32_t* ids;
    int32_t *cnt, *stopped;
    hipStream_t st;

    StopTracker(mg_sessions* ss, int max_tok, const int32_t* stops, int n_stops, const int32_t* out_ids_d,
                hipStream_t stream)
        : s(ss), S(ss->n), max_tokens(max_tok), cut(max_tok), set{}, ids(out_ids_d), st(stream) {
        set.n = n_stops;
        for (int k = 0; k < n_stops; k++) set.id[k] = stops[k];
        if (!s->stop_host) {
            HIPCHECK(hipHostMalloc((void**)&s->stop_host, mg_sessions::kStopRing * sizeof(int32_t)));
            for (hipEvent_t& e : s->stop_ev) HIPCHECK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        }
        s->stop_count.ensure((size_t)S * 4);
        s->stopped.ensure(16);
        cnt = s->stop_count.as<int32_t>();
        stopped = s->stopped.as<int32_t>();
        hipLaunchKernelGGL(stop_init_kernel, dim3((S + 255) / 256), dim3(256), 0, st, S, cnt, stopped);
        HIPCHECK(hipGetLastError());
    }
    // Without stop tokens no reply ends early: nothing to scan or copy (finish() gives every session `cut`
    // columns); the event alone still keeps the host within kLag steps of the device, so that a
    // cancellation takes effect at the next column.
    void scan(int col) {
        const int slot = col % mg_sessions::kStopRing;
        if (set.n == 0) {
            HIPCHECK(hipEventRecord(s->stop_ev[slot], st));
            return;
        }
        hipLaunchKernelGGL(stop_scan_kernel, dim3((S + 255) / 256), dim3(256), 0, st, S, col, ids, max_tokens, set, cnt,
                           stopped);
        HIPCHECK(hipGetLastError());
        HIPCHECK(hipMemcpyAsync(s->stop_host + slot, stopped, 4, hipMemcpyDeviceToHost, st));
        HIPCHECK(hipEventRecord(s->stop_ev[slot], st));
    }
    bool cancelled() const {
        const volatile int32_t* f = s->m->cancel.load(std::memory_order_acquire);
        return f && *f != 0;
    }
    bool keep_going(int k) {
        const int c = k - 1 - kLag;
        if (c >= 0) {
            const int slot = c % mg_sessions::kStopRing;
            HIPCHECK(hipEventSynchronize(s->stop_ev[slot]));
            if (set.n > 0 && s->stop_host[slot] >= S) return false;
        }
        if (cancelled()) {
            cut = k;
            return false;
        }
        return true;
    }
    void finish() {
        hipLaunchKernelGGL(stop_finish_kernel, dim3((S + 255) / 256), dim3(256), 0, st, S, cut, cnt);
        HIPCHECK(hipGetLastError());
    }
};

// Outputs of a batched decode: device calls leave ids (and probabilities) where they were written and
// only move the reply lengths; host calls copy everything back and wait.
void copy_decode_outputs(bool dev, int S, int max_tokens, const int32_t* oi, const double* op, const int32_t* cnt,
                         int32_t* out_ids, double* out_probs, int32_t* out_counts, hipStream_t st) {
    if (dev) {
        HIPCHECK(hipMemcpyAsync(out_counts, cnt, (size_t)S * 4, hipMemcpyDeviceToDevice, st));
        return;
    }
    HIPCHECK(hipMemcpyAsync(out_ids, oi, (size_t)S * max_tokens * 4, hipMemcpyDeviceToHost, st));
    if (out_probs && op) HIPCHECK(hipMemcpyAsync(out_probs, op, (size_t)S * max_tokens * 8, hipMemcpyDeviceToHost, st));
    HIPCHECK(hipMemcpyAsync(out_counts, cnt, (size_t)S * 4, hipMemcpyDeviceToHost, st));
    HIPCHECK(hipStreamSynchronize(st));
}

}  // namespace
}  // namespace mg

using namespace mg;

// Workspace of the allocation-free decode step (mg_sessions_step_noalloc): one copy of this array per GPU
// the library runs on, held until the process ends. Host code never uses its name as an address (the
// name is a host-side stand-in): kernels get the per-device address scratch_setup resolves.
constexpr size_t kScratchBytes = 64ull << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxScratchDevices] = {};

// Ordering of the allocation-free calls of one device: each model enqueues on its own stream, so a call
// from another stream than the previous call's first waits on the device for the event that call
// recorded (set up with the array; the mutex orders the host side).
struct ScratchOrder {
    std::mutex mu;
    hipEvent_t ev = nullptr;
    hipStream_t last = nullptr;
    bool used = false;
};
ScratchOrder g_scratch_order[kMaxScratchDevices];

// Resolves this device's copy of `scratch`, once per device, with that device current (mg_model_load).
void scratch_setup(int device) {
    require(device >= 0 && device < kMaxScratchDevices, "device index beyond the scratch table");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return;
    void* p = nullptr;
    HIPCHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    require(p != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
    HIPCHECK(hipEventCreateWithFlags(&g_scratch_order[device].ev, hipEventDisableTiming));
    g_scratch_ptr[device] = (uint8_t*)p;
}

uint8_t* scratch_ptr(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return (device >= 0 && device < kMaxScratchDevices) ? g_scratch_ptr[device] : nullptr;
}

}  // namespace

extern "C" {

const char* mg_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"

void mg::set_last_error(const std::string& msg) { g_last_error = msg; }

extern "C" {

int mg_model_load(const uint8_t* data, size_t n, int max_context, mg_model** out) {
    return guarded([&] {
        require(data != nullptr && out != nullptr, "mg_model_load: null argument");
        *out = nullptr;
        HostModel hm = decode_model_file(data, n);
        validate_for_engine(hm);
        std::unique_ptr<mg_model> m(new mg_model());
        HIPCHECK(hipGetDevice(&m->device));
        scratch_setup(m->device);
        build_device_model(m.get(), hm, max_context);
        HIPCHECK(hipStreamCreateWithFlags(&m->own_stream, hipStreamNonBlocking));
        m->stream = m->own_stream;
        HIPCHECK(hipDeviceSynchronize());
        *out = m.release();
        return MG_OK;
    });
}

int mg_model_file_info(const uint8_t* data, size_t n, int max_context, mg_model_info_t* info) {
    return guarded([&] {
        require(data != nullptr && info != nullptr, "mg_model_file_info: null argument");
        HostModel hm = decode_model_file(data, n);
        validate_for_engine(hm);
        std::vector<DevBlock> blocks(hm.blocks.size());
        for (size_t b = 0; b < hm.blocks.size(); b++) {
            blocks[b].steps = hm.blocks[b].steps;
            blocks[b].dil_base = hm.blocks[b].dilation_base;
            blocks[b].init_dil = hm.blocks[b].initial_dilation;
        }
        int ctx = max_context > 0 ? max_context : hm.context_size;
        ctx = ctx < 64 ? 128 : ctx;
        info->vocab_size = hm.V; info->state_size = hm.D; info->hidden_size = hm.H;
        info->num_blocks = (int)hm.blocks.size(); info->attn_heads = hm.attn_heads; info->attn_window = hm.attn_window;
        info->max_context = ctx; info->tied_embed = hm.tied ? 1 : 0;
        info->norm_ring = norm_ring_of(blocks);
        info->attn_cache = hm.attn_window > 0 ? hm.attn_window : ctx;
        info->num_params = hm.num_params;
        return MG_OK;
    });
}

int mg_model_info(const mg_model* m, mg_model_info_t* info) {
    return guarded([&] {
        require(m && info, "mg_model_info: null argument");
        info->vocab_size = m->V; info->state_size = m->D; info->hidden_size = m->H;
        info->num_blocks = (int)m->blocks.size(); info->attn_heads = m->heads; info->attn_window = m->window;
        info->max_context = m->max_context; info->tied_embed = m->tied ? 1 : 0;
        info->norm_ring = m->ring; info->attn_cache = m->cap; info->num_params = m->num_params;
        return MG_OK;
    });
}

int mg_model_set_stream(mg_model* m, void* stream) {
    return guarded([&] {
        require(m != nullptr, "mg_model_set_stream: null model");
        std::lock_guard<std::mutex> lk(m->mu);
        m->stream = stream ? (hipStream_t)stream : m->own_stream;
        return MG_OK;
    });
}

void* mg_model_stream(const mg_model* m) { return m ? (void*)m->stream : nullptr; }

int mg_model_profile(mg_model* m, int on) {
    return guarded([&] {
        require(m != nullptr, "mg_model_profile: null model");
        Guard g(m);
        if (on) {
            m->prof.used = 0;
            m->prof.recs.clear();
        }
        m->prof.on = on != 0;
        return MG_OK;
    });
}

int mg_model_profile_read(mg_model* m, mg_kernel_time_t* out, int max) {
    return guarded([&] {
        require(m != nullptr && (out != nullptr || max == 0), "mg_model_profile_read: null argument");
        Guard g(m);
        HIPCHECK(hipStreamSynchronize(m->stream));
        double ms[K_NCLASS] = {0}, by[K_NCLASS] = {0}, op[K_NCLASS] = {0};
        long long n[K_NCLASS] = {0};
        for (auto& r : m->prof.recs) {
            float t = 0;
            HIPCHECK(hipEventElapsedTime(&t, m->prof.pool[r.start], m->prof.pool[r.start + 1]));
            ms[r.cls] += t;
            by[r.cls] += r.bytes;
            op[r.cls] += r.ops;
            n[r.cls]++;
        }
        int k = 0;
        for (int c = 0; c < K_NCLASS; c++) {
            if (!n[c]) continue;
            if (k < max) {
                std::memset(out[k].name, 0, sizeof(out[k].name));
                std::strncpy(out[k].name, kClassNames[c], sizeof(out[k].name) - 1);
                out[k].launches = n[c];
                out[k].total_ms = ms[c];
                out[k].bytes = by[c];
                out[k].ops = op[c];
            }
            k++;
        }
        return k;
    });
}

int mg_model_set_cancel(mg_model* m, const volatile int32_t* flag) {
    return guarded([&] {
        require(m != nullptr, "mg_model_set_cancel: null model");
        m->cancel.store(flag, std::memory_order_release);  // no lock: a decode in progress may hold it
        return MG_OK;
    });
}

int mg_model_sync(mg_model* m) {
    return guarded([&] {
        require(m != nullptr, "mg_model_sync: null model");
        Guard g(m);
        HIPCHECK(hipStreamSynchronize(m->stream));
        return MG_OK;
    });
}

void mg_model_free(mg_model* m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (mg_sessions* s = m->gen_cache.exchange(nullptr)) mg_sessions_free(s);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->own_stream) (void)hipStreamDestroy(m->own_stream);
    delete m;
}

int mg_forward_batch(mg_model* m, const int32_t* ids, int B, int T, float* logits, float* logprob, float* probs,
                     float* bits, int flags) {
    return guarded([&] {
        require(m && ids, "mg_forward_batch: null argument");
        require(B >= 0 && T >= 0, "mg_forward_batch: negative shape");
        if (B == 0 || T == 0) return MG_OK;
        Guard gd(m);
        hipStream_t s = m->stream;
        const bool dev = flags & MG_PTR_DEVICE;
        const int V = m->V;
        int chunk = (int)std::max<long long>(1, std::min<long long>(B, pass_tokens(m) / std::max(T, 1)));
        ensure_ws(m, chunk * T);
        Workspace& w = ws_of(m);
        Staging st;
        for (int b0 = 0; b0 < B; b0 += chunk) {
            const int Bc = std::min(chunk, B - b0);
            const int M = Bc * T;
            const size_t row0 = (size_t)b0 * T;
            int32_t* ids_d = w.ids.as<int32_t>();
            if (dev) HIPCHECK(hipMemcpyAsync(ids_d, ids + row0, (size_t)M * 4, hipMemcpyDeviceToDevice, s));
            else HIPCHECK(hipMemcpyAsync(ids_d, ids + row0, (size_t)M * 4, hipMemcpyHostToDevice, s));
            hipLaunchKernelGGL(targets_kernel, dim3((M + 255) / 256), dim3(256), 0, s, M, T, ids_d, w.tgt.as<int32_t>());
            HIPCHECK(hipGetLastError());
            BodyCtx c;
            c.B = Bc; c.T = T; c.ids = ids_d;
            run_body(m, c, s);
            float* lg = nullptr;
            if (logits) lg = dev ? logits + row0 * V : st.out<float>((size_t)M * V);
            HeadCombineArgs hc;
            hc.lse = w.lse.as<float>();
            hc.logprob = w.logprob.as<float>();
            run_head(m, M, nullptr, w.tgt.as<int32_t>(), lg, hc, s);
            if (logprob) {
                if (dev) HIPCHECK(hipMemcpyAsync(logprob + row0, w.logprob.p, (size_t)M * 4, hipMemcpyDeviceToDevice, s));
                else HIPCHECK(hipMemcpyAsync(logprob + row0, w.logprob.p, (size_t)M * 4, hipMemcpyDeviceToHost, s));
            }
            if (bits) {
                float* bd = dev ? bits + b0 : st.out<float>((size_t)Bc);
                ProfScope ps(m->prof, K_BITS, s, (double)M * 8.0 + 4.0 * Bc);
                HIPCHECK(launch_bits(Bc, T, w.logprob.as<float>(), ids_d, V, bd, s));
                if (!dev) HIPCHECK(hipMemcpyAsync(bits + b0, bd, (size_t)Bc * 4, hipMemcpyDeviceToHost, s));
            }
            if (probs) {
                float* pd = dev ? probs + row0 * V : st.out<float>((size_t)M * V);
                GemmArgs g = lx_args(w.nl.as<int8_t>(), w.ns.as<float>(), m->headw, m->Vp, m->Dp, M, V, m->head_scale);
                g.bias = m->headb; g.out = pd; g.ldo = V; g.lse = w.lse.as<float>();
                gemm(m, EPI_PROBS, g, s);
                if (!dev) HIPCHECK(hipMemcpyAsync(probs + row0 * V, pd, (size_t)M * V * 4, hipMemcpyDeviceToHost, s));
            }
            if (logits && !dev) HIPCHECK(hipMemcpyAsync(logits + row0 * V, lg, (size_t)M * V * 4, hipMemcpyDeviceToHost, s));
            if (!dev) {
                HIPCHECK(hipStreamSynchronize(s));
                st.bufs.clear();
            }
        }
        return MG_OK;
    });
}

int mg_score_sequences(mg_model* m, const int32_t* tokens, const long long* offsets, int n_seq, int context,
                       float* logprob) {
    return guarded([&] {
        require(m && offsets && logprob, "mg_score_sequences: null argument");
        require(n_seq >= 0, "mg_score_sequences: negative sequence count");
        // window() slices tokens[len-contextSize:], which panics in the reference for a negative size
        // (internal/eval/suite.go:196-198); a context of 0 scores nothing
        require(context >= 0, "mg_score_sequences: negative context");
        require(offsets[0] >= 0, "mg_score_sequences: negative offset");
        long long n_targets = 0;
        for (int q = 0; q < n_seq; q++) {
            require(offsets[q + 1] >= offsets[q], "mg_score_sequences: offsets must not decrease");
            n_targets += std::max<long long>(offsets[q + 1] - offsets[q] - 1, 0);
        }
        const long long n_tok = offsets[n_seq];
        require(n_tok == 0 || tokens, "mg_score_sequences: null tokens");
        const float qnan = std::numeric_limits<float>::quiet_NaN();
        std::fill(logprob, logprob + n_targets, qnan);
        // window(tokens[:t], contextSize) (internal/eval/suite.go:196-198), then Call's truncation to
        // maxContext; an empty window gives no logits and nothing is scored (internal/eval/eval.go:27-33)
        const int W = std::min(context, m->max_context);
        if (n_targets == 0 || W <= 0) return MG_OK;

        // One row per window: the first W targets of a sequence share the row of its first W tokens (the
        // prefix of target t is tokens[0..t), fresh from position 0); every later target t has its own row
        // tokens[t-W .. t), scored at its last position.
        struct Row {
            long long start, out;
            int len, first, count;
        };
        std::vector<Row> rows;
        long long out0 = 0;
        for (int q = 0; q < n_seq; q++) {
            const long long off = offsets[q], L = offsets[q + 1] - offsets[q];
            if (L < 2) continue;
            const int n0 = (int)std::min<long long>(L - 1, W);
            rows.push_back({off, out0, n0, 0, n0});
            for (long long t = W + 1; t < L; t++) rows.push_back({off + t - W, out0 + t - 1, W, W - 1, 1});
            out0 += L - 1;
        }
        std::stable_sort(rows.begin(), rows.end(), [](const Row& a, const Row& b) { return a.len > b.len; });

        long long row_tokens = 0;
        for (const Row& r : rows) row_tokens += r.len;
        // every chunk holds at most `cap` row tokens (cap >= the longest row, so a chunk is never empty)
        Guard gd(m);
        const long long cap =
            std::max<long long>(rows.empty() ? 1 : rows[0].len, std::min<long long>(pass_tokens(m), row_tokens));
        const size_t max_rows = std::min<size_t>(rows.size(), (size_t)cap);

        hipStream_t s = m->stream;
        ensure_ws(m, (int)cap);
        Workspace& w = ws_of(m);
        Staging st;
        int32_t* tok_d = st.in(tokens, (size_t)n_tok, s);
        long long* start_d = st.out<long long>(max_rows);
        int32_t* len_d = st.out<int32_t>(max_rows);
        std::vector<long long> h_start;
        std::vector<int32_t> h_len, h_map, h_tgt;
        std::vector<float> h_lp;
        for (size_t r0 = 0; r0 < rows.size();) {
            const int T = rows[r0].len;
            const size_t r1 = std::min(rows.size(), r0 + (size_t)(cap / T));
            const int B = (int)(r1 - r0);
            h_start.clear(); h_len.clear(); h_map.clear(); h_tgt.clear();
            for (size_t r = r0; r < r1; r++) {
                const Row& row = rows[r];
                h_start.push_back(row.start);
                h_len.push_back(row.len);
                for (int k = 0; k < row.count; k++) {
                    const int pos = row.first + k;
                    h_map.push_back((int32_t)((r - r0) * T + pos));
                    h_tgt.push_back(tokens[row.start + pos + 1]);
                }
            }
            const int Ms = (int)h_map.size();
            HIPCHECK(hipMemcpyAsync(start_d, h_start.data(), (size_t)B * 8, hipMemcpyHostToDevice, s));
            HIPCHECK(hipMemcpyAsync(len_d, h_len.data(), (size_t)B * 4, hipMemcpyHostToDevice, s));
            HIPCHECK(hipMemcpyAsync(w.rowmap.p, h_map.data(), (size_t)Ms * 4, hipMemcpyHostToDevice, s));
            HIPCHECK(hipMemcpyAsync(w.tgt.p, h_tgt.data(), (size_t)Ms * 4, hipMemcpyHostToDevice, s));
            int32_t* ids_d = w.ids.as<int32_t>();
            hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)(((long long)B * T + 255) / 256)), dim3(256), 0, s, B, T,
                               tok_d, start_d, len_d, ids_d);
            HIPCHECK(hipGetLastError());
            BodyCtx c;
            c.B = B; c.T = T; c.ids = ids_d;
            run_body(m, c, s);
            HeadCombineArgs hc;
            hc.logprob = w.logprob.as<float>();
            run_head(m, Ms, w.rowmap.as<int32_t>(), w.tgt.as<int32_t>(), nullptr, hc, s);
            h_lp.resize(Ms);
            HIPCHECK(hipMemcpyAsync(h_lp.data(), w.logprob.p, (size_t)Ms * 4, hipMemcpyDeviceToHost, s));
            HIPCHECK(hipStreamSynchronize(s));
            size_t k = 0;
            for (size_t r = r0; r < r1; r++)
                for (int j = 0; j < rows[r].count; j++) logprob[rows[r].out + j] = h_lp[k++];
            r0 = r1;
        }
        return MG_OK;
    });
}

int mg_model_call(mg_model* m, const int32_t* ids, int n, double* logits) {
    return guarded([&] {
        require(m && logits, "mg_model_call: null argument");
        if (n <= 0) return 0;
        if (n > m->max_context) {  // quant.Model.prefill keeps the most recent maxContext tokens
            ids += n - m->max_context;
            n = m->max_context;
        }
        std::vector<float> all((size_t)n * m->V);
        int rc = mg_forward_batch(m, ids, 1, n, all.data(), nullptr, nullptr, nullptr, 0);
        if (rc != MG_OK) return rc;
        for (int v = 0; v < m->V; v++) logits[v] = (double)all[(size_t)(n - 1) * m->V + v];
        return m->V;
    });
}

namespace {

// A new set's state: empty norm rings, latches and K/V rings, every position 0 (on the model's stream).
void clear_sessions(mg_sessions* s) {
    mg_model* m = s->m;
    HIPCHECK(launch_fill_f32(s->norm_ring.as<float>(), (long long)(s->norm_ring.n / 4), 0.0f, m->stream));
    HIPCHECK(launch_fill_f32(s->g.as<float>(), (long long)(s->g.n / 4), 0.0f, m->stream));
    HIPCHECK(launch_fill_f32(s->kring.as<float>(), (long long)(s->kring.n / 4), 0.0f, m->stream));
    HIPCHECK(launch_fill_f32(s->vring.as<float>(), (long long)(s->vring.n / 4), 0.0f, m->stream));
    if (s->kv_packed) {  // zero words decode to zero under any scale; the scales start at 1
        HIPCHECK(launch_fill_f32(s->kscale.as<float>(), (long long)(s->kscale.n / 4), 1.0f, m->stream));
        HIPCHECK(launch_fill_f32(s->vscale.as<float>(), (long long)(s->vscale.n / 4), 1.0f, m->stream));
    }
    HIPCHECK(launch_fill_i32(s->pos.as<int32_t>(), s->n, 0, m->stream));
}

}  // namespace

int mg_sessions_create(mg_model* m, int n, int context, mg_sessions** out) {
    return guarded([&] {
        require(m && out, "mg_sessions_create: null argument");
        require(n > 0, "mg_sessions_create: n must be positive");
        *out = nullptr;
        Guard gd(m);
        std::unique_ptr<mg_sessions> s(new mg_sessions());
        s->m = m;
        s->n = n;
        s->window = (context > 0 && context < m->max_context) ? context : m->max_context;
        const size_t Dp = m->Dp, D = m->D;
        s->norm_ring.ensure(std::max<size_t>(16, (size_t)m->nbs * n * m->ring * Dp * 4));
        s->g.ensure(std::max<size_t>(16, (size_t)m->nbs * n * Dp * 4));
        s->kv_packed = kv_rings_packed(m, n);
        // packed: 3 bytes per element and a 4-byte scale per (head, slot) row; fp32: 4 bytes per element
        const size_t ring_bytes = (size_t)m->nattn * n * m->cap * D * (s->kv_packed ? 3 : 4);
        s->kring.ensure(std::max<size_t>(16, ring_bytes));
        s->vring.ensure(std::max<size_t>(16, ring_bytes));
        if (s->kv_packed) {
            s->kscale.ensure(std::max<size_t>(16, (size_t)m->nattn * n * m->heads * m->cap * 4));
            s->vscale.ensure(std::max<size_t>(16, (size_t)m->nattn * n * m->heads * m->cap * 4));
        }
        s->pos.ensure((size_t)n * 4);
        s->next_ids.ensure((size_t)n * 4);
        clear_sessions(s.get());
        HIPCHECK(hipStreamSynchronize(m->stream));
        *out = s.release();
        return MG_OK;
    });
}

extern "C++" {
namespace mg {

int generate_sessions_acquire(mg_model* m, int n, int context, mg_sessions** out) {
    mg_sessions* s = m->gen_cache.exchange(nullptr);
    const int window = (context > 0 && context < m->max_context) ? context : m->max_context;
    if (s && (s->n != n || s->window != window)) {
        mg_sessions_free(s);
        s = nullptr;
    }
    if (!s) return mg_sessions_create(m, n, context, out);
    std::unique_ptr<mg_sessions, void (*)(mg_sessions*)> hold(s, mg_sessions_free);
    return guarded([&] {
        Guard gd(m);
        clear_sessions(hold.get());  // on the model's stream, ahead of the call's prefill
        *out = hold.release();
        return MG_OK;
    });
}

void generate_sessions_release(mg_model* m, mg_sessions* s) {
    if (mg_sessions* old = m->gen_cache.exchange(s)) mg_sessions_free(old);
}

}  // namespace mg
}  // extern "C++"

namespace {

// Batched prefill on device-resident windowed prompts; leaves the head statistics in ws.
void prefill_device(mg_sessions* s, const int32_t* prompts_d, const int32_t* lens_d, int max_len, float* logits_d,
                    HeadCombineArgs hc, hipStream_t st) {
    mg_model* m = s->m;
    const int S = s->n;
    const int Tw = std::min(max_len, s->window);
    ensure_ws(m, S * Tw);
    Workspace& w = ws_of(m);
    w.tmp.ensure((size_t)S * Tw * 4);
    int32_t* ids_w = w.tmp.as<int32_t>();
    int32_t* lens_w = w.lens.as<int32_t>();
    hipLaunchKernelGGL(window_ids_kernel, dim3(S), dim3(128), 0, st, S, max_len, s->window, Tw, prompts_d, lens_d, ids_w, lens_w);
    HIPCHECK(hipGetLastError());
    BodyCtx c;
    c.B = S; c.T = Tw; c.ids = ids_w; c.sess = s; c.lens = lens_w;
    run_body(m, c, st);
    hipLaunchKernelGGL(last_rows_kernel, dim3((S + 255) / 256), dim3(256), 0, st, S, Tw, lens_w, w.rowmap.as<int32_t>());
    HIPCHECK(hipGetLastError());
    run_head(m, S, w.rowmap.as<int32_t>(), nullptr, logits_d, hc, st);
    HIPCHECK(launch_set_pos(S, lens_w, s->pos.as<int32_t>(), 0, st));
}

// The one-workgroup-per-session step for this set, when the option and the shapes allow it (automatically
// for sets of up to kStep1MaxSessions).
// The arguments both single-kernel steps share.
bool step1_args_fill(mg_sessions* s, const int32_t* ids_d, float* logits_d, const HeadCombineArgs& hc, Step1Args& a) {
    mg_model* m = s->m;
    a.S = s->n; a.D = m->D; a.Dp = m->Dp; a.H = m->H; a.Hp = m->Hp; a.V = m->V; a.Vp = m->Vp;
    a.NpD = m->NpD; a.Np3 = m->Np3; a.heads = m->nattn ? m->heads : 0; a.window = m->window; a.cap = m->cap;
    a.ring = m->ring; a.nblocks = (int)m->blocks.size(); a.blocks = m->s1blocks;
    a.emb = m->emb; a.emb_scale = m->emb_scale; a.headw = m->headw; a.headb = m->headb; a.head_scale = m->head_scale;
    a.final_norm = m->final_norm; a.latch_base = m->latch_base;
    a.pos = s->pos.as<int32_t>(); a.g = s->g.as<float>(); a.norm_ring = s->norm_ring.as<float>();
    if (s->kv_packed) {
        a.kpack = s->kring.as<uint32_t>(); a.vpack = s->vring.as<uint32_t>();
        a.kscale = s->kscale.as<float>(); a.vscale = s->vscale.as<float>();
    } else {
        a.kring = s->kring.as<float>(); a.vring = s->vring.as<float>();
    }
    a.ids = ids_d; a.logits = logits_d; a.argmax = hc.argmax; a.prob = hc.prob; a.next_ids = hc.next_ids;
    a.out_ids = hc.out_ids; a.out_probs = hc.out_probs; a.out_ld = hc.out_ld; a.out_col = hc.out_col; a.col = hc.col;
    a.done = hc.done;
    return true;
}

bool step1_args(mg_sessions* s, const int32_t* ids_d, float* logits_d, const HeadCombineArgs& hc, Step1Args& a) {
    mg_model* m = s->m;
    const int mode = option(OPT_STEP_KERNEL);
    if (mode == 1 || mode == 3 || (mode == 0 && s->n > kStep1MaxSessions) || !m->s1blocks) return false;
    return step1_args_fill(s, ids_d, logits_d, hc, a) && step1_fits(a);
}

// The decode attention of the tiled step (between its segments): its shape, for the fit check.
AttnStepArgs step_attn_args(mg_sessions* s, int ab) {
    mg_model* m = s->m;
    Workspace& w = ws_of(m);
    AttnStepArgs aa;
    aa.S = s->n; aa.D = m->D; aa.Dp = m->Dp; aa.heads = m->heads; aa.window = m->window; aa.cap = m->cap;
    aa.pos = s->pos.as<int32_t>(); aa.qkv = w.qkv.as<float>();
    ring_args(s, ab, aa);
    aa.xl = w.nl.as<int8_t>(); aa.xs = w.ns.as<float>();
    return aa;
}

// Algorithmic work of one segment of the tiled step over S sessions (the profiler's figures): int8 MACs x 2
// of its matrix products at the unpadded shapes; the bytes memory must move: its weights once, and per
// session the state rows in and out (cur, blockIn), the latch state and norm ring per block step, the
// attention output's limbs in, q/k/v out, and the logits when they are written.
void tile_work(const mg_model* m, int S, int seg_block, bool seg_out, bool logits, double& bytes, double& ops) {
    const double D = m->D, H = m->H, V = m->V, Dp = m->Dp;
    double macs = 0, wbytes = 0, per = 0;
    int b = seg_block;
    if (seg_out) {
        macs += D * D; wbytes += (double)m->Dp * m->NpD;
        per += 8.0 * Dp + 3.0 * Dp + 4;  // cur and blockIn in, attention limbs and scale in
        b++;
    }
    bool ended = false;
    for (; b < (int)m->blocks.size() && !ended; b++) {
        const DevBlock& B = m->blocks[b];
        for (int st = 0; st < B.steps; st++) {
            macs += D * D + 3.0 * D * 2.0 * H + H * 2.0 * D;
            wbytes += (double)m->Dp * m->NpD + 3.0 * m->Dp * 2.0 * m->Hp + (double)m->Hp * 2.0 * m->Dp;
            per += 8.0 * D + 8.0 * D;  // g read and written, norm ring slot written and the left row read
        }
        if (B.attn) {
            macs += 3.0 * D * D; wbytes += (double)m->Dp * m->Np3;
            per += 12.0 * D + 8.0 * Dp;  // q, k, v and the state rows out
            ended = true;
        }
    }
    if (!ended) {
        macs += D * V; wbytes += (double)m->Dp * m->Vp;
        per += 24.0 + (logits ? 4.0 * V : 0.0);
    }
    ops = 2.0 * S * macs;
    bytes = wbytes + S * per;
}

// The tiled step (16 sessions per workgroup), when the option and the shapes allow it: automatic for
// sets larger than the fused step takes.
bool tile_args(mg_sessions* s, const int32_t* ids_d, float* logits_d, const HeadCombineArgs& hc, TileStepArgs& a) {
    mg_model* m = s->m;
    const int mode = option(OPT_STEP_KERNEL);
    if (!(mode == 3 || mode == 0) || !m->s1blocks) return false;
    Step1Args& b = a;
    if (!step1_args_fill(s, ids_d, logits_d, hc, b)) return false;
    if (m->nattn && !attention_step_rows_fits(step_attn_args(s, 0))) return false;
    return tile_step_fits(a);
}

void step_device(mg_sessions* s, const int32_t* ids_d, float* logits_d, HeadCombineArgs hc, hipStream_t st) {
    mg_model* m = s->m;
    const int S = s->n;
    Step1Args s1;
    if (!hc.lse && !hc.logprob && step1_args(s, ids_d, logits_d, hc, s1)) {
        {
            ProfScope ps(m->prof, K_STEP1, st);
            HIPCHECK(launch_step1(s1, st));
        }
        if (hc.col) HIPCHECK(launch_advance(const_cast<int32_t*>(hc.col), st));
        return;
    }
    TileStepArgs ta;
    if (!hc.lse && !hc.logprob && tile_args(s, ids_d, logits_d, hc, ta)) {
        ensure_ws(m, S);
        Workspace& w = ws_of(m);
        ta.cur = w.cur.as<float>(); ta.bin = w.bin.as<float>(); ta.qkv = w.qkv.as<float>();
        ta.att_xl = w.nl.as<int8_t>(); ta.att_xs = w.ns.as<float>();
        int ab = 0;
        for (;;) {
            {
                double bytes = 0, ops = 0;
                if (m->prof.on) tile_work(m, S, ta.seg_block, ta.seg_out != 0, logits_d != nullptr, bytes, ops);
                ProfScope ps(m->prof, K_TILE_STEP, st, bytes, ops);
                HIPCHECK(launch_tile_step(ta, st));
            }
            int next = ta.seg_out ? ta.seg_block + 1 : ta.seg_block;
            while (next < (int)m->blocks.size() && !m->blocks[next].attn) next++;
            if (next >= (int)m->blocks.size()) break;
            {
                // the segment ended with block next's projection: its attention, output limbs to w.nl/w.ns
                AttnStepArgs aa = step_attn_args(s, ab);
                aa.done = hc.done;
                ProfScope ps(m->prof, K_ATTN_STEP, st);
                HIPCHECK(launch_attention_step_rows(aa, st));
            }
            ab++;
            ta.seg_block = next;
            ta.seg_out = 1;
        }
        if (hc.col) HIPCHECK(launch_advance(const_cast<int32_t*>(hc.col), st));
        return;
    }
    ensure_ws(m, S);
    BodyCtx c;
    c.B = S; c.T = 1; c.ids = ids_d; c.sess = s; c.step = true;
    run_body(m, c, st);
    run_head(m, S, nullptr, nullptr, logits_d, hc, st);
    HIPCHECK(launch_set_pos(S, nullptr, s->pos.as<int32_t>(), 1, st, const_cast<int32_t*>(hc.col)));
}

}  // namespace

int mg_sessions_prefill(mg_sessions* s, const int32_t* prompts, const int32_t* lens, int max_len, float* logits,
                        int32_t* argmax, double* prob, int flags) {
    return guarded([&] {
        require(s && prompts && lens, "mg_sessions_prefill: null argument");
        require(max_len > 0, "mg_sessions_prefill: max_len must be positive");
        mg_model* m = s->m;
        Guard gd(m);
        hipStream_t st = m->stream;
        const bool dev = flags & MG_PTR_DEVICE;
        const int S = s->n;
        if (!dev)
            for (int i = 0; i < S; i++)
                require(lens[i] >= 1 && lens[i] <= max_len, "mg_sessions_prefill: lengths must be in 1..max_len");
        Staging sg;
        const int32_t* p_d = dev ? prompts : sg.in(prompts, (size_t)S * max_len, st);
        const int32_t* l_d = dev ? lens : sg.in(lens, (size_t)S, st);
        float* lg = logits ? (dev ? logits : sg.out<float>((size_t)S * m->V)) : nullptr;
        HeadCombineArgs hc;
        hc.argmax = argmax ? (dev ? argmax : sg.out<int32_t>(S)) : nullptr;
        hc.prob = prob ? (dev ? prob : sg.out<double>(S)) : nullptr;
        prefill_device(s, p_d, l_d, max_len, lg, hc, st);
        if (!dev) {
            if (logits) HIPCHECK(hipMemcpyAsync(logits, lg, (size_t)S * m->V * 4, hipMemcpyDeviceToHost, st));
            if (argmax) HIPCHECK(hipMemcpyAsync(argmax, hc.argmax, (size_t)S * 4, hipMemcpyDeviceToHost, st));
            if (prob) HIPCHECK(hipMemcpyAsync(prob, hc.prob, (size_t)S * 8, hipMemcpyDeviceToHost, st));
            HIPCHECK(hipStreamSynchronize(st));
        }
        return MG_OK;
    });
}

namespace {

// The device column counter of a batched decode, set to 1 (the prefill wrote column 0).
const int32_t* start_columns(mg_sessions* s, hipStream_t st) {
    s->col.ensure(4);
    HIPCHECK(launch_fill_i32(s->col.as<int32_t>(), 1, 1, st));
    return s->col.as<int32_t>();
}

// One decode step of every session (step_device), replayed from a captured HIP graph when the options
// allow it and the profiler is off: a step is ~10 launches per block of a few microseconds each at small
// batches, and the graph removes their host-side enqueue cost. Batched decodes pass the output column
// through hc.col (device memory the step advances), so one graph serves every column. The graph is
// captured again when the workspace was reallocated, an option changed or the arguments differ; if
// capture fails the set falls back to launching kernel by kernel.
// Steps of a batched greedy decode replayed from one graph (where the decode has no per-step host work).
constexpr int kStepsPerGraph = 8;

// `nsteps` consecutive steps (1, or kStepsPerGraph for a batched decode whose output column advances on
// the device) replayed from one captured graph, or launched kernel by kernel where graphs are off.
void step_graphed(mg_sessions* s, const int32_t* ids_d, float* logits_d, const HeadCombineArgs& hc, hipStream_t st,
                  int nsteps = 1) {
    mg_model* m = s->m;
    const int mode = option(OPT_STEP_GRAPH);
    auto& G = nsteps == 1 ? s->graph : s->graph_multi;
    // A step that is one kernel (the single-workgroup step, outside a batched decode) is launched directly
    // unless graphs are forced: a graph launch costs more than the one kernel launch it would replace.
    Step1Args one;
    const bool one_kernel = mode == 0 && !hc.col && !hc.lse && !hc.logprob && step1_args(s, ids_d, logits_d, hc, one);
    if (mode == 1 || m->prof.on || G.failed || one_kernel) {
        for (int i = 0; i < nsteps; i++) step_device(s, ids_d, logits_d, hc, st);
        return;
    }
    ensure_ws(m, s->n);  // before any capture: no allocation may happen inside one
    const void* ptrs[mg_sessions::StepGraph::kKey] = {ids_d, logits_d, hc.argmax, hc.prob, hc.next_ids, hc.out_ids, hc.out_probs,
                                hc.col, (const void*)(intptr_t)hc.out_ld, (const void*)(intptr_t)hc.out_col,
                                hc.lse, hc.done};
    const bool same = G.exec && G.ws_gen == ws_of(m).gen && G.opts == options_key() &&
                      std::equal(ptrs, ptrs + G.kKey, G.ptrs);
    if (!same) {
        G.reset();
        hipGraph_t graph = nullptr;
        bool ok = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) == hipSuccess;
        if (ok) {
            try {
                for (int i = 0; i < nsteps; i++) step_device(s, ids_d, logits_d, hc, st);
            } catch (const Error&) {
                ok = false;
            }
            ok = hipStreamEndCapture(st, &graph) == hipSuccess && ok && graph;
        }
        if (ok) ok = hipGraphInstantiateWithFlags(&G.exec, graph, 0) == hipSuccess;
        if (graph) (void)hipGraphDestroy(graph);
        if (!ok) {
            (void)hipGetLastError();
            G.reset();
            G.failed = true;
            for (int i = 0; i < nsteps; i++) step_device(s, ids_d, logits_d, hc, st);
            return;
        }
        G.ws_gen = ws_of(m).gen;
        G.opts = options_key();
        std::copy(ptrs, ptrs + G.kKey, G.ptrs);
    }
    HIPCHECK(hipGraphLaunch(G.exec, st));
}

}  // namespace

int mg_sessions_step(mg_sessions* s, const int32_t* ids, float* logits, int32_t* argmax, double* prob, int flags) {
    return guarded([&] {
        require(s && ids, "mg_sessions_step: null argument");
        mg_model* m = s->m;
        Guard gd(m);
        hipStream_t st = m->stream;
        const bool dev = flags & MG_PTR_DEVICE;
        const int S = s->n;
        if (dev) {
            HeadCombineArgs hc;
            hc.argmax = argmax;
            hc.prob = prob;
            step_graphed(s, ids, logits, hc, st);
            return MG_OK;
        }
        // host pointers: the set's own device buffers and pinned mirror [ids | logits | argmax | prob].
        // When the one-workgroup step runs, its single kernel reads the ids from and writes the outputs to
        // the pinned mirror itself (no copies); otherwise the mirror is staged through the device buffers.
        auto up = [](size_t b) { return (b + 255) / 256 * 256; };
        const size_t o_lg = up((size_t)S * 4), o_am = o_lg + up((size_t)S * m->V * 4), o_pb = o_am + up((size_t)S * 4),
                     total = o_pb + (size_t)S * 8;
        if (s->io.n < total) {
            s->io.ensure(total);
            if (s->io_host) (void)hipHostFree(s->io_host);
            s->io_host = s->io_host_dev = nullptr;
            HIPCHECK(hipHostMalloc((void**)&s->io_host, total, hipHostMallocCoherent | hipHostMallocMapped));
            HIPCHECK(hipHostGetDevicePointer((void**)&s->io_host_dev, s->io_host, 0));
        }
        uint8_t* h = s->io_host;
        std::memcpy(h, ids, (size_t)S * 4);
        Step1Args probe;
        const bool direct = step1_args(s, nullptr, nullptr, HeadCombineArgs{}, probe);
        uint8_t* d = direct ? s->io_host_dev : s->io.as<uint8_t>();
        if (!direct) HIPCHECK(hipMemcpyAsync(d, h, (size_t)S * 4, hipMemcpyHostToDevice, st));
        HeadCombineArgs hc;
        hc.argmax = argmax ? (int32_t*)(d + o_am) : nullptr;
        hc.prob = prob ? (double*)(d + o_pb) : nullptr;
        float* lg = logits ? (float*)(d + o_lg) : nullptr;
        step_graphed(s, (const int32_t*)d, lg, hc, st);
        if (!direct) {
            if (logits) HIPCHECK(hipMemcpyAsync(h + o_lg, lg, (size_t)S * m->V * 4, hipMemcpyDeviceToHost, st));
            if (argmax) HIPCHECK(hipMemcpyAsync(h + o_am, hc.argmax, (size_t)S * 4, hipMemcpyDeviceToHost, st));
            if (prob) HIPCHECK(hipMemcpyAsync(h + o_pb, hc.prob, (size_t)S * 8, hipMemcpyDeviceToHost, st));
        }
        HIPCHECK(hipStreamSynchronize(st));
        if (logits) std::memcpy(logits, h + o_lg, (size_t)S * m->V * 4);
        if (argmax) std::memcpy(argmax, h + o_am, (size_t)S * 4);
        if (prob) std::memcpy(prob, h + o_pb, (size_t)S * 8);
        return MG_OK;
    });
}

int mg_sessions_step_noalloc(mg_sessions* s, const int32_t* ids, float* logits, int32_t* argmax, double* prob) {
    return guarded([&] {
        require(s && ids, "mg_sessions_step_noalloc: null argument");
        mg_model* m = s->m;
        Guard gd(m);
        uint8_t* base = scratch_ptr(m->device);
        require(base != nullptr, "mg_sessions_step_noalloc: the scratch array of this device is not set up");
        Workspace view;
        const size_t need = carve_ws(m, view, s->n, nullptr);
        if (need > kScratchBytes)
            throw Error(MG_ERR_INVALID, "mg_sessions_step_noalloc: " + std::to_string(s->n) + " sessions of this model need " +
                                            std::to_string(need) + " bytes of scratch; it holds " +
                                            std::to_string(kScratchBytes) + " (use mg_sessions_step)");
        carve_ws(m, view, s->n, base);
        // the view replaces the model's workspace for this call only; the profiler (which creates events)
        // is paused
        struct Use {
            mg_model* m;
            bool prof;
            ~Use() {
                m->wsp = nullptr;
                m->prof.on = prof;
            }
        } use{m, m->prof.on};
        m->wsp = &view;
        m->prof.on = false;
        HeadCombineArgs hc;
        hc.argmax = argmax;
        hc.prob = prob;
        // after the previous allocation-free call of this device, whichever stream it was on (not under
        // stream capture, where a wait on an event recorded outside the capture is not allowed: a caller
        // capturing these calls orders them itself)
        ScratchOrder& o = g_scratch_order[m->device];
        std::lock_guard<std::mutex> lk(o.mu);
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        HIPCHECK(hipStreamIsCapturing(m->stream, &cs));
        const bool capturing = cs != hipStreamCaptureStatusNone;
        if (!capturing && o.used && o.last != m->stream) HIPCHECK(hipStreamWaitEvent(m->stream, o.ev, 0));
        step_device(s, ids, logits, hc, m->stream);
        if (!capturing) {
            HIPCHECK(hipEventRecord(o.ev, m->stream));
            o.last = m->stream;
            o.used = true;
        }
        return MG_OK;
    });
}

int mg_sessions_decode_greedy(mg_sessions* s, const int32_t* prompts, const int32_t* lens, int max_len,
                              int max_tokens, int32_t* out_ids, double* out_probs, int flags) {
    return guarded([&] {
        require(s && prompts && lens && out_ids, "mg_sessions_decode_greedy: null argument");
        require(max_len > 0 && max_tokens >= 0, "mg_sessions_decode_greedy: bad lengths");
        if (max_tokens == 0) return MG_OK;
        mg_model* m = s->m;
        Guard gd(m);
        hipStream_t st = m->stream;
        const bool dev = flags & MG_PTR_DEVICE;
        const int S = s->n;
        if (!dev)
            for (int i = 0; i < S; i++)
                require(lens[i] >= 1 && lens[i] <= max_len, "mg_sessions_decode_greedy: lengths must be in 1..max_len");
        Staging sg;
        const int32_t* p_d = dev ? prompts : sg.in(prompts, (size_t)S * max_len, st);
        const int32_t* l_d = dev ? lens : sg.in(lens, (size_t)S, st);
        int32_t* oi = dev ? out_ids : sg.out<int32_t>((size_t)S * max_tokens);
        double* op = out_probs ? (dev ? out_probs : sg.out<double>((size_t)S * max_tokens)) : nullptr;
        HeadCombineArgs hc;
        hc.next_ids = s->next_ids.as<int32_t>();
        hc.out_ids = oi; hc.out_probs = op; hc.out_ld = max_tokens; hc.out_col = 0;
        prefill_device(s, p_d, l_d, max_len, nullptr, hc, st);
        hc.col = start_columns(s, st);
        int k = 1;
        for (; k + kStepsPerGraph <= max_tokens; k += kStepsPerGraph)
            step_graphed(s, s->next_ids.as<int32_t>(), nullptr, hc, st, kStepsPerGraph);
        for (; k < max_tokens; k++) step_graphed(s, s->next_ids.as<int32_t>(), nullptr, hc, st);
        if (!dev) {
            HIPCHECK(hipMemcpyAsync(out_ids, oi, (size_t)S * max_tokens * 4, hipMemcpyDeviceToHost, st));
            if (out_probs) HIPCHECK(hipMemcpyAsync(out_probs, op, (size_t)S * max_tokens * 8, hipMemcpyDeviceToHost, st));
            HIPCHECK(hipStreamSynchronize(st));
        }
        return MG_OK;
    });
}

int mg_sessions_decode_greedy_until(mg_sessions* s, const int32_t* prompts, const int32_t* lens, int max_len,
                                    int max_tokens, const int32_t* stops, int n_stops, int32_t* out_ids,
                                    double* out_probs, int32_t* out_counts, int flags) {
    return guarded([&] {
        require(s && prompts && lens && out_ids && out_counts, "mg_sessions_decode_greedy_until: null argument");
        require(max_len > 0 && max_tokens >= 0, "mg_sessions_decode_greedy_until: bad lengths");
        require(n_stops >= 0 && n_stops <= kMaxStops && (n_stops == 0 || stops),
                "mg_sessions_decode_greedy_until: at most 8 stop tokens");
        mg_model* m = s->m;
        Guard gd(m);
        hipStream_t st = m->stream;
        const bool dev = flags & MG_PTR_DEVICE;
        const int S = s->n;
        if (!dev)
            for (int i = 0; i < S; i++)
                require(lens[i] >= 1 && lens[i] <= max_len,
                        "mg_sessions_decode_greedy_until: lengths must be in 1..max_len");
        if (max_tokens == 0) {
            if (!dev) std::fill(out_counts, out_counts + S, 0);
            else HIPCHECK(launch_fill_i32(out_counts, S, 0, st));
            return MG_OK;
        }
        Staging sg;
        const int32_t* p_d = dev ? prompts : sg.in(prompts, (size_t)S * max_len, st);
        const int32_t* l_d = dev ? lens : sg.in(lens, (size_t)S, st);
        int32_t* oi = dev ? out_ids : sg.out<int32_t>((size_t)S * max_tokens);
        double* op = out_probs ? (dev ? out_probs : sg.out<double>((size_t)S * max_tokens)) : nullptr;
        StopTracker tr(s, max_tokens, stops, n_stops, oi, st);
        HeadCombineArgs hc;
        hc.next_ids = s->next_ids.as<int32_t>();
        hc.out_ids = oi; hc.out_probs = op; hc.out_ld = max_tokens; hc.out_col = 0;
        prefill_device(s, p_d, l_d, max_len, nullptr, hc, st);
        tr.scan(0);
        const bool first = tr.keep_going(0);  // false: cancelled before the first token
        hc.col = start_columns(s, st);
        hc.done = tr.cnt;  // sessions past their stop token need no further steps
        for (int k = 1; first && k < max_tokens && tr.keep_going(k); k++) {
            step_graphed(s, s->next_ids.as<int32_t>(), nullptr, hc, st);
            tr.scan(k);
        }
        tr.finish();
        copy_decode_outputs(dev, S, max_tokens, oi, op, tr.cnt, out_ids, out_probs, out_counts, st);
        return MG_OK;
    });
}

int mg_sessions_decode_sample(mg_sessions* s, const int32_t* prompts, const int32_t* lens, int max_len, int max_tokens,
                              const mg_sampling_t* sp, const uint64_t* seeds, const int32_t* stops, int n_stops,
                              int32_t* out_ids, int32_t* out_counts, int flags) {
    return guarded([&] {
        require(s && prompts && lens && sp && seeds && out_ids && out_counts, "mg_sessions_decode_sample: null argument");
        require(max_len > 0 && max_tokens >= 0, "mg_sessions_decode_sample: bad lengths");
        require(n_stops >= 0 && n_stops <= kMaxStops && (n_stops == 0 || stops),
                "mg_sessions_decode_sample: at most 8 stop tokens");
        mg_model* m = s->m;
        if (m->V > kMaxSampleVocab)
            throw Error(MG_ERR_UNSUPPORTED, "mg_sessions_decode_sample: vocabularies above " +
                                                std::to_string(kMaxSampleVocab) + " tokens are not supported");
        Guard gd(m);
        hipStream_t st = m->stream;
        const bool dev = flags & MG_PTR_DEVICE;
        const int S = s->n, V = m->V;
        if (!dev)
            for (int i = 0; i < S; i++)
                require(lens[i] >= 1 && lens[i] <= max_len, "mg_sessions_decode_sample: lengths must be in 1..max_len");
        if (max_tokens == 0) {
            if (!dev) std::fill(out_counts, out_counts + S, 0);
            else HIPCHECK(launch_fill_i32(out_counts, S, 0, st));
            return MG_OK;
        }
        Staging sg;
        const int32_t* p_d = dev ? prompts : sg.in(prompts, (size_t)S * max_len, st);
        const int32_t* l_d = dev ? lens : sg.in(lens, (size_t)S, st);
        const uint64_t* seed_d = dev ? seeds : sg.in(seeds, (size_t)S, st);
        int32_t* oi = dev ? out_ids : sg.out<int32_t>((size_t)S * max_tokens);
        s->logits.ensure((size_t)S * V * 4);
        float* lg = s->logits.as<float>();
        StopTracker tr(s, max_tokens, stops, n_stops, oi, st);
        SampleArgs sa;
        sa.n = S; sa.V = V; sa.n2 = sample_n2(V);
        sa.logits32 = lg; sa.ld = V;
        if (sp->penalize_prompt) {
            sa.prefix = p_d; sa.prefix_ld = max_len; sa.prefix_len = l_d;
        }
        sa.hist = oi; sa.hist_ld = max_tokens; sa.trigram = true;
        sa.p.temperature = sp->temperature; sa.p.rep_penalty = sp->rep_penalty;
        sa.p.top_p = sp->top_p; sa.p.top_k = sp->top_k;
        sa.seeds = seed_d;
        sa.out = oi; sa.out_ld = max_tokens;
        sa.next_ids = s->next_ids.as<int32_t>();
        s->sample_ws.ensure(sample_scratch_bytes(S, V));
        sa.scratch = s->sample_ws.as<double>();
        sa.sums = sa.scratch + (size_t)S * V;
        sa.flags = (int32_t*)(sa.sums + S);
        auto pick = [&](int col) {
            sa.col = col; sa.step = col; sa.out_col = col;
            ProfScope ps(m->prof, K_SAMPLE, st);
            HIPCHECK(launch_sample(sa, st));
            tr.scan(col);
        };
        HeadCombineArgs hc;  // the sampler, not the argmax, picks each token
        prefill_device(s, p_d, l_d, max_len, lg, hc, st);
        pick(0);
        const bool first = tr.keep_going(0);  // false: cancelled before the first token
        if (n_stops > 0) hc.done = tr.cnt;  // sessions past their stop token need no further steps
        for (int k = 1; first && k < max_tokens && tr.keep_going(k); k++) {
            step_graphed(s, s->next_ids.as<int32_t>(), lg, hc, st);
            pick(k);
        }
        tr.finish();
        copy_decode_outputs(dev, S, max_tokens, oi, nullptr, tr.cnt, out_ids, nullptr, out_counts, st);
        return MG_OK;
    });
}

int mg_sample_logits(const double* logits, int n, int V, const int32_t* recent, const int32_t* recent_len,
                     int recent_ld, const mg_sampling_t* sp, const double* u, int32_t* out) {
    return guarded([&] {
        require(logits && sp && u && out && (recent == nullptr || recent_len), "mg_sample_logits: null argument");
        require(n >= 0 && V > 0 && recent_ld >= 0, "mg_sample_logits: bad shape");
        if (V > kMaxSampleVocab)
            throw Error(MG_ERR_UNSUPPORTED, "mg_sample_logits: vocabularies above " + std::to_string(kMaxSampleVocab) +
                                                " tokens are not supported");
        if (n == 0) return MG_OK;
        int dev = 0;
        HIPCHECK(hipGetDevice(&dev));
        hipStream_t st = nullptr;
        Staging sg;
        SampleArgs sa;
        sa.n = n; sa.V = V; sa.n2 = sample_n2(V);
        sa.logits64 = sg.in(logits, (size_t)n * V, st); sa.ld = V;
        if (recent) {
            for (int i = 0; i < n; i++)
                require(recent_len[i] >= 0 && recent_len[i] <= recent_ld, "mg_sample_logits: bad recent length");
            sa.prefix = sg.in(recent, (size_t)n * recent_ld, st);
            sa.prefix_ld = recent_ld;
            sa.prefix_len = sg.in(recent_len, (size_t)n, st);
        }
        sa.p.temperature = sp->temperature; sa.p.rep_penalty = sp->rep_penalty;
        sa.p.top_p = sp->top_p; sa.p.top_k = sp->top_k;
        sa.u = sg.in(u, (size_t)n, st);
        int32_t* o = sg.out<int32_t>((size_t)n);
        sa.out = o; sa.out_ld = 1;
        sa.scratch = sg.out<double>(sample_scratch_bytes(n, V) / sizeof(double));
        sa.sums = sa.scratch + (size_t)n * V;
        sa.flags = (int32_t*)(sa.sums + n);
        HIPCHECK(launch_sample(sa, st));
        HIPCHECK(hipMemcpyAsync(out, o, (size_t)n * 4, hipMemcpyDeviceToHost, st));
        HIPCHECK(hipStreamSynchronize(st));
        return MG_OK;
    });
}

long long mg_sessions_state_bytes(const mg_sessions* s) {
    if (!s) return -1;
    // quantSeqState.bytes (internal/quant/stream.go:87-101): CA caches at 8 bytes per element, attention
    // rings and score scratch at 4.
    const mg_model* m = s->m;
    long long n = 3LL * m->D + (long long)m->nbs * ((long long)m->ring * m->D + m->D);
    long long n32 = m->nattn > 0 ? 2LL * m->cap : 0;
    n32 += (long long)m->nattn * 2 * m->cap * m->D;
    return n * 8 + n32 * 4;
}

long long mg_sessions_device_bytes(const mg_sessions* s) {
    if (!s) return -1;
    const mg_model* m = s->m;
    // packed rings: 3 bytes per element and a 4-byte scale per (head, slot) row of each ring
    const long long rings = s->kv_packed ? (long long)m->nattn * 2 * m->cap * ((long long)m->D * 3 + m->heads * 4)
                                         : (long long)m->nattn * 2 * m->cap * m->D * 4;
    return (long long)m->nbs * (m->ring + 1) * m->Dp * 4 + rings + 8;
}

int mg_sessions_count(const mg_sessions* s) { return s ? s->n : -1; }

void mg_sessions_free(mg_sessions* s) {
    if (!s) return;
    (void)hipSetDevice(s->m->device);
    (void)hipStreamSynchronize(s->m->stream);
    delete s;
}

int mg_gemm_i8(const int8_t* A, int M, int K, const int8_t* W, int N, const float* scale, float* C, int32_t* acc,
               int flags, void* stream) {
    return guarded([&] {
        require(A && W && scale && (C || acc), "mg_gemm_i8: null argument");
        require(M >= 0 && K > 0 && N > 0, "mg_gemm_i8: bad shape");
        if (M == 0) return MG_OK;
        hipStream_t st = (hipStream_t)stream;
        const bool dev = flags & MG_PTR_DEVICE;
        const int Kp = round_up(K, GEMM_BK), Np = round_up(N, GEMM_BN);
        Staging sg;
        // Operands in the kernel's padded layout when K or N is not a multiple of the tile; otherwise
        // device operands are used in place.
        const int8_t* a_d = A;
        const int8_t* w_d = W;
        if (!dev || Kp != K) {
            int8_t* ap = sg.out<int8_t>((size_t)M * Kp);
            if (Kp != K) HIPCHECK(hipMemsetAsync(ap, 0, (size_t)M * Kp, st));
            HIPCHECK(hipMemcpy2DAsync(ap, Kp, A, K, K, M, dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st));
            a_d = ap;
        }
        if (!dev || Kp != K || Np != N) {
            int8_t* wp = sg.out<int8_t>((size_t)Np * Kp);
            HIPCHECK(hipMemsetAsync(wp, 0, (size_t)Np * Kp, st));
            HIPCHECK(hipMemcpy2DAsync(wp, Kp, W, K, K, N, dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st));
            w_d = wp;
        }
        const float* s_d = dev ? scale : sg.in(scale, (size_t)N, st);
        float* c_d = C ? (dev ? C : sg.out<float>((size_t)M * N)) : nullptr;
        int32_t* i_d = acc ? (dev ? acc : sg.out<int32_t>((size_t)M * N)) : nullptr;
        if (!c_d) c_d = sg.out<float>((size_t)M * N);
        GemmArgs g;
        g.A = a_d; g.a_row = Kp;
        g.W = w_d; g.ldw = Kp; g.Np = Np; g.Kp = Kp; g.M = M; g.nvalid = N;
        g.wscale_n = s_d; g.out = c_d; g.ldo = N; g.out_i32 = i_d;
        HIPCHECK(launch_gemm_c2(g, st));
        if (dev && !sg.bufs.empty()) HIPCHECK(hipStreamSynchronize(st));  // padded copies die on return
        if (!dev) {
            if (C) HIPCHECK(hipMemcpyAsync(C, c_d, (size_t)M * N * 4, hipMemcpyDeviceToHost, st));
            if (acc) HIPCHECK(hipMemcpyAsync(acc, i_d, (size_t)M * N * 4, hipMemcpyDeviceToHost, st));
            HIPCHECK(hipStreamSynchronize(st));
        }
        return MG_OK;
    });
}

int mg_quantize_f32(const float* w, long long n, int8_t* q, float* scale, int flags, void* stream) {
    return guarded([&] {
        require(w && q && scale, "mg_quantize_f32: null argument");
        require(n >= 0, "mg_quantize_f32: negative length");
        hipStream_t st = (hipStream_t)stream;
        const bool dev = flags & MG_PTR_DEVICE;
        if (n == 0) {  // NewTensorF32 of an empty slice: empty tensor, scale 0
            if (dev) HIPCHECK(hipMemsetAsync(scale, 0, 4, st));
            else *scale = 0.0f;
            return MG_OK;
        }
        Staging sg;
        const float* w_d = dev ? w : sg.in(w, (size_t)n, st);
        int8_t* q_d = dev ? q : sg.out<int8_t>((size_t)n);
        float* s_d = dev ? scale : sg.out<float>(1);
        float* tmp = sg.out<float>(4);
        HIPCHECK(launch_quantize(w_d, n, q_d, s_d, tmp, st));
        if (!dev) {
            HIPCHECK(hipMemcpyAsync(q, q_d, (size_t)n, hipMemcpyDeviceToHost, st));
            HIPCHECK(hipMemcpyAsync(scale, s_d, 4, hipMemcpyDeviceToHost, st));
            HIPCHECK(hipStreamSynchronize(st));
        } else {
            HIPCHECK(hipStreamSynchronize(st));  // the temporaries above are released on return
        }
        return MG_OK;
    });
}

int mg_engine_option(int opt, int value) {
    const int prev = set_option(opt, value);
    if (prev < 0) {
        g_last_error = "mg_engine_option: unknown option " + std::to_string(opt) + " or value " + std::to_string(value);
        return MG_ERR_INVALID;
    }
    return prev;
}

}  // extern "C"
