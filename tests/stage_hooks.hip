// Test hooks: single-stage launches of the engine's own kernels on caller-owned device buffers, so that
// a test can give one stage exactly the inputs the oracle gets and compare its output bit for bit. Test
// infrastructure only: not part of the engine's C ABI (include/mignon_hip.h), built by
// tests/stage_hooks.py into tests/_build/libmg_stage_hooks.so against the engine library, whose
// launchers it calls. Every hook launches on the null stream, waits for it, and returns the HIP status
// (0 = success).
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace {

int finish(hipError_t launched) {
    if (launched != hipSuccess) return (int)launched;
    return (int)hipStreamSynchronize(nullptr);
}

}  // namespace

extern "C" {

// Digest of the engine headers this library was compiled against (the loader compares it with the
// current headers': a stale library would pass misplaced argument fields to the engine's launchers).
const char* mgt_headers_digest(void) { return MGT_HEADERS_DIGEST; }

// The row kernel in ROW_SRC mode over M rows of D values (row stride Dp, a multiple of 64): RMSNorm with
// gamma (null: a copy) into nout ([M][Dp], or null), and the limb expansion into the GEMM operand layout
// (limbs: [ceil(M/16)][Dp/64][3][1 KiB], lscale: [M]; both null for none).
int mgt_row(const float* x, int M, int D, int Dp, const float* gamma, float* nout, int8_t* limbs, float* lscale) {
    mg::RowArgs r;
    r.M = M; r.D = D; r.Dp = Dp; r.mode = mg::ROW_SRC;
    r.src = x; r.lds = Dp; r.gamma = gamma; r.nout = nout; r.limbs = limbs; r.lscale = lscale;
    return finish(mg::launch_row(r, nullptr));
}

// The latch scan (scan_kernel) over B sequences of T positions: g[m] for every row m from lambda and the
// normalised rows ([B*T][Dp] each).
int mgt_latch_scan(const float* lam, const float* nf, int B, int T, int D, int Dp, float* g) {
    mg::ScanArgs a;
    a.B = B; a.T = T; a.D = D; a.Dp = Dp; a.lam = lam; a.nf = nf; a.g = g;
    return finish(mg::launch_scan(a, nullptr));
}

// Batched attention over B sequences of T positions (qkv: [B*T][3D], att: [B*T][Dp]). kernel 0: the
// launcher's own choice under the engine's attention option; 1: the one-wave-per-(row, head) kernel.
int mgt_attention(const float* qkv, int B, int T, int D, int Dp, int heads, int window, int cap, float* att,
                  int kernel) {
    if (kernel == 1) {
        mg::AttnWaveArgs w;
        w.rows = B * T; w.T = T; w.D = D; w.Dp = Dp; w.heads = heads; w.dh = heads > 0 ? D / heads : 0;
        w.window = window; w.cap = cap; w.qkv = qkv; w.att = att;
        return finish(mg::launch_attention_wave(w, nullptr));
    }
    mg::AttnArgs a;
    a.B = B; a.T = T; a.D = D; a.Dp = Dp; a.heads = heads; a.window = window; a.cap = cap;
    a.qkv = qkv; a.att = att;
    return finish(mg::launch_attention(a, nullptr));
}

// Decode attention of S sessions at positions pos[i] (qkv: [S][3D]; kring, vring: [S][heads][cap][D/heads],
// the new key and value are written to slot pos % cap). kernel 0: launch_attention_step's choice (by
// cache size); 1: the one-wave-per-(row, head) kernel; 2: the kernel fused with the limb expansion of its
// output (xl, xs instead of att).
int mgt_attention_step(const int32_t* pos, const float* qkv, float* kring, float* vring, int S, int D, int Dp,
                       int heads, int window, int cap, float* att, int8_t* xl, float* xs, int kernel) {
    if (kernel == 1) {
        mg::AttnWaveArgs w;
        w.rows = S; w.D = D; w.Dp = Dp; w.heads = heads; w.dh = heads > 0 ? D / heads : 0;
        w.window = window; w.cap = cap; w.step = true; w.qkv = qkv; w.pos = pos; w.kring = kring;
        w.vring = vring; w.att = att;
        return finish(mg::launch_attention_wave(w, nullptr));
    }
    mg::AttnStepArgs a;
    a.S = S; a.D = D; a.Dp = Dp; a.heads = heads; a.window = window; a.cap = cap;
    a.pos = pos; a.qkv = qkv; a.kring = kring; a.vring = vring; a.att = att;
    if (kernel == 2) {
        if (!mg::attention_step_rows_fits(a)) return (int)hipErrorInvalidValue;
        a.xl = xl; a.xs = xs;
        return finish(mg::launch_attention_step_rows(a, nullptr));
    }
    return finish(mg::launch_attention_step(a, nullptr));
}

// Decode attention on packed rings (kpack/vpack: [S][heads][cap][3 dh / 4] words, kscale/vscale:
// [S][heads][cap]); kernel 0: launch_attention_step's choice (attention_step_rk), 2: the kernel fused
// with the limb expansion of its output (xl, xs instead of att), with the rings' loads chosen by their
// size (these tests' rings are small: cached), 3: the same kernel with the rings streamed.
int mgt_attention_step_packed(const int32_t* pos, const float* qkv, uint32_t* kpack, uint32_t* vpack, float* kscale,
                              float* vscale, int S, int D, int Dp, int heads, int window, int cap, float* att,
                              int8_t* xl, float* xs, int kernel) {
    mg::AttnStepArgs a;
    a.S = S; a.D = D; a.Dp = Dp; a.heads = heads; a.window = window; a.cap = cap;
    a.pos = pos; a.qkv = qkv; a.att = att;
    a.kpack = kpack; a.vpack = vpack; a.kscale = kscale; a.vscale = vscale;
    if (kernel == 2 || kernel == 3) {
        if (!mg::attention_step_rows_fits(a)) return (int)hipErrorInvalidValue;
        a.xl = xl; a.xs = xs;
        a.stream_rings = kernel == 3 ? 1 : -1;
        return finish(mg::launch_attention_step_rows(a, nullptr));
    }
    return finish(mg::launch_attention_step(a, nullptr));
}

// A batched prefill's K/V export into packed rings: B sequences of T rows of qkv ([B][T][3D]), the last
// min(lens[b], cap) positions of each.
int mgt_export_kv_packed(int B, int T, int D, int heads, int cap, const int32_t* lens, const float* qkv,
                         uint32_t* kpack, uint32_t* vpack, float* kscale, float* vscale) {
    return finish(mg::launch_export_kv_packed(B, T, D, heads, cap, lens, qkv, kpack, vpack, kscale, vscale, nullptr));
}

}  // extern "C"
