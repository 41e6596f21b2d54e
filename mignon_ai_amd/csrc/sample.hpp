// Device token sampling (sample.hip): generate.SampleRawLogitsAdvanced and sampleContinuation's per-step
// rules over rows of logits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace mg {

constexpr int kRepWindow = 6;          // generate.ChatRepetitionWindow (internal/generate/constants.go:11)
constexpr int kMaxSampleVocab = 8192;  // rows are sorted in LDS: 12 bytes per entry of the padded vocabulary

struct SampleParams {
    double temperature = 0.0, rep_penalty = 1.0, top_p = 1.0;
    int top_k = 0;
};

struct SampleArgs {
    int n = 0, V = 0, n2 = 0;             // rows, vocabulary, vocabulary padded to a power of two
    const float* logits32 = nullptr;      // [n][ld] fp32 logits, or
    const double* logits64 = nullptr;     // [n][ld] float64 logits
    long long ld = 0;
    // repetition window: the last tokens of prefix[row][0..prefix_len[row]) then hist[row][0..col)
    const int32_t* prefix = nullptr;
    int prefix_ld = 0;
    const int32_t* prefix_len = nullptr;
    const int32_t* hist = nullptr;        // generated tokens [n][hist_ld]
    int hist_ld = 0, col = 0;
    bool trigram = false;                 // ban the token that followed an earlier copy of the last two
    SampleParams p;
    const double* u = nullptr;            // [n] uniforms in [0, 1), or
    const uint64_t* seeds = nullptr;      // [n] generator seeds, drawn at `step`
    int step = 0;
    int32_t* out = nullptr;               // chosen token -> out[row * out_ld + out_col]
    int out_ld = 1, out_col = 0;
    int32_t* next_ids = nullptr;          // [n] or null
    // Workspace of the three-pass form of sampled draws (temperature above 0.001): the exponentials
    // [n][V] and the rows' sums [n]. Without it one kernel does everything, the sequential float64 sum of
    // each row in one lane of its workgroup.
    double* scratch = nullptr;
    double* sums = nullptr;
    // [n] per-row flags of the same workspace: set for the rows whose top-p mass is not reached within
    // the candidates taken one by one, which then take the full sort
    int32_t* flags = nullptr;
};
// Bytes of SampleArgs::scratch, SampleArgs::sums and SampleArgs::flags for n rows of V tokens, laid out
// in that order (sums at scratch + n * V, flags right after the sums).
size_t sample_scratch_bytes(int n, int V);

int sample_n2(int V);
size_t sample_lds_bytes(int V);
hipError_t launch_sample(const SampleArgs& a, hipStream_t s);

}  // namespace mg
