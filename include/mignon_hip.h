/*
 * mignon_hip.h -- C ABI of the MI355X (gfx950) batched INT8 engine for mignon-ai's Hybrid NCA model.
 *
 * The reference engine is Go (internal/quant over internal/kernels); this ABI is what its cgo binding
 * would call. Each entry point names the reference interface it replaces. Conventions:
 *   - Every function returns MG_OK (0) or a negative MG_ERR_* code; mg_last_error() gives the message
 *     (thread-local). Go panics cannot cross cgo, so the reference's panics become error codes too.
 *   - Handles own their device memory and one HIP stream; calls on one handle are serialised (the
 *     reference serialises a model and its sessions on one mutex, internal/quant/model.go:67,123).
 *   - Array arguments are host pointers unless MG_PTR_DEVICE is passed in `flags`; then every array of
 *     that call is a device pointer and the work is only enqueued on the handle's stream (call
 *     mg_model_sync to wait). Host-pointer calls return when their outputs are written.
 *   - Optional outputs may be NULL.
 */
#ifndef MIGNON_HIP_H
#define MIGNON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MG_OK 0
#define MG_ERR_INVALID (-1)     /* bad argument or shape (the reference panics or returns nil) */
#define MG_ERR_FORMAT (-2)      /* damaged or unsupported model file (quant.Decode's errors) */
#define MG_ERR_DEVICE (-3)      /* HIP runtime error */
#define MG_ERR_NOMEM (-4)       /* device allocation failed */
#define MG_ERR_UNSUPPORTED (-5) /* valid model the engine does not run (e.g. head width not compiled) */

#define MG_PTR_DEVICE 1 /* all array arguments of the call are device pointers; the call is asynchronous */

typedef struct mg_model mg_model;
typedef struct mg_sessions mg_sessions;

typedef struct {
    int vocab_size;    /* quant.Model.VocabSize  (internal/quant/model.go:71-74) */
    int state_size;    /* quant.Model.StateSize  (internal/quant/model.go:76-79) */
    int hidden_size;   /* quant.Model.HiddenSize (internal/quant/model.go:81-84) */
    int num_blocks;    /* quant.Model.NumBlocks  (internal/quant/model.go:86-89) */
    int attn_heads;    /* metadata attn_heads (internal/checkpoint/checkpoint.go:29) */
    int attn_window;   /* metadata attn_window (internal/checkpoint/checkpoint.go:30) */
    int max_context;   /* quant.Model.maxContext after NewModel's defaulting (internal/quant/model.go:91-95) */
    int tied_embed;
    int norm_ring;     /* quant.Model.normRing (internal/quant/stream.go:37-47) */
    int attn_cache;    /* quant.Model.attnCache (internal/quant/attention.go:46-52) */
    long long num_params; /* quant.Model.NumParams (internal/quant/checkpoint.go:91-104) */
} mg_model_info_t;

/* Thread-local message of the last failed call on this thread. */
const char* mg_last_error(void);

/* Decodes an INT8 model file (binary mignon.model/1 or legacy JSON) and uploads it to the current HIP
 * device. Replaces quant.Decode + quant.NewModel (internal/quant/checkpoint.go:162-212,
 * internal/quant/model.go:90-118) and pkg/model.Decode for INT8 files (pkg/model/model.go:59-117).
 * max_context <= 0 takes the file's metadata context_size; below 64 it becomes 128 as in NewModel. */
int mg_model_load(const uint8_t* data, size_t n, int max_context, mg_model** out);

/* Decodes and validates a model file without touching the GPU (quant.Decode's checks,
 * internal/quant/checkpoint.go:162-225) and reports what mg_model_load would build. */
int mg_model_file_info(const uint8_t* data, size_t n, int max_context, mg_model_info_t* info);

/* quant.Model accessors (internal/quant/model.go:71-89, internal/quant/checkpoint.go:91-104). */
int mg_model_info(const mg_model* m, mg_model_info_t* info);

/* Replaces the handle's stream (NULL restores the library's own stream). */
int mg_model_set_stream(mg_model* m, void* hip_stream);
void* mg_model_stream(const mg_model* m);

/* Kernel timing (no reference counterpart; measurement support). While on, every kernel launch of the
 * handle is bracketed by HIP events on its stream; mg_model_profile_read waits for the stream and
 * returns per-class launch counts, summed durations and the summed algorithmic work of those launches:
 * bytes = HBM bytes each launch must move (its operands read once, its results written once; 0 where the
 * host cannot know it, e.g. decode attention's spans), ops = int8 multiply-accumulates x 2 (GEMMs only,
 * unpadded shapes, one pass per weight matrix). At most max entries; returns the class count. */
typedef struct {
    char name[32];
    long long launches;
    double total_ms;
    double bytes;
    double ops;
} mg_kernel_time_t;
int mg_model_profile(mg_model* m, int on);
int mg_model_profile_read(mg_model* m, mg_kernel_time_t* out, int max);

/* Cancellation: generate's Cancel hook, checked before each token (internal/generate/greedy.go:29,68-70,
 * internal/generate/sample.go:204-206), which pkg/infer.Generate wires to its context
 * (pkg/infer/infer.go:73-95). flag is caller-owned memory (NULL removes it) that any thread may set at any
 * time, also while a call on m runs; this call takes no lock. While *flag is nonzero, a batched decode on
 * m (mg_sessions_decode_greedy_until, mg_sessions_decode_sample, mg_generate_greedy, mg_generate_sample)
 * enqueues no further token: every reply is cut before the first column not yet started, and the call
 * returns MG_OK with out_counts giving the lengths of the replies produced so far. A flag already set when
 * the call starts gives empty replies (after the prefill, as the reference's loop). */
int mg_model_set_cancel(mg_model* m, const volatile int32_t* flag);
int mg_model_sync(mg_model* m);
void mg_model_free(mg_model* m);

/* quant.Model.Call / Forward (internal/quant/model.go:120-137): next-token logits after the last
 * token, window truncated to max_context. logits: host double[V]. Returns V, or 0 for empty input. */
int mg_model_call(mg_model* m, const int32_t* ids, int n, double* logits);

/* Teacher-forced batch: B sequences of T tokens, every position's next-token distribution at once.
 * Position t of sequence b gives the logits Call(ids[b][0..t]) gives (internal/quant/stream.go:11-17;
 * beyond max_context the positions follow a streaming session, internal/quant/session.go:41-56).
 *   logits  [B][T][V] fp32
 *   logprob [B][T]    fp32: log-softmax of target ids[b][t+1] under position t (eval.logProb,
 *                     internal/eval/suite.go:200-208); NaN for t = T-1 and for out-of-range targets
 *   probs   [B][T][V] fp32 softmax probabilities
 *   bits    [B]       fp32: bits per token over the sequence's targets (eval nll.score +
 *                     tokenizer.BitsPerByte with tokens for bytes, internal/eval/eval.go:25-48) */
int mg_forward_batch(mg_model* m, const int32_t* ids, int B, int T, float* logits, float* logprob, float* probs,
                     float* bits, int flags);

/* n streaming sessions (quant.Model.NewSession, internal/quant/session.go:20-28): window =
 * min(max_context, context) when context > 0. State lives in device memory, constant per session. */
int mg_sessions_create(mg_model* m, int n, int context, mg_sessions** out);

/* quantSession.Prefill for every session at once (internal/quant/session.go:30-39): prompts
 * [n][max_len] with lengths lens[n] (1..max_len); prompts longer than the window keep their last
 * window tokens. Outputs describe the next token after each prompt:
 *   logits [n][V] fp32, argmax [n] (first maximum, internal/generate/greedy.go:89-102),
 *   prob [n] double = 1 / sum exp(l - max) (argmaxProb, internal/generate/greedy.go:89-102; the sum is
 *   accumulated in fp32 from the head's per-tile statistics, so the value has fp32 accuracy, about 1e-6
 *   relative, where the reference sums math.Exp in float64). */
int mg_sessions_prefill(mg_sessions* s, const int32_t* prompts, const int32_t* lens, int max_len, float* logits,
                        int32_t* argmax, double* prob, int flags);

/* quantSession.Append for every session (internal/quant/session.go:41-56): ids [n]. */
int mg_sessions_step(mg_sessions* s, const int32_t* ids, float* logits, int32_t* argmax, double* prob, int flags);

/* No counterpart in the reference: mg_sessions_step for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same kernels and results as
 * mg_sessions_step with MG_PTR_DEVICE, but it allocates nothing: its workspace is a static 64 MiB array
 * per GPU (held until the process ends) instead of the model's workspace. All pointers are device
 * pointers; logits, argmax and prob may be NULL. A set whose sessions need more than 64 MiB of workspace
 * (about 4300 sessions of c4's D256/H512/V4096 model, fewer for wider models) is MG_ERR_INVALID. Calls on
 * one GPU share the array, so each call is ordered after the previous one on that GPU: a call enqueued on
 * another stream (another model's) first waits on the device for the previous call's work. Under stream
 * capture that wait is not recorded: callers capturing these calls from several streams order them
 * themselves, or calls that overlap in time race. The step is enqueued on the model's stream and not
 * waited for. */
int mg_sessions_step_noalloc(mg_sessions* s, const int32_t* ids, float* logits, int32_t* argmax, double* prob);

/* generate.greedyLoop for every session without stop tokens (internal/generate/greedy.go:63-87):
 * Prefill(prompt), then max_tokens tokens, each the first-maximum argmax with its probability, with
 * Append after every token but the last. out_ids [n][max_tokens], out_probs [n][max_tokens]. */
int mg_sessions_decode_greedy(mg_sessions* s, const int32_t* prompts, const int32_t* lens, int max_len,
                              int max_tokens, int32_t* out_ids, double* out_probs, int flags);

/* generate.greedyLoop with stop tokens (internal/generate/greedy.go:63-87) for every session: as
 * mg_sessions_decode_greedy, and each session's reply ends before the first of its n_stops (<= 8) stop
 * ids; out_counts[n] receives the reply lengths. Entries of out_ids / out_probs past a session's count
 * are unspecified: decoding ends once every session has stopped. Sessions that stopped are still stepped
 * until all have (the reference's loop never Appends the stop token), so the set's state afterwards is
 * unspecified: Prefill again before reusing it (as mg_generate_greedy does with a fresh set). */
int mg_sessions_decode_greedy_until(mg_sessions* s, const int32_t* prompts, const int32_t* lens, int max_len,
                                    int max_tokens, const int32_t* stops, int n_stops, int32_t* out_ids,
                                    double* out_probs, int32_t* out_counts, int flags);

/* generate.Sampling's numeric fields (internal/generate/chat.go:43-55): temperature <= 0.001 is argmax;
 * rep_penalty > 1 scales down the last 6 tokens' logits; top_k <= 0 and top_p >= 0.9999 disable
 * truncation. penalize_prompt: the repetition window starts in the prompt (generate.Text) rather than
 * in the reply (generate.Chat). */
typedef struct {
    double temperature, rep_penalty, top_p;
    int top_k, penalize_prompt;
} mg_sampling_t;

/* generate.SampleRawLogitsAdvanced (internal/generate/sample.go:31-171) for n rows of float64 logits [n][V]
 * (V <= 8192): repetition penalty over recent[i][0..recent_len[i]) (recent_ld per row; recent may be NULL),
 * then argmax, temperature sampling or top-k / top-p truncated sampling with the uniform u[i] in [0, 1)
 * standing for the reference's rand.Float64(). Candidates of equal probability sort by token id (the
 * reference's sort leaves their order open). out[n]. Runs on the current device. */
int mg_sample_logits(const double* logits, int n, int V, const int32_t* recent, const int32_t* recent_len,
                     int recent_ld, const mg_sampling_t* sp, const double* u, int32_t* out);

/* generate.sampleContinuation (internal/generate/sample.go:196-247) for every session: Prefill, then per
 * step the trigram ban over the reply, SampleRawLogitsAdvanced over the last 6 tokens of (prompt if
 * penalize_prompt) + reply, a stop before any of the n_stops (<= 8) stop ids, Append. The reference
 * draws from Go's global math/rand, randomly seeded; here session i's draw at step k is the (k+1)-th
 * output of SplitMix64 seeded with seeds[i], top 53 bits over 2^53. out_ids [n][max_tokens],
 * out_counts[n] and the set's state afterwards as mg_sessions_decode_greedy_until. Vocabularies up to
 * 8192 tokens. */
int mg_sessions_decode_sample(mg_sessions* s, const int32_t* prompts, const int32_t* lens, int max_len, int max_tokens,
                              const mg_sampling_t* sp, const uint64_t* seeds, const int32_t* stops, int n_stops,
                              int32_t* out_ids, int32_t* out_counts, int flags);

/* quantSession.StateBytes (internal/quant/session.go:65-68, formula internal/quant/stream.go:87-101). */
long long mg_sessions_state_bytes(const mg_sessions* s);
/* Device bytes actually held per session. */
long long mg_sessions_device_bytes(const mg_sessions* s);
int mg_sessions_count(const mg_sessions* s);
void mg_sessions_free(mg_sessions* s);

/* eval nll.score's per-target log-probabilities over many token sequences in one batched pass
 * (internal/eval/eval.go:25-50, window internal/eval/suite.go:196-198, logProb :200-208). Sequence q is
 * tokens[offsets[q] .. offsets[q+1]); each of its targets t = 1..len-1 is scored from
 * window(seq[:t], context) (then Call's truncation to max_context), as log-softmax of seq[t].
 * logprob receives, sequence after sequence, max(len-1, 0) fp32 values; NaN marks a target that is not
 * scored (id outside [0, V), or context 0). A negative context is MG_ERR_INVALID (the reference's window()
 * panics on it). offsets has n_seq+1 entries. Host pointers. */
int mg_score_sequences(mg_model* m, const int32_t* tokens, const long long* offsets, int n_seq, int context,
                       float* logprob);

/* ---- Text: the tokenizer stored in a model file and the generation / evaluation drivers over it ---- */
typedef struct mg_tokenizer mg_tokenizer;

/* tokenizer.FromVocabAndMerges on a model file's header after tokenizer.CheckFormat
 * (internal/quant/checkpoint.go:201-207, internal/tokenizer/tokenizer.go:60-72, format.go:12-17).
 * *out = NULL (and MG_OK) when the file has no vocabulary; MG_ERR_FORMAT for any other format version. */
int mg_tokenizer_load(const uint8_t* data, size_t n, mg_tokenizer** out);
void mg_tokenizer_free(mg_tokenizer* t);
/* Tokenizer.VocabSize (internal/tokenizer/tokenizer.go:86-90). */
int mg_tokenizer_vocab_size(const mg_tokenizer* t);
/* PadTokenID (0 when absent), UnkTokenID, UserTokenID, BotTokenID, EOSTokenID (-1 when absent)
 * (internal/tokenizer/tokenizer.go:320-347). */
#define MG_TOKEN_PAD 0
#define MG_TOKEN_UNK 1
#define MG_TOKEN_USER 2
#define MG_TOKEN_BOT 3
#define MG_TOKEN_EOS 4
int mg_tokenizer_special(const mg_tokenizer* t, int which);
/* Encode (internal/tokenizer/tokenizer.go:268-318), EncodePrompt / EncodeReply (template.go:11-21) of
 * UTF-8 text of n bytes. Writes at most cap ids and returns how many the text encodes to. */
#define MG_ENCODE_TEXT 0
#define MG_ENCODE_PROMPT 1
#define MG_ENCODE_REPLY 2
long long mg_tokenizer_encode(mg_tokenizer* t, const char* text, size_t n, int mode, int32_t* ids, long long cap);
/* Decode (internal/tokenizer/tokenizer.go:348-367): writes at most cap bytes (no terminator) and returns
 * the decoded length in bytes. */
long long mg_tokenizer_decode(const mg_tokenizer* t, const int32_t* ids, long long n, char* out, long long cap);
/* Decode of n rows at once, for a batch of replies (infer.Generate's Result.Text: strings.TrimSpace of
 * the decoded reply, pkg/infer/infer.go:76-79): row i is counts[i] ids at ids + i*ld; with trim != 0 each
 * row's text loses its leading and trailing white space (unicode.IsSpace). The texts are written one
 * after another into out (at most cap bytes, no terminators) and row i's text is
 * out[offsets[i], offsets[i+1]) (offsets: n + 1 entries, always written). Returns the total length in
 * bytes; when it exceeds cap, out holds only the texts that fit whole. */
long long mg_tokenizer_decode_rows(const mg_tokenizer* t, const int32_t* ids, const int32_t* counts, int n, int ld,
                                   int trim, char* out, long long cap, long long* offsets);
/* The vocabulary entry of id (Tokenizer.Vocab[id]): writes at most cap bytes (no terminator) and returns
 * its length, or MG_ERR_INVALID for an id outside the vocabulary. */
long long mg_tokenizer_token(const mg_tokenizer* t, int id, char* out, long long cap);
/* TokenBytes (internal/tokenizer/bytes.go:13-22): out[V]. */
int mg_tokenizer_token_bytes(const mg_tokenizer* t, int32_t* out);
/* splitWords (internal/tokenizer/pretokenize.go:39-67): the end offset (bytes) of every pre-token of the
 * text; writes at most cap and returns the count. */
long long mg_pretokenize(const char* text, size_t n, long long* ends, long long cap);

/* infer.Generate's greedy branch (pkg/infer/infer.go:64-84, generate.DecodeGreedy and greedyLoop,
 * internal/generate/greedy.go:43-102) for n prompts at once, on device sessions of window `context`:
 * each prompt (UTF-8, prompt_lens[i] bytes) goes through the chat template when chat != 0; the reply
 * stops before <EOS>, <USER> or <BOT> or after max_tokens (> 0) tokens. out_ids / out_probs are
 * [n][max_tokens]; out_counts[i] is the reply length. Decode the ids with mg_tokenizer_decode and trim
 * surrounding whitespace for infer.Result.Text. The session set a call decodes on stays allocated in m
 * afterwards (cleared and reused by the next mg_generate_* call with as many non-empty prompts and the same
 * window, replaced otherwise, freed by mg_model_free); calls running at once on m use sets of their own. */
int mg_generate_greedy(mg_model* m, mg_tokenizer* t, const char* const* prompts, const size_t* prompt_lens, int n,
                       int context, int max_tokens, int chat, int32_t* out_ids, double* out_probs,
                       int32_t* out_counts);

/* infer.Generate's sampling branch (pkg/infer/infer.go:85-95) for n prompts at once: generate.Chat when
 * chat != 0 (the prompt trimmed of surrounding whitespace, an empty one getting no reply, the chat template,
 * the repetition window over the reply; internal/generate/chat.go:104-140), generate.Text otherwise (the
 * prompt as is, the window starting in the prompt; chat.go:62-70). sp->penalize_prompt is ignored. Replies
 * stop before <EOS>, <USER> or <BOT> or after max_tokens (> 0) tokens; seeds[i] seeds prompt i's draws
 * (mg_sessions_decode_sample). out_ids [n][max_tokens], out_counts[n]. Its session set is kept in m as
 * mg_generate_greedy's is (one set for both). */
int mg_generate_sample(mg_model* m, mg_tokenizer* t, const char* const* prompts, const size_t* prompt_lens, int n,
                       int context, int max_tokens, int chat, const mg_sampling_t* sp, const uint64_t* seeds,
                       int32_t* out_ids, int32_t* out_counts);

/* eval.HeldOut (internal/eval/eval.go:12-17). */
typedef struct {
    double loss, ppl, bpb;
    long long tokens;
} mg_heldout_t;
/* eval.Perplexity (internal/eval/eval.go:50-75; per_doc == 0: text is one stream, max_count caps the
 * targets) and eval.PerplexityPerDoc (internal/eval/perdoc.go:12-48; per_doc != 0: documents split on
 * "<EOS>", each scored from a fresh <EOS>, max_count caps the documents), all targets in one batched pass
 * (mg_score_sequences). max_count <= 0: no cap. */
int mg_perplexity(mg_model* m, mg_tokenizer* t, const char* text, size_t n, int context, int max_count, int per_doc,
                  mg_heldout_t* out);

/* Standalone INT8 GEMM (kernels.MatVecInt8 per row, internal/kernels/int8.go:31-41, on integer
 * activations): acc[m][n] = sum_k A[m][k]*W[n][k] exactly in int32, C[m][n] = float(acc)*scale[n].
 * A [M][K], W [N][K] (one row per output channel), scale [N], C [M][N], acc [M][N] (optional).
 * stream: HIP stream for MG_PTR_DEVICE calls (NULL = default stream). */
int mg_gemm_i8(const int8_t* A, int M, int K, const int8_t* W, int N, const float* scale, float* C, int32_t* acc,
               int flags, void* stream);

/* quant.NewTensorF32 (internal/quant/tensor.go:12-42) on the GPU: scale = max|w|/127, q = clamp(round
 * half away from zero (w/scale), +-127); an all-zero tensor gets scale 1. */
int mg_quantize_f32(const float* w, long long n, int8_t* q, float* scale, int flags, void* stream);

/* Engine options, no reference counterpart: where two implementations of a stage exist, which one runs,
 * for every model of the process. Value 0 (the default) chooses automatically.
 *   MG_OPT_GEMM_KERNEL: MG_GEMM_STREAM streams weight tiles through LDS per token block;
 *     MG_GEMM_SLAB holds a weight slab in LDS and streams token tiles through it (used where the slab
 *     fits). Both give bit-identical results; automatic picks the slab kernel for large batches.
 *   MG_OPT_ATTENTION_KERNEL: MG_ATTN_EXACT keeps the reference's sequential dot-product and softmax
 *     order (bit-identical given equal inputs); MG_ATTN_MFMA computes scores and P.V on the matrix
 *     cores (fp32, other summation order); MG_ATTN_FUSED also computes the attention projection inside
 *     the attention kernel, per sequence and head (teacher-forced batches of 128-token sequences, head
 *     width 32 or 64), with results bit-identical to MG_ATTN_MFMA. Automatic fuses where that applies,
 *     else picks the matrix cores where they apply (head width a multiple of 4 up to 64, attended span
 *     up to 64 keys, or longer spans for narrower heads).
 *   MG_OPT_SCAN_KERNEL: MG_SCAN_SEPARATE writes the latch state of every position, then limb-expands
 *     the rule input [n | left | g] in a second kernel; MG_SCAN_FUSED does both in one pass without
 *     writing the latch state. Both give byte-identical operands. The fused kernel applies where the
 *     sequence length is a multiple of 16 and the padded width at most 1024; elsewhere the separate
 *     kernels run whatever the option says. Automatic fuses where it applies to batches of many
 *     sequences (one workgroup per sequence).
 *   MG_OPT_STEP_GRAPH: MG_STEP_EAGER launches a decode step's kernels one at a time; MG_STEP_GRAPH
 *     captures a step's launches as a HIP graph once and replays it while the step's buffers and
 *     arguments are unchanged (identical results, less host time per step). Automatic uses the graph.
 *   MG_OPT_STEP_KERNEL: MG_STEP_LAYERED runs a decode step layer by layer (about ten kernels per block,
 *     each over all sessions); MG_STEP_FUSED runs each session's whole step in one workgroup, where the
 *     model fits it (state size up to 512, at most 8 heads of width 16, 32 or 64, caches of at most 64
 *     positions); MG_STEP_TILED runs the step for 16 sessions per workgroup, one kernel per stretch
 *     between attention blocks and the decode attention kernel between them (state size up to 512, hidden
 *     size up to 1024, caches of at most 64 positions); identical results. Automatic fuses sets of up to
 *     256 sessions and tiles larger ones, where the model fits. The fused step's one
 *     kernel reads the ids of an mg_sessions_step call with host pointers from, and writes its outputs
 *     to, the set's pinned host buffers directly (no copies between host and device buffers).
 *   MG_OPT_OPERANDS: MG_OPERANDS_LIMBS writes the limb planes of every GEMM operand of a batched forward
 *     in a pass of their own; MG_OPERANDS_FP32 lets the highway GEMM read the GLU output, and the
 *     attention's output projection the attention output, as fp32 rows (each expanded to base-256 digit
 *     planes as it is loaded, with the row's scale from maxima its producer writes), where the weight-
 *     stationary kernel runs them; results agree within 2e-7 of the row's largest value per operand
 *     element. Automatic is MG_OPERANDS_FP32.
 *   MG_OPT_KV_RINGS (read when a session set is created, fixed for its life): MG_KV_FP32 keeps each
 *     attention block's key and value rings as fp32 rows, as the reference's session does
 *     (internal/quant/stream.go:19-35); MG_KV_PACKED keeps each (head, position) row as 24-bit mantissas
 *     with one power-of-two scale per row (every element within 2^-24 of the row's largest magnitude of
 *     its fp32 value, the precision the engine's limb planes give every matrix operand), 3 bytes per
 *     element: decode attention, which reads the whole window every step, moves 3/4 of the bytes. Packed
 *     rings apply where the fused decode attention kernel takes the model (head width a multiple of 4 up
 *     to 64, caches of at most 64 positions, at most 16 heads); elsewhere fp32. The layered, fused and
 *     tiled steps give bit-identical results to each other under either format. Automatic is
 *     MG_KV_PACKED for sets of more than 256 sessions (where decode attention streams many rings) and
 *     MG_KV_FP32 for smaller ones (a step that is a chain of dependent phases, which decoding lengthens).
 * value < 0 only reads the option. Returns the previous value, or MG_ERR_INVALID. */
#define MG_OPT_GEMM_KERNEL 0
#define MG_OPT_ATTENTION_KERNEL 1
#define MG_OPT_SCAN_KERNEL 2
#define MG_OPT_STEP_GRAPH 3
#define MG_STEP_EAGER 1
#define MG_STEP_GRAPH 2
#define MG_OPT_STEP_KERNEL 4
#define MG_STEP_LAYERED 1
#define MG_STEP_FUSED 2
#define MG_STEP_TILED 3
#define MG_SCAN_SEPARATE 1
#define MG_SCAN_FUSED 2
#define MG_GEMM_STREAM 1
#define MG_GEMM_SLAB 2
#define MG_ATTN_EXACT 1
#define MG_ATTN_MFMA 2
#define MG_ATTN_FUSED 3
#define MG_OPT_OPERANDS 5
#define MG_OPERANDS_LIMBS 1
#define MG_OPERANDS_FP32 2
#define MG_OPT_KV_RINGS 6
#define MG_KV_FP32 1
#define MG_KV_PACKED 2
int mg_engine_option(int option, int value);

#ifdef __cplusplus
}
#endif

#endif /* MIGNON_HIP_H */
