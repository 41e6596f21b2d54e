// Text layer of the library (host code over the public C ABI): the tokenizer of a model file, batched greedy
// generation (infer.Generate's greedy branch) and held-out scoring (eval.Perplexity, PerplexityPerDoc).
// The network runs through mg_sessions_* and mg_score_sequences; nothing here touches the GPU directly.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/mignon_hip.h"
#include "model_file.hpp"
#include "text_abi.hpp"
#include "tokenizer.hpp"

struct mg_tokenizer {
    std::unique_ptr<mg::Tokenizer> tok;
};

namespace {

struct AbiError : std::runtime_error {
    int code;
    AbiError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void need(bool ok, const std::string& msg) {
    if (!ok) throw AbiError(MG_ERR_INVALID, msg);
}

// an engine call's failure keeps the engine's message and code
void engine(int rc) {
    if (rc < 0) throw AbiError(rc, mg_last_error());
}

// runs an entry point's body; an exception becomes its error code (negative) and mg_last_error()
template <class F>
auto guarded(F&& f) -> decltype(f()) {
    using R = decltype(f());
    try {
        return f();
    } catch (const AbiError& e) {
        mg::set_last_error(e.what());
        return (R)e.code;
    } catch (const mg::TokenizerFormatError& e) {
        mg::set_last_error(e.what());
        return (R)MG_ERR_FORMAT;
    } catch (const mg::FormatError& e) {
        mg::set_last_error(e.what());
        return (R)MG_ERR_FORMAT;
    } catch (const std::bad_alloc&) {
        mg::set_last_error("host allocation failed");
        return (R)MG_ERR_NOMEM;
    } catch (const std::exception& e) {
        mg::set_last_error(e.what());
        return (R)MG_ERR_FORMAT;
    }
}

constexpr const char* kDocSeparator = "<EOS>";  // data.DocSeparator (internal/data/data.go:11)
constexpr const char* kDocPadding = "\n\n";      // docPadding (internal/eval/perdoc.go:34-36)

// splitDocs (internal/eval/perdoc.go:39-48): split on the separator, strip one blank line each side,
// drop empty documents
std::vector<std::string> split_docs(const std::string& text) {
    std::vector<std::string> docs;
    const size_t sep = std::strlen(kDocSeparator), pad = std::strlen(kDocPadding);
    size_t pos = 0;
    for (;;) {
        const size_t e = text.find(kDocSeparator, pos);
        std::string d = text.substr(pos, e == std::string::npos ? std::string::npos : e - pos);
        if (d.compare(0, pad, kDocPadding) == 0) d.erase(0, pad);
        if (d.size() >= pad && d.compare(d.size() - pad, pad, kDocPadding) == 0) d.erase(d.size() - pad);
        if (!d.empty()) docs.push_back(std::move(d));
        if (e == std::string::npos) break;
        pos = e + sep;
    }
    return docs;
}

// strings.TrimSpace: the byte range of text without leading and trailing unicode.IsSpace runes
std::pair<size_t, size_t> trim_space(const char* text, size_t n) {
    const unsigned char* t = (const unsigned char*)text;
    size_t b = 0, e = 0;
    bool any = false;
    for (size_t i = 0; i < n;) {
        int w;
        const bool space = mg::char_class(mg::decode_rune(t + i, n - i, w)) == mg::CLS_SPACE;
        if (!space) {
            if (!any) b = i;
            any = true;
            e = i + w;
        }
        i += w;
    }
    return any ? std::make_pair(b, e) : std::make_pair(size_t(0), size_t(0));
}

}  // namespace

extern "C" {

int mg_tokenizer_load(const uint8_t* data, size_t n, mg_tokenizer** out) {
    return guarded([&] {
        need(data != nullptr && out != nullptr, "mg_tokenizer_load: null argument");
        *out = nullptr;
        const mgjson::Value hdr = mg::parse_model_header(data, n, nullptr, nullptr);
        std::unique_ptr<mg::Tokenizer> t(mg::Tokenizer::from_header(hdr));
        if (t) {
            *out = new mg_tokenizer();
            (*out)->tok = std::move(t);
        }
        return MG_OK;
    });
}

void mg_tokenizer_free(mg_tokenizer* t) { delete t; }

int mg_tokenizer_vocab_size(const mg_tokenizer* t) { return t ? (int)t->tok->vocab.size() : 0; }

int mg_tokenizer_special(const mg_tokenizer* t, int which) {
    if (!t) return -1;
    switch (which) {
        case MG_TOKEN_PAD: return t->tok->pad_id();
        case MG_TOKEN_UNK: return t->tok->lookup(mg::Tokenizer::kUnk, -1);
        case MG_TOKEN_USER: return t->tok->user_id();
        case MG_TOKEN_BOT: return t->tok->bot_id();
        case MG_TOKEN_EOS: return t->tok->eos_id();
        default:
            mg::set_last_error("mg_tokenizer_special: unknown token kind " + std::to_string(which));
            return MG_ERR_INVALID;
    }
}

long long mg_tokenizer_encode(mg_tokenizer* t, const char* text, size_t n, int mode, int32_t* ids, long long cap) {
    return guarded(
        [&]() -> long long {
            need(t != nullptr && (text != nullptr || n == 0), "mg_tokenizer_encode: null argument");
            need(cap >= 0 && (ids != nullptr || cap == 0), "mg_tokenizer_encode: bad output buffer");
            std::vector<int32_t> out;
            out.reserve(n / 2 + 2);
            if (mode == MG_ENCODE_TEXT) t->tok->encode(text, n, out);
            else if (mode == MG_ENCODE_PROMPT) t->tok->encode_prompt(text, n, out);
            else if (mode == MG_ENCODE_REPLY) t->tok->encode_reply(text, n, out);
            else need(false, "mg_tokenizer_encode: unknown mode " + std::to_string(mode));
            const long long k = std::min<long long>(cap, (long long)out.size());
            if (k) std::memcpy(ids, out.data(), (size_t)k * 4);
            return (long long)out.size();
        });
}

long long mg_tokenizer_decode(const mg_tokenizer* t, const int32_t* ids, long long n, char* out, long long cap) {
    return guarded(
        [&]() -> long long {
            need(t != nullptr && (ids != nullptr || n == 0) && n >= 0, "mg_tokenizer_decode: bad input");
            need(cap >= 0 && (out != nullptr || cap == 0), "mg_tokenizer_decode: bad output buffer");
            std::string s;
            t->tok->decode(ids, (size_t)n, s);
            const long long k = std::min<long long>(cap, (long long)s.size());
            if (k) std::memcpy(out, s.data(), (size_t)k);
            return (long long)s.size();
        });
}

long long mg_tokenizer_decode_rows(const mg_tokenizer* t, const int32_t* ids, const int32_t* counts, int n, int ld,
                                   int trim, char* out, long long cap, long long* offsets) {
    return guarded([&]() -> long long {
        need(t != nullptr && n >= 0 && offsets != nullptr && (n == 0 || (ids && counts)),
             "mg_tokenizer_decode_rows: null argument");
        need(ld >= 0 && cap >= 0 && (out != nullptr || cap == 0), "mg_tokenizer_decode_rows: bad buffer");
        std::string s;
        long long pos = 0;
        offsets[0] = 0;
        for (int i = 0; i < n; i++) {
            need(counts[i] >= 0 && counts[i] <= ld, "mg_tokenizer_decode_rows: row length outside 0..ld");
            s.clear();
            t->tok->decode(ids + (size_t)i * ld, (size_t)counts[i], s);
            size_t b = 0, e = s.size();
            if (trim) std::tie(b, e) = trim_space(s.data(), s.size());
            const long long len = (long long)(e - b);
            if (pos + len <= cap && len) std::memcpy(out + pos, s.data() + b, (size_t)len);
            pos += len;
            offsets[i + 1] = pos;
        }
        return pos;
    });
}

long long mg_tokenizer_token(const mg_tokenizer* t, int id, char* out, long long cap) {
    return guarded([&]() -> long long {
        need(t != nullptr && id >= 0 && (size_t)id < t->tok->vocab.size(), "mg_tokenizer_token: id outside the vocabulary");
        need(cap >= 0 && (out != nullptr || cap == 0), "mg_tokenizer_token: bad output buffer");
        const std::string& s = t->tok->vocab[id];
        const long long k = std::min<long long>(cap, (long long)s.size());
        if (k) std::memcpy(out, s.data(), (size_t)k);
        return (long long)s.size();
    });
}

int mg_tokenizer_token_bytes(const mg_tokenizer* t, int32_t* out) {
    return guarded([&] {
        need(t != nullptr && out != nullptr, "mg_tokenizer_token_bytes: null argument");
        const std::vector<int32_t> b = t->tok->token_bytes();
        std::memcpy(out, b.data(), b.size() * 4);
        return MG_OK;
    });
}

long long mg_pretokenize(const char* text, size_t n, long long* ends, long long cap) {
    return guarded(
        [&]() -> long long {
            need(text != nullptr || n == 0, "mg_pretokenize: null text");
            need(cap >= 0 && (ends != nullptr || cap == 0), "mg_pretokenize: bad output buffer");
            long long k = 0;
            mg::split_words(text, n, [&](size_t, size_t e) {
                if (k < cap) ends[k] = (long long)e;
                k++;
            });
            return k;
        });
}

int mg_generate_greedy(mg_model* m, mg_tokenizer* t, const char* const* prompts, const size_t* prompt_lens, int n,
                       int context, int max_tokens, int chat, int32_t* out_ids, double* out_probs,
                       int32_t* out_counts) {
    return guarded([&] {
        need(m && t && out_counts && (n == 0 || (prompts && prompt_lens && out_ids && out_probs)),
             "mg_generate_greedy: null argument");
        need(n >= 0 && max_tokens > 0, "mg_generate_greedy: n must be >= 0 and max_tokens > 0");
        if (n == 0) return MG_OK;
        std::vector<std::vector<int32_t>> ctx(n);
        std::vector<int> live;
        int L = 0;
        for (int i = 0; i < n; i++) {
            out_counts[i] = 0;
            need(prompts[i] != nullptr || prompt_lens[i] == 0, "mg_generate_greedy: null prompt");
            if (chat) t->tok->encode_prompt(prompts[i], prompt_lens[i], ctx[i]);
            else t->tok->encode(prompts[i], prompt_lens[i], ctx[i]);
            if (!ctx[i].empty()) {  // an empty context prefills to no logits: no reply (greedy.go:66-67)
                live.push_back(i);
                L = std::max<int>(L, (int)ctx[i].size());
            }
        }
        if (live.empty()) return MG_OK;
        const int S = (int)live.size();
        std::vector<int32_t> arr((size_t)S * L, t->tok->pad_id()), lens(S);
        for (int r = 0; r < S; r++) {
            const auto& c = ctx[live[r]];
            std::copy(c.begin(), c.end(), arr.begin() + (size_t)r * L);
            lens[r] = (int32_t)c.size();
        }
        std::vector<int32_t> ids((size_t)S * max_tokens), counts(S);
        std::vector<double> probs((size_t)S * max_tokens);
        // greedyLoop stops before <EOS>, <USER> or <BOT> (those the vocabulary has)
        std::vector<int32_t> stops;
        for (int id : {t->tok->eos_id(), t->tok->user_id(), t->tok->bot_id()})
            if (id >= 0) stops.push_back(id);
        mg_sessions* ss = nullptr;
        engine(mg::generate_sessions_acquire(m, S, context, &ss));
        const int rc = mg_sessions_decode_greedy_until(ss, arr.data(), lens.data(), L, max_tokens, stops.data(),
                                                       (int)stops.size(), ids.data(), probs.data(), counts.data(), 0);
        mg::generate_sessions_release(m, ss);
        engine(rc);
        for (int r = 0; r < S; r++) {
            const int i = live[r], k = counts[r];
            std::copy_n(ids.begin() + (size_t)r * max_tokens, k, out_ids + (size_t)i * max_tokens);
            std::copy_n(probs.begin() + (size_t)r * max_tokens, k, out_probs + (size_t)i * max_tokens);
            out_counts[i] = k;
        }
        return MG_OK;
    });
}

int mg_generate_sample(mg_model* m, mg_tokenizer* t, const char* const* prompts, const size_t* prompt_lens, int n,
                       int context, int max_tokens, int chat, const mg_sampling_t* sp, const uint64_t* seeds,
                       int32_t* out_ids, int32_t* out_counts) {
    return guarded([&] {
        need(m && t && sp && out_counts && (n == 0 || (prompts && prompt_lens && seeds && out_ids)),
             "mg_generate_sample: null argument");
        need(n >= 0 && max_tokens > 0, "mg_generate_sample: n must be >= 0 and max_tokens > 0");
        if (n == 0) return MG_OK;
        std::vector<std::vector<int32_t>> ctx(n);
        std::vector<int> live;
        int L = 0;
        for (int i = 0; i < n; i++) {
            out_counts[i] = 0;
            need(prompts[i] != nullptr || prompt_lens[i] == 0, "mg_generate_sample: null prompt");
            if (chat) {  // ChatWithHistory (internal/generate/chat.go:104-130): a trimmed prompt, no history
                const auto r = trim_space(prompts[i], prompt_lens[i]);
                if (r.second == r.first) continue;
                t->tok->encode_prompt(prompts[i] + r.first, r.second - r.first, ctx[i]);
            } else {  // Text (chat.go:62-70)
                t->tok->encode(prompts[i], prompt_lens[i], ctx[i]);
            }
            if (!ctx[i].empty()) {
                live.push_back(i);
                L = std::max<int>(L, (int)ctx[i].size());
            }
        }
        if (live.empty()) return MG_OK;
        const int S = (int)live.size();
        std::vector<int32_t> arr((size_t)S * L, t->tok->pad_id()), lens(S), ids((size_t)S * max_tokens), counts(S);
        std::vector<uint64_t> sd(S);
        for (int r = 0; r < S; r++) {
            const auto& c = ctx[live[r]];
            std::copy(c.begin(), c.end(), arr.begin() + (size_t)r * L);
            lens[r] = (int32_t)c.size();
            sd[r] = seeds[live[r]];
        }
        // Text penalises repeats of the prompt's last tokens; Chat's repetition window starts in the reply
        mg_sampling_t p = *sp;
        p.penalize_prompt = chat ? 0 : 1;
        std::vector<int32_t> stops;
        for (int id : {t->tok->eos_id(), t->tok->user_id(), t->tok->bot_id()})
            if (id >= 0) stops.push_back(id);
        mg_sessions* ss = nullptr;
        engine(mg::generate_sessions_acquire(m, S, context, &ss));
        const int rc = mg_sessions_decode_sample(ss, arr.data(), lens.data(), L, max_tokens, &p, sd.data(), stops.data(),
                                                 (int)stops.size(), ids.data(), counts.data(), 0);
        mg::generate_sessions_release(m, ss);
        engine(rc);
        for (int r = 0; r < S; r++) {
            const int i = live[r], k = counts[r];
            std::copy_n(ids.begin() + (size_t)r * max_tokens, k, out_ids + (size_t)i * max_tokens);
            out_counts[i] = k;
        }
        return MG_OK;
    });
}

int mg_perplexity(mg_model* m, mg_tokenizer* t, const char* text, size_t n, int context, int max_count, int per_doc,
                  mg_heldout_t* out) {
    return guarded([&] {
        need(m && t && out && (text || n == 0), "mg_perplexity: null argument");
        *out = mg_heldout_t{0, 0, 0, 0};
        std::vector<int32_t> tokens;
        std::vector<long long> offsets{0};
        if (per_doc) {
            std::vector<std::string> docs = split_docs(std::string(text, n));
            if (max_count > 0 && (int)docs.size() > max_count) docs.resize(max_count);
            const int eos = t->tok->eos_id();
            for (const auto& d : docs) {
                tokens.push_back(eos);
                t->tok->encode(d.data(), d.size(), tokens);
                offsets.push_back((long long)tokens.size());
            }
        } else {
            if (n == 0) return MG_OK;
            t->tok->encode(text, n, tokens);
            if (tokens.size() < 2) return MG_OK;
            long long num = (long long)tokens.size() - 1;
            if (max_count > 0 && num > max_count) num = max_count;
            tokens.resize((size_t)num + 1);
            offsets.push_back((long long)tokens.size());
        }
        const int n_seq = (int)offsets.size() - 1;
        if (n_seq == 0) return MG_OK;
        long long n_targets = 0;
        for (int q = 0; q < n_seq; q++) n_targets += std::max<long long>(offsets[q + 1] - offsets[q] - 1, 0);
        std::vector<float> lp((size_t)n_targets);
        engine(mg_score_sequences(m, tokens.data(), offsets.data(), n_seq, context, lp.data()));
        // nll.score / nll.result (internal/eval/eval.go:27-50): nats and bytes of the scored targets, in order
        const std::vector<int32_t> tb = t->tok->token_bytes();
        double nats = 0.0;
        long long bytes = 0, count = 0, k = 0;
        for (int q = 0; q < n_seq; q++)
            for (long long p = offsets[q] + 1; p < offsets[q + 1]; p++, k++) {
                if (std::isnan(lp[k])) continue;
                nats -= (double)lp[k];
                const int32_t tg = tokens[p];
                if (tg >= 0 && (size_t)tg < tb.size()) bytes += tb[tg];
                count++;
            }
        if (count == 0) return MG_OK;
        const double avg = nats / (double)count;
        out->loss = avg;
        out->ppl = std::exp(avg);
        out->bpb = bytes > 0 ? nats / (std::log(2.0) * (double)bytes) : 0.0;  // tokenizer.BitsPerByte
        out->tokens = count;
        return MG_OK;
    });
}

}  // extern "C"
