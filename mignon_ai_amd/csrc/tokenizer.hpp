// Byte-pair-encoding tokenizer of a model file (host code): the trained vocabulary and merge table that
// travel in the file's JSON header, with the reference's encoding rules (internal/tokenizer, format
// version 2):
//   - pre-tokenization (splitWords, internal/tokenizer/pretokenize.go:19-67): runs of one character class,
//     every decimal digit alone, at most 128 bytes, a single ' ' before a word or punctuation run joining it;
//   - per pre-token, the adjacent pair of lowest merge rank merges first, the leftmost on a tie, until no
//     ranked pair is left; pieces missing from the vocabulary become <UNK> (encodeWord, tokenizer.go:179-232);
//   - registered "<...>" tokens are taken whole (Encode, tokenizer.go:264-311);
//   - decoding skips <PAD> <EOS> <USER> <BOT> and writes U+FFFD for <UNK> (Decode, tokenizer.go:355-375).
// Text is UTF-8 bytes and is decoded as Go decodes strings: each invalid byte is one U+FFFD rune.
#pragma once

#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "json.hpp"
#include "unicode_classes.hpp"

namespace mg {

constexpr int kTokenizerFormat = 2;   // tokenizer.FormatVersion (internal/tokenizer/format.go:8)
constexpr size_t kMaxWordBytes = 128;  // maxWordBytes (internal/tokenizer/pretokenize.go:7)

enum CharClass { CLS_WORD = 0, CLS_SPACE = 1, CLS_PUNCT = 2, CLS_DIGIT = 3 };

inline int char_class(uint32_t r) {
    if (r < 0x80) {
        // ASCII directly; the table's first entries say the same
        if (r == ' ' || (r >= 0x09 && r <= 0x0D)) return CLS_SPACE;
        if (r >= '0' && r <= '9') return CLS_DIGIT;
        if ((r >= 0x21 && r <= 0x2F) || (r >= 0x3A && r <= 0x40) || (r >= 0x5B && r <= 0x60) ||
            (r >= 0x7B && r <= 0x7E))
            return CLS_PUNCT;
        return CLS_WORD;
    }
    int lo = 0, hi = kCharRanges - 1;
    while (lo <= hi) {
        const int mid = (lo + hi) >> 1;
        const CharRange& c = kCharRangeTable[mid];
        if (r < c.lo) hi = mid - 1;
        else if (r > c.hi) lo = mid + 1;
        else return c.cls;
    }
    return CLS_WORD;
}

// utf8.DecodeRuneInString: the rune at s and its width; an invalid or truncated encoding is (U+FFFD, 1).
inline uint32_t decode_rune(const unsigned char* s, size_t n, int& w) {
    const uint32_t bad = 0xFFFD;
    w = 1;
    const unsigned b0 = s[0];
    if (b0 < 0x80) return b0;
    auto cont = [&](size_t i, unsigned lo, unsigned hi) { return i < n && s[i] >= lo && s[i] <= hi; };
    if (b0 >= 0xC2 && b0 <= 0xDF) {
        if (!cont(1, 0x80, 0xBF)) return bad;
        w = 2;
        return ((b0 & 0x1F) << 6) | (s[1] & 0x3F);
    }
    if (b0 >= 0xE0 && b0 <= 0xEF) {
        const unsigned lo = b0 == 0xE0 ? 0xA0 : 0x80, hi = b0 == 0xED ? 0x9F : 0xBF;
        if (!cont(1, lo, hi) || !cont(2, 0x80, 0xBF)) return bad;
        w = 3;
        return ((b0 & 0x0F) << 12) | ((s[1] & 0x3F) << 6) | (s[2] & 0x3F);
    }
    if (b0 >= 0xF0 && b0 <= 0xF4) {
        const unsigned lo = b0 == 0xF0 ? 0x90 : 0x80, hi = b0 == 0xF4 ? 0x8F : 0xBF;
        if (!cont(1, lo, hi) || !cont(2, 0x80, 0xBF) || !cont(3, 0x80, 0xBF)) return bad;
        w = 4;
        return ((b0 & 0x07) << 18) | ((s[1] & 0x3F) << 12) | ((s[2] & 0x3F) << 6) | (s[3] & 0x3F);
    }
    return bad;
}

inline void put_rune(std::string& o, uint32_t cp) {
    if (cp < 0x80) {
        o += (char)cp;
    } else if (cp < 0x800) {
        o += (char)(0xC0 | (cp >> 6));
        o += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        o += (char)(0xE0 | (cp >> 12));
        o += (char)(0x80 | ((cp >> 6) & 0x3F));
        o += (char)(0x80 | (cp & 0x3F));
    } else {
        o += (char)(0xF0 | (cp >> 18));
        o += (char)(0x80 | ((cp >> 12) & 0x3F));
        o += (char)(0x80 | ((cp >> 6) & 0x3F));
        o += (char)(0x80 | (cp & 0x3F));
    }
}

// splitWords: calls emit(begin, end) with the byte range of every pre-token, in order.
template <class F>
void split_words(const char* text, size_t n, F&& emit) {
    const unsigned char* t = (const unsigned char*)text;
    size_t start = 0, i = 0;
    int cur = CLS_SPACE;
    while (i < n) {
        int w;
        const int c = char_class(decode_rune(t + i, n - i, w));
        if (i == start) {
            cur = c;
        } else if (!(c == cur && c != CLS_DIGIT && i - start < kMaxWordBytes)) {
            if (cur == CLS_SPACE && c != CLS_SPACE && t[i - 1] == ' ') {
                if (i - 1 > start) emit(start, i - 1);  // the space right before the run belongs to it
                start = i - 1;
            } else {
                emit(start, i);
                start = i;
            }
            cur = c;
        }
        i += w;
    }
    if (start < n) emit(start, n);
}

class TokenizerFormatError : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

struct Tokenizer {
    std::vector<std::string> vocab;
    std::unordered_map<std::string, int> id;
    std::unordered_map<std::string, int> rank;  // pair1 + '\0' + pair2 -> merge rank
    std::unordered_map<std::string, std::vector<int32_t>> cache;
    std::mutex cache_mu;
    // what Decode writes for each id: 0 its vocabulary text, 1 nothing (<PAD>, <EOS>, <USER>, <BOT>),
    // 2 U+FFFD (<UNK>); fixed at construction so that decoding compares no strings
    std::vector<uint8_t> decode_kind;

    static constexpr const char* kPad = "<PAD>";
    static constexpr const char* kUnk = "<UNK>";
    static constexpr const char* kUser = "<USER>";
    static constexpr const char* kBot = "<BOT>";
    static constexpr const char* kEos = "<EOS>";

    // tokenizer.FromVocabAndMerges (tokenizer.go:60-72): a repeated token or pair keeps its last index
    Tokenizer(std::vector<std::string> v, const std::vector<std::pair<std::string, std::string>>& merges)
        : vocab(std::move(v)) {
        id.reserve(vocab.size() * 2);
        for (size_t i = 0; i < vocab.size(); i++) id[vocab[i]] = (int)i;
        rank.reserve(merges.size() * 2);
        for (size_t r = 0; r < merges.size(); r++) rank[pair_key(merges[r].first, merges[r].second)] = (int)r;
        decode_kind.resize(vocab.size(), 0);
        for (size_t i = 0; i < vocab.size(); i++) {
            const std::string& s = vocab[i];
            if (s == kPad || s == kEos || s == kUser || s == kBot) decode_kind[i] = 1;
            else if (s == kUnk) decode_kind[i] = 2;
        }
    }

    // The tokenizer of a parsed model-file header, after tokenizer.CheckFormat on its metadata
    // (quant.Decode, internal/quant/checkpoint.go:201-207); nullptr when the file has no vocabulary.
    static Tokenizer* from_header(const mgjson::Value& hdr) {
        const mgjson::Value* v = hdr.get("vocab");
        if (!v || v->kind != mgjson::Value::Array || v->arr.empty()) return nullptr;
        int version = 0;
        if (const mgjson::Value* meta = hdr.get("metadata")) version = (int)meta->number_or("tokenizer_version", 0);
        if (version != kTokenizerFormat)
            throw TokenizerFormatError("tokenizer format version " + std::to_string(version) +
                                       " is not supported (want " + std::to_string(kTokenizerFormat) +
                                       "): retrain the model");
        std::vector<std::string> vocab;
        vocab.reserve(v->arr.size());
        for (const auto& e : v->arr) {
            if (e.kind != mgjson::Value::String) throw TokenizerFormatError("vocab entries must be strings");
            vocab.push_back(e.str);
        }
        std::vector<std::pair<std::string, std::string>> merges;
        if (const mgjson::Value* m = hdr.get("merges"); m && m->kind == mgjson::Value::Array) {
            merges.reserve(m->arr.size());
            for (const auto& e : m->arr) {
                const mgjson::Value* a = e.get("pair1");
                const mgjson::Value* b = e.get("pair2");
                merges.emplace_back(a && a->kind == mgjson::Value::String ? a->str : std::string(),
                                    b && b->kind == mgjson::Value::String ? b->str : std::string());
            }
        }
        return new Tokenizer(std::move(vocab), merges);
    }

    static std::string pair_key(const std::string& a, const std::string& b) {
        std::string k;
        k.reserve(a.size() + b.size() + 1);
        k += a;
        k += '\0';
        k += b;
        return k;
    }

    int lookup(const char* tok, int missing) const {
        auto it = id.find(tok);
        return it == id.end() ? missing : it->second;
    }
    int pad_id() const { return lookup(kPad, 0); }
    int unk_id() const { return lookup(kUnk, 0); }
    int user_id() const { return lookup(kUser, -1); }
    int bot_id() const { return lookup(kBot, -1); }
    int eos_id() const { return lookup(kEos, -1); }

    std::vector<int32_t> encode_word(const char* w, size_t n) const {
        std::vector<std::string> toks;
        toks.reserve(n);
        const unsigned char* s = (const unsigned char*)w;
        for (size_t i = 0; i < n;) {
            int k;
            const uint32_t r = decode_rune(s + i, n - i, k);
            std::string piece;
            put_rune(piece, r);
            toks.push_back(std::move(piece));
            i += k;
        }
        std::string key;
        while (toks.size() > 1) {
            int best_rank = 0x7fffffff, best = -1;
            for (size_t i = 0; i + 1 < toks.size(); i++) {
                key.assign(toks[i]);
                key += '\0';
                key += toks[i + 1];
                auto it = rank.find(key);
                if (it != rank.end() && it->second < best_rank) {
                    best_rank = it->second;
                    best = (int)i;
                }
            }
            if (best < 0) break;
            toks[best] += toks[best + 1];
            toks.erase(toks.begin() + best + 1);
        }
        const int unk = unk_id();
        std::vector<int32_t> ids(toks.size());
        for (size_t i = 0; i < toks.size(); i++) {
            auto it = id.find(toks[i]);
            ids[i] = it == id.end() ? unk : it->second;
        }
        return ids;
    }

    void encode_plain(const char* text, size_t n, std::vector<int32_t>& out) {
        split_words(text, n, [&](size_t b, size_t e) {
            std::string w(text + b, e - b);
            {
                std::lock_guard<std::mutex> lk(cache_mu);
                auto it = cache.find(w);
                if (it != cache.end()) {
                    out.insert(out.end(), it->second.begin(), it->second.end());
                    return;
                }
            }
            std::vector<int32_t> enc = encode_word(w.data(), w.size());
            out.insert(out.end(), enc.begin(), enc.end());
            std::lock_guard<std::mutex> lk(cache_mu);
            cache.emplace(std::move(w), std::move(enc));
        });
    }

    bool is_special(const std::string& s) const {
        return s.size() >= 2 && s.front() == '<' && s.back() == '>' && id.count(s);
    }

    // Encode: registered "<...>" tokens whole, everything else through encode_plain.
    void encode(const char* text, size_t n, std::vector<int32_t>& out) {
        if (n == 0) return;
        if (!std::memchr(text, '<', n)) {
            encode_plain(text, n, out);
            return;
        }
        size_t pos = 0;
        while (pos < n) {
            const char* lt = (const char*)std::memchr(text + pos, '<', n - pos);
            if (!lt) {
                encode_plain(text + pos, n - pos, out);
                break;
            }
            const size_t s = lt - text;
            const char* gt = (const char*)std::memchr(text + s, '>', n - s);
            if (!gt) {
                encode_plain(text + pos, n - pos, out);
                break;
            }
            const size_t e = gt - text + 1;
            std::string cand(text + s, e - s);
            if (is_special(cand)) {
                if (s > pos) encode_plain(text + pos, s - pos, out);
                out.push_back(id.at(cand));
                pos = e;
            } else {
                encode_plain(text + pos, s + 1 - pos, out);
                pos = s + 1;
            }
        }
    }

    // the chat template (internal/tokenizer/template.go:12-21): <USER> prompt <BOT>
    void encode_prompt(const char* text, size_t n, std::vector<int32_t>& out) {
        out.push_back(user_id());
        encode(text, n, out);
        out.push_back(bot_id());
    }

    // EncodeReply (template.go:23-26): reply <EOS>
    void encode_reply(const char* text, size_t n, std::vector<int32_t>& out) {
        encode(text, n, out);
        out.push_back(eos_id());
    }

    void decode(const int32_t* ids, size_t n, std::string& out) const {
        for (size_t i = 0; i < n; i++) {
            const int32_t t = ids[i];
            if (t < 0 || (size_t)t >= vocab.size()) continue;
            const uint8_t k = decode_kind[t];
            if (k == 1) continue;
            if (k == 2) out += "\xEF\xBF\xBD";
            else out += vocab[t];
        }
    }

    // TokenBytes (internal/tokenizer/bytes.go:13-22): bytes of text each id decodes to
    std::vector<int32_t> token_bytes() const {
        std::vector<int32_t> b(vocab.size());
        std::string s;
        for (size_t i = 0; i < vocab.size(); i++) {
            s.clear();
            const int32_t t = (int32_t)i;
            decode(&t, 1, s);
            b[i] = (int32_t)s.size();
        }
        return b;
    }
};

}  // namespace mg
