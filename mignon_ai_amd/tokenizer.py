"""Byte-pair-encoding tokenizer of a mignon-ai model file, host side (the model's own vocabulary and merge
table travel in the file header).

Mirrors internal/tokenizer (format version 2): pre-tokenization (pretokenize.go:9-67), rank-ordered
pair merges within each pre-token (tokenizer.go:190-232), atomic special tokens (tokenizer.go:264-311),
decoding that skips turn markers (tokenizer.go:355-375) and the chat template (template.go:12-35).
Training (bpe_train.go) is not part of the inference path and is not provided.
"""
from __future__ import annotations

import json
import struct
import unicodedata

PAD, UNK, USER, BOT, EOS = "<PAD>", "<UNK>", "<USER>", "<BOT>", "<EOS>"
FORMAT_VERSION = 2  # internal/tokenizer/format.go:8
MAX_WORD_BYTES = 128  # pretokenize.go:7

# character classes of pretokenize.go:11-33 (Go's unicode.IsSpace / IsPunct / IsSymbol / IsDigit)
_WORD, _SPACE, _PUNCT, _DIGIT = 0, 1, 2, 3
_LATIN1_SPACE = set("\t\n\v\f\r \x85\xa0")
_OTHER_SPACE = {0x1680, 0x2028, 0x2029, 0x202F, 0x205F, 0x3000} | set(range(0x2000, 0x200B))


def _class(ch: str) -> int:
    o = ord(ch)
    if (o <= 0xFF and ch in _LATIN1_SPACE) or (o > 0xFF and o in _OTHER_SPACE):
        return _SPACE
    cat = unicodedata.category(ch)
    if cat[0] in "PS":
        return _PUNCT
    if cat == "Nd":
        return _DIGIT
    return _WORD


def split_words(text: str) -> list[str]:
    """splitWords: runs of one class, each digit alone, at most MAX_WORD_BYTES bytes; a single space
    before a word or punctuation run joins that run. The pieces concatenate back to text."""
    out = []
    if not text:
        return out
    chars = list(text)
    offs = []  # byte offset of every character (Go ranges over a string by byte index)
    pos = 0
    for ch in chars:
        offs.append(pos)
        pos += len(ch.encode("utf-8"))
    start_ci = 0
    cur = _SPACE
    for ci, ch in enumerate(chars):
        c = _class(ch)
        if ci == start_ci:
            cur = c
            continue
        if c == cur and c != _DIGIT and offs[ci] - offs[start_ci] < MAX_WORD_BYTES:
            continue
        if cur == _SPACE and c != _SPACE and chars[ci - 1] == " ":
            if ci - 1 > start_ci:
                out.append("".join(chars[start_ci:ci - 1]))
            start_ci = ci - 1
        else:
            out.append("".join(chars[start_ci:ci]))
            start_ci = ci
        cur = c
    if start_ci < len(chars):
        out.append("".join(chars[start_ci:]))
    return out


class TokenizerError(ValueError):
    pass


def read_header(data: bytes) -> dict:
    """The JSON header of a binary model file (internal/binfmt/binfmt.go: "MGNN", uint16 version,
    uint8 kind, uint8 reserved, uint32 header length, header)."""
    if len(data) < 12 or data[:4] != b"MGNN":
        raise TokenizerError("not a binary model file")
    n = struct.unpack_from("<I", data, 8)[0]
    if 12 + n > len(data):
        raise TokenizerError("model file header is truncated")
    return json.loads(data[12:12 + n])


class Tokenizer:
    """tokenizer.Tokenizer as FromVocabAndMerges builds it (tokenizer.go:62-75)."""

    def __init__(self, vocab: list[str], merges: list[tuple[str, str]]):
        self.vocab = list(vocab)
        self.token_to_id = {}
        for i, s in enumerate(self.vocab):
            self.token_to_id[s] = i  # later duplicates win, as Go's map assignment does
        self.ranks = {}
        for r, (a, b) in enumerate(merges):
            self.ranks[a + "\x00" + b] = r  # a repeated pair keeps its last rank (initRanks)
        self._cache: dict[str, list[int]] = {}

    @classmethod
    def from_model_file(cls, data: bytes) -> "Tokenizer | None":
        """The tokenizer stored in a binary model file (quant.Decode, internal/quant/checkpoint.go:201-207);
        None when the file has no vocabulary."""
        return cls.from_header(read_header(data))

    @classmethod
    def from_header(cls, hdr: dict) -> "Tokenizer | None":
        vocab = hdr.get("vocab") or []
        if not vocab:
            return None
        version = (hdr.get("metadata") or {}).get("tokenizer_version", 0)
        if version != FORMAT_VERSION:
            raise TokenizerError(f"tokenizer format version {version} is not supported (want {FORMAT_VERSION}): "
                                 "retrain the model")
        merges = [(m["pair1"], m["pair2"]) for m in (hdr.get("merges") or [])]
        return cls(vocab, merges)

    def vocab_size(self) -> int:
        return len(self.vocab)

    def _special(self, tok: str) -> int:
        return self.token_to_id.get(tok, -1)

    def eos_id(self) -> int:
        return self._special(EOS)

    def user_id(self) -> int:
        return self._special(USER)

    def bot_id(self) -> int:
        return self._special(BOT)

    def pad_id(self) -> int:
        return self.token_to_id.get(PAD, 0)

    def _encode_word(self, word: str) -> list[int]:
        toks = list(word)
        while len(toks) > 1:
            best_rank, best = None, -1
            for i in range(len(toks) - 1):
                r = self.ranks.get(toks[i] + "\x00" + toks[i + 1])
                if r is not None and (best_rank is None or r < best_rank):
                    best_rank, best = r, i
            if best < 0:
                break
            toks = toks[:best] + [toks[best] + toks[best + 1]] + toks[best + 2:]
        unk = self.token_to_id.get(UNK, 0)
        return [self.token_to_id.get(t, unk) for t in toks]

    def _encode_plain(self, text: str) -> list[int]:
        ids = []
        for w in split_words(text):
            enc = self._cache.get(w)
            if enc is None:
                enc = self._encode_word(w)
                self._cache[w] = enc
            ids.extend(enc)
        return ids

    def _is_special(self, s: str) -> bool:
        return s.startswith("<") and s.endswith(">") and s in self.token_to_id

    def encode(self, text: str) -> list[int]:
        """Encode: registered "<...>" tokens are taken whole, the rest is BPE-encoded."""
        if not text:
            return []
        if "<" not in text:
            return self._encode_plain(text)
        ids = []
        rem = text
        while rem:
            s = rem.find("<")
            if s < 0:
                ids.extend(self._encode_plain(rem))
                break
            e = rem.find(">", s)
            if e < 0:
                ids.extend(self._encode_plain(rem))
                break
            cand = rem[s:e + 1]
            if self._is_special(cand):
                if s > 0:
                    ids.extend(self._encode_plain(rem[:s]))
                ids.append(self.token_to_id[cand])
                rem = rem[e + 1:]
            else:
                ids.extend(self._encode_plain(rem[:s + 1]))
                rem = rem[s + 1:]
        return ids

    def decode(self, ids) -> str:
        """Decode: turn markers and padding print nothing, <UNK> prints U+FFFD."""
        out = []
        for i in ids:
            i = int(i)
            if 0 <= i < len(self.vocab):
                t = self.vocab[i]
                if t in (PAD, EOS, USER, BOT):
                    continue
                out.append("�" if t == UNK else t)
        return "".join(out)

    # chat template (template.go:12-35): <USER> prompt <BOT> response <EOS>
    def encode_prompt(self, prompt: str) -> list[int]:
        return [self.user_id()] + self.encode(prompt) + [self.bot_id()]

    def encode_reply(self, reply: str) -> list[int]:
        return self.encode(reply) + [self.eos_id()]

    def drop_oldest_turns(self, history: list[int], max_len: int) -> list[int]:
        eos = self.eos_id()
        history = list(history)
        while len(history) > max(max_len, 0):
            if eos not in history:
                return []
            history = history[history.index(eos) + 1:]
        return history
