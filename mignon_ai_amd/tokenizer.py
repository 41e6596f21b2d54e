"""Python binding of the library's tokenizer (mignon_ai_amd/csrc/tokenizer.hpp through the C ABI): the
byte-pair-encoding tokenizer stored in a model file, with the reference's interface (internal/tokenizer:
Encode, Decode, EncodePrompt, EncodeReply, DropOldestTurns, TokenBytes, special-token ids).

Text may be str (encoded as UTF-8) or bytes; decode returns str (invalid UTF-8 bytes, which only a
vocabulary built from invalid text could produce, are replaced).
"""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import check, lib, ptr

PAD, UNK, USER, BOT, EOS = "<PAD>", "<UNK>", "<USER>", "<BOT>", "<EOS>"
_SPECIAL = {PAD: 0, UNK: 1, USER: 2, BOT: 3, EOS: 4}  # MG_TOKEN_*
_MODE = {"text": 0, "prompt": 1, "reply": 2}        # MG_ENCODE_*


def _bytes(text) -> bytes:
    return text.encode("utf-8") if isinstance(text, str) else bytes(text)


def split_words(text) -> list[str | bytes]:
    """splitWords (internal/tokenizer/pretokenize.go:39-67): the pre-tokens of text, in order (str in,
    str out; bytes in, bytes out)."""
    b = _bytes(text)
    n = check(lib().mg_pretokenize(b, len(b), None, 0))
    ends = np.empty(max(n, 1), np.int64)
    check(lib().mg_pretokenize(b, len(b), ptr(ends), n))
    out, start = [], 0
    for e in ends[:n]:
        out.append(b[start:int(e)])
        start = int(e)
    return [w.decode("utf-8") for w in out] if isinstance(text, str) else out


class Tokenizer:
    """tokenizer.Tokenizer of a model file (quant.Decode's FromVocabAndMerges after CheckFormat)."""

    def __init__(self, handle):
        self._h = handle
        self._vocab = None

    @classmethod
    def from_model_file(cls, data: bytes) -> "Tokenizer | None":
        buf = (ctypes.c_uint8 * len(data)).from_buffer_copy(data)
        h = ctypes.c_void_p()
        check(lib().mg_tokenizer_load(buf, len(data), ctypes.byref(h)))
        return cls(h) if h.value else None

    @classmethod
    def load(cls, path: str) -> "Tokenizer | None":
        with open(path, "rb") as f:
            return cls.from_model_file(f.read())

    def close(self):
        if getattr(self, "_h", None):
            lib().mg_tokenizer_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def handle(self):
        return self._h

    def vocab_size(self) -> int:
        return lib().mg_tokenizer_vocab_size(self._h)

    def token(self, i: int) -> str:
        """Vocab[i]."""
        n = check(lib().mg_tokenizer_token(self._h, int(i), None, 0))
        buf = ctypes.create_string_buffer(max(n, 1))
        check(lib().mg_tokenizer_token(self._h, int(i), buf, n))
        return buf.raw[:n].decode("utf-8", errors="replace")

    @property
    def vocab(self) -> list[str]:
        if self._vocab is None:
            self._vocab = [self.token(i) for i in range(self.vocab_size())]
        return self._vocab

    def special(self, name: str) -> int:
        return lib().mg_tokenizer_special(self._h, _SPECIAL[name])

    def pad_id(self) -> int:
        return self.special(PAD)

    def unk_id(self) -> int:
        return self.special(UNK)

    def user_id(self) -> int:
        return self.special(USER)

    def bot_id(self) -> int:
        return self.special(BOT)

    def eos_id(self) -> int:
        return self.special(EOS)

    def _encode(self, text, mode: str) -> list[int]:
        b = _bytes(text)
        n = check(lib().mg_tokenizer_encode(self._h, b, len(b), _MODE[mode], None, 0))
        ids = np.empty(max(n, 1), np.int32)
        check(lib().mg_tokenizer_encode(self._h, b, len(b), _MODE[mode], ptr(ids), n))
        return ids[:n].tolist()

    def encode(self, text) -> list[int]:
        return self._encode(text, "text")

    def encode_prompt(self, prompt) -> list[int]:
        """EncodePrompt (internal/tokenizer/template.go:11-16): <USER> prompt <BOT>."""
        return self._encode(prompt, "prompt")

    def encode_reply(self, reply) -> list[int]:
        """EncodeReply (internal/tokenizer/template.go:18-21): reply <EOS>."""
        return self._encode(reply, "reply")

    def decode_bytes(self, ids) -> bytes:
        a = np.ascontiguousarray(np.asarray(list(ids) if not isinstance(ids, np.ndarray) else ids, np.int32))
        n = check(lib().mg_tokenizer_decode(self._h, ptr(a), a.size, None, 0))
        buf = ctypes.create_string_buffer(max(n, 1))
        check(lib().mg_tokenizer_decode(self._h, ptr(a), a.size, buf, n))
        return buf.raw[:n]

    def decode(self, ids) -> str:
        return self.decode_bytes(ids).decode("utf-8", errors="replace")

    def decode_rows(self, ids, counts, trim: bool = False) -> list[str]:
        """mg_tokenizer_decode_rows: Decode of every row of a [n][ld] id matrix (row i: its first counts[i]
        ids), each text trimmed of surrounding white space (strings.TrimSpace) when trim is set, in one
        call; invalid UTF-8 reads as U+FFFD."""
        ids = np.ascontiguousarray(ids, np.int32)
        counts = np.ascontiguousarray(counts, np.int32)
        n, ld = ids.shape
        if getattr(self, "_max_token_bytes", None) is None:
            self._max_token_bytes = max(self.token_bytes(), default=0)
        cap = int(counts.sum()) * self._max_token_bytes
        buf = ctypes.create_string_buffer(max(cap, 1))
        off = np.empty(n + 1, np.int64)
        total = check(lib().mg_tokenizer_decode_rows(self._h, ptr(ids), ptr(counts), n, ld, int(trim), buf, cap,
                                                     ptr(off)))
        raw = ctypes.string_at(buf, total)
        o = off.tolist()
        return [raw[o[i]:o[i + 1]].decode("utf-8", errors="replace") for i in range(n)]

    def piece_texts(self) -> list[str]:
        """Decode([id]) for every id (cached): the text each token contributes; Decode of a sequence is the
        concatenation of its tokens' texts."""
        if getattr(self, "_pieces", None) is None:
            self._pieces = [self.decode([i]) for i in range(self.vocab_size())]
        return self._pieces

    def token_bytes(self) -> list[int]:
        out = np.empty(self.vocab_size(), np.int32)
        check(lib().mg_tokenizer_token_bytes(self._h, ptr(out)))
        return out.tolist()

    def drop_oldest_turns(self, history: list[int], max_len: int) -> list[int]:
        """DropOldestTurns (internal/tokenizer/template.go:23-35): whole turns, each ending in <EOS>, leave
        the front of history until at most max_len tokens remain; nothing remains without a complete turn."""
        eos = self.eos_id()
        history = list(history)
        while len(history) > max(max_len, 0):
            if eos not in history:
                return []
            history = history[history.index(eos) + 1:]
        return history
