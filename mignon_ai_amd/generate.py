"""Text generation through the library: infer.Generate (pkg/infer/infer.go:64-96) over batched device
sessions, with the tokenizer stored in the model file. Temperature 0 decodes greedily
(generate.DecodeGreedy / greedyLoop, internal/generate/greedy.go:43-102; mg_generate_greedy); above 0 the
reply is sampled (generate.Chat / Text over sampleContinuation, internal/generate/chat.go,
sample.go; mg_generate_sample), each prompt's draws seeded by its own seed.

    g = Generator.load("orders.mgn")
    g.generate("unpaid orders").text
    g.generate_batch(requests, max_tokens=80)
    g.generate_batch(requests, temperature=0.7, top_k=40, top_p=0.9, rep_penalty=1.2, seeds=range(len(requests)))
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

from ._lib import Sampling, check, lib, ptr
from .model import Model, read_metadata
from .tokenizer import Tokenizer

CHAT_MAX_RESPONSE_TOKENS = 60  # internal/generate/constants.go:6 (infer.DefaultMaxTokens)
TASK_CHAT = "chat"             # model.TaskChat
# unicode.IsSpace, what strings.TrimSpace removes (Python's str.strip() without arguments removes more)
GO_SPACE = "\t\n\v\f\r \x85\xa0\u1680\u2000\u2001\u2002\u2003\u2004\u2005\u2006\u2007\u2008\u2009\u200a" \
           "\u2028\u2029\u202f\u205f\u3000"


def trim_space(text: str) -> str:
    """strings.TrimSpace."""
    return text.strip(GO_SPACE)


@dataclass
class Piece:
    """generate.Piece / infer.Token: one generated token's text and probability."""
    text: str
    prob: float


class Result:
    """infer.Result: the reply, trimmed of surrounding whitespace, and its tokens (built on first use from
    the token ids, their probabilities and the tokenizer's per-token texts).

    A batch of thousands of replies would otherwise leave several garbage-collected containers per reply
    (a dict, two lists), whose count sets off Python's cyclic collector over the whole heap several times
    per batch; the ids and probabilities are therefore kept as the call's own numpy arrays (with row
    set: the batch's matrices, of which this reply is the first n entries of that row) and turned into
    lists when first read, and the fields live in slots. The lists are kept once built (so edits to them
    stay) and may be replaced by assignment; once both have been read the reply holds no reference to the
    batch's matrices."""
    __slots__ = ("text", "_ids", "_probs", "_texts", "_row", "_n")

    def __init__(self, text: str, ids=(), probs=(), texts: list[str] | None = None, row: int | None = None,
                 n: int = 0):
        self.text = text
        self._ids = ids      # token ids: a sequence, or the batch's id matrix
        self._probs = probs  # their probabilities (empty when sampled), or the batch's matrix
        self._texts = texts
        self._row = row
        self._n = n

    def _mine(self, a):
        if self._row is None or not isinstance(a, np.ndarray) or a.ndim != 2:
            return a
        return a[self._row, :self._n]

    @property
    def ids(self) -> list[int]:
        if not isinstance(self._ids, list):
            self._ids = np.asarray(self._mine(self._ids), np.int64).tolist()
        return self._ids

    @ids.setter
    def ids(self, v):
        self._ids = list(v)

    @property
    def probs(self) -> list[float]:
        if not isinstance(self._probs, list):
            self._probs = np.asarray(self._mine(self._probs), np.float64).tolist()
        return self._probs

    @probs.setter
    def probs(self, v):
        self._probs = list(v)

    def __eq__(self, other) -> bool:
        if not isinstance(other, Result):
            return NotImplemented
        return (self.text, self.ids, self.probs) == (other.text, other.ids, other.probs)

    __hash__ = None

    def __repr__(self) -> str:
        return f"Result(text={self.text!r}, ids={self.ids!r}, probs={self.probs!r})"

    @property
    def tokens(self) -> list[Piece]:
        return [Piece(self._texts[t], p) for t, p in zip(self.ids, self.probs)]

    @property
    def min_prob(self) -> float:
        """infer.Result.MinProb (pkg/infer/infer.go:54-62)."""
        return min(self.probs, default=1.0)


class Generator:
    """A model, its tokenizer and metadata (what pkg/infer.Load returns) on the GPU."""

    def __init__(self, model: Model, tok: Tokenizer, metadata: dict):
        if tok is None:
            raise ValueError("the model file has no tokenizer")
        self.model, self.tok, self.metadata = model, tok, metadata

    @classmethod
    def from_bytes(cls, data: bytes, max_context: int = 0) -> "Generator":
        return cls(Model(data, max_context), Tokenizer.from_model_file(data), read_metadata(data))

    @classmethod
    def load(cls, path: str, max_context: int = 0) -> "Generator":
        with open(path, "rb") as f:
            return cls.from_bytes(f.read(), max_context)

    def task(self) -> str:
        return self.metadata.get("task", "")

    def context_size(self) -> int:
        """model.Model.ContextSize: the metadata's context_size."""
        return int(self.metadata.get("context_size", 0))

    def generate(self, prompt, max_tokens: int = 0, temperature: float = 0.0, top_k: int = 0, top_p: float = 0.0,
                 rep_penalty: float = 0.0, seed: int | None = None) -> Result:
        """infer.Generate with infer.Options' fields."""
        return self.generate_batch([prompt], max_tokens, temperature, top_k, top_p, rep_penalty,
                                   None if seed is None else [seed])[0]

    def generate_batch(self, prompts, max_tokens: int = 0, temperature: float = 0.0, top_k: int = 0,
                       top_p: float = 0.0, rep_penalty: float = 0.0, seeds=None) -> list[Result]:
        """infer.Generate for every prompt, all decoded together on device sessions. When sampling, seeds[i]
        (a 64-bit integer) fixes prompt i's draws; without seeds they are drawn from os.urandom, as the
        reference's global generator is seeded at random."""
        if max_tokens <= 0:
            max_tokens = CHAT_MAX_RESPONSE_TOKENS
        n = len(prompts)
        if n == 0:
            return []
        chat = self.task() == TASK_CHAT
        enc = [p.encode("utf-8") if isinstance(p, str) else bytes(p) for p in prompts]
        arr = (ctypes.c_char_p * n)(*enc)
        lens = (ctypes.c_size_t * n)(*[len(b) for b in enc])
        ids = np.empty((n, max_tokens), np.int32)
        counts = np.empty(n, np.int32)
        texts = self.tok.piece_texts()
        if temperature <= 0:
            probs = np.empty((n, max_tokens), np.float64)
            check(lib().mg_generate_greedy(self.model.handle, self.tok.handle, arr, lens, n, self.context_size(),
                                           max_tokens, int(chat), ptr(ids), ptr(probs), ptr(counts)))
            # infer.Result.Text: strings.TrimSpace of the decoded reply (pkg/infer/infer.go:76-79)
            replies = self.tok.decode_rows(ids, counts, trim=True)
            cl = counts.tolist()
            return [Result(replies[i], ids, probs, texts, i, cl[i]) for i in range(n)]
        sp = Sampling(temperature=temperature, rep_penalty=rep_penalty, top_p=top_p if top_p > 0 else 1.0,
                      top_k=top_k, penalize_prompt=0)
        if seeds is None:
            seeds = np.frombuffer(os.urandom(8 * n), np.uint64)
        sd = np.ascontiguousarray(np.asarray([int(x) & (2 ** 64 - 1) for x in seeds], np.uint64))
        if sd.size != n:
            raise ValueError("one seed per prompt")
        check(lib().mg_generate_sample(self.model.handle, self.tok.handle, arr, lens, n, self.context_size(),
                                       max_tokens, int(chat), ctypes.byref(sp), ptr(sd), ptr(ids), ptr(counts)))
        replies = self.tok.decode_rows(ids, counts, trim=chat)
        cl = counts.tolist()
        return [Result(replies[i], ids, (), texts, i, cl[i]) for i in range(n)]  # Tokens stay empty
