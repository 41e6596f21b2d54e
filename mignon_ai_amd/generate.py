"""Text generation through the library: infer.Generate's greedy branch (pkg/infer/infer.go:64-84;
generate.DecodeGreedy / greedyLoop, internal/generate/greedy.go:43-102) over batched device sessions,
with the tokenizer stored in the model file (mg_generate_greedy).

    g = Generator.load("orders.mgn")
    g.generate("unpaid orders").text
    g.generate_batch(requests, max_tokens=80)
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from ._lib import check, lib, ptr
from .model import Model, read_metadata
from .tokenizer import Tokenizer

CHAT_MAX_RESPONSE_TOKENS = 60  # internal/generate/constants.go:6 (infer.DefaultMaxTokens)
TASK_CHAT = "chat"             # model.TaskChat


@dataclass
class Piece:
    """generate.Piece / infer.Token: one generated token's text and probability."""
    text: str
    prob: float


@dataclass
class Result:
    """infer.Result: the reply, trimmed of surrounding whitespace, and its tokens (built on first use from
    the token ids, their probabilities and the tokenizer's per-token texts)."""
    text: str
    ids: list[int] = field(default_factory=list)
    probs: list[float] = field(default_factory=list)
    _texts: list[str] | None = field(default=None, repr=False, compare=False)

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

    def generate(self, prompt, max_tokens: int = 0) -> Result:
        """infer.Generate with Temperature 0."""
        return self.generate_batch([prompt], max_tokens)[0]

    def generate_batch(self, prompts, max_tokens: int = 0) -> list[Result]:
        """infer.Generate for every prompt, all decoded together on device sessions."""
        if max_tokens <= 0:
            max_tokens = CHAT_MAX_RESPONSE_TOKENS
        n = len(prompts)
        if n == 0:
            return []
        enc = [p.encode("utf-8") if isinstance(p, str) else bytes(p) for p in prompts]
        arr = (ctypes.c_char_p * n)(*enc)
        lens = (ctypes.c_size_t * n)(*[len(b) for b in enc])
        ids = np.empty((n, max_tokens), np.int32)
        probs = np.empty((n, max_tokens), np.float64)
        counts = np.empty(n, np.int32)
        check(lib().mg_generate_greedy(self.model.handle, self.tok.handle, arr, lens, n, self.context_size(),
                                       max_tokens, int(self.task() == TASK_CHAT), ptr(ids), ptr(probs), ptr(counts)))
        texts = self.tok.piece_texts()
        out = []
        for i in range(n):
            k = int(counts[i])
            row = ids[i, :k].tolist()
            out.append(Result("".join([texts[t] for t in row]).strip(), row, probs[i, :k].tolist(), texts))
        return out
