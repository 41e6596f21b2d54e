"""Greedy text generation over a session provider, host side.

Mirrors internal/generate/greedy.go (DecodeGreedy, greedyLoop, argmaxProb) and the greedy branch of
pkg/infer.Generate (pkg/infer/infer.go:64-84): the prompt goes through the chat template when the model's
task is "chat", the reply stops before <EOS>, <USER> or <BOT>, and every token comes with the softmax
probability the model gave it. A session provider is anything with new_session(context_size) returning
an object with prefill(tokens) -> logits and append(token) -> logits (infer.SessionProvider); the GPU
Model is one.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .tokenizer import Tokenizer, read_header

CHAT_MAX_RESPONSE_TOKENS = 60  # internal/generate/constants.go:6; infer.DefaultMaxTokens (pkg/infer/infer.go:22)
TASK_CHAT = "chat"  # model.TaskChat


def argmax_prob(logits) -> tuple[int, float]:
    """argmaxProb (greedy.go:89-102): the first maximum and its softmax probability, in float64."""
    vals = [float(v) for v in logits]
    best = 0
    for i, v in enumerate(vals):
        if v > vals[best]:
            best = i
    s = 0.0
    for v in vals:
        s += math.exp(v - vals[best])
    return best, 1.0 / s


def greedy_loop(session, context, max_tokens: int, stops=()) -> tuple[list[int], list[float]]:
    """greedyLoop (greedy.go:63-87) without a constraint or cancellation: no Append after the last token."""
    ids, probs = [], []
    logits = session.prefill(list(context))
    while len(ids) < max_tokens and logits is not None and len(logits) > 0:
        best, prob = argmax_prob(logits)
        if best in stops:
            break
        ids.append(best)
        probs.append(prob)
        if len(ids) < max_tokens:
            logits = session.append(best)
    return ids, probs


@dataclass
class Piece:
    text: str
    prob: float


@dataclass
class Greedy:
    """generate.Greedy: the decoded reply (untrimmed) and its pieces."""
    text: str
    pieces: list[Piece] = field(default_factory=list)
    ids: list[int] = field(default_factory=list)


def decode_greedy(provider, tok: Tokenizer, prompt: str, context_size: int, max_tokens: int,
                  chat: bool = True) -> Greedy:
    """DecodeGreedy (greedy.go:43-57)."""
    context = tok.encode_prompt(prompt) if chat else tok.encode(prompt)
    ids, probs = greedy_loop(provider.new_session(context_size), context, max_tokens,
                             stops=(tok.eos_id(), tok.user_id(), tok.bot_id()))
    return Greedy(text=tok.decode(ids), pieces=[Piece(tok.decode([i]), p) for i, p in zip(ids, probs)], ids=ids)


@dataclass
class Result:
    """infer.Result: the trimmed reply and each token's text and probability."""
    text: str
    tokens: list[Piece] = field(default_factory=list)

    @property
    def min_prob(self) -> float:
        return min((p.prob for p in self.tokens), default=1.0)


class Generator:
    """A model, its tokenizer and metadata, as pkg/infer.Load returns them (model.Model).

    `provider` runs the network: the GPU Model by default (Generator.load); tests pass the CPU oracle."""

    def __init__(self, provider, tok: Tokenizer, metadata: dict):
        if tok is None:
            raise ValueError("the model file has no tokenizer")
        self.provider, self.tok, self.metadata = provider, tok, metadata

    @classmethod
    def from_bytes(cls, data: bytes, provider=None) -> "Generator":
        hdr = read_header(data)
        if provider is None:
            from .model import Model
            provider = Model(data)
        return cls(provider, Tokenizer.from_header(hdr), hdr.get("metadata") or {})

    @classmethod
    def load(cls, path: str, provider=None) -> "Generator":
        with open(path, "rb") as f:
            return cls.from_bytes(f.read(), provider)

    def task(self) -> str:
        return self.metadata.get("task", "")

    def context_size(self) -> int:
        return int(self.metadata.get("context_size", 0))

    def generate(self, prompt: str, max_tokens: int = 0) -> Result:
        """infer.Generate with greedy options (Temperature 0)."""
        if max_tokens <= 0:
            max_tokens = CHAT_MAX_RESPONSE_TOKENS
        g = decode_greedy(self.provider, self.tok, prompt, self.context_size(), max_tokens,
                          chat=self.task() == TASK_CHAT)
        return Result(text=g.text.strip(), tokens=g.pieces)

    def generate_batch(self, prompts: list[str], max_tokens: int = 0) -> list[Result]:
        """generate() for many prompts in one batch of device sessions: every prompt's greedy tokens
        come from one batched decode (mg_sessions_decode_greedy), cut at the first stop token, which
        gives the same reply as the per-prompt loop (a greedy choice depends only on the tokens before
        it). The provider must offer sessions(n, context_size) (the GPU Model does)."""
        if max_tokens <= 0:
            max_tokens = CHAT_MAX_RESPONSE_TOKENS
        if not prompts:
            return []
        chat = self.task() == TASK_CHAT
        ctxs = [self.tok.encode_prompt(p) if chat else self.tok.encode(p) for p in prompts]
        live = [i for i, c in enumerate(ctxs) if c]  # an empty context prefills to nothing: no reply
        out = [Result(text="") for _ in prompts]
        if not live:
            return out
        L = max(len(ctxs[i]) for i in live)
        arr = np.full((len(live), L), self.tok.pad_id(), np.int32)
        lens = np.empty(len(live), np.int32)
        for r, i in enumerate(live):
            arr[r, :len(ctxs[i])] = ctxs[i]
            lens[r] = len(ctxs[i])
        sess = self.provider.sessions(len(live), self.context_size())
        try:
            ids, probs = sess.decode_greedy(arr, max_tokens, lens)
        finally:
            sess.close()
        stops = {self.tok.eos_id(), self.tok.user_id(), self.tok.bot_id()}
        for r, i in enumerate(live):
            row = [int(t) for t in ids[r]]
            n = next((k for k, t in enumerate(row) if t in stops), len(row))
            pieces = [Piece(self.tok.decode([t]), float(p)) for t, p in zip(row[:n], probs[r, :n])]
            out[i] = Result(text=self.tok.decode(row[:n]).strip(), tokens=pieces)
        return out
