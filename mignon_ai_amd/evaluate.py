"""Held-out scoring through the library: eval.Perplexity and eval.PerplexityPerDoc (internal/eval/eval.go:50-75,
internal/eval/perdoc.go:12-48) with every target of the text scored in one batched pass on the GPU
(mg_perplexity over mg_score_sequences), instead of one Call per target.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import HeldOut as _HeldOut
from ._lib import check, lib, ptr
from .model import Model
from .tokenizer import Tokenizer


@dataclass
class HeldOut:
    """eval.HeldOut: loss (nats per token), perplexity, bits per byte of text, scored tokens."""
    loss: float
    ppl: float
    bpb: float
    tokens: int


def _run(model: Model, tok: Tokenizer, text, context: int, max_count: int, per_doc: bool) -> HeldOut:
    b = text.encode("utf-8") if isinstance(text, str) else bytes(text)
    h = _HeldOut()
    check(lib().mg_perplexity(model.handle, tok.handle, b, len(b), int(context), int(max_count), int(per_doc),
                              ctypes.byref(h)))
    return HeldOut(h.loss, h.ppl, h.bpb, h.tokens)


def perplexity(model: Model, tok: Tokenizer, text, context: int, max_tokens: int = 0) -> HeldOut:
    """eval.Perplexity: text as one stream; each of the first max_tokens targets (all when <= 0) scored
    from the context tokens before it."""
    return _run(model, tok, text, context, max_tokens, False)


def perplexity_per_doc(model: Model, tok: Tokenizer, text, context: int, max_docs: int = 0) -> HeldOut:
    """eval.PerplexityPerDoc: documents split on <EOS>, each scored from a fresh <EOS>."""
    return _run(model, tok, text, context, max_docs, True)


def score_sequences(model: Model, seqs, context: int) -> list[np.ndarray]:
    """Per-target log-probabilities of each token sequence (mg_score_sequences): entry t-1 of sequence q is
    log p(seq[t] | window(seq[:t], context)); NaN where the reference scores nothing."""
    seqs = [np.ascontiguousarray(s, np.int32) for s in seqs]
    offsets = np.zeros(len(seqs) + 1, np.int64)
    for i, s in enumerate(seqs):
        offsets[i + 1] = offsets[i] + len(s)
    tokens = np.concatenate(seqs) if seqs else np.zeros(0, np.int32)
    counts = [max(len(s) - 1, 0) for s in seqs]
    lp = np.empty(max(sum(counts), 1), np.float32)
    check(lib().mg_score_sequences(model.handle, ptr(tokens) if tokens.size else None, ptr(offsets), len(seqs),
                                   int(context), ptr(lp)))
    out, k = [], 0
    for c in counts:
        out.append(lp[k:k + c].copy())
        k += c
    return out
