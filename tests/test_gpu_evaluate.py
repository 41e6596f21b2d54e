"""Held-out scoring on the GPU (mg_score_sequences, mg_perplexity) against the oracle's restatement of
eval.Perplexity / PerplexityPerDoc (oracle/text.py, one oracle Call per target, internal/eval/eval.go:25-75,
internal/eval/perdoc.go:12-48): every target's log-probability within 1e-4 (of max(1, |ref|)), the same
targets scored, and loss, perplexity and bits per byte within 1e-5 relative."""
import json
import os

import numpy as np
import pytest

from helpers import EQUIV_CASES, GOLDEN, equiv_model_bytes, oracle_model
from mignon_ai_amd import Model
from mignon_ai_amd.evaluate import perplexity, perplexity_per_doc, score_sequences
from mignon_ai_amd.tokenizer import Tokenizer
from oracle import text as T

pytestmark = pytest.mark.gpu

ORDERS = os.path.join(GOLDEN, "orders.mgn")
LP_TOL = 1e-4


@pytest.fixture(scope="module")
def orders():
    with open(ORDERS, "rb") as f:
        data = f.read()
    return Model(data), Tokenizer.from_model_file(data), oracle_model(data), T.Tokenizer.from_model_file(data)


@pytest.fixture(scope="module")
def corpus():
    """The order-search pairs as chat turns, one document per pair."""
    with open(os.path.join(GOLDEN, "orders_handwritten.json")) as f:
        pairs = json.load(f)
    return [f"<USER>{p['instruction']}<BOT>{p['output']}<EOS>" for p in pairs]


def _terms_close(got, want):
    got = np.asarray(got, np.float64)
    assert len(got) == len(want)
    for g, w in zip(got, want):
        if w is None:
            assert np.isnan(g)
        else:
            assert abs(g - w) <= LP_TOL * max(1.0, abs(w)), (g, w)


def _held_close(got, want):
    assert got.tokens == want["tokens"]
    for k in ("loss", "ppl", "bpb"):
        assert getattr(got, k) == pytest.approx(want[k], rel=1e-5, abs=1e-12), k


@pytest.mark.parametrize("context", [128, 24, 1])
def test_perplexity_stream(orders, corpus, context):
    """eval.Perplexity over the corpus as one stream; context 24 and 1 slide the window past the first
    targets (one row per later target)."""
    gm, gt, om, ot = orders
    text = "".join(corpus[:40])
    want = T.perplexity(om.call, ot, text.encode(), context)
    _held_close(perplexity(gm, gt, text, context), want)


def test_perplexity_max_tokens(orders, corpus):
    gm, gt, om, ot = orders
    text = "".join(corpus[:10])
    _held_close(perplexity(gm, gt, text, 32, max_tokens=50), T.perplexity(om.call, ot, text.encode(), 32, 50))
    assert perplexity(gm, gt, "", 32).tokens == 0
    assert perplexity(gm, gt, "o", 32).tokens == 0
    assert perplexity(gm, gt, text, 0).tokens == 0


def test_perplexity_per_doc(orders, corpus):
    """eval.PerplexityPerDoc: the chat turns, separated by <EOS> and blank lines, each scored from <EOS>."""
    gm, gt, om, ot = orders
    docs = [c.replace("<EOS>", "") for c in corpus[:60]]
    text = "\n\n<EOS>\n\n".join(docs)
    want = T.perplexity_per_doc(om.call, ot, text.encode(), 16)
    _held_close(perplexity_per_doc(gm, gt, text, 16), want)
    want = T.perplexity_per_doc(om.call, ot, text.encode(), 16, max_docs=7)
    _held_close(perplexity_per_doc(gm, gt, text, 16, max_docs=7), want)


def test_score_sequences_edges(orders):
    """Per-target terms: empty and one-token sequences have no targets, an id outside the vocabulary is
    embedded as 0 and not scored as a target, and a context above max_context is cut to it."""
    gm, gt, om, _ = orders
    rng = np.random.default_rng(5)
    V = gm.vocab_size()
    seqs = [rng.integers(0, V, 300), np.zeros(0, np.int64), np.array([7]), rng.integers(0, V, 5),
            np.array([5, V + 3, 9, -2, 11])]
    for context in (0, 8, 200):
        got = score_sequences(gm, seqs, context)
        for s, g in zip(seqs, got):
            _terms_close(g, T.score(om.call, [int(x) for x in s], context))
    # the reference's window() panics on a negative context: an error here, not a silent NaN result
    from mignon_ai_amd import MignonError
    with pytest.raises(MignonError):
        score_sequences(gm, seqs, -1)


@pytest.mark.parametrize("case", list(EQUIV_CASES))
def test_score_sequences_architectures(case):
    """The reference's equivalence architectures (internal/quant/equivalence_test.go:34-49): long ragged
    sequences with windows shorter and longer than the sequences."""
    data = equiv_model_bytes(case)
    gm, om = Model(data), oracle_model(data)
    rng = np.random.default_rng(17)
    seqs = [rng.integers(0, 16, n) for n in (90, 3, 41, 130)]
    for context in (5, 40):
        for s, g in zip(seqs, score_sequences(gm, seqs, context)):
            _terms_close(g, T.score(om.call, [int(x) for x in s], context))
