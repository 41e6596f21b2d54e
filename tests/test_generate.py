"""The oracle's text path (oracle/text.py over the CPU oracle model) on the reference's trained order-search
model: the reference's own known answers, which pin the restatement end to end (tokenizer, chat template,
greedy loop and the model), and the greedy loop's rules. The library is checked against this oracle on the
GPU (tests/test_gpu_generate.py).

Known answers (the model is the reference's examples/order-search/orders.mgn):
  - packages/mignon-web/README.md:9-10: "unpaid electronics orders over $500 from last month" ->
    "orders find --status unpaid --category electronics --min-amount 500 --when last-month";
  - packages/mignon-web/test/mignon.test.mjs:17-22 (reply shape, probabilities) and :40-44 (maxTokens);
  - research/FINDINGS.md:23: the 168 hand-written requests of examples/order-search/handwritten.json
    (tests/golden/orders_handwritten.json) are answered at 96-99% (the page's customer-name correction
    included; here replies are compared as the model writes them, case-insensitively as check.js does).
"""
import json
import os

import pytest

from helpers import GOLDEN, oracle_model
from oracle import text as T

ORDERS = os.path.join(GOLDEN, "orders.mgn")
REQUEST = "unpaid electronics orders over $500 from last month"
ANSWER = b"orders find --status unpaid --category electronics --min-amount 500 --when last-month"
MAX_REPLY_TOKENS = 80  # examples/order-search/orders.js:20
CONTEXT = 128          # the file's metadata context_size


@pytest.fixture(scope="module")
def orders():
    with open(ORDERS, "rb") as f:
        data = f.read()
    return oracle_model(data), T.Tokenizer.from_model_file(data), T.read_header(data)["metadata"]


def handwritten():
    with open(os.path.join(GOLDEN, "orders_handwritten.json")) as f:
        return json.load(f)


def test_metadata(orders):
    _, _, meta = orders
    assert meta["task"] == "chat" and meta["context_size"] == CONTEXT


def test_readme_answer(orders):
    m, tok, _ = orders
    text, ids, probs = T.generate(m, tok, REQUEST, CONTEXT)
    assert text == ANSWER
    # mignon.test.mjs:19-22
    assert text.startswith(b"orders find ")
    assert b"--status unpaid" in text and b"--min-amount 500" in text
    assert len(ids) > 3 and 0 < min(probs) <= 1
    assert b"".join(tok.decode([i]) for i in ids).strip() == text


def test_max_tokens_limits_reply(orders):
    m, tok, _ = orders
    assert len(T.generate(m, tok, "unpaid orders", CONTEXT, 2)[1]) <= 2
    assert T.generate(m, tok, "unpaid orders", CONTEXT)[0].startswith(b"orders find ")


def test_handwritten_requests(orders):
    m, tok, _ = orders
    pairs = handwritten()
    ok = sum(T.generate(m, tok, p["instruction"].strip(), CONTEXT, MAX_REPLY_TOKENS)[0].decode().lower()
             == p["output"].lower() for p in pairs)
    assert ok / len(pairs) >= 0.96, f"{ok}/{len(pairs)}"


def test_replies_are_canonical_encodings(orders):
    """The model was trained on text encoded by the reference's tokenizer, so the tokens it emits for a
    reply are the reference encoding of that reply: the restated encoder gives back the same ids."""
    m, tok, _ = orders
    for p in handwritten()[:60]:
        _, ids, _ = T.generate(m, tok, p["instruction"].strip(), CONTEXT, MAX_REPLY_TOKENS)
        assert tok.encode(tok.decode(ids)) == ids


class _Scripted:
    """A session whose logits name the next token: script[i] is the argmax after i generated tokens."""

    def __init__(self, script, V=8):
        self.script, self.V, self.appended = script, V, []

    def _logits(self):
        lg = [0.0] * self.V
        k = len(self.appended)
        if k < len(self.script):
            lg[self.script[k]] = 5.0
        return lg

    def prefill(self, ids):
        return self._logits() if ids else None

    def append(self, t):
        self.appended.append(t)
        return self._logits()


def test_greedy_loop_rules():
    """greedyLoop (internal/generate/greedy.go:63-87): stop before a stop token, no Append after the last
    token, nothing from an empty prefill."""
    s = _Scripted([5, 6, 4, 7])
    ids, probs = T.greedy_loop(s, [1, 2], 10, stops=(4,))
    assert ids == [5, 6] and s.appended == [5, 6] and len(probs) == 2
    s = _Scripted([5, 6, 7])
    ids, _ = T.greedy_loop(s, [1], 2, stops=(4,))
    assert ids == [5, 6] and s.appended == [5]
    assert T.greedy_loop(_Scripted([5]), [], 5) == ([], [])


def test_argmax_prob():
    """argmaxProb (greedy.go:89-102): the first maximum; probability 1/sum exp(l - max)."""
    assert T.argmax_prob([0.0, 3.0, 3.0, 1.0])[0] == 1
    b, p = T.argmax_prob([0.0, 0.0])
    assert b == 0 and p == pytest.approx(0.5)
    assert T.argmax_prob([2.0]) == (0, 1.0)


def test_perplexity_closed_forms():
    """nll.score / result / BitsPerByte (internal/eval/eval.go:27-50, internal/tokenizer/bytes.go:5-11) on a
    model whose logits are uniform over V = 5 tokens: every target costs ln 5 nats, so loss = ln 5,
    PPL = 5 and BPB = ln 5 * tokens / (ln 2 * bytes)."""
    import math
    tok = T.Tokenizer(["<PAD>", "<UNK>", "<EOS>", "ab", "c"], [("a", "b")])

    def call(ids):
        return [0.0] * 5
    r = T.perplexity(call, tok, b"abcab", context=2)
    # tokens ab c ab: 2 targets (c, ab) of 1 + 2 bytes
    assert r["tokens"] == 2
    assert r["loss"] == pytest.approx(math.log(5))
    assert r["ppl"] == pytest.approx(5)
    assert r["bpb"] == pytest.approx(2 * math.log(5) / (math.log(2) * 3))
    assert T.perplexity(call, tok, b"abcab", context=2, max_tokens=1)["tokens"] == 1
    assert T.perplexity(call, tok, b"ab", context=2)["tokens"] == 0      # fewer than 2 tokens
    assert T.perplexity(call, tok, b"abcab", context=0)["tokens"] == 0   # empty windows score nothing
    # documents: split on <EOS>, one blank line stripped each side, each scored from a fresh <EOS>
    assert T.split_docs(b"\n\nab\n\n<EOS>\n\n<EOS>c") == [b"ab", b"c"]
    d = T.perplexity_per_doc(call, tok, b"ab<EOS>c<EOS>", context=4)
    assert d["tokens"] == 2
    assert T.perplexity_per_doc(call, tok, b"ab<EOS>c<EOS>", context=4, max_docs=1)["tokens"] == 1


def test_score_windows(orders):
    """window(tokens[:t], context) (internal/eval/suite.go:196-198): target t is scored from the last
    `context` tokens before it, as a fresh Call."""
    m, tok, _ = orders
    ids = tok.encode("orders find --status unpaid --when last-month")
    terms = T.score(m.call, ids, 4)
    for t in (1, 3, len(ids) - 1):
        want = T.log_prob(m.call(ids[max(0, t - 4):t]), ids[t])
        assert terms[t - 1] == want


def test_result_fields_from_batch_matrices():
    """generate.Result over a batch's id and probability matrices (the library's batched replies): its
    ids and probs are the row's first n entries, built once and kept, so edits persist and assignment
    replaces them; once both are read the reply no longer refers to the matrices."""
    import numpy as np
    from mignon_ai_amd.generate import Result
    ids = np.arange(12, dtype=np.int32).reshape(3, 4)
    probs = np.linspace(0.1, 0.9, 12).reshape(3, 4)
    r = Result("x", ids, probs, ["t%d" % i for i in range(12)], row=1, n=3)
    assert r.ids == [4, 5, 6] and r.probs == pytest.approx(list(probs[1, :3]))
    r.ids.append(7)
    assert r.ids == [4, 5, 6, 7]
    r.probs = [0.5]
    assert r.probs == [0.5] and r.min_prob == 0.5
    assert not isinstance(r._ids, np.ndarray) and not isinstance(r._probs, np.ndarray)
    assert [p.text for p in Result("y", ids, probs, ["t%d" % i for i in range(12)], row=0, n=2).tokens] == ["t0", "t1"]
