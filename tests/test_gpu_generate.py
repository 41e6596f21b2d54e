"""The library's text layer on the GPU against the oracle's text path (oracle/text.py over the CPU oracle), on
the reference's trained order-search model (tests/golden/orders.mgn): the README's known answer, and every
reply to the 168 hand-written requests identical (tokens, text; probabilities within 1e-4), for one prompt
at a time and all prompts in one batch."""
import ctypes
import json
import os

import numpy as np
import pytest

from helpers import GOLDEN, oracle_model
from mignon_ai_amd._lib import check, lib, ptr
from mignon_ai_amd.generate import Generator
from oracle import text as T

pytestmark = pytest.mark.gpu

ORDERS = os.path.join(GOLDEN, "orders.mgn")
REQUEST = "unpaid electronics orders over $500 from last month"
ANSWER = "orders find --status unpaid --category electronics --min-amount 500 --when last-month"
MAX_REPLY_TOKENS = 80  # examples/order-search/orders.js:20
CONTEXT = 128
PROB_RTOL = 1e-4


@pytest.fixture(scope="module")
def data():
    with open(ORDERS, "rb") as f:
        return f.read()


@pytest.fixture(scope="module")
def gpu(data):
    return Generator.from_bytes(data)


@pytest.fixture(scope="module")
def ref(data):
    return oracle_model(data), T.Tokenizer.from_model_file(data)


@pytest.fixture(scope="module")
def requests_():
    with open(os.path.join(GOLDEN, "orders_handwritten.json")) as f:
        return [p["instruction"].strip() for p in json.load(f)]


def _check(got, ref, prompt, max_tokens=MAX_REPLY_TOKENS, chat=True):
    m, tok = ref
    text, ids, probs = T.generate(m, tok, prompt, CONTEXT, max_tokens, chat=chat)
    assert got.ids == ids, prompt
    assert got.text == text.decode(), prompt
    assert np.all(np.abs(np.array([p.prob for p in got.tokens]) - np.array(probs)) <= PROB_RTOL * np.array(probs))


def test_readme_answer_on_gpu(gpu):
    r = gpu.generate(REQUEST)
    assert r.text == ANSWER
    assert len(r.tokens) > 3 and 0 < r.min_prob <= 1
    assert "".join(p.text for p in r.tokens).strip() == r.text


def test_replies_match_oracle(gpu, ref, requests_):
    for q in requests_[::6]:
        _check(gpu.generate(q, MAX_REPLY_TOKENS), ref, q)


def test_batched_replies_match_oracle(gpu, ref, requests_):
    got = gpu.generate_batch(requests_, MAX_REPLY_TOKENS)
    assert len(got) == len(requests_)
    for q, g in zip(requests_, got):
        _check(g, ref, q)


def test_batches_of_one_size_in_a_row(gpu, ref, requests_):
    """The model keeps mg_generate_*'s session set for the next call of the same size: the second batch
    starts from cleared state, not from the first batch's."""
    a, b = requests_[:8], requests_[8:16][::-1]
    gpu.generate_batch(a, MAX_REPLY_TOKENS)
    for q, g in zip(b, gpu.generate_batch(b, MAX_REPLY_TOKENS)):
        _check(g, ref, q)


def test_max_tokens_and_empty_batch(gpu, ref):
    got = gpu.generate_batch(["unpaid orders", REQUEST], 2)
    assert all(len(r.tokens) <= 2 for r in got)
    for q, g in zip(["unpaid orders", REQUEST], got):
        _check(g, ref, q, max_tokens=2)
    assert gpu.generate_batch([]) == []
    assert len(gpu.generate("unpaid orders").tokens) <= 60  # infer.DefaultMaxTokens


def test_plain_continuation_and_empty_prompt(gpu, ref):
    """DecodeGreedy with Chat false continues the raw text; an empty plain prompt prefills nothing and gets
    no reply (greedy.go:43-49,66-67)."""
    prompts = [b"orders find --status", b"", b"unpaid"]
    n, K = len(prompts), 12
    arr = (ctypes.c_char_p * n)(*prompts)
    lens = (ctypes.c_size_t * n)(*[len(p) for p in prompts])
    ids = np.full((n, K), -7, np.int32)
    probs = np.zeros((n, K))
    counts = np.full(n, -1, np.int32)
    check(lib().mg_generate_greedy(gpu.model.handle, gpu.tok.handle, arr, lens, n, CONTEXT, K, 0, ptr(ids),
                                   ptr(probs), ptr(counts)))
    m, tok = ref
    for i, p in enumerate(prompts):
        _, want, _ = T.generate(m, tok, p, CONTEXT, K, chat=False)
        assert counts[i] == len(want) and ids[i, :counts[i]].tolist() == want
    assert counts[1] == 0
