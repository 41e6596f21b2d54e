"""Greedy chat generation on the GPU engine against the CPU oracle, on the reference's trained
order-search model (tests/golden/orders.mgn): the README's known answer, and every reply to the 168
hand-written requests identical (tokens and text), one session at a time and as one batch of sessions."""
import json
import os

import numpy as np
import pytest

from helpers import GOLDEN, oracle_model
from mignon_ai_amd.generate import Generator

pytestmark = pytest.mark.gpu

ORDERS = os.path.join(GOLDEN, "orders.mgn")
REQUEST = "unpaid electronics orders over $500 from last month"
ANSWER = "orders find --status unpaid --category electronics --min-amount 500 --when last-month"
MAX_REPLY_TOKENS = 80  # examples/order-search/orders.js:20
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
    return Generator.from_bytes(data, provider=oracle_model(data))


@pytest.fixture(scope="module")
def requests_():
    with open(os.path.join(GOLDEN, "orders_handwritten.json")) as f:
        return [p["instruction"].strip() for p in json.load(f)]


def _same(a, b, what):
    assert a.text == b.text, f"{what}: {a.text!r} != {b.text!r}"
    assert [p.text for p in a.tokens] == [p.text for p in b.tokens], what
    pa = np.array([p.prob for p in a.tokens])
    pb = np.array([p.prob for p in b.tokens])
    assert np.all(np.abs(pa - pb) <= PROB_RTOL * pb), what


def test_readme_answer_on_gpu(gpu):
    r = gpu.generate(REQUEST)
    assert r.text == ANSWER
    assert len(r.tokens) > 3 and 0 < r.min_prob <= 1


def test_replies_match_oracle(gpu, ref, requests_):
    for q in requests_[::4]:
        _same(gpu.generate(q, MAX_REPLY_TOKENS), ref.generate(q, MAX_REPLY_TOKENS), q)


def test_batched_replies_match_oracle(gpu, ref, requests_):
    got = gpu.generate_batch(requests_, MAX_REPLY_TOKENS)
    assert len(got) == len(requests_)
    for q, g in zip(requests_, got):
        _same(g, ref.generate(q, MAX_REPLY_TOKENS), q)


def test_batched_max_tokens_and_empty(gpu):
    got = gpu.generate_batch(["unpaid orders", REQUEST], 2)
    assert all(len(r.tokens) <= 2 for r in got)
    assert gpu.generate_batch([]) == []
