"""Cancellation of batched decodes (mg_model_set_cancel): generate's Cancel hook, checked before each token
(internal/generate/greedy.go:68-70, internal/generate/sample.go:204-206; pkg/infer.Generate's context,
pkg/infer/infer.go:73-95). A flag set before the call gives empty replies; a flag set by another thread
while the decode runs cuts every reply at one column, and what was produced equals the uncancelled decode's
prefix."""
import ctypes
import os
import threading
import time

import numpy as np
import pytest

from helpers import GOLDEN, model_bytes
from mignon_ai_amd import Model, synth
from mignon_ai_amd.generate import Generator

pytestmark = pytest.mark.gpu


def test_cancel_before_start():
    data = model_bytes("c3")
    spec = synth.CONFIGS["c3"]["spec"]
    m = Model(data)
    flag = ctypes.c_int32(1)
    m.set_cancel(flag)
    prompts = synth.token_ids(61, "cancel:pre", (8, 6), spec.V)
    ids, probs, counts = m.sessions(8).decode_greedy_until(prompts, 20, [])
    assert not counts.any()
    ids, counts = m.sessions(8).decode_sample(prompts, 20, list(range(8)), temperature=0.8)
    assert not counts.any()
    flag.value = 0  # cleared: the next call runs to the end
    ids, probs, counts = m.sessions(8).decode_greedy_until(prompts, 20, [])
    assert (counts == 20).all()
    m.set_cancel(None)


def test_cancel_from_another_thread():
    """c1's model decoding 4000 tokens per session (a few hundred ms of launches); another thread sets the
    flag after 30 ms."""
    data = model_bytes("c1")
    spec = synth.CONFIGS["c1"]["spec"]
    m = Model(data)
    S, G = 16, 4000
    prompts = synth.token_ids(62, "cancel:mid", (S, 8), spec.V)
    full_ids, full_probs, full_counts = m.sessions(S).decode_greedy_until(prompts, G, [])
    assert (full_counts == G).all()
    flag = ctypes.c_int32(0)
    m.set_cancel(flag)
    out = {}

    def run():
        out["r"] = m.sessions(S).decode_greedy_until(prompts, G, [])

    th = threading.Thread(target=run)
    th.start()
    time.sleep(0.03)
    flag.value = 1
    th.join(timeout=120)
    assert not th.is_alive()
    ids, probs, counts = out["r"]
    k = int(counts[0])
    print(f"cancelled after {k} of {G} tokens")
    assert (counts == k).all() and k < G
    assert np.array_equal(ids[:, :k], full_ids[:, :k])
    assert np.array_equal(probs[:, :k], full_probs[:, :k])
    m.set_cancel(None)


def test_generate_cancelled_before_start():
    with open(os.path.join(GOLDEN, "orders.mgn"), "rb") as f:
        g = Generator.from_bytes(f.read())
    flag = ctypes.c_int32(1)
    g.model.set_cancel(flag)
    res = g.generate_batch(["unpaid orders", "refunds from last week"], 40)
    assert all(r.text == "" and not r.ids for r in res)
    res = g.generate_batch(["unpaid orders"], 40, temperature=0.7, seeds=[3])
    assert res[0].text == "" and not res[0].ids
    flag.value = 0
    assert g.generate_batch(["unpaid orders"], 40)[0].ids
    g.model.set_cancel(None)
