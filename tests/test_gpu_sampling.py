"""The library's device sampler against the oracle's restatement of the reference sampler
(oracle/text.py; internal/generate/sample.go:31-247): the same token for the same logits and draw, row by
row (mg_sample_logits); every token of a sampled batched decode equal to what the restatement picks from
the engine's own logits at each step (mg_sessions_decode_sample); and sampled chat on the reference's
trained orders.mgn equal to the oracle's end to end (mg_generate_sample)."""
import json
import os

import numpy as np
import pytest

from helpers import GOLDEN, model_bytes, oracle_model
from mignon_ai_amd import MignonError, Model, sample_logits, synth
from mignon_ai_amd.generate import Generator
from oracle import text as T

pytestmark = pytest.mark.gpu

PARAMS = [  # temperature, top_k, top_p, rep_penalty
    (0.0, 0, 1.0, 1.0), (0.0, 0, 1.0, 1.3), (0.7, 0, 1.0, 1.0), (1.0, 0, 1.0, 1.2), (1.3, 40, 1.0, 1.0),
    (0.8, 0, 0.9, 1.0), (0.7, 40, 0.9, 1.2), (1.0, 1, 1.0, 1.0), (2.0, 0, 0.5, 1.5), (1.0, 5000, 0.999, 1.0),
]


# vocabulary sizes across every exponentials-kernel instantiation (4 values per thread up to 1024, 8 up to
# 2048, 16 up to 4096, 32 above), uneven sizes inside each
@pytest.mark.parametrize("V", [4, 300, 301, 1500, 2048, 3000, 4096, 8192])
def test_sampler_matches_oracle(V):
    rng = np.random.default_rng(V)
    n = 24
    logits = rng.normal(0, 3, (n, V))
    logits[:, :2] = logits[:, 2:4]                 # exact ties in probability
    logits[3, :] = 1.0                            # a flat row
    if V >= 1024:
        # a first batch of equal values that all pass the first threshold and are dropped again once
        # later batches raise it (the truncated draw's mid-row refilter)
        logits[5, :512] = -5.0
    recent = [list(rng.integers(-2, V + 2, rng.integers(0, 7))) for _ in range(n)]
    u = rng.random(n)
    for temp, k, p, rp in PARAMS:
        got = sample_logits(logits, recent, temp, k, p, rp, u)
        want = [T.sample_raw_logits(logits[i], [int(x) for x in recent[i]], temp, rp, k, p, u[i]) for i in range(n)]
        assert got.tolist() == want, (temp, k, p, rp)


def test_sampler_rejects_large_vocabulary():
    with pytest.raises(MignonError):
        sample_logits(np.zeros((1, 8193)), None, 1.0, 0, 1.0, 1.0, np.zeros(1))


def _replay(gm, prompts, lens, G, seeds, temp, k, p, rp, penalize, stops):
    """sampleContinuation per session, stepping the engine's sessions one token at a time and choosing each
    token with the restated sampler from the engine's logits."""
    S = len(prompts)
    ss = gm.sessions(S)
    lg, _, _ = ss.prefill(prompts, lens)
    gen = [[] for _ in range(S)]
    done = [False] * S
    for step in range(G):
        nxt = np.zeros(S, np.int32)
        for i in range(S):
            row = [float(x) for x in lg[i]]
            g = gen[i]
            if len(g) >= 2:
                for j in range(len(g) - 2):
                    if g[j] == g[-2] and g[j + 1] == g[-1]:
                        row[g[j + 2]] = -1.7976931348623157e308
            recent = (list(prompts[i, :lens[i]]) if penalize else []) + g
            t = T.sample_raw_logits(row, [int(x) for x in recent[-6:]], temp, rp, k, p, T.uniform_draw(seeds[i], step))
            nxt[i] = t
            if not done[i]:
                if t in stops:
                    done[i] = True
                else:
                    g.append(t)
        if all(done) or step == G - 1:
            break
        lg, _, _ = ss.step(nxt)
    return gen


@pytest.mark.parametrize("cfg,params", [("c3", (1.0, 0, 1.0, 1.2, False)), ("c3", (0.8, 40, 0.9, 1.3, True)),
                                        ("c3", (0.0, 0, 1.0, 1.5, True)), ("c4", (0.7, 40, 0.9, 1.2, False))])
def test_decode_sample_matches_replay(cfg, params):
    """c4: the benchmarked sampled workload's shape (V 4096) and parameters."""
    temp, k, p, rp, penalize = params
    data = model_bytes(cfg)
    spec = synth.CONFIGS[cfg]["spec"]
    gm = Model(data)
    S, P, G = 12, 10, 24
    prompts = synth.token_ids(5, "sample:prompts", (S, P), spec.V)
    lens = np.random.default_rng(4).integers(1, P + 1, S).astype(np.int32)
    seeds = [1000 + 7 * i for i in range(S)]
    stops = [int(prompts[0, 0]), int(prompts[1, 0])]
    ids, counts = gm.sessions(S).decode_sample(prompts, G, seeds, temp, k, p, rp, penalize, stops, lens)
    want = _replay(gm, prompts, lens, G, seeds, temp, k, p, rp, penalize, set(stops))
    for i in range(S):
        assert ids[i, :counts[i]].tolist() == want[i], i


def test_sampled_chat_matches_oracle():
    with open(os.path.join(GOLDEN, "orders.mgn"), "rb") as f:
        data = f.read()
    with open(os.path.join(GOLDEN, "orders_handwritten.json")) as f:
        requests = [p["instruction"] for p in json.load(f)][:48]
    g = Generator.from_bytes(data)
    om, ot = oracle_model(data), T.Tokenizer.from_model_file(data)
    seeds = [31 * i + 5 for i in range(len(requests))]
    for temp, k, p, rp in [(0.7, 40, 0.9, 1.2), (1.5, 0, 0.0, 0.0)]:
        got = g.generate_batch(requests + ["   "], 80, temp, k, p, rp, seeds + [1])
        for q, s, r in zip(requests, seeds, got):
            text, ids = T.generate_sample(om, ot, q, 128, 80, temp, k, p if p > 0 else 1.0, rp, s)
            assert r.ids == ids and r.text == text, q
            assert r.tokens == [] or all(isinstance(t.prob, float) for t in r.tokens)
        assert got[-1].text == "" and got[-1].ids == []   # a blank chat prompt gets no reply
    # the same seed gives the same reply; a plain-text model path continues the raw prompt
    a = g.generate("unpaid orders", 40, 1.0, seed=9)
    b = g.generate("unpaid orders", 40, 1.0, seed=9)
    assert a.ids == b.ids
