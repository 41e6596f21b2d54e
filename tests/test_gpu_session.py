"""Streaming sessions and batched greedy decode through the C ABI."""
import numpy as np
import pytest

from helpers import EQUIV_CASES, assert_close, equiv_model_bytes, model_bytes, oracle_model
from mignon_ai_amd import MignonError, Model, synth

pytestmark = pytest.mark.gpu

WINDOW, TOKENS, PREFILL = 12, 40, 5  # internal/quant/session_test.go:9-13


@pytest.mark.parametrize("case", list(EQUIV_CASES))
def test_session_matches_oracle(case):
    """TestQuantSessionMatchesCall's sequence (internal/quant/session_test.go:18-52) on the GPU engine,
    each output checked against the oracle's session."""
    data = equiv_model_bytes(case)
    gm = Model(data)
    om = oracle_model(data)
    rng = np.random.default_rng(9)
    toks = rng.integers(0, 16, TOKENS).astype(np.int32)
    gs = gm.new_session(WINDOW)
    os_ = om.new_session(WINDOW)
    assert_close(gs.prefill(toks[:PREFILL]), os_.prefill(toks[:PREFILL]), what="prefill")
    for i in range(PREFILL, TOKENS):
        assert_close(gs.append(toks[i]), os_.append(toks[i]), what=f"append {i}")
    long = toks[:2 * WINDOW]
    assert_close(gs.prefill(long), os_.prefill(long), what="long prefill")
    assert gs.state_bytes() == os_.state_bytes()


def test_batched_sessions_match_forward():
    """Session Prefill + Append per position equals the teacher-forced batch (both on the GPU)."""
    data = model_bytes("c3")
    spec = synth.CONFIGS["c3"]["spec"]
    gm = Model(data)
    S, P, G = 16, 8, 24
    ids = synth.token_ids(4, "c3:sess", (S, P + G), spec.V)
    full = gm.forward_batch(ids)["logits"]
    ss = gm.sessions(S)
    lg, am, pb = ss.prefill(ids[:, :P])
    assert_close(lg, full[:, P - 1], what="prefill")
    assert np.array_equal(am, lg.argmax(-1))
    for t in range(P, P + G):
        lg, am, pb = ss.step(ids[:, t])
        assert_close(lg, full[:, t], what=f"step {t}")


def test_ragged_prefill():
    data = model_bytes("c3")
    spec = synth.CONFIGS["c3"]["spec"]
    gm = Model(data)
    om = oracle_model(data)
    lens = np.array([1, 5, 32, 17], np.int32)
    ids = synth.token_ids(5, "c3:ragged", (4, 32), spec.V)
    ss = gm.sessions(4)
    lg, am, pb = ss.prefill(ids, lens)
    for i, L in enumerate(lens):
        assert_close(lg[i], om.call(ids[i, :L]), what=f"session {i}")
    nxt = synth.token_ids(6, "c3:ragged2", (4,), spec.V)
    lg2, _, _ = ss.step(nxt)
    for i, L in enumerate(lens):
        assert_close(lg2[i], om.call(np.concatenate([ids[i, :L], nxt[i:i + 1]])), what=f"session {i} step")


def test_greedy_decode_matches_oracle():
    """Config-4 shape, a subset of sessions: greedy tokens identical to the oracle's greedyLoop."""
    data = model_bytes("c4")
    spec = synth.CONFIGS["c4"]["spec"]
    gm = Model(data)
    om = oracle_model(data)
    S, P, G = 8, 32, 64
    prompts = synth.token_ids(3, "c4:prompts", (S, P), spec.V)
    ss = gm.sessions(S)
    ids, probs = ss.decode_greedy(prompts, G)
    rid, rprob = om.greedy(prompts, G)
    assert np.array_equal(ids, rid)
    assert np.allclose(probs, rprob, rtol=1e-4)


def _first_stop(row, stops, G):
    for k, t in enumerate(row):
        if int(t) in stops:
            return k
    return G


def test_greedy_until_stops():
    """greedyLoop with stop tokens (internal/generate/greedy.go:63-87) on device sessions: each reply is the
    stop-free greedy decode cut before its first stop token, with the same probabilities, whether sessions
    stop early, at the first token, or never (the loop ends once every session has stopped)."""
    data = model_bytes("c3")
    spec = synth.CONFIGS["c3"]["spec"]
    gm = Model(data)
    S, P, G = 64, 12, 40
    prompts = synth.token_ids(8, "until:prompts", (S, P), spec.V)
    lens = np.random.default_rng(2).integers(1, P + 1, S).astype(np.int32)
    full_ids, full_probs = gm.sessions(S).decode_greedy(prompts, G, lens)
    vals, freq = np.unique(full_ids, return_counts=True)
    frequent = [int(v) for v in vals[np.argsort(-freq)][:3]]
    v0, f0 = np.unique(full_ids[:, 0], return_counts=True)
    first = [int(v) for v in v0[np.argsort(-f0)][:8]]
    cases = [frequent, first, [], [spec.V + 5]]
    for stops in cases:
        ids, probs, counts = gm.sessions(S).decode_greedy_until(prompts, G, stops, lens)
        for i in range(S):
            k = _first_stop(full_ids[i], set(stops), G)
            assert counts[i] == k, (stops, i)
            assert np.array_equal(ids[i, :k], full_ids[i, :k])
            assert np.array_equal(probs[i, :k], full_probs[i, :k])
    # every session stops at its first token: all counts 0
    same = np.repeat(prompts[:1], S, axis=0)
    one = np.full(S, lens[0], np.int32)
    _, _, counts = gm.sessions(S).decode_greedy_until(same, G, [int(full_ids[0, 0])], one)
    assert not counts.any()
    with pytest.raises(MignonError):
        gm.sessions(S).decode_greedy_until(prompts, G, list(range(9)), lens)


@pytest.mark.parametrize("D,heads,context,window", [(32, 2, 256, 0), (128, 2, 256, 0), (64, 1, 64, 0),
                                                    (40, 2, 128, 30)])
def test_decode_attention_kernels(D, heads, context, window):
    """Streamed steps through each decode-attention kernel equal the teacher-forced batch: caches of more
    than 64 positions with keys and values staged in LDS (head width 16), one lane per key where that
    staging would not fit (head width 64, cache 256), and caches of at most 64 positions with key rows in
    registers (head widths 64 and 20, the last with a window of 30 inside a 128-token context); the last
    step also against the oracle."""
    from helpers import tiny_spec, uniform_model_bytes
    spec = tiny_spec([(1, 2, 1), (1, 2, 1)], V=64, D=D, H=32, heads=heads, window=window, context=context)
    data = uniform_model_bytes(spec, scale=0.3)
    gm = Model(data)
    S = 6
    T = min(100, context)
    P = T // 3
    ids = synth.token_ids(12, f"dec-attn{D}-{heads}-{context}-{window}", (S, T), spec.V)
    full = gm.forward_batch(ids)["logits"]
    ss = gm.sessions(S)
    lg, _, _ = ss.prefill(ids[:, :P])
    assert_close(lg, full[:, P - 1], what="prefill")
    for t in range(P, T):
        lg, _, _ = ss.step(ids[:, t])
        assert_close(lg, full[:, t], what=f"step {t}")
    assert_close(lg[:2], oracle_model(data).forward_all(ids[:2])[:, -1], what="oracle, last step")
