"""Decode steps replayed from a captured HIP graph (MG_OPT_STEP_GRAPH) against the same steps launched one
kernel at a time: bitwise-identical logits, argmax and probabilities on every replay, with the program's own
eager work and synchronisations between replays, including work that reallocates the workspace (the graph
must be captured again) and a change of output buffers."""
import numpy as np
import pytest

from helpers import assert_close, equiv_model_bytes, model_bytes, oracle_model
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore_graph():
    prev = engine_option("step_graph", "auto")
    yield
    engine_option("step_graph", prev)


def _run(data, mode, prompts, steps, spec, interleave):
    engine_option("step_graph", mode)
    m = Model(data)
    S = prompts.shape[0]
    ss = m.sessions(S)
    ss.prefill(prompts)
    outs = []
    for k in range(steps.shape[0]):
        outs.append(ss.step(steps[k]))
        if interleave and k == 3:
            # eager work on the same model between replays: a batch larger than anything before, so the
            # workspace is reallocated and the step must be captured again
            m.forward_batch(synth.token_ids(5, "graph:batch", (64, 24), spec.V))
        if interleave and k == 6:
            ss.step(steps[k], logits=False)  # other output pointers: another capture, then back
    return outs


@pytest.mark.parametrize("cfg", ["c3", "c1"])
def test_graph_replays_equal_eager(restore_graph, cfg):
    data = model_bytes(cfg)
    spec = synth.CONFIGS[cfg]["spec"]
    prompts = synth.token_ids(3, f"graph:{cfg}", (6, 9), spec.V)
    steps = synth.token_ids(4, f"graph:{cfg}:steps", (10, 6), spec.V)
    eager = _run(data, "off", prompts, steps, spec, True)
    graph = _run(data, "on", prompts, steps, spec, True)
    for k, (a, b) in enumerate(zip(eager, graph)):
        for x, y in zip(a, b):
            assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"step {k}"


def test_graph_single_session_matches_oracle(restore_graph):
    """One session's Appends through the graph path (host pointers, the per-set pinned buffers) against
    the oracle, past the attention window."""
    engine_option("step_graph", "on")
    data = equiv_model_bytes("2blk attn window")
    gm, om = Model(data), oracle_model(data)
    toks = np.random.default_rng(21).integers(0, 16, 40).astype(np.int32)
    gs, os_ = gm.new_session(12), om.new_session(12)
    assert_close(gs.prefill(toks[:5]), os_.prefill(toks[:5]), what="prefill")
    for i in range(5, 40):
        assert_close(gs.append(toks[i]), os_.append(toks[i]), what=f"append {i}")


@pytest.mark.parametrize("cfg", ["c4", "c3"])
def test_graph_decodes_equal_eager(restore_graph, cfg):
    """Batched decodes (greedy, greedy with stop tokens, sampled) replay one captured step for every column
    (the column advances in device memory; the greedy decode replays eight steps per graph, then single
    steps for the rest): the same tokens, probabilities and reply lengths as launching each step kernel by
    kernel, with eager work on the model between the calls (a second greedy decode, of exactly two
    eight-step graphs, after the workspace was reallocated)."""
    data = model_bytes(cfg)
    spec = synth.CONFIGS[cfg]["spec"]
    prompts = synth.token_ids(11, f"graph-dec:{cfg}", (24, 7), spec.V)
    lens = (np.arange(24) % 7 + 1).astype(np.int32)
    res = {}
    for mode in ("off", "on"):
        engine_option("step_graph", mode)
        m = Model(data)
        ss = m.sessions(24)
        a = ss.decode_greedy(prompts, 30, lens)
        m.forward_batch(synth.token_ids(12, "graph-dec:batch", (40, 16), spec.V))
        stops = [int(x) for x in a[0][:3, 5]]  # tokens that do occur, so some replies stop early
        b = ss.decode_greedy_until(prompts, 30, stops, lens)
        c = ss.decode_sample(prompts, 30, list(range(24)), temperature=0.8, top_k=20, top_p=0.9, rep_penalty=1.1,
                             stops=stops, lens=lens)
        m.forward_batch(synth.token_ids(13, "graph-dec:batch2", (80, 16), spec.V))
        d = ss.decode_greedy(prompts, 17, lens)
        res[mode] = (a, b, c, d)
    (ea, eb, ec, ed), (ga, gb, gc, gd) = res["off"], res["on"]
    assert np.array_equal(ea[0], ga[0]) and np.array_equal(ea[1].view(np.uint64), ga[1].view(np.uint64))
    assert np.array_equal(ed[0], gd[0]) and np.array_equal(ed[1].view(np.uint64), gd[1].view(np.uint64))
    assert np.array_equal(eb[2], gb[2]) and (eb[2] < 30).any()
    for i in range(24):
        k = eb[2][i]
        assert np.array_equal(eb[0][i, :k], gb[0][i, :k])
        assert np.array_equal(eb[1][i, :k].view(np.uint64), gb[1][i, :k].view(np.uint64))
        assert np.array_equal(ec[0][i, :ec[1][i]], gc[0][i, :gc[1][i]])
    assert np.array_equal(ec[1], gc[1])
