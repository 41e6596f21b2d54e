"""The one-workgroup-per-session decode step (MG_STEP_FUSED, automatic for sets of up to 256 sessions)
against the layer-by-layer step (MG_STEP_LAYERED): logits, argmax and probabilities identical bit for bit
step after step (the same limb arithmetic, reductions, attention and head statistics), greedy decodes
identical, and sessions against the oracle. Models: c1 (no attention), c3 (4 heads of 32), c4 (8 heads
of 32, three blocks), and the reference's equivalence architectures (blocks without attention, windows
of 12, dilations 1 and 2)."""
import numpy as np
import pytest

from helpers import EQUIV_CASES, assert_close, equiv_model_bytes, model_bytes, oracle_model
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore_step():
    prev = engine_option("step_kernel", "auto")
    yield
    engine_option("step_kernel", prev)


def _steps(data, V, mode, S, P, n, seed):
    engine_option("step_kernel", mode)
    m = Model(data)
    ss = m.sessions(S)
    prompts = synth.token_ids(seed, "s1:p", (S, P), V)
    outs = [ss.prefill(prompts)]
    for k in range(n):
        outs.append(ss.step(synth.token_ids(seed, f"s1:{k}", (S,), V)))
    return outs


def _same(a, b):
    for k, (x, y) in enumerate(zip(a, b)):
        for u, v in zip(x, y):
            assert np.array_equal(u.view(np.uint8), v.view(np.uint8)), f"step {k}"


@pytest.mark.parametrize("cfg", ["c1", "c3", "c4"])
def test_fused_step_equals_layered(restore_step, cfg):
    spec = synth.CONFIGS[cfg]["spec"]
    data = model_bytes(cfg)
    a = _steps(data, spec.V, "layered", 5, 9, 12, 3)
    b = _steps(data, spec.V, "fused", 5, 9, 12, 3)
    _same(a, b)


@pytest.mark.parametrize("case", list(EQUIV_CASES))
def test_fused_step_equivalence_architectures(restore_step, case):
    """TestQuantSessionMatchesCall's sequence on the fused step, against the oracle's session and the
    layered step (internal/quant/session_test.go:18-52)."""
    data = equiv_model_bytes(case)
    om = oracle_model(data)
    toks = np.random.default_rng(19).integers(0, 16, 40).astype(np.int32)
    res = {}
    for mode in ("layered", "fused"):
        engine_option("step_kernel", mode)
        gs = Model(data).new_session(12)
        out = [gs.prefill(toks[:5])]
        out += [gs.append(t) for t in toks[5:]]
        res[mode] = out
    os_ = om.new_session(12)
    ref = [os_.prefill(toks[:5])] + [os_.append(t) for t in toks[5:]]
    for i, (x, y, r) in enumerate(zip(res["layered"], res["fused"], ref)):
        assert np.array_equal(x.view(np.uint64), y.view(np.uint64)), f"position {i}"
        assert_close(y, r, what=f"position {i}")


def test_fused_greedy_decode(restore_step):
    spec = synth.CONFIGS["c4"]["spec"]
    data = model_bytes("c4")
    prompts = synth.token_ids(7, "s1:greedy", (6, 32), spec.V)
    res = {}
    for mode in ("layered", "fused"):
        engine_option("step_kernel", mode)
        res[mode] = Model(data).sessions(6).decode_greedy(prompts, 40)
    assert np.array_equal(res["layered"][0], res["fused"][0])
    assert np.array_equal(res["layered"][1].view(np.uint64), res["fused"][1].view(np.uint64))
    rid, _ = oracle_model(data).greedy(prompts[:2], 40)
    assert np.array_equal(res["fused"][0][:2], rid)
