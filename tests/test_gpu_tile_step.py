"""The tiled decode step (MG_STEP_TILED: 16 sessions per workgroup, one kernel per stretch between
attention blocks, decode attention between them; automatic for sets larger than the fused step takes)
against the layer-by-layer step (MG_STEP_LAYERED): logits, argmax and probabilities identical bit for bit
step after step, for sets that fill tiles exactly and sets that leave the last tile partial; greedy
decodes identical; sessions against the oracle. Models: c1 (no attention), c3 (4 heads of 32), c4 (8 heads
of 32, three blocks), the reference's trained orders.mgn (heads of 24) and the reference's equivalence
architectures (blocks without attention, windows of 12, dilations 1 and 2)."""
import os

import numpy as np
import pytest

from helpers import EQUIV_CASES, assert_close, equiv_model_bytes, model_bytes, oracle_model
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture
def restore_step():
    prev = engine_option("step_kernel", "auto")
    yield
    engine_option("step_kernel", prev)


def _steps(data, V, mode, S, P, n, seed, logits=True):
    engine_option("step_kernel", mode)
    m = Model(data)
    ss = m.sessions(S)
    prompts = synth.token_ids(seed, "ts:p", (S, P), V)
    outs = [ss.prefill(prompts, logits=logits)]
    for k in range(n):
        outs.append(ss.step(synth.token_ids(seed, f"ts:{k}", (S,), V), logits=logits))
    return outs


def _same(a, b):
    for k, (x, y) in enumerate(zip(a, b)):
        for u, v in zip(x, y):
            if u is None:
                assert v is None
                continue
            assert np.array_equal(u.view(np.uint8), v.view(np.uint8)), f"step {k}"


@pytest.mark.parametrize("cfg,S", [("c1", 21), ("c3", 16), ("c3", 37), ("c4", 5), ("c4", 48)])
def test_tiled_step_equals_layered(restore_step, cfg, S):
    spec = synth.CONFIGS[cfg]["spec"]
    data = model_bytes(cfg)
    a = _steps(data, spec.V, "layered", S, 9, 10, 3)
    b = _steps(data, spec.V, "tiled", S, 9, 10, 3)
    _same(a, b)


def test_tiled_step_without_logits(restore_step):
    spec = synth.CONFIGS["c3"]["spec"]
    data = model_bytes("c3")
    a = _steps(data, spec.V, "layered", 19, 7, 6, 5, logits=False)
    b = _steps(data, spec.V, "tiled", 19, 7, 6, 5, logits=False)
    _same(a, b)


def test_tiled_step_real_model(restore_step):
    """orders.mgn: state size 96, hidden 160, heads of width 24 (the fused step does not take them)."""
    with open(os.path.join(GOLDEN, "orders.mgn"), "rb") as f:
        data = f.read()
    a = _steps(data, 2048, "layered", 40, 12, 8, 9)
    b = _steps(data, 2048, "tiled", 40, 12, 8, 9)
    _same(a, b)


@pytest.mark.parametrize("case", list(EQUIV_CASES))
def test_tiled_step_equivalence_architectures(restore_step, case):
    """TestQuantSessionMatchesCall's sequence on the tiled step, against the oracle's session and the
    layered step (internal/quant/session_test.go:18-52)."""
    data = equiv_model_bytes(case)
    om = oracle_model(data)
    toks = np.random.default_rng(19).integers(0, 16, 40).astype(np.int32)
    res = {}
    for mode in ("layered", "tiled"):
        engine_option("step_kernel", mode)
        gs = Model(data).new_session(12)
        out = [gs.prefill(toks[:5])]
        out += [gs.append(t) for t in toks[5:]]
        res[mode] = out
    os_ = om.new_session(12)
    ref = [os_.prefill(toks[:5])] + [os_.append(t) for t in toks[5:]]
    for i, (x, y, r) in enumerate(zip(res["layered"], res["tiled"], ref)):
        assert np.array_equal(x.view(np.uint64), y.view(np.uint64)), f"position {i}"
        assert_close(y, r, what=f"position {i}")


def test_tiled_greedy_decode(restore_step):
    spec = synth.CONFIGS["c4"]["spec"]
    data = model_bytes("c4")
    prompts = synth.token_ids(7, "ts:greedy", (40, 32), spec.V)
    res = {}
    for mode in ("layered", "tiled"):
        engine_option("step_kernel", mode)
        res[mode] = Model(data).sessions(40).decode_greedy(prompts, 40)
    assert np.array_equal(res["layered"][0], res["tiled"][0])
    assert np.array_equal(res["layered"][1].view(np.uint64), res["tiled"][1].view(np.uint64))
    rid, _ = oracle_model(data).greedy(prompts[:2], 40)
    assert np.array_equal(res["tiled"][0][:2], rid)


def test_zero_step_block_all_step_kernels(restore_step):
    """A block with no rule steps (its input is the previous block's state plus the residual, then its
    attention): the layered, fused and tiled steps, bit for bit, against the oracle's session; the batched
    forward against the oracle's Call."""
    from helpers import tiny_spec, uniform_model_bytes
    spec = tiny_spec([(2, 2, 1), (0, 2, 1), (1, 2, 2)], heads=2, context=64)
    data = uniform_model_bytes(spec)
    om = oracle_model(data)
    toks = np.random.default_rng(23).integers(0, 16, 40).astype(np.int32)
    res = {}
    for mode in ("layered", "fused", "tiled"):
        engine_option("step_kernel", mode)
        gs = Model(data).new_session(12)
        out = [gs.prefill(toks[:5])]
        out += [gs.append(t) for t in toks[5:]]
        res[mode] = out
    os_ = om.new_session(12)
    ref = [os_.prefill(toks[:5])] + [os_.append(t) for t in toks[5:]]
    for i, r in enumerate(ref):
        assert np.array_equal(res["layered"][i].view(np.uint32), res["fused"][i].view(np.uint32)), f"fused {i}"
        assert np.array_equal(res["layered"][i].view(np.uint32), res["tiled"][i].view(np.uint32)), f"tiled {i}"
        assert_close(res["tiled"][i], r, what=f"position {i}")
    ids = toks[:24].reshape(2, 12)
    got = Model(data).call(ids[0])
    assert_close(got, om.call(ids[0]), what="call")
