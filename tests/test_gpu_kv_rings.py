"""Session K/V ring formats (MG_OPT_KV_RINGS): packed rings (24-bit mantissas with a power-of-two scale
per head row, automatic where the fused decode attention takes the model) against fp32 rings, on the same
model and prompts: logits within the parity bar of each other and of the oracle, greedy tokens identical;
the layered, fused and tiled steps bit-identical to each other under either format; the set's device
bytes. Models: c3 (4 heads of 32), c4 (8 heads of 32, three blocks) and the reference's trained orders.mgn
(heads of 24)."""
import os

import numpy as np
import pytest

from helpers import assert_close, model_bytes, oracle_model
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture
def restore():
    prev = engine_option("kv_rings", "auto"), engine_option("step_kernel", "auto")
    yield
    engine_option("kv_rings", prev[0])
    engine_option("step_kernel", prev[1])


def _steps(data, V, rings, mode, S, P, n, seed):
    engine_option("kv_rings", rings)
    engine_option("step_kernel", mode)
    m = Model(data)
    ss = m.sessions(S)
    prompts = synth.token_ids(seed, "kv:p", (S, P), V)
    outs = [ss.prefill(prompts)]
    for k in range(n):
        outs.append(ss.step(synth.token_ids(seed, f"kv:{k}", (S,), V)))
    return outs, ss.device_bytes(), prompts


def _model(cfg):
    if cfg == "orders":
        with open(os.path.join(GOLDEN, "orders.mgn"), "rb") as f:
            return f.read(), None
    return model_bytes(cfg), synth.CONFIGS[cfg]["spec"].V


@pytest.mark.parametrize("cfg,S", [("c3", 37), ("c4", 48), ("orders", 20)])
def test_packed_against_fp32_rings(restore, cfg, S):
    data, V = _model(cfg)
    if V is None:
        V = Model(data).vocab_size()
    P, n = 40, 30  # past the 64-slot cache, so the rings wrap
    fp, b32, prompts = _steps(data, V, "fp32", "auto", S, P, n, 9)
    pk, bpk, _ = _steps(data, V, "packed", "auto", S, P, n, 9)
    assert bpk < b32
    for k, (x, y) in enumerate(zip(fp, pk)):
        assert_close(y[0], x[0], what=f"step {k} logits")
        assert np.array_equal(np.argmax(y[0], -1), np.argmax(x[0], -1)), f"step {k} argmax"
    # against the oracle: one session's whole history through Call
    ids = np.concatenate([prompts[0], [synth.token_ids(9, f"kv:{k}", (S,), V)[0] for k in range(n)]])
    om = oracle_model(data)
    assert_close(pk[-1][0][0], om.call(ids), what="last step vs oracle")


@pytest.mark.parametrize("rings", ["fp32", "packed"])
@pytest.mark.parametrize("cfg,S", [("c3", 21), ("c4", 40)])
def test_step_kernels_identical_under_either_format(restore, rings, cfg, S):
    data, V = _model(cfg)
    runs = {mode: _steps(data, V, rings, mode, S, 9, 12, 4)[0] for mode in ("layered", "fused", "tiled")}
    for mode in ("fused", "tiled"):
        for k, (x, y) in enumerate(zip(runs["layered"], runs[mode])):
            for u, v in zip(x, y):
                if u is not None:
                    assert np.array_equal(u.view(np.uint8), v.view(np.uint8)), f"{mode} step {k}"
