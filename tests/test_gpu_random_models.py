"""Randomly drawn architectures through every path, against the oracle.

Each seed draws a model the reference could build: state size, hidden size, blocks with their rule steps
and dilations (a block may have none), attention heads of any width dividing the state, windowed or full
attention, vocabulary size, tied or untied head, context. Parameters are uniform like the reference's
equivalence models (internal/quant/equivalence_test.go:63-73), then quantised per tensor. Each model runs
(1) a teacher-forced batch (every position's logits) and (2) a set of streaming sessions: a ragged prefill
then single steps (internal/quant/session.go:11-68), once with each decode-step implementation that takes
the model (layer by layer, one workgroup per session, one per 16 sessions; the others fall back to the
layered step), each output checked against the oracle's Call / session at the 1e-4 bar. The sizes keep the oracle to a fraction of a second per model."""
import numpy as np
import pytest

from helpers import assert_close, oracle_model, uniform_model_bytes
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu

SEEDS = list(range(24))


def draw_spec(seed):
    rng = np.random.default_rng(1000 + seed)
    D = int(rng.choice([8, 12, 24, 40, 64, 72, 96, 128, 136]))
    H = int(rng.choice([D, 2 * D, D + 8, 3 * D // 2 + 4]))
    nblocks = int(rng.integers(1, 4))
    blocks = []
    for b in range(nblocks):
        steps = int(rng.integers(0 if nblocks > 1 else 1, 4))
        blocks.append((steps, int(rng.integers(1, 4)), int(rng.integers(1, 4))))
    if all(s == 0 for s, _, _ in blocks):
        blocks[0] = (1,) + blocks[0][1:]
    divisors = [h for h in range(1, 9) if D % h == 0]
    heads = int(rng.choice([0] + divisors))
    window = int(rng.choice([0, 3, 16, 64])) if heads else 0
    context = int(rng.choice([64, 128, 200]))
    V = int(rng.choice([16, 97, 300]))
    tied = bool(rng.integers(0, 2))
    return synth.ModelSpec(V=V, D=D, H=H, blocks=[synth.BlockSpec(*b) for b in blocks], heads=heads,
                           window=window, context=context, tied=tied)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_model_forward_and_sessions(seed):
    spec = draw_spec(seed)
    data = uniform_model_bytes(spec, seed=50 + seed, scale=0.4)
    gm, om = Model(data), oracle_model(data)
    rng = np.random.default_rng(seed)
    what = f"seed {seed}: {spec}"

    # teacher-forced batch: every position of every sequence, against Call on each prefix; with the
    # automatic kernel choice, then with the weight-stationary GEMM, the fused scan, the fused attention and
    # the fp32 operands forced (where the shapes take them), then the streaming GEMM, the separate scan, the
    # reference-order attention and limb-plane operands
    B, T = 3, int(rng.choice([7, 16, 33, 128]))
    ids = rng.integers(0, spec.V, (B, T)).astype(np.int32)
    ref = om.forward_all(ids)
    combos = [None, dict(gemm="slab", scan="fused", attention="fused", operands="fp32"),
              dict(gemm="stream", scan="separate", attention="exact", operands="limbs")]
    for combo in combos:
        prev = {k: engine_option(k) for k in ("gemm", "scan", "attention", "operands")}
        try:
            for k, v in (combo or {}).items():
                engine_option(k, v)
            got = gm.forward_batch(ids, logits=True)["logits"]
        finally:
            for k, v in prev.items():
                engine_option(k, v)
        assert_close(got, ref, what=f"forward {combo}, {what}")

    # sessions: ragged prefill, then steps
    S, ctx = 5, int(rng.choice([12, 40, spec.context]))
    P, G = 9, 6
    toks = rng.integers(0, spec.V, (S, P + G)).astype(np.int32)
    lens = rng.integers(1, P + 1, S).astype(np.int32)
    want = []
    osess = [om.new_session(ctx) for _ in range(S)]
    want.append([osess[i].prefill(toks[i, :lens[i]]) for i in range(S)])
    for t in range(P, P + G):
        want.append([osess[i].append(int(toks[i, t])) for i in range(S)])
    prev = engine_option("step_kernel")
    try:
        for mode in ("layered", "fused", "tiled"):
            engine_option("step_kernel", mode)
            ss = gm.sessions(S, ctx)
            lg, _, _ = ss.prefill(toks[:, :P], lens)
            for i in range(S):
                assert_close(lg[i], want[0][i], what=f"{mode} prefill {i}, {what}")
            for k, t in enumerate(range(P, P + G)):
                lg, _, _ = ss.step(toks[:, t])
                for i in range(S):
                    assert_close(lg[i], want[k + 1][i], what=f"{mode} step {t} session {i}, {what}")
    finally:
        engine_option("step_kernel", prev)
