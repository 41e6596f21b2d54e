"""The head GEMMs' integer join of the two lower digit-plane sums (254 p1 + p2 in one 24-bit multiply-add,
for K <= 512) at its bound and just past it. Decode steps of a model of state width 512 (K = 512, the
widest the single-kernel step takes) and of width 320 (the widest the tiled step takes) are bit-identical
between the layer-by-layer step and those kernels, and its sessions match the oracle. The batched forward
at widths 512 and 576 (K = 576: the three-term join) is bit-identical between the streaming and
weight-stationary GEMM kernels and matches the oracle."""
import numpy as np
import pytest

from helpers import assert_close, oracle_model, tiny_spec, uniform_model_bytes
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore():
    # both GEMM kernels on limb-plane operands (the fp32-operand GEMM is weight-stationary only)
    prev = {k: engine_option(k) for k in ("step_kernel", "gemm", "operands")}
    engine_option("operands", "limbs")
    yield
    for k, v in prev.items():
        engine_option(k, v)


def _model(D, heads=8):
    spec = tiny_spec([(1, 2, 1), (1, 2, 2)], heads=heads, window=16, V=300, D=D, H=D, context=64, tied=False)
    return spec, uniform_model_bytes(spec, scale=0.3)


def _same(a, b, what):
    for k, (x, y) in enumerate(zip(a, b)):
        for u, v in zip(x, y):
            assert np.array_equal(u.view(np.uint8), v.view(np.uint8)), f"{what}: step {k}"


# (state width, heads, step kernels): 512 is the widest the single-kernel step takes, 320 the widest the
# tiled step's LDS takes
@pytest.mark.parametrize("D,heads,modes", [(512, 8, ("fused",)), (320, 5, ("fused", "tiled"))])
def test_k512_decode_steps(restore, D, heads, modes):
    spec, data = _model(D, heads)
    prompts = synth.token_ids(61, f"k512:p{D}", (5, 9), spec.V)
    steps = synth.token_ids(62, f"k512:s{D}", (8, 5), spec.V)
    kernels = {"fused": "session_step", "tiled": "tile_step"}
    res = {}
    for mode in ("layered",) + modes:
        engine_option("step_kernel", mode)
        m = Model(data)
        ss = m.sessions(5)
        res[mode] = [ss.prefill(prompts)]
        m.profile(True)
        res[mode] += [ss.step(steps[k]) for k in range(8)]
        m.profile(False)
        if mode in kernels:
            n = m.profile_read().get(kernels[mode], (0,))[0]
            assert n > 0 and n % 8 == 0, f"{mode}: {n} launches of {kernels[mode]} in 8 steps"
    for mode in modes:
        _same(res["layered"], res[mode], f"layered vs {mode} step")
    om = oracle_model(data)
    for i in (0, 4):
        seq = np.concatenate([prompts[i], steps[:, i]])
        assert_close(res[modes[0]][-1][0][i], om.call(seq), what=f"session {i} vs oracle")


@pytest.mark.parametrize("D", [512, 576])
def test_k512_batched_forward(restore, D):
    spec, data = _model(D)
    ids = synth.token_ids(63, f"k512:f{D}", (3, 40), spec.V)
    out = {}
    for mode in ("stream", "slab"):
        engine_option("gemm", mode)
        out[mode] = Model(data).forward_batch(ids, logits=True, probs=True, logprob=True)
    for k in out["stream"]:
        assert np.array_equal(out["stream"][k].view(np.uint32), out["slab"][k].view(np.uint32)), k
    assert_close(out["slab"]["logits"], oracle_model(data).forward_all(ids), what=f"D{D} forward vs oracle")
