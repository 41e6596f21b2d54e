"""The two limb-expanded GEMM kernels (streaming and weight-stationary) accumulate the same exact int32
sums and share one epilogue, so every model output must be bit-identical between them (with every operand
as limb planes); both are also checked against the oracle. Covers ragged token counts (not multiples of 16 or 128), a single token,
K of 2..18 K steps, every epilogue (latch, GLU, highway, QKV, residual, logits, probabilities) and an
odd vocabulary."""
import numpy as np
import pytest

from helpers import GOLDEN, assert_close, model_bytes, oracle_model, tiny_spec, uniform_model_bytes
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore_selection():
    # both kernels on limb-plane operands: the fp32-operand GEMM (weight-stationary only) has tests of its own
    prev = engine_option("gemm", "auto")
    prev_ops = engine_option("operands", "limbs")
    yield
    engine_option("gemm", prev)
    engine_option("operands", prev_ops)


def _both(m, ids, **kw):
    engine_option("gemm", "stream")
    a = m.forward_batch(ids, **kw)
    engine_option("gemm", "slab")
    b = m.forward_batch(ids, **kw)
    return a, b


def _same(a, b):
    for k in a:
        assert np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)), k


@pytest.mark.parametrize("shape", [(1, 1), (3, 37), (5, 130), (2, 300)])
def test_kernels_identical_c1(restore_selection, shape):
    data = model_bytes("c1")
    m = Model(data)
    ids = synth.token_ids(21, f"kern{shape}", shape, 512)
    a, b = _both(m, ids, logits=True, logprob=True, bits=True)
    _same(a, b)
    assert_close(b["logits"], oracle_model(data).forward_all(ids), what=f"c1 slab {shape}")


def test_kernels_identical_real_model(restore_selection):
    with open(f"{GOLDEN}/orders.mgn", "rb") as f:
        data = f.read()
    m = Model(data)
    ids = synth.token_ids(22, "kern-orders", (3, 129), 2048)
    a, b = _both(m, ids, logits=True, probs=True)
    _same(a, b)
    assert_close(b["logits"], oracle_model(data).forward_all(ids), what="orders.mgn slab")


def test_kernels_identical_untied_odd_vocab(restore_selection):
    spec = tiny_spec([(2, 2, 1), (1, 2, 2)], V=130, D=48, H=40, heads=3, window=7, tied=False)
    data = uniform_model_bytes(spec, scale=0.3)
    m = Model(data)
    ids = synth.token_ids(23, "kern-untied", (4, 45), 130)
    a, b = _both(m, ids, logits=True, logprob=True)
    _same(a, b)
    assert_close(b["logits"], oracle_model(data).forward_all(ids), what="untied slab")


def test_kernels_identical_c3_batch(restore_selection):
    """A batch large enough for several slab runs per channel slab."""
    data = model_bytes("c3")
    m = Model(data)
    ids = synth.token_ids(24, "kern-c3", (96, 128), 2048)
    a, b = _both(m, ids, logits=True, logprob=True, bits=True)
    _same(a, b)
    sub = [0, 95]
    assert_close(b["logits"][sub], oracle_model(data).forward_all(ids[sub]), what="c3 slab")


def test_kernels_identical_c5_shape(restore_selection):
    """c5's widths: the GLU GEMM's 18 K steps (K 1152), the highway's 16 (K 1024), the 6-step latch, QKV,
    out, logits and probabilities GEMMs, and a vocabulary of 64 channel slabs."""
    data = model_bytes("c5")
    m = Model(data)
    ids = synth.token_ids(26, "kern-c5", (3, 128), 8192)
    a, b = _both(m, ids, logits=True, logprob=True, probs=True, bits=True)
    _same(a, b)
    assert_close(b["logits"][:1], oracle_model(data).forward_all(ids[:1]), what="c5 slab")


def test_sessions_identical(restore_selection):
    data = model_bytes("c4")
    prompts = synth.token_ids(25, "kern-c4", (64, 9), 4096)
    engine_option("gemm", "stream")
    i1, p1 = Model(data).sessions(64).decode_greedy(prompts, 6)
    engine_option("gemm", "slab")
    i2, p2 = Model(data).sessions(64).decode_greedy(prompts, 6)
    assert np.array_equal(i1, i2) and np.array_equal(p1, p2)
