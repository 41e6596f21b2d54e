"""The two batched attention kernels: the reference-order kernel (sequential DotF32 / softmax order) and
the matrix-core kernel (fp32 MFMA, other summation order). Both must match the oracle within the
engine's tolerance, and each other to 5e-5, for windowed and full-context attention, head widths
4..32, sequences longer than the context (streaming semantics) and ragged lengths."""
import numpy as np
import pytest

from helpers import GOLDEN, assert_close, model_bytes, oracle_model, rel_err, tiny_spec, uniform_model_bytes
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore_selection():
    prev = engine_option("attention", "auto")
    yield
    engine_option("attention", prev)


def _both(data, ids):
    m = Model(data)
    engine_option("attention", "exact")
    a = m.forward_batch(ids)["logits"]
    engine_option("attention", "mfma")
    b = m.forward_batch(ids)["logits"]
    ref = oracle_model(data).forward_all(ids)
    assert_close(a, ref, what="exact attention")
    assert_close(b, ref, what="mfma attention")
    # the two differ by fp32 summation order only; a trained model amplifies that to ~1e-5
    assert rel_err(b, a).max() < 5e-5
    return a, b


@pytest.mark.parametrize("window,context,T", [(7, 64, 45), (64, 64, 130), (0, 64, 50), (0, 64, 200), (0, 128, 150),
                                              (0, 256, 300), (100, 256, 180), (7, 64, 64), (64, 64, 128),
                                              (0, 64, 192), (30, 128, 160)])
def test_windows_and_lengths(restore_selection, window, context, T):
    """Key spans of 7..256 (1 to 17 blocks of 16 keys) and sequences past the context."""
    spec = tiny_spec([(2, 2, 1), (1, 2, 2)], V=96, D=64, H=48, heads=4, window=window, context=context)
    data = uniform_model_bytes(spec, scale=0.3)
    ids = synth.token_ids(31, f"attn{window}-{context}-{T}", (3, T), 96)
    _both(data, ids)


@pytest.mark.parametrize("D,heads,T", [(8, 2, 70), (48, 3, 70), (96, 4, 70), (128, 4, 70), (8, 2, 48), (48, 3, 80),
                                        (96, 4, 96), (128, 8, 64), (128, 4, 32)])
def test_head_widths(restore_selection, D, heads, T):
    """Head widths 4..32, whole and partial 16-query tiles."""
    spec = tiny_spec([(1, 2, 1), (1, 2, 1)], V=64, D=D, H=32, heads=heads, window=20)
    data = uniform_model_bytes(spec, scale=0.3)
    ids = synth.token_ids(32, f"attn-d{D}-{T}", (2, T), 64)
    _both(data, ids)


def test_real_model(restore_selection):
    with open(f"{GOLDEN}/orders.mgn", "rb") as f:
        data = f.read()
    ids = synth.token_ids(33, "attn-orders", (3, 140), 2048)
    _both(data, ids)


def test_c3_subset(restore_selection):
    data = model_bytes("c3")
    ids = synth.token_ids(34, "attn-c3", (4, 128), 2048)
    _both(data, ids)
