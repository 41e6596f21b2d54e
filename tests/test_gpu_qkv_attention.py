"""The attention projection fused with matrix-core attention (MG_ATTN_FUSED, automatic for teacher-forced
batches of 128-token sequences with head width 32 or 64) against the separate QKV GEMM + attention kernel
(MG_ATTN_MFMA): the fused kernel takes the same q, k and v sums and runs the same attention arithmetic, so
logits and log-probs must be identical bit for bit; and against the oracle. Shapes: c5 (D384, 6 heads of
64, window 64), c3 (D128, 4 heads of 32), a full-context model (window 0, cap 128: nine key blocks), a
short window (three key blocks), and batches whose sequence count leaves a partial run of sequences."""
import numpy as np
import pytest

from helpers import assert_close, model_bytes, oracle_model
from mignon_ai_amd import Model, engine_option, mgnn, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore_attention():
    # the output projection on the attention output's limb planes in both modes (the separate kernels
    # write no per-head maxima, so only the fused mode could take the fp32 operand)
    prev = engine_option("attention", "auto")
    prev_ops = engine_option("operands", "limbs")
    yield
    engine_option("attention", prev)
    engine_option("operands", prev_ops)


def _both(data, ids, logits):
    out = {}
    for mode in ("mfma", "fused"):
        engine_option("attention", mode)
        m = Model(data)
        out[mode] = m.forward_batch(ids, logits=logits, logprob=True)
    return out


def _check(data, ids, n_oracle=1, logits=True):
    out = _both(data, ids, logits)
    for k in out["mfma"]:
        a, b = out["mfma"][k], out["fused"][k]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), k
    if logits:
        assert_close(out["fused"]["logits"][:n_oracle], oracle_model(data).forward_all(ids[:n_oracle]),
                     what="fused")


@pytest.mark.parametrize("cfg,B", [("c5", 3), ("c3", 37)])
def test_fused_equals_separate(restore_attention, cfg, B):
    spec = synth.CONFIGS[cfg]["spec"]
    ids = synth.token_ids(31, f"qkvatt:{cfg}", (B, 128), spec.V)
    _check(model_bytes(cfg), ids)


def test_fused_partial_run(restore_attention):
    """1025 sequences of c3: two sequences per workgroup run, the last run holding one (log-probs compared,
    each of which depends on every logit of its row through the log-sum-exp)."""
    spec = synth.CONFIGS["c3"]["spec"]
    ids = synth.token_ids(33, "qkvatt:c3:big", (1025, 128), spec.V)
    _check(model_bytes("c3"), ids, logits=False)


@pytest.mark.parametrize("D,heads,window,context", [(64, 2, 0, 128), (128, 2, 20, 128), (256, 8, 64, 128)])
def test_fused_shapes(restore_attention, D, heads, window, context):
    spec = synth.ModelSpec(V=300, D=D, H=2 * D, blocks=[synth.BlockSpec(1, 2, 1)] * 2, heads=heads, window=window,
                           context=context)
    data = mgnn.build_model_file(spec, 17, O.quantize)
    ids = synth.token_ids(32, f"qkvatt:{D}:{window}", (9, 128), spec.V)
    _check(data, ids, n_oracle=2)
