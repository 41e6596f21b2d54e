"""Attention at every shape the reference runs (internal/quant/attention.go:46-104 takes any D/heads and any
cache): the `pro` and `xl` presets' head widths 56 and 72 (internal/train/presets.go:133-173), widths that
are not a multiple of 4 or wider than 128, and full-context models whose cache holds 512 or 2048 positions,
streaming past their context (the genbench full-attention candidate, internal/genbench/genbench_test.go:28,
92-123). Batched forward (both attention kernels) and sessions, each against the oracle."""
import numpy as np
import pytest

from helpers import assert_close, oracle_model, rel_err, tiny_spec, uniform_model_bytes
from mignon_ai_amd import Model, engine_option, mgnn, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore_selection():
    prev = engine_option("attention", "auto")
    yield
    engine_option("attention", prev)


def preset_bytes(D, H, heads, window=64, context=128, V=512, blocks=2, seed=5):
    spec = synth.ModelSpec(V=V, D=D, H=H, blocks=[synth.BlockSpec(1, 2, 1)] * blocks, heads=heads, window=window,
                           context=context)
    return spec, mgnn.build_model_file(spec, seed, O.quantize)


def forward_both(data, ids):
    m = Model(data)
    ref = oracle_model(data).forward_all(ids)
    out = {}
    for mode in ("exact", "mfma"):
        engine_option("attention", mode)
        out[mode] = m.forward_batch(ids)["logits"]
        assert_close(out[mode], ref, what=f"{mode} attention")
    assert rel_err(out["mfma"], out["exact"]).max() < 5e-5
    assert np.array_equal(out["exact"].argmax(-1), ref.argmax(-1))


def session_run(data, ids, P, ctx=0):
    """Prefill P tokens, then append the rest one by one; every output against the oracle's session."""
    gm = Model(data)
    om = oracle_model(data)
    gs = gm.new_session(ctx)
    os_ = om.new_session(ctx)
    assert_close(gs.prefill(ids[:P]), os_.prefill(ids[:P]), what="prefill")
    for t in range(P, len(ids)):
        assert_close(gs.append(ids[t]), os_.append(ids[t]), what=f"append {t}")


@pytest.mark.parametrize("name,D,H", [("pro", 224, 448), ("xl", 288, 576)])
def test_presets_forward(restore_selection, name, D, H):
    """The pro (head width 56) and xl (72) shapes, 4 heads, window 64, past the 128-token context."""
    spec, data = preset_bytes(D, H, 4)
    ids = synth.token_ids(41, f"preset-{name}", (3, 140), spec.V)
    forward_both(data, ids)


@pytest.mark.parametrize("name,D,H", [("pro", 224, 448), ("xl", 288, 576)])
def test_presets_sessions(name, D, H):
    spec, data = preset_bytes(D, H, 4)
    ids = synth.token_ids(42, f"preset-sess-{name}", (150,), spec.V)
    session_run(data, ids, 20)
    # a batch of sessions equals the teacher-forced batch
    gm = Model(data)
    S, P, T = 5, 9, 90
    ids2 = synth.token_ids(43, f"preset-batch-{name}", (S, T), spec.V)
    full = gm.forward_batch(ids2)["logits"]
    ss = gm.sessions(S)
    lg, _, _ = ss.prefill(ids2[:, :P])
    assert_close(lg, full[:, P - 1], what="prefill")
    for t in range(P, T):
        lg, _, _ = ss.step(ids2[:, t])
        assert_close(lg, full[:, t], what=f"step {t}")


@pytest.mark.parametrize("D,heads,window", [(60, 4, 20), (36, 2, 0), (6, 6, 9), (288, 1, 20), (256, 1, 0),
                                            (40, 5, 0), (216, 3, 64), (120, 8, 17)])
def test_any_head_width(restore_selection, D, heads, window):
    """Head widths 15, 18, 1, 288, 256, 8, 72, 15: not a multiple of 4, past 128, or one element."""
    spec = tiny_spec([(1, 2, 1), (1, 2, 2)], V=48, D=D, H=40, heads=heads, window=window, context=64)
    data = uniform_model_bytes(spec, scale=0.2)
    ids = synth.token_ids(44, f"width-{D}-{heads}-{window}", (2, 80), spec.V)
    forward_both(data, ids)
    session_run(data, ids[0], 11)


def test_full_context_512_streaming(restore_selection):
    """A full-attention model with a 512-position cache: the batch runs past the context (streaming
    positions attend the last 512), and a session streams 600 tokens through its ring."""
    spec = tiny_spec([(1, 2, 1), (1, 2, 1)], V=64, D=32, H=48, heads=2, window=0, context=512)
    data = uniform_model_bytes(spec, scale=0.3)
    ids = synth.token_ids(45, "ctx512", (2, 600), spec.V)
    forward_both(data, ids)
    session_run(data, ids[0], 100)
    # a session window shorter than the context truncates the prefill and then streams
    session_run(data, ids[1][:260], 230, ctx=200)


def test_genbench_full_attention_2048():
    """genbench's hybrid full-attention candidate at context 2048 on the medium shape (D128, H256, 4 heads,
    window 0): prefill of context - 64 tokens, then 64 appends (internal/genbench/genbench_test.go:88-123),
    each against the oracle; and the teacher-forced batch over the full context."""
    spec = synth.ModelSpec(V=2048, D=128, H=256, blocks=[synth.BlockSpec(1, 2, 1)] * 2, heads=4, window=0,
                           context=2048)
    data = mgnn.build_model_file(spec, 6, O.quantize)
    ids = (synth.token_ids(46, "genbench2048", (2048,), 1000)).astype(np.int32)
    session_run(data, ids, 2048 - 64, ctx=2048)
    gm = Model(data)
    ref = oracle_model(data).forward_all(ids[None, :])
    got = gm.forward_batch(ids[None, :])["logits"]
    assert_close(got, ref, what="batched forward, 2048 positions")
