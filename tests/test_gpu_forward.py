"""Teacher-forced batched forward through the C ABI against the oracle's streaming engine.

Bar (north star): logits within 1e-4 relative (per element, against max(|ref|, rms of the row)) and
identical argmax wherever the oracle's top-2 gap is not a near-tie."""
import numpy as np
import pytest

from helpers import RTOL, assert_close, model_bytes, oracle_model, rel_err
from mignon_ai_amd import Model, synth

pytestmark = pytest.mark.gpu


def _argmax_agree(got, ref):
    a = got.argmax(-1)
    b = ref.argmax(-1)
    srt = np.sort(ref, axis=-1)
    gap = srt[..., -1] - srt[..., -2]
    scale = np.maximum(np.abs(srt[..., -1]), np.sqrt(np.mean(ref.astype(np.float64) ** 2, axis=-1)))
    near_tie = gap <= 2 * RTOL * scale
    bad = (a != b) & ~near_tie
    return int(bad.sum()), int(near_tie.sum())


@pytest.mark.parametrize("name,B,T", [("c1", 64, 128), ("c3", 4, 128), ("c5", 2, 128)])
def test_forward_logits_match_oracle(name, B, T):
    data = model_bytes(name)
    spec = synth.CONFIGS[name]["spec"]
    ids = synth.token_ids(7, name + ":ids", (B, T), spec.V)
    gm = Model(data)
    out = gm.forward_batch(ids, logits=True, logprob=True, bits=True)
    om = oracle_model(data)
    ref = om.forward_all(ids)
    worst = assert_close(out["logits"], ref, what=f"{name} logits")
    print(f"{name}: max rel err {worst:.2e}")
    bad, ties = _argmax_agree(out["logits"], ref)
    assert bad == 0, f"{bad} argmax mismatches outside near-ties ({ties} near-ties)"
    # log-probs of the targets (eval.logProb in float64 on the oracle's logits)
    r64 = ref.astype(np.float64)
    mx = r64.max(-1, keepdims=True)
    lse = mx[..., 0] + np.log(np.exp(r64 - mx).sum(-1))
    tg = ids[:, 1:]
    want = np.take_along_axis(r64[:, :-1], tg[..., None], -1)[..., 0] - lse[:, :-1]
    assert np.allclose(out["logprob"][:, :-1], want, rtol=0, atol=1e-4 * np.maximum(1, np.abs(want)).max())
    assert np.all(np.isnan(out["logprob"][:, -1]))
    bits = -want.sum(1) / (np.log(2) * (T - 1))
    assert np.allclose(out["bits"], bits, rtol=1e-5)


def test_forward_probs_c1():
    data = model_bytes("c1")
    spec = synth.CONFIGS["c1"]["spec"]
    ids = synth.token_ids(8, "c1:probs", (8, 128), spec.V)
    gm = Model(data)
    out = gm.forward_batch(ids, logits=True, probs=True)
    l = out["logits"].astype(np.float64)
    p = np.exp(l - l.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    assert np.all(rel_err(out["probs"], p) <= 1e-4)
    assert np.allclose(out["probs"].sum(-1), 1.0, atol=1e-4)


def test_call_matches_oracle_and_truncates():
    data = model_bytes("c3")
    spec = synth.CONFIGS["c3"]["spec"]
    gm = Model(data)
    om = oracle_model(data)
    ids = synth.token_ids(9, "c3:call", (200,), spec.V)
    for n in (1, 2, 65, 128, 200):
        got = gm.call(ids[:n])
        ref = om.call(ids[:n])
        assert_close(got, ref, what=f"Call n={n}")
    assert gm.call(np.zeros(0, np.int32)) is None


def test_forward_out_of_range_ids_clamp():
    data = model_bytes("c1")
    gm = Model(data)
    om = oracle_model(data)
    ids = np.array([[5, -3, 600, 511, 512, 0, 7, 100000]], np.int32)
    out = gm.forward_batch(ids)
    ref = om.forward_all(ids)
    assert_close(out["logits"], ref)


@pytest.mark.parametrize("heads", [0, 2])
def test_block_residual_paths(heads):
    """The inter-block residual is added by a block's last GEMM (out projection, or the last highway)
    when the next block has steps, and by the row kernel otherwise: blocks without steps (attention only,
    or nothing but the residual) between blocks with steps, decoded through both routes, against the
    oracle; then the same model through sessions (prefill and streamed steps)."""
    from helpers import tiny_spec, uniform_model_bytes
    spec = tiny_spec([(2, 2, 1), (0, 2, 1), (1, 2, 1), (2, 3, 1)], V=61, D=24, H=20, heads=heads,
                     window=9 if heads else 0)
    data = uniform_model_bytes(spec, scale=0.4)
    gm = Model(data)
    om = oracle_model(data)
    ids = synth.token_ids(41, f"resid{heads}", (3, 40), spec.V)
    assert_close(gm.forward_batch(ids)["logits"], om.forward_all(ids), what=f"blocks with and without steps, heads {heads}")
    ss = gm.sessions(3)
    lg, am, pb = ss.prefill(ids[:, :20])
    assert_close(lg, om.forward_all(ids[:, :20])[:, -1], what="session prefill")
    for t in range(20, 24):
        lg, am, pb = ss.step(ids[:, t])
        assert_close(lg, om.forward_all(ids[:, :t + 1])[:, -1], what=f"session step {t}")
