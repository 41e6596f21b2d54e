"""Model-level pins of the oracle (CPU): what makes its restatement of the reference engine trustworthy.

- The reference's own invariants: streaming session == Call, bit for bit
  (internal/quant/session_test.go:18-52), and bounded session state (:54-90).
- An independent float64, step-major restatement (tests/ref_f64.py) agrees to 1e-5 relative on the
  reference's six equivalence architectures, on the benchmark configurations and on the reference's own
  trained model file (examples/order-search/orders.mgn, copied to tests/golden/).
- Closed forms that a dropped term would break: identity blocks (highway gate closed) leave
  cur = 2^(blocks-1) * embedding; a zero attention output projection is the identity.
"""
import numpy as np
import pytest

import ref_f64
from helpers import EQUIV_CASES, GOLDEN, equiv_model_bytes, model_bytes, oracle_model, rel_err, tiny_spec, uniform_model_bytes
from mignon_ai_amd import mgnn, synth
from oracle import oracle as O

WINDOW, TOKENS, PREFILL = 12, 40, 5


def orders_bytes():
    with open(f"{GOLDEN}/orders.mgn", "rb") as f:
        return f.read()


@pytest.mark.parametrize("case", list(EQUIV_CASES))
def test_session_matches_call_bitwise(case):
    """TestQuantSessionMatchesCall: every session output equals Call over the whole sequence so far."""
    om = oracle_model(equiv_model_bytes(case))
    rng = np.random.default_rng(9)
    toks = rng.integers(0, 16, TOKENS).astype(np.int32)
    s = om.new_session(WINDOW)
    window = list(toks[:PREFILL])
    assert np.array_equal(s.prefill(window), om.call(window))
    for i in range(PREFILL, TOKENS):
        window.append(toks[i])
        assert np.array_equal(s.append(toks[i]), om.call(window)), i
    long = toks[:2 * WINDOW]
    assert np.array_equal(s.prefill(long), om.call(long[-WINDOW:]))


@pytest.mark.parametrize("case", ["2blk", "2blk attn window"])
def test_session_state_is_bounded(case):
    """TestQuantSessionStateIsBounded / ...WindowedAttentionIsBounded, plus the byte formula of
    quantSeqState.bytes (internal/quant/stream.go:87-101)."""
    c = EQUIV_CASES[case]
    om = oracle_model(equiv_model_bytes(case))
    s = om.new_session(WINDOW)
    s.prefill([1, 2])
    before = s.state_bytes()
    for i in range(10 * om.max_context):
        s.append(i % 16)
    assert s.state_bytes() == before
    D = 8
    steps = sum(b[0] for b in c["blocks"])
    ring = 1 + max(ref_f64.step_dilation(b[2], b[1], st) for b in c["blocks"] for st in range(b[0]))
    n = 3 * D + steps * (ring * D + D)
    cap = c.get("window", 0) or om.max_context
    n32 = (2 * cap + len(c["blocks"]) * 2 * cap * D) if c.get("heads") else 0
    assert before == n * 8 + n32 * 4


@pytest.mark.parametrize("case", list(EQUIV_CASES))
def test_oracle_matches_f64_restatement_equiv_cases(case):
    rm = O.read_model(equiv_model_bytes(case))
    om = O.OracleModel(rm)
    ids = np.array([2, 5, 7, 1, 9, 3, 11, 4, 0, 15, 6, 8, 2, 2, 13, 1, 0, 5, 9, 9] * 4, np.int32)
    got = om.forward_all(ids[None])[0]
    ref = ref_f64.forward(rm, ids, om.max_context)
    assert rel_err(got, ref).max() < 1e-5


@pytest.mark.parametrize("name", ["c1", "c3"])
def test_oracle_matches_f64_restatement_configs(name):
    rm = O.read_model(model_bytes(name))
    om = O.OracleModel(rm)
    ids = synth.token_ids(3, "f64", (70,), rm.V)
    got = om.forward_all(ids[None])[0]
    assert rel_err(got, ref_f64.forward(rm, ids, om.max_context)).max() < 1e-5


def test_oracle_matches_f64_restatement_real_model():
    """The reference's trained 538k-parameter model: 2 hybrid blocks, 4 heads of width 24."""
    rm = O.read_model(orders_bytes())
    om = O.OracleModel(rm)
    assert (rm.V, rm.D, rm.H, rm.heads, rm.window, len(rm.blocks)) == (2048, 96, 160, 4, 64, 2)
    ids = (np.arange(1, 150, dtype=np.int32) * 7) % 2048
    got = om.forward_all(ids[None])[0]
    assert rel_err(got, ref_f64.forward(rm, ids, om.max_context)).max() < 1e-5


def _spec_q(spec, seed=5, tweak=None):
    w = synth.float_weights(spec, seed, std=0.05)
    if tweak:
        tweak(w)
    q = {}
    for k, v in w.items():
        if synth.is_matrix(k):
            q[k], q[k + ".scale"] = O.quantize(v)
        else:
            q[k] = v
    return q


def test_identity_blocks_closed_form():
    """Highway gates shut (gate bias -100: sigmoidClamped = 0) make each rule step the identity, so the
    inter-block residual doubles the embedding per block. Without a final norm the logits are then
    exactly s_e * Emb . (2^(B-1) e) + head_b in closed form."""
    spec = tiny_spec([(2, 2, 1), (1, 2, 2), (1, 2, 1)], V=40, D=24, H=16)

    def shut(w):
        for b in range(3):
            w[f"b{b}.b2"][spec.D:] = -100.0
        w["head_b"][:] = np.linspace(-1, 1, spec.V).astype(np.float32)

    q = _spec_q(spec, tweak=shut)
    q["final_norm"] = np.zeros(0, np.float32)
    rm = O.read_model(mgnn.encode(spec, q))
    om = O.OracleModel(rm)
    ids = np.array([3, 17, 39, 0, 8], np.int32)
    got = om.forward_all(ids[None])[0]
    E = rm.embed.astype(np.float64).reshape(spec.V, spec.D) * float(rm.embed_scale)
    cur = 4.0 * E[ids]
    want = cur @ rm.embed.astype(np.float64).reshape(spec.V, spec.D).T * float(rm.embed_scale) + rm.head_b
    assert rel_err(got, want).max() < 1e-6


def test_zero_output_projection_is_identity():
    """W_o = 0 (the reference's own attention init, internal/nn/attention.go:40-52) adds exactly zero."""
    base = tiny_spec([(2, 2, 1), (1, 2, 2)], V=40, D=32, H=16)
    attn = tiny_spec([(2, 2, 1), (1, 2, 2)], V=40, D=32, H=16, heads=4, window=5)
    q = _spec_q(attn)
    for b in range(2):
        q[f"b{b}.out"] = np.zeros_like(q[f"b{b}.out"])
    qb = {k: v for k, v in q.items() if not any(x in k for x in ("attn_norm", "qkv", "out"))}
    ids = np.array([[1, 5, 9, 30, 2, 2, 7, 39, 11, 4]], np.int32)
    with_attn = O.OracleModel(O.read_model(mgnn.encode(attn, q))).forward_all(ids)
    without = O.OracleModel(O.read_model(mgnn.encode(base, qb))).forward_all(ids)
    assert np.array_equal(with_attn, without)


@pytest.mark.parametrize("name", ["c1", "c3", "c4", "c5"])
def test_num_params_matches_reference_layout(name):
    """quant.Model.NumParams equals the full-precision layout's count (binary_test.go:27-30)."""
    spec = synth.CONFIGS[name]["spec"]
    rm = O.read_model(model_bytes(name))
    n = rm.embed.size + sum(b.w1.size + b.b1.size + b.w2.size + b.b2.size + b.gamma.size + b.wsel.size +
                            (b.attn["norm"].size + b.attn["qkv"].size + b.attn["wo"].size if b.attn else 0)
                            for b in rm.blocks) + rm.final_norm.size + rm.head_b.size
    assert n == spec.n_params
    assert {"c1": 34560, "c3": 954496, "c4": 5187840, "c5": 18700672}[name] == n


def test_real_model_param_count():
    rm = O.read_model(orders_bytes())
    n = rm.embed.size + sum(b.w1.size + b.b1.size + b.w2.size + b.b2.size + b.gamma.size + b.wsel.size +
                            b.attn["norm"].size + b.attn["qkv"].size + b.attn["wo"].size for b in rm.blocks)
    n += rm.final_norm.size + rm.head_b.size
    assert n == 538080


def test_untied_head():
    spec = tiny_spec([(1, 2, 1)], V=50, D=16, H=8, tied=False)
    data = uniform_model_bytes(spec)
    rm = O.read_model(data)
    assert not rm.tied and rm.head_w.size == 50 * 16
    om = O.OracleModel(rm)
    ids = np.array([1, 2, 49, 3], np.int32)
    assert rel_err(om.forward_all(ids[None])[0], ref_f64.forward(rm, ids, om.max_context)).max() < 1e-5
