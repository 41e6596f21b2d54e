"""The GEMMs that read the GLU output (the highway GEMM) and the fused attention's output (the output
projection) as fp32 rows, expanding each row to three base-256 digit planes as they load it with the scale
taken from partial maxima its producer wrote (MG_OPERANDS_FP32, automatic wherever the weight-stationary
kernel runs them), against the same forward with a row pass writing limb planes before each of those
GEMMs (MG_OPERANDS_LIMBS) and against the oracle.

Both paths hold every operand element within 2e-7 of its row's largest magnitude, so their outputs agree
far inside the 1e-4 bar: they are compared at 3e-5 (the trained orders.mgn differs by 1.0e-5, the
synthetic models by less), and each against the oracle at 1e-4. The per-class
launch counts show that the fp32 path ran (the row passes of h and of the attention output are gone).
Shapes: c5 (highway K 1024 in 16 K steps, output projection K 384 over six 64-wide heads), c3 (four heads of
32, K 256), c1 (no attention, two rule steps), ragged token counts (rows past the batch in the last tile),
the reference's trained orders.mgn (hidden size 160: the GLU output's padding columns meet zero weights;
24-wide heads, so its attention output keeps the row pass), and an untied head with an odd vocabulary.
With the fused scan, the RMSNorm before each later block's latch GEMM happens inside that GEMM (from
statistics the previous block's last GEMM writes) and its row pass is gone too."""
import numpy as np
import pytest

from helpers import GOLDEN, assert_close, model_bytes, oracle_model, rel_err, tiny_spec, uniform_model_bytes
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def slab_forced():
    # small batches take the weight-stationary kernels (and with them the fp32 operands) and the fused scan
    # (which the RMSNorm inside the latch GEMM needs) only when forced
    prev = engine_option("gemm", "slab")
    prev_scan = engine_option("scan", "fused")
    prev_ops = engine_option("operands")
    yield
    engine_option("gemm", prev)
    engine_option("scan", prev_scan)
    engine_option("operands", prev_ops)


def _run(data, ids, **kw):
    out, rows = {}, {}
    for mode in ("limbs", "fp32"):
        engine_option("operands", mode)
        m = Model(data)
        m.profile(True)
        out[mode] = m.forward_batch(ids, **kw)
        prof = m.profile_read()
        m.profile(False)
        rows[mode] = prof.get("row_norm_pack", (0,))[0]
    return out, rows


def removed_passes(D, H, heads, steps, nattn, T, chained=0):
    """Row passes the fp32 operands take away from one forward: h's per rule step when its padded width
    (a multiple of 64) is at least 128 (two K steps) and has at most 16 channel tiles of partial maxima; the
    attention output's per attention block where the fused attention runs (128-token sequences, heads of
    32 or 64) and the padded state is at least 128 wide; and the RMSNorm before the latch GEMM of each of
    the `chained` blocks whose input the previous block added into blockIn, where the fused scan runs
    (sequence lengths a multiple of 16) and the padded state is at least 128 wide."""
    Hp, Dp = -(-H // 64) * 64, -(-D // 64) * 64
    n = steps if 128 <= Hp <= 1024 else 0
    if nattn and T == 128 and D // heads in (32, 64) and 128 <= Dp <= 384:
        n += nattn
    if T % 16 == 0 and Dp >= 128:
        n += chained
    return n


def _check(data, ids, removed, n_oracle=1, **kw):
    out, rows = _run(data, ids, logits=True, **kw)
    for k in out["limbs"]:
        a, b = out["fp32"][k], out["limbs"][k]
        if k == "logprob":  # the last position has no target: NaN in both
            assert np.isnan(a[:, -1]).all() and np.isnan(b[:, -1]).all()
            a, b = a[:, :-1], b[:, :-1]
        print(f"{k}: fp32 vs limb operands {float(rel_err(a, b).max()):.2e}")
    assert rows["limbs"] - rows["fp32"] == removed, (rows, removed)
    ref = oracle_model(data).forward_all(ids[:n_oracle])
    e_fp32 = assert_close(out["fp32"]["logits"][:n_oracle], ref, what="fp32 operands vs oracle")
    e_limbs = assert_close(out["limbs"]["logits"][:n_oracle], ref, what="limb operands vs oracle")
    print(f"worst relative error against the oracle: fp32 operands {e_fp32:.2e}, limb operands {e_limbs:.2e}")
    if "probs" in out["fp32"]:
        r = ref.astype(np.float64)
        pr = np.exp(r - r.max(-1, keepdims=True))
        pr /= pr.sum(-1, keepdims=True)
        p_fp32 = assert_close(out["fp32"]["probs"][:n_oracle], pr, what="fp32 operands: probabilities vs oracle")
        p_limbs = assert_close(out["limbs"]["probs"][:n_oracle], pr, what="limb operands: probabilities vs oracle")
        print(f"probabilities against the oracle: fp32 operands {p_fp32:.2e}, limb operands {p_limbs:.2e}")


def _removed(spec, T):
    chained = sum(1 for i in range(1, len(spec.blocks))
                  if spec.blocks[i].steps > 0 and (spec.heads > 0 or spec.blocks[i - 1].steps > 0))
    return removed_passes(spec.D, spec.H, spec.heads, sum(b.steps for b in spec.blocks),
                          len(spec.blocks) if spec.heads else 0, T, chained)


@pytest.mark.parametrize("cfg,shape", [("c5", (3, 128)), ("c3", (5, 128)), ("c3", (2, 61)), ("c1", (3, 37))])
def test_fp32_operands(slab_forced, cfg, shape):
    spec = synth.CONFIGS[cfg]["spec"]
    ids = synth.token_ids(41, f"fp32ops:{cfg}:{shape}", shape, spec.V)
    removed = _removed(spec, shape[1])
    assert removed > 0 or cfg == "c1"  # c1's 64-wide h is one K step: its row pass stays
    _check(model_bytes(cfg), ids, removed, logprob=True, bits=shape[1] > 1)


def test_fp32_operands_real_model(slab_forced):
    """orders.mgn: D96 H160 (h padded to 192: three channel tiles of maxima, padding columns), 2 blocks,
    4 heads of 24 (the attention output keeps its row pass)."""
    with open(f"{GOLDEN}/orders.mgn", "rb") as f:
        data = f.read()
    ids = synth.token_ids(42, "fp32ops:orders", (3, 128), 2048)
    _check(data, ids, removed_passes(96, 160, 4, 2, 2, 128, 1), n_oracle=2, probs=True)


def test_fp32_operands_untied_no_attention(slab_forced):
    spec = tiny_spec([(2, 2, 1), (1, 2, 2)], V=131, D=48, H=72, tied=False)
    data = uniform_model_bytes(spec, scale=0.3)
    ids = synth.token_ids(43, "fp32ops:untied", (4, 45), 131)
    _check(data, ids, _removed(spec, 45), n_oracle=4, logprob=True)


def test_fp32_operands_automatic_batch():
    """Without forcing: a batch of 8192 rows takes the weight-stationary kernels and the fp32 operands by
    itself; sequences at both ends against the oracle."""
    prev = engine_option("operands", "auto")
    try:
        data = model_bytes("c3")
        ids = synth.token_ids(44, "fp32ops:auto", (64, 128), 2048)
        m = Model(data)
        m.profile(True)
        got = m.forward_batch(ids, logits=True)["logits"]
        rows_auto = m.profile_read()["row_norm_pack"][0]
        m.profile(False)
        engine_option("operands", "limbs")
        m2 = Model(data)
        m2.profile(True)
        want = m2.forward_batch(ids, logits=True)["logits"]
        rows_limbs = m2.profile_read()["row_norm_pack"][0]
        assert rows_auto < rows_limbs, (rows_auto, rows_limbs)
        assert_close(got, want, rtol=1e-5, what="automatic vs limb operands")
        sub = [0, 63]
        assert_close(got[sub], oracle_model(data).forward_all(ids[sub]), what="automatic vs oracle")
    finally:
        engine_option("operands", prev)
