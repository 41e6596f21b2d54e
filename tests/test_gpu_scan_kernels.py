"""The fused latch scan + rule-input packing (one kernel, no latch state written) and the separate path
(the scan writes the latch state of every position, then the row kernel packs [n | left | g]) build
byte-identical GEMM operands, so every model output must be bit-identical between them; the fused path is
also checked against the oracle. In a batched forward without a session export the fused kernel does not
read the normalised rows n but recomputes them from the norm's source rows and the row kernel's 1/rms per
row, so the bit equality also pins that recomputation. Covers dilations 1..32 (left neighbours up to two tiles back), padded
widths (D not a multiple of 64), several blocks and steps, 16..256-token sequences, the session export of
the latch state at each prompt's last position (ragged prefill lengths, then greedy steps), and lengths
that are not a multiple of 16 (where the separate kernels run whatever the option says)."""
import numpy as np
import pytest

from helpers import assert_close, model_bytes, oracle_model, tiny_spec, uniform_model_bytes
from mignon_ai_amd import Model, engine_option, synth

pytestmark = pytest.mark.gpu


@pytest.fixture
def restore_selection():
    prev = engine_option("scan", "auto")
    yield
    engine_option("scan", prev)


def _both(m, ids, **kw):
    engine_option("scan", "separate")
    a = m.forward_batch(ids, **kw)
    engine_option("scan", "fused")
    b = m.forward_batch(ids, **kw)
    return a, b


def _same(a, b):
    for k in a:
        assert np.array_equal(np.asarray(a[k]).view(np.uint32), np.asarray(b[k]).view(np.uint32)), k


def test_scan_fused_dilations(restore_selection):
    # dilations 1, 2, 4, 8, 16, 32 in the first block, 2 and 6 in the second; D = 40 pads to 64
    spec = tiny_spec([(6, 2, 1), (2, 3, 2)], V=97, D=40, H=24, heads=2, window=9, context=256)
    data = uniform_model_bytes(spec, scale=0.3)
    m = Model(data)
    ids = synth.token_ids(31, "scan-dil", (3, 96), spec.V)
    a, b = _both(m, ids, logits=True, logprob=True)
    _same(a, b)
    assert_close(b["logits"], oracle_model(data).forward_all(ids), what="fused scan, dilations to 32")


@pytest.mark.parametrize("shape", [(1, 16), (5, 128), (2, 256)])
def test_scan_fused_c3(restore_selection, shape):
    data = model_bytes("c3")
    spec = synth.CONFIGS["c3"]["spec"]
    m = Model(data)
    ids = synth.token_ids(32, f"scan-c3{shape}", shape, spec.V)
    a, b = _both(m, ids, logits=True, logprob=True, bits=True)
    _same(a, b)
    if shape[0] * shape[1] <= 640:
        assert_close(b["logits"], oracle_model(data).forward_all(ids), what=f"fused scan c3 {shape}")


def test_scan_unfusable_length(restore_selection):
    # T = 37: the fused kernel does not apply; "fused" falls back to the separate kernels
    data = model_bytes("c1")
    spec = synth.CONFIGS["c1"]["spec"]
    m = Model(data)
    ids = synth.token_ids(33, "scan-37", (3, 37), spec.V)
    a, b = _both(m, ids, logits=True)
    _same(a, b)
    assert_close(b["logits"], oracle_model(data).forward_all(ids), what="T=37")


def test_scan_fused_session_export(restore_selection):
    """Prefill exports each session's latch state at its last prompt position; the greedy steps that
    follow read it, so they agree between the two paths only if the exported state does."""
    data = model_bytes("c3")
    spec = synth.CONFIGS["c3"]["spec"]
    m = Model(data)
    lens = np.array([1, 5, 32, 17, 16, 31], np.int32)
    ids = synth.token_ids(34, "scan-sess", (6, 32), spec.V)
    out = {}
    for mode in ("separate", "fused"):
        engine_option("scan", mode)
        ss = m.sessions(6)
        lg, am, pb = ss.prefill(ids, lens)
        steps = [lg]
        for t in range(6):
            lg, am, pb = ss.step(am)
            steps.append(lg)
        out[mode] = np.stack(steps)
        ss.close()
    assert np.array_equal(out["separate"].view(np.uint32), out["fused"].view(np.uint32))
    om = oracle_model(data)
    for i, L in enumerate(lens):
        assert_close(out["fused"][0, i], om.call(ids[i, :L]), what=f"session {i} prefill")
