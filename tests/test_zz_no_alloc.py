"""mg_sessions_step_noalloc (the decode step that allocates nothing: its workspace is the library's static
per-GPU scratch array) against mg_sessions_step on device pointers: bitwise-identical logits, argmax and
probabilities, on two calls in a row for a set of 48 sessions and then two for a smaller set of 8 (the
scratch keeps the earlier call's contents, which must not matter), plus the size limit, and two models on
their own streams sharing the GPU's array."""
import numpy as np
import pytest

from helpers import model_bytes
from mignon_ai_amd import MignonError, Model, synth

pytestmark = pytest.mark.gpu


def _pair(m, S, spec, tag):
    prompts = synth.token_ids(7, f"noalloc:{tag}", (S, 9), spec.V)
    a, b = m.sessions(S), m.sessions(S)
    a.prefill(prompts)
    b.prefill(prompts)
    return a, b


def test_noalloc_step_equals_step():
    import torch
    data = model_bytes("c4")
    spec = synth.CONFIGS["c4"]["spec"]
    m = Model(data)
    stream = torch.cuda.current_stream().cuda_stream
    m.set_stream(stream)
    for S in (48, 8):
        a, b = _pair(m, S, spec, str(S))
        for k in range(2):
            ids = torch.from_numpy(synth.token_ids(8, f"noalloc:{S}:{k}", (S,), spec.V)).cuda()
            outs = []
            for sess, fn in ((a, a.step_device), (b, b.step_noalloc)):
                lg = torch.full((S, spec.V), float("nan"), dtype=torch.float32, device="cuda")
                am = torch.full((S,), -1, dtype=torch.int32, device="cuda")
                pb = torch.full((S,), float("nan"), dtype=torch.float64, device="cuda")
                fn(ids, lg, am, pb)
                outs.append((lg, am, pb))
            torch.cuda.synchronize()
            print(f"S={S} call {k}: argmax[:4] {outs[0][1][:4].tolist()}")
            for x, y in zip(*outs):
                assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), f"S={S} call {k}"
            assert bool(torch.isfinite(outs[1][0]).all())


def test_noalloc_step_rejects_sets_beyond_the_scratch():
    """3000 sessions of c5's D384/H1024/V8192 model need about 75 MB of workspace (the array holds 64 MiB):
    refused on the host, before any launch; the ordinary step still runs them."""
    import torch
    data = model_bytes("c5")
    spec = synth.CONFIGS["c5"]["spec"]
    m = Model(data)
    S = 3000
    big = m.sessions(S)
    ids = torch.zeros(S, dtype=torch.int32, device="cuda")
    am = torch.empty(S, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    with pytest.raises(MignonError, match="scratch"):
        big.step_noalloc(ids, None, am, None)
    big.step_device(ids, None, am, None)
    m.sync()
    assert int(am.min()) >= 0


def test_noalloc_two_models_on_one_gpu():
    """Two models on their own streams calling the allocation-free step one after the other from one
    thread: the second call waits on the device for the first (they share the GPU's scratch array), so
    both equal their models' ordinary steps bit for bit; then in the other order, twice."""
    import torch
    data = model_bytes("c4")
    spec = synth.CONFIGS["c4"]["spec"]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    models = [Model(data), Model(data)]
    for m, st in zip(models, streams):
        m.set_stream(st.cuda_stream)
    S = 96
    pairs = [_pair(m, S, spec, f"two:{i}") for i, m in enumerate(models)]
    torch.cuda.synchronize()
    for k, order in enumerate(((0, 1), (1, 0), (0, 1))):
        ids = [torch.from_numpy(synth.token_ids(9, f"two:{k}:{i}", (S,), spec.V)).cuda() for i in range(2)]
        torch.cuda.synchronize()
        got, want = {}, {}
        for i in order:  # back to back on two streams
            lg = torch.full((S, spec.V), float("nan"), dtype=torch.float32, device="cuda")
            am = torch.full((S,), -1, dtype=torch.int32, device="cuda")
            torch.cuda.synchronize()
            pairs[i][1].step_noalloc(ids[i], lg, am, None)
            got[i] = (lg, am)
        for m in models:
            m.sync()
        for i in range(2):
            lg = torch.full((S, spec.V), float("nan"), dtype=torch.float32, device="cuda")
            am = torch.full((S,), -1, dtype=torch.int32, device="cuda")
            pairs[i][0].step_device(ids[i], lg, am, None)
            models[i].sync()
            want[i] = (lg, am)
        for i in range(2):
            assert torch.equal(got[i][0].view(torch.uint8), want[i][0].view(torch.uint8)), (k, i)
            assert torch.equal(got[i][1], want[i][1]), (k, i)
