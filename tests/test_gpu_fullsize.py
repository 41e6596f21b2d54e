"""The benchmark's own workloads at the sizes it times them, on device.

c5 runs as one pass of 2^21 tokens, whose probability rows sit up to 1.7e10 elements past the base, so the
test reaches the 64-bit offsets that smaller batches never touch. Checks: every probability row sums to
one; every sequence's bits per token equals -log2 of its gathered target probabilities (eval nll.score,
internal/eval/eval.go:25-48); the log-probs equal the log of those probabilities; and four sequences (0,
8191, 8192, 16383) against the oracle at 1e-4. A batch of more tokens than one pass holds (the c1 model,
17,000 x 128 tokens) checks the passes' boundary: log-probs and bits of sequences on both sides of it
against the oracle.

c2's timed call writes no int32 output, so its tiles leave through the LDS-staged row-segment stores; over
all 262,144 rows it must equal, bit for bit, the call that also writes the int32 accumulators (whose rows
test_gpu_gemm.py pins against exact integer arithmetic), and sampled rows must equal the oracle's exact
GEMM."""
import numpy as np
import pytest

from helpers import model_bytes, oracle_model, rel_err
from mignon_ai_amd import Model, gemm_i8_device, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def test_c5_full_size_device():
    import torch
    data = model_bytes("c5")
    cfg = synth.CONFIGS["c5"]
    spec = cfg["spec"]
    B, T, V = cfg["B"], cfg["T"], spec.V
    ids_np = synth.token_ids(1, "c5:ids", (B, T), V)  # the benchmark's input
    m = Model(data)
    s = torch.cuda.Stream()
    m.set_stream(s.cuda_stream)
    ids = torch.from_numpy(ids_np).cuda()
    probs = torch.empty((B, T, V), dtype=torch.float32, device="cuda")  # 68.7 GB
    bits = torch.empty(B, dtype=torch.float32, device="cuda")
    logprob = torch.empty((B, T), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        m.forward_batch_device(ids, probs=probs, bits=bits, logprob=logprob)
    m.sync()
    flat = probs.view(-1, V)
    # every row of both passes sums to one (float64 sums, in chunks of 65536 rows)
    worst = 0.0
    for r0 in range(0, flat.shape[0], 65536):
        worst = max(worst, float((flat[r0:r0 + 65536].double().sum(-1) - 1.0).abs().max()))
    print(f"c5 full: worst |row sum - 1| = {worst:.2e} over {flat.shape[0]} rows")
    assert worst < 5e-5
    assert bool(torch.isfinite(flat[:: 4099]).all())
    # bits per token of all 16384 sequences from the gathered target probabilities
    tp = torch.gather(probs[:, :-1], 2, ids[:, 1:].long()[..., None])[..., 0].double()
    want_bits = (-torch.log2(tp)).mean(1)
    e_bits = float(((bits.double() - want_bits).abs() / want_bits.abs()).max())
    print(f"c5 full: worst bits relative error {e_bits:.2e}")
    assert e_bits < 1e-5
    e_lp = float((logprob[:, :-1].double() - torch.log(tp)).abs().max())
    assert e_lp < 2e-5
    assert bool(torch.isnan(logprob[:, -1]).all())
    # sequences at the pass boundaries against the oracle
    sub = [0, 8191, 8192, B - 1]
    ref = oracle_model(data).forward_all(ids_np[sub]).astype(np.float64)
    p = np.exp(ref - ref.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    got = probs[sub].cpu().numpy()
    e = float(rel_err(got, p).max())
    print(f"c5 full: sequences {sub} max relative error {e:.2e}")
    assert e <= 1e-4
    tgt = ids_np[sub][:, 1:]
    ref_bits = -np.log2(np.take_along_axis(p[:, :-1], tgt[..., None], -1)[..., 0]).mean(1)
    assert np.allclose(bits[sub].cpu().numpy(), ref_bits, rtol=1e-5)


def test_c2_full_size_fp32_only_device():
    import torch
    c = synth.C2
    M, K, N = c["M"], c["K"], c["N"]
    A = ((synth.u64_stream(1, "A", M * K) % np.uint64(255)).astype(np.int64) - 127).astype(np.int8).reshape(M, K)
    W = ((synth.u64_stream(1, "W", N * K) % np.uint64(255)).astype(np.int64) - 127).astype(np.int8).reshape(N, K)
    sc = (1e-3 + 9e-3 * synth.uniform(1, "s", N)).astype(np.float32)  # the benchmark's operands
    dA, dW, ds = (torch.from_numpy(x).cuda() for x in (A, W, sc))
    C1 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    C2 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    acc = torch.empty((M, N), dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    gemm_i8_device(dA, dW, ds, C1, None, stream)  # the timed call: fp32 only
    gemm_i8_device(dA, dW, ds, C2, acc, stream)
    torch.cuda.synchronize()
    assert torch.equal(C1.view(torch.int32), C2.view(torch.int32))
    # C == float(acc) * s over every row, bit for bit
    assert torch.equal(C1.view(torch.int32), (acc.float() * ds[None, :]).view(torch.int32))
    rows = np.unique(np.concatenate([np.arange(128), np.arange(M - 128, M),
                                     (synth.u64_stream(3, "rows", 4096) % np.uint64(M)).astype(np.int64)]))
    Cr, accr = O.gemm_i8_exact(A[rows], W, sc)
    got = C1[torch.from_numpy(rows).cuda()].cpu().numpy()
    assert np.array_equal(got.view(np.uint32), Cr.view(np.uint32))
    assert np.array_equal(acc[torch.from_numpy(rows).cuda()].cpu().numpy(), accr)


def test_batch_over_two_passes():
    """17,000 sequences of 128 tokens: more than the 2^21 tokens of one workspace pass, so the batch runs
    in two and the second starts at sequence 16384. Per-token log-probs and bits per token of sequences
    around that boundary (and the first and last) against the oracle."""
    import torch
    data = model_bytes("c1")
    spec = synth.CONFIGS["c1"]["spec"]
    B, T = 17000, 128
    assert B * T > (1 << 21)
    ids_np = synth.token_ids(7, "two-pass", (B, T), spec.V)
    m = Model(data)
    ids = torch.from_numpy(ids_np).cuda()
    logprob = torch.empty((B, T), dtype=torch.float32, device="cuda")
    bits = torch.empty(B, dtype=torch.float32, device="cuda")
    m.forward_batch_device(ids, logprob=logprob, bits=bits)
    m.sync()
    lp, bt = logprob.cpu().numpy(), bits.cpu().numpy()
    om = oracle_model(data)
    sub = [0, 16383, 16384, 16385, B - 1]
    ref = om.forward_all(ids_np[sub])
    for k, b in enumerate(sub):
        r = ref[k].astype(np.float64)
        mx = r.max(-1, keepdims=True)
        lse = mx[:, 0] + np.log(np.exp(r - mx).sum(-1))
        want = r[np.arange(T - 1), ids_np[b, 1:]] - lse[:-1]
        assert np.abs(lp[b, :-1] - want).max() < 2e-5 * max(1.0, np.abs(want).max()), b
        want_bits = -(want / np.log(2)).mean()
        assert abs(bt[b] - want_bits) < 1e-5 * abs(want_bits), b
