"""Config-2 INT8 GEMM through the C ABI against the oracle's exact integer GEMM.

Bar: int32 accumulators bit-exact; fp32 outputs bit-exact (the reference's DotInt8F32 on integer
activations is exact while sum|a*w| < 2^24, then MatVecInt8 multiplies once by the scale)."""
import numpy as np
import pytest

from mignon_ai_amd import gemm_i8, synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _operands(M, K, N, seed, lo=-127, hi=127):
    A = (synth.u64_stream(seed, "A", M * K) % np.uint64(hi - lo + 1)).astype(np.int64) + lo
    W = (synth.u64_stream(seed, "W", N * K) % np.uint64(hi - lo + 1)).astype(np.int64) + lo
    s = (1e-3 + 9e-3 * synth.uniform(seed, "s", N)).astype(np.float32)
    return A.astype(np.int8).reshape(M, K), W.astype(np.int8).reshape(N, K), s


@pytest.mark.parametrize("M,K,N", [(64, 384, 512), (1, 384, 512), (100, 37, 5), (130, 100, 130), (257, 1152, 256),
                                   (64, 64, 128), (3, 1, 1)])
def test_gemm_small_exact(M, K, N):
    A, W, s = _operands(M, K, N, 11 + M + K + N)
    A[0, 0] = -128
    W[0, -1] = -128
    C, acc = gemm_i8(A, W, s, want_acc=True)
    Cr, accr = O.gemm_i8_exact(A, W, s)
    assert np.array_equal(acc, accr)
    assert np.array_equal(C.view(np.uint32), Cr.view(np.uint32))


def test_gemm_matches_faithful_dot():
    # the oracle's DotInt8F32 restatement (AVX2 accumulation order) on integer activations equals the
    # exact integer result at the config-2 width, so the GPU result is the reference's own result
    A, W, s = _operands(8, 384, 64, 5)
    C = gemm_i8(A, W, s)
    for m in range(8):
        ref = O.matvec_i8(W.ravel(), 384, 1.0, A[m].astype(np.float32), rows=64) * 1.0
        want = np.array([np.float32(ref[n]) * s[n] for n in range(64)], np.float32)
        assert np.array_equal(C[m].view(np.uint32), want.view(np.uint32))


def test_gemm_config2_full():
    c = synth.C2
    M, K, N = c["M"], c["K"], c["N"]
    A, W, s = _operands(M, K, N, 2)
    C, acc = gemm_i8(A, W, s, want_acc=True)
    rows = np.unique(np.concatenate([np.arange(64), np.arange(M - 64, M),
                                     (synth.u64_stream(2, "rows", 2048) % np.uint64(M)).astype(np.int64)]))
    Cr, accr = O.gemm_i8_exact(A[rows], W, s)
    assert np.array_equal(acc[rows], accr)
    assert np.array_equal(C[rows].view(np.uint32), Cr.view(np.uint32))
    # size-independent property over every row: C == float(acc) * s bit-exactly, and column sums of the
    # int32 accumulators equal (sum over rows of A) . W computed in int64
    assert np.array_equal(C.view(np.uint32), (acc.astype(np.float32) * s[None, :]).view(np.uint32))
    colsum = acc.astype(np.int64).sum(axis=0)
    want = A.astype(np.int64).sum(axis=0) @ W.astype(np.int64).T
    assert np.array_equal(colsum, want)


@pytest.mark.parametrize("M,K,N", [(1000, 384, 512), (256, 64, 130), (128, 1152, 256)])
def test_gemm_fp32_only(M, K, N):
    """Without the int32 output, whole 64 x 128 tiles leave through LDS as row segments (the config-2
    bench's call); partial tiles (the last rows, the last channels) take the direct stores. Both
    bit-exact."""
    A, W, s = _operands(M, K, N, 17 + M + N)
    C = gemm_i8(A, W, s)
    Cr, _ = O.gemm_i8_exact(A, W, s)
    assert np.array_equal(C.view(np.uint32), Cr.view(np.uint32))
