"""Pins of the oracle's kernel-level restatements (CPU).

Each pin is chosen so that a plausible mistake fails it: the reference's own known answers and
tolerances, closed forms, and inputs on which the reference's accumulation order, rounding mode or
fused/unfused choice changes the bits."""
import math

import numpy as np
import pytest

from oracle import oracle as O

F = np.float32


def bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


# ---- quant.NewTensorF32 (internal/quant/tensor.go:12-42) -------------------------------------------

def test_quantizer_known_answer():
    # internal/quant/tensor_test.go:7-22: dequantised within 0.05; closed form scale = 2/127 in fp32
    w = np.array([-1.5, -0.75, 0.0, 0.33, 1.25, 2.0], np.float32)
    q, s = O.quantize(w)
    assert bits(s) == 0x3c810204
    assert q.tolist() == [-95, -48, 0, 21, 79, 127]
    assert np.all(np.abs(q.astype(np.float32) * s - w) <= 0.05)


def test_quantizer_rounds_half_away_and_special_tensors():
    # 127 sets scale 1, so w/scale is exact: math.Round sends x.5 away from zero (banker's would not)
    q, s = O.quantize(np.array([127.0, 0.5, -0.5, 2.5, -2.5, 126.5], np.float32))
    assert s == 1.0 and q.tolist() == [127, 1, -1, 3, -3, 127]
    q, s = O.quantize(np.zeros(7, np.float32))
    assert s == 1.0 and not q.any()
    q, s = O.quantize(np.zeros(0, np.float32))
    assert s == 0.0


# ---- kernels.DotInt8F32 (internal/kernels/int8.go:8-29, vec_amd64.s:603-679) ----------------------

def test_dot_i8_reference_tolerance():
    # TestDotInt8F32MatchesReference (internal/kernels/int8_test.go:15-38)
    rng = np.random.default_rng(1)
    for n in range(101):
        x = rng.standard_normal(n).astype(np.float32)
        w = rng.integers(-128, 128, n).astype(np.int8)
        if n:
            w[0], w[-1] = -128, 127
        want = float(np.dot(x.astype(np.float64), w.astype(np.float64)))
        mag = float(np.abs(x.astype(np.float64) * w).sum())
        got = float(O.dot_i8_f32(x, w))
        assert abs(got - want) <= 1e-5 * mag + 1e-6, n


def test_dot_i8_exact_on_integers():
    rng = np.random.default_rng(2)
    for n in (1, 7, 31, 32, 33, 384, 1040):
        x = rng.integers(-127, 128, n)
        w = rng.integers(-127, 128, n)
        assert O.dot_i8_f32(x.astype(np.float32), w.astype(np.int8)) == np.float32(int(np.dot(x, w)))


def test_dot_i8_accumulator_tree():
    # 2^24 in lane 0 of Y0 plus 1s in lane 0 of Y4 and Y5: (Y0+Y1)+(Y4+Y5) keeps both (2^24 + 2), a
    # sequential sum or the 4-accumulator pure-Go fallback rounds each 1 away (2^24).
    x = np.zeros(32, np.float32)
    x[0], x[16], x[24] = 2.0 ** 24, 1.0, 1.0
    assert O.dot_i8_f32(x, np.ones(32, np.int8)) == F(2.0 ** 24 + 2)


def test_dot_i8_unfused_tail():
    # element 33 is in the scalar tail: product rounded, then added (an FMA would keep 2^-24)
    x = np.zeros(33, np.float32)
    x[0] = -1.0
    x[32] = 1.0 + 2.0 ** -12
    w = np.ones(33, np.int8)
    # (1+2^-12)*1 is exact, so fused and unfused agree here; use w=3 to force a product rounding
    w[32] = 3
    got = O.dot_i8_f32(x, w)
    p = F(x[32] * F(3))
    assert got == F(p + F(-1.0))


def test_matvec_reference_case():
    # TestMatVecInt8 (internal/kernels/int8_test.go:52-77): rows 5, cols 37, stride 40, 1e-4 absolute
    rng = np.random.default_rng(2)
    w = rng.integers(-128, 128, 5 * 40).astype(np.int8)
    x = rng.standard_normal(37).astype(np.float32)
    bias = np.array([0.5, -1, 2, 0, 3], np.float32)
    y = O.matvec_i8(w, 40, 0.01, x, bias, rows=5)
    for r in range(5):
        want = bias[r] + 0.01 * np.dot(w[r * 40:r * 40 + 37].astype(np.float64), x.astype(np.float64))
        assert abs(y[r] - want) <= 1e-4


# ---- kernels.DotF32 (dotProductASM_F32, vec_amd64.s:4-63) -----------------------------------------

def test_dot_f32_tree_and_tail():
    # v[0] = a0[0]+a1[0] = 2^24+1 rounds to 2^24, v[4] = 1+1 = 2, fold v[0]+v[4] = 2^24+2 exactly;
    # summing left to right gives 2^24.
    x = np.zeros(16, np.float32)
    x[0], x[4], x[8], x[12] = 2.0 ** 24, 1.0, 1.0, 1.0
    assert O.dot_f32(x, np.ones(16, np.float32)) == F(2.0 ** 24 + 2)
    # scalar tail: mul then add. x*x = 1 + 2^-11 + 2^-24 rounds to 1 + 2^-11 (tie to even), then -1:
    # 2^-11. An FMA would return 2^-11 + 2^-24.
    x = np.zeros(17, np.float32)
    y = np.zeros(17, np.float32)
    x[0], y[0] = -1.0, 1.0
    x[16] = y[16] = 1.0 + 2.0 ** -12
    assert O.dot_f32(x, y) == F(2.0 ** -11)


def test_dot_f32_fma_in_chunks():
    # inside a 16-chunk the accumulation is fused: fma(x, x, 0) then the fold; with one element the
    # product 1+2^-11+2^-24 is rounded once by the FMA into the zero accumulator: same as unfused,
    # so check the fused path with a non-zero accumulator: lane 0 gets -1 first, then (1+2^-12)^2.
    x = np.zeros(32, np.float32)
    y = np.zeros(32, np.float32)
    x[0], y[0] = -1.0, 1.0
    x[16] = y[16] = 1.0 + 2.0 ** -12
    assert O.dot_f32(x, y) == F(2.0 ** -11 + 2.0 ** -24)


# ---- FastExpF32 / vecExpASM_F32 (vec_ops.go:104-138, vec_amd64.s:281-430) --------------------------

def test_fast_exp_accuracy_and_special_values():
    xs = np.linspace(-87, 87, 20001, dtype=np.float32)
    got = np.array([O.fast_exp(x) for x in xs], np.float64)
    ref = np.exp(xs.astype(np.float64))
    # reference bar 1e-4 (accuracy_test.go:10-33); the degree-5 polynomial measures 3.3e-6, and dropping
    # its last term would give ~4e-5
    assert np.max(np.abs(got - ref) / ref) < 5e-6
    assert O.fast_exp(0.0) == 1.0
    assert O.fast_exp(-100.0) == 0.0  # clamped to -88: k = -127 builds a zero 2^k
    assert O.fast_exp(100.0) == O.fast_exp(88.0)  # the vector path clamps; it does not return MaxFloat32
    assert O.fast_exp(88.0) == pytest.approx(math.exp(88.0), rel=1e-5)


def test_sigmoid_clamped_bounds():
    assert O.sigmoid_clamped(15.0) == F(1.0 / (1.0 + F(math.exp(-15.0))))
    assert O.sigmoid_clamped(15.0) != 1.0
    assert O.sigmoid_clamped(np.nextafter(F(15), F(16))) == 1.0
    assert O.sigmoid_clamped(np.nextafter(F(-15), F(-16))) == 0.0
    assert O.sigmoid_clamped(0.0) == 0.5


# ---- RMSNorm, softmax, AddScaled ------------------------------------------------------------------

@pytest.mark.parametrize("D", [1, 7, 8, 16, 24, 96, 128, 384])
def test_rmsnorm_closed_form(D):
    g = np.linspace(0.5, 1.5, D).astype(np.float32)
    c = F(3.0)
    out = O.rmsnorm(np.full(D, c), g)
    rms = F(math.sqrt(float(F(F(D * 9.0) / F(D)) + F(1e-5))))
    inv = F(1.0) / rms
    assert np.array_equal(bits(out), bits(F(c * inv) * g))
    rng = np.random.default_rng(D)
    x = rng.standard_normal(D).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-5) * g
    assert np.allclose(O.rmsnorm(x, g), ref, rtol=2e-6, atol=1e-7)
    assert not O.rmsnorm(np.zeros(D, np.float32), g).any()


def test_softmax():
    rng = np.random.default_rng(4)
    for n in (1, 5, 8, 9, 64):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        p = O.softmax(x)
        e = np.exp(x.astype(np.float64) - x.max())
        assert np.allclose(p, e / e.sum(), rtol=1e-5, atol=1e-7)
        assert abs(float(p.astype(np.float64).sum()) - 1) < 1e-6
    assert np.all(O.softmax(np.full(6, 2.5, np.float32)) == F(1 / 6))


def test_add_scaled_fused_chunks_unfused_tail():
    a = F(1.0 + 2.0 ** -12)
    y = np.full(9, -1.0, np.float32)
    x = np.full(9, a, np.float32)
    out = O.add_scaled(y, x, a)
    assert out[0] == F(2.0 ** -11 + 2.0 ** -24)  # fused (8-chunk)
    assert out[8] == F(2.0 ** -11)               # scalar tail: product rounded first


def test_latch_base_closed_form():
    # sigmoid(base_d) reproduces decay_d = 2^(-1/T_d), T geometric from 1.5 to 64 (ca/layout.go:60-85)
    for D in (1, 2, 32, 384):
        b = O.latch_base(D).astype(np.float64)
        T = np.full(D, 1.5) if D == 1 else 1.5 * (64 / 1.5) ** (np.arange(D) / (D - 1))
        assert np.allclose(1 / (1 + np.exp(-b)), 2.0 ** (-1 / T), rtol=1e-6)


def test_avx2_dot_paths_match_scalar_restatement():
    """The oracle's AVX2 dot kernels (used for speed) give the scalar restatement's exact bits."""
    if not O.has_avx2():
        pytest.skip("host has no AVX2/FMA")
    rng = np.random.default_rng(12)
    try:
        for n in list(range(0, 70)) + [96, 127, 128, 384, 1000, 1152]:
            x = (rng.standard_normal(n) * rng.choice([1e-3, 1, 1e3])).astype(np.float32)
            y = rng.standard_normal(n).astype(np.float32)
            w = rng.integers(-128, 128, n).astype(np.int8)
            O.force_scalar(False)
            a, b = O.dot_f32(x, y), O.dot_i8_f32(x, w)
            O.force_scalar(True)
            assert bits(a) == bits(O.dot_f32(x, y)) and bits(b) == bits(O.dot_i8_f32(x, w)), n
    finally:
        O.force_scalar(False)


# ---- the latch recurrence and attention over whole sequences (the stage-level pins' oracle) --------

def test_latch_seq_closed_forms():
    rng = np.random.default_rng(21)
    B, T, D = 2, 19, 13
    nf = rng.standard_normal((B, T, D)).astype(np.float32)
    # lambda = 0: the latch is the normalised cell itself; lambda = 1: it stays at its zero start
    assert np.array_equal(bits(O.latch_seq(np.zeros((B, T, D), np.float32), nf)), bits(nf))
    assert not O.latch_seq(np.ones((B, T, D), np.float32), nf).any()
    # constant lambda and cell: g_t = n (1 - lambda^(t+1))
    lam = np.full((1, T, 1), 0.75, np.float32)
    g = O.latch_seq(lam, np.full((1, T, 1), 2.0, np.float32))[0, :, 0]
    assert np.allclose(g, 2.0 * (1 - 0.75 ** np.arange(1, T + 1)), rtol=1e-6)
    # random inputs against the float64 recurrence
    lam = rng.uniform(0, 1, (B, T, D)).astype(np.float32)
    g = O.latch_seq(lam, nf)
    ref = np.zeros((B, D))
    for t in range(T):
        ref = lam[:, t] * ref + (1 - lam[:, t].astype(np.float64)) * nf[:, t]
        assert np.allclose(g[:, t], ref, rtol=1e-5, atol=1e-6)


def test_latch_seq_rounds_each_product():
    # updateLatch rounds lam*g and (1-lam)*n separately (stream.go:202; Go fuses nothing on amd64): on
    # these inputs a fused multiply-add gives a different float32
    rng = np.random.default_rng(5)
    hits = 0
    for _ in range(200):
        lam = rng.uniform(0, 1, (1, 2, 1)).astype(np.float32)
        n = rng.standard_normal((1, 2, 1)).astype(np.float32)
        g0 = F(F(F(1) - lam[0, 0, 0]) * n[0, 0, 0])
        b = F(F(F(1) - lam[0, 1, 0]) * n[0, 1, 0])
        sep = F(F(lam[0, 1, 0] * g0) + b)
        fused = F(float(lam[0, 1, 0]) * float(g0) + float(b))
        got = O.latch_seq(lam, n)[0, 1, 0]
        assert bits(got) == bits(sep)
        hits += bits(sep) != bits(fused)
    assert hits > 0


def _attn_f64(qkv, heads, window, cap):
    B, T, D3 = qkv.shape
    D = D3 // 3
    dh = D // heads
    out = np.zeros((B, T, D))
    for b in range(B):
        for t in range(T):
            lo = max(t - window + 1 if window > 0 else 0, t - cap + 1, 0)
            for h in range(heads):
                sl = slice(h * dh, (h + 1) * dh)
                q = qkv[b, t, sl].astype(np.float64)
                k = qkv[b, lo:t + 1, D:2 * D][:, sl].astype(np.float64)
                v = qkv[b, lo:t + 1, 2 * D:][:, sl].astype(np.float64)
                s = k @ q / np.sqrt(dh)
                p = np.exp(s - s.max())
                out[b, t, sl] = (p / p.sum()) @ v
    return out


@pytest.mark.parametrize("D,heads,T,window,cap", [(16, 2, 12, 0, 128), (24, 3, 20, 4, 128), (12, 1, 30, 0, 8),
                                                 (56, 1, 9, 0, 128), (72, 4, 15, 6, 10)])
def test_attend_seq_against_float64(D, heads, T, window, cap):
    rng = np.random.default_rng(D + T)
    qkv = rng.standard_normal((2, T, 3 * D)).astype(np.float32)
    got = O.attend_seq(qkv, heads, window, cap)
    assert np.allclose(got, _attn_f64(qkv, heads, window, cap), rtol=2e-5, atol=2e-6)


def test_attend_seq_special_cases():
    rng = np.random.default_rng(8)
    D, T = 24, 11
    qkv = rng.standard_normal((1, T, 3 * D)).astype(np.float32)
    v = qkv[:, :, 2 * D:]
    # one attended position (position 0, window 1, a ring of 1): the output is that value, bit for bit
    assert np.array_equal(bits(O.attend_seq(qkv, 2, 0, 128)[:, 0]), bits(v[:, 0]))
    for window, cap in ((1, 128), (0, 1)):
        assert np.array_equal(bits(O.attend_seq(qkv, 3, window, cap)), bits(v))
    # equal keys: uniform weights, the output is the mean of the attended values
    same = qkv.copy()
    same[:, :, D:2 * D] = same[:, :1, D:2 * D]
    got = O.attend_seq(same, 2, 0, 128)
    mean = np.cumsum(v.astype(np.float64), axis=1) / np.arange(1, T + 1)[None, :, None]
    assert np.allclose(got, mean, rtol=1e-5, atol=1e-6)
    # a window of w equals a ring of w positions
    assert np.array_equal(bits(O.attend_seq(qkv, 2, 4, 128)), bits(O.attend_seq(qkv, 2, 0, 4)))
