"""The packed K/V ring format's host codec (tests/helpers.kv_pack / kv_unpack), which the GPU tests of the
packed rings compare the engine's ring bytes with: a known answer worked by hand, exactness where the
format is exact, the error bound it promises, and its edge cases."""
import numpy as np

from helpers import kv_pack, kv_unpack


def test_known_answer():
    # amax 1 = 0.5 * 2^1: e = 1 - 23 = -22, mantissas 2^22, -2^22, 2^21, 2^20 (0x400000, 0xC00000,
    # 0x200000, 0x100000) packed low byte first
    w, s = kv_pack(np.array([1.0, -1.0, 0.5, 0.25], np.float32))
    assert w.tolist() == [0x00400000, 0x0000C000, 0x10000020]
    assert s == np.float32(2.0 ** -22)
    assert kv_unpack(w, s).tolist() == [1.0, -1.0, 0.5, 0.25]


def test_exact_where_representable():
    # values on the row's 2^e grid with |m| < 2^23 come back bit for bit, in every slot of a group
    rng = np.random.default_rng(5)
    m = rng.integers(-(1 << 23) + 1, 1 << 23, size=(64, 32))
    m[:, 0] = (1 << 22) + rng.integers(0, 1 << 22, size=64)  # sets amax's binade: E - 23 = e
    x = np.ldexp(m.astype(np.float64), -30).astype(np.float32)
    w, s = kv_pack(x)
    assert np.all(s == np.float32(2.0 ** -30))
    assert np.array_equal(kv_unpack(w, s), x)


def test_error_bound_and_largest_element():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((2000, 32)) * np.exp(rng.uniform(-20, 20, (2000, 1)))).astype(np.float32)
    got = kv_unpack(*kv_pack(x)).astype(np.float64)
    amax = np.abs(x).max(-1, keepdims=True).astype(np.float64)
    # every element within half a mantissa step: 2^e / 2 = 2^(E - 24) <= amax * 2^-23, as amax >= 2^(E - 1)
    assert np.all(np.abs(got - x) <= amax * 2.0 ** -23)
    # the largest element keeps 23 significant bits: relative error at most 2^-23
    i = np.abs(x).argmax(-1)
    big = x[np.arange(len(x)), i].astype(np.float64)
    assert np.all(np.abs(got[np.arange(len(x)), i] - big) <= np.abs(big) * 2.0 ** -23)


def test_edge_cases():
    z, s = kv_pack(np.zeros((3, 8), np.float32))
    assert not z.any() and np.all(kv_unpack(z, s) == 0)
    # a row whose largest element rounds up to 2^23 is clamped to 2^23 - 1
    x = np.array([np.float32(np.nextafter(np.float32(1.0), np.float32(0.0))), 0, 0, 0], np.float32)
    w, s = kv_pack(x)
    assert s == np.float32(2.0 ** -23)
    assert kv_unpack(w, s)[0] == np.float32((2 ** 23 - 1) * 2.0 ** -23)
    # tiny rows keep the scale a normal float (e >= -120)
    w, s = kv_pack(np.array([1e-38, 0, 0, 0], np.float32))
    assert s == np.float32(2.0 ** -120)
