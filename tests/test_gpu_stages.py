"""Stage-level parity: single kernels of the engine given exactly the oracle's inputs (through the stage
hooks, tests/stage_hooks.hip) and compared with the oracle bit for bit, for the stages whose arithmetic
follows the reference's order of operations:

- RMSNorm rows (row_kernel): nn.RMSNormForwardF32 (internal/nn/rmsnorm.go:14-32), DotF32's partial-sum
  order, tails of 8 and of single elements;
- the latch scan (scan_kernel): updateLatch's recurrence (internal/quant/stream.go:195-205);
- attention (attention_kernel under the exact option, attention_wave_kernel for every other head width,
  and the decode kernels attention_step_rk / _lds / plain / wave): attendPosition's scores, FastExp
  softmax and AddScaledF32 (internal/quant/attention.go:82-101), windows and rings;
- the limb expansion (row kernel; decode attention fused with it): digits in [-127, 127], the row scale
  amax/127, the representation bound, and the fused kernel's limbs equal to the row kernel's limbs of
  the same (bit-identical) attention output.
The matrix-core attention kernel is checked at its tolerance against the same oracle output."""
import numpy as np
import pytest
import torch

import stage_hooks as H
from helpers import assert_close, kv_pack, kv_unpack
from mignon_ai_amd import engine_option
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.cpu().numpy()


def pad_cols(x, Dp):
    out = np.zeros(x.shape[:-1] + (Dp,), np.float32)
    out[..., :x.shape[-1]] = x
    return out


def p64(D):
    return (D + 63) // 64 * 64


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture
def restore_attention():
    prev = engine_option("attention", "auto")
    yield
    engine_option("attention", prev)


def _rows(rng, M, D):
    # rows of different magnitudes, one all-zero row and one with a single non-zero element
    x = rng.standard_normal((M, D)).astype(np.float32)
    x *= (10.0 ** rng.uniform(-3, 3, (M, 1))).astype(np.float32)
    x[min(3, M - 1)] = 0
    x[min(5, M - 1)] = 0
    x[min(5, M - 1), D // 2] = -7.25
    return x


@pytest.mark.parametrize("D", [1, 7, 8, 15, 16, 24, 100, 384, 1000, 1024])
def test_rmsnorm_rows_bitwise(D):
    rng = np.random.default_rng(D)
    M, Dp = 37, p64(D)
    x = _rows(rng, M, D)
    gamma = rng.uniform(0.5, 1.5, D).astype(np.float32)
    xd, gd = dev(pad_cols(x, Dp)), dev(pad_cols(gamma, Dp))
    nout = torch.full((M, Dp), float("nan"), device="cuda")
    H.call("mgt_row", H.ptr(xd), M, D, Dp, H.ptr(gd), H.ptr(nout), None, None)
    got = host(nout)
    ref = np.stack([O.rmsnorm(x[m], gamma) for m in range(M)])
    assert np.array_equal(bits(got[:, :D]), bits(ref))
    assert not got[:, D:].any()


def _unpack_limbs(xl, M, Dp):
    """[ceil(M/16)][Dp/64][3][1 KiB] operand layout -> digits [3][M][Dp]: lane 16g + token holds channels
    64ks + 16g .. + 15 of that token."""
    kc = Dp // 64
    a = xl.reshape(-1, kc, 3, 4, 16, 16)  # tile, K step, limb, g, token, byte
    d = a.transpose(2, 0, 4, 1, 3, 5).reshape(3, -1, Dp)  # limb, tile*16 + token, 64ks + 16g + byte
    return d[:, :M].astype(np.int64)


def _split_limbs(x, inv):
    """The engine's digit definition (split_limbs in csrc/common.hpp), float32 throughout."""
    y = np.float32(x * inv)
    q0 = np.clip(np.rint(y), -127, 127).astype(np.float32)
    y1 = np.float32((y - q0) * np.float32(254))
    q1 = np.clip(np.rint(y1), -127, 127).astype(np.float32)
    y2 = np.float32((y1 - q1) * np.float32(254))
    q2 = np.clip(np.rint(y2), -127, 127).astype(np.float32)
    return np.stack([q0, q1, q2]).astype(np.int64)


@pytest.mark.parametrize("D", [64, 100, 384, 1024])
def test_limb_expansion(D):
    rng = np.random.default_rng(100 + D)
    M, Dp = 35, p64(D)
    x = _rows(rng, M, D)
    xl = torch.zeros(((M + 15) // 16) * 3 * Dp * 16, dtype=torch.int8, device="cuda")
    xs = torch.zeros(M, device="cuda")
    xd = dev(pad_cols(x, Dp))
    H.call("mgt_row", H.ptr(xd), M, D, Dp, None, None, H.ptr(xl), H.ptr(xs))
    q = _unpack_limbs(host(xl), M, Dp)
    s = host(xs)
    amax = np.abs(x).max(1)
    nz = amax >= 1e-30
    assert np.array_equal(bits(s[nz]), bits(amax[nz] / np.float32(127)))
    assert not s[~nz].any() and not q[:, ~nz].any()
    assert np.abs(q).max() <= 127 and not q[:, :, D:].any()
    inv = np.where(nz, np.float32(127) / np.where(nz, amax, 1), 0).astype(np.float32)
    assert np.array_equal(q[:, :, :D], _split_limbs(x, inv[:, None]))
    rec = (q[0] + q[1] / 254.0 + q[2] / 254.0 ** 2)[:, :D] * s[:, None].astype(np.float64)
    bound = s.astype(np.float64) * (0.5 / 64516 + 2.0 ** -23 * 127) + 1e-45
    assert np.all(np.abs(rec - x) <= bound[:, None])


@pytest.mark.parametrize("B,T,D", [(3, 37, 100), (2, 128, 384), (1, 5, 1)])
def test_latch_scan_bitwise(B, T, D):
    rng = np.random.default_rng(T * D)
    Dp = p64(D)
    lam = rng.uniform(0, 1, (B, T, D)).astype(np.float32)
    lam[:, ::7] = 0.0  # g = n exactly
    lam[:, 3::11] = 1.0  # g unchanged
    nf = rng.standard_normal((B, T, D)).astype(np.float32)
    ld, nd = dev(pad_cols(lam, Dp)), dev(pad_cols(nf, Dp))
    g = torch.full((B * T, Dp), float("nan"), device="cuda")
    H.call("mgt_latch_scan", H.ptr(ld), H.ptr(nd), B, T, D, Dp, H.ptr(g))
    ref = O.latch_seq(lam, nf).reshape(B * T, D)
    assert np.array_equal(bits(host(g)[:, :D]), bits(ref))


ATT_CASES = [
    # D, heads, T, window, cap
    (64, 2, 40, 0, 128),    # dh 32, full causal
    (96, 4, 33, 5, 128),    # dh 24, window 5
    (128, 8, 64, 12, 64),   # dh 16, window 12
    (48, 3, 50, 0, 16),     # ring of 16 < T
    (224, 4, 20, 0, 128),   # dh 56 (the pro preset's width): the wave kernel
    (288, 4, 20, 7, 128),   # dh 72 (the xl preset's width): the wave kernel
    (40, 1, 9, 1, 128),     # window 1: each position attends to itself only
]


def _qkv(rng, B, T, D):
    return (rng.standard_normal((B, T, 3 * D)) * 2).astype(np.float32)


@pytest.mark.parametrize("D,heads,T,window,cap", ATT_CASES)
def test_attention_bitwise(restore_attention, D, heads, T, window, cap):
    rng = np.random.default_rng(D + T)
    B, Dp = 3, p64(D)
    qkv = _qkv(rng, B, T, D)
    ref = O.attend_seq(qkv, heads, window, cap)
    if window == 1:
        assert np.array_equal(bits(ref), bits(qkv[:, :, 2 * D:]))
    q = dev(qkv.reshape(B * T, 3 * D))
    for option, kernel in (("exact", 0), ("exact", 1)):
        engine_option("attention", option)
        att = torch.full((B * T, Dp), float("nan"), device="cuda")
        H.call("mgt_attention", H.ptr(q), B, T, D, Dp, heads, window, cap, H.ptr(att), kernel)
        got = host(att)[:, :D].reshape(B, T, D)
        assert np.array_equal(bits(got), bits(ref)), (option, kernel)
    # the matrix-core kernel, where it applies: its own summation order, within the parity bar
    engine_option("attention", "mfma")
    att = torch.full((B * T, Dp), float("nan"), device="cuda")
    H.call("mgt_attention", H.ptr(q), B, T, D, Dp, heads, window, cap, H.ptr(att), 0)
    assert_close(host(att)[:, :D].reshape(B, T, D).astype(np.float64), ref, what="mfma attention")


STEP_CASES = [
    # D, heads, window, cap, kernels
    (64, 2, 0, 32, (0, 1, 2)),    # dh 32, cache <= 64: attention_step_rk, the fused rows kernel
    (256, 8, 0, 64, (0, 1, 2)),   # c4's shape
    (64, 2, 0, 128, (0, 1)),      # the LDS kernel
    (128, 2, 0, 256, (0, 1)),     # dh 64, 256 positions: the plain kernel
    (96, 4, 6, 64, (0, 1, 2)),    # window 6 inside a cache of 64
    (224, 4, 0, 40, (0, 1)),      # dh 56: the wave kernel
]


@pytest.mark.parametrize("D,heads,window,cap,kernels", STEP_CASES)
def test_decode_attention_bitwise(D, heads, window, cap, kernels):
    rng = np.random.default_rng(D * cap + window)
    dh, Dp = D // heads, p64(D)
    # sessions at positions 0, 1, cap - 1, cap, cap + 5 and 2cap + 3 (the ring wrapped)
    pos = np.array([0, 1, cap - 1, cap, cap + 5, 2 * cap + 3], np.int32)
    S, T = len(pos), int(pos.max()) + 1
    qkv = _qkv(rng, S, T, D)
    ref = O.attend_seq(qkv, heads, window, cap)  # [S][T][D]
    want = np.stack([ref[i, p] for i, p in enumerate(pos)])
    # slots outside a session's span hold stale values (as in a ring that has been written before)
    kr = (rng.standard_normal((S, heads, cap, dh)) * 1e3).astype(np.float32)
    vr = (rng.standard_normal((S, heads, cap, dh)) * 1e3).astype(np.float32)
    for i, p in enumerate(pos):
        for j in range(max(0, p - cap + 1), p):  # the ring before position p (slot j % cap)
            kr[i, :, j % cap] = qkv[i, j, D:2 * D].reshape(heads, dh)
            vr[i, :, j % cap] = qkv[i, j, 2 * D:].reshape(heads, dh)
    rows = np.stack([qkv[i, p] for i, p in enumerate(pos)])
    pd, rd = dev(pos), dev(rows)
    for kernel in kernels:
        k, v = dev(kr), dev(vr)
        att = torch.full((S, Dp), float("nan"), device="cuda")
        xl = torch.zeros(((S + 15) // 16) * 3 * Dp * 16, dtype=torch.int8, device="cuda")
        xs = torch.zeros(S, device="cuda")
        H.call("mgt_attention_step", H.ptr(pd), H.ptr(rd), H.ptr(k), H.ptr(v), S, D, Dp, heads, window, cap,
               H.ptr(att), H.ptr(xl), H.ptr(xs), kernel)
        for i, p in enumerate(pos):  # the new key and value went to slot p % cap
            assert np.array_equal(host(k)[i, :, p % cap], rows[i, D:2 * D].reshape(heads, dh))
            assert np.array_equal(host(v)[i, :, p % cap], rows[i, 2 * D:].reshape(heads, dh))
        if kernel == 2:
            # limbs of the output: those the row kernel makes of the oracle's (bit-identical) output
            rl = torch.zeros_like(xl)
            rs = torch.zeros_like(xs)
            wd = dev(pad_cols(want, Dp))
            H.call("mgt_row", H.ptr(wd), S, D, Dp, None, None, H.ptr(rl), H.ptr(rs))
            assert np.array_equal(host(xl), host(rl)) and np.array_equal(bits(host(xs)), bits(host(rs)))
        else:
            assert np.array_equal(bits(host(att)[:, :D]), bits(want)), kernel


PACKED_CASES = [
    # D, heads, window, cap
    (64, 2, 0, 32),     # dh 32
    (256, 8, 0, 64),    # c4's shape
    (96, 4, 6, 64),     # window 6 inside a cache of 64
    (80, 4, 0, 48),     # dh 20: groups of a row not 16-byte aligned
    (512, 8, 0, 64),    # dh 64
]


@pytest.mark.parametrize("D,heads,window,cap", PACKED_CASES)
@pytest.mark.parametrize("kernel", [0, 2, 3])
def test_decode_attention_packed_rings(D, heads, window, cap, kernel):
    """Decode attention on packed rings (attention_step_rk through launch_attention_step, and the rows
    kernel with cached and with streamed ring loads; the streamed form is taken for heads of up to 32):
    the output is bit-identical to the reference order over the rings' decoded values (the current
    position's key and value in fp32), and the new row is written exactly as the host codec packs it."""
    rng = np.random.default_rng(D * cap + window + 7)
    dh, Dp = D // heads, p64(D)
    pos = np.array([0, 1, cap - 1, cap, cap + 5, 2 * cap + 3], np.int32)
    S, T = len(pos), int(pos.max()) + 1
    qkv = _qkv(rng, S, T, D)
    # stale rows outside a span, as in a ring written before
    kr = (rng.standard_normal((S, heads, cap, dh)) * 1e3).astype(np.float32)
    vr = (rng.standard_normal((S, heads, cap, dh)) * 1e3).astype(np.float32)
    want = np.empty((S, D), np.float32)
    for i, p in enumerate(pos):
        seq = qkv[i].copy()
        for j in range(max(0, p - cap + 1), p):  # the ring before position p (slot j % cap)
            kr[i, :, j % cap] = seq[j, D:2 * D].reshape(heads, dh)
            vr[i, :, j % cap] = seq[j, 2 * D:].reshape(heads, dh)
            # the oracle sees the values the ring holds
            seq[j, D:2 * D] = kv_unpack(*kv_pack(seq[j, D:2 * D].reshape(heads, dh))).ravel()
            seq[j, 2 * D:] = kv_unpack(*kv_pack(seq[j, 2 * D:].reshape(heads, dh))).ravel()
        want[i] = O.attend_seq(seq[None, :p + 1], heads, window, cap)[0, p]
    kw, ks = kv_pack(kr)
    vw, vs_ = kv_pack(vr)
    rows = np.stack([qkv[i, p] for i, p in enumerate(pos)])
    pd, rd = dev(pos), dev(rows)
    k, v = dev(kw.view(np.int32)), dev(vw.view(np.int32))
    kscl, vscl = dev(ks), dev(vs_)
    att = torch.full((S, Dp), float("nan"), device="cuda")
    xl = torch.zeros(((S + 15) // 16) * 3 * Dp * 16, dtype=torch.int8, device="cuda")
    xs = torch.zeros(S, device="cuda")
    H.call("mgt_attention_step_packed", H.ptr(pd), H.ptr(rd), H.ptr(k), H.ptr(v), H.ptr(kscl), H.ptr(vscl), S, D,
           Dp, heads, window, cap, H.ptr(att), H.ptr(xl), H.ptr(xs), kernel)
    nk, nv = kv_pack(rows[:, D:2 * D].reshape(S, heads, dh)), kv_pack(rows[:, 2 * D:].reshape(S, heads, dh))
    gk, gv = host(k).view(np.uint32), host(v).view(np.uint32)
    for i, p in enumerate(pos):  # the new key and value went to slot p % cap, packed as the codec packs them
        assert np.array_equal(gk[i, :, p % cap], nk[0][i]) and np.array_equal(host(kscl)[i, :, p % cap], nk[1][i])
        assert np.array_equal(gv[i, :, p % cap], nv[0][i]) and np.array_equal(host(vscl)[i, :, p % cap], nv[1][i])
    if kernel >= 2:
        rl = torch.zeros_like(xl)
        rs = torch.zeros_like(xs)
        wd = dev(pad_cols(want, Dp))
        H.call("mgt_row", H.ptr(wd), S, D, Dp, None, None, H.ptr(rl), H.ptr(rs))
        assert np.array_equal(host(xl), host(rl)) and np.array_equal(bits(host(xs)), bits(host(rs)))
    else:
        assert np.array_equal(bits(host(att)[:, :D]), bits(want))


@pytest.mark.parametrize("D,heads", [(96, 4), (256, 8), (64, 1), (32, 2), (16, 2), (8, 2)])
def test_export_kv_packed(D, heads):
    """A prefill's K/V export into packed rings: the last min(len, cap) positions of each sequence, each
    (head, position) row packed as the host codec packs it; other slots untouched. Head widths 24 (the LDS
    kernel) and 32, 64, 16, 8, 4 (the DPP kernel: a row's groups on an aligned half-row, row, quad, pair,
    single lane)."""
    rng = np.random.default_rng(11 + D)
    B, T, cap = 5, 40, 16
    dh = D // heads
    qkv = _qkv(rng, B, T, D)
    lens = np.array([1, 7, 16, 17, 40], np.int32)
    words = rng.integers(0, 1 << 32, size=(2, B, heads, cap, 3 * dh // 4), dtype=np.uint64).astype(np.uint32)
    scl = rng.standard_normal((2, B, heads, cap)).astype(np.float32)
    dk, dv = dev(words[0].view(np.int32)), dev(words[1].view(np.int32))
    dks, dvs = dev(scl[0]), dev(scl[1])
    dl, dq = dev(lens), dev(qkv)  # referenced until the hook returns
    H.call("mgt_export_kv_packed", B, T, D, heads, cap, H.ptr(dl), H.ptr(dq), H.ptr(dk), H.ptr(dv), H.ptr(dks),
           H.ptr(dvs))
    got_w = [host(dk).view(np.uint32), host(dv).view(np.uint32)]
    got_s = [host(dks), host(dvs)]
    for part in range(2):
        ew, es = words[part].copy(), scl[part].copy()
        for b in range(B):
            for p in range(max(0, lens[b] - cap), lens[b]):
                w, s_ = kv_pack(qkv[b, p, (1 + part) * D:(2 + part) * D].reshape(heads, dh))
                ew[b, :, p % cap], es[b, :, p % cap] = w, s_
        assert np.array_equal(got_w[part], ew) and np.array_equal(bits(got_s[part]), bits(es))
