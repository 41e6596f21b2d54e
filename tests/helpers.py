"""Shared test helpers: seeded models, the oracle, the parity tolerance."""
from __future__ import annotations

import functools
import os

import numpy as np

from mignon_ai_amd import mgnn, synth
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")

# The north-star tolerance for dequantised fp32 activations and logits: 1e-4 relative, measured per
# element against max(|ref|, rms of the reference row) so that near-zero logits are not held to an
# absolute 1e-12.
RTOL = 1e-4


def rel_err(got, ref, axis=-1):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=axis, keepdims=True))
    denom = np.maximum(np.abs(ref), rms)
    denom = np.where(denom == 0, 1.0, denom)
    return np.abs(got - ref) / denom


def assert_close(got, ref, rtol=RTOL, what="values"):
    e = rel_err(got, ref)
    worst = float(e.max()) if e.size else 0.0
    assert worst <= rtol, f"{what}: max relative error {worst:.3e} > {rtol:.0e}"
    return worst


def kv_pack(x):
    """The packed K/V ring format (the engine's packed session rings; no reference counterpart): each row
    x[..., :dh] (dh a multiple of 4) as dh/4 groups of three uint32 words holding four 24-bit
    two's-complement mantissas m, and one scale 2^e per row, so that the element is m * 2^e. e = E - 23 for
    the row's largest magnitude amax = f * 2^E (f in [0.5, 1)), at least -120; m = round half to even of
    x * 2^-e, clamped to +-(2^23 - 1). Returns (words uint32 [..., 3 dh / 4], scales float32 [...])."""
    x = np.asarray(x, np.float32)
    e = np.maximum(np.frexp(np.abs(x).max(-1))[1] - 23, -120)
    m = np.clip(np.rint(np.ldexp(x, -e[..., None])), -8388607, 8388607).astype(np.int64) & 0xFFFFFF
    u = m.reshape(*m.shape[:-1], -1, 4)
    w = np.stack([u[..., 0] | (u[..., 1] << 24), (u[..., 1] >> 8) | (u[..., 2] << 16),
                  (u[..., 2] >> 16) | (u[..., 3] << 8)], -1) & 0xFFFFFFFF
    return w.reshape(*x.shape[:-1], -1).astype(np.uint32), np.ldexp(np.float32(1), e).astype(np.float32)


def kv_unpack(words, scales):
    """Inverse of kv_pack: fp32 rows [..., dh] (exact: a 24-bit integer times a power of two)."""
    w = np.asarray(words, np.int64).reshape(*np.shape(words)[:-1], -1, 3)
    u = np.stack([w[..., 0], (w[..., 0] >> 24) | (w[..., 1] << 8), (w[..., 1] >> 16) | (w[..., 2] << 16),
                  w[..., 2] >> 8], -1) & 0xFFFFFF
    m = np.where(u >= 1 << 23, u - (1 << 24), u).reshape(*np.shape(words)[:-1], -1)
    return (m.astype(np.float64) * np.asarray(scales, np.float64)[..., None]).astype(np.float32)


@functools.lru_cache(maxsize=None)
def model_bytes(name: str, seed: int = 1) -> bytes:
    spec = synth.CONFIGS[name]["spec"]
    return mgnn.build_model_file(spec, seed, O.quantize)


def tiny_spec(blocks, heads=0, window=0, V=16, D=8, H=12, context=64, tied=True):
    return synth.ModelSpec(V=V, D=D, H=H, blocks=[synth.BlockSpec(*b) for b in blocks], heads=heads, window=window,
                           context=context, tied=tied)


def uniform_model_bytes(spec, seed=3, scale=0.5) -> bytes:
    """Every parameter uniform in [-scale, scale] (vectors too), like the reference's equivalence models
    (internal/quant/equivalence_test.go:63-73), then the per-tensor quantiser."""
    w = synth.float_weights(spec, seed)
    q = {}
    for i, (k, v) in enumerate(sorted(w.items())):
        u = (synth.uniform(seed, "u:" + k, v.size) * 2 - 1) * scale
        v = u.astype(np.float32).reshape(v.shape)
        if synth.is_matrix(k):
            q[k], q[k + ".scale"] = O.quantize(v)
        else:
            q[k] = v
    return mgnn.encode(spec, q)


# The reference's quantEquivCases (internal/quant/equivalence_test.go:34-49): one and two blocks,
# context sizes and attention sublayers.
EQUIV_CASES = {
    "1blk": dict(blocks=[(3, 2, 1)], context=64),
    "2blk": dict(blocks=[(2, 2, 1), (2, 2, 2)], context=64),
    "2blk ctx=256": dict(blocks=[(2, 2, 1), (2, 2, 2)], context=256),
    "1blk attn": dict(blocks=[(3, 2, 1)], context=64, heads=2),
    "2blk attn": dict(blocks=[(2, 2, 1), (2, 2, 2)], context=64, heads=2),
    "2blk attn window": dict(blocks=[(2, 2, 1), (2, 2, 2)], context=64, heads=4, window=3),
}


def equiv_model_bytes(name: str) -> bytes:
    c = EQUIV_CASES[name]
    spec = tiny_spec(c["blocks"], heads=c.get("heads", 0), window=c.get("window", 0), context=c["context"])
    return uniform_model_bytes(spec)


def oracle_model(data: bytes, max_context=None) -> O.OracleModel:
    return O.OracleModel(O.read_model(data), max_context)
