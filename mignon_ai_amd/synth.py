"""Seeded synthetic models and inputs for the five benchmark configurations.

Weights follow the benchmark definition: every matrix (embedding, W1, W2, W_select, QKV, Out) is drawn
N(0, 0.02); vectors take the reference initialisation (internal/ca/model.go:126-174): gamma, attention
norms and the final norm 1, b1 0, b2 0 on the value half and -1.386 on the gate half, head bias 0.
Heads are tied. Every matrix is then quantised with the reference's per-tensor quantiser
(quant.NewTensorF32, internal/quant/tensor.go:12-42), supplied by the caller.

Random numbers: a counter-based splitmix64 stream per tensor, so any tensor can be regenerated alone:
  u64(seed, tag, i) = mix64(seed ^ mix64(tag) + (i + 1) * 0x9E3779B97F4A7C15)
with mix64 the splitmix64 finaliser. Uniforms in [0, 1) take the top 53 bits; normals use Box-Muller
on consecutive pairs (u1 = 1 - uniform, u2 = uniform): z = sqrt(-2 ln u1) cos(2 pi u2), computed in
float64 and rounded to float32 after scaling. Token ids are (u64 >> 11) mod V.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix64(z):
    z = np.asarray(z, np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _tag_hash(tag: str) -> np.uint64:
    h = np.uint64(1469598103934665603)  # FNV-1a 64
    with np.errstate(over="ignore"):
        for ch in tag.encode():
            h = (h ^ np.uint64(ch)) * np.uint64(1099511628211)
    return _mix64(h)


def u64_stream(seed: int, tag: str, n: int) -> np.ndarray:
    base = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) ^ _tag_hash(tag)
    i = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(base + i * _GAMMA)


def uniform(seed: int, tag: str, n: int) -> np.ndarray:
    return (u64_stream(seed, tag, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, tag: str, n: int, std: float) -> np.ndarray:
    m = (n + 1) // 2
    u = uniform(seed, tag, 2 * m)
    u1 = 1.0 - u[0::2]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:n] * std).astype(np.float32)


def token_ids(seed: int, tag: str, shape, V: int) -> np.ndarray:
    n = int(np.prod(shape))
    return ((u64_stream(seed, tag, n) >> np.uint64(11)) % np.uint64(V)).astype(np.int32).reshape(shape)


@dataclass
class BlockSpec:
    steps: int = 1
    dilation_base: int = 2
    initial_dilation: int = 1


@dataclass
class ModelSpec:
    V: int
    D: int
    H: int
    blocks: list = field(default_factory=list)
    heads: int = 0
    window: int = 0
    context: int = 128
    tied: bool = True

    @property
    def n_params(self) -> int:
        """Parameter count of the reference layout (internal/ca/layout.go:96-162)."""
        D, H, V = self.D, self.H, self.V
        n = V * D
        for _ in self.blocks:
            n += 2 * H * (3 * D + 1) + 2 * D * (H + 1) + D + D * D
            if self.heads > 0:
                n += D + 4 * D * D
        n += D
        n += V if self.tied else V * (D + 1)
        return n


# The five benchmark configurations. c3's "dilation cap 16" is inert under the reference's
# BuildBlockConfigs (every block has one step, so no dilation is ever multiplied): the blocks keep
# initial dilation 1 as BuildBlockConfigs(2, 1, 2) produces (internal/ca/model.go:33-59).
CONFIGS = {
    "c1": dict(spec=ModelSpec(V=512, D=32, H=64, blocks=[BlockSpec(2, 2, 1)]), B=64, T=128),
    "c3": dict(spec=ModelSpec(V=2048, D=128, H=256, blocks=[BlockSpec(1, 2, 1)] * 2, heads=4, window=64),
               B=1024, T=128),
    "c4": dict(spec=ModelSpec(V=4096, D=256, H=512, blocks=[BlockSpec(1, 2, 1)] * 3, heads=8, window=64),
               B=4096, P=32, G=64),
    "c5": dict(spec=ModelSpec(V=8192, D=384, H=1024, blocks=[BlockSpec(1, 2, 1)] * 4, heads=6, window=64),
               B=16384, T=128),
}
C2 = dict(M=262144, K=384, N=512)


def float_weights(spec: ModelSpec, seed: int, std: float = 0.02) -> dict:
    """Full-precision synthetic weights, keyed like the checkpoint fields."""
    D, H, V = spec.D, spec.H, spec.V
    w = {"embed": normal(seed, "embed", V * D, std)}
    for b in range(len(spec.blocks)):
        p = f"b{b}."
        w[p + "w1"] = normal(seed, p + "w1", 2 * H * 3 * D, std)
        w[p + "b1"] = np.zeros(2 * H, np.float32)
        w[p + "w2"] = normal(seed, p + "w2", 2 * D * H, std)
        w[p + "b2"] = np.concatenate([np.zeros(D, np.float32), np.full(D, -1.386, np.float32)])
        w[p + "gamma"] = np.ones(D, np.float32)
        w[p + "wsel"] = normal(seed, p + "wsel", D * D, std)
        if spec.heads > 0:
            w[p + "attn_norm"] = np.ones(D, np.float32)
            w[p + "qkv"] = normal(seed, p + "qkv", 3 * D * D, std)
            w[p + "out"] = normal(seed, p + "out", D * D, std)
    w["final_norm"] = np.ones(D, np.float32)
    w["head_b"] = np.zeros(V, np.float32)
    if not spec.tied:
        w["head_w"] = normal(seed, "head_w", V * D, std)
    return w


MATRICES = ("embed", "w1", "w2", "wsel", "qkv", "out", "head_w")


def is_matrix(key: str) -> bool:
    return key.split(".")[-1] in MATRICES
