"""Float64, step-major restatement of the reference INT8 model for small shapes (test infrastructure).

The oracle (oracle/mgn_oracle.cpp) runs the reference's position-major fp32 streaming engine with its
exact rounding points. This module computes the same function a different way -- whole sequences one
rule step at a time (the float engine's order, internal/ca/forward.go:99-142), in float64, with plain
numpy reductions -- so that a structural mistake in either (a wrong gather index, a latch recurrence
off by one, a window bound, a missing residual) shows up as a large disagreement, while legitimate
fp32-vs-fp64 rounding stays far below the tolerance.
"""
from __future__ import annotations

import numpy as np


def sig(x):
    x = np.asarray(x, np.float64)
    out = 1.0 / (1.0 + np.exp(-np.clip(x, -15, 15)))
    return np.where(x > 15, 1.0, np.where(x < -15, 0.0, out))


def rmsnorm(x, g):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-5) * g


def step_dilation(initial, base, step):
    d = initial
    for _ in range(step):
        if d >= 32:
            break
        d *= base
    return min(d, 32)


def latch_base(D):
    d = np.arange(D, dtype=np.float64)
    td = np.full(D, 1.5) if D == 1 else 1.5 * (64 / 1.5) ** (d / (D - 1))
    lam = np.float32(2.0 ** (-1.0 / td)).astype(np.float64)
    return np.log(lam / (1 - lam))


def forward(rm, ids, max_context=128):
    """All-position logits [T, V] of one sequence (streaming semantics)."""
    D, H, V = rm.D, rm.H, rm.V
    ids = np.where((ids < 0) | (ids >= V), 0, ids)
    T = len(ids)
    emb = rm.embed.astype(np.float64).reshape(V, D)
    cur = emb[ids] * float(rm.embed_scale)
    block_in = cur.copy()
    base = latch_base(D)
    for b, blk in enumerate(rm.blocks):
        if b > 0:
            block_in = block_in + cur
            cur = block_in.copy()
        w1 = blk.w1.astype(np.float64).reshape(2 * H, 3 * D)
        w2 = blk.w2.astype(np.float64).reshape(2 * D, H)
        ws = blk.wsel.astype(np.float64).reshape(D, D)
        for step in range(blk.steps):
            dil = step_dilation(blk.initial_dilation, blk.dilation_base, step)
            n = rmsnorm(cur, blk.gamma.astype(np.float64)) if len(blk.gamma) == D else cur.copy()
            lam = sig(n @ ws.T * float(blk.ssel) + base)
            g = np.zeros(D)
            G = np.empty_like(n)
            for t in range(T):
                g = lam[t] * g + (1 - lam[t]) * n[t]
                G[t] = g
            left = np.zeros_like(n)
            if dil < T:
                left[dil:] = n[:T - dil]
            x = np.concatenate([n, left, G], axis=1)
            hid = x @ w1.T * float(blk.s1) + blk.b1.astype(np.float64)
            h = hid[:, :H] * sig(hid[:, H:])
            o = h @ w2.T * float(blk.s2) + blk.b2.astype(np.float64)
            gate = sig(o[:, D:])
            cur = (1 - gate) * cur + gate * o[:, :D]
        if blk.attn is not None:
            a = blk.attn
            heads = rm.heads
            dh = D // heads
            an = rmsnorm(cur, a["norm"].astype(np.float64))
            qkv = an @ a["qkv"].astype(np.float64).reshape(3 * D, D).T * float(a["sqkv"])
            q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
            cap = rm.window if rm.window > 0 else max_context
            att = np.zeros((T, D))
            for t in range(T):
                ws_ = t - rm.window + 1 if (rm.window > 0 and t - rm.window + 1 > 0) else 0
                lo = max(ws_, t - cap + 1)
                for hh in range(heads):
                    sl = slice(hh * dh, (hh + 1) * dh)
                    s = k[lo:t + 1, sl] @ q[t, sl] / np.sqrt(dh)
                    p = np.exp(s - s.max())
                    p /= p.sum()
                    att[t, sl] = p @ v[lo:t + 1, sl]
            cur = cur + att @ a["wo"].astype(np.float64).reshape(D, D).T * float(a["so"])
    fn = rmsnorm(cur, rm.final_norm.astype(np.float64)) if len(rm.final_norm) == D else cur
    hw = rm.embed if rm.tied else rm.head_w
    hs = rm.embed_scale if rm.tied else rm.head_scale
    logits = fn @ hw.astype(np.float64).reshape(V, D).T * float(hs)
    if len(rm.head_b):
        logits = logits + rm.head_b.astype(np.float64)
    return logits
