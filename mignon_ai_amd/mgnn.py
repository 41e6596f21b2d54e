"""Writer for the reference's binary INT8 model file (mignon.model/1, kind Int8).

Container (internal/binfmt/binfmt.go:1-78): "MGNN", uint16 version 1, uint8 kind 2, uint8 0, uint32
header length, the JSON header, then every weight array as a uint32 element count followed by int8
bytes or little-endian float32. The header is the checkpoint with its arrays emptied
(internal/quant/checkpoint.go:104-131); arrays follow quant.CheckpointJSON.arrays
(internal/quant/checkpoint.go:74-89). The format is the drop-in boundary, so it is kept byte-for-byte.
"""
from __future__ import annotations

import json
import struct

import numpy as np

from .synth import ModelSpec


def encode(spec: ModelSpec, q: dict, metadata: dict | None = None) -> bytes:
    """q maps checkpoint keys (see synth.float_weights) to int8 arrays (matrices, with a matching
    "<key>.scale" float) or float32 arrays (vectors)."""
    D, H, V = spec.D, spec.H, spec.V

    def tensor(k):
        return {"data": None, "scale": float(np.float32(q[k + ".scale"]))}

    blocks = []
    for b, bs in enumerate(spec.blocks):
        p = f"b{b}."
        blk = {"steps": bs.steps, "dilation_base": bs.dilation_base, "initial_dilation": bs.initial_dilation,
               "rule_w1": tensor(p + "w1"), "rule_b1": None, "rule_w2": tensor(p + "w2"), "rule_b2": None,
               "rule_w_select": tensor(p + "wsel")}
        if spec.heads > 0:
            blk["attn"] = {"norm": None, "qkv": tensor(p + "qkv"), "out": tensor(p + "out")}
        blocks.append(blk)
    meta = {"blocks": len(spec.blocks), "state_size": D, "hidden_size": H, "steps": spec.blocks[0].steps,
            "dilation_base": spec.blocks[0].dilation_base, "context_size": spec.context}
    if spec.tied:
        meta["tied_embed"] = True
    if spec.heads > 0:
        meta["attn_heads"] = spec.heads
        meta["attn_window"] = spec.window
    meta.update(metadata or {})
    header = {"vocab_size": V, "state_size": D, "hidden_size": H, "tied_embed": spec.tied,
              "embed": tensor("embed"), "blocks": blocks,
              "head_w": tensor("head_w") if not spec.tied else {"data": None, "scale": 0},
              "head_b": None, "metadata": meta}
    hjson = json.dumps(header, separators=(",", ":")).encode()

    arrays = [("i8", q["embed"])]
    for b in range(len(spec.blocks)):
        p = f"b{b}."
        arrays += [("i8", q[p + "w1"]), ("f32", q[p + "b1"]), ("i8", q[p + "w2"]), ("f32", q[p + "b2"]),
                   ("f32", q[p + "gamma"]), ("i8", q[p + "wsel"])]
        if spec.heads > 0:
            arrays += [("f32", q[p + "attn_norm"]), ("i8", q[p + "qkv"]), ("i8", q[p + "out"])]
    arrays += [("f32", q["final_norm"]), ("i8", q["head_w"] if not spec.tied else np.zeros(0, np.int8)),
               ("f32", q["head_b"])]

    parts = [b"MGNN", struct.pack("<HBBI", 1, 2, 0, len(hjson)), hjson]
    for dt, a in arrays:
        a = np.ascontiguousarray(a, np.int8 if dt == "i8" else "<f4")
        parts.append(struct.pack("<I", a.size))
        parts.append(a.tobytes())
    return b"".join(parts)


def build_model_file(spec: ModelSpec, seed: int, quantize) -> bytes:
    """Synthetic model file: seeded float weights, per-tensor quantised by `quantize(w) -> (q, scale)`."""
    from .synth import float_weights, is_matrix

    w = float_weights(spec, seed)
    q = {}
    for k, v in w.items():
        if is_matrix(k):
            q[k], q[k + ".scale"] = quantize(v)
        else:
            q[k] = v
    return encode(spec, q)
