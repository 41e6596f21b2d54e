"""Model-file format: the product's writer, the oracle's reader and the product's C++ loader agree, and
damaged files are rejected (internal/binfmt/binfmt.go, internal/quant/checkpoint.go,
internal/quant/binary_test.go). CPU only: the product loader is exercised through mg_model_file_info,
which decodes and validates without touching the GPU."""
import ctypes
import json
import struct

import numpy as np
import pytest

from helpers import GOLDEN, equiv_model_bytes, model_bytes, tiny_spec, uniform_model_bytes
from mignon_ai_amd import _lib, mgnn, synth
from oracle import oracle as O


def product_info(data: bytes, max_context: int = 0):
    info = _lib.ModelInfo()
    buf = (ctypes.c_uint8 * max(len(data), 1)).from_buffer_copy(data or b"\0")
    rc = _lib.lib().mg_model_file_info(buf, len(data), max_context, ctypes.byref(info))
    return rc, info


def _damaged(good: bytes):
    """TestBinaryFileRejectsDamage's cases (internal/quant/binary_test.go:58-75)."""
    return {
        "cut in the arrays": good[:-5],
        "cut in the header": good[:20],
        "trailing bytes": good + bytes([1, 2, 3]),
        "wrong version": good[:4] + bytes([9, 0]) + good[6:],
        "wrong kind": good[:6] + bytes([7]) + good[7:],
        "full-precision kind": good[:6] + bytes([1]) + good[7:],
        "empty": b"",
    }


def test_damaged_files_rejected_by_both_readers():
    good = equiv_model_bytes("2blk attn")
    assert product_info(good)[0] == 0
    O.read_model(good)
    for name, data in _damaged(good).items():
        with pytest.raises(Exception):
            O.read_model(data)
        rc, _ = product_info(data)
        assert rc == _lib.MG_ERR_FORMAT, name
        assert _lib.lib().mg_last_error(), name


def test_wrong_rule_shape_rejected():
    """checkBlockShapes (internal/quant/checkpoint.go:214-225): |W1| must be 2*H*3*D."""
    good = model_bytes("c1")
    n = struct.unpack_from("<I", good, 8)[0]
    hdr = json.loads(good[12:12 + n])
    hdr["hidden_size"] = 65
    h2 = json.dumps(hdr).encode()
    bad = good[:8] + struct.pack("<I", len(h2)) + h2 + good[12 + n:]
    assert product_info(bad)[0] == _lib.MG_ERR_FORMAT
    assert b"rule_w1" in _lib.lib().mg_last_error()
    with pytest.raises(O.ModelFileError):
        O.read_model(bad)


def _json_checkpoint(data: bytes) -> bytes:
    """The legacy JSON form of a binary file (quant.Save writes CheckpointJSON with inline arrays)."""
    rm = O.read_model(data)
    n = struct.unpack_from("<I", data, 8)[0]
    cp = json.loads(data[12:12 + n])
    cp["embed"]["data"] = rm.embed.tolist()
    for b, rb in zip(cp["blocks"], rm.blocks):
        b["rule_w1"]["data"] = rb.w1.tolist()
        b["rule_b1"] = rb.b1.tolist()
        b["rule_w2"]["data"] = rb.w2.tolist()
        b["rule_b2"] = rb.b2.tolist()
        b["gamma"] = rb.gamma.tolist()
        b["rule_w_select"]["data"] = rb.wsel.tolist()
        if rb.attn is not None:
            b["attn"]["norm"] = rb.attn["norm"].tolist()
            b["attn"]["qkv"]["data"] = rb.attn["qkv"].tolist()
            b["attn"]["out"]["data"] = rb.attn["wo"].tolist()
    cp["final_norm"] = rm.final_norm.tolist()
    cp["head_b"] = rm.head_b.tolist()
    return json.dumps(cp).encode()


def test_json_file_matches_binary():
    """TestBinaryFileMatchesJSON (internal/quant/binary_test.go:14-56): same model either way."""
    data = equiv_model_bytes("2blk attn window")
    js = _json_checkpoint(data)
    assert len(data) < len(js) / 2
    a, b = O.OracleModel(O.read_model(data)), O.OracleModel(O.read_model(js))
    ctx = [2, 7, 14, 3, 9]
    assert np.array_equal(a.call(ctx), b.call(ctx))
    ra, ia = product_info(data)
    rb, ib = product_info(js)
    assert ra == rb == 0
    assert [getattr(ia, f) for f, _ in _lib.ModelInfo._fields_] == [getattr(ib, f) for f, _ in _lib.ModelInfo._fields_]


def test_writer_round_trip_and_header_shape():
    spec = synth.CONFIGS["c3"]["spec"]
    w = synth.float_weights(spec, 1)
    data = model_bytes("c3")
    rm = O.read_model(data)
    q, s = O.quantize(w["b1.w1"])
    assert np.array_equal(rm.blocks[1].w1, q) and rm.blocks[1].s1 == s
    assert np.array_equal(rm.blocks[0].b2, w["b0.b2"])
    n = struct.unpack_from("<I", data, 8)[0]
    hdr = json.loads(data[12:12 + n])
    # what Go's encoder puts in the header: arrays emptied to null, omitempty fields absent
    assert hdr["embed"]["data"] is None and hdr["head_b"] is None
    assert "gamma" not in hdr["blocks"][0] and "final_norm" not in hdr
    assert hdr["metadata"]["attn_heads"] == 4 and hdr["metadata"]["attn_window"] == 64
    assert data[:4] == b"MGNN" and struct.unpack_from("<HBB", data, 4) == (1, 2, 0)


@pytest.mark.parametrize("name", ["c1", "c3", "c4", "c5"])
def test_product_loader_info(name):
    spec = synth.CONFIGS[name]["spec"]
    rc, info = product_info(model_bytes(name))
    assert rc == 0
    assert (info.vocab_size, info.state_size, info.hidden_size, info.num_blocks) == (spec.V, spec.D, spec.H, len(spec.blocks))
    assert (info.attn_heads, info.attn_window, info.tied_embed) == (spec.heads, spec.window, 1)
    assert info.max_context == 128 and info.num_params == spec.n_params
    assert info.norm_ring == (3 if name == "c1" else 2)  # dilations {1,2} -> 2+1; {1} -> 1+1
    assert info.attn_cache == (spec.window or 128)


def test_product_loader_real_model():
    with open(f"{GOLDEN}/orders.mgn", "rb") as f:
        rc, info = product_info(f.read())
    assert rc == 0
    assert (info.vocab_size, info.state_size, info.hidden_size, info.num_blocks, info.attn_heads) == (2048, 96, 160, 2, 4)
    assert info.num_params == 538080 and info.max_context == 128 and info.attn_cache == 64


def test_max_context_defaulting():
    """quant.NewModel: a context below ca.DefaultMinContextSize (64) becomes 128 (model.go:91-95)."""
    data = model_bytes("c1")
    assert product_info(data, 32)[1].max_context == 128
    assert product_info(data, 64)[1].max_context == 64
    assert product_info(data, 300)[1].max_context == 300


def test_splitmix64_stream_matches_published_sequence():
    """The synthetic generator's mix is splitmix64: from state 0 its outputs are the published
    0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f (Vigna's reference implementation)."""
    from mignon_ai_amd.synth import _GAMMA, _mix64
    i = np.arange(1, 4, dtype=np.uint64)
    with np.errstate(over="ignore"):
        got = _mix64(i * _GAMMA)
    assert [int(x) for x in got] == [0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f]


def test_synthetic_models_are_deterministic():
    spec = tiny_spec([(1, 2, 1)], V=20, D=8, H=8)
    assert uniform_model_bytes(spec, seed=4) == uniform_model_bytes(spec, seed=4)
    assert uniform_model_bytes(spec, seed=4) != uniform_model_bytes(spec, seed=5)
