"""safetensors IO (browsergrad_amd/jit/safetensors.py) on CPU.

Pinned against the format's own implementation, the ``safetensors`` 0.8.0
package (its numpy API): files it writes load bit-exactly, files this module
writes load bit-exactly with it.  The reference's tests
(packages/browsergrad-jit/tests-integration/safetensors.test.ts) are
restated: 3-tensor round trip with names in order, every dtype preserved,
the ``dtype=`` cast, BF16 and HTTP refusals.  The GPT-2 name mapping is
checked by evaluating one block (graph oracle) from Hugging Face-named
weights against the same block built from the weights directly.
"""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest
import safetensors.numpy as stnp

from browsergrad_amd.jit import configs
from browsergrad_amd.jit.safetensors import (SafetensorsFormatError, gpt2_block_params, load_safetensors,
                                             parse_header, save_safetensors)
from browsergrad_amd.jit.tensor import Session, autocast
from oracle import graph as G


def host(t):
    return t.session.buffers.get(t.uop.inputs[0].arg)


def test_round_trip_three_tensors_through_bytes():
    # safetensors.test.ts:23-61
    rng = np.random.default_rng(0)
    data = {"x": rng.standard_normal((2, 3)).astype(np.float32), "y": np.arange(5, dtype=np.int64),
            "z": rng.standard_normal((4,)).astype(np.float16)}
    blob = save_safetensors(data)
    s = Session()
    out = load_safetensors(blob, session=s)
    assert list(out) == ["x", "y", "z"]
    for k, v in data.items():
        got = host(out[k])
        assert got.dtype == v.dtype and np.array_equal(got, v)


@pytest.mark.parametrize("np_dtype", ["float32", "float16", "float64", "int64", "int32", "int16", "int8", "uint8",
                                      "uint16", "uint32", "uint64", "bool"])
def test_every_dtype_matches_the_format_library(np_dtype, tmp_path):
    # safetensors.test.ts:63-99 (dtype preservation), both directions against safetensors 0.8.0
    rng = np.random.default_rng(1)
    if np_dtype == "bool":
        a = rng.integers(0, 2, (3, 5)).astype(bool)
    elif np_dtype.startswith(("int", "uint")):
        a = rng.integers(0, 100, (3, 5)).astype(np_dtype)
    else:
        a = rng.standard_normal((3, 5)).astype(np_dtype)
    theirs = stnp.save({"t": a, "empty": np.zeros((0, 4), np_dtype)})
    s = Session()
    mine = load_safetensors(theirs, session=s)
    assert mine["t"].dtype == np_dtype and np.array_equal(host(mine["t"]), a)
    assert host(mine["empty"]).shape == (0, 4)
    back = stnp.load(save_safetensors({"t": a}))
    assert back["t"].dtype == a.dtype and np.array_equal(back["t"], a)
    p = tmp_path / "f.safetensors"
    save_safetensors({"t": a}, str(p), metadata={"k": "v"})
    assert np.array_equal(stnp.load_file(str(p))["t"], a)
    assert np.array_equal(host(load_safetensors(f"file://{p}", session=Session())["t"]), a)


def test_dtype_cast_argument():
    # safetensors.test.ts:101-125
    blob = save_safetensors({"w": np.ones((2, 2), np.float16)})
    out = load_safetensors(blob, session=Session(), dtype="float32")
    assert out["w"].dtype == "float32" and out["w"].uop.op == "CAST"


def test_bf16_and_http_are_refused():
    # safetensors.test.ts:127-171
    header = json.dumps({"w": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 4]}},
                        separators=(",", ":")).encode()
    blob = struct.pack("<Q", len(header)) + header + b"\0" * 4
    with pytest.raises(NotImplementedError, match=r"BF16.*PRD-010"):
        load_safetensors(blob, session=Session())
    with pytest.raises(NotImplementedError, match=r"HTTP.*PRD-008\.2"):
        load_safetensors("https://example.invalid/model.safetensors")


def _blob(header, data=b""):
    h = json.dumps(header).encode() if not isinstance(header, bytes) else header
    return struct.pack("<Q", len(h)) + h + data


def test_malformed_files_are_refused():
    with pytest.raises(SafetensorsFormatError, match="too small"):
        parse_header(b"\0" * 4)
    with pytest.raises(SafetensorsFormatError, match="header is empty"):
        parse_header(struct.pack("<Q", 0))
    with pytest.raises(SafetensorsFormatError, match="past the end of the input"):
        parse_header(struct.pack("<Q", 64) + b"{}")
    with pytest.raises(SafetensorsFormatError, match="ceiling"):
        parse_header(struct.pack("<Q", 200 * 1024 * 1024))
    with pytest.raises(SafetensorsFormatError, match="not a JSON object"):
        parse_header(_blob(b"{nope"))
    with pytest.raises(SafetensorsFormatError, match="start with"):
        parse_header(_blob([1, 2]))
    with pytest.raises(SafetensorsFormatError, match="not UTF-8"):
        parse_header(_blob(b'{"\xff": 1}'))
    with pytest.raises(SafetensorsFormatError, match="needs 8"):
        load_safetensors(_blob({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 4),
                         session=Session())
    with pytest.raises(SafetensorsFormatError, match="past the end"):
        load_safetensors(_blob({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, b"\0" * 4),
                         session=Session())
    with pytest.raises(SafetensorsFormatError, match="dtype code 'F8'"):
        load_safetensors(_blob({"a": {"dtype": "F8", "shape": [1], "data_offsets": [0, 1]}}, b"\0"),
                         session=Session())
    with pytest.raises(SafetensorsFormatError, match="shape must be"):
        load_safetensors(_blob({"a": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 1]}}, b"\0"),
                         session=Session())
    with pytest.raises(SafetensorsFormatError, match="unexpected field"):
        load_safetensors(_blob({"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1], "x": 0}}, b"\0"),
                         session=Session())
    with pytest.raises(SafetensorsFormatError, match="no safetensors code"):
        save_safetensors({"c": np.zeros(2, np.complex64)})
    with pytest.raises(SafetensorsFormatError, match="str to str"):
        save_safetensors({"a": np.zeros(1, np.float32)}, metadata={"k": 1})
    with pytest.raises(SafetensorsFormatError, match="reserved"):
        save_safetensors({"__metadata__": np.zeros(1, np.float32)})
    with pytest.raises(TypeError, match="neither a Tensor nor a NumPy array"):
        save_safetensors({"a": [1.0]})


def test_format_rules_beyond_the_reference():
    """Rules of the format description that the reference's reader does not
    enforce: duplicate keys, string-only metadata, and tensors that tile the
    data buffer (no gap, overlap or trailing bytes)."""
    rec = lambda lo, hi: {"dtype": "U8", "shape": [hi - lo], "data_offsets": [lo, hi]}  # noqa: E731
    dup = b'{"a":' + json.dumps(rec(0, 1)).encode() + b',"a":' + json.dumps(rec(1, 2)).encode() + b"}"
    with pytest.raises(SafetensorsFormatError, match="appears twice"):
        load_safetensors(_blob(dup, b"\0\0"), session=Session())
    with pytest.raises(SafetensorsFormatError, match="gap at byte 0"):
        load_safetensors(_blob({"a": rec(1, 2)}, b"\0\0"), session=Session())
    with pytest.raises(SafetensorsFormatError, match="overlaps"):
        load_safetensors(_blob({"a": rec(0, 2), "b": rec(1, 2)}, b"\0\0"), session=Session())
    with pytest.raises(SafetensorsFormatError, match="cover only 1"):
        load_safetensors(_blob({"a": rec(0, 1)}, b"\0\0"), session=Session())
    with pytest.raises(SafetensorsFormatError, match="__metadata__"):
        load_safetensors(_blob({"__metadata__": {"k": 3}, "a": rec(0, 1)}, b"\0"), session=Session())
    # Tiling holds in any header order; zero-length tensors may sit anywhere.
    ok = {"b": rec(2, 3), "e": rec(3, 3), "a": rec(0, 2), "__metadata__": {"k": "v"}}
    out = load_safetensors(_blob(ok, b"\1\2\3"), session=Session())
    assert list(out) == ["b", "e", "a"]
    assert host(out["a"]).tolist() == [1, 2] and host(out["b"]).tolist() == [3] and host(out["e"]).size == 0


def test_writer_aligns_the_data_buffer():
    for n in range(1, 12):
        blob = save_safetensors({"x" * n: np.arange(3, dtype=np.float64)}, metadata={"m": "y" * n})
        (hlen,) = struct.unpack("<Q", blob[:8])
        assert (8 + hlen) % 8 == 0 and blob[8:9] == b"{"
        assert np.array_equal(stnp.load(blob)["x" * n], np.arange(3, dtype=np.float64))


def _gpt2_hf_weights(rng, emb):
    f = lambda *s: (rng.standard_normal(s) * 0.02).astype(np.float32)  # noqa: E731
    return {
        "h.0.ln_1.weight": (1 + f(emb)).astype(np.float32), "h.0.ln_1.bias": f(emb),
        "h.0.attn.c_attn.weight": f(emb, 3 * emb), "h.0.attn.c_attn.bias": f(3 * emb),
        "h.0.attn.c_proj.weight": f(emb, emb), "h.0.attn.c_proj.bias": f(emb),
        "h.0.ln_2.weight": (1 + f(emb)).astype(np.float32), "h.0.ln_2.bias": f(emb),
        "h.0.mlp.c_fc.weight": f(emb, 4 * emb), "h.0.mlp.c_fc.bias": f(4 * emb),
        "h.0.mlp.c_proj.weight": f(4 * emb, emb), "h.0.mlp.c_proj.bias": f(emb),
    }


def test_gpt2_names_map_onto_the_block():
    rng = np.random.default_rng(3)
    heads, emb, bsz, seq = 2, 128, 2, 16
    hf = _gpt2_hf_weights(rng, emb)
    x = rng.standard_normal((bsz, seq, emb)).astype(np.float32)

    s1 = Session()
    p1 = gpt2_block_params(load_safetensors(stnp.save(hf), session=s1), 0)
    with autocast("float16"):
        y1 = configs.gpt2_block(s1.from_numpy(x, "x"), p1, heads)

    s2 = Session()
    direct = {
        "ln1_w": hf["h.0.ln_1.weight"], "ln1_b": hf["h.0.ln_1.bias"],
        "w_qkv": np.ascontiguousarray(hf["h.0.attn.c_attn.weight"].T), "b_qkv": hf["h.0.attn.c_attn.bias"],
        "w_o": np.ascontiguousarray(hf["h.0.attn.c_proj.weight"].T), "b_o": hf["h.0.attn.c_proj.bias"],
        "ln2_w": hf["h.0.ln_2.weight"], "ln2_b": hf["h.0.ln_2.bias"],
        "w_up": np.ascontiguousarray(hf["h.0.mlp.c_fc.weight"].T), "b_up": hf["h.0.mlp.c_fc.bias"],
        "w_down": np.ascontiguousarray(hf["h.0.mlp.c_proj.weight"].T), "b_down": hf["h.0.mlp.c_proj.bias"],
    }
    p2 = {k: s2.from_numpy(v, k) for k, v in direct.items()}
    with autocast("float16"):
        y2 = configs.gpt2_block(s2.from_numpy(x, "x"), p2, heads)
    a = G.evaluate(y1.uop, s1.buffers)
    b = G.evaluate(y2.uop, s2.buffers)
    assert a.shape == (bsz, seq, emb) and np.array_equal(a, b)
    with pytest.raises(KeyError, match="h.1.ln_1.weight"):
        gpt2_block_params(load_safetensors(stnp.save(hf), session=Session()), 1)
