"""The checkpoint probe (weights_io::probe, src/weights_io.rs:208-297) and the
safetensors header reader behind bark_hip_load_safetensors, on the CPU: layout,
tensor and weight counts, architecture from shapes, release name, sharded
checkpoints, JSON edge cases (escapes, unicode names, nesting) and malformed
files. ModelInfo::check_architecture (src/weights_io.rs:173-195) on top."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest


def header_file(path, entries, metadata=None, raw_header=None, pad=0):
    """entries: name -> (dtype, shape); data bytes are zeros of the right size"""
    size = {"BF16": 2, "F16": 2, "F32": 4, "U32": 4, "I64": 8}
    h, off = {}, 0
    if metadata is not None:
        h["__metadata__"] = metadata
    for name, (dt, shape) in entries.items():
        n = int(np.prod(shape)) * size[dt]
        h[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + n]}
        off += n
    text = raw_header if raw_header is not None else json.dumps(h).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"\0" * (off + pad))


def small_model(dt="BF16", layers=2, ffn=64, hidden=16, vocab=33):
    e = {"decoder.embedding.weight": (dt, (vocab, 8)), "encoder.subsampling.linear.weight": (dt, (hidden, 32))}
    for l in range(layers):
        e[f"encoder.layers.{l}.feed_forward1.linear1.weight"] = (dt, (ffn, hidden))
        e[f"encoder.layers.{l}.norm_out.weight"] = (dt, (hidden,))
        e[f"encoder.layers.{l}.conv.norm.num_batches_tracked"] = ("I64", ())
    return e


def test_probe_single_file(pkg, tmp_path):
    e = small_model()
    header_file(tmp_path / "model.safetensors", e, metadata={"format": "pt"})
    info = pkg.probe(tmp_path)
    weights = sum(int(np.prod(s)) for d, s in e.values() if d != "I64")
    assert info == {"release": None, "layout": "bf16", "tensors": len(e), "weights": weights, "layers": 2,
                    "hidden": 16, "ffn": 64, "vocab": 33}
    assert pkg.probe(tmp_path / "model.safetensors")["layers"] == 2  # the file itself
    with pytest.raises(pkg.HipError, match="this checkpoint is 2x16"):
        pkg.check_architecture(info)


def test_probe_full_architecture_passes_the_check(pkg, tmp_path):
    e = small_model(layers=24, ffn=4096, hidden=1024, vocab=8193)
    header_file(tmp_path / "model.safetensors", e)
    info = pkg.probe(tmp_path)
    pkg.check_architecture(info)
    assert info["layout"] == "bf16" and info["layers"] == 24


def test_probe_layouts(pkg, tmp_path):
    for dt, want in (("F16", "f16"), ("F32", "f32")):
        d = tmp_path / dt
        d.mkdir()
        header_file(d / "model.safetensors", small_model(dt))
        assert pkg.probe(d)["layout"] == want
    # 4-bit code words: eight weights each, hidden from the packed columns
    d = tmp_path / "lowbit"
    d.mkdir()
    e = small_model("BF16")
    e["encoder.layers.0.feed_forward1.linear1.weight"] = ("U32", (64, 2))
    e["encoder.layers.0.feed_forward1.linear1.levels"] = ("F16", (64, 4))
    header_file(d / "model.safetensors", e)
    with pytest.raises(pkg.HipError, match="lowbit.json is missing"):
        pkg.probe(d)
    (d / "lowbit.json").write_text("{}")
    (d / "bark3.json").write_text(json.dumps({"source": 'Underdog-Bark-3.0-"Plus"'}))
    info = pkg.probe(d)
    dense = sum(int(np.prod(s)) for n, (t, s) in e.items() if t not in ("I64", "U32") and not n.endswith(".levels"))
    assert info["layout"] == "low-bit" and info["hidden"] == 16 and info["weights"] == dense + 64 * 2 * 8
    assert info["release"] == 'Underdog-Bark-3.0-"Plus"'


def test_probe_sharded(pkg, tmp_path):
    e = small_model(layers=3)
    names = sorted(e)
    shards = {"a.safetensors": names[::2], "b.safetensors": names[1::2]}
    for f, ns in shards.items():
        header_file(tmp_path / f, {n: e[n] for n in ns})
    wm = {n: f for f, ns in shards.items() for n in ns}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {"x": 1}, "weight_map": wm}))
    info = pkg.probe(tmp_path)
    assert info["layers"] == 3 and info["tensors"] == len(e)
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"x": "../escape.safetensors"}}))
    with pytest.raises(pkg.HipError, match="plain file names"):
        pkg.probe(tmp_path)


def test_json_edge_cases(pkg, tmp_path):
    e = small_model()
    h = {"__metadata__": {"note": "tab\t \"quoted\" \\ slash/ é \U0001F600", "nested": {"a": [1, 2.5e3, -3, True,
                                                                                                   False, None]}}}
    off = 0
    for name, (dt, shape) in e.items():
        n = int(np.prod(shape)) * {"BF16": 2, "I64": 8}[dt]
        h[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + n]}
        off += n
    odd = "encoder.layers.1.café \"x\"\U0001F600.weight"
    h[odd] = {"dtype": "F32", "shape": [1], "data_offsets": [off, off + 4]}
    text = json.dumps(h, ensure_ascii=True).encode()  # \\uXXXX escapes incl. a surrogate pair
    with open(tmp_path / "model.safetensors", "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"\0" * (off + 4))
    info = pkg.probe(tmp_path)
    assert info["tensors"] == len(e) + 1 and info["layers"] == 2


@pytest.mark.parametrize("raw,match", [
    (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},}', "malformed JSON header"),
    (b'{"a": "\\q"}', "bad escape"),
    (b'[' * 100 + b']' * 100, "nesting too deep"),
    (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4000]}}', "data outside the file"),
    (b'{"a": {"dtype": "F32", "shape": [1.5], "data_offsets": [0, 4]}}', "expected an integer"),
    (b'{"a": {"dtype": "F32", "shape": [1]}}', "malformed tensor entry"),
    (b'{"a": 1} x', "trailing data"),
    # 2^63 and above would be undefined in a cast to int64: rejected first
    (b'{"a": {"dtype": "F32", "shape": [9223372036854775808], "data_offsets": [0, 4]}}', "below 2\\^53"),
    (b'{"a": {"dtype": "F32", "shape": [1e300], "data_offsets": [0, 4]}}', "below 2\\^53"),
    # each entry is fine, their product wraps a 64-bit count: rejected, not wrapped
    (b'{"a": {"dtype": "F32", "shape": [4294967296, 4294967296, 16], "data_offsets": [0, 4]}}', "overflows"),
    (b'{"a": {"dtype": "F32", "shape": [134217728, 134217728], "data_offsets": [0, 4]}}', "overflows"),
])
def test_malformed_headers(pkg, tmp_path, raw, match):
    header_file(tmp_path / "model.safetensors", {}, raw_header=raw, pad=16)
    with pytest.raises(pkg.HipError, match=match):
        pkg.probe(tmp_path)


def test_not_safetensors(pkg, tmp_path):
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(pkg.HipError, match="not a safetensors file"):
        pkg.probe(tmp_path)
    with pytest.raises(pkg.HipError, match="no such checkpoint"):
        pkg.probe(tmp_path / "nope.safetensors")
    header_file(tmp_path / "model.safetensors", {"x.weight": ("F32", (2,))})
    with pytest.raises(pkg.HipError, match="no feed_forward1"):
        pkg.probe(tmp_path)
