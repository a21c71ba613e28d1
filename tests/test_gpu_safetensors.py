"""Safetensors ingest (TensorReader, src/weights_io.rs:46-127) through the C ABI
(bark_hip_load_safetensors): a handle loaded from a checkpoint file — single
file, or a directory with an index and shards; BF16, F16 and F32 entries —
gives bit-identical encoder and decoder results to one loaded tensor by tensor
with the same values."""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def write_safetensors(path, tensors):
    """tensors: name -> (dtype, array); BF16 arrays are f32 values already
    representable in bf16, stored as their upper 16 bits."""
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (dtype, a) in tensors.items():
        if dtype == "BF16":
            raw = (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16).tobytes()
        elif dtype == "F16":
            raw = np.ascontiguousarray(a, np.float16).tobytes()
        else:
            raw = np.ascontiguousarray(a, np.float32).tobytes()
        header[name] = {"dtype": dtype, "shape": list(np.shape(a)), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def checkpoint(pkg, synth, dtype_of):
    src, dec = synth.SynthCheckpoint(seed=1, n_layers=1), synth.SynthTdt(seed=0)
    out = {name: (dtype_of(name, src.read(name)), src.read(name)) for name in pkg.tensor_names(1, True)}
    for name in pkg.TDT_SHAPES:
        v = dec.read(name)
        out[name] = ("F16" if v.ndim == 2 and name != "decoder.embedding.weight" else "F32", v)
    out["encoder.layers.0.conv.norm.num_batches_tracked"] = ("I64", np.zeros(1))  # skipped by the loader
    return src, dec, out


def results(enc, synth):
    pooler, _ = enc.encode_mel(synth.mel(400, 2))
    return pooler, enc.tdt_decode(synth.pooler(200, 1))


@pytest.fixture(scope="module")
def reference(pkg, synth):
    src, dec = synth.SynthCheckpoint(seed=1, n_layers=1), synth.SynthTdt(seed=0)
    enc = pkg.HipEncoder.load_with(src, 0, 1, decoder=dec)
    try:
        yield results(enc, synth)
    finally:
        enc.close()


def test_single_file_bf16(pkg, synth, reference, tmp_path):
    print("case safetensors single file", flush=True)
    _, _, t = checkpoint(pkg, synth, lambda n, v: "BF16")
    t.pop("encoder.layers.0.conv.norm.num_batches_tracked")
    write_safetensors(tmp_path / "model.safetensors", t)
    enc = pkg.HipEncoder(0, 1)
    try:
        enc.load_safetensors(tmp_path)  # the directory form: model.safetensors
        enc.finalize()
        pooler, toks = results(enc, synth)
    finally:
        enc.close()
    np.testing.assert_array_equal(pooler, reference[0])
    np.testing.assert_array_equal(toks, reference[1])


def test_sharded_mixed_dtypes(pkg, synth, reference, tmp_path):
    print("case safetensors sharded", flush=True)
    dt = lambda n, v: "F16" if n.endswith("_proj.weight") else ("F32" if "norm" in n else "BF16")
    _, _, t = checkpoint(pkg, synth, dt)
    i64 = t.pop("encoder.layers.0.conv.norm.num_batches_tracked")
    names = sorted(t)
    shards = {"model-00001-of-00002.safetensors": names[::2], "model-00002-of-00002.safetensors": names[1::2]}
    for fname, ns in shards.items():
        write_safetensors(tmp_path / fname, {n: t[n] for n in ns})
    # an integer entry the loader skips, in its own shard
    with open(tmp_path / "extra.safetensors", "wb") as f:
        h = json.dumps({"encoder.layers.0.conv.norm.num_batches_tracked":
                        {"dtype": "I64", "shape": [], "data_offsets": [0, 8]}}).encode()
        h += b" " * (-len(h) % 8)
        f.write(struct.pack("<Q", len(h)) + h + struct.pack("<q", 0))
    wm = {n: f for f, ns in shards.items() for n in ns}
    wm["encoder.layers.0.conv.norm.num_batches_tracked"] = "extra.safetensors"
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": wm}))
    enc = pkg.HipEncoder(0, 1)
    try:
        enc.load_safetensors(str(tmp_path))
        enc.finalize()
        pooler, toks = results(enc, synth)
    finally:
        enc.close()
    np.testing.assert_array_equal(pooler, reference[0])
    np.testing.assert_array_equal(toks, reference[1])


def test_errors(pkg, synth, tmp_path):
    print("case safetensors errors", flush=True)
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    enc = pkg.HipEncoder(0, 1)
    try:
        with pytest.raises(pkg.HipError, match="not a safetensors file"):
            enc.load_safetensors(bad)
        trunc = tmp_path / "trunc.safetensors"
        h = json.dumps({"decoder.lstm.bias_ih_l0": {"dtype": "F32", "shape": [2560], "data_offsets": [0, 10240]}}).encode()
        trunc.write_bytes(struct.pack("<Q", len(h)) + h + b"\0" * 100)
        with pytest.raises(pkg.HipError, match="data outside the file"):
            enc.load_safetensors(trunc)
        with pytest.raises(pkg.HipError, match="no such checkpoint"):
            enc.load_safetensors(tmp_path / "missing.safetensors")
        part = tmp_path / "part.safetensors"
        _, _, t = checkpoint(pkg, synth, lambda n, v: "BF16")
        t.pop("encoder.layers.0.conv.norm.num_batches_tracked")
        t.pop("encoder.layers.0.norm_out.bias")
        write_safetensors(part, t)
        enc.load_safetensors(part)
        with pytest.raises(pkg.HipError, match="missing tensor encoder.layers.0.norm_out.bias"):
            enc.finalize()
    finally:
        enc.close()
