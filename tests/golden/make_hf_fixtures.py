"""Writes tests/golden/hf_parakeet.npz — golden vectors from an implementation
independent of both the reference and the oracle: transformers' Parakeet
encoder modules (transformers 5.15.0, models/parakeet/modeling_parakeet.py:
ParakeetEncoderRelPositionalEncoding, ParakeetEncoderBlock,
ParakeetEncoderSubsamplingConv2D), which the reference states it matches
(src/encoder/shader_sources.rs:7, src/mel.rs:1-3).

Weights come from SynthCheckpoint(seed=5, style="rich", attn_std=0.1: sharp,
position-sensitive attention) with the linear and
depthwise weights pre-rounded to f16, so the oracle's own f16 weight rounding
(src/cpu/mod.rs:33-37) changes nothing and both sides multiply identical
values. Settings that match the reference encoder: no linear / conv biases,
scale_input=False, eager attention, eval mode.

Cases: blocks at t = 5 and 23 (one 256-query block of the CPU path); blocks at
t = 300 and 600 (two and three 256-query blocks, src/cpu/layer.rs:251-294: the
position-window start j0 of the later blocks), stored at rows around the block
boundaries; a block over 300 padded frames with a boolean attention mask of 257
valid frames (keys past the sequence masked, padded rows zeroed before the
depthwise conv) whose valid rows must equal a 257-frame block; the position
table; the conv front end unmasked and with n_valid < n_frames.

Front-end masks: transformers masks after every Conv2d (also the pointwise
ones), the reference after conv1 and after each depthwise conv only
(src/sub.rs:259-273). Both agree on every valid output row when the second
valid length vlen2 = conv_len(conv_len(n_valid)) is even; when it is odd the
last valid row differs (its depthwise window reads one pointwise output row
past vlen2, bias + ReLU in the reference, zero in transformers). The fixture
holds one case of each parity; the test compares all valid rows of the even
case and all but the last of the odd one.

Run in the build container only (the GPU box never needs it):
    python tests/golden/make_hf_fixtures.py
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent / "hf_parakeet.npz"
SEED = 5
ATTN_STD = 0.1


def load_synth():
    name = "bark3_wgpu_amd"
    init = ROOT / "bark3-wgpu_amd" / "__init__.py"
    spec = importlib.util.spec_from_file_location(name, init, submodule_search_locations=[str(init.parent)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    import importlib as il

    return il.import_module("bark3_wgpu_amd.synth")


def f16(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float16).astype(np.float32)


def main() -> None:
    from transformers.models.parakeet.configuration_parakeet import ParakeetEncoderConfig
    from transformers.models.parakeet.modeling_parakeet import (
        ParakeetEncoderBlock,
        ParakeetEncoderRelPositionalEncoding,
        ParakeetEncoderSubsamplingConv2D,
    )

    synth = load_synth()
    src = synth.SynthCheckpoint(seed=SEED, n_layers=1, style="rich", attn_std=ATTN_STD)
    cfg = ParakeetEncoderConfig(
        hidden_size=1024, num_hidden_layers=1, num_attention_heads=8, intermediate_size=4096,
        attention_bias=False, convolution_bias=False, conv_kernel_size=9, subsampling_factor=8,
        subsampling_conv_channels=256, num_mel_bins=128, scale_input=False, dropout=0.0,
        dropout_positions=0.0, layerdrop=0.0, activation_dropout=0.0, attention_dropout=0.0,
    )
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)

    block = ParakeetEncoderBlock(cfg, 0).eval()
    sd = {}
    for name, t in list(block.state_dict().items()):
        if name.endswith("num_batches_tracked"):
            sd[name] = t
            continue
        full = f"encoder.layers.0.{name}"
        v = src.read(full).astype(np.float32)
        if synth.is_linear(full) or name == "conv.depthwise_conv.weight":
            v = f16(v)
        sd[name] = torch.from_numpy(v.reshape(t.shape))
    block.load_state_dict(sd, strict=True)

    sub = ParakeetEncoderSubsamplingConv2D(cfg).eval()
    sd = {}
    for name, t in sub.state_dict().items():
        full = f"encoder.subsampling.{name}"
        v = src.read(full).astype(np.float32)
        if name == "linear.weight":
            v = f16(v)
        sd[name] = torch.from_numpy(v.reshape(t.shape))
    sub.load_state_dict(sd, strict=True)

    posenc = ParakeetEncoderRelPositionalEncoding(cfg)
    out = {"seed": np.array(SEED), "attn_std": np.array(ATTN_STD)}
    rng = np.random.default_rng(SEED)
    with torch.no_grad():
        for t in (5, 23):
            x = rng.standard_normal((t, 1024), dtype=np.float32)
            xt = torch.from_numpy(x)[None]
            pos = posenc(xt)
            y = block(xt, position_embeddings=pos)
            out[f"block_x_{t}"] = x
            out[f"block_y_{t}"] = y[0].numpy()
        x = torch.zeros((1, 9, 1024))
        out["pos_9"] = posenc(x)[0].numpy()
        mel = rng.standard_normal((61, 128), dtype=np.float32)
        out["sub_mel"] = mel
        out["sub_y"] = sub(torch.from_numpy(mel)[None])[0].numpy()
        # several 256-query blocks: inputs stored as f16 values (exact in
        # f32), outputs at rows around the block boundaries
        for t, rows in ((300, list(range(0, 8)) + list(range(248, 264)) + list(range(292, 300))),
                        (600, list(range(0, 4)) + list(range(252, 260)) + list(range(508, 516))
                         + list(range(596, 600)))):
            x = f16(rng.standard_normal((t, 1024), dtype=np.float32))
            xt = torch.from_numpy(x)[None]
            y = block(xt, position_embeddings=posenc(xt))[0].numpy()
            out[f"wblock_x_{t}"] = x.astype(np.float16)
            out[f"wblock_rows_{t}"] = np.array(rows, np.int32)
            out[f"wblock_y_{t}"] = y[rows]
        # padded batch row: 300 frames of which the first 257 are valid
        t_pad, t_valid = 300, 257
        x = f16(rng.standard_normal((t_pad, 1024), dtype=np.float32))
        xt = torch.from_numpy(x)[None]
        valid = torch.arange(t_pad) < t_valid
        mask = (valid[:, None] & valid[None, :])[None, None]
        y = block(xt, position_embeddings=posenc(xt), attention_mask=mask)[0].numpy()
        out["mblock_x"] = x.astype(np.float16)
        rows = list(range(0, 8)) + list(range(232, t_valid))
        out["mblock_valid"] = np.array(t_valid)
        out["mblock_rows"] = np.array(rows, np.int32)
        out["mblock_y"] = y[rows]
        # masked front end: (n_frames, n_valid) with vlen2 even, then odd
        for tag, (nf, nv) in (("even", (200, 150)), ("odd", (200, 145))):
            mel = rng.standard_normal((nf, 128), dtype=np.float32)
            am = (torch.arange(nf) < nv)[None].to(torch.int64)
            out[f"subm_{tag}_mel"] = mel
            out[f"subm_{tag}_valid"] = np.array(nv)
            out[f"subm_{tag}_y"] = sub(torch.from_numpy(mel)[None], attention_mask=am)[0].numpy()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): " + ", ".join(f"{k}{v.shape}" for k, v in out.items()))


if __name__ == "__main__":
    main()
