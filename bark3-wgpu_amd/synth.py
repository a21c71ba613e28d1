"""Seeded synthetic checkpoints with the reference's tensor names and shapes.

A `SynthCheckpoint` behaves like the reference's `WeightSource`
(src/weights.rs:22-36): `read(name)` returns the tensor's values widened to f32
(what `RawTensor::to_f32` yields for a bf16 checkpoint) and `read_lowbit(name)`
returns the 4-bit form of a linear weight, or None.

attn_std scales q/k/relative_k projections and bias_u/bias_v (default 0.02,
like every other weight); golden fixtures raise it so that attention is sharp
and its position term dominates.

Styles:
  "baseline" - the BASELINE.json configs literally: every weight N(0, 0.02)
               stored as bf16, LayerNorm 1/0, BatchNorm mean 0 var 1 w 1 b 0,
               biases 0, bias_u/bias_v N(0, 0.02).
  "rich"     - non-trivial values for every parameter (LayerNorm/BatchNorm
               affine terms, biases, BN statistics) and front-end convolutions
               scaled by 1/sqrt(fan-in), so tests exercise every term.

4-bit linears (lowbit=True): "lut16" gives the generic format of config 1
(codes uniform in 0..15, each row's table = 16 sorted N(0, 0.02) draws as f16);
"levels" gives the reference's LowBitTensor format (k levels per row, codes in
0..2k, src/bark.rs:31-48,597-611).
"""
from __future__ import annotations

import zlib
from typing import Optional

import numpy as np

from . import LowBitTensor, Lut4Tensor

LINEAR_SUFFIXES = (
    "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
    "self_attn.relative_k_proj.weight", "self_attn.o_proj.weight",
    "feed_forward1.linear1.weight", "feed_forward1.linear2.weight",
    "feed_forward2.linear1.weight", "feed_forward2.linear2.weight",
    "conv.pointwise_conv1.weight", "conv.pointwise_conv2.weight",
)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """f32 -> nearest-even bf16 -> f32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def shape_of(name: str) -> tuple:
    if name.startswith("encoder.subsampling.layers."):
        i, kind = name.split(".")[3], name.split(".")[4]
        if kind == "bias":
            return (256,)
        return (256, 256, 1, 1) if i in ("3", "6") else (256, 1, 3, 3)
    if name == "encoder.subsampling.linear.weight":
        return (1024, 4096)
    if name == "encoder.subsampling.linear.bias":
        return (1024,)
    if name == "encoder_projector.weight":
        return (640, 1024)
    if name == "encoder_projector.bias":
        return (640,)
    suffix = name.split(".", 3)[3]
    table = {
        "feed_forward1.linear1.weight": (4096, 1024), "feed_forward2.linear1.weight": (4096, 1024),
        "feed_forward1.linear2.weight": (1024, 4096), "feed_forward2.linear2.weight": (1024, 4096),
        "conv.pointwise_conv1.weight": (2048, 1024, 1), "conv.pointwise_conv2.weight": (1024, 1024, 1),
        "conv.depthwise_conv.weight": (1024, 1, 9),
        "self_attn.bias_u": (8, 128), "self_attn.bias_v": (8, 128),
    }
    if suffix in table:
        return table[suffix]
    if suffix.endswith("_proj.weight"):
        return (1024, 1024)
    return (1024,)


def is_linear(name: str) -> bool:
    if name == "encoder.subsampling.linear.weight":
        return True
    return name.startswith("encoder.layers.") and name.split(".", 3)[3] in LINEAR_SUFFIXES


class SynthCheckpoint:
    def __init__(self, seed: int = 0, n_layers: int = 24, style: str = "rich", lowbit: bool = False,
                 lowbit_format: str = "lut16", k_lev: int = 2, attn_std: float = 0.02):
        assert style in ("rich", "baseline") and lowbit_format in ("lut16", "levels")
        self.seed, self.n_layers, self.style, self.attn_std = seed, n_layers, style, attn_std
        self.lowbit, self.lowbit_format, self.k_lev = lowbit, lowbit_format, k_lev

    def _rng(self, name: str, salt: int = 0) -> np.random.Generator:
        return np.random.default_rng([self.seed, zlib.crc32(name.encode()), salt])

    # -- WeightSource ---------------------------------------------------------
    def read_lowbit(self, name: str):
        if not (self.lowbit and is_linear(name)):
            return None
        rows, cols = shape_of(name)[:2]
        rng = self._rng(name, 1)
        if self.lowbit_format == "lut16":
            codes = rng.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
            lut = np.sort(rng.standard_normal((rows, 16), dtype=np.float32) * 0.02, axis=1)
            return Lut4Tensor(codes, lut.astype(np.float16).view(np.uint16), rows, cols)
        k = self.k_lev
        sym = rng.integers(0, 2 * k + 1, size=(rows, cols), dtype=np.uint32)
        words = np.zeros((rows, cols // 8), np.uint32)
        for e in range(8):
            words |= sym[:, e::8] << np.uint32(4 * e)
        lev = np.zeros((rows, 4), np.float16)
        lev[:, :k] = np.sort(np.abs(rng.standard_normal((rows, k), dtype=np.float32)) * 0.02 + 1e-3, axis=1)
        return LowBitTensor(words, lev.view(np.uint16), k, rows, cols)

    def read(self, name: str) -> np.ndarray:
        low = self.read_lowbit(name)
        if low is not None:
            return dequant(low)
        shp = shape_of(name)
        rng = self._rng(name)
        n = int(np.prod(shp))
        suffix = name.split(".")[-1]
        rich = self.style == "rich"
        if suffix in ("running_mean",):
            v = rng.standard_normal(n, dtype=np.float32) * 0.1 if rich else np.zeros(n, np.float32)
        elif suffix in ("running_var",):
            v = rng.uniform(0.5, 1.5, n).astype(np.float32) if rich else np.ones(n, np.float32)
        elif ("norm" in name and suffix == "weight") and "subsampling" not in name:
            v = 1.0 + rng.standard_normal(n, dtype=np.float32) * 0.1 if rich else np.ones(n, np.float32)
        elif suffix == "bias" and "norm" in name:
            v = rng.standard_normal(n, dtype=np.float32) * 0.1 if rich else np.zeros(n, np.float32)
        elif suffix == "bias":
            v = rng.standard_normal(n, dtype=np.float32) * 0.02 if rich else np.zeros(n, np.float32)
        else:
            std = 0.02
            if any(k in name for k in ("q_proj", "k_proj", "relative_k_proj", "bias_u", "bias_v")):
                std = self.attn_std  # larger values make attention peaky and position-sensitive
            if rich and name.startswith("encoder.subsampling.layers."):
                std = 1.0 / 3.0 if shp[1] == 1 else 1.0 / 16.0
            v = rng.standard_normal(n, dtype=np.float32) * std
        return round_bf16(v).reshape(shp)


def dequant(t) -> np.ndarray:
    """4-bit tensor -> f32 weight values (BarkContainer::read of a Levels2
    entry, src/bark.rs:379-391; lut16: w = lut16[row][code])."""
    if isinstance(t, Lut4Tensor):
        lo = (t.codes & 0xF).astype(np.intp)
        hi = (t.codes >> 4).astype(np.intp)
        codes = np.empty((t.rows, t.cols), np.intp)
        codes[:, 0::2], codes[:, 1::2] = lo, hi
        lut = t.lut16.view(np.float16).astype(np.float32)
        return np.take_along_axis(lut, codes, axis=1)
    codes = np.empty((t.rows, t.cols), np.intp)
    for e in range(8):
        codes[:, e::8] = (t.codes >> np.uint32(4 * e)) & 0xF
    lev = t.levels.view(np.float16).astype(np.float32)
    k = t.k
    table = np.zeros((t.rows, 16), np.float32)
    for c in range(1, 16):
        mag, neg = (c - 1, False) if c <= k else (c - k - 1, True)
        val = lev[:, mag] if mag < k else np.zeros(t.rows, np.float32)
        table[:, c] = -val if neg else val
    return np.take_along_axis(table, codes, axis=1)


def mel(frames: int, seed: int = 0) -> np.ndarray:
    """Synthetic log-mel features (frames, 128) ~ N(0, 1)."""
    return np.random.default_rng([seed, 7]).standard_normal((frames, 128), dtype=np.float32)


class SynthTdt:
    """Seeded TDT decoder weights under the reference's names (TDT_SHAPES).

    LSTM and projection entries ~ U(-1/sqrt(640), 1/sqrt(640)) (torch's LSTM /
    Linear initialisation), embedding N(0, 1), joint head N(0, 1/sqrt(640))
    with biases N(0, 0.1), the blank row's bias raised by `blank_bias` and the
    duration rows' by (dur0_bias, 0.5, 0.3, 0, -0.3), so that blanks, tokens and
    every duration occur. A dur0_bias near -0.6 makes runs of duration-0
    tokens that the step guard ends. Matrices hold f16-representable values
    (the decoder keeps them as f16), vectors f32.
    """

    def __init__(self, seed: int = 0, blank_bias: float = 2.5, dur0_bias: float = -1.5):
        self.seed, self.blank_bias, self.dur0_bias = seed, blank_bias, dur0_bias

    def read(self, name: str) -> np.ndarray:
        from . import TDT_SHAPES

        shp = TDT_SHAPES[name]
        rng = np.random.default_rng([self.seed, zlib.crc32(name.encode()), 5])
        k = 1.0 / np.sqrt(640.0)
        if name == "decoder.embedding.weight":
            return rng.standard_normal(shp, dtype=np.float32)
        if name.startswith("decoder."):
            v = rng.uniform(-k, k, shp).astype(np.float32)
        elif name == "joint.head.weight":
            v = (rng.standard_normal(shp, dtype=np.float32) * k).astype(np.float32)
        else:
            v = rng.standard_normal(shp, dtype=np.float32) * np.float32(0.1)
            if name == "joint.head.bias":
                v[8192] += np.float32(self.blank_bias)
                v[8193:] += np.asarray((self.dur0_bias, 0.5, 0.3, 0.0, -0.3), np.float32)
        return v.astype(np.float16).astype(np.float32) if len(shp) == 2 else v


def pooler(t: int, seed: int = 0) -> np.ndarray:
    """Synthetic encoder output (t, 640) ~ N(0, 1)."""
    return np.random.default_rng([seed, 11]).standard_normal((t, 640), dtype=np.float32)
