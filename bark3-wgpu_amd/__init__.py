"""MI355X (gfx950) HIP backend for the bark3 Conformer encoder — Python host layer.

This module is the host-side mirror of the reference's encoder surface over the
C ABI in include/bark_hip.h (libbark_hip.so, built in-tree by build.py):

  reference (Rust)                               here
  ---------------------------------------------  ----------------------------------
  Backend {Auto, Cpu, Gpu} (src/inference.rs:60)  Backend (+ HIP)
  Encoder::load_with(gpu, &dyn WeightSource)      HipEncoder.load_with(src)
    (src/encoder.rs:412)
  Encoder::encode(sub_rows, t, dump) -> EncodeOut HipEncoder.encode(sub_rows, t, dump)
    (src/encoder.rs:1985, :1974-1981)
  SubGpu::run + Encoder::encode_pre               HipEncoder.encode_mel(mel, n_valid)
    (src/sub_gpu.rs:574, src/encoder.rs:2005)
  LowBitTensor (src/bark.rs:31-48)                LowBitTensor
  WeightSource::{read, read_lowbit}               any object with read()/read_lowbit()
    (src/weights.rs:22-36)

Errors raise HipError with the library's message (the reference returns
anyhow::Error). The library must be built: there is no CPU fallback in this
module — a missing libbark_hip.so or a missing GPU raises.
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

__all__ = [
    "Backend",
    "EncodeOut",
    "HipEncoder",
    "HipError",
    "LowBitTensor",
    "Lut4Tensor",
    "lib",
    "lib_path",
    "lowbit_linear",
    "lowbit_linear_noalloc",
    "tensor_names",
    "conv_len",
    "HEADER_SYMBOLS",
]

_PKG = Path(__file__).resolve().parent
_LIB_PATH = _PKG / "libbark_hip.so"
_lib: Optional[ctypes.CDLL] = None

HIDDEN, LAYERS, PROJ, MEL = 1024, 24, 640, 128


class HipError(RuntimeError):
    """An error reported by libbark_hip (the reference's anyhow::Error)."""


class Backend(enum.Enum):
    """src/inference.rs:60-67, with the HIP backend added (the enum is
    #[non_exhaustive] there, so the new variant is not a breaking change)."""

    AUTO = "auto"
    CPU = "cpu"
    GPU = "gpu"
    HIP = "hip"


@dataclass
class LowBitTensor:
    """The reference's low-bit layout (src/bark.rs:31-48): `codes` rows x
    ceil(cols/8) u32 words, nibble col&7 of word col>>3; `levels` rows x 4 f16
    bits (zero padded); `k` levels in use per row (1..3)."""

    codes: np.ndarray
    levels: np.ndarray
    k: int
    rows: int
    cols: int


@dataclass
class Lut4Tensor:
    """Generic 4-bit layout: `codes` rows x cols/2 bytes (low nibble = even
    column), `lut16` rows x 16 f16 bits; weight = lut16[row][code]."""

    codes: np.ndarray
    lut16: np.ndarray
    rows: int
    cols: int


@dataclass
class EncodeOut:
    """src/encoder.rs:1974-1981: pooler (t, 640) f32 and, when asked for, the
    pre-norm residual (t, 1024) of one block."""

    pooler: np.ndarray
    block: Optional[np.ndarray] = None


def conv_len(l: int) -> int:
    """src/sub.rs:11-13"""
    return (l + 2 - 3) // 2 + 1


def lib_path() -> Path:
    return _LIB_PATH


# Every function declared in include/bark_hip.h, with its ctypes signature.
_c = ctypes
_SIGS = {
    "bark_hip_last_error": (_c.c_char_p, []),
    "bark_hip_device_count": (_c.c_int, []),
    "bark_hip_create": (_c.c_int, [_c.c_int, _c.c_int, _c.POINTER(_c.c_void_p)]),
    "bark_hip_destroy": (None, [_c.c_void_p]),
    "bark_hip_set_f32": (_c.c_int, [_c.c_void_p, _c.c_char_p, _c.c_void_p, _c.POINTER(_c.c_int64), _c.c_int]),
    "bark_hip_set_f16": (_c.c_int, [_c.c_void_p, _c.c_char_p, _c.c_void_p, _c.c_int64, _c.c_int64]),
    "bark_hip_set_lowbit": (
        _c.c_int,
        [_c.c_void_p, _c.c_char_p, _c.c_void_p, _c.c_void_p, _c.c_uint32, _c.c_int64, _c.c_int64],
    ),
    "bark_hip_set_lut4": (_c.c_int, [_c.c_void_p, _c.c_char_p, _c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int64]),
    "bark_hip_load_safetensors": (_c.c_int, [_c.c_void_p, _c.c_char_p]),
    "bark_hip_probe": (_c.c_int, [_c.c_char_p, _c.c_char_p, _c.c_size_t]),
    "bark_hip_finalize": (_c.c_int, [_c.c_void_p]),
    "bark_hip_encode_sub": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_int32, _c.c_void_p, _c.c_void_p]),
    "bark_hip_encode_mel": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_int32, _c.POINTER(_c.c_int32), _c.c_void_p, _c.c_size_t],
    ),
    "bark_hip_encode_mel_batch": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_void_p, _c.c_size_t],
    ),
    "bark_hip_encode_mel_batch_device": (
        _c.c_int,
        [
            _c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_void_p,
            _c.c_void_p, _c.c_size_t, _c.c_void_p,
        ],
    ),
    "bark_hip_set_mel_filters": (_c.c_int, [_c.c_void_p, _c.c_void_p]),
    "bark_hip_mel": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_size_t, _c.c_void_p, _c.c_void_p],
    ),
    "bark_hip_mel_device": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_size_t, _c.c_void_p, _c.c_void_p, _c.c_void_p],
    ),
    "bark_hip_encode_wave_batch": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_void_p, _c.c_size_t],
    ),
    "bark_hip_tdt_decode": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_size_t, _c.POINTER(_c.c_int32)],
    ),
    "bark_hip_tdt_decode_device": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_size_t, _c.POINTER(_c.c_int32), _c.c_void_p],
    ),
    "bark_hip_tdt_decode_batch": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_size_t, _c.c_void_p],
    ),
    "bark_hip_tdt_decode_batch_device": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_size_t, _c.c_void_p, _c.c_void_p],
    ),
    "bark_hip_transcribe_wave_batch": (
        _c.c_int,
        [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_void_p, _c.c_size_t, _c.c_void_p],
    ),
    "bark_hip_profile": (_c.c_int, [_c.c_void_p, _c.c_int]),
    "bark_hip_profile_only": (_c.c_int, [_c.c_void_p, _c.c_char_p]),
    "bark_hip_profile_report": (_c.c_int, [_c.c_void_p, _c.c_char_p, _c.c_size_t]),
    "bark_hip_lowbit_linear": (
        _c.c_int,
        [
            _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int32,
            _c.c_int32, _c.c_int32, _c.c_int32, _c.c_void_p,
        ],
    ),
    "bark_hip_lowbit_linear_noalloc": (
        _c.c_int,
        [
            _c.c_void_p, _c.c_int32, _c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int32,
            _c.c_int32, _c.c_int32, _c.c_int32, _c.c_void_p,
        ],
    ),
}
HEADER_SYMBOLS = tuple(_SIGS)


def lib() -> ctypes.CDLL:
    """Load libbark_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise HipError(f"{_LIB_PATH} is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(str(_LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != 0:
        msg = lib().bark_hip_last_error().decode(errors="replace")
        raise HipError(f"libbark_hip error {rc}: {msg}")


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def tensor_names(n_layers: int = LAYERS, front_end: bool = True) -> list[str]:
    """The tensor names the encoder reads, in load order (src/encoder.rs:423-604,
    src/sub.rs:85-89)."""
    names = []
    if front_end:
        for i in (0, 2, 3, 5, 6):
            names += [f"encoder.subsampling.layers.{i}.weight", f"encoder.subsampling.layers.{i}.bias"]
    names += ["encoder.subsampling.linear.weight", "encoder.subsampling.linear.bias"]
    per = [
        "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
        "self_attn.relative_k_proj.weight", "self_attn.o_proj.weight",
        "feed_forward1.linear1.weight", "feed_forward1.linear2.weight",
        "feed_forward2.linear1.weight", "feed_forward2.linear2.weight",
        "conv.pointwise_conv1.weight", "conv.pointwise_conv2.weight", "conv.depthwise_conv.weight",
        "conv.norm.weight", "conv.norm.bias", "conv.norm.running_mean", "conv.norm.running_var",
        "self_attn.bias_u", "self_attn.bias_v",
    ]
    for n in ("norm_feed_forward1", "norm_self_att", "norm_conv", "norm_feed_forward2", "norm_out"):
        per += [f"{n}.weight", f"{n}.bias"]
    for l in range(n_layers):
        names += [f"encoder.layers.{l}.{p}" for p in per]
    names += ["encoder_projector.weight", "encoder_projector.bias"]
    return names


# The greedy TDT decoder's tensors and shapes (TdtDecoder::from_source,
# src/tdt.rs:130-162).
TDT_SHAPES = {
    "decoder.embedding.weight": (8193, 640),
    "decoder.lstm.weight_ih_l0": (2560, 640), "decoder.lstm.weight_ih_l1": (2560, 640),
    "decoder.lstm.weight_hh_l0": (2560, 640), "decoder.lstm.weight_hh_l1": (2560, 640),
    "decoder.lstm.bias_ih_l0": (2560,), "decoder.lstm.bias_ih_l1": (2560,),
    "decoder.lstm.bias_hh_l0": (2560,), "decoder.lstm.bias_hh_l1": (2560,),
    "decoder.decoder_projector.weight": (640, 640), "decoder.decoder_projector.bias": (640,),
    "joint.head.weight": (8198, 640), "joint.head.bias": (8198,),
}


def probe(path) -> dict:
    """What a safetensors checkpoint holds, from its header(s) alone
    (weights_io::probe, src/weights_io.rs:208-297); needs no GPU."""
    import json

    buf = ctypes.create_string_buffer(4096)
    _check(lib().bark_hip_probe(str(path).encode(), buf, len(buf)))
    return json.loads(buf.value.decode())


# The architecture this build runs (src/lib.rs cfg: LAYERS, HIDDEN, FFN, VOCAB).
ARCH = {"layers": 24, "hidden": 1024, "ffn": 4096, "vocab": 8193}


def check_architecture(info: dict) -> None:
    """ModelInfo::check_architecture (src/weights_io.rs:173-195): refuse a
    checkpoint whose shape differs from the compiled-in constants, naming both."""
    got = tuple(info[k] for k in ("layers", "hidden", "ffn", "vocab"))
    want = tuple(ARCH[k] for k in ("layers", "hidden", "ffn", "vocab"))
    if got != want:
        raise HipError(
            f"this checkpoint is {got[0]}x{got[1]} (ffn {got[2]}, vocab {got[3]}), but this build is compiled for "
            f"{want[0]}x{want[1]} (ffn {want[2]}, vocab {want[3]}): it is a different Parakeet variant, not a Bark 3.0 "
            "release")


class HipEncoder:
    """The HIP encoder on one device (Encoder, src/encoder.rs:89-139,412-830)."""

    def __init__(self, device: int = 0, n_layers: int = LAYERS):
        L = lib()
        h = ctypes.c_void_p()
        _check(L.bark_hip_create(int(device), int(n_layers), ctypes.byref(h)))
        self._h = h
        self.n_layers = n_layers
        self.finalized = False

    # -- weight ingest ------------------------------------------------------
    def set_tensor(self, name: str, value) -> None:
        L, n = lib(), name.encode()
        if isinstance(value, LowBitTensor):
            codes = np.ascontiguousarray(value.codes, dtype=np.uint32)
            levels = np.ascontiguousarray(value.levels, dtype=np.uint16)
            _check(L.bark_hip_set_lowbit(self._h, n, _ptr(codes), _ptr(levels), value.k, value.rows, value.cols))
        elif isinstance(value, Lut4Tensor):
            codes = np.ascontiguousarray(value.codes, dtype=np.uint8)
            lut = np.ascontiguousarray(value.lut16, dtype=np.uint16)
            _check(L.bark_hip_set_lut4(self._h, n, _ptr(codes), _ptr(lut), value.rows, value.cols))
        else:
            arr = np.asarray(value)
            if arr.dtype == np.float16:
                a16 = np.ascontiguousarray(arr).view(np.uint16)
                rows = a16.shape[0] if a16.ndim > 1 else 1
                _check(L.bark_hip_set_f16(self._h, n, _ptr(a16), rows, a16.size // rows))
            else:
                a32 = np.ascontiguousarray(arr, dtype=np.float32)
                shape = (ctypes.c_int64 * max(a32.ndim, 1))(*(a32.shape or (1,)))
                _check(L.bark_hip_set_f32(self._h, n, _ptr(a32), shape, max(a32.ndim, 1)))

    def load_safetensors(self, path) -> None:
        """Stage every tensor this handle reads from a safetensors checkpoint
        (a file, or a directory with model.safetensors or an index and shards)."""
        _check(lib().bark_hip_load_safetensors(self._h, str(path).encode()))

    def finalize(self) -> None:
        _check(lib().bark_hip_finalize(self._h))
        self.finalized = True

    @classmethod
    def load_with(cls, src, device: int = 0, n_layers: int = LAYERS, front_end: bool = True,
                  decoder=None) -> "HipEncoder":
        """Read every encoder tensor from `src` (read / read_lowbit, like the
        reference's WeightSource) and upload it; with `decoder` (a source of
        the TDT_SHAPES tensors), the greedy TDT decoder's weights too."""
        enc = cls(device, n_layers)
        for name in tensor_names(n_layers, front_end):
            low = src.read_lowbit(name) if hasattr(src, "read_lowbit") else None
            enc.set_tensor(name, low if low is not None else src.read(name))
        if decoder is not None:
            for name in TDT_SHAPES:
                enc.set_tensor(name, decoder.read(name))
        enc.finalize()
        return enc

    # -- forward ------------------------------------------------------------
    def encode(self, sub_rows: np.ndarray, t_real: int, dump_layer: Optional[int] = None) -> EncodeOut:
        sub = np.ascontiguousarray(sub_rows, dtype=np.float32).reshape(-1)
        if sub.size < t_real * 4096:
            raise HipError("sub_rows holds fewer than t_real x 4096 values")
        pooler = np.empty((t_real, PROJ), np.float32)
        block = np.empty((t_real, HIDDEN), np.float32) if dump_layer is not None else None
        _check(
            lib().bark_hip_encode_sub(
                self._h, _ptr(sub), t_real, -1 if dump_layer is None else int(dump_layer), _ptr(pooler),
                _ptr(block) if block is not None else None,
            )
        )
        return EncodeOut(pooler, block)

    def encode_mel(self, mel: np.ndarray, n_valid: Optional[int] = None) -> tuple[np.ndarray, int]:
        m = np.ascontiguousarray(mel, dtype=np.float32)
        frames = m.shape[0]
        t = conv_len(conv_len(conv_len(frames)))
        out = np.empty((t, PROJ), np.float32)
        t_out = ctypes.c_int32()
        _check(
            lib().bark_hip_encode_mel(
                self._h, _ptr(m), frames, frames if n_valid is None else int(n_valid), ctypes.byref(t_out),
                _ptr(out), out.size,
            )
        )
        return out, t_out.value

    def encode_mel_batch(self, mels: Sequence[np.ndarray], n_valid: Optional[Sequence[int]] = None) -> list[np.ndarray]:
        frames = np.array([m.shape[0] for m in mels], np.int32)
        valid = frames.copy() if n_valid is None else np.asarray(n_valid, np.int32)
        cat = np.ascontiguousarray(np.concatenate([np.asarray(m, np.float32) for m in mels]), np.float32)
        ts = [conv_len(conv_len(conv_len(int(f)))) for f in frames]
        out = np.empty((sum(ts), PROJ), np.float32)
        t_out = np.zeros(len(mels), np.int32)
        _check(
            lib().bark_hip_encode_mel_batch(
                self._h, _ptr(cat), _ptr(frames), _ptr(valid), len(mels), _ptr(t_out), _ptr(out), out.size
            )
        )
        res, row = [], 0
        for t in t_out:
            res.append(out[row : row + t])
            row += int(t)
        return res

    def encode_mel_batch_device(self, d_mel: int, frames: Sequence[int], valid: Sequence[int], d_pooler: int,
                                cap: int, stream: int = 0) -> np.ndarray:
        """Device pointers in and out (inputs already resident in HBM); queued
        on `stream` without synchronising. Returns the per-utterance T."""
        fr = np.asarray(frames, np.int32)
        va = np.asarray(valid, np.int32)
        t_out = np.zeros(len(fr), np.int32)
        _check(
            lib().bark_hip_encode_mel_batch_device(
                self._h, ctypes.c_void_p(d_mel), _ptr(fr), _ptr(va), len(fr), _ptr(t_out), ctypes.c_void_p(d_pooler),
                int(cap), ctypes.c_void_p(stream) if stream else None,
            )
        )
        return t_out

    def set_mel_filters(self, filters: Optional[np.ndarray] = None) -> None:
        """MelFrontend::new (src/mel.rs:25): the 128 x 257 filterbank (default:
        the slaney filterbank of mel.slaney_mel_filters)."""
        if filters is None:
            from .mel import slaney_mel_filters

            filters = slaney_mel_filters()
        f = np.ascontiguousarray(filters, dtype=np.float32)
        if f.shape != (MEL, 257):
            raise ValueError(f"mel filters must be ({MEL}, 257), got {f.shape}")
        _check(lib().bark_hip_set_mel_filters(self._h, _ptr(f)))

    def mel(self, wave: np.ndarray) -> tuple[np.ndarray, int, int]:
        """MelFrontend::compute (src/mel.rs:41): (features (frames, 128) f32,
        frames, valid) of a 16 kHz mono wave."""
        w = np.ascontiguousarray(wave, dtype=np.float32)
        if w.ndim != 1 or w.size == 0:
            raise ValueError("wave must be a non-empty 1-D array")
        nf = 1 + w.size // 160
        out = np.empty((nf, MEL), np.float32)
        fr = np.zeros(1, np.int32)
        va = np.zeros(1, np.int32)
        _check(lib().bark_hip_mel(self._h, _ptr(w), w.size, _ptr(out), out.size, _ptr(fr), _ptr(va)))
        return out, int(fr[0]), int(va[0])

    def mel_device(self, d_wave: int, n_samples: int, d_features: int, cap: int, stream: int = 0) -> tuple[int, int]:
        """Device pointers in and out, queued on `stream` without synchronising;
        returns (frames, valid)."""
        fr = np.zeros(1, np.int32)
        va = np.zeros(1, np.int32)
        _check(
            lib().bark_hip_mel_device(
                self._h, ctypes.c_void_p(d_wave), int(n_samples), ctypes.c_void_p(d_features), int(cap), _ptr(fr),
                _ptr(va), ctypes.c_void_p(stream) if stream else None,
            )
        )
        return int(fr[0]), int(va[0])

    def encode_wave_batch(self, waves: Sequence[np.ndarray]) -> list[np.ndarray]:
        """Log-mel of each 16 kHz wave and one batched encode (chunked
        transcription's per-chunk mel + encoder); one pooler per wave."""
        ws = [np.ascontiguousarray(w, dtype=np.float32) for w in waves]
        n = np.asarray([w.size for w in ws], np.int64)
        flat = np.ascontiguousarray(np.concatenate(ws))
        t_exp = [conv_len(conv_len(conv_len(1 + int(k) // 160))) for k in n]
        out = np.empty((sum(t_exp), PROJ), np.float32)
        t_out = np.zeros(len(ws), np.int32)
        _check(lib().bark_hip_encode_wave_batch(self._h, _ptr(flat), _ptr(n), len(ws), _ptr(t_out), _ptr(out),
                                                out.size))
        res, row = [], 0
        for t in t_out:
            res.append(out[row : row + int(t)])
            row += int(t)
        return res

    def tdt_decode(self, pooler: np.ndarray) -> np.ndarray:
        """TdtDecoder::decode (src/tdt.rs:318): greedy TDT tokens of a pooler
        (T, 640) as an (n, 3) u32 array of {id, frame, dur}."""
        p = np.ascontiguousarray(pooler, dtype=np.float32)
        if p.ndim != 2 or p.shape[1] != PROJ:
            raise ValueError("pooler must be (T, 640)")
        t = p.shape[0]
        cap = t * 14 + 64
        out = np.zeros((cap, 3), np.uint32)
        n = ctypes.c_int32()
        _check(lib().bark_hip_tdt_decode(self._h, _ptr(p) if t else None, t, _ptr(out), cap, ctypes.byref(n)))
        return out[: n.value].copy()

    def tdt_decode_device(self, d_pooler: int, t_len: int, stream: int = 0) -> np.ndarray:
        """The same on a device pooler pointer (GpuTdtDecoder::decode_async)."""
        cap = t_len * 14 + 64
        out = np.zeros((cap, 3), np.uint32)
        n = ctypes.c_int32()
        _check(
            lib().bark_hip_tdt_decode_device(
                self._h, ctypes.c_void_p(d_pooler), int(t_len), _ptr(out), cap, ctypes.byref(n),
                ctypes.c_void_p(stream) if stream else None,
            )
        )
        return out[: n.value].copy()

    def tdt_decode_batch(self, poolers: Sequence[np.ndarray]) -> list[np.ndarray]:
        """Greedy TDT decoding of several poolers together (every launch
        advances all of them); one (n, 3) u32 token array per pooler."""
        ps = [np.ascontiguousarray(p, dtype=np.float32).reshape(-1, PROJ) for p in poolers]
        t = np.asarray([p.shape[0] for p in ps], np.int32)
        flat = np.ascontiguousarray(np.concatenate(ps)) if t.sum() else np.zeros((1, PROJ), np.float32)
        cap = int(sum(int(k) * 14 + 64 for k in t))
        out = np.zeros((cap, 3), np.uint32)
        counts = np.zeros(len(ps), np.int32)
        _check(lib().bark_hip_tdt_decode_batch(self._h, _ptr(flat), _ptr(t), len(ps), _ptr(out), cap, _ptr(counts)))
        res, row = [], 0
        for c in counts:
            res.append(out[row : row + int(c)].copy())
            row += int(c)
        return res

    def transcribe_wave_batch(self, waves: Sequence[np.ndarray]) -> list[np.ndarray]:
        """Log-mel, one batched encode and the greedy TDT decode of every 16 kHz
        wave, poolers kept on the device; one (n, 3) u32 token array per wave."""
        ws = [np.ascontiguousarray(w, dtype=np.float32) for w in waves]
        n = np.asarray([w.size for w in ws], np.int64)
        flat = np.ascontiguousarray(np.concatenate(ws))
        ts = [conv_len(conv_len(conv_len(1 + int(k) // 160))) for k in n]
        cap = sum(t * 14 + 64 for t in ts)
        out = np.zeros((cap, 3), np.uint32)
        counts = np.zeros(len(ws), np.int32)
        t_out = np.zeros(len(ws), np.int32)
        _check(lib().bark_hip_transcribe_wave_batch(self._h, _ptr(flat), _ptr(n), len(ws), _ptr(t_out), _ptr(out),
                                                    cap, _ptr(counts)))
        res, row = [], 0
        for c in counts:
            res.append(out[row : row + int(c)].copy())
            row += int(c)
        return res

    def profile(self, enable: bool = True) -> None:
        """Per-operator HIP-event timing of the forward (BARK3_ENC_PROFILE)."""
        _check(lib().bark_hip_profile(self._h, 1 if enable else 0))

    def profile_only(self, label: str | None) -> None:
        """Time only the launches labelled `label` (None = all)."""
        _check(lib().bark_hip_profile_only(self._h, label.encode() if label else None))

    def profile_report(self) -> dict:
        """{label: {count, ms, flops, bytes}} since the last report."""
        import json

        buf = ctypes.create_string_buffer(1 << 16)
        _check(lib().bark_hip_profile_report(self._h, buf, len(buf)))
        return json.loads(buf.value.decode())

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().bark_hip_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def lowbit_linear_noalloc(A: int, a_dtype: int, codes: int, lut16: int, C: int, c_dtype: int, T: int, K: int,
                          N: int, stream: int = 0) -> None:
    """bark_hip_lowbit_linear_noalloc: the isolated linear without any device
    allocation (partial sums in a fixed per-GPU array; calls that overlap on
    one GPU race)."""
    _check(
        lib().bark_hip_lowbit_linear_noalloc(
            ctypes.c_void_p(A), a_dtype, ctypes.c_void_p(codes), ctypes.c_void_p(lut16), ctypes.c_void_p(C), c_dtype,
            T, K, N, ctypes.c_void_p(stream) if stream else None,
        )
    )


def lowbit_linear(A: int, a_dtype: int, codes: int, lut16: int, C: int, c_dtype: int, T: int, K: int, N: int,
                  stream: int = 0) -> None:
    """The isolated 4-bit level-table linear on device pointers (see
    bark_hip_lowbit_linear); queued on `stream`, not synchronised."""
    _check(
        lib().bark_hip_lowbit_linear(
            ctypes.c_void_p(A), a_dtype, ctypes.c_void_p(codes), ctypes.c_void_p(lut16), ctypes.c_void_p(C), c_dtype,
            T, K, N, ctypes.c_void_p(stream) if stream else None,
        )
    )
