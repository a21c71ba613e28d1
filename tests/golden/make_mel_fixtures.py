"""Writes tests/golden/mel_fixture.npz — expected log-mel features of seeded
synthetic waves from an implementation independent of both the reference and
the oracle: torch.stft (center=True, pad_mode="constant", the symmetric
400-point Hann window zero-padded to 512) in float64, |X|^2, the reference's
own filterbank data file (data/mel_filters.f32, read as data), ln(. + 2^-24),
per-bin normalisation over the valid frames with the sample std (N - 1) and
zeroed padded frames — the feature pipeline of src/mel.rs:41-140, which the
reference states matches transformers' ParakeetFeatureExtractor. Also stores
a digest of the filterbank (per-row first / last nonzero bin, count, sum) and
four full rows, so the package's own filterbank is checked without the data
file.

Run in the build container only:  python tests/golden/make_mel_fixtures.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "mel_fixture.npz"
REF_FILTERS = Path("/root/reference/data/mel_filters.f32")
SR = 16000


def waves():
    rng = np.random.default_rng(2024)
    t = np.arange(19237) / SR  # 1.2 s and a partial hop
    chirp = 0.3 * np.sin(2 * np.pi * (200 + 1500 * t) * t)
    a = (chirp + 0.05 * rng.standard_normal(t.size)).astype(np.float32)
    a[6000:7000] = 0.0  # silence inside
    b = (0.2 * rng.standard_normal(1283)).astype(np.float32)  # 8 valid frames
    c = (0.1 * rng.standard_normal(170)).astype(np.float32)   # one valid frame
    return {"a": a, "b": b, "c": c}


def expected(wave: np.ndarray, filters: np.ndarray):
    x = torch.from_numpy(wave.astype(np.float64))
    pre = torch.cat([x[:1], x[1:] - 0.97 * x[:-1]])
    win = torch.hann_window(400, periodic=False, dtype=torch.float64)
    st = torch.stft(pre, 512, hop_length=160, win_length=400, window=win, center=True, pad_mode="constant",
                    return_complex=True)
    power = st.real ** 2 + st.imag ** 2  # (257, n_frames)
    mel = torch.log(torch.from_numpy(filters.astype(np.float64)) @ power + 2.0 ** -24).T
    n_frames, n_valid = 1 + wave.size // 160, wave.size // 160
    assert mel.shape[0] == n_frames
    out = torch.zeros_like(mel)
    if n_valid:
        v = mel[:n_valid]
        mean = v.mean(0)
        std = torch.sqrt(((v - mean) ** 2).sum(0) / max(n_valid - 1, 1))
        out[:n_valid] = (v - mean) / (std + 1e-5)
    return out.numpy().astype(np.float32), n_frames, n_valid


def main():
    filters = np.fromfile(REF_FILTERS, dtype=np.float32).reshape(128, 257)
    data = {}
    for k, w in waves().items():
        f, nf, nv = expected(w, filters)
        data[f"wave_{k}"] = w
        data[f"feat_{k}"] = f
        data[f"frames_{k}"] = np.int64(nf)
        data[f"valid_{k}"] = np.int64(nv)
    nz = filters != 0
    first = nz.argmax(1)
    last = 256 - nz[:, ::-1].argmax(1)
    data["filt_digest"] = np.stack([first, last, nz.sum(1)], 1).astype(np.int64)
    data["filt_rowsum"] = filters.astype(np.float64).sum(1)
    data["filt_rows_idx"] = np.array([0, 1, 64, 127], dtype=np.int64)
    data["filt_rows"] = filters[[0, 1, 64, 127]]
    np.savez_compressed(OUT, **data)
    print("wrote", OUT)


if __name__ == "__main__":
    main()
