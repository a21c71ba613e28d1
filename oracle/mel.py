"""Log-mel front end, numpy restatement — TEST INFRASTRUCTURE ONLY.

Follows MelFrontend::compute (src/mel.rs:41-140): preemphasis 0.97 in f32
(:45-49); frames = 1 + len/hop, valid = len/hop (:51-52); each frame is the
center-padded (zeros outside the wave) 512-sample window starting at
t*160 - 256, multiplied by the symmetric 400-point Hann window placed at
offset 56 (:28-35, :58-68); power spectrum |FFT|^2 of bins 0..256 (:70); mel
= filters (128 x 257) . power summed over the filters' nonzero entries, then
ln(s + 2^-24) (:80-93); per-bin mean and sample std (N - 1) over the valid
frames, (x - mean) / (std + 1e-5) on valid frames, zeros on padded frames
(:103-131). The FFT, the filterbank product and the statistics run in float64
here (the reference uses rustfft and f32 sums), so agreement is to rounding.
Pinned by tests/golden/mel_fixture.npz (torch.stft pipeline, tests/golden/
make_mel_fixtures.py) in tests/test_oracle_mel.py.
"""
from __future__ import annotations

import numpy as np

HOP = 160
N_FFT = 512
WIN = 400


def window() -> np.ndarray:
    """Symmetric Hann of WIN points, zero-padded to N_FFT (f32, src/mel.rs:28-35)."""
    w = np.zeros(N_FFT, dtype=np.float32)
    i = np.arange(WIN, dtype=np.float32)
    w[(N_FFT - WIN) // 2 : (N_FFT - WIN) // 2 + WIN] = np.float32(0.5) * (
        np.float32(1.0) - np.cos(np.float32(2.0 * np.pi) * i / np.float32(WIN - 1)))
    return w


def features(wave: np.ndarray, filters: np.ndarray):
    """(frames (n_frames, 128) f32, n_frames, n_valid)."""
    x = np.asarray(wave, dtype=np.float32)
    pre = x.copy()
    pre[1:] = x[1:] - np.float32(0.97) * x[:-1]
    n = pre.size
    n_frames, n_valid = 1 + n // HOP, n // HOP
    padded = np.zeros(n + N_FFT, dtype=np.float64)
    padded[N_FFT // 2 : N_FFT // 2 + n] = pre
    idx = np.arange(n_frames)[:, None] * HOP + np.arange(N_FFT)[None, :]
    frames = padded[idx] * window().astype(np.float64)[None, :]
    spec = np.fft.rfft(frames, axis=1)
    power = (spec.real ** 2 + spec.imag ** 2)
    mel = np.log(power @ filters.astype(np.float64).T + 2.0 ** -24)  # (n_frames, 128)
    out = np.zeros((n_frames, filters.shape[0]), dtype=np.float32)
    if n_valid > 0:
        v = mel[:n_valid]
        mean = v.mean(axis=0)
        std = np.sqrt(((v - mean) ** 2).sum(axis=0) / max(n_valid - 1, 1))
        out[:n_valid] = ((v - mean) / (std + 1e-5)).astype(np.float32)
    return out, n_frames, n_valid
