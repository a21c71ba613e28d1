"""Host side of the log-mel front end: the 128 x 257 slaney filterbank.

The reference ships this filterbank as data (data/mel_filters.f32, loaded by
src/inference.rs:46,480 into MelFrontend::new, src/mel.rs:25-38); it is
librosa.filters.mel(sr=16000, n_fft=512, n_mels=128, fmin=0, fmax=8000,
norm="slaney"), the filterbank transformers' ParakeetFeatureExtractor uses.
This module computes it from that published construction (slaney mel scale:
linear below 1 kHz at 200/3 Hz per mel, logarithmic above with step
ln(6.4)/27; triangular filters between adjacent mel points on the 257 FFT bin
frequencies; each triangle scaled by 2 / (its upper - lower edge in Hz)),
with librosa's roundings: each triangle is computed in float64 and stored as
float32, then scaled in float64 and rounded to float32 again.
"""
from __future__ import annotations

import numpy as np

SR = 16000
N_FFT = 512
N_MELS = 128


def _hz_to_mel(f):
    f = np.asarray(f, dtype=np.float64)
    f_sp = 200.0 / 3.0
    mels = f / f_sp
    min_log_hz = 1000.0
    min_log_mel = min_log_hz / f_sp
    logstep = np.log(6.4) / 27.0
    return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-300) / min_log_hz) / logstep, mels)


def _mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    f_sp = 200.0 / 3.0
    freqs = f_sp * m
    min_log_hz = 1000.0
    min_log_mel = min_log_hz / f_sp
    logstep = np.log(6.4) / 27.0
    return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), freqs)


def slaney_mel_filters(sr: int = SR, n_fft: int = N_FFT, n_mels: int = N_MELS) -> np.ndarray:
    """(n_mels, 1 + n_fft // 2) float32 filterbank."""
    fftfreqs = np.linspace(0.0, sr / 2.0, 1 + n_fft // 2)
    mel_pts = np.linspace(_hz_to_mel(0.0), _hz_to_mel(sr / 2.0), n_mels + 2)
    mel_f = _mel_to_hz(mel_pts)
    fdiff = np.diff(mel_f)
    ramps = mel_f[:, None] - fftfreqs[None, :]
    w = np.zeros((n_mels, fftfreqs.size), dtype=np.float32)
    for i in range(n_mels):
        lower = -ramps[i] / fdiff[i]
        upper = ramps[i + 2] / fdiff[i + 1]
        w[i] = np.maximum(0.0, np.minimum(lower, upper))
    enorm = 2.0 / (mel_f[2 : n_mels + 2] - mel_f[:n_mels])
    return (w.astype(np.float64) * enorm[:, None]).astype(np.float32)
