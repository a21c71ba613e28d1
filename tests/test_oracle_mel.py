"""The log-mel front end's oracle (oracle/mel.py) and the package's slaney
filterbank against tests/golden/mel_fixture.npz — features from an independent
torch.stft pipeline with the reference's own filterbank data file, written by
tests/golden/make_mel_fixtures.py — and, where the reference checkout is
present, against that data file itself (src/inference.rs:46,480)."""
from __future__ import annotations

import importlib
from pathlib import Path

import numpy as np
import pytest

from oracle import mel as omel

GOLD = Path(__file__).resolve().parent / "golden" / "mel_fixture.npz"
REF_FILTERS = Path("/root/reference/data/mel_filters.f32")
TOL = 5e-4  # f32 window / preemphasis in the oracle vs f64 torch pipeline


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


@pytest.fixture(scope="module")
def filters(pkg):
    return importlib.import_module("bark3_wgpu_amd.mel").slaney_mel_filters()


def test_filterbank_matches_digest(gold, filters):
    nz = filters != 0
    first = nz.argmax(1)
    last = 256 - nz[:, ::-1].argmax(1)
    assert np.array_equal(np.stack([first, last, nz.sum(1)], 1), gold["filt_digest"])
    assert np.allclose(filters.astype(np.float64).sum(1), gold["filt_rowsum"], rtol=0, atol=1e-7)
    rows = filters[gold["filt_rows_idx"]]
    assert np.array_equal(rows.view(np.uint32), gold["filt_rows"].view(np.uint32))


@pytest.mark.skipif(not REF_FILTERS.exists(), reason="reference checkout absent")
def test_filterbank_bit_exact_to_reference_data(filters):
    ref = np.fromfile(REF_FILTERS, dtype=np.float32).reshape(128, 257)
    assert np.array_equal(filters.view(np.uint32), ref.view(np.uint32))


def test_window_closed_form():
    w = omel.window()
    assert w[:56].max() == 0 and w[456:].max() == 0  # zero padding around the 400 taps
    assert w[56] == 0 and w[455] == 0  # symmetric Hann ends
    assert np.allclose(w[56:456], w[56:456][::-1], atol=1e-7)
    assert abs(w[56 + 199] - 1.0) < 1e-4 and abs(w[56 + 200] - 1.0) < 1e-4


@pytest.mark.parametrize("k", ["a", "b", "c"])
def test_oracle_features_vs_torch_stft(gold, filters, k):
    f, nf, nv = omel.features(gold[f"wave_{k}"], filters)
    assert (nf, nv) == (int(gold[f"frames_{k}"]), int(gold[f"valid_{k}"]))
    assert np.abs(f - gold[f"feat_{k}"]).max() <= TOL
    assert not f[nv:].any()  # padded frames are zero


def test_oracle_catches_a_wrong_hop(gold, filters, monkeypatch):
    """A planted mistake (hop 161) must fail the fixture comparison."""
    monkeypatch.setattr(omel, "HOP", 161)
    f, nf, nv = omel.features(gold["wave_a"], filters)
    assert f.shape != gold["feat_a"].shape or np.abs(f - gold["feat_a"]).max() > TOL
