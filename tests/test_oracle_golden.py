"""The oracle's Conformer block, position table and conv front end against
golden vectors from transformers' Parakeet modules (tests/golden/hf_parakeet.npz,
written by tests/golden/make_hf_fixtures.py). This pins the conventions a
restatement could misread identically in oracle and kernel: rel-shift
direction, bias_u on content vs bias_v on position, interleaved sin/cos, the
half-step FFN residuals, GLU halves, flatten order of the front end."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from conftest import rel_max_abs

GOLD = Path(__file__).resolve().parent / "golden" / "hf_parakeet.npz"
TOL = 5e-3  # bounded by the oracle's f16 rounding of K, V and relK


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


@pytest.fixture(scope="module")
def src(gold, synth):
    return synth.SynthCheckpoint(seed=int(gold["seed"]), n_layers=1, style="rich", attn_std=float(gold["attn_std"]))


@pytest.mark.parametrize("t", [5, 23])
def test_block_matches_transformers(oracle, gold, src, t):
    """One block (incl. norm_out). The oracle rounds K, V and relK to f16 as the
    reference does (src/cpu/ops.rs:258-259, src/cpu/layer.rs:234-247); the HF
    module keeps them f32, which bounds the agreement at ~1e-3."""
    enc = oracle.Encoder(src, n_layers=1)
    got = enc.block(0, gold[f"block_x_{t}"])
    err = rel_max_abs(got, gold[f"block_y_{t}"])
    print(f"block t={t}: rel max-abs vs transformers {err:.2e}")
    assert err < TOL


def test_block_shift_direction_matters(oracle, gold, src):
    """Guard on the check above: reversing the time axis of the input (which
    flips the sign of every relative position) must move the result far beyond
    the tolerance, so the fixture can tell a mirrored rel-shift apart."""
    enc = oracle.Encoder(src, n_layers=1)
    x = gold["block_x_23"]
    flipped = enc.block(0, x[::-1].copy())[::-1]
    err = rel_max_abs(flipped, gold["block_y_23"])
    print(f"mirrored positions: rel max-abs {err:.2e}")
    assert err > 10 * TOL


def test_pos_embed_matches_transformers(oracle, gold):
    got = oracle.pos_embed(9)
    assert np.max(np.abs(got - gold["pos_9"])) < 2e-6


def test_front_end_matches_transformers(oracle, gold, src):
    """Conv stack + flatten (src/sub.rs) followed by the f16-rounded sub
    linear + bias, against ParakeetEncoderSubsamplingConv2D."""
    sub = oracle.subsample(src, gold["sub_mel"])
    w = oracle.round_f16(src.read("encoder.subsampling.linear.weight")).astype(np.float64)
    b = src.read("encoder.subsampling.linear.bias").astype(np.float64)
    y = sub.astype(np.float64) @ w.T + b
    err = rel_max_abs(y, gold["sub_y"])
    print(f"front end: rel max-abs vs transformers {err:.2e}")
    assert err < 1e-5
