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


def _rows_err(got, want):
    return float(np.max(np.abs(got - want)) / np.max(np.abs(want)))


@pytest.mark.parametrize("t", [300, 600])
def test_block_query_windows_match_transformers(oracle, gold, src, t):
    """Blocks of 300 and 600 frames: the CPU path attends in 256-query blocks
    whose position window starts at j0 = floor((T-1-i_max)/128)*128
    (src/cpu/layer.rs:251-294); the later blocks' windows are only exercised
    past 256 frames. Rows around the block boundaries are compared."""
    enc = oracle.Encoder(src, n_layers=1)
    x = gold[f"wblock_x_{t}"].astype(np.float32)
    rows = gold[f"wblock_rows_{t}"]
    got = enc.block(0, x)[rows]
    err = _rows_err(got, gold[f"wblock_y_{t}"])
    print(f"block t={t} rows {rows.min()}..{rows.max()}: rel max-abs vs transformers {err:.2e}")
    assert err < TOL


def test_block_with_attention_mask_matches_transformers(oracle, gold, src):
    """A padded batch row: 300 frames with a boolean attention mask of 257
    valid ones (keys past the sequence masked, padded rows zeroed before the
    depthwise conv). Its valid rows equal a 257-frame block, the semantics of
    the per-sequence length masks (config 4); a guard shows the fixture tells
    masked from unmasked apart."""
    enc = oracle.Encoder(src, n_layers=1)
    tv = int(gold["mblock_valid"])
    x = gold["mblock_x"].astype(np.float32)
    rows = gold["mblock_rows"]
    err = _rows_err(enc.block(0, x[:tv])[rows], gold["mblock_y"])
    unmasked = _rows_err(enc.block(0, x)[rows], gold["mblock_y"])
    print(f"masked block {tv} of {x.shape[0]}: rel max-abs {err:.2e}; without the mask {unmasked:.2e}")
    assert err < TOL
    assert unmasked > 10 * TOL


@pytest.mark.parametrize("tag", ["even", "odd"])
def test_masked_front_end_matches_transformers(oracle, gold, src, tag):
    """n_valid < n_frames: time positions past the valid length are zeroed
    after conv1 and after each depthwise conv (src/sub.rs:259-300).
    transformers also masks after the pointwise convs; the two agree on every
    valid output row when vlen2 is even (all compared, and a guard shows the
    unmasked front end misses the last ones), and on all but the last valid
    row when vlen2 is odd, where the last row must differ: its depthwise
    window reads one pointwise output row past vlen2, which the reference
    leaves at bias + ReLU and transformers zeroes."""
    mel = gold[f"subm_{tag}_mel"]
    nv = int(gold[f"subm_{tag}_valid"])
    c = lambda l: (l - 1) // 2 + 1  # noqa: E731
    v2 = c(c(nv))
    v3 = c(v2)
    assert (v2 % 2 == 0) == (tag == "even")
    w = oracle.round_f16(src.read("encoder.subsampling.linear.weight")).astype(np.float64)
    b = src.read("encoder.subsampling.linear.bias").astype(np.float64)
    want = gold[f"subm_{tag}_y"]
    y = oracle.subsample(src, mel, n_valid=nv).astype(np.float64) @ w.T + b
    if tag == "even":
        err = rel_max_abs(y[:v3], want[:v3])
        y0 = oracle.subsample(src, mel).astype(np.float64) @ w.T + b
        miss = rel_max_abs(y0[:v3], want[:v3])
        print(f"masked front end (even, n_valid={nv}, {v3} rows): rel max-abs {err:.2e}; unmasked {miss:.2e}")
        assert err < 1e-5 and miss > 1e-3
    else:
        err = rel_max_abs(y[: v3 - 1], want[: v3 - 1])
        last = float(np.max(np.abs(y[v3 - 1] - want[v3 - 1])) / np.max(np.abs(want[: v3])))
        print(f"masked front end (odd, n_valid={nv}): first {v3 - 1} rows {err:.2e}; last valid row {last:.2e}")
        assert err < 1e-5 and last > 1e-3
