"""The greedy TDT decoder's oracle (oracle/tdt.py) against
tests/golden/tdt_fixture.npz — decodes by transformers' ParakeetRNNTDecoder /
ParakeetTDTJointNetwork (torch nn.LSTM) stepped with the TDT rule, written by
tests/golden/make_tdt_fixtures.py — plus the step guard and mistakes planted
in the oracle that the fixture must catch."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import tdt as otdt

GOLD = Path(__file__).resolve().parent / "golden" / "tdt_fixture.npz"
CASES = {  # name -> (SynthTdt kwargs, pooler frames, pooler seed), as the fixture script
    "base": (dict(seed=0), 300, 0),
    "dur0": (dict(seed=0, dur0_bias=-0.8), 300, 0),
    "short": (dict(seed=0), 7, 3),
}


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


@pytest.fixture(scope="module")
def decoders(synth):
    return {k: otdt.Decoder(synth.SynthTdt(**kw)) for k, (kw, _, _) in CASES.items()}


def test_weight_digest(synth, gold):
    src = synth.SynthTdt(seed=0)
    names = ("decoder.embedding.weight", "decoder.lstm.weight_hh_l1", "joint.head.weight", "joint.head.bias")
    got = np.array([float(np.asarray(src.read(n), np.float64).sum()) for n in names])
    np.testing.assert_array_equal(got, gold["digest"])


@pytest.mark.parametrize("case", list(CASES))
def test_decode_vs_fixture(synth, gold, decoders, case):
    _, frames, pseed = CASES[case]
    toks, margins = decoders[case].decode(synth.pooler(frames, pseed), with_margins=True)
    np.testing.assert_array_equal(toks, gold[f"{case}_tokens"])
    assert len(margins) == int(gold[f"{case}_steps"])


@pytest.mark.parametrize("case", list(CASES))
def test_first_scores_vs_fixture(synth, gold, decoders, case):
    """joint scores of the first steps at the fixture's rows (8 best tokens,
    5 durations), both in float64"""
    d = decoders[case]
    _, frames, pseed = CASES[case]
    pooler = synth.pooler(frames, pseed).astype(np.float64)
    ref = gold[f"{case}_scores"]
    h, c, dec = d.start()
    frame = 0
    for s in range(ref.shape[0]):
        sc = d.scores(pooler[frame], dec)
        rows = ref[s, 0].astype(np.int64)
        np.testing.assert_allclose(sc[rows], ref[s, 1], rtol=0, atol=1e-9)
        tok, dur = int(np.argmax(sc[: otdt.VOCAB])), int(np.argmax(sc[otdt.VOCAB :]))
        if tok == otdt.BLANK:
            frame += max(dur, 1)
        else:
            d.lstm_step(d.embed[tok], h, c)
            dec = d.project(h[1])
            frame += dur


def test_cases_cover_the_rules(gold):
    """blank and token steps, every duration, duration-0 tokens, end on frames"""
    base, dur0 = gold["base_tokens"], gold["dur0_tokens"]
    assert len(base) < int(gold["base_steps"])  # blanks happened
    assert set(np.unique(base[:, 2])) == {1, 2, 3, 4}
    assert (dur0[:, 2] == 0).sum() >= 5
    assert np.all(np.diff(base[:, 1].astype(np.int64)) >= 0)
    assert int(base[-1, 1]) < 300


def test_step_guard(synth):
    """a run of duration-0 tokens ends at T * 14 + 64 steps (src/tdt.rs:381-392)"""
    d = otdt.Decoder(synth.SynthTdt(seed=0, dur0_bias=-0.6))
    t = 100
    toks, margins = d.decode(synth.pooler(t, 0), with_margins=True)
    assert len(margins) == t * 14 + 64
    assert len(toks) > t * 10 and np.all(toks[:, 1] < t)


def test_empty_pooler(synth):
    d = otdt.Decoder(synth.SynthTdt(seed=0))
    assert d.decode(np.zeros((0, 640), np.float32)).shape == (0, 3)


@pytest.mark.parametrize("mistake", ["gate_order", "blank_min_step", "no_bias_hh"])
def test_planted_mistakes_are_caught(synth, gold, mistake):
    """each plausible slip in the oracle changes the fixture's decode"""
    d = otdt.Decoder(synth.SynthTdt(seed=0))
    if mistake == "gate_order":  # i and f rows swapped
        for l in (0, 1):
            for m in (d.w_ih, d.w_hh):
                m[l] = np.concatenate([m[l][640:1280], m[l][:640], m[l][1280:]])
            d.b[l] = np.concatenate([d.b[l][640:1280], d.b[l][:640], d.b[l][1280:]])
    elif mistake == "no_bias_hh":
        src = synth.SynthTdt(seed=0)
        d.b = [np.asarray(src.read(f"decoder.lstm.bias_ih_l{l}"), np.float64) for l in (0, 1)]
    else:  # blanks advance by their duration only, so a blank of duration 0 stays
        d = otdt.Decoder(synth.SynthTdt(seed=0, dur0_bias=-0.8))
        toks = _decode_without_blank_min(d, synth.pooler(300, 0))
        assert not np.array_equal(toks, gold["dur0_tokens"])
        return
    toks = d.decode(synth.pooler(300, 0))
    assert not np.array_equal(toks, gold["base_tokens"])


def _decode_without_blank_min(d, pooler):
    """the loop with `frame += dur` for blanks too (the slip)"""
    pooler = pooler.astype(np.float64)
    t_len = pooler.shape[0]
    h, c, dec = d.start()
    frame = guard = 0
    out = []
    while frame < t_len and guard < t_len * 14 + 64:
        guard += 1
        tok, dur, _, _ = d.joint(pooler[frame], dec)
        if tok != otdt.BLANK:
            out.append((tok, frame, dur))
            d.lstm_step(d.embed[tok], h, c)
            dec = d.project(h[1])
        frame += dur
    return np.asarray(out, np.uint32).reshape(-1, 3)


class _NanDurations:
    """SynthTdt with NaN duration biases: no duration row qualifies"""

    def __init__(self, synth, **kw):
        self.src = synth.SynthTdt(**kw)

    def read(self, name):
        v = np.array(self.src.read(name), copy=True)
        if name == "joint.head.bias":
            v[otdt.VOCAB:] = np.nan
        return v


def test_no_duration_row_ends_the_decode(synth):
    """the reference's scan keeps duration row 0 when no score beats -inf; its
    u32 duration 0 - 8193 wraps and moves the frame past T (src/tdt.rs:236-263,
    287, 396-410): one step, and a token (if any) records the wrapped value"""
    d = otdt.Decoder(_NanDurations(synth, seed=0, blank_bias=-5.0))
    toks, margins = d.decode(synth.pooler(50, 0), with_margins=True)
    assert len(margins) == 1
    assert toks.shape == (1, 3) and toks[0, 1] == 0 and toks[0, 2] == (1 << 32) - otdt.VOCAB
    d = otdt.Decoder(_NanDurations(synth, seed=0, blank_bias=50.0))
    toks, margins = d.decode(synth.pooler(50, 0), with_margins=True)
    assert len(margins) == 1 and toks.shape == (0, 3)


def test_nan_pooler_entries_act_as_zero(synth):
    """max(enc + dec, 0) gives 0 for NaN as Rust's f32::max (and for -inf)"""
    d = otdt.Decoder(synth.SynthTdt(seed=0))
    p = synth.pooler(60, 3)
    p[10:20] = np.nan
    q = p.copy()
    q[10:20] = -np.inf
    np.testing.assert_array_equal(d.decode(p), d.decode(q))
