"""Greedy TDT decoder, numpy restatement — TEST INFRASTRUCTURE ONLY.

Follows TdtDecoder::decode_rayon (src/tdt.rs:374-414) with the pieces it calls:
  start state .. h = c = 0, one LSTM step on the blank (8192) embedding, then
                 dec = proj_w h1 + proj_b (:382-385, project :515-529);
  lstm_step .... per layer gates = b_ih + b_hh + w_ih x + w_hh h in PyTorch's
                 row order i, f, g, o; c = f c + i g; h = o tanh(c); layer 1
                 takes the new h0 (:179-214);
  joint ........ x = max(enc + dec, 0) (NaN -> 0, f32::max); scores = head_w x
                 + head_b; token = first row of the highest score above -inf
                 among rows 0..8192 (NaN never qualifies; none: 0), duration
                 likewise over rows 8193..8197 minus 8193 (none: 0 - 8193,
                 which as a u32 moves the frame past T and ends the loop)
                 (:217-288);
  loop ......... stop when frame >= T or after T * (10 + 4) + 64 steps; blank:
                 frame += max(dur, 1); token: emit {id, frame, dur}, LSTM step
                 on its embedding, new dec, frame += dur (:386-412).
Arithmetic is float64 on the f16-rounded matrices (the reference keeps them as
f16 and sums in f32), so scores agree with it to f32 rounding. Each step also
records its decision margins (best minus runner-up score, token and duration),
so a comparison can show that the decisions are not near-ties.
Pinned by tests/golden/tdt_fixture.npz (transformers' ParakeetRNNTDecoder /
ParakeetTDTJointNetwork with torch.nn.LSTM, tests/golden/make_tdt_fixtures.py)
in tests/test_oracle_tdt.py.
"""
from __future__ import annotations

import numpy as np

DH = 640
VOCAB = 8193
N_DUR = 5
BLANK = 8192
MAX_SYMBOLS = 10


class Decoder:
    def __init__(self, src):
        """src.read(name) -> array, the reference's tensor names."""
        f16 = lambda n: np.asarray(src.read(n), np.float32).astype(np.float16).astype(np.float64)
        f32 = lambda n: np.asarray(src.read(n), np.float32).astype(np.float64)
        self.embed = f32("decoder.embedding.weight")
        self.w_ih = [f16(f"decoder.lstm.weight_ih_l{l}") for l in (0, 1)]
        self.w_hh = [f16(f"decoder.lstm.weight_hh_l{l}") for l in (0, 1)]
        self.b = [f32(f"decoder.lstm.bias_ih_l{l}") + f32(f"decoder.lstm.bias_hh_l{l}") for l in (0, 1)]
        self.proj_w = f16("decoder.decoder_projector.weight")
        self.proj_b = f32("decoder.decoder_projector.bias")
        self.head_w = f16("joint.head.weight")
        self.head_b = f32("joint.head.bias")

    def lstm_step(self, x, h, c):
        for l in range(2):
            g = self.b[l] + self.w_ih[l] @ (x if l == 0 else h[0]) + self.w_hh[l] @ h[l]
            i, f, gg, o = g[:DH], g[DH:2 * DH], g[2 * DH:3 * DH], g[3 * DH:]
            sig = lambda v: 1.0 / (1.0 + np.exp(-v))
            c[l] = sig(f) * c[l] + sig(i) * np.tanh(gg)
            h[l] = sig(o) * np.tanh(c[l])

    def project(self, h1):
        return self.proj_w @ h1 + self.proj_b

    def scores(self, enc, dec):
        """joint scores of the 8193 token rows and 5 duration rows; max(x, 0)
        returns 0 for NaN like Rust's f32::max"""
        return self.head_w @ np.fmax(enc + dec, 0.0) + self.head_b

    def start(self):
        """(h, c, dec) after the start step on the blank embedding"""
        h = [np.zeros(DH), np.zeros(DH)]
        c = [np.zeros(DH), np.zeros(DH)]
        self.lstm_step(self.embed[BLANK], h, c)
        return h, c, self.project(h[1])

    def joint(self, enc, dec):
        s = self.scores(enc, dec)
        tok_s, dur_s = s[:VOCAB], s[VOCAB:]
        tok, dur = first_max(tok_s), first_max(dur_s)
        # no qualifying duration row: row 0, whose u32 duration 0 - 8193 wraps
        dur = dur if dur is not None else -VOCAB
        return (tok if tok is not None else 0), dur, margin(tok_s, tok or 0), margin(dur_s, max(dur, 0))

    def decode(self, pooler, t_len=None, with_margins=False):
        pooler = np.asarray(pooler, np.float32).astype(np.float64)
        t_len = pooler.shape[0] if t_len is None else t_len
        h, c, dec = self.start()
        tokens, margins = [], []
        frame = guard = 0
        max_steps = t_len * (MAX_SYMBOLS + 4) + 64
        while frame < t_len:
            guard += 1
            if guard > max_steps:
                break
            tok, dur, mt, md = self.joint(pooler[frame], dec)
            margins.append((mt, md))
            if dur < 0:  # the wrapped duration moves the frame past any T
                if tok != BLANK:
                    tokens.append((tok, frame, dur % (1 << 32)))
                break
            if tok == BLANK:
                frame += max(dur, 1)
            else:
                tokens.append((tok, frame, dur))
                self.lstm_step(self.embed[tok], h, c)
                dec = self.project(h[1])
                frame += dur
        out = np.asarray(tokens, np.uint32).reshape(-1, 3)
        return (out, np.asarray(margins).reshape(-1, 2)) if with_margins else out


def first_max(scores):
    """the reference's scan (src/tdt.rs:236-263): the first row with the highest
    score above -inf; NaN never qualifies; None when no row does"""
    ok = scores > -np.inf  # False for NaN
    if not ok.any():
        return None
    best = scores[ok].max()
    return int(np.flatnonzero(ok & (scores == best))[0])


def margin(scores, best):
    """best score minus the highest other score (inf when there is no other)."""
    if scores.size < 2:
        return np.inf
    rest = np.delete(scores, best)
    return float(scores[best] - rest.max())
