"""Writes tests/golden/tdt_fixture.npz — greedy TDT decodes of seeded synthetic
decoder weights and poolers, computed with an implementation independent of
both the reference and the oracle: transformers' ParakeetRNNTDecoder (torch
nn.Embedding + 2-layer nn.LSTM + decoder_projector) and
ParakeetTDTJointNetwork (relu, head over 8193 tokens + 5 durations) built
from the default ParakeetTDTConfig, run in float64, stepped with the TDT rule
of transformers' ParakeetTDTGenerationMixin (token and duration argmax; a
blank with duration 0 advances one frame; the decoder state changes only on a
token) and the reference's step guard T * 14 + 64 (src/tdt.rs:381). Per case
it stores the tokens {id, frame, dur}, the number of steps, and the joint
scores of the first steps at the best rows, plus a digest of the weights so a
change of the seeded generator is caught.

Run in the build container only:  python tests/golden/make_tdt_fixtures.py
"""
from __future__ import annotations

import importlib
import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent / "tdt_fixture.npz"

# (name, SynthTdt kwargs, pooler frames, pooler seed)
CASES = [
    ("base", dict(seed=0), 300, 0),
    ("dur0", dict(seed=0, dur0_bias=-0.8), 300, 0),
    ("short", dict(seed=0), 7, 3),
]
SCORE_STEPS = 3
DIGEST_NAMES = ("decoder.embedding.weight", "decoder.lstm.weight_hh_l1", "joint.head.weight", "joint.head.bias")


def synth():
    """The package's synth module (the package directory's name has a dash, so
    it is loaded by path)."""
    name = "bark3_wgpu_amd"
    if name not in sys.modules:
        init = ROOT / "bark3-wgpu_amd" / "__init__.py"
        spec = importlib.util.spec_from_file_location(name, init, submodule_search_locations=[str(init.parent)])
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
    return importlib.import_module(name + ".synth")


def build(src):
    from transformers.models.parakeet.configuration_parakeet import ParakeetTDTConfig
    from transformers.models.parakeet.modeling_parakeet import ParakeetRNNTDecoder, ParakeetTDTJointNetwork

    cfg = ParakeetTDTConfig()
    dec, joint = ParakeetRNNTDecoder(cfg).double(), ParakeetTDTJointNetwork(cfg).double()
    t = lambda n: torch.from_numpy(np.asarray(src.read(n), np.float64))
    with torch.no_grad():
        dec.embedding.weight.copy_(t("decoder.embedding.weight"))
        for l in (0, 1):
            for kind in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
                getattr(dec.lstm, f"{kind}_l{l}").copy_(t(f"decoder.lstm.{kind}_l{l}"))
        dec.decoder_projector.weight.copy_(t("decoder.decoder_projector.weight"))
        dec.decoder_projector.bias.copy_(t("decoder.decoder_projector.bias"))
        joint.head.weight.copy_(t("joint.head.weight"))
        joint.head.bias.copy_(t("joint.head.bias"))
    return cfg, dec, joint


@torch.no_grad()
def run(cfg, dec, joint, pooler):
    T = pooler.shape[0]
    enc = torch.from_numpy(pooler.astype(np.float64))

    def step(token, state):
        out, state = dec.lstm(dec.embedding(torch.tensor([[token]])), state)
        return dec.decoder_projector(out)[0, 0], state

    d, state = step(cfg.blank_token_id, None)
    frame, steps, tokens, scores = 0, 0, [], []
    while frame < T and steps < T * (cfg.max_symbols_per_step + 4) + 64:
        steps += 1
        logits = joint(d, enc[frame])
        tok = int(logits[: cfg.vocab_size].argmax())
        dur = int(logits[cfg.vocab_size :].argmax())
        if len(scores) < SCORE_STEPS:
            top = torch.topk(logits[: cfg.vocab_size], 8).indices
            rows = torch.cat([top, torch.arange(cfg.vocab_size, cfg.vocab_size + 5)])
            scores.append(np.stack([rows.numpy().astype(np.float64), logits[rows].numpy()]))
        if tok == cfg.blank_token_id:
            frame += max(dur, 1)
        else:
            tokens.append((tok, frame, dur))
            d, state = step(tok, state)
            frame += dur
    return np.asarray(tokens, np.uint32).reshape(-1, 3), steps, np.stack(scores)


def main():
    s = synth()
    out = {}
    for name, kw, frames, pseed in CASES:
        src = s.SynthTdt(**kw)
        cfg, dec, joint = build(src)
        toks, steps, scores = run(cfg, dec, joint, s.pooler(frames, pseed))
        out[f"{name}_tokens"], out[f"{name}_steps"], out[f"{name}_scores"] = toks, np.int64(steps), scores
        print(name, "steps", steps, "tokens", len(toks), "durations", np.bincount(toks[:, 2], minlength=5))
    src = s.SynthTdt(seed=0)
    out["digest"] = np.array([float(np.asarray(src.read(n), np.float64).sum()) for n in DIGEST_NAMES])
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
