"""GPU parity of the encoder against the CPU oracle (the reference CPU path
restated), through the C ABI. Tolerance (BASELINE): relative max-abs error
<= 1e-2 per block; measured values are printed per case."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_max_abs

pytestmark = pytest.mark.gpu

TOL = 1e-2


@pytest.fixture(scope="module")
def one_layer(pkg, synth, oracle):
    out = {}
    for key in ("f16", "4bit", "sharp"):
        # "sharp": attention projections at std 0.1 so softmax rows are peaky and
        # the relative-position term dominates the scores
        src = synth.SynthCheckpoint(seed=1, n_layers=1, style="rich", lowbit=key != "f16",
                                    attn_std=0.1 if key == "sharp" else 0.02)
        out[key] = (src, pkg.HipEncoder.load_with(src, n_layers=1, front_end=False), oracle.Encoder(src, 1))
    yield out
    for _, enc, _ in out.values():
        enc.close()


@pytest.mark.parametrize("kind", ["f16", "4bit", "sharp"])
@pytest.mark.parametrize("t", [1, 5, 17, 64, 129, 188, 300])
def test_one_block(one_layer, kind, t):
    src, enc, orc = one_layer[kind]
    print(f"case one_block {kind} t={t}", flush=True)
    sub = np.random.default_rng([t, 2]).standard_normal((t, 4096), dtype=np.float32)
    got = enc.encode(sub, t, dump_layer=0)
    want_pool, want_dump = orc.encode_dump(sub, t)
    e_blk = rel_max_abs(got.block, want_dump[0])
    e_pool = rel_max_abs(got.pooler, want_pool)
    print(f"  block err {e_blk:.3e}  pooler err {e_pool:.3e}")
    assert np.all(np.isfinite(got.pooler))
    assert e_blk <= TOL and e_pool <= TOL
