"""A 1,000-step BERT-tiny run (b32 s128, V 30522, masked rows 832, dropout 0.1, AdamW with warmup)
on the MI355X against the CPU oracle's run of the same seed and inputs.

The oracle's run takes hours on one core, so its outputs are fixtures written by
tests/golden/make_oracle_losses.py (`bert_tiny 1000`): the 1,001 losses (every step's and the
final one) and the L2 norm of every parameter tensor after the run. The bar is the reference's run
tolerance (crates/modelspec-runtime/tests/common/mod.rs:17-40): every loss within
1e-4 + 1e-3 |c|, and each parameter tensor's norm within what that elementwise bound allows,
1e-3 ||c|| + 1e-4 sqrt(size) (the attention key biases, whose exact gradient is zero, hold only
rounding noise of order 1e-7 in both runs, so their norms agree only to that absolute term)."""
import os

import numpy as np
import pytest

from modelspec_amd import api

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_bert_tiny_tracks_the_oracle_over_1000_steps(ctx):
    want_l = np.load(os.path.join(GOLDEN, "oracle_losses_bert_tiny_1000.npy"))
    want_n = np.load(os.path.join(GOLDEN, "oracle_param_norms_bert_tiny_1000.npy"))
    print("bert_tiny 1000 steps", flush=True)
    got_l, got_p, _ = ctx.train_config("bert_tiny", steps=1000)
    assert got_l.shape == want_l.shape
    assert np.all(np.isfinite(got_l))
    ok = np.abs(got_l - want_l) <= 1e-4 + 1e-3 * np.abs(want_l)
    assert ok.all(), (np.flatnonzero(~ok)[:5], got_l[~ok][:5], want_l[~ok][:5])
    # The run trains: the last losses are well below the first.
    assert want_l[-10:].mean() < want_l[:10].mean() - 1.0
    step_ir, _ = api.compile_config("bert_tiny", -1, 1000)
    sizes = [int(np.prod(s)) for _, s in api.param_shapes(step_ir)]
    parts = np.split(got_p.astype(np.float64), np.cumsum(sizes)[:-1])
    got_n = np.array([np.sqrt(np.sum(p * p)) for p in parts])
    bound = 1e-3 * want_n + 1e-4 * np.sqrt(np.array(sizes, np.float64))
    assert np.all(np.abs(got_n - want_n) <= bound), float(np.max(np.abs(got_n - want_n) / bound))
