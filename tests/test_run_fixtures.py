"""The committed oracle runs are current: their programs hash to what the configs compile to now
(BLAKE3 of the printed step and forward programs), their first loss (before any update, so
independent of the run's length) is the oracle's own bit for bit, their parameter sample is the
documented seeded one, and they hold one norm per parameter tensor. A failure here asks for the
fixture to be rewritten (tests/golden/make_oracle_losses.py), not for the device to be fixed."""
import numpy as np
import pytest

from modelspec_amd import api

import run_fixtures

RUNS = [("mlp_classifier", 1000), ("transformer_block", 500), ("bert_tiny", 1000)]


@pytest.mark.parametrize("config,steps", RUNS)
def test_fixture_is_current(oracle, config, steps):
    if not run_fixtures.available(config, steps):
        pytest.skip(f"no committed oracle run of {config} for {steps} steps")
    import sys, os
    sys.path.insert(0, run_fixtures.GOLDEN)
    import make_oracle_losses as mk
    losses, norms, idx, val, meta = run_fixtures.load(config, steps)
    assert meta == mk.program_hashes(config, steps)
    step_ir, _ = api.compile_config(config, -1, steps)
    sizes = [int(np.prod(s)) for _, s in api.param_shapes(step_ir)]
    assert norms.shape == (len(sizes),) and np.all(norms > 0)
    assert losses.shape == (steps + 1,) and losses.dtype == np.float32
    assert np.array_equal(idx, np.arange(sum(sizes)) if idx.size == sum(sizes) else mk.sample_indices(sizes))
    assert val.size == idx.size and np.all(np.isfinite(val))
    first, _, _ = oracle.train(config, steps=1)
    assert np.float32(first[0]).tobytes() == losses[0].tobytes()
