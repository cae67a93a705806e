"""Runs compiled from .mspec sources on the MI355X: a config file trains exactly as the built-in
config it restates (same program, so bit-identical losses and parameters), and within the run
tolerance of the CPU oracle's run of the same file."""
import numpy as np
import pytest

from modelspec_amd import api

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("config", ["bert_micro", "mlp_classifier", "linear_regression"])
def test_a_config_file_trains_as_its_builtin(ctx, oracle, config):
    print(config, flush=True)
    steps = 20 if config != "bert_micro" else -1
    got_l, got_p, _ = ctx.train_config(api.config_file(config), steps=steps)
    want_l, want_p, _ = ctx.train_config(config, steps=steps)
    assert got_l.tobytes() == want_l.tobytes() and got_p.tobytes() == want_p.tobytes()
    ref_l, ref_p, _ = oracle.train(api.config_file(config), steps=steps)
    assert np.all(np.abs(got_l - ref_l) <= 1e-4 + 1e-3 * np.abs(ref_l)), (got_l, ref_l)
    assert np.all(np.abs(got_p - ref_p) <= 1e-4 + 1e-3 * np.abs(ref_p))
