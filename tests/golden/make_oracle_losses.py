"""Writes the per-step losses of the CPU oracle's run of a config to tests/golden/ as
`oracle_losses_<config>_<steps>.npy` (float32, one loss per step plus the final evaluation, the
array `Oracle.train` returns), and the L2 norm (float64) of each parameter tensor after the run,
in the step program's parameter order, as `oracle_param_norms_<config>_<steps>.npy`, for runs too
long to repeat inside a test:

  python tests/golden/make_oracle_losses.py bert_tiny 1000
  python tests/golden/make_oracle_losses.py bert_mini_mixed 2

The oracle is deterministic (fixed seeds, -ffp-contract=off, no threads), so a rerun reproduces
each file byte for byte."""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle_lib  # noqa: E402
from modelspec_amd import api  # noqa: E402


def param_norms(config, steps, params):
    """The L2 norm of each parameter tensor of the flat `params`, in parameter order."""
    step_ir, _ = api.compile_config(config, -1, steps)
    sizes = [int(np.prod(shape)) for _, shape in api.param_shapes(step_ir)]
    if sum(sizes) != params.size:
        raise ValueError("parameter count differs from the step program's")
    parts = np.split(params.astype(np.float64), np.cumsum(sizes)[:-1])
    return np.array([np.sqrt(np.sum(p * p)) for p in parts])


def main(config, steps):
    t = time.time()
    losses, params, _ = oracle_lib.Oracle().train(config, steps=steps)
    path = os.path.join(HERE, f"oracle_losses_{config}_{steps}.npy")
    np.save(path, losses.astype(np.float32))
    np.save(os.path.join(HERE, f"oracle_param_norms_{config}_{steps}.npy"), param_norms(config, steps, params))
    print(path, losses.size, f"{time.time() - t:.0f} s", flush=True)


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]))
