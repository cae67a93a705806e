"""Writes the per-step losses of the CPU oracle's run of a config to tests/golden/ as
`oracle_losses_<config>_<steps>.npy` (float32, one loss per step plus the final evaluation, the
array `Oracle.train` returns), for runs too long to repeat inside a test:

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


def main(config, steps):
    t = time.time()
    losses, _, _ = oracle_lib.Oracle().train(config, steps=steps)
    path = os.path.join(HERE, f"oracle_losses_{config}_{steps}.npy")
    np.save(path, losses.astype(np.float32))
    print(path, losses.size, f"{time.time() - t:.0f} s", flush=True)


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]))
