"""Writes the CPU oracle's run of a config to tests/golden/, for runs too long to repeat inside a
test:

- `oracle_losses_<config>_<steps>.npy`: float32, one loss per step plus the final evaluation (the
  array `Oracle.train` returns);
- `oracle_param_norms_<config>_<steps>.npy`: float64, the L2 norm of each parameter tensor after
  the run, in the step program's parameter order;
- `oracle_params_<config>_<steps>.npz`: `idx` (int32, ascending flat indices into the parameter
  vector; empty when it would be every index) and `val` (float32, the oracle's final parameters
  there). Every element when the model has at most 262,144 parameters; otherwise a seeded sample,
  stratified by tensor, of about 65,536 elements plus up to 1,024 of each tensor
  (`sample_indices`);
- `oracle_meta_<config>_<steps>.json`: the BLAKE3 of the printed step and forward programs the
  run compiled, so a test can tell a stale fixture (a changed config or optimizer) from a wrong
  device result.

  python tests/golden/make_oracle_losses.py bert_tiny 1000
  python tests/golden/make_oracle_losses.py transformer_block 500
  python tests/golden/make_oracle_losses.py mlp_classifier 1000
  python tests/golden/make_oracle_losses.py bert_mini_mixed 2

The oracle is deterministic (fixed seeds, -ffp-contract=off, no threads), so a rerun reproduces
each file byte for byte."""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle_lib  # noqa: E402
from modelspec_amd import api  # noqa: E402

FULL_LIMIT = 262144
SAMPLE = 65536
PER_TENSOR = 1024


def tensor_sizes(config, steps):
    step_ir, _ = api.compile_config(config, -1, steps)
    return [int(np.prod(shape)) for _, shape in api.param_shapes(step_ir)]


def sample_indices(sizes):
    """Flat parameter indices the fixture keeps: all of them for a small model, else per tensor
    min(size, 1024 + round(65536 * size / total)) distinct indices drawn by a fixed seed."""
    total = sum(sizes)
    if total <= FULL_LIMIT:
        return np.arange(total, dtype=np.int64)
    rng = np.random.default_rng(0x6d7378)
    out, off = [], 0
    for n in sizes:
        k = min(n, PER_TENSOR + int(round(SAMPLE * n / total)))
        out.append(off + np.sort(rng.choice(n, size=k, replace=False)))
        off += n
    return np.concatenate(out).astype(np.int64)


def param_norms(config, steps, params):
    """The L2 norm of each parameter tensor of the flat `params`, in parameter order."""
    sizes = tensor_sizes(config, steps)
    if sum(sizes) != params.size:
        raise ValueError("parameter count differs from the step program's")
    parts = np.split(params.astype(np.float64), np.cumsum(sizes)[:-1])
    return np.array([np.sqrt(np.sum(p * p)) for p in parts])


def program_hashes(config, steps):
    """BLAKE3 (hex) of the printed step and forward programs of the config at this step count."""
    step_ir, forward_ir = api.compile_config(config, -1, steps)
    b3 = oracle_lib.Oracle().blake3
    return {"config": config, "steps": steps, "step_ir_blake3": b3(step_ir.encode()).hex(),
            "forward_ir_blake3": b3(forward_ir.encode()).hex()}


def main(config, steps):
    t = time.time()
    losses, params, _ = oracle_lib.Oracle().train(config, steps=steps)
    stem = f"{config}_{steps}"
    np.save(os.path.join(HERE, f"oracle_losses_{stem}.npy"), losses.astype(np.float32))
    np.save(os.path.join(HERE, f"oracle_param_norms_{stem}.npy"), param_norms(config, steps, params))
    idx = sample_indices(tensor_sizes(config, steps))
    kept = idx if idx.size < params.size else np.zeros(0, np.int64)
    np.savez(os.path.join(HERE, f"oracle_params_{stem}.npz"), idx=kept.astype(np.int32),
             val=params[idx].astype(np.float32))
    with open(os.path.join(HERE, f"oracle_meta_{stem}.json"), "w") as f:
        json.dump(program_hashes(config, steps), f, indent=1)
        f.write("\n")
    print(stem, losses.size, idx.size, f"{time.time() - t:.0f} s", flush=True)


if __name__ == "__main__":
    main(sys.argv[1], int(sys.argv[2]))
