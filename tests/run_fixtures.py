"""The committed oracle runs of tests/golden/ (written by tests/golden/make_oracle_losses.py) and
the reference's run tolerance applied to them (crates/modelspec-runtime/tests/common/mod.rs:17-40):
every loss and every kept parameter element within 1e-4 + 1e-3 |c|; an attention key bias, whose
exact gradient is zero so that both backends carry only rounding noise there, within
1e-4 + steps * lr * 1e-3 (zero_gradient_bound); and every other tensor within the reference's
whole-tensor bound ||g - c|| <= 1e-4 ||c||, estimated from its kept elements."""
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
RUN_ATOL, RUN_RTOL = 1e-4, 1e-3


def path(kind, config, steps, ext):
    return os.path.join(GOLDEN, f"oracle_{kind}_{config}_{steps}.{ext}")


def available(config, steps):
    return all(os.path.exists(path(k, config, steps, e))
               for k, e in (("losses", "npy"), ("param_norms", "npy"), ("params", "npz"), ("meta", "json")))


def load(config, steps):
    """(losses, norms, idx, val, meta) of a committed run; idx is every index when stored empty."""
    losses = np.load(path("losses", config, steps, "npy"))
    norms = np.load(path("param_norms", config, steps, "npy"))
    with np.load(path("params", config, steps, "npz")) as z:
        idx, val = z["idx"].astype(np.int64), z["val"]
    if idx.size == 0:
        idx = np.arange(val.size, dtype=np.int64)
    with open(path("meta", config, steps, "json")) as f:
        meta = json.load(f)
    return losses, norms, idx, val, meta


def param_tolerance(step_ir, steps, lr, key_biases):
    """Per-element absolute tolerance of the flat parameter vector (before the relative term)."""
    from modelspec_amd import api
    atol = []
    for p, shape in api.param_shapes(step_ir):
        n = int(np.prod(shape))
        atol.append(np.full(n, RUN_ATOL + (steps * lr * 1e-3 if p in key_biases else 0.0)))
    return np.concatenate(atol)


def check_run(got_losses, got_params, config, steps, lr, step_ir, key_biases, l2_bound=True):
    """Asserts a device run against the committed oracle run of (config, steps); with l2_bound
    also the reference's whole-tensor bound on every tensor but the key biases."""
    want_l, want_n, idx, val, _ = load(config, steps)
    assert got_losses.shape == want_l.shape, (got_losses.shape, want_l.shape)
    assert np.all(np.isfinite(got_losses))
    ok = np.abs(got_losses - want_l) <= RUN_ATOL + RUN_RTOL * np.abs(want_l)
    assert ok.all(), (config, np.flatnonzero(~ok)[:5], got_losses[~ok][:5], want_l[~ok][:5])
    atol = param_tolerance(step_ir, steps, lr, key_biases)
    g = got_params[idx]
    bad = np.abs(g - val) > atol[idx] + RUN_RTOL * np.abs(val)
    assert not bad.any(), (config, int(bad.sum()), idx[bad][:5], g[bad][:5], val[bad][:5])
    # The reference's whole-tensor bound of a run (run_within, tests/common/mod.rs:469-485):
    # ||g - c|| <= 1e-4 ||c|| for every tensor but the key biases, with ||g - c||^2 estimated from
    # the tensor's kept elements (all of them for a tensor of at most 1,024 elements or a fully
    # stored run; a seeded uniform sample otherwise, scaled by size / kept).
    from modelspec_amd import api
    norm_frac = 0.0
    start = 0
    for k, (p, shape) in enumerate(api.param_shapes(step_ir)):
        n = int(np.prod(shape))
        sel = (idx >= start) & (idx < start + n)
        start += n
        if p in key_biases or not sel.any() or want_n[k] == 0.0:
            continue
        est = np.sqrt(np.sum((g[sel].astype(np.float64) - val[sel]) ** 2) * n / sel.sum())
        frac = est / (1e-4 * want_n[k])
        norm_frac = max(norm_frac, frac)
        print(f"  {p}: ||g - c|| {est:.3e} = {frac:.3f} of 1e-4 ||c|| ({want_n[k]:.4e})", flush=True)
        assert frac <= 1.0 or not l2_bound, (config, p, est, want_n[k])
    # The margins, for the record: the largest difference of each kind as a fraction of its bound.
    loss_frac = float(np.max(np.abs(got_losses - want_l) / (RUN_ATOL + RUN_RTOL * np.abs(want_l))))
    param_frac = float(np.max(np.abs(g - val) / (atol[idx] + RUN_RTOL * np.abs(val))))
    print(f"{config} {steps} steps: worst loss {loss_frac:.3f}, worst parameter {param_frac:.3f} of the tolerance "
          f"({len(idx)} parameter elements), worst tensor ||g - c|| {norm_frac:.3f} of 1e-4 ||c||", flush=True)
