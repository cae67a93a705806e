"""Whole training runs on the MI355X against the CPU oracle on the same seed and inputs.

Tolerances are the reference's run tolerances (crates/modelspec-runtime/tests/common/mod.rs:17-40):
every loss and parameter within 1e-4 + 1e-3 |c|, an attention key bias (whose exact gradient is
zero, so both backends carry rounding noise there) within 1e-4 + steps * lr * 1e-3."""
import numpy as np
import pytest

from modelspec_amd import api

pytestmark = pytest.mark.gpu

RUN_ATOL, RUN_RTOL = 1e-4, 1e-3


def key_biases(step_ir):
    """Parameters read only by an AddRows whose result is only an Attention's key operand."""
    lines = [l.split(" ", 1)[1] if l.split(" ", 1)[0] in ("forward", "loss", "gradient", "optimizer") else l
             for l in step_ir.splitlines() if "%" in l and "= " in l and not l.startswith("output")]
    nodes = {}
    for l in lines:
        vid, rest = l.split(":", 1)
        body = rest.split("= ", 1)[1]
        op = body.split()[0]
        operands = [w.strip(",") for w in body.split()[1:] if w.startswith("%")]
        nodes[vid] = (op, operands, body)
    readers = lambda v: [(i, n[0], n[1].index(v)) for i, n in nodes.items() if v in n[1]]
    out = set()
    for vid, (op, _, body) in nodes.items():
        if op != "ParamRead":
            continue
        path = body.split("@")[1].split()[0]
        rs = readers(vid)
        fwd = [r for r in rs if r[1] == "AddRows" and r[2] == 1]
        if fwd and any(n[1] == "Attention" and n[2] == 1 for n in readers(fwd[0][0])):
            out.add(path)
    return out


def compare_runs(config, got, want, step_ir, steps, lr):
    (gl, gp, _), (wl, wp, _) = got, want
    assert np.all(np.isfinite(gl))
    ok = np.abs(gl - wl) <= RUN_ATOL + RUN_RTOL * np.abs(wl)
    assert ok.all(), (config, np.flatnonzero(~ok)[:5], gl[~ok][:5], wl[~ok][:5])
    biases = key_biases(step_ir)
    off = 0
    for path, shape in api.param_shapes(step_ir):
        n = int(np.prod(shape))
        g, w = gp[off:off + n], wp[off:off + n]
        off += n
        atol = RUN_ATOL + (steps * lr * 1e-3 if path in biases else 0.0)
        bad = np.abs(g - w) > atol + RUN_RTOL * np.abs(w)
        assert not bad.any(), (config, path, float(np.max(np.abs(g - w))))


def test_linear_regression_is_bit_identical_to_the_golden_run(ctx, oracle):
    got = ctx.train_config("linear_regression")
    want = oracle.train("linear_regression")
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


@pytest.mark.parametrize("config,steps,lr", [
    ("mnist_mlp", 100, 0.1),
    ("mlp_micro", -1, 0.01),
    ("mlp_classifier", 200, 0.01),
    ("block_micro", -1, 1e-3),
    ("bert_micro", -1, 3e-3),
    ("bert_cpu", 100, 3e-3),
])
def test_run_tracks_the_oracle(ctx, oracle, config, steps, lr):
    step_ir, _ = api.compile_config(config, -1, steps)
    n = steps if steps >= 0 else api.config_steps(config)
    got = ctx.train_config(config, steps=steps)
    want = oracle.train(config, steps=steps)
    compare_runs(config, got, want, step_ir, n, lr)


@pytest.mark.parametrize("config,steps,lr", [("bert_tiny", 2, 1e-4), ("transformer_block", 2, 1e-3)])
def test_full_size_steps_track_the_oracle(ctx, oracle, config, steps, lr):
    step_ir, _ = api.compile_config(config, -1, steps)
    got = ctx.train_config(config, steps=steps)
    want = oracle.train(config, steps=steps)
    compare_runs(config, got, want, step_ir, steps, lr)


@pytest.mark.parametrize("config", ["bert_micro", "transformer_block"])
def test_finalize_inside_adamw_is_bit_identical_to_separate_launches(ctx, config):
    """MSX_FUSE_OPTIMIZER (the default) sums the deferred reductions inside the AdamW launch; the
    separate finalize and AdamW launches give the same bits in every loss and parameter."""
    steps = 6
    try:
        ctx.set_fusion(optimizer=False)
        apart = ctx.train_config(config, steps=steps)
        ctx.set_fusion(optimizer=True)
        fused = ctx.train_config(config, steps=steps)
    finally:
        ctx.set_fusion()
    assert np.array_equal(apart[0], fused[0])
    assert np.array_equal(apart[1], fused[1])
