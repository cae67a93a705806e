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


def test_linear_regression_on_the_baseline_distribution(ctx, oracle):
    """BASELINE configs[0] as stated there: x ~ U(-1, 1) [8, 4], w_true ~ U(-1, 1) [4, 1] and
    y = x w_true + N(0, 0.01) noise (standard deviation 0.01), a fresh batch each step, SGD lr 0.1
    for 500 steps from the seed-42 xavier initialisation. The same step program and inputs go to
    the oracle one step at a time (its printed step program: loss, gradient and updated weight);
    the device run must equal it bit for bit, as the golden run does."""
    steps = 500
    step_ir, fwd = api.compile_config("linear_regression")
    rng = np.random.default_rng(20250101)
    w_true = rng.uniform(-1, 1, (4, 1))
    batches = []
    for _ in range(steps):
        x = rng.uniform(-1, 1, (8, 4))
        y = x @ w_true + rng.normal(0, 0.01, (8, 1))
        batches.append({"x": x.astype(np.float32).reshape(-1), "y": y.astype(np.float32).reshape(-1)})
    w0 = oracle.init_params("linear_regression", 4)
    want_l, w = [], w0.copy()
    for b in batches:
        loss, w = oracle.run_program(step_ir, {"x": b["x"], "y": b["y"]}, params=[w], outputs=(0, 2))
        want_l.append(loss[0])
    ctx.load(step_ir, fwd, 42, 1)
    ctx.set_params([w0])
    got_l = ctx.run_steps(batches)
    got_w = ctx.read_param(0, 4)
    assert np.array_equal(np.asarray(got_l, np.float32), np.asarray(want_l, np.float32))
    assert np.array_equal(got_w, w)
    assert want_l[-1] < 1e-3 < want_l[0]  # it fits the teacher down to the noise


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
