"""Held-out evaluation on the MI355X (msx_evaluate, msx_train_config_eval) against the CPU oracle's
tally of crates/modelspec-runtime/src/train/eval.rs.

The device reduces each batch's logits to row losses and hits (held_out_rows) and adds them into
an f64 sum and a count (held_out_sum). On logits handed over as inputs the hits, the correct and
selected counts and the weight sum are exact, and the numerator is within 1e-5 of the sum of the
absolute terms (each row's exp sum is a tree here, ascending in the oracle). Over a training run
the logits themselves come from the device's kernels, so the loss is held to the reference's run
tolerance, 1e-4 + 1e-3 |c| (crates/modelspec-runtime/tests/common/mod.rs:17-40), and the accuracy
to two rows of the selected ones (a near-tie may resolve the other way)."""
import numpy as np
import pytest

from modelspec_amd import api

pytestmark = pytest.mark.gpu


def logits_forward(rows, v):
    """A forward program whose prediction is its input `x`: the held-out reduction alone."""
    _, fwd = api.compile_config("mlp_micro")
    params = [l for l in fwd.splitlines() if l.startswith("param ")]
    return "\n".join(params + [
        f'%0: Tensor<f32, [{rows}, {v}]> = Input "x"',
        f'%1: Tensor<i32, [{rows}]> = Input "labels"',
        f'%2: Tensor<f32, [{rows}]> = Input "weights"',
        "%3: Tensor<f32, []> = CrossEntropy %0, %1, %2",
        "output %3",
        "output %0",
    ]) + "\n"


def load_logits(ctx, rows, v):
    step, _ = api.compile_config("mlp_micro")
    ctx.load(step, logits_forward(rows, v), 0, 1)


def batches_of(logits, labels, weights):
    return [{"x": logits[b], "labels": labels[b], "weights": weights[b]} for b in range(logits.shape[0])]


@pytest.mark.parametrize("v", [10, 1001, 30522])
def test_the_device_reduction_matches_the_tally(ctx, oracle, v):
    rng = np.random.default_rng(v)
    batches, rows = 3, 37
    print(f"held-out reduction v={v}", flush=True)
    logits = (rng.standard_normal((batches, rows, v)) * 4).astype(np.float32)
    labels = rng.integers(0, v, (batches, rows)).astype(np.int32)
    weights = rng.choice(np.array([0.0, 1.0, 0.5, 2.0], np.float32), (batches, rows))
    # Ties: the first largest wins (label at the first copy hits, at the second does not).
    logits[0, 0, :] = 0.0
    logits[0, 0, min(3, v - 1)] = 5.0
    logits[0, 1, :] = 0.0
    labels[0, 0] = 0 if v == 1 else min(3, v - 1)
    weights[0, :2] = 1.0
    if v > 4:
        logits[0, 1, 1] = logits[0, 1, 4] = 5.0
        labels[0, 1] = 4
        # Rows whose label is the largest logit, so the count is not trivially small.
        for r in range(2, rows, 3):
            labels[1, r] = int(np.argmax(logits[1, r]))
    load_logits(ctx, rows, v)
    got = ctx.evaluate(batches_of(logits, labels, weights), "labels", "weights")
    want = oracle.held_out_tally(logits, labels, weights)
    assert got["correct"] == want["correct"] and got["selected"] == want["selected"]
    assert got["denominator"] == want["denominator"]
    x = logits.astype(np.float64).reshape(-1, v)
    m = x.max(axis=1)
    nll = m + np.log(np.exp(x - m[:, None]).sum(axis=1)) - x[np.arange(x.shape[0]), labels.reshape(-1)]
    scale = float(np.sum(np.abs(weights.reshape(-1) * nll)))
    assert abs(got["numerator"] - want["numerator"]) <= 1e-5 * scale + 1e-6
    assert abs(got["loss"] - want["loss"]) <= 1e-5 * abs(want["loss"]) + 1e-6
    assert got["accuracy"] == want["accuracy"]


def test_non_finite_logits_poison_the_loss_as_in_the_tally(ctx, oracle):
    rows, v = 6, 8
    logits = np.zeros((1, rows, v), np.float32)
    logits[0, :, 2] = 1.0
    labels = np.full((1, rows), 2, np.int32)
    weights = np.ones((1, rows), np.float32)
    load_logits(ctx, rows, v)
    # -inf entries beside a finite maximum are ordinary: exp(-inf) = 0.
    logits[0, 1, 5] = -np.inf
    got = ctx.evaluate(batches_of(logits, labels, weights), "labels", "weights")
    want = oracle.held_out_tally(logits, labels, weights)
    assert np.isfinite(got["loss"]) and abs(got["loss"] - want["loss"]) <= 1e-6
    assert got["correct"] == want["correct"] == rows
    for case, value in (("nan", np.nan), ("+inf", np.inf)):
        bad = logits.copy()
        bad[0, 3, 6] = value
        w = weights.copy()
        w[0, 3] = 0.0  # a weight of 0 does not hide a non-finite nll: 0 * NaN is NaN
        got = ctx.evaluate(batches_of(bad, labels, w), "labels", "weights")
        want = oracle.held_out_tally(bad, labels, w)
        assert np.isnan(got["loss"]) and np.isnan(want["loss"]), case
        assert got["correct"] == want["correct"], case
    # Nothing selected: 0 and 0, not NaN (tests/adversary_heldout.rs:1-6).
    got = ctx.evaluate(batches_of(logits, labels, np.zeros_like(weights)), "labels", "weights")
    assert got["loss"] == 0.0 and got["accuracy"] == 0.0 and got["selected"] == 0
    every = np.full((1, rows, v), -np.inf, np.float32)
    got = ctx.evaluate(batches_of(every, labels, weights), "labels", "weights")
    assert np.isnan(got["loss"]) and np.isnan(oracle.held_out_tally(every, labels, weights)["loss"])


def test_a_label_outside_the_classes_is_a_data_error(ctx):
    rows, v = 4, 5
    load_logits(ctx, rows, v)
    logits = np.zeros((1, rows, v), np.float32)
    labels = np.array([[0, 1, 5, 2]], np.int32)
    with pytest.raises(api.MsxError) as e:
        ctx.evaluate(batches_of(logits, labels, np.ones((1, rows), np.float32)), "labels", "weights")
    assert e.value.code == -2


@pytest.mark.parametrize("config,steps,every,batches", [("mlp_micro", 20, 5, 3), ("bert_cpu", 30, 10, 4)])
def test_evaluations_of_a_run_track_the_oracle(ctx, oracle, config, steps, every, batches):
    print(f"held-out run {config}", flush=True)
    losses, evals, _, _ = ctx.train_config_eval(config, every, batches, steps=steps)
    want = oracle.train_eval(config, steps, every, batches)
    assert [s for s, _ in evals] == [s for s, _, _ in want]
    for (step, got), (_, host, _) in zip(evals, want):
        assert abs(got["loss"] - host[0]) <= 1e-4 + 1e-3 * abs(host[0]), (step, got, host)
        assert abs(got["accuracy"] - host[1]) <= 2.0 / max(1, got["selected"]) + 1e-6, (step, got, host)


def test_bert_tiny_evaluation_is_the_forward_loss_on_one_batch(ctx, oracle):
    # Over one batch the held-out loss is that batch's cross_entropy (eval.rs:24-30): the device's
    # reduction and its forward-loss kernels, two different paths, agree at full size.
    print("held-out bert_tiny", flush=True)
    losses, evals, _, _ = ctx.train_config_eval("bert_tiny", 2, 1, steps=2)
    assert [s for s, _ in evals] == [0, 2] and np.all(np.isfinite(losses))
    for step, m in evals:
        # Zipf ids under BERT masking select about 15 % of the 4096 rows.
        assert 400 < m["selected"] < 900 and m["denominator"] == m["selected"]
        assert 9.0 < m["loss"] < 11.5 and 0.0 <= m["accuracy"] < 0.05, (step, m)
    step_ir, fwd = api.compile_config("bert_tiny", -1, 2)
    ctx.load(step_ir, fwd, 42, 1)
    n = api.param_count(step_ir)
    init = oracle.init_params("bert_tiny", n)
    sizes = [int(np.prod(s)) for _, s in api.param_shapes(step_ir)]
    ctx.set_params(np.split(init, np.cumsum(sizes)[:-1]))
    # Held-out batch 0 is the batch drawn at step id 2^63.
    full = oracle.step_inputs("bert_tiny", 1 << 63, steps=2)
    batch = {k: full[k] for k in ("ids", "positions", "key_mask", "labels", "weights")}
    got = ctx.evaluate([batch], "labels", "weights")
    loss, _ = ctx.forward(batch)
    assert abs(got["loss"] - loss) <= 1e-5 * abs(loss), (got, loss)
    # The run's own evaluation at step 0 read the same parameters and batch: the same bits.
    assert np.float32(got["loss"]).tobytes() == np.float32(evals[0][1]["loss"]).tobytes()
    assert got["correct"] == evals[0][1]["correct"] and got["selected"] == int((batch["weights"] > 0).sum())
