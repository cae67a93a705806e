"""Held-out evaluation on the CPU: the oracle's tally (crates/modelspec-runtime/src/train/eval.rs:
520-601) pinned against the reference's own known answers (eval.rs:603-634, runner.rs:633-638),
against the forward program's CrossEntropy on one batch (eval.rs:24-30: over one batch the loss
is the bits of that batch's cross_entropy), against float64 brute force over several batches,
and the host's finishing of device sums (HeldOut::metrics_of_sums, eval.rs:299-339) against the
tally's own division."""
import numpy as np
import pytest

from ops_lib import Draw, Prog


def tally(oracle, logits, labels, weights):
    return oracle.held_out_tally(logits, labels, weights)


def test_a_row_of_equal_logits_has_the_nll_ln_v(oracle):
    # eval.rs:607-611: row_nll([0; 4], 2) == ln 4 in f32.
    got = tally(oracle, np.zeros((1, 1, 4), np.float32), np.array([[2]]), np.ones((1, 1), np.float32))
    assert np.float32(got["loss"]).tobytes() == np.float32(np.log(np.float32(4.0))).tobytes()


def test_a_tie_goes_to_the_lowest_id_and_a_nan_row_never_hits(oracle):
    # runner.rs:633-638 and eval.rs:628-633: argmax([1, 3, 3, 2]) = 1; a row with a NaN has none.
    row = np.array([1.0, 3.0, 3.0, 2.0], np.float32)
    logits = np.stack([row, row, np.array([1.0, np.nan, 0.0, 0.0], np.float32)])[None]
    w = np.array([[1.0, 1.0, 0.0]], np.float32)
    got = tally(oracle, logits, np.array([[1, 2, 0]]), w)
    assert got["correct"] == 1 and got["selected"] == 2 and got["accuracy"] == np.float32(0.5)
    # The NaN row has weight 0, yet its nll is NaN and 0 * NaN poisons the numerator.
    assert np.isnan(got["loss"])


def test_one_batch_is_the_bits_of_its_cross_entropy(oracle):
    d = Draw(11)
    rows, V = 9, 13
    x = d.values(rows * V).reshape(rows, V)
    labels = np.array([0, 12, 5, 5, 3, 7, 1, 2, 11], np.int32)
    w = np.array([1.0, 0.0, 2.0, 0.5, 1.0, 0.0, 3.0, 1.0, 0.25], np.float32)
    p = Prog()
    xi, li, wi = p.input("x", (rows, V)), p.input("labels", (rows,), "i32"), p.input("w", (rows,))
    p.out(p.op("CrossEntropy", [xi, li, wi], ()))
    ce = oracle.run_program(p.text(), {"x": x, "labels": labels, "w": w}, (), outputs=(0,))[0]
    got = tally(oracle, x[None], labels[None], w[None])
    assert np.float32(got["loss"]).tobytes() == np.float32(ce[0]).tobytes()


@pytest.mark.parametrize("v", [1, 7, 1000])
def test_several_batches_against_float64(oracle, v):
    rng = np.random.default_rng(v)
    batches, rows = 3, 17
    logits = (rng.standard_normal((batches, rows, v)) * 3).astype(np.float32)
    labels = rng.integers(0, v, (batches, rows)).astype(np.int32)
    weights = rng.choice(np.array([0.0, 1.0, 0.5, 2.0], np.float32), (batches, rows))
    got = tally(oracle, logits, labels, weights)
    x = logits.astype(np.float64).reshape(-1, v)
    m = x.max(axis=1)
    nll = m + np.log(np.exp(x - m[:, None]).sum(axis=1)) - x[np.arange(x.shape[0]), labels.reshape(-1)]
    w = weights.reshape(-1).astype(np.float64)
    assert abs(got["numerator"] - np.sum(w * nll)) <= 1e-5 * np.sum(np.abs(w * nll)) + 1e-6
    assert got["denominator"] == np.sum(w)
    want = np.float32(np.sum(w * nll) / np.sum(w))
    assert abs(got["loss"] - want) <= 1e-6 * abs(want) + 1e-7
    # np.argmax takes the first largest, the reference rule.
    sel = w > 0
    hits = np.argmax(logits.reshape(-1, v), axis=1) == labels.reshape(-1)
    assert got["selected"] == sel.sum() and got["correct"] == (hits & sel).sum()


def test_no_weight_gives_zero_loss_and_accuracy(oracle):
    x = np.ones((2, 3, 4), np.float32)
    got = tally(oracle, x, np.zeros((2, 3), np.int32), np.zeros((2, 3), np.float32))
    assert got["loss"] == 0.0 and got["accuracy"] == 0.0 and got["selected"] == 0


def test_a_label_outside_the_classes_is_refused(oracle):
    with pytest.raises(ValueError, match="label"):
        tally(oracle, np.zeros((1, 2, 3), np.float32), np.array([[0, 3]]), np.ones((1, 2), np.float32))


@pytest.mark.parametrize("config", ["mlp_micro", "bert_micro"])
def test_the_host_finishes_device_sums_to_the_tally(oracle, config):
    # Every evaluation of a run: the host's metrics_of_sums over the sums equals the tally's own
    # loss and accuracy bit for bit; step 0 and the last step are evaluated, and every multiple.
    evals = oracle.train_eval(config, 6, 4, 2)
    assert [s for s, _, _ in evals] == [0, 4, 6]
    for step, host, own in evals:
        assert np.float32(host[0]).tobytes() == np.float32(own[0]).tobytes(), step
        assert host[1] == own[1], step
        assert np.isfinite(host[0]) and host[0] > 0
