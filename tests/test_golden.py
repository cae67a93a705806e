"""The reference's own golden files, reproduced by the host compiler and the CPU oracle.

- crates/modelspec-cli/tests/golden/linear_regression.training.ir and mnist_mlp.training.ir:
  lowering, autodiff order and SGD attachment (ir/print.rs text), byte for byte.
- crates/modelspec-cli/tests/golden/linear_regression.train.stdout: a whole 500-step CPU run
  (blake3 path ids, Philox streams 0/1/2, xavier, Box-Muller, the teacher, matmul, mse, SGD and
  the print format), byte for byte.
"""
import os

import numpy as np

from modelspec_amd import api

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def read(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return f.read()


def rust_display(x):
    """Rust's `{}` of an f32: shortest round-trip digits, never an exponent."""
    return np.format_float_positional(np.float32(x), unique=True, trim="-")


def test_training_ir_goldens():
    for config, golden in [("linear_regression", "linear_regression.training.ir"),
                           ("mnist_mlp", "mnist_mlp.training.ir")]:
        step_ir, _ = api.compile_config(config)
        assert step_ir == read(golden), config


def test_linear_regression_run_reproduces_the_golden_stdout(oracle):
    losses, params, _ = oracle.train("linear_regression")
    init = oracle.init_params("linear_regression", 4)
    fmt = lambda v: "[" + ", ".join(rust_display(x) for x in v) + "]"
    lines = [f"init @LinearReg.w: Tensor<f32, [4, 1]> = {fmt(init)}"]
    for k in range(0, 501):
        if k % 50 == 0 or k == 500:
            lines.append(f"step {k} loss {rust_display(losses[k])}")
    lines.append(f"param @LinearReg.w: Tensor<f32, [4, 1]> = {fmt(params)}")
    assert "\n".join(lines) + "\n" == read("linear_regression.train.stdout")


def test_every_config_round_trips_through_the_parser():
    for config in api.CONFIGS:
        step_ir, forward_ir = api.compile_config(config)
        assert api.check_ir(step_ir) == step_ir, config


def test_bert_tiny_step_gathers_832_masked_rows():
    step_ir, forward_ir = api.compile_config("bert_tiny")
    assert 'Input "masked.rows"' in step_ir and "Tensor<i32, [832]>" in step_ir
    assert 'Input "masked.weights.weights"' in step_ir and 'Input "masked.labels.labels"' in step_ir
    ce = [l for l in step_ir.splitlines() if "= CrossEntropy " in l]
    assert len(ce) == 1 and ce[0].startswith("loss ")
    # The gathered head: the logits the loss reads are [832, 30522]; the full head stays for the
    # forward program, which computes [4096, 30522].
    assert "Tensor<f32, [832, 30522]> = AddRows" in step_ir
    assert "Tensor<f32, [4096, 30522]> = AddRows" in forward_ir
    sites = [l for l in step_ir.splitlines() if l.split("= ")[-1].startswith("Input \"BertTiny.forward.dropout#")]
    assert len(sites) == 5
    assert "Dropout" not in forward_ir
    # 41 parameters, 4,367,290 floats (V = 30522).
    shapes = api.param_shapes(step_ir)
    assert len(shapes) == 41
    assert sum(int(np.prod(s)) for _, s in shapes) == 4367290
    # AdamW with the example's hyperparameters.
    assert "optimizer adamw lr = 0.0001 weight_decay = 0.01 beta1 = 0.9 beta2 = 0.999 eps = 1e-6 warmup_steps = 100" in step_ir


def test_default_masked_rows_capacity():
    # crates/modelspec-cli/src/train.rs:380-389: 832 for 4096 rows at 0.15.
    import math
    def cap(rows, rate):
        bound = rows * rate + 8 * math.sqrt(rows * rate * (1 - rate))
        return min(rows, -(-math.ceil(bound) // 64) * 64)
    assert cap(4096, 0.15) == 832
    step_ir, _ = api.compile_config("bert_micro")
    assert f"Tensor<i32, [{cap(128, 0.15)}]> = Input \"masked.rows\"" in step_ir


def test_the_1000_step_fixture_starts_where_the_oracle_does(oracle):
    """tests/golden/oracle_losses_bert_tiny_1000.npy is the oracle's BERT-tiny run: its first loss
    (before any update, so independent of the run's length) is the oracle's, bit for bit, and the
    parameter-norm fixture has one norm per parameter tensor of the step program."""
    from modelspec_amd import api
    golden = os.path.join(os.path.dirname(__file__), "golden")
    want = np.load(os.path.join(golden, "oracle_losses_bert_tiny_1000.npy"))
    norms = np.load(os.path.join(golden, "oracle_param_norms_bert_tiny_1000.npy"))
    assert want.shape == (1001,) and want.dtype == np.float32
    step_ir, _ = api.compile_config("bert_tiny", -1, 1000)
    assert norms.shape == (len(api.param_shapes(step_ir)),) and np.all(norms > 0)
    got, _, _ = oracle.train("bert_tiny", steps=1)
    assert np.float32(got[0]).tobytes() == want[0].tobytes()
