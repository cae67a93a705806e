"""The whole compiled step's gradients against central differences of its own loss, on the
oracle: pins the autodiff assembly (adjoint sums, the tied token table's two contributions, the
masked-row gather's scatter, dropout through DropoutGrad) beyond the two IR goldens, the check
crates/modelspec-runtime/tests/gradients_bert_cpu.rs makes for the hidden-32 twin."""
import numpy as np
import pytest

from modelspec_amd import api


def step_program_inputs(oracle, config, step_ir):
    inputs = oracle.step_inputs(config, 0)
    for path, shape in api.param_shapes(step_ir):
        for m in "mv":
            if f'Input "optimizer.{m}@{path}"' in step_ir:
                inputs[f"optimizer.{m}@{path}"] = np.zeros(int(np.prod(shape)), np.float32)
    return inputs


@pytest.mark.parametrize("config", ["bert_micro", "block_micro", "mlp_micro"])
def test_step_gradients_match_central_differences(oracle, config):
    step_ir, _ = api.compile_config(config)
    shapes = api.param_shapes(step_ir)
    sizes = [int(np.prod(s)) for _, s in shapes]
    flat = oracle.init_params(config, sum(sizes))
    params = np.split(flat, np.cumsum(sizes)[:-1])
    inputs = step_program_inputs(oracle, config, step_ir)
    grads_out = [l for l in step_ir.splitlines() if l.startswith("output") and "gradient @" in l]
    paths = [l.split("gradient @")[1] for l in grads_out]
    n_out = 1 + len(paths)
    outs = oracle.run_program(step_ir, inputs, params, seed=42, outputs=tuple(range(n_out)))
    loss0 = outs[0][0]
    assert np.isfinite(loss0)
    rng = np.random.default_rng(0)
    checked = 0
    for k, path in enumerate(paths):
        idx = [p for p, _ in shapes].index(path)
        g = outs[1 + k]
        # The largest gradient entries, where the f32 loss resolves the difference well.
        for e in np.argsort(-np.abs(g))[:2]:
            if abs(g[e]) < 2e-3:
                continue
            eps = np.float32(1e-2 if abs(params[idx][e]) < 1 else 1e-2 * abs(params[idx][e]))
            def loss_at(delta):
                ps = [p.copy() for p in params]
                ps[idx][e] = np.float32(ps[idx][e] + delta)
                return float(oracle.run_program(step_ir, inputs, ps, seed=42, outputs=(0,))[0][0])
            fd = (loss_at(eps) - loss_at(-eps)) / (2 * float(eps))
            assert abs(fd - g[e]) <= 0.05 * abs(g[e]) + 2e-4, (path, int(e), float(g[e]), fd)
            checked += 1
    assert checked >= 4
    del rng
