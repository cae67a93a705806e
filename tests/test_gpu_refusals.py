"""The step path's refusals on the MI355X, through msx_run_steps: the checks the reference makes
before a step reads an id, a label, a weight or a key mask (crates/modelspec-runtime/src/cpu/
interpreter.rs:700-715, 1146-1175, 1240-1262) are MSX_E_DATA, a refused step changes nothing,
and a loss that stops being finite is MSX_E_NONFINITE (E-TRAIN-001) naming its step
(train/runner.rs:410-470)."""
import re

import numpy as np
import pytest

from modelspec_amd import api

pytestmark = pytest.mark.gpu


def table_rows(step_ir, input_name):
    """Rows of the table an Embedding reads with the ids input `input_name`."""
    lines = step_ir.splitlines()
    ids = next(re.search(r"%(\d+):", l).group(1) for l in lines if f'Input "{input_name}"' in l)
    emb = next(l for l in lines if re.search(rf"= Embedding %\d+, %{ids}\b", l))
    table = re.search(r"Embedding %(\d+),", emb).group(1)
    decl = next(l for l in lines if re.search(rf"%{table}:", l))
    return int(re.search(r"\[(\d+),", decl).group(1))


def loaded(ctx, oracle, config):
    step_ir, fwd = api.compile_config(config)
    ctx.load_packed(None)
    ctx.load(step_ir, fwd, 42, 1)
    sizes = [int(np.prod(s)) for _, s in api.param_shapes(step_ir)]
    params = np.split(oracle.init_params(config, sum(sizes)), np.cumsum(sizes)[:-1])
    ctx.set_params(params)
    return step_ir, sizes, params


def refused(ctx, inputs, pattern):
    with pytest.raises(api.MsxError) as e:
        ctx.run_steps([inputs])
    assert e.value.code == -2, (e.value.code, str(e.value))
    assert re.search(pattern, str(e.value)), str(e.value)


def bert_cases(step_ir, good):
    v = table_rows(step_ir, "ids")
    p = table_rows(step_ir, "positions")
    b, s = 8, 16
    cases = []

    def case(name, key, fn, pattern):
        x = {k: a.copy() for k, a in good.items()}
        fn(x[key])
        cases.append((name, x, pattern))

    case("id = rows", "ids", lambda a: a.__setitem__(5, v), "E-DATA-011.*`ids`")
    case("id < 0", "ids", lambda a: a.__setitem__(0, -1), "E-DATA-011.*`ids`")
    case("position = rows", "positions", lambda a: a.__setitem__(3, p), "E-DATA-011.*`positions`")
    case("label = V", "masked.labels.labels", lambda a: a.__setitem__(0, v), "E-DATA-011.*labels")
    case("negative weight", "masked.weights.weights", lambda a: a.__setitem__(1, -0.5), "loss weight 1")
    case("NaN weight", "masked.weights.weights", lambda a: a.__setitem__(2, np.nan), "loss weight 2")
    case("inf weight", "masked.weights.weights", lambda a: a.__setitem__(2, np.inf), "loss weight 2")
    case("key mask 0.5", "key_mask", lambda a: a.__setitem__(7, 0.5), "key mask .*other than 0 and 1")
    case("no unmasked key", "key_mask", lambda a: a.__setitem__(slice(2 * s, 3 * s), 0.0), "sequence 2 has no unmasked key")
    assert good["key_mask"].size == b * s
    return cases


def test_step_inputs_outside_their_domain_are_refused_and_change_nothing(ctx, oracle):
    config = "bert_micro"
    step_ir, sizes, params = loaded(ctx, oracle, config)
    good = oracle.step_inputs(config, 0)
    for name, bad, pattern in bert_cases(step_ir, good):
        print("refusal", config, name, flush=True)
        refused(ctx, bad, pattern)
    # Every refusal happened before the step: the parameters are the initial ones and the next
    # step's loss is the oracle's first loss.
    for k, c in enumerate(sizes):
        assert np.array_equal(ctx.read_param(k, c), params[k]), k
    loss = ctx.run_steps([good])[0]
    want = oracle.train(config, steps=1)[0][0]
    assert abs(loss - want) <= 1e-4 + 1e-3 * abs(want), (loss, want)


def test_a_label_outside_the_classes_is_refused_without_a_gather(ctx, oracle):
    config = "mlp_micro"
    loaded(ctx, oracle, config)
    good = oracle.step_inputs(config, 0)
    for v in (10, -1):
        bad = {k: a.copy() for k, a in good.items()}
        bad["labels"][3] = v
        print("refusal", config, "label", v, flush=True)
        refused(ctx, bad, "E-DATA-011.*`labels`")
    bad = {k: a.copy() for k, a in good.items()}
    bad["weights"][0] = -1.0
    refused(ctx, bad, "loss weight 0")


def test_a_non_finite_loss_stops_at_its_step(ctx, oracle):
    """Three good steps, then a batch whose features overflow the logits: the loss of the fourth
    step (step 3 of the steps run since the parameters were set) is not finite, and the call
    names it."""
    config = "mlp_micro"
    loaded(ctx, oracle, config)
    ctx.run_steps([oracle.step_inputs(config, k) for k in range(3)])
    bad = oracle.step_inputs(config, 3)
    bad["x"] = np.full_like(bad["x"], 3e38)
    print("non-finite loss", config, flush=True)
    with pytest.raises(api.MsxError) as e:
        ctx.run_steps([bad, oracle.step_inputs(config, 4)])
    assert e.value.code == -4
    assert re.search(r"E-TRAIN-001.*step 3\b", str(e.value)), str(e.value)
