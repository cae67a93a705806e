"""This backend's launch and buffer plans checked against the reference's own Kernel IR goldens
(crates/modelspec-cli/tests/golden/{linear_regression,mnist_mlp}.kernel.ir, copied under
tests/golden/): every fusion group of the reference's step and forward plans is one launch here,
completing the same value, with the same fused operation chain or epilogue, in an order that keeps
every buffer dependency of the reference plan; operands the reference reads transposed are read in
place here too (no Transpose launch); every value a reference dispatch writes has storage here
(the arena, or the gradient arena for a gradient the optimizer reads). Planned without a device
(msx_plan), so this runs on the CPU.

Where this backend plans differently, by design: the reference's one sgd_update kernel a parameter
is one optimizer launch over the flat parameter arena; a RecordLoss launch appends the step's loss
to the device loss log (the reference's loss slots, kernel.rs:1515; where a cross-entropy loss
launch forms the loss, that launch appends it); weight-gradient GEMMs that only the optimizer reads
run on the side stream."""
import os

import pytest

from modelspec_amd import api

import kernel_ir

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def plans(config):
    ref = kernel_ir.parse_reference(open(os.path.join(GOLDEN, f"{config}.kernel.ir")).read())
    step_ir, forward_ir = api.compile_config(config)
    ours = kernel_ir.parse_plan(api.plan(step_ir, forward_ir))
    return ref, ours, step_ir


def label(kernel):
    """The fused chain as this backend names it: Sub>Mul for the reference's Sub>Mul@0."""
    return ">".join(op.split("@")[0] for op in kernel["ops"])


@pytest.mark.parametrize("config", ["linear_regression", "mnist_mlp"])
@pytest.mark.parametrize("which", ["step", "forward"])
def test_every_reference_fusion_group_is_one_launch(config, which):
    ref, ours, step_ir = plans(config)
    launches = ours[which]["launches"]
    assert not any(l["what"].startswith("Transpose") for l in launches)
    placed = {}
    for d in ref["plans"][which]:
        k = ref["kernels"][d["kernel"]]
        if k["kind"] == "sgd_update":
            hits = [i for i, l in enumerate(launches) if l["what"] in ("SGD", "AdamW")]
        else:
            hits = [i for i, l in enumerate(launches) if d["value"] in l["values"]]
        assert len(hits) == 1, (config, which, d, [l["what"] for l in launches])
        what = launches[hits[0]]["what"]
        if k["kind"] == "matmul":
            assert what.startswith("MatMul"), what
            if k["epilogue"]:
                assert f"+{k['epilogue']} %" in what, (k, what)
        elif k["kind"] == "elementwise":
            assert what.startswith(label(k)), (k, what)
        elif k["kind"] == "loss_sum":
            assert what.startswith(k["ops"][0]), (k, what)
        placed[(d["kernel"], d["value"])] = hits[0]
    # Buffer dependencies of the reference plan keep their order here.
    ds = ref["plans"][which]
    for i, a in enumerate(ds):
        for b in ds[i + 1:]:
            if set(a["writes"]) & set(b["reads"]):
                pa, pb = placed[(a["kernel"], a["value"])], placed[(b["kernel"], b["value"])]
                assert pa < pb or ref["kernels"][b["kernel"]]["kind"] == "sgd_update", (a, b)
    # Every launch here is a reference group, or the loss log (step), or the loss (forward: the
    # reference's forward plan is the prediction's; this backend's forward program also gives the
    # final and held-out loss).
    groups = set(placed.values())
    extra = [l["what"].split()[0] for i, l in enumerate(launches) if i not in groups]
    assert extra == (["RecordLoss"] if which == "step" else ["Mse"]), extra


@pytest.mark.parametrize("config", ["linear_regression", "mnist_mlp"])
def test_every_value_a_reference_dispatch_writes_has_storage(config):
    ref, ours, step_ir = plans(config)
    gradients = {int(l.split("%")[1].split()[0]) for l in step_ir.splitlines()
                 if l.startswith("output %") and " gradient @" in l}
    for which in ("step", "forward"):
        slices = ours[which]["slices"]
        launches = ours[which]["launches"]
        for d in ref["plans"][which]:
            k = ref["kernels"][d["kernel"]]
            if k["kind"] == "sgd_update":
                continue  # the parameter arena, updated in place
            stored = lambda v: v in slices or (which == "step" and v in gradients)
            if k["epilogue"]:
                # A group with an epilogue stores its epilogue's value (the reference's buffer of the
                # dispatch holds it too): the other value of the launch completing d.
                owner = next(l for l in launches if d["value"] in l["values"])
                assert any(stored(v) for v in owner["values"] if v != d["value"]), (config, which, d, owner)
            else:
                assert stored(d["value"]), (config, which, d)


def test_the_forward_program_is_the_reference_tensor_ir_with_the_prediction():
    """golden/linear_regression.tensor.ir is the reference's lowered forward program; this
    backend's forward program is it with the prediction appended as a second output (held-out
    evaluation and synthetic teacher targets read it)."""
    _, forward_ir = api.compile_config("linear_regression")
    want = open(os.path.join(GOLDEN, "linear_regression.tensor.ir")).read()
    assert forward_ir == want + "output %3\n"


def test_bert_tiny_step_plan_takes_the_fused_paths():
    """The BERT-tiny step (the benchmark and the 1,000-step parity run) plans the fusions the GPU
    op tests check one by one: the Embedding gathers inside the LayerNorm pass, the masked-row
    scatter with its DropoutGrad, the Q/K/V input-gradient chains as K-segment GEMMs (one ending in
    a DropoutGrad epilogue), the loss summed and logged by a block of the optimizer launch (with the
    deferred column finalize), the EmbeddingGrad plans made on the host, and no Dropout,
    DropoutGrad, Embedding, RecordLoss, loss, finalize or EmbeddingPlan launch of its own."""
    step_ir, forward_ir = api.compile_config("bert_tiny")
    launches = kernel_ir.parse_plan(api.plan(step_ir, forward_ir))["step"]["launches"]
    whats = [l["what"] for l in launches]
    assert any(w.startswith("LayerNorm+fused") and w.count(" embedding %") == 2 for w in whats), whats
    assert any(w.startswith("EmbeddingGrad") and "+DropoutGrad %" in w for w in whats), whats
    chains = [w for w in whats if w.startswith("MatMul") and w.count(" (+) ") == 2]
    assert len(chains) == 2 and sum("+DropoutGrad %" in w for w in chains) == 1, chains
    assert any(w.startswith("ColumnFinalize") and "+ AdamW + CrossEntropyRows" in w and "+RecordLoss" in w
               for w in whats), whats
    assert not any(w.split()[0] in ("Dropout", "DropoutGrad", "Embedding", "RecordLoss", "AdamW") for w in whats), whats
    assert sum(w.startswith("CrossEntropyRows") for w in whats) == 1, whats
    # The EmbeddingGrad plans of the host-staged ids are made by the host with the step's inputs.
    assert not any(w.startswith("EmbeddingPlan") for w in whats), whats
