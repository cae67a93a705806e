"""Hip artifacts on the MI355X: an artifact written from a loaded step reads back, validates, and
loads into a run bit-identical to the step it was written from; an altered artifact is refused
with the reference's codes (crates/modelspec-core/src/artifact.rs:1-35, 330-520: 002 for a module
or manifest changed after sealing, 004 for a missing, longer or stray module file, 001 for the
manifest itself)."""
import json
import os
import shutil

import numpy as np
import pytest

from modelspec_amd import api

pytestmark = pytest.mark.gpu

KEYS = ["format_version", "artifact_id", "backend", "artifact_hash", "source_hash", "ir_hash", "fast_math",
        "deterministic", "compiler_version", "schema_hash", "parameters", "data", "kernels", "plan", "forward_plan",
        "buffers", "loss_view", "prediction_view"]


def written(ctx, oracle, tmp_path, config="bert_micro"):
    step_ir, fwd = api.compile_config(config)
    ctx.load_packed(None)
    ctx.load(step_ir, fwd, 42, 1)
    path = tmp_path / "art"
    h = ctx.write_artifact(path)
    return path, h, step_ir, fwd


def run_steps(ctx, oracle, config, steps):
    step_ir, _ = api.compile_config(config)
    n = api.param_count(step_ir)
    sizes = [int(np.prod(s)) for _, s in api.param_shapes(step_ir)]
    ctx.set_params(np.split(oracle.init_params(config, n), np.cumsum(sizes)[:-1]))
    losses = ctx.run_steps([oracle.step_inputs(config, k, steps=20) for k in range(steps)])
    return losses, np.concatenate([ctx.read_param(k, c) for k, c in enumerate(sizes)])


def test_an_artifact_round_trips_and_runs_as_its_step(ctx, oracle, tmp_path):
    path, h, step_ir, fwd = written(ctx, oracle, tmp_path)
    m = json.load(open(path / "artifact.json"))
    assert list(m)[:len(KEYS)] == KEYS and m["backend"] == "Hip" and m["format_version"] == 1
    assert m["artifact_hash"] == h and m["artifact_id"][14] == "8"
    assert m["ir_hash"] == oracle.blake3(step_ir.encode()).hex()
    assert m["schema_hash"] == oracle.schema_hash("bert_micro")
    assert all(p["canonical_parameter_id"] == oracle.canonical_id(p["path"]) for p in m["parameters"])
    assert len(m["plan"]) > 10 and all(k["kind"] == "code_object" for k in m["kernels"])
    assert sorted(os.listdir(path / "kernels")) == sorted(k["kernel_module_id"] + ".hsaco" for k in m["kernels"])
    assert api.check_artifact(path) == m["artifact_id"]
    # The same step writes the same artifact.
    assert ctx.write_artifact(tmp_path / "again") == h
    # A run of the loaded artifact is the run of the step, bit for bit.
    want_l, want_p = run_steps(ctx, oracle, "bert_micro", 4)
    ctx.load_artifact(path, 42)
    got_l, got_p = run_steps(ctx, oracle, "bert_micro", 4)
    assert got_l.tobytes() == want_l.tobytes() and got_p.tobytes() == want_p.tobytes()


@pytest.mark.parametrize("case,code", [("manifest", "E-ARTIFACT-002"), ("module", "E-ARTIFACT-002"),
                                       ("missing", "E-ARTIFACT-004"), ("stray", "E-ARTIFACT-004"),
                                       ("longer", "E-ARTIFACT-004"), ("version", "E-ARTIFACT-001")])
def test_an_altered_artifact_is_refused(ctx, oracle, tmp_path, case, code):
    path, _, _, _ = written(ctx, oracle, tmp_path)
    bad = tmp_path / "bad"
    shutil.copytree(path, bad)
    kdir = bad / "kernels"
    first = sorted(os.listdir(kdir))[0]
    if case == "manifest":
        text = open(bad / "artifact.json").read().replace('"fast_math": false', '"fast_math": true', 1)
        open(bad / "artifact.json", "w").write(text)
    elif case == "module":
        b = bytearray(open(kdir / first, "rb").read())
        b[-1] ^= 1
        open(kdir / first, "wb").write(bytes(b))
    elif case == "missing":
        os.remove(kdir / first)
    elif case == "stray":
        open(kdir / "extra.hsaco", "wb").write(b"\x7fELF")
    elif case == "longer":
        open(kdir / first, "ab").write(b"\0")
    else:
        text = open(bad / "artifact.json").read().replace('"format_version": 1', '"format_version": 2', 1)
        open(bad / "artifact.json", "w").write(text)
    with pytest.raises(api.MsxError) as e:
        api.check_artifact(bad)
    assert e.value.code == -7 and code in str(e.value), str(e.value)
    with pytest.raises(api.MsxError):
        ctx.load_artifact(bad, 42)
