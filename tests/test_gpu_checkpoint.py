"""Checkpoints on the MI355X: a device run resumed from its own mid-run checkpoint equals the
device run that never stopped, bit for bit (the step's kernels are deterministic), on synthetic
and packed data, with AdamW moments; and checkpoints move between the device and the CPU oracle
(crates/modelspec-runtime/src/train/checkpoint.rs: loaded into the CPU backend whatever device
wrote it), the continued runs agreeing at the reference's run tolerance
(crates/modelspec-runtime/tests/common/mod.rs:17-40)."""
import numpy as np
import pytest

from modelspec_amd import api
from test_gpu_packed import write_corpus
from test_gpu_train import compare_runs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("config,total,cut,packed", [
    ("linear_regression", 50, 20, False),
    ("mlp_micro", 20, 7, False),
    ("bert_micro", 20, 8, False),
    ("bert_micro", 20, 8, True),
])
def test_a_resumed_device_run_equals_one_that_never_stopped(ctx, tmp_path, config, total, cut, packed):
    print(f"resume {config} packed={packed}", flush=True)
    corpus = write_corpus(tmp_path / "corpus", 16, 300, 40, 20) if packed else None
    path = tmp_path / "run.msckpt"
    whole_l, whole_p, _ = ctx.train_checkpointed(config, total, packed=corpus, every=cut, path=path)
    rest_l, rest_p, start = ctx.train_checkpointed(config, total - cut, packed=corpus,
                                                   resume=tmp_path / f"run-{cut}.msckpt",
                                                   path=tmp_path / "again.msckpt")
    assert start == cut
    assert rest_p.tobytes() == whole_p.tobytes()
    assert rest_l.tobytes() == whole_l[cut:].tobytes()
    assert open(tmp_path / "again.msckpt", "rb").read() == open(path, "rb").read()


@pytest.mark.parametrize("config,total,cut,lr", [("mlp_micro", 20, 7, 0.01), ("bert_micro", 20, 8, 3e-3)])
def test_checkpoints_move_between_the_device_and_the_oracle(ctx, oracle, tmp_path, config, total, cut, lr):
    print(f"interchange {config}", flush=True)
    step_ir, _ = api.compile_config(config)
    # Device -> oracle: the oracle continues the device's mid-run state; so does the device.
    ctx.train_checkpointed(config, total, every=cut, path=tmp_path / "dev.msckpt")
    dev_l, dev_p, _ = ctx.train_checkpointed(config, total - cut, resume=tmp_path / f"dev-{cut}.msckpt")
    orc_l, orc_p, start = oracle.train_ckpt(config, total - cut, resume=tmp_path / f"dev-{cut}.msckpt")
    assert start == cut
    compare_runs(config, (dev_l, dev_p, None), (orc_l, orc_p, None), step_ir, total - cut, lr)
    # Oracle -> device.
    oracle.train_ckpt(config, total, every=cut, path=tmp_path / "orc.msckpt")
    orc_l, orc_p, _ = oracle.train_ckpt(config, total - cut, resume=tmp_path / f"orc-{cut}.msckpt")
    dev_l, dev_p, start = ctx.train_checkpointed(config, total - cut, resume=tmp_path / f"orc-{cut}.msckpt")
    assert start == cut
    compare_runs(config, (dev_l, dev_p, None), (orc_l, orc_p, None), step_ir, total - cut, lr)


def test_a_checkpoint_loads_into_a_loaded_step(ctx, oracle, tmp_path):
    # msx_checkpoint_write / msx_checkpoint_read on a loaded step: the state reads back exactly.
    step_ir, fwd = api.compile_config("bert_micro")
    ctx.load_packed(None)
    ctx.load(step_ir, fwd, 42, 1)
    n = api.param_count(step_ir)
    sizes = [int(np.prod(s)) for _, s in api.param_shapes(step_ir)]
    ctx.set_params(np.split(oracle.init_params("bert_micro", n), np.cumsum(sizes)[:-1]))
    ctx.run_steps([oracle.step_inputs("bert_micro", k, steps=20) for k in range(3)])
    before = [ctx.read_param(k, c) for k, c in enumerate(sizes)]
    moments = [(ctx.read_moment(k, "m", c), ctx.read_moment(k, "v", c)) for k, c in enumerate(sizes)]
    ctx.checkpoint_write(tmp_path / "s.msckpt", 3)
    ctx.set_params([np.zeros(c, np.float32) for c in sizes])
    assert ctx.checkpoint_read(tmp_path / "s.msckpt", resume=True) == 3
    for k, c in enumerate(sizes):
        assert ctx.read_param(k, c).tobytes() == before[k].tobytes()
        assert ctx.read_moment(k, "m", c).tobytes() == moments[k][0].tobytes()
        assert ctx.read_moment(k, "v", c).tobytes() == moments[k][1].tobytes()
    lr_ir, lr_fwd = api.compile_config("linear_regression")
    ctx.load(lr_ir, lr_fwd, 42, 1)
    with pytest.raises(api.MsxError) as e:
        ctx.checkpoint_read(tmp_path / "s.msckpt")
    assert e.value.code == -6 and "E-CKPT-003" in str(e.value)
