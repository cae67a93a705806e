"""The packed data path on the MI355X: batches drawn, masked and gathered on the device from a
corpus resident in HBM (hip/data.hip) against the oracle's CPU rows of the same draw
(crates/modelspec-runtime/src/dataset/mlm.rs:717-788, train/masked.rs:97-118), bit for bit;
whole runs on a packed directory against the oracle at the reference's run tolerance
(crates/modelspec-runtime/tests/common/mod.rs:17-40); the gather's refusal E-DATA-012."""
import numpy as np
import pytest

from modelspec_amd import api
from test_gpu_train import compare_runs

pytestmark = pytest.mark.gpu

SEED = 42  # the BERT configs' seed


def write_corpus(path, seq, vocab, train_seqs, heldout_seqs, seed=5, selection_rate=0.15):
    rng = np.random.default_rng(seed)
    def ids(n):
        x = rng.integers(5, vocab, n * seq).astype(np.int32)
        x[::11] = rng.integers(0, 5, x[::11].size)
        return x
    api.write_packed(path, ids(train_seqs), ids(heldout_seqs), seq, vocab, selection_rate=selection_rate)
    return str(path)


def step_inputs_without_data(oracle, config, step, steps):
    """The host inputs of a step other than its batch and gather: dropout tokens, AdamW scalars."""
    full = oracle.step_inputs(config, step, steps=steps)
    keep = {k: v for k, v in full.items()
            if k not in ("ids", "positions", "key_mask", "labels", "weights") and not k.startswith("masked.")}
    keep["data.step"] = np.array([step & 0xFFFFFFFF, step >> 32], np.uint32).view(np.int32)
    return keep


@pytest.mark.parametrize("config,seq,vocab,train_seqs,rows,cap", [
    ("bert_micro", 16, 300, 40, 128, 64),
    ("bert_tiny", 128, 30522, 96, 4096, 832),
])
def test_device_draws_are_the_oracle_rows_bit_for_bit(ctx, oracle, tmp_path, config, seq, vocab, train_seqs, rows, cap):
    path = write_corpus(tmp_path / config, seq, vocab, train_seqs, 2 * rows // seq)
    try:
        check_device_draws(ctx, oracle, path, config, seq, train_seqs, rows, cap)
    finally:
        ctx.load_packed(None)


def check_device_draws(ctx, oracle, path, config, seq, train_seqs, rows, cap):
    steps = 8
    step_ir, fwd = api.compile_config(config, -1, steps)
    ctx.load_packed(path)
    ctx.load(step_ir, fwd, SEED, 1)
    n = api.param_count(step_ir)
    sizes = [int(np.prod(s)) for _, s in api.param_shapes(step_ir)]
    ctx.set_params(np.split(oracle.init_params(config, n), np.cumsum(sizes)[:-1]))
    per_epoch = train_seqs // (rows // seq)
    for step in (0, 1, per_epoch + 1):
        print(f"device draw {config} step {step}", flush=True)
        inputs = step_inputs_without_data(oracle, config, step, steps)
        ctx.run_steps([inputs])
        want = oracle.corpus_draw(config, path, 0, step, rows, cap)
        for name in ("ids", "positions"):
            assert ctx.read_input(0, name, rows).tobytes() == want[name].tobytes(), (config, step, name)
        assert np.all(ctx.read_input(0, "key_mask", rows, np.float32) == 1.0)
        # The step program reads labels and weights only through the gather; the forward program,
        # on the same draw, reads them whole.
        ctx.forward({"data.step": inputs["data.step"]})
        for name, dt in (("ids", np.int32), ("labels", np.int32), ("weights", np.float32)):
            assert ctx.read_input(1, name, rows, dt).tobytes() == want[name].tobytes(), (config, step, name)
        assert ctx.read_input(0, "masked.rows", cap).tobytes() == want["g_rows"].tobytes()
        assert ctx.read_input(0, "masked.labels.labels", cap).tobytes() == want["g_labels"].tobytes()
        assert ctx.read_input(0, "masked.weights.weights", cap, np.float32).tobytes() == want["g_weights"].tobytes()
    # Every held-out batch in stored order; the forward program keeps the last one's rows.
    m = ctx.evaluate([], "labels", "weights")
    last = (2 * rows // seq) // (rows // seq) - 1
    want = oracle.corpus_draw(config, path, 1, last, rows)
    assert ctx.read_input(1, "ids", rows).tobytes() == want["ids"].tobytes()
    assert ctx.read_input(1, "weights", rows, np.float32).tobytes() == want["weights"].tobytes()
    assert np.isfinite(m["loss"]) and m["selected"] > 0


@pytest.mark.parametrize("config,steps,every,lr", [("bert_micro", 20, 5, 3e-3), ("bert_cpu", 30, 10, 3e-3)])
def test_a_packed_run_tracks_the_oracle(ctx, oracle, tmp_path, config, steps, every, lr):
    path = write_corpus(tmp_path / config, 16, 300, 40, 20)
    print(f"packed run {config}", flush=True)
    gl, gp, gev = ctx.train_packed(config, path, steps, every, 0)
    wl, wp, wev = oracle.train_packed(config, path, steps, every, 0)
    step_ir, _ = api.compile_config(config, -1, steps)
    compare_runs(config, (gl, gp, None), (wl, wp, None), step_ir, steps, lr)
    assert [s for s, _ in gev] == [s for s, _, _ in wev]
    for (step, got), (_, host, _) in zip(gev, wev):
        assert abs(got["loss"] - host[0]) <= 1e-4 + 1e-3 * abs(host[0]), (step, got, host)
        assert abs(got["accuracy"] - host[1]) <= 2.0 / max(1, got["selected"]) + 1e-6, (step, got, host)


def test_a_gather_too_small_for_the_selection_is_refused(ctx, tmp_path):
    path = write_corpus(tmp_path / "dense", 16, 300, 40, 20, selection_rate=0.9)
    with pytest.raises(api.MsxError) as e:
        ctx.train_packed("bert_micro", path, 2)
    assert e.value.code == -2 and "E-DATA-012" in str(e.value)
