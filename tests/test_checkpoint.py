"""The .msckpt v1 checkpoint on the CPU (crates/modelspec-runtime/src/train/checkpoint.rs, the
format of the reference's DESIGN.md 6.2): the byte layout the reference's own tests check
(tests/checkpoint.rs:50-180), the refusals in the reference's order and codes, resumed runs equal
to runs that never stopped (SGD, and AdamW with its moments, which the reference cannot resume),
and the schema hash against the reference's artifact fixture."""
import json
import os
import struct

import numpy as np
import pytest

NIL = "00000000-0000-0000-0000-000000000000"


def parse(path):
    b = open(path, "rb").read()
    msize = struct.unpack_from("<Q", b, 16)[0]
    return b, json.loads(b[56:56 + msize]), msize


def test_the_schema_hash_is_the_reference_artifacts(oracle):
    # core/tests/fixtures/adversary_transposed_base_linear_regression/artifact.json:11.
    assert oracle.schema_hash("linear_regression") == "a3c150bea8dcd814ba09eeea6f77739aa6bb61ccd311cbf19669b3edb53e4868"


@pytest.mark.parametrize("v,text", [(1.0, "1.0"), (0.5, "0.5"), (0.1, "0.1"), (100.0, "100.0"), (0.001, "0.001"),
                                    (123.456, "123.456"), (-2.5, "-2.5"), (0.0, "0.0"),
                                    (float(np.float32(0.1)), "0.10000000149011612")])
def test_floats_are_written_as_serde_json_writes_them(oracle, v, text):
    assert oracle.json_f64(v) == text
    assert float(oracle.json_f64(v)) == v


def test_floats_read_back_exactly(oracle):
    rng = np.random.default_rng(0)
    for v in list(rng.standard_normal(200) * 10.0 ** rng.integers(-30, 30, 200)) + [1e-6, 1e16, 1e-5, 5e-324]:
        assert float(oracle.json_f64(float(v))) == float(v)


def test_the_header_and_payload_have_the_documented_layout(oracle, tmp_path):
    path = tmp_path / "lr.msckpt"
    losses, params, start = oracle.train_ckpt("linear_regression", 5, path=path)
    assert start == 0
    b, m, msize = parse(path)
    # tests/checkpoint.rs:50-83.
    assert b[0:4] == b"MSCK" and struct.unpack_from("<I", b, 4)[0] == 1
    assert b[8:12] == bytes([4, 3, 2, 1]) and struct.unpack_from("<I", b, 12)[0] == 0
    signed = bytearray(b[:56 + msize])
    signed[24:56] = bytes(32)
    assert oracle.blake3(bytes(signed)) == b[24:56]
    assert m["file_size"] == len(b) and m["alignment"] == 64 and m["step"] == 5
    assert m["optimizer_slots"] == [] and m["optimizer"] == {"kind": "Sgd", "learning_rate": float(np.float32(0.1))}
    assert m["rng"] == {"algorithm": "Philox4x32x10", "seed": 42, "counter": 0}
    assert m["schema_hash"] == oracle.schema_hash("linear_regression")
    # tests/checkpoint.rs:85-123: 64-byte aligned, zero gaps, payload hash, the values themselves.
    (rec,) = m["parameters"]
    assert rec == {"path": "LinearReg.w", "dtype": "F32", "shape": [4, 1], "offset": rec["offset"], "length": 16}
    assert rec["offset"] % 64 == 0 and rec["offset"] >= 56 + msize and rec["offset"] + 16 == len(b)
    assert not any(b[56 + msize:rec["offset"]])
    assert oracle.blake3(b[rec["offset"]:]).hex() == m["payload_hash"]
    assert np.frombuffer(b[rec["offset"]:], "<f4").tobytes() == params.tobytes()
    # The id: blake3 of the manifest with the nil UUID in its place (checkpoint.rs:497-503).
    unnamed = b[56:56 + msize].replace(m["checkpoint_id"].encode(), NIL.encode())
    assert oracle.uuid_of(list(oracle.blake3(b"modelspec-checkpoint-id/1\n" + unnamed))) == m["checkpoint_id"]
    # Compact JSON, the reference's field order.
    assert list(m) == ["checkpoint_id", "file_size", "alignment", "schema_hash", "step", "payload_hash", "optimizer",
                       "optimizer_slots", "rng", "parameters"]
    assert b" " not in b[56:56 + msize]


def test_the_same_state_writes_the_same_bytes(oracle, tmp_path):
    oracle.train_ckpt("mlp_micro", 3, path=tmp_path / "a.msckpt")
    oracle.train_ckpt("mlp_micro", 3, path=tmp_path / "b.msckpt")
    oracle.train_ckpt("mlp_micro", 4, path=tmp_path / "c.msckpt")
    a, b, c = (open(tmp_path / f, "rb").read() for f in ("a.msckpt", "b.msckpt", "c.msckpt"))
    assert a == b and a != c


def test_an_adamw_checkpoint_carries_its_moments(oracle, tmp_path):
    path = tmp_path / "bm.msckpt"
    oracle.train_ckpt("bert_micro", 6, path=path)
    b, m, _ = parse(path)
    opt = m["optimizer"]
    assert opt["kind"] == "AdamW" and set(opt) == {"kind", "learning_rate", "weight_decay", "beta1", "beta2",
                                                   "epsilon", "schedule"}
    slots = m["optimizer_slots"]
    paths = sorted({r["path"] for r in m["parameters"]})
    assert [r["path"] for r in m["parameters"]] == paths
    assert sorted((r["path"], r["slot"]) for r in slots) == [(r["path"], r["slot"]) for r in slots]
    assert {r["slot"] for r in slots} == {"m", "v"} and len(slots) == 2 * len(paths)
    for r in slots:
        v = np.frombuffer(b[r["offset"]:r["offset"] + r["length"]], "<f4")
        assert np.any(v != 0) and (r["slot"] == "m" or np.all(v >= 0))


@pytest.mark.parametrize("config,total,cut", [("linear_regression", 50, 20), ("mlp_micro", 20, 7), ("bert_micro", 20, 8)])
def test_a_resumed_run_equals_one_that_never_stopped(oracle, tmp_path, config, total, cut):
    # tests/checkpoint.rs:149-178, and AdamW (bert_micro: dropout, gather, moments, schedule). The
    # checkpoint is the one a whole run writes after `cut` updates, so the learning-rate schedule
    # of both runs ends at `total`.
    path = tmp_path / "run.msckpt"
    whole_l, whole_p, _ = oracle.train_ckpt(config, total, every=cut, path=path)
    rest_l, rest_p, start = oracle.train_ckpt(config, total - cut, resume=tmp_path / f"run-{cut}.msckpt")
    assert start == cut
    assert rest_p.tobytes() == whole_p.tobytes()
    assert rest_l.tobytes() == whole_l[cut:].tobytes()
    # The end checkpoint of the resumed run is the whole run's, byte for byte.
    oracle.train_ckpt(config, total - cut, resume=tmp_path / f"run-{cut}.msckpt", path=tmp_path / "again.msckpt")
    assert open(tmp_path / "again.msckpt", "rb").read() == open(path, "rb").read()


def test_checkpoints_every_n_updates(oracle, tmp_path):
    path = tmp_path / "run.msckpt"
    oracle.train_ckpt("mlp_micro", 10, every=4, path=path)
    assert sorted(os.listdir(tmp_path)) == ["run-4.msckpt", "run-8.msckpt", "run.msckpt"]
    assert parse(tmp_path / "run-8.msckpt")[1]["step"] == 8 and parse(path)[1]["step"] == 10


def damaged(oracle, tmp_path, edit):
    path = tmp_path / "ck.msckpt"
    oracle.train_ckpt("mlp_micro", 2, path=path)
    b = bytearray(open(path, "rb").read())
    out = tmp_path / "bad.msckpt"
    open(out, "wb").write(bytes(edit(b)))
    with pytest.raises(RuntimeError) as e:
        oracle.train_ckpt("mlp_micro", 1, resume=out)
    return str(e.value)


@pytest.mark.parametrize("case,code", [
    ("magic", "E-CKPT-001"), ("version", "E-CKPT-001"), ("endian", "E-CKPT-001"), ("reserved", "E-CKPT-001"),
    ("short", "E-CKPT-002"), ("manifest_size", "E-CKPT-002"), ("checksum", "E-CKPT-001"), ("manifest", "E-CKPT-001"),
    ("gap", "E-CKPT-002"), ("payload", "E-CKPT-004"), ("tail", "E-CKPT-002"),
])
def test_a_damaged_file_is_refused_with_the_reference_code(oracle, tmp_path, case, code):
    def edit(b):
        msize = struct.unpack_from("<Q", b, 16)[0]
        if case == "magic": b[0] ^= 1
        elif case == "version": b[4] = 2
        elif case == "endian": b[8:12] = bytes([1, 2, 3, 4])
        elif case == "reserved": b[12] = 1
        elif case == "short": return b[:40]
        elif case == "manifest_size": b[16:24] = struct.pack("<Q", len(b))
        elif case == "checksum": b[30] ^= 1
        elif case == "manifest": b[60] ^= 1
        elif case == "gap":
            first = min(r["offset"] for r in json.loads(b[56:56 + msize])["parameters"])
            if first == 56 + msize:
                pytest.skip("no gap before the first tensor")
            b[first - 1] = 7
        elif case == "payload": b[-5] ^= 1
        elif case == "tail": b += bytes(64)
        return b
    assert code in damaged(oracle, tmp_path, edit)


def test_another_model_is_refused(oracle, tmp_path):
    # tests/checkpoint.rs:211-231: refused at the first parameter path that differs.
    path = tmp_path / "lr.msckpt"
    oracle.train_ckpt("linear_regression", 2, path=path)
    with pytest.raises(RuntimeError, match="E-CKPT-003.*path"):
        oracle.train_ckpt("mlp_micro", 1, resume=path)


DIVERGING = """model LinearReg {
    param w: Tensor<f32, [4, 1]> = xavier_uniform();

    fn forward(x: Tensor<f32, [8, 4]>) -> Tensor<f32, [8, 1]> {
        return matmul(x, w);
    }
}

train Fit {
    model = LinearReg;
    input x: Tensor<f32, [8, 4]>;
    target y: Tensor<f32, [8, 1]>;
    loss = mse(model.forward(x), y);
    optimizer = sgd(lr = 1e30);
    steps = 6;
    seed = 42;
    device = cpu;
}
"""


def test_a_diverged_run_stops_and_writes_no_later_checkpoint(oracle, tmp_path):
    """cli/src/train.rs:39-44: a run whose loss stops being finite stops with E-TRAIN-001, and the
    state is checked where it is read back, so no checkpoint holds a non-finite loss's state. At
    lr 1e30 the first update leaves finite parameters of order 1e30 (written at step 1) and the
    loss of step 1 overflows; the read-back before the step-2 checkpoint shows it."""
    src = tmp_path / "diverge.mspec"
    src.write_text(DIVERGING)
    path = tmp_path / "run.msckpt"
    with pytest.raises(RuntimeError, match=r"E-TRAIN-001.*step 1\b"):
        oracle.train_ckpt(str(src), 6, every=1, path=str(path))
    assert (tmp_path / "run-1.msckpt").exists()
    assert not (tmp_path / "run-2.msckpt").exists()
    assert not path.exists()
    with pytest.raises(RuntimeError, match="E-TRAIN-001"):
        oracle.train(str(src))


def test_a_parameter_that_overflows_is_named_by_its_path(oracle, tmp_path):
    """runner.rs:156-227: with the losses finite, the diagnostic names the parameters the update
    left non-finite by canonical path. At lr 1e38 the first SGD update overflows w to inf while the
    loss of step 0 is finite; a one-step run reads it back after its last update."""
    src = tmp_path / "overflow.mspec"
    src.write_text(DIVERGING.replace("lr = 1e30", "lr = 1e38").replace("steps = 6", "steps = 1"))
    with pytest.raises(RuntimeError, match=r"E-TRAIN-001: the update of step 1 leaves a parameter not finite: @\S*w"):
        oracle.train(str(src))
