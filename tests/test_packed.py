"""The packed masked-language-model data path on the CPU: the directory format and its refusals
(crates/modelspec-runtime/src/dataset/mlm.rs:588-662, train/data.rs:1448-1640), uuid_of and
binding_id (dataset/mod.rs:212-239, mlm.rs:161-185), the epoch order (mlm.rs:665-680) and the
oracle's rows of a draw (mlm.rs:717-788) against the reference's own tests of them
(tests/mlm.rs, tests/adversary_mlm_batches.rs, dataset/mod.rs:233-239) and what the rules fix."""
import json
import os

import numpy as np
import pytest

from modelspec_amd import api

SEQ, V = 16, 300


def corpus(rng, sequences, specials_every=7):
    ids = rng.integers(5, V, sequences * SEQ).astype(np.int32)
    ids[::specials_every] = rng.integers(0, 5, ids[::specials_every].size)
    return ids


@pytest.fixture
def packed(tmp_path):
    rng = np.random.default_rng(3)
    path = tmp_path / "packed"
    api.write_packed(path, corpus(rng, 40), corpus(rng, 20), SEQ, V)
    return str(path)


def test_uuid_of_marks_version_8_and_the_variant(oracle):
    # dataset/mod.rs:233-239.
    assert oracle.uuid_of([0xFF] * 32) == "ffffffff-ffff-8fff-bfff-ffffffffffff"
    assert oracle.uuid_of([0] * 32) == "00000000-0000-8000-8000-000000000000"
    # The reference's artifact fixture: artifact_id is uuid_of(artifact_hash)
    # (core/tests/fixtures/adversary_transposed_base_linear_regression/artifact.json:3-5).
    digest = bytes.fromhex("23cb168aea426941cbb843cd379283a76510f4cc29490a98381350fed3d26ca8")
    assert oracle.uuid_of(list(digest)) == "23cb168a-ea42-8941-8bb8-43cd379283a7"


def test_binding_id_hashes_the_ids_the_length_and_the_rates(oracle):
    bert = [0.15, 0.8, 0.1, 0.1]
    a = oracle.binding_id(api.DATASET_ID, api.TOKENIZER_ID, SEQ, bert)
    assert a is not None and a[14] == "8"
    # One ulp of any rate, the length, or either id moves it (tests/adversary_mlm_batches.rs:373-396).
    for k in range(4):
        r = list(bert)
        r[k] = float(np.nextafter(r[k], 1.0))
        assert oracle.binding_id(api.DATASET_ID, api.TOKENIZER_ID, SEQ, r) != a
    assert oracle.binding_id(api.DATASET_ID, api.TOKENIZER_ID, SEQ + 1, bert) != a
    assert oracle.binding_id(api.TOKENIZER_ID, api.DATASET_ID, SEQ, bert) != a
    assert oracle.binding_id("not-a-uuid", api.TOKENIZER_ID, SEQ, bert) is None
    # By the formula: blake3(dataset 16 bytes || tokenizer 16 bytes || seq_len LE || 4 rates LE).
    raw = bytes.fromhex(api.DATASET_ID.replace("-", "")) + bytes.fromhex(api.TOKENIZER_ID.replace("-", ""))
    raw += SEQ.to_bytes(8, "little") + np.array(bert, "<f8").tobytes()
    assert oracle.uuid_of(list(oracle.blake3(raw))) == a


def test_the_artifact_fixture_pins_multi_block_blake3(oracle):
    # ir_hash of the reference's artifact fixture is blake3 of the printed training step of
    # linear regression (903 bytes, 15 blocks of one chunk), which tests/golden holds byte for byte.
    here = os.path.dirname(os.path.abspath(__file__))
    text = open(os.path.join(here, "golden", "linear_regression.training.ir"), "rb").read()
    assert len(text) > 64
    assert oracle.blake3(text).hex() == "84b42026bf9b34acda2576ba079637bc2118546f9bb65926c157a5d08e34e05a"


@pytest.mark.parametrize("n", [1, 2, 3, 17, 100])
def test_epoch_order_is_a_permutation_sorted_by_the_tag_5_key(oracle, n):
    seed = 0x0123456789ABCDEF
    for epoch in (0, 1, 1 << 32):
        order = oracle.epoch_order(seed, epoch, n)
        assert sorted(order.tolist()) == list(range(n))
        key = lambda i: (lambda w: (w[1] << 32) | w[0])(
            oracle.philox([i, 5, epoch & 0xFFFFFFFF, epoch >> 32], [seed & 0xFFFFFFFF, seed >> 32]))
        keys = [(key(i), i) for i in range(n)]
        assert order.tolist() == [i for _, i in sorted(keys)]
    assert n < 3 or not np.array_equal(oracle.epoch_order(seed, 0, n), oracle.epoch_order(seed, 1, n))


def test_a_packed_directory_reads_back_and_records_what_pack_records(packed):
    b = json.load(open(os.path.join(packed, "binding.json")))
    p = json.load(open(os.path.join(packed, "packed.json")))
    assert b["seq_len"] == SEQ and b["masking_policy"] == {
        "selection_rate": 0.15, "mask_fraction": 0.8, "random_fraction": 0.1, "keep_fraction": 0.1}
    assert p["binding_id"] == b["binding_id"] and p["vocabulary_size"] == V
    assert [s["role"] for s in p["splits"]] == ["Train", "HeldOut"]
    assert [s["sequence_count"] for s in p["splits"]] == [40, 20]
    assert p["heldout_unigram_baseline_nats"] > 0


def loads(oracle, path):
    try:
        oracle.corpus_draw("bert_cpu", path, 0, 0, 2 * SEQ)
        return None
    except RuntimeError as e:
        return str(e)


def rewrite(path, name, edit):
    full = os.path.join(path, name)
    data = open(full, "rb").read()
    open(full, "wb").write(edit(data))


@pytest.mark.parametrize("case", ["flip", "short", "id", "binding", "vocab", "rate"])
def test_a_damaged_directory_is_refused_naming_the_file(oracle, packed, case):
    assert loads(oracle, packed) is None
    if case == "flip":      # tests/adversary_mlm_batches.rs:350-371
        rewrite(packed, "train.tokens", lambda d: d[:5] + bytes([d[5] ^ 1]) + d[6:])
        want = "train.tokens"
    elif case == "short":
        rewrite(packed, "heldout.tokens", lambda d: d[:-4])
        want = "heldout.tokens"
    elif case == "id":
        rng = np.random.default_rng(1)
        api.write_packed(packed, np.full(40 * SEQ, 7, np.int32), corpus(rng, 20), SEQ, V)
        rewrite(packed, "train.tokens", lambda d: np.full(40 * SEQ, V, np.int32).tobytes())
        want = "train.tokens"
    elif case == "binding":
        rewrite(packed, "binding.json", lambda d: d.replace(b'"seq_len": 16', b'"seq_len": 17'))
        want = "binding.json"
    elif case == "vocab":   # tests/adversary_mlm_batches.rs:277-302
        rewrite(packed, "packed.json", lambda d: d.replace(b'"vocabulary_size": 300', b'"vocabulary_size": 5'))
        want = "packed.json"
    else:
        rewrite(packed, "binding.json", lambda d: d.replace(b'"selection_rate": 0.15', b'"selection_rate": 0.25'))
        want = "binding.json"
    err = loads(oracle, packed)
    assert err is not None and want in err, err


def test_a_program_of_another_vocabulary_is_refused(tmp_path, oracle):
    rng = np.random.default_rng(2)
    path = str(tmp_path / "wide")
    api.write_packed(path, rng.integers(5, 400, 40 * SEQ), rng.integers(5, 400, 20 * SEQ), SEQ, 400)
    with pytest.raises(RuntimeError, match="E-DATA-006"):
        oracle.corpus_draw("bert_cpu", path, 0, 0, 2 * SEQ)


def test_a_draw_follows_the_tag_3_derivation(oracle, packed):
    # tests/mlm.rs:195-240 and tests/adversary_mlm_batches.rs:139-200: every row from its block.
    seed = 42  # the config's seed
    train = np.fromfile(os.path.join(packed, "train.tokens"), "<i4").reshape(-1, SEQ)
    heldout = np.fromfile(os.path.join(packed, "heldout.tokens"), "<i4").reshape(-1, SEQ)
    B = 2
    per_epoch = train.shape[0] // B
    seen = []
    for role, step in [(0, 0), (0, 1), (0, per_epoch + 3), (1, 0), (1, 9), (1, 10)]:
        d = oracle.corpus_draw("bert_cpu", packed, role, step, B * SEQ)
        if role == 0:
            order = oracle.epoch_order(seed, step // per_epoch, train.shape[0])
            seqs = order[(step % per_epoch) * B:(step % per_epoch + 1) * B]
            src = train[seqs].reshape(-1)
            draw_id = step
            seen.append(tuple(seqs))
        else:
            b = step % (heldout.shape[0] // B)
            src = heldout[b * B:(b + 1) * B].reshape(-1)
            draw_id = step + (1 << 63)
        assert np.array_equal(d["labels"], src)
        assert np.array_equal(d["positions"], np.tile(np.arange(SEQ), B))
        for r in range(B * SEQ):
            w = oracle.philox([r, 3, draw_id & 0xFFFFFFFF, draw_id >> 32], [seed, 0])
            u = lambda x: (x + 0.5) / 2.0 ** 32
            label = int(src[r])
            selected = label >= 5 and u(w[0]) < 0.15
            assert (d["weights"][r] == 1.0) == selected and d["weights"][r] in (0.0, 1.0)
            if not selected:
                want = label
            elif u(w[1]) < 0.8:
                want = 4
            elif u(w[1]) < 0.8 + 0.1:
                want = 5 + ((w[2] * (V - 5)) >> 32)
            else:
                want = label
            assert d["ids"][r] == want, (role, step, r)
    assert len(set(seen)) > 1


def test_masking_proportions(oracle, tmp_path):
    # tests/mlm.rs:101-190: over 20 000 positions the selected share is within 0.01 of 0.15 and the
    # mask / random / keep shares of the selected within 0.02 of 0.8 / 0.1 / 0.1; no special token
    # is selected.
    rng = np.random.default_rng(9)
    path = str(tmp_path / "prop")
    api.write_packed(path, corpus(rng, 400), corpus(rng, 20), SEQ, V)
    sel = masked = rand = kept = total = 0
    for step in range(760):
        d = oracle.corpus_draw("bert_cpu", path, 0, step, 2 * SEQ)
        special = d["labels"] < 5
        s = d["weights"] == 1.0
        assert not np.any(s & special) and np.array_equal(d["ids"][~s], d["labels"][~s])
        total += int((~special).sum())
        sel += int(s.sum())
        masked += int((d["ids"][s] == 4).sum())
        kept += int((d["ids"][s] == d["labels"][s]).sum())
    rand = sel - masked - kept
    assert total >= 20000
    assert abs(sel / total - 0.15) < 0.01
    assert abs(masked / sel - 0.8) < 0.02 and abs(rand / sel - 0.1) < 0.02 and abs(kept / sel - 0.1) < 0.02


def test_the_gather_of_a_draw_holds_its_selected_rows(oracle, packed):
    # train/masked.rs:97-118: rows of non-zero weight ascending, then row 0 / label 0 / +0.
    rows, cap = 8 * SEQ, 64
    for step in range(3):
        d = oracle.corpus_draw("bert_micro", packed, 0, step, rows, cap)
        sel = np.flatnonzero(d["weights"])
        n = sel.size
        assert np.array_equal(d["g_rows"][:n], sel)
        assert np.array_equal(d["g_labels"][:n], d["labels"][sel]) and np.all(d["g_weights"][:n] == 1.0)
        assert not d["g_rows"][n:].any() and not d["g_labels"][n:].any()
        assert np.all(d["g_weights"][n:].view(np.uint32) == 0)


def test_a_packed_run_evaluates_the_held_out_split(oracle, packed):
    losses, params, evals = oracle.train_packed("bert_cpu", packed, 6, 3, 0)
    assert np.all(np.isfinite(losses)) and losses.size == 7
    assert [s for s, _, _ in evals] == [0, 3, 6]
    for _, host, own in evals:
        assert np.float32(host[0]).tobytes() == np.float32(own[0]).tobytes() and host[1] == own[1]


def test_a_gather_too_small_for_the_selection_is_refused(oracle, tmp_path):
    rng = np.random.default_rng(4)
    path = str(tmp_path / "dense")
    api.write_packed(path, rng.integers(5, V, 40 * SEQ), rng.integers(5, V, 20 * SEQ), SEQ, V, selection_rate=0.9)
    with pytest.raises(RuntimeError, match="E-DATA-012"):
        oracle.train_packed("bert_micro", path, 2)
