"""Known answers of the host draws: Philox4x32-10 (Random123 KATs, train/init.rs:424-449),
BLAKE3 (the empty input, init.rs:451-455), the dropout keep threshold at its edges
(spirv/emit/rowwise.rs:1960-2005), and the AdamW schedule and bias corrections against their
closed forms (ir/training.rs:209-230)."""
import numpy as np


def test_philox_kats(oracle):
    kats = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for counter, key, want in kats:
        assert oracle.philox(counter, key) == want


def test_blake3_empty_and_canonical_id(oracle):
    assert oracle.blake3(b"").hex() == "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"
    assert oracle.canonical_id("") == 0xA6A1F9F5B94913AF
    assert oracle.canonical_id("LinearReg.w") != oracle.canonical_id("LinearReg.b")


def test_dropout_ids_differ_by_site_and_step(oracle):
    a = oracle.dropout_id("BertTiny.forward.dropout#0", 0)
    assert a != oracle.dropout_id("BertTiny.forward.dropout#0", 1)
    assert a != oracle.dropout_id("BertTiny.forward.dropout#1", 0)


def test_dropout_id_is_the_first_8_le_bytes_of_blake3_of_site_then_le_step(oracle):
    """train/init.rs:136-146: blake3(site bytes, then step as 8 little-endian bytes), its first 8
    bytes read little-endian. BLAKE3 itself is pinned by the known answers above. Steps above
    2^32 and with distinct bytes catch a 4-byte or big-endian step; two sites catch a dropped
    site."""
    for site in ("BertTiny.forward.dropout#0", "Block.forward.dropout#12", ""):
        for step in (0, 1, 255, 256, 999, 0x0102030405060708, (1 << 32) + 7, (1 << 64) - 1):
            digest = oracle.blake3(site.encode() + step.to_bytes(8, "little"))
            assert oracle.dropout_id(site, step) == int.from_bytes(digest[:8], "little"), (site, step)


def uniform(w):
    return (w + 0.5) / 4294967296.0


def test_keep_threshold_is_the_keep_rule_at_its_edges(oracle):
    exact = (np.float32(uniform(12345)), np.float32(uniform(1 << 23)))
    ps = [0.0, np.finfo(np.float32).tiny, 0.1, 0.25, 0.3, 0.5, 0.9, exact[0], exact[1],
          1.0 - np.finfo(np.float32).eps / 2]
    for p in ps:
        p = float(np.float32(p))
        t = oracle.dropout_threshold(p)
        assert uniform(t) >= p, p
        if t > 0:
            assert not uniform(t - 1) >= p, p
    assert oracle.dropout_threshold(0.0) == 0


def test_threshold_keeps_what_the_rule_keeps(oracle):
    seed, id_ = 0x0123456789ABCDEF, 0xFEEDBEEFDEADF00D
    for p in (0.1, 0.25, 0.5):
        t = oracle.dropout_threshold(p)
        for i in range(0, 4096, 7):
            w = oracle.philox([i, 4, id_ & 0xFFFFFFFF, id_ >> 32], [seed & 0xFFFFFFFF, seed >> 32])[0]
            assert (w >= t) == oracle.dropout_keeps(seed, id_, i, p)


def powi(a, b):
    """compiler-rt __powidf2: the lowering of Rust's f64::powi."""
    r = 1.0
    while True:
        if b & 1:
            r *= a
        b //= 2
        if b == 0:
            break
        a *= a
    return r


def test_adamw_scalars_closed_form(oracle):
    lr, steps, warmup = np.float32(1e-4), 1000, 100
    for t in (1, 2, 50, 100, 101, 500, 999, 1000):
        got = oracle.adamw_scalars(lr, t, steps, warmup)
        peak = float(lr)
        rate = peak * t / warmup if t <= warmup else peak * (steps - t) / (steps - warmup)
        c1 = 1.0 / (1.0 - powi(float(np.float32(0.9)), t))
        c2 = 1.0 / (1.0 - powi(float(np.float32(0.999)), t))
        assert got[0] == np.float32(rate) and got[1] == np.float32(c1) and got[2] == np.float32(c2), t
