"""Mixed precision on the MI355X (the BERT-base config's f16 MFMA with f32 accumulation and
dynamic loss scaling). The reference trains in f32 only, so there is no reference oracle for this
path: parity is pinned by what the arithmetic fixes and held against the f32 oracle at a stated
looser tolerance.

- A mixed GEMM equals the float64 product of its operands rounded to f16 (round to nearest even),
  up to f32 accumulation: |g - c16| <= 1e-5 * sum |a16 b16| + 1e-30.
- A mixed training run tracks the f32 oracle's run of the same program: every loss within
  2e-2 |c| + 2e-3 (the f16 rounding of each GEMM operand, 2^-11 relative, through 20 AdamW steps).
- Loss scaling: a step whose scaled gradients overflow changes no parameter and halves the scale."""
import os

import numpy as np
import pytest

from modelspec_amd import api
from ops_lib import Prog, fast_values

pytestmark = pytest.mark.gpu


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


@pytest.fixture
def mixed(ctx):
    ctx.set_precision(True)
    yield ctx
    ctx.set_precision(False)


@pytest.mark.parametrize("m,k,n,ta,tb", [(128, 96, 80, False, False), (300, 770, 129, True, False),
                                         (64, 4096, 128, False, True), (832, 128, 4001, True, True),
                                         (33, 45, 17, False, False), (1000, 2100, 3000, False, False),
                                         (777, 2900, 520, True, True), (2880, 768, 4100, False, True)])
def test_a_mixed_gemm_is_the_product_of_f16_operands(mixed, m, k, n, ta, tb):
    a = fast_values(21, m * k, 0.25).reshape((k, m) if ta else (m, k))
    b = fast_values(22, k * n, 0.25).reshape((n, k) if tb else (k, n))
    p = Prog()
    ai, bi = p.input("a", a.shape), p.input("b", b.shape)
    lhs = p.op("Transpose", [ai], (m, k)) if ta else ai
    rhs = p.op("Transpose", [bi], (k, n)) if tb else bi
    p.out(p.op("MatMul", [lhs, rhs], (m, n)))
    prog = mixed.program(p.text())
    prog.run({"a": a, "b": b})
    got = prog.output(0, m * n).reshape(m, n).astype(np.float64)
    A = f16(a.T if ta else a)
    Bm = f16(b.T if tb else b)
    want = A @ Bm
    bound = 1e-5 * (np.abs(A) @ np.abs(Bm)) + 1e-30
    assert np.all(np.abs(got - want) <= bound), float(np.max(np.abs(got - want) / bound))
    # Against the f32 operands the error is the f16 rounding: 2^-11 of each operand's magnitude.
    exact = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 2.0 ** -10 * (np.abs(A) @ np.abs(Bm)) + 1e-6)


@pytest.mark.parametrize("rows,m,n", [(4096, 768, 3072), (2880, 768, 768), (256, 64, 96), (16384, 128, 256),
                                      (100, 40, 24), (1000, 36, 52)])
def test_a_mixed_weight_gradient_takes_the_bias_gradient(mixed, rows, m, n):
    """dW = x^T dy beside db = SumRows(dy), and the transposed form dW^T = dy^T x (the sums as row
    sums of the left operand). Where the f16 GEMM reads both operands' f16 copies (rows whole
    16-byte groups, K a multiple of 32) it takes db from its fragments: the f32 sum of dy rounded to
    f16, |db - sum f16(dy)| <= 1e-5 sum |f16(dy)|. Elsewhere db is the separate f32 column sum of
    dy itself (within 1e-5 of the float64 sum). Both within 2^-10 of the float64 sum of dy."""
    x, dy = fast_values(41, rows * m, 0.5).reshape(rows, m), fast_values(42, rows * n, 0.5).reshape(rows, n)
    p = Prog()
    xi, di = p.input("x", (rows, m)), p.input("dy", (rows, n))
    dw = p.op("MatMul", [p.op("Transpose", [xi], (m, rows)), di], (m, n))
    db = p.op("SumRows", [di], (n,))
    dwt = p.op("MatMul", [p.op("Transpose", [di], (n, rows)), xi], (n, m))
    p.out(dw, db, dwt)
    prog = mixed.program(p.text())
    prog.run({"x": x, "dy": dy})
    gw = prog.output(0, m * n).reshape(m, n).astype(np.float64)
    gb = prog.output(1, n).astype(np.float64)
    gt = prog.output(2, n * m).reshape(n, m).astype(np.float64)
    X, D = f16(x), f16(dy)
    r = np.abs(X.T) @ np.abs(D)
    assert np.all(np.abs(gw - X.T @ D) <= 1e-5 * r + 1e-30)
    assert np.all(np.abs(gt - D.T @ X) <= 1e-5 * r.T + 1e-30)
    fused = m % 8 == 0 and n % 8 == 0 and rows % 32 == 0
    want = D.sum(0) if fused else dy.astype(np.float64).sum(0)
    mag = np.abs(D).sum(0)
    assert np.all(np.abs(gb - want) <= 1e-5 * mag + 1e-30), float(np.max(np.abs(gb - want) / mag))
    assert np.all(np.abs(gb - dy.astype(np.float64).sum(0)) <= 2.0 ** -10 * mag)


@pytest.mark.parametrize("B,S,H,heads,masked", [(2, 128, 128, 2, True), (32, 176, 768, 12, True), (16, 272, 256, 16, False),
                                                (2, 64, 256, 2, True), (4, 256, 256, 4, True), (2, 512, 128, 2, False),
                                                (8, 128, 768, 12, True)])
def test_mixed_attention_and_gradients(mixed, oracle, B, S, H, heads, masked):
    """Attention on the f16 MFMA (q, k, v, P, dO and dS rounded to f16, f32 accumulation and softmax
    statistics) against the oracle's f32 values: within 1e-3 + 4e-3 (|c| + r), r the f32 test's
    magnitude bound, i.e. a few f16 roundings (2^-11 each) of the terms. 64-wide heads over rows
    that are multiples of 128 take the f16-copy kernels (flash16), the others attention.hip's."""
    from test_gpu_ops import both
    n = B * S * H
    q, k, v, G = (fast_values(s, n, 0.5).reshape(B * S, H) for s in (12, 13, 14, 15))
    mask = np.ones((B, S), np.float32)
    if masked:
        rng = np.random.default_rng(1)
        mask[rng.random((B, S)) < 0.3] = 0.0
        mask[:, 0] = 1.0
    p = Prog()
    qi, ki, vi = p.input("q", (B * S, H)), p.input("k", (B * S, H)), p.input("v", (B * S, H))
    mi, Gi = p.input("mask", (B, S)), p.input("G", (B * S, H))
    attr = f"[heads = {heads}]"
    outs = [p.op("Attention", [qi, ki, vi, mi], (B * S, H), attr)]
    for op in ("AttentionGradQ", "AttentionGradK", "AttentionGradV"):
        outs.append(p.op(op, [qi, ki, vi, mi, Gi], (B * S, H), attr))
    got, want = both(mixed, oracle, p.out(*outs), {"q": q, "k": k, "v": v, "mask": mask, "G": G}, (0, 1, 2, 3))
    d = H // heads
    r = np.abs(v).max() + np.abs(G).max() * (np.abs(q).max() + np.abs(k).max()) * np.sqrt(d) * 2
    for idx, (g, w) in enumerate(zip(got, want)):
        err = np.abs(g.astype(np.float64) - w) / (1e-3 + 4e-3 * (np.abs(w) + r))
        assert np.all(err <= 1.0), (idx, float(err.max()))
        # Not the f32 path: f16 rounding shows (the f32 kernels agree to 1e-5 + 1e-4 (|c| + r)).
        if idx == 0:
            assert np.max(np.abs(g - w)) > 1e-6
    if masked:
        dead = np.flatnonzero(mask.reshape(-1) == 0)
        for g in (got[2], got[3]):
            assert np.all(g.reshape(B * S, H)[dead] == 0)


def test_a_mixed_run_tracks_the_f32_oracle(ctx, oracle):
    got_l, got_p, _ = ctx.train_config("bert_micro_mixed")
    want_l, want_p, _ = oracle.train("bert_micro")
    assert np.all(np.isfinite(got_l))
    err = np.abs(got_l - want_l)
    assert np.all(err <= 2e-2 * np.abs(want_l) + 2e-3), (got_l, want_l)
    # Parameters: the bulk close to the f32 run (AdamW normalises each update, so an element with
    # a near-zero gradient may move by up to lr per step either way).
    close = np.abs(got_p - want_p) <= 1e-2 * np.abs(want_p) + 3e-3
    assert close.mean() > 0.99, close.mean()
    assert ctx.loss_scale() == (65536.0, 0)


def test_gemm_only_values_are_kept_as_f16_copies_alone(ctx):
    """The BERT FFN's GELU output and the gradient of its pre-activation are read only by f16 GEMMs
    (and the bias-gradient sums those take): their producers write the f16 copy alone. The run
    itself is checked against the f32 oracle by the test above."""
    _, _, loss, rows = api.bench_config(ctx, "bert_micro_mixed", 1, 2, profile_reps=1)
    only = [r[0] for r in rows if "(f16 only)" in r[0]]
    assert np.isfinite(loss)
    assert any("+Gelu" in w for w in only) and any("+GeluGrad" in w for w in only), only
    assert all("k_gemm_lds16" in r[4] for r in rows if "(f16 only)" in r[0])


GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_the_seq_512_mixed_config_trains_and_tracks_the_f32_oracle(ctx):
    # The oracle's f32 run of this config takes a minute on one core: its losses are a fixture
    # written by tests/golden/make_oracle_losses.py.
    print("bert_mini_mixed", flush=True)
    got_l, _, _ = ctx.train_config("bert_mini_mixed", steps=2)
    want_l = np.load(os.path.join(GOLDEN, "oracle_losses_bert_mini_mixed_2.npy"))
    assert np.all(np.isfinite(got_l))
    assert np.all(np.abs(got_l - want_l) <= 2e-2 * np.abs(want_l) + 2e-3), (got_l, want_l)
    losses, _, _ = ctx.train_config("bert_mini_mixed")
    assert np.all(np.isfinite(losses)) and losses[-1] < losses[0]


def test_an_overflowing_step_is_skipped_and_halves_the_scale(ctx, oracle):
    config = "bert_micro_mixed"
    step_ir, fwd = api.compile_config(config)
    ctx.load_packed(None)
    ctx.set_precision(True, loss_scale=1e38)
    try:
        ctx.load(step_ir, fwd, 42, 1)
    finally:
        ctx.set_precision(False)
    n = api.param_count(step_ir)
    sizes = [int(np.prod(s)) for _, s in api.param_shapes(step_ir)]
    init = oracle.init_params(config, n)
    ctx.set_params(np.split(init, np.cumsum(sizes)[:-1]))
    # The same batch three times: with no update in between, the three losses are one value.
    losses = ctx.run_steps([oracle.step_inputs(config, 0, steps=20)] * 3)
    after = np.concatenate([ctx.read_param(k, c) for k, c in enumerate(sizes)])
    assert after.tobytes() == init.tobytes()
    assert np.all(np.isfinite(losses)) and losses[0] == losses[1] == losses[2]
    scale, skipped = ctx.loss_scale()
    assert skipped == 3 and scale == np.float32(1e38) / 8


def test_the_bert_base_config_takes_two_steps(ctx):
    """BERT-base (12 layers, H 768, V 30522, batch 32, seq 512) at its full shape: no oracle run
    finishes at this size, so the check is what initialisation fixes. With xavier weights the first
    loss is within 3 nats of ln V (logits of order one). The step after it is finite and the scale
    has not overflowed."""
    print("bert_base", flush=True)
    losses, _, _ = ctx.train_config("bert_base", steps=2)
    assert np.all(np.isfinite(losses)), losses
    assert abs(losses[0] - np.log(30522)) < 3.0, losses
    assert ctx.loss_scale() == (65536.0, 0)


def test_the_bert_base_config_trains_for_its_whole_run(ctx):
    """BERT-base mixed for the config's whole run (200 steps, AdamW with warm-up, dynamic loss
    scale): every loss finite, the run learning (the last ten losses below the first ten), and at
    most a few steps skipped for an overflow of the scaled gradients (the scale starts at 2^16)."""
    steps = api.config_steps("bert_base")
    print("bert_base", steps, flush=True)
    losses, _, _ = ctx.train_config("bert_base")
    assert len(losses) == steps + 1 and np.all(np.isfinite(losses)), losses
    assert losses[-10:].mean() < losses[:10].mean(), (losses[:10], losses[-10:])
    scale, skipped = ctx.loss_scale()
    assert skipped <= 8 and scale >= 1.0, (scale, skipped)
