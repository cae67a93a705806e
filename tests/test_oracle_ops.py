"""The CPU oracle, op by op, against what the mathematics fixes: float64 restatements of each
forward op (numpy), central differences of those for every gradient op (the scheme of
crates/modelspec-runtime/tests/common/finite_difference.rs), exact integer work (gathers,
scatters, dropout masks) and the f64-rounded whole-tensor sums (interpreter.rs:1900-1912)."""
import numpy as np
import pytest

from ops_lib import (Draw, Prog, attention64, central_difference, cross_entropy64, gelu64, layer_norm64,
                     within)


def run(oracle, p, inputs, params=(), outputs=(0,), seed=0):
    return oracle.run_program(p.text(), inputs, params, seed=seed, outputs=outputs)


def test_matmul_plain_and_transposed(oracle):
    d = Draw(1)
    a = d.values(5 * 7).reshape(5, 7)
    b = d.values(7 * 3).reshape(7, 3)
    at = np.ascontiguousarray(a.T)
    bt = np.ascontiguousarray(b.T)
    p = Prog()
    x = p.input("a", (5, 7))
    y = p.input("b", (7, 3))
    xt = p.input("at", (7, 5))
    yt = p.input("bt", (3, 7))
    m0 = p.op("MatMul", [x, y], (5, 3))
    t1 = p.op("Transpose", [xt], (5, 7))
    m1 = p.op("MatMul", [t1, y], (5, 3))
    t2 = p.op("Transpose", [yt], (7, 3))
    m2 = p.op("MatMul", [x, t2], (5, 3))
    p.out(m0, m1, m2)
    outs = run(oracle, p, {"a": a, "b": b, "at": at, "bt": bt}, outputs=(0, 1, 2))
    ref = a.astype(np.float64) @ b.astype(np.float64)
    r = np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64)
    for o in outs:
        ok, worst = within(o.reshape(5, 3), ref, r)
        assert ok, worst
    # The three layouts round identically (the k = 0 product first, then fma in ascending k).
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_matmul_first_product_then_fma_chain(oracle):
    a = np.array([[1.0 + 2 ** -12, 3.0]], np.float32)
    b = np.array([[1.0 - 2 ** -12], [2 ** -30]], np.float32)
    p = Prog()
    m = p.op("MatMul", [p.input("a", (1, 2)), p.input("b", (2, 1))], (1, 1))
    (o,) = run(oracle, p.out(m), {"a": a, "b": b})
    first = np.float32(a[0, 0]) * np.float32(b[0, 0])  # rounded once
    want = np.float32(np.float64(a[0, 1]) * np.float64(b[1, 0]) + np.float64(first))  # fma: one rounding
    assert o[0] == want


def test_layer_norm_and_its_gradients(oracle):
    d = Draw(2)
    rows, h = 6, 8
    x = d.values(rows * h).reshape(rows, h)
    gamma = d.values(h, 0.5)
    beta = d.values(h, 0.5)
    G = d.values(rows * h).reshape(rows, h)
    p = Prog()
    xi, gi, bi, Gi = p.input("x", (rows, h)), p.input("g", (h,)), p.input("b", (h,)), p.input("G", (rows, h))
    y = p.op("LayerNorm", [xi, gi, bi], (rows, h))
    dx = p.op("LayerNormGradX", [xi, gi, Gi], (rows, h))
    dg = p.op("LayerNormGradGamma", [xi, Gi], (h,))
    db = p.op("SumRows", [Gi], (h,))
    p.out(y, dx, dg, db)
    oy, odx, odg, odb = run(oracle, p, {"x": x, "g": gamma, "b": beta, "G": G}, outputs=(0, 1, 2, 3))
    ok, worst = within(oy.reshape(rows, h), layer_norm64(x, gamma, beta), np.abs(layer_norm64(x, gamma, beta)) + 4)
    assert ok, worst
    f_x = lambda xx: float(np.sum(layer_norm64(xx, gamma, beta) * G))
    fd = central_difference(f_x, x)
    assert np.allclose(odx.reshape(rows, h), fd, rtol=1e-3, atol=1e-3)
    f_g = lambda gg: float(np.sum(layer_norm64(x, gg, beta) * G))
    assert np.allclose(odg, central_difference(f_g, gamma), rtol=1e-3, atol=1e-3)
    assert np.allclose(odb, G.astype(np.float64).sum(axis=0), rtol=1e-5, atol=1e-5)


def test_gelu_and_its_gradient(oracle):
    d = Draw(3)
    x = d.values(64)
    G = d.values(64)
    p = Prog()
    xi, Gi = p.input("x", (64,)), p.input("G", (64,))
    y = p.op("Gelu", [xi], (64,))
    dy = p.op("GeluGrad", [xi, Gi], (64,))
    oy, ody = run(oracle, p.out(y, dy), {"x": x, "G": G}, outputs=(0, 1))
    ok, worst = within(oy, gelu64(x), np.abs(gelu64(x)))
    assert ok, worst
    fd = central_difference(lambda xx: float(np.sum(gelu64(xx) * G)), x)
    assert np.allclose(ody, fd, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("masked", [False, True])
def test_attention_and_its_gradients(oracle, masked):
    d = Draw(4)
    B, S, H, heads = 2, 4, 8, 2
    q = d.values(B * S * H, 0.5).reshape(B * S, H)
    k = d.values(B * S * H, 0.5).reshape(B * S, H)
    v = d.values(B * S * H, 0.5).reshape(B * S, H)
    G = d.values(B * S * H, 0.5).reshape(B * S, H)
    mask = np.ones((B, S), np.float32)
    if masked:
        mask[0, 1] = 0.0
        mask[1, 3] = 0.0
    p = Prog()
    qi, ki, vi = p.input("q", (B * S, H)), p.input("k", (B * S, H)), p.input("v", (B * S, H))
    mi, Gi = p.input("mask", (B, S)), p.input("G", (B * S, H))
    attr = f"[heads = {heads}]"
    o = p.op("Attention", [qi, ki, vi, mi], (B * S, H), attr)
    dq = p.op("AttentionGradQ", [qi, ki, vi, mi, Gi], (B * S, H), attr)
    dk = p.op("AttentionGradK", [qi, ki, vi, mi, Gi], (B * S, H), attr)
    dv = p.op("AttentionGradV", [qi, ki, vi, mi, Gi], (B * S, H), attr)
    oo, odq, odk, odv = run(oracle, p.out(o, dq, dk, dv), {"q": q, "k": k, "v": v, "mask": mask, "G": G},
                            outputs=(0, 1, 2, 3))
    ref = attention64(q, k, v, mask, heads)
    assert np.allclose(oo.reshape(B * S, H), ref, rtol=1e-5, atol=1e-5)
    for got, wrt in [(odq, "q"), (odk, "k"), (odv, "v")]:
        def f(t, wrt=wrt):
            args = {"q": q, "k": k, "v": v}
            args[wrt] = t
            return float(np.sum(attention64(args["q"], args["k"], args["v"], mask, heads) * G))
        fd = central_difference(f, {"q": q, "k": k, "v": v}[wrt])
        assert np.allclose(got.reshape(B * S, H), fd, rtol=1e-3, atol=1e-4), wrt
    # A masked key's dK and dV rows are +0 (interpreter.rs:1053-1119).
    if masked:
        rows = [1, S + 3]
        assert np.all(odk.reshape(B * S, H)[rows] == 0) and np.all(odv.reshape(B * S, H)[rows] == 0)


def test_cross_entropy_and_its_gradient(oracle):
    d = Draw(5)
    rows, V = 5, 11
    x = d.values(rows * V).reshape(rows, V)
    labels = np.array([0, 3, 10, 7, 2], np.int32)
    w = np.array([1.0, 0.0, 2.0, 1.0, 0.5], np.float32)
    p = Prog()
    xi, li, wi = p.input("x", (rows, V)), p.input("labels", (rows,), "i32"), p.input("w", (rows,))
    loss = p.op("CrossEntropy", [xi, li, wi], ())
    one = p.scalar(1.0)
    g = p.op("CrossEntropyGrad", [xi, li, wi, one], (rows, V))
    ol, og = run(oracle, p.out(loss, g), {"x": x, "labels": labels, "w": w}, outputs=(0, 1))
    assert abs(ol[0] - cross_entropy64(x, labels, w)) <= 1e-5 + 1e-5 * abs(ol[0])
    fd = central_difference(lambda xx: cross_entropy64(xx, labels, w), x)
    assert np.allclose(og.reshape(rows, V), fd, rtol=1e-4, atol=1e-6)
    # All weights zero: the loss and every gradient element are +0.
    ol0, og0 = run(oracle, p, {"x": x, "labels": labels, "w": np.zeros(rows, np.float32)}, outputs=(0, 1))
    assert ol0[0] == 0.0 and np.all(og0 == 0.0)


def test_cross_entropy_refuses_a_label_outside_the_classes(oracle):
    p = Prog()
    xi, li, wi = p.input("x", (2, 3)), p.input("labels", (2,), "i32"), p.input("w", (2,))
    p.out(p.op("CrossEntropy", [xi, li, wi], ()))
    with pytest.raises(RuntimeError, match="label"):
        run(oracle, p, {"x": np.zeros((2, 3), np.float32), "labels": np.array([0, 3], np.int32),
                        "w": np.ones(2, np.float32)})


def test_embedding_and_its_gradient_are_exact(oracle):
    d = Draw(6)
    rows, h, n = 7, 5, 12
    table = d.values(rows * h).reshape(rows, h)
    ids = np.array([3, 0, 3, 6, 1, 3, 0, 2, 2, 6, 5, 3], np.int32)
    G = d.values(n * h).reshape(n, h)
    p = Prog()
    ti, ii, Gi = p.input("t", (rows, h)), p.input("ids", (n,), "i32"), p.input("G", (n, h))
    e = p.op("Embedding", [ti, ii], (n, h))
    g = p.op("EmbeddingGrad", [ii, Gi], (rows, h), f"[{rows}]")
    oe, og = run(oracle, p.out(e, g), {"t": table, "ids": ids, "G": G}, outputs=(0, 1))
    assert np.array_equal(oe.reshape(n, h), table[ids])
    want = np.zeros((rows, h), np.float32)
    for kk, i in enumerate(ids):  # ascending k, one f32 rounding per add, from +0
        want[i] = want[i] + G[kk]
    assert np.array_equal(og.reshape(rows, h).view(np.uint32), want.view(np.uint32))


def test_dropout_masks_follow_the_keep_rule(oracle):
    d = Draw(7)
    n = 97
    x = d.values(n)
    token = np.array([0x1234567, -0x2345678], np.int32)
    seed = 42
    p = Prog()
    xi, ti, gi = p.input("x", (n,)), p.input("tok", (2,), "i32"), p.input("G", (n,))
    y = p.op("Dropout", [xi, ti], (n,), "[p = 0.1, site = tok]")
    dy = p.op("DropoutGrad", [ti, gi], (n,), "[p = 0.1, site = tok]")
    oy, ody = run(oracle, p.out(y, dy), {"x": x, "tok": token, "G": x}, seed=seed, outputs=(0, 1))
    tid = (int(token[0]) & 0xFFFFFFFF) | ((int(token[1]) & 0xFFFFFFFF) << 32)
    scale = np.float32(1.0) / (np.float32(1.0) - np.float32(0.1))
    want = np.array([x[i] * scale if oracle.dropout_keeps(seed, tid, i, 0.1) else 0.0 for i in range(n)], np.float32)
    assert np.array_equal(oy, want) and np.array_equal(ody, want)


def test_whole_tensor_sums_are_f64_rounded_once(oracle):
    d = Draw(8)
    a = d.values(1000)
    b = d.values(1000)
    p = Prog()
    ai, bi = p.input("a", (10, 100)), p.input("b", (10, 100))
    s = p.op("ReduceSum", [ai], ())
    m = p.op("ReduceMean", [ai], ())
    e = p.op("Mse", [ai, bi], ())
    os_, om, oe = run(oracle, p.out(s, m, e), {"a": a, "b": b}, outputs=(0, 1, 2))
    acc = 0.0
    for v in a:  # sequential f64 from the first term
        acc += float(v)
    assert os_[0] == np.float32(acc) and om[0] == np.float32(acc / 1000.0)
    diff = a.astype(np.float64) - b.astype(np.float64)
    assert abs(oe[0] - np.sum(diff * diff) / 1000.0) <= 1e-6 * abs(oe[0])


def test_softmax_and_its_gradient(oracle):
    d = Draw(9)
    x = d.values(4 * 6).reshape(4, 6)
    G = d.values(4 * 6).reshape(4, 6)
    p = Prog()
    xi, Gi = p.input("x", (4, 6)), p.input("G", (4, 6))
    y = p.op("Softmax", [xi], (4, 6))
    dy = p.op("SoftmaxGrad", [y, Gi], (4, 6))
    oy, ody = run(oracle, p.out(y, dy), {"x": x, "G": G}, outputs=(0, 1))

    def sm(t):
        t = t - t.max(axis=1, keepdims=True)
        e = np.exp(t)
        return e / e.sum(axis=1, keepdims=True)
    assert np.allclose(oy.reshape(4, 6), sm(x.astype(np.float64)), rtol=1e-6, atol=1e-7)
    fd = central_difference(lambda t: float(np.sum(sm(t) * G)), x)
    assert np.allclose(ody.reshape(4, 6), fd, rtol=1e-4, atol=1e-6)
