"""Each HIP kernel against the CPU oracle on the same inputs, through the C ABI (msx_prog_*).

Tolerance per kernel (common/mod.rs:17-40): |g - c| <= 1e-5 + 1e-4 * r, r = |c| elementwise and
the sum of |terms| for contractions and sums. Integer and indexing work (gathers, the sorted-segment
scatter, dropout masks) must match bit for bit."""
import numpy as np
import pytest

from ops_lib import Draw, Prog, fast_values, within

pytestmark = pytest.mark.gpu


def both(ctx, oracle, p, inputs, outputs, seed=0, params=()):
    text = p.text()
    want = oracle.run_program(text, inputs, params, seed=seed, outputs=outputs)
    prog = ctx.program(text, seed)
    try:
        prog.run(inputs, params)
        got = [prog.output(k, w.size) for k, w in zip(outputs, want)]
    finally:
        prog.close()
    return got, want


@pytest.mark.parametrize("m,k,n,ta,tb", [
    (5, 7, 3, False, False), (64, 64, 64, False, False), (130, 70, 33, True, False),
    (33, 129, 65, False, True), (128, 4096, 128, True, False), (832, 128, 1000, False, True),
    (100, 3000, 17, True, True),
])
def test_matmul(ctx, oracle, m, k, n, ta, tb):
    a = fast_values(1, m * k).reshape((k, m) if ta else (m, k))
    b = fast_values(2, k * n).reshape((n, k) if tb else (k, n))
    p = Prog()
    ai = p.input("a", a.shape)
    bi = p.input("b", b.shape)
    lhs = p.op("Transpose", [ai], (m, k)) if ta else ai
    rhs = p.op("Transpose", [bi], (k, n)) if tb else bi
    p.out(p.op("MatMul", [lhs, rhs], (m, n)))
    (g,), (w,) = both(ctx, oracle, p, {"a": a, "b": b}, (0,))
    A = (a.T if ta else a).astype(np.float64)
    B = (b.T if tb else b).astype(np.float64)
    ok, worst = within(g, w, (np.abs(A) @ np.abs(B)).reshape(-1))
    assert ok, worst


@pytest.mark.parametrize("m,k,n,ta,tb,bias", [
    (1000, 64, 2200, False, True, True),    # both operands contiguous along K, ragged tiles
    (520, 96, 4100, False, False, False),   # A along K, B along N; K tiles of 32
    (2048, 80, 1028, True, False, True),    # neither along K (128 x 128 tiles)
    (1500, 48, 1500, True, True, False),    # A along M, B along K
    (100, 8192, 200, False, False, True),   # deep K: split-K slices and their sum
    (36, 9216, 64, True, True, False),      # deep K, split, a 36-row operand along its rows
    (36, 9000, 64, True, True, False),      # a K tail on an unpadded operand: the other kernel
])
def test_large_gemm_layouts(ctx, oracle, m, k, n, ta, tb, bias):
    """The GEMMs of 2^21 outputs or more (or K of 8192 or more) run the direct-to-LDS kernel when
    their layout allows: every pair of operand layouts, partial edge tiles, split-K with its slice
    sum, and the bias epilogue, against the oracle."""
    a = fast_values(91, m * k).reshape((k, m) if ta else (m, k))
    b = fast_values(92, k * n).reshape((n, k) if tb else (k, n))
    bv = fast_values(93, n)
    p = Prog()
    ai, bi_ = p.input("a", a.shape), p.input("b", b.shape)
    lhs = p.op("Transpose", [ai], (m, k)) if ta else ai
    rhs = p.op("Transpose", [bi_], (k, n)) if tb else bi_
    y = p.op("MatMul", [lhs, rhs], (m, n))
    inputs = {"a": a, "b": b}
    if bias:
        y = p.op("AddRows", [y, p.input("bias", (n,))], (m, n))
        inputs["bias"] = bv
    (g,), (w,) = both(ctx, oracle, p.out(y), inputs, (0,))
    A = np.abs(a.T if ta else a).astype(np.float64)
    B = np.abs(b.T if tb else b).astype(np.float64)
    r = A @ B + (np.abs(bv) if bias else 0)
    ok, worst = within(g, w, r.reshape(-1))
    assert ok, worst


@pytest.mark.parametrize("rows,m,n", [(2048, 1024, 2048), (1024, 4096, 512)])
def test_large_weight_gradient_takes_the_bias_gradient(ctx, oracle, rows, m, n):
    """dW = x^T dy with db = SumRows(dy) on the direct-to-LDS kernel (the column sums of its right
    operand from the fragments the MFMAs read), and the transposed form (dW^T = dy^T x, the sums
    as row sums of its left operand)."""
    x, dy = fast_values(94, rows * m).reshape(rows, m), fast_values(95, rows * n).reshape(rows, n)
    p = Prog()
    xi, di = p.input("x", (rows, m)), p.input("dy", (rows, n))
    dw = p.op("MatMul", [p.op("Transpose", [xi], (m, rows)), di], (m, n))
    db = p.op("SumRows", [di], (n,))
    dwt = p.op("MatMul", [p.op("Transpose", [di], (n, rows)), xi], (n, m))
    (gw, gb, gt), (ww, wb, wt) = both(ctx, oracle, p.out(dw, db, dwt), {"x": x, "dy": dy}, (0, 1, 2))
    r = np.abs(x.T).astype(np.float64) @ np.abs(dy)
    assert within(gw, ww, r.reshape(-1))[0]
    assert within(gb, wb, np.abs(dy).astype(np.float64).sum(0))[0]
    assert within(gt, wt, r.T.reshape(-1))[0]


def test_matmul_with_bias_epilogue_and_sum_rows(ctx, oracle):
    m, k, n = 4096, 128, 128
    x, w, bias = fast_values(3, m * k).reshape(m, k), fast_values(4, k * n, 0.1).reshape(k, n), fast_values(5, n)
    p = Prog()
    xi, wi, bi = p.input("x", (m, k)), p.input("w", (k, n)), p.input("b", (n,))
    y = p.op("AddRows", [p.op("MatMul", [xi, wi], (m, n)), bi], (m, n))
    s = p.op("SumRows", [y], (n,))
    (gy, gs), (wy, ws) = both(ctx, oracle, p.out(y, s), {"x": x, "w": w, "b": bias}, (0, 1))
    r = (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64) + np.abs(bias)).reshape(-1)
    assert within(gy, wy, r)[0]
    assert within(gs, ws, np.abs(wy.reshape(m, n)).sum(axis=0))[0]


@pytest.mark.parametrize("rows,m,n", [(7, 5, 3), (4096, 128, 128), (4096, 512, 128), (4096, 128, 512),
                                      (832, 128, 30522), (300, 33, 70)])
def test_weight_gradient_gemm_takes_the_bias_gradient(ctx, oracle, rows, m, n):
    """dW = x^T dy with db = SumRows(dy) read from the same GEMM's tiles (with and without split-K)."""
    x, dy = fast_values(31, rows * m).reshape(rows, m), fast_values(32, rows * n).reshape(rows, n)
    p = Prog()
    xi, di = p.input("x", (rows, m)), p.input("dy", (rows, n))
    dw = p.op("MatMul", [p.op("Transpose", [xi], (m, rows)), di], (m, n))
    db = p.op("SumRows", [di], (n,))
    (gw, gb), (ww, wb) = both(ctx, oracle, p.out(dw, db), {"x": x, "dy": dy}, (0, 1))
    assert within(gw, ww, (np.abs(x.T).astype(np.float64) @ np.abs(dy)).reshape(-1))[0]
    assert within(gb, wb, np.abs(dy).astype(np.float64).sum(0))[0]


@pytest.mark.parametrize("rows,h", [(16384, 768), (16384, 3072), (2458, 30522), (33, 5)])
def test_column_sums_of_a_tall_matrix(ctx, oracle, rows, h):
    """SumRows on its own (no GEMM to fuse into): partial column sums over row chunks, then the
    chunk sums. 16384 x 768 is a shape where the requested chunk count leaves an empty last chunk."""
    x = fast_values(35, rows * h).reshape(rows, h)
    p = Prog()
    xi = p.input("x", (rows, h))
    (g,), (w,) = both(ctx, oracle, p.out(p.op("SumRows", [xi], (h,))), {"x": x}, (0,))
    assert within(g, w, np.abs(x).astype(np.float64).sum(0))[0]


@pytest.mark.parametrize("r,k,v,h", [(832, 64, 1001, 32), (300, 128, 30522, 64)])
def test_column_sums_of_a_row_padded_gemm_output(ctx, oracle, r, k, v, h):
    """A GEMM output whose width is not a multiple of 4, read by GEMMs and by a column sum of its
    own: its rows are padded in HBM, and the column-sum launch reads them at that pitch."""
    x, w, w2 = fast_values(61, r * k).reshape(r, k), fast_values(62, k * v).reshape(k, v), fast_values(63, v * h).reshape(v, h)
    p = Prog()
    xi, wi, w2i = p.input("x", (r, k)), p.input("w", (k, v)), p.input("w2", (v, h))
    y = p.op("MatMul", [xi, wi], (r, v))
    cs = p.op("SumRows", [y], (v,))
    z = p.op("MatMul", [y, w2i], (r, h))
    (gs, gz), (ws, wz) = both(ctx, oracle, p.out(cs, z), {"x": x, "w": w, "w2": w2}, (0, 1))
    ay = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64)
    assert within(gs, ws, ay.sum(0))[0]
    assert within(gz, wz, (ay @ np.abs(w2)).reshape(-1))[0]


@pytest.mark.parametrize("v,h,r,n", [(1000, 64, 96, 256), (30522, 128, 832, 4096)])
def test_tied_decoder_gradients(ctx, oracle, v, h, r, n):
    """The tied-embedding decoder's graph: logits = h E^T, dX = dl E, the decoder weight gradient
    computed transposed (with the bias sums as row sums of its left operand) and added to the
    embedding gradient by the scatter."""
    E, x = fast_values(51, v * h).reshape(v, h), fast_values(52, r * h).reshape(r, h)
    dl, G = fast_values(53, r * v).reshape(r, v), fast_values(54, n * h).reshape(n, h)
    ids = embedding_ids("zipf", v, n, np.random.default_rng(5))
    p = Prog()
    Ei, xi, di, ii, Gi = p.input("E", (v, h)), p.input("x", (r, h)), p.input("dl", (r, v)), p.input("ids", (n,), "i32"), p.input("G", (n, h))
    t1 = p.op("Transpose", [Ei], (h, v))
    logits = p.op("MatMul", [xi, t1], (r, v))
    dx = p.op("MatMul", [di, p.op("Transpose", [t1], (v, h))], (r, h))
    dw = p.op("MatMul", [p.op("Transpose", [xi], (h, r)), di], (h, v))
    db = p.op("SumRows", [di], (v,))
    eg = p.op("EmbeddingGrad", [ii, Gi], (v, h), f"[{v}]")
    total = p.op("Add", [p.op("Transpose", [dw], (v, h)), eg], (v, h))
    got, want = both(ctx, oracle, p.out(logits, dx, db, total), {"E": E, "x": x, "dl": dl, "ids": ids, "G": G}, (0, 1, 2, 3))
    ax, aE, adl = (np.abs(a).astype(np.float64) for a in (x, E, dl))
    assert within(got[0], want[0], (ax @ aE.T).reshape(-1))[0]
    assert within(got[1], want[1], (adl @ aE).reshape(-1))[0]
    assert within(got[2], want[2], adl.sum(0))[0]
    seg = np.zeros((v, h))
    np.add.at(seg, ids, np.abs(G).astype(np.float64))
    assert within(got[3], want[3], ((ax.T @ adl).T + seg).reshape(-1))[0]


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("v,h,r,n,g_const", [(1000, 64, 96, 256, True), (1001, 64, 96, 256, False),
                                             (30522, 128, 832, 4096, True)])
def test_decoder_cross_entropy_head(ctx, oracle, request, v, h, r, n, g_const, fused):
    """The masked-LM head as the step has it: logits = x E^T + b, the cross-entropy loss and
    gradient, dX, the transposed dW with the bias sums as row sums, added to the embedding
    gradient; the upstream gradient a constant or computed. Vocabularies that are not a multiple of
    4 keep the logits and their gradient in rows padded to 64 floats. `fused`: the cross-entropy
    folded into the head GEMMs (msx_set_fusion)."""
    ctx.set_fusion(ce_head=fused)
    request.addfinalizer(lambda: ctx.set_fusion(ce_head=False))
    E, x, b = fast_values(61, v * h).reshape(v, h), fast_values(62, r * h).reshape(r, h), fast_values(63, v, 0.5)
    G = fast_values(64, n * h).reshape(n, h)
    rng = np.random.default_rng(7)
    labels = rng.integers(0, v, r).astype(np.int32)
    w = (rng.random(r) < 0.8).astype(np.float32)
    ids = embedding_ids("zipf", v, n, rng)
    p = Prog()
    Ei, xi, bi = p.input("E", (v, h)), p.input("x", (r, h)), p.input("b", (v,))
    li, wi, ii, Gi = p.input("labels", (r,), "i32"), p.input("w", (r,)), p.input("ids", (n,), "i32"), p.input("G", (n, h))
    t1 = p.op("Transpose", [Ei], (h, v))
    logits = p.op("AddRows", [p.op("MatMul", [xi, t1], (r, v)), bi], (r, v))
    loss = p.op("CrossEntropy", [logits, li, wi], ())
    gs = p.scalar(1.0) if g_const else p.op("Mul", [p.scalar(0.5), p.scalar(2.0)], ())
    dl = p.op("CrossEntropyGrad", [logits, li, wi, gs], (r, v))
    db = p.op("SumRows", [dl], (v,))
    dx = p.op("MatMul", [dl, p.op("Transpose", [t1], (v, h))], (r, h))
    dw = p.op("MatMul", [p.op("Transpose", [xi], (h, r)), dl], (h, v))
    total = p.op("Add", [p.op("Transpose", [dw], (v, h)), p.op("EmbeddingGrad", [ii, Gi], (v, h), f"[{v}]")], (v, h))
    inputs = {"E": E, "x": x, "b": b, "labels": labels, "w": w, "ids": ids, "G": G}
    got, want = both(ctx, oracle, p.out(loss, dx, db, total), inputs, (0, 1, 2, 3))
    lg = x.astype(np.float64) @ E.T.astype(np.float64) + b
    pr = np.exp(lg - lg.max(1, keepdims=True))
    pr /= pr.sum(1, keepdims=True)
    adl = (pr + (np.arange(v)[None, :] == labels[:, None])) * w[:, None] / w.sum()
    aE, ax = np.abs(E).astype(np.float64), np.abs(x).astype(np.float64)
    assert within(got[0], want[0], np.abs(want[0]) + 10)[0]
    assert within(got[1], want[1], (adl @ aE).reshape(-1) + 1e-3)[0]
    assert within(got[2], want[2], adl.sum(0) + 1e-3)[0]
    seg = np.zeros((v, h))
    np.add.at(seg, ids, np.abs(G).astype(np.float64))
    assert within(got[3], want[3], ((ax.T @ adl).T + seg).reshape(-1) + 1e-3)[0]


@pytest.mark.parametrize("act,m,k,n", [("Gelu", 4096, 128, 512), ("Relu", 64, 784, 256), ("Gelu", 33, 70, 129)])
def test_gemm_epilogues(ctx, oracle, act, m, k, n):
    """Activation, activation gradient and residual add written by the GEMM that produces their
    input: y = x W + b, a = act(y) (y kept for the gradient), act'(y) (r W), q + dy W^T."""
    x, W, b = fast_values(71, m * k).reshape(m, k), fast_values(72, k * n, 0.1).reshape(k, n), fast_values(73, n)
    dy, r, q = fast_values(74, m * n).reshape(m, n), fast_values(75, m * k).reshape(m, k), fast_values(76, m * k).reshape(m, k)
    p = Prog()
    xi, wi, bi = p.input("x", (m, k)), p.input("W", (k, n)), p.input("b", (n,))
    di, ri, qi = p.input("dy", (m, n)), p.input("r", (m, k)), p.input("q", (m, k))
    y = p.op("AddRows", [p.op("MatMul", [xi, wi], (m, n)), bi], (m, n))
    a = p.op(act, [y], (m, n))
    g = p.op(act + "Grad", [y, p.op("MatMul", [ri, wi], (m, n))], (m, n))
    z = p.op("Add", [qi, p.op("MatMul", [di, p.op("Transpose", [wi], (n, k))], (m, k))], (m, k))
    got, want = both(ctx, oracle, p.out(a, g, z), {"x": x, "W": W, "b": b, "dy": dy, "r": r, "q": q}, (0, 1, 2))
    aW = np.abs(W).astype(np.float64)
    ry = np.abs(x) @ aW + np.abs(b)
    assert within(got[0], want[0], (ry * 1.2 + 1e-3).reshape(-1))[0]
    assert within(got[1], want[1], ((np.abs(r) @ aW) * 1.2 * (1 + ry) + 1e-3).reshape(-1))[0]
    assert within(got[2], want[2], (np.abs(q) + np.abs(dy) @ aW.T).reshape(-1))[0]


@pytest.mark.parametrize("m,k,n", [(4096, 128, 128), (37, 64, 40)])
def test_gemm_chain_with_dropout_gradient(ctx, oracle, m, k, n):
    """q + d1 W1^T + d2 W2^T + d3 W3^T (a chain of like GEMMs added into one value, run as one
    GEMM over three K segments) followed by the DropoutGrad that is its only reader (applied in
    the GEMM's epilogue): values within the per-kernel tolerance of the oracle, zeros exactly where
    the mask drops."""
    q = fast_values(91, m * n).reshape(m, n)
    ds = [fast_values(92 + i, m * k).reshape(m, k) for i in range(3)]
    Ws = [fast_values(95 + i, n * k, 0.1).reshape(n, k) for i in range(3)]
    token = np.array([0x13579, -0x2468], np.int32)
    p = Prog()
    qi, ti = p.input("q", (m, n)), p.input("tok", (2,), "i32")
    acc = qi
    for i in range(3):
        di, wi = p.input(f"d{i}", (m, k)), p.input(f"W{i}", (n, k))
        acc = p.op("Add", [acc, p.op("MatMul", [di, p.op("Transpose", [wi], (k, n))], (m, n))], (m, n))
    z = p.op("DropoutGrad", [ti, acc], (m, n), "[p = 0.1, site = tok]")
    inputs = {"q": q, "tok": token, **{f"d{i}": ds[i] for i in range(3)}, **{f"W{i}": Ws[i] for i in range(3)}}
    (g,), (w,) = both(ctx, oracle, p.out(z), inputs, (0,), seed=7)
    r = np.abs(q).astype(np.float64) + sum(np.abs(d).astype(np.float64) @ np.abs(W).T.astype(np.float64) for d, W in zip(ds, Ws))
    assert np.array_equal(g == 0, w == 0)
    assert within(g, w, (r / 0.9).reshape(-1))[0]


def test_embedding_gradient_with_its_dropout_gradient(ctx, oracle):
    """EmbeddingGrad over step-input ids (the sorted-segment path) and a DropoutGrad of it written by
    the same apply pass: both bit for bit."""
    n, rows, h = 832, 4096, 128
    ids = np.random.default_rng(5).integers(0, rows, n).astype(np.int32)
    ids[700:] = 0  # padding slots all naming row 0: one long segment
    G = fast_values(98, n * h).reshape(n, h)
    token = np.array([0x2222, 0x7777], np.int32)
    p = Prog()
    ii, gi, ti = p.input("ids", (n,), "i32"), p.input("G", (n, h)), p.input("tok", (2,), "i32")
    e = p.op("EmbeddingGrad", [ii, gi], (rows, h), "[%d]" % rows)
    d = p.op("DropoutGrad", [ti, e], (rows, h), "[p = 0.1, site = tok]")
    got, want = both(ctx, oracle, p.out(e, d), {"ids": ids, "G": G, "tok": token}, (0, 1), seed=3)
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))


@pytest.mark.parametrize("rows,h", [(6, 8), (4096, 128), (832, 128), (33, 200), (100, 768)])
def test_layer_norm_family(ctx, oracle, rows, h):
    x = fast_values(6, rows * h).reshape(rows, h)
    gamma, beta = fast_values(7, h, 0.5), fast_values(8, h, 0.5)
    G = fast_values(9, rows * h).reshape(rows, h)
    p = Prog()
    xi, gi, bi, Gi = p.input("x", (rows, h)), p.input("g", (h,)), p.input("b", (h,)), p.input("G", (rows, h))
    y = p.op("LayerNorm", [xi, gi, bi], (rows, h))
    dx = p.op("LayerNormGradX", [xi, gi, Gi], (rows, h))
    dg = p.op("LayerNormGradGamma", [xi, Gi], (h,))
    db = p.op("SumRows", [Gi], (h,))
    got, want = both(ctx, oracle, p.out(y, dx, dg, db), {"x": x, "g": gamma, "b": beta, "G": G}, (0, 1, 2, 3))
    # r: the magnitude of each term: |xhat| |gamma| + |beta| for y; sums of |terms| for the grads.
    xhat = np.abs((x - x.mean(1, keepdims=True)) / x.std(1, keepdims=True))
    assert within(got[0], want[0], (xhat * np.abs(gamma) + np.abs(beta) + 1).reshape(-1))[0]
    rx = (np.abs(G) * np.abs(gamma)).sum(1, keepdims=True) / h * (1 + xhat) / x.std(1, keepdims=True)
    assert within(got[1], want[1], (np.abs(want[1].reshape(rows, h)) + rx).reshape(-1))[0]
    assert within(got[2], want[2], (np.abs(G) * xhat).sum(0))[0]
    assert within(got[3], want[3], np.abs(G).astype(np.float64).sum(0))[0]


def test_layer_norm_gamma_gradient_alone(ctx, oracle):
    rows, h = 512, 128
    x, G = fast_values(41, rows * h).reshape(rows, h), fast_values(42, rows * h).reshape(rows, h)
    p = Prog()
    xi, Gi = p.input("x", (rows, h)), p.input("G", (rows, h))
    (g,), (w,) = both(ctx, oracle, p.out(p.op("LayerNormGradGamma", [xi, Gi], (h,))), {"x": x, "G": G}, (0,))
    xhat = np.abs((x - x.mean(1, keepdims=True)) / x.std(1, keepdims=True))
    assert within(g, w, (np.abs(G) * xhat).sum(0))[0]


def test_gelu_relu_elementwise(ctx, oracle):
    n = 4096 * 512
    x, G = fast_values(10, n), fast_values(11, n)
    p = Prog()
    xi, Gi = p.input("x", (n,)), p.input("G", (n,))
    outs = [p.op("Gelu", [xi], (n,)), p.op("GeluGrad", [xi, Gi], (n,)), p.op("Relu", [xi], (n,)),
            p.op("ReluGrad", [xi, Gi], (n,)), p.op("Add", [xi, Gi], (n,)), p.op("Mul", [xi, Gi], (n,)),
            p.op("Sub", [xi, Gi], (n,))]
    got, want = both(ctx, oracle, p.out(*outs), {"x": x, "G": G}, tuple(range(len(outs))))
    for k, (g, w) in enumerate(zip(got, want)):
        if k >= 2:  # relu, add, mul, sub: one correctly rounded operation, bit for bit
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), k
        else:
            assert within(g, w, np.abs(w) + np.abs(x) * 1e-2)[0], k


@pytest.mark.parametrize("B,S,H,heads,masked", [
    (2, 16, 32, 2, False), (2, 16, 32, 2, True), (32, 128, 128, 2, False), (4, 128, 128, 2, True),
    (2, 24, 32, 2, True),  # S not a multiple of 16: the scalar path
    (2, 64, 256, 2, False),  # head width 128
    (2, 512, 128, 2, True),  # keys and queries streamed through LDS in two chunks
    (1, 320, 256, 2, False),  # head width 128 in three chunks, the last one shorter
    # 4096 or more 16-row tiles: blocks of four waves streaming 32-row tiles, the last one of 16 rows
    (16, 272, 256, 16, True),  # head width 16
    (32, 176, 768, 12, True),  # head width 64 (the BERT-base heads)
])
def test_attention_and_gradients(ctx, oracle, B, S, H, heads, masked):
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
    got, want = both(ctx, oracle, p.out(*outs), {"q": q, "k": k, "v": v, "mask": mask, "G": G}, (0, 1, 2, 3))
    d = H // heads
    # r: sum over keys of |p| |v|-like terms, bounded by the largest row magnitudes.
    scale = np.abs(v).max() + np.abs(G).max() * (np.abs(q).max() + np.abs(k).max()) * np.sqrt(d) * 2
    for idx, (g, w) in enumerate(zip(got, want)):
        ok, worst = within(g, w, np.abs(w) + scale)
        assert ok, (idx, worst)
    if masked:
        dead = np.flatnonzero(mask.reshape(-1) == 0)
        for g in (got[2], got[3]):
            assert np.all(g.reshape(B * S, H)[dead] == 0)


def test_cross_entropy_and_gradient_full_head(ctx, oracle):
    rows, V = 832, 30522
    x = fast_values(16, rows * V).reshape(rows, V)
    rng = np.random.default_rng(2)
    labels = rng.integers(0, V, rows).astype(np.int32)
    w = (rng.random(rows) < 0.75).astype(np.float32)
    p = Prog()
    xi, li, wi = p.input("x", (rows, V)), p.input("labels", (rows,), "i32"), p.input("w", (rows,))
    loss = p.op("CrossEntropy", [xi, li, wi], ())
    g = p.op("CrossEntropyGrad", [xi, li, wi, p.scalar(1.0)], (rows, V))
    (gl, gg), (wl, wg) = both(ctx, oracle, p.out(loss, g), {"x": x, "labels": labels, "w": w}, (0, 1))
    assert within(gl, wl, np.abs(wl) + 10)[0]
    assert within(gg, wg, np.abs(wg) + 1.0 / w.sum())[0]


def embedding_ids(kind, rows, n, rng):
    if kind == "zipf":  # hot rows, as token ids
        ranks = np.arange(1, rows - 4)
        prob = ranks ** -1.1
        return (5 + rng.choice(len(ranks), n, p=prob / prob.sum())).astype(np.int32)
    if kind == "positions":  # every row n / rows times, as position ids
        return np.tile(np.arange(rows, dtype=np.int32), n // rows + 1)[:n]
    if kind == "same":  # one segment holding every position
        return np.full(n, rows // 2, np.int32)
    return rng.integers(0, rows, n).astype(np.int32)


@pytest.mark.parametrize("kind,rows,h,n", [
    ("zipf", 30522, 128, 4096), ("positions", 128, 128, 4096), ("same", 50, 64, 3000), ("uniform", 7, 130, 1),
    ("uniform", 1000, 96, 1500), ("zipf", 40000, 128, 2048), ("uniform", 32768, 8, 16384),
    ("zipf", 30522, 768, 2048), ("same", 5, 128, 8192), ("uniform", 3, 33, 600), ("positions", 512, 256, 8000),
    ("zipf", 4096, 128, 832), ("zipf", 30522, 768, 16384), ("same", 5, 64, 16384), ("positions", 512, 64, 12288),
])
def test_embedding_gather_and_sorted_segment_scatter_are_bit_exact(ctx, oracle, kind, rows, h, n):
    rng = np.random.default_rng(3)
    ids = embedding_ids(kind, rows, n, rng)
    table = fast_values(17, rows * h).reshape(rows, h)
    G = fast_values(18, n * h).reshape(n, h)
    p = Prog()
    ti, ii, Gi = p.input("t", (rows, h)), p.input("ids", (n,), "i32"), p.input("G", (n, h))
    e = p.op("Embedding", [ti, ii], (n, h))
    dg = p.op("EmbeddingGrad", [ii, Gi], (rows, h), f"[{rows}]")
    got, want = both(ctx, oracle, p.out(e, dg), {"t": table, "ids": ids, "G": G}, (0, 1))
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))


@pytest.mark.parametrize("pad_kind", ["signed_zeros", "one_nonzero", "cancelling", "zero_column_groups"])
def test_scatter_of_padding_slots_is_bit_exact(ctx, oracle, pad_kind):
    """The masked-row scatter's shape: 832 gathered rows back into 4096 positions, the last 218
    slots padding that all name row 0 (one long segment). Rows of +0/-0 in the padding are left
    out of the device's add chain; the sum must still equal the oracle's sequential one bit for
    bit: all signed zeros (+0), one nonzero padding row, x then -x then -0 rows (the exact zero of
    a cancellation is +0), and rows that are zero in some 32-column groups only."""
    rows, h, n, pad = 4096, 128, 832, 218
    rng = np.random.default_rng(9)
    ids = np.concatenate([np.sort(rng.choice(np.arange(1, rows), n - pad, replace=False)),
                          np.zeros(pad, np.int64)]).astype(np.int32)
    G = fast_values(18, n * h).reshape(n, h).copy()
    zeros = np.where(rng.random((pad, h)) < 0.5, np.float32(-0.0), np.float32(0.0)).astype(np.float32)
    G[n - pad:] = zeros
    if pad_kind == "one_nonzero":
        G[n - pad + 101, 37:70] = fast_values(5, 33)
    elif pad_kind == "cancelling":
        G[n - pad + 3] = fast_values(6, h)
        G[n - pad + 150] = -G[n - pad + 3]
    elif pad_kind == "zero_column_groups":
        for r in range(0, pad, 3):
            g = rng.integers(0, 4)
            G[n - pad + r, 32 * g:32 * g + 32] = fast_values(100 + r, 32)
    p = Prog()
    ii, Gi = p.input("ids", (n,), "i32"), p.input("G", (n, h))
    dg = p.op("EmbeddingGrad", [ii, Gi], (rows, h), f"[{rows}]")
    got, want = both(ctx, oracle, p.out(dg), {"ids": ids, "G": G}, (0,))
    assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32))
    if pad_kind == "signed_zeros":
        assert np.all(got[0][0].view(np.uint32) == 0)  # +0, never -0


def test_dropout_masks_are_bit_exact_at_full_size(ctx, oracle):
    n = 4096 * 128
    x = fast_values(19, n)
    token = np.array([-0x1357, 0x2468ACE], np.int32)
    p = Prog()
    xi, ti = p.input("x", (n,)), p.input("tok", (2,), "i32")
    y = p.op("Dropout", [xi, ti], (n,), "[p = 0.1, site = tok]")
    dy = p.op("DropoutGrad", [ti, xi], (n,), "[p = 0.1, site = tok]")
    got, want = both(ctx, oracle, p.out(y, dy), {"x": x, "tok": token}, (0, 1), seed=42)
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
    kept = np.mean(got[0] != 0) / np.mean(x != 0)  # x holds planted zeros
    assert 0.88 < kept < 0.92


@pytest.mark.parametrize("rows,h", [(4096, 128), (37, 200), (1000, 768), (64, 256), (33, 1024)])
def test_fused_layer_norm_neighbours(ctx, oracle, rows, h):
    """LayerNorm(e1 + e2) followed by a Dropout, and LayerNorm(a + Dropout(b)) with the residual sum
    kept for the backward, as the fused pass runs them: values within the per-kernel tolerance of
    the oracle, dropout masks bit for bit."""
    e1, e2 = fast_values(81, rows * h).reshape(rows, h), fast_values(82, rows * h).reshape(rows, h)
    a, b = fast_values(83, rows * h).reshape(rows, h), fast_values(84, rows * h).reshape(rows, h)
    gamma, beta, G = fast_values(85, h, 0.5), fast_values(86, h, 0.5), fast_values(87, rows * h).reshape(rows, h)
    t1, t2 = np.array([11, -3], np.int32), np.array([0x7123, 99], np.int32)
    p = Prog()
    ei, fi, ai, bi = (p.input(nm, (rows, h)) for nm in ("e1", "e2", "a", "b"))
    gi, be, Gi = p.input("gamma", (h,)), p.input("beta", (h,)), p.input("G", (rows, h))
    ti1, ti2 = p.input("t1", (2,), "i32"), p.input("t2", (2,), "i32")
    x1 = p.op("Add", [ei, fi], (rows, h))
    y1 = p.op("Dropout", [p.op("LayerNorm", [x1, gi, be], (rows, h)), ti1], (rows, h), "[p = 0.1, site = t1]")
    d2 = p.op("Dropout", [bi, ti2], (rows, h), "[p = 0.1, site = t2]")
    s2 = p.op("Add", [ai, d2], (rows, h))
    y2 = p.op("LayerNorm", [s2, gi, be], (rows, h))
    dx2 = p.op("LayerNormGradX", [s2, gi, Gi], (rows, h))
    # LayerNorm backward passes that also write the dropout / GELU gradient of their dx.
    Gb = p.input("Gb", (rows, h))
    da = p.op("DropoutGrad", [ti1, p.op("LayerNormGradX", [x1, gi, Gi], (rows, h))], (rows, h), "[p = 0.1, site = t1]")
    dxb = p.op("LayerNormGradX", [s2, gi, Gb], (rows, h))
    gb = p.op("GeluGrad", [ai, dxb], (rows, h))
    # LayerNorm of a gather of a residual sum (the masked rows of the last layer): only those rows.
    nr = max(1, rows // 5)
    ids = np.random.default_rng(9).permutation(rows)[:nr].astype(np.int32)
    ii, ti3, G3 = p.input("ids", (nr,), "i32"), p.input("t3", (2,), "i32"), p.input("G3", (nr, h))
    e3 = p.op("Embedding", [p.op("Add", [ai, p.op("Dropout", [bi, ti3], (rows, h), "[p = 0.1, site = t3]")], (rows, h)), ii],
              (nr, h))
    y3 = p.op("LayerNorm", [e3, gi, be], (nr, h))
    dx3 = p.op("LayerNormGradX", [e3, gi, G3], (nr, h))
    inputs = {"e1": e1, "e2": e2, "a": a, "b": b, "gamma": gamma, "beta": beta, "G": G, "t1": t1, "t2": t2,
              "Gb": fast_values(88, rows * h).reshape(rows, h), "ids": ids, "t3": np.array([5, 6], np.int32),
              "G3": fast_values(89, nr * h).reshape(nr, h)}
    got, want = both(ctx, oracle, p.out(y1, y2, dx2, s2, da, dxb, gb, y3, dx3), inputs, tuple(range(9)), seed=5)
    assert within(got[7], want[7], np.ones(nr * h) * (4 * np.abs(gamma).max() + np.abs(beta).max() + 1))[0]
    assert within(got[8], want[8], np.abs(want[8]) * 0.01 + 0.05 * np.abs(want[8]).max())[0]
    for gg, ww in zip(got[4:], want[4:]):
        assert np.array_equal(gg == 0, ww == 0) or gg is got[5]
        assert within(gg, ww, np.abs(ww) * 0.01 + 0.05 * np.abs(ww).max())[0]
    r_ln = (4 * np.abs(gamma) + np.abs(beta) + 1)[None, :] * np.ones((rows, 1))
    assert np.array_equal(got[0] == 0, want[0] == 0)
    assert within(got[0], want[0], (r_ln / 0.9).reshape(-1))[0]
    assert within(got[1], want[1], r_ln.reshape(-1))[0]
    assert np.array_equal(got[3].view(np.uint32), want[3].view(np.uint32))  # a + dropout(b): exact
    rx = (np.abs(G) * np.abs(gamma)).sum(1, keepdims=True) / h * 8 / np.abs(want[3].reshape(rows, h)).std(1, keepdims=True)
    assert within(got[2], want[2], (np.abs(want[2].reshape(rows, h)) + rx).reshape(-1))[0]


def test_whole_tensor_sums(ctx, oracle):
    n = 1 << 16
    a, b = fast_values(20, n), fast_values(21, n)
    p = Prog()
    ai, bi = p.input("a", (256, 256)), p.input("b", (256, 256))
    outs = [p.op("ReduceSum", [ai], ()), p.op("ReduceMean", [ai], ()), p.op("Mse", [ai, bi], ())]
    got, want = both(ctx, oracle, p.out(*outs), {"a": a, "b": b}, (0, 1, 2))
    r = [np.abs(a).sum(), np.abs(a).mean(), ((a - b) ** 2).mean()]
    for g, w, rr in zip(got, want, r):
        assert within(g, w, rr, atol=1e-6, rtol=1e-6)[0]


def test_transpose_and_broadcast(ctx, oracle):
    x = fast_values(22, 130 * 70).reshape(130, 70)
    p = Prog()
    xi = p.input("x", (130, 70))
    t = p.op("Transpose", [xi], (70, 130))
    s = p.op("ReduceSum", [xi], ())
    bcast = p.op("BroadcastScalar", [s], (3, 5), "[3, 5]")
    got, want = both(ctx, oracle, p.out(t, bcast), {"x": x}, (0, 1))
    assert np.array_equal(got[0], want[0])
    assert within(got[1], want[1], np.abs(x).sum())[0]
