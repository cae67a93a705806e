"""The reference's hand-computed CPU goldens, f32 column (crates/modelspec-runtime/tests/
cpu_golden.rs:145-416), run on the oracle and compared bit for bit. Every expected value is exact
in f32, and each case is built so that a wrong accumulation order, a fused first product, a
running f32 sum where the reference sums in f64, or a dropped sign of zero gives other bits."""
import numpy as np
import pytest

from ops_lib import Prog

BIG = 9007199254740992.0  # 2^53
A4 = [1.0, 2.0, 3.0, 4.0]
B4 = [10.0, 20.0, 30.0, 40.0]


def f32(values):
    out = np.array(values, np.float64).astype(np.float32)
    assert np.array_equal(out.astype(np.float64), np.array(values, np.float64)), "not exact in f32"
    return out


def unary(oracle, shape, data, build, out_shape):
    p = Prog()
    x = p.input("x", shape)
    p.out(build(p, x, out_shape))
    return oracle.run_program(p.text(), {"x": f32(data)})[0]


def binary(oracle, a_shape, a, b_shape, b, name, out_shape):
    p = Prog()
    x, y = p.input("a", a_shape), p.input("b", b_shape)
    p.out(p.op(name, [x, y], out_shape))
    return oracle.run_program(p.text(), {"a": f32(a), "b": f32(b)})[0]


def same_bits(got, want):
    want = f32(want)
    assert got.shape == want.shape and got.view(np.uint32).tolist() == want.view(np.uint32).tolist(), (got, want)


@pytest.mark.parametrize("name,a_shape,a,b_shape,b,want", [
    ("Add", (2, 2), A4, (2, 2), B4, [11.0, 22.0, 33.0, 44.0]),            # cpu_golden.rs:181-186
    ("Add", (2, 2), A4, (), [0.5], [1.5, 2.5, 3.5, 4.5]),                 # :188-193
    ("Add", (), [0.5], (2, 2), A4, [1.5, 2.5, 3.5, 4.5]),                 # :195-200
    ("Add", (), [0.5], (), [-2.0], [-1.5]),                               # :202-207
    ("Sub", (2, 2), A4, (2, 2), B4, [-9.0, -18.0, -27.0, -36.0]),         # :209-214
    ("Sub", (2, 2), A4, (), [0.5], [0.5, 1.5, 2.5, 3.5]),                 # :216-221
    ("Sub", (), [0.5], (2, 2), A4, [-0.5, -1.5, -2.5, -3.5]),             # :223-228
    ("Mul", (2, 2), A4, (2, 2), B4, [10.0, 40.0, 90.0, 160.0]),           # :230-235
    ("Mul", (2, 2), A4, (), [0.5], [0.5, 1.0, 1.5, 2.0]),                 # :237-242
    ("Mul", (), [-3.0], (2, 2), A4, [-3.0, -6.0, -9.0, -12.0]),           # :244-249
    ("Add", (1,), [16777216.0], (1,), [1.0], [16777216.0]),               # :251-256, f32 rounding
    ("ReluGrad", (2, 3), [-1.0, 0.0, 2.0, -0.0, 3.0, -4.0], (2, 3), [5.0, 6.0, 7.0, 8.0, 9.0, 10.0],
     [0.0, 0.0, 7.0, 0.0, 9.0, 0.0]),                                     # :265-272
])
def test_elementwise(oracle, name, a_shape, a, b_shape, b, want):
    out_shape = a_shape if len(a_shape) >= len(b_shape) else b_shape
    same_bits(binary(oracle, a_shape, a, b_shape, b, name, out_shape), want)


def test_relu_broadcast_and_transpose(oracle):
    same_bits(unary(oracle, (2, 3), [-2.0, -0.0, 0.0, 0.5, 3.0, -7.0], lambda p, x, s: p.op("Relu", [x], s), (2, 3)),
              [0.0, 0.0, 0.0, 0.5, 3.0, 0.0])                             # :258-263
    same_bits(unary(oracle, (), [1.5], lambda p, x, s: p.op("BroadcastScalar", [x], s, "[2, 3]"), (2, 3)),
              [1.5] * 6)                                                  # :274-280
    same_bits(unary(oracle, (2, 3), [1, 2, 3, 4, 5, 6], lambda p, x, s: p.op("Transpose", [x], s), (3, 2)),
              [1.0, 4.0, 2.0, 5.0, 3.0, 6.0])                             # :282-289


def test_matmul_cases(oracle):
    # :291-309 a plain 2x3 by 3x4 product.
    same_bits(binary(oracle, (2, 3), [1, 2, 3, 4, 5, 6], (3, 4), list(range(1, 13)), "MatMul", (2, 4)),
              [38.0, 44.0, 50.0, 56.0, 83.0, 98.0, 113.0, 128.0])
    # :311-320 ascending accumulation over k: products [2^53, 1, -2^53, 1] give 1, the other row 0.
    same_bits(binary(oracle, (2, 4), [BIG, 1.0, -BIG, 1.0, 1.0, BIG, 1.0, -BIG], (4, 1), [1.0] * 4, "MatMul",
                     (2, 1)), [1.0, 0.0])
    # :322-330 the accumulator starts at the first product: -0 + -0 stays -0.
    same_bits(binary(oracle, (1, 2), [-1.0, -1.0], (2, 1), [0.0, 0.0], "MatMul", (1, 1)), [-0.0])
    # :332-344 each later product is fused into its sum: 2^-24, where a rounded product gives 0.
    e = 1.0 + 2.0 ** -12
    same_bits(binary(oracle, (1, 2), [-(1.0 + 2.0 ** -11), e], (2, 1), [1.0, e], "MatMul", (1, 1)), [2.0 ** -24])


def test_reductions(oracle):
    red = lambda name: (lambda p, x, s: p.op(name, [x], s))
    same_bits(unary(oracle, (2, 3), [1, 2, 3, 4, 5, 6], red("ReduceSum"), ()), [21.0])          # :346-353
    same_bits(unary(oracle, (2, 2), [BIG, 1.0, -BIG, 1.0], red("ReduceSum"), ()), [1.0])        # :355-360
    same_bits(unary(oracle, (2,), [-0.0, -0.0], red("ReduceSum"), ()), [-0.0])                  # :362-365
    same_bits(unary(oracle, (3,), [1, 2, 3], red("ReduceMean"), ()), [2.0])                     # :367-374
    same_bits(unary(oracle, (2, 3), [1, 2, 3, 4, 5, 3], red("ReduceMean"), ()), [3.0])
    same_bits(unary(oracle, (2, 2), [BIG, 1.0, -BIG, 1.0], red("ReduceMean"), ()), [0.25])      # :376-382


def test_mse(oracle):
    same_bits(binary(oracle, (2, 3), [3, 5, 4, 0, 1, 7], (2, 3), [2, 3, 2, 1, 3, 5], "Mse", ()), [3.0])  # :384-398
    # :400-416 squared differences summed in row-major order in f64, rounded once.
    same_bits(binary(oracle, (2, 2), [1.5, 134217728.0, 1.5, 1.5], (2, 2), [0.25, 0.0, 0.25, 0.25], "Mse", ()),
              [4503599627370496.0])
    same_bits(binary(oracle, (2, 2), [1.0, 4096.0, 1.0, 1.0], (2, 2), [0.125, 0.0, 0.125, 0.125], "Mse", ()),
              [4194304.5])
