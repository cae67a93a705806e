"""Per-op test programs (ir/print.rs text), inputs and float64 references shared by the oracle
tests (CPU) and the HIP parity tests (GPU).

Inputs follow crates/modelspec-runtime/tests/common/mod.rs:123-160: SplitMix64 draws in
[-4, 4) with +0 and -0 planted every 7th element. Tolerances follow common/mod.rs:17-40:
|g - c| <= 1e-5 + 1e-4 * r per kernel, r = |c| for elementwise results and the sum of the
absolute terms for sums and contractions.
"""
import numpy as np

ATOL, RTOL = 1e-5, 1e-4


class Draw:
    """SplitMix64 values in [-4, 4), +0 / -0 planted every 7th element (common/mod.rs:123-160)."""

    def __init__(self, seed):
        self.state = seed & 0xFFFFFFFFFFFFFFFF
        self.calls = 0

    def _next(self):
        M = 0xFFFFFFFFFFFFFFFF
        self.state = (self.state + 0x9E3779B97F4A7C15) & M
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)

    def values(self, count, scale=1.0):
        zero_at = (3 + self.calls) % 7
        self.calls += 1
        out = np.empty(count, np.float32)
        for i in range(count):
            if i % 7 == zero_at:
                out[i] = 0.0 if i % 14 == zero_at else -0.0
            else:
                out[i] = np.float32((self._next() >> 40) / float(1 << 24) * 8.0 - 4.0)
        return (out * np.float32(scale)).astype(np.float32)


def fast_values(seed, count, scale=1.0):
    """The same distribution for large tensors, drawn with numpy (zeros planted every 7th)."""
    rng = np.random.default_rng(seed)
    v = (rng.random(count, dtype=np.float64) * 8.0 - 4.0).astype(np.float32) * np.float32(scale)
    v[3::7] = 0.0
    v[10::14] = -0.0
    return v.astype(np.float32)


def within(g, c, r, atol=ATOL, rtol=RTOL):
    """Elementwise |g - c| <= atol + rtol * r; returns (ok, worst excess ratio)."""
    g = np.asarray(g, np.float64)
    c = np.asarray(c, np.float64)
    bound = atol + rtol * np.asarray(r, np.float64)
    err = np.abs(g - c)
    return bool(np.all(err <= bound)), float(np.max(err / bound)) if err.size else 0.0


class Prog:
    """A Tensor IR program in the printed form the C ABI parses."""

    def __init__(self, model="T"):
        self.model = model
        self.params = []
        self.lines = []
        self.outs = []
        self.n = 0

    def param(self, name, shape, init="xavier_uniform"):
        self.params.append(f"param @{self.model}.{name}: {ty(shape)} = {init}")
        return len(self.params) - 1

    def _node(self, shape, body, dtype="f32"):
        i = self.n
        self.n += 1
        self.lines.append(f"%{i}: {ty(shape, dtype)} = {body}")
        return i

    def input(self, name, shape, dtype="f32"):
        return self._node(shape, f'Input "{name}"', dtype)

    def read(self, param, shape):
        path = self.params[param].split(":")[0][len("param @"):]
        return self._node(shape, f"ParamRead @{path}")

    def scalar(self, v):
        return self._node((), f"Scalar {float(np.float32(v))!r}")

    def op(self, name, operands, shape, attr=None):
        ops = ", ".join(f"%{o}" for o in operands)
        body = name + (f" {attr}" if attr else "") + (f" {ops}" if ops else "")
        return self._node(shape, body)

    def out(self, *ids):
        self.outs += list(ids)
        return self

    def text(self):
        return "\n".join(self.params + self.lines + [f"output %{o}" for o in self.outs]) + "\n"


def ty(shape, dtype="f32"):
    return f"Tensor<{dtype}, [{', '.join(str(d) for d in shape)}]>"


# ---- float64 references ---------------------------------------------------------------------
GELU_S = float(np.float32(0.7978845608028654))
GELU_C = float(np.float32(0.044715))


def gelu64(x):
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def layer_norm64(x, g, b):
    x = np.asarray(x, np.float64)
    m = x.mean(axis=1, keepdims=True)
    v = ((x - m) ** 2).mean(axis=1, keepdims=True)
    return (x - m) / np.sqrt(v + 1e-12) * g + b


def attention64(q, k, v, mask, heads):
    """q [B*L, H], k/v [B*S, H], mask [B, S]: masked softmax(q k^T / sqrt(d)) v per head."""
    B, S = mask.shape
    L = q.shape[0] // B
    H = q.shape[1]
    d = H // heads
    out = np.zeros((B * L, H))
    for b in range(B):
        keys = mask[b] != 0
        for a in range(heads):
            cs = slice(a * d, (a + 1) * d)
            qb = q[b * L:(b + 1) * L, cs].astype(np.float64)
            kb = k[b * S:(b + 1) * S, cs].astype(np.float64)[keys]
            vb = v[b * S:(b + 1) * S, cs].astype(np.float64)[keys]
            s = qb @ kb.T / np.sqrt(d)
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b * L:(b + 1) * L, cs] = p @ vb
    return out


def cross_entropy64(logits, labels, w):
    x = np.asarray(logits, np.float64)
    m = x.max(axis=1, keepdims=True)
    lse = (m + np.log(np.exp(x - m).sum(axis=1, keepdims=True)))[:, 0]
    loss = lse - x[np.arange(x.shape[0]), labels]
    den = np.sum(np.asarray(w, np.float64))
    return 0.0 if den == 0 else float(np.sum(w * loss) / den)


def central_difference(f, x, eps=1e-6):
    """d f / d x of a scalar float64 function, by central differences, element by element."""
    x = np.array(x, np.float64)
    g = np.zeros_like(x)
    flat, gflat = x.reshape(-1), g.reshape(-1)
    for i in range(flat.size):
        keep = flat[i]
        flat[i] = keep + eps
        up = f(x)
        flat[i] = keep - eps
        down = f(x)
        flat[i] = keep
        gflat[i] = (up - down) / (2 * eps)
    return g
