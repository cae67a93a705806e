"""msx_evaluate_static, the held-out evaluation that allocates no device memory, against
msx_evaluate on the same batches: the same kernels over the same logits, so every metric is
bit-identical. Two calls in a row, the second on a smaller batch, so the static array's leftover
rows and sums from the first call must not leak into the second; then a batch above the array's
65,536 rows is refused."""
import numpy as np
import pytest

from modelspec_amd import api

pytestmark = pytest.mark.gpu


def logits_forward(rows, v):
    """A forward program whose prediction is its input `x`: the held-out reduction alone."""
    _, fwd = api.compile_config("mlp_micro")
    params = [l for l in fwd.splitlines() if l.startswith("param ")]
    return "\n".join(params + [
        f'%0: Tensor<f32, [{rows}, {v}]> = Input "x"',
        f'%1: Tensor<i32, [{rows}]> = Input "labels"',
        f'%2: Tensor<f32, [{rows}]> = Input "weights"',
        "%3: Tensor<f32, []> = CrossEntropy %0, %1, %2",
        "output %3",
        "output %0",
    ]) + "\n"


def batches(rng, n, rows, v):
    logits = (rng.standard_normal((n, rows, v)) * 3).astype(np.float32)
    labels = rng.integers(0, v, (n, rows)).astype(np.int32)
    weights = rng.choice(np.array([0.0, 1.0, 0.5, 2.0], np.float32), (n, rows))
    for b in range(n):
        hit = rng.integers(0, rows, rows // 3)
        logits[b, hit, labels[b, hit]] += 20.0
    return [{"x": logits[b], "labels": labels[b], "weights": weights[b]} for b in range(n)]


def same(a, b):
    for k in ("numerator", "denominator", "correct", "selected", "loss", "accuracy"):
        assert a[k] == b[k] or (np.isnan(a[k]) and np.isnan(b[k])), (k, a[k], b[k])


def test_the_static_evaluation_equals_the_allocating_one(ctx):
    step, _ = api.compile_config("mlp_micro")
    rng = np.random.default_rng(11)
    for rows, v, n in ((4096, 512, 3), (1000, 37, 2)):
        print(f"static evaluation rows={rows} v={v} batches={n}", flush=True)
        ctx.load(step, logits_forward(rows, v), 0, 1)
        bs = batches(rng, n, rows, v)
        got = ctx.evaluate_static(bs, "labels", "weights")
        want = ctx.evaluate(bs, "labels", "weights")
        same(got, want)
        assert got["selected"] > 0 and got["correct"] > 0
    print("static evaluation over the limit", flush=True)
    ctx.load(step, logits_forward(65537, 2), 0, 1)
    with pytest.raises(api.MsxError, match="exceeds 65536"):
        ctx.evaluate_static(batches(rng, 1, 65537, 2), "labels", "weights")


def test_static_evaluations_from_two_threads_do_not_mix(ctx):
    """Two contexts on one device, each on its own thread, call the static evaluation in turn
    with different batches (ctypes releases the GIL for the call, so the calls overlap): the
    per-device lock keeps each call's sums its own, equal to that context's allocating result."""
    import threading
    step, _ = api.compile_config("mlp_micro")
    rng = np.random.default_rng(5)
    other = api.Context(0)
    try:
        jobs = []
        for c, (rows, v) in ((ctx, (4096, 512)), (other, (3000, 129))):
            c.load(step, logits_forward(rows, v), 0, 1)
            bs = batches(rng, 2, rows, v)
            jobs.append((c, bs, c.evaluate(bs, "labels", "weights")))
        errors = []

        def run(c, bs, want):
            try:
                for _ in range(20):
                    same(c.evaluate_static(bs, "labels", "weights"), want)
            except Exception as e:  # noqa: BLE001 - reported on the main thread
                errors.append(e)

        print("static evaluation on two threads", flush=True)
        threads = [threading.Thread(target=run, args=j) for j in jobs]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=100)
        assert not any(t.is_alive() for t in threads)
        assert not errors, errors
    finally:
        other.close()
