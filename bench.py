"""Benchmark of the BERT-tiny masked-LM training step on one MI355X;
with `--config bert_base`, of the BERT-base mixed-precision step.

One step = forward + backward + AdamW of BERT-tiny (2 layers, hidden 128, 2 heads, FFN 512,
V = 30522, batch 32, seq 128, dropout 0.1, the masked-row gather of 832 rows) on synthetic Zipf
tokens with BERT masking, captured once in a hipGraph and relaunched per step. The timed region
holds only device work: every step's host inputs (tokens, masks, dropout ids, AdamW scalars) are
made before it and staged per step through pinned memory.

Prints one JSON line: the median ms/step (the metric), tokens/s, the roofline fraction of the
dominant kernel (algorithmic FLOP or bytes per launch over its mean launch time, timed with HIP
events on the run's stream), and the CPU oracle (a single-threaded restatement of the reference
interpreter) timed on a bounded sample of the same step on this host.

BERT-base (12 layers, H 768, 12 heads, FFN 3072, V 30522, batch 32, seq 512) runs its GEMMs and
attention as f16 MFMA with f32 accumulation, f32 master weights and activations, and dynamic loss
scaling from 2^16; its GEMM and f16 attention launches are priced against the f16 MFMA peak. One oracle step of it is ~10^13 flop of scalar code (hours), so that line carries no CPU
baseline.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM = 8.0e12          # bytes/s, MI355X
PEAK_FP32_MFMA = 157.3e12  # flop/s, dense
PEAK_FP16_MFMA = 2.5e15    # flop/s, dense
WORKLOADS = {
    "bert_tiny": {
        "metric": "BERT-tiny b32 s128 train ms/step (median) + per-kernel % of MFMA/HBM roofline",
        "tokens": 32 * 128, "dtype": "f32", "mixed": False,
        "config": {"workload": "bert_tiny masked-LM train step (fwd + bwd + AdamW), 2 layers, H 128, 2 heads, "
                               "FFN 512, V 30522, dropout 0.1, masked-row gather 832",
                   "global_batch": 32, "seq_len": 128, "parallelism": "single-gpu"}},
    "bert_base": {
        "metric": "BERT-base b32 s512 mixed-precision train ms/step (median) + per-kernel % of MFMA/HBM roofline",
        "tokens": 32 * 512, "dtype": "f16 MFMA / f32 accumulate, f32 master weights", "mixed": True,
        "config": {"workload": "bert_base masked-LM train step (fwd + bwd + AdamW, dynamic loss scale from 2^16), "
                               "12 layers, H 768, 12 heads, FFN 3072, V 30522, dropout 0.1, masked-row gather 15%",
                   "global_batch": 32, "seq_len": 512, "parallelism": "single-gpu"}},
}

def roofline(rows, mixed=False):
    """The launch with the largest mean time, and every launch's fraction of its roofline. Under
    mixed precision a GEMM's and the f16 attention kernels' (`k_attn_*_h16`) peak is the f16 MFMA
    one; an f32 attention kernel is priced at the f32 MFMA peak."""
    table = []
    for what, ms, flop, nbytes, kernels, _ in rows:
        if ms <= 0:
            continue
        if flop > 0:
            f32_attn = "attn" in kernels and "_h16" not in kernels
            peak = PEAK_FP16_MFMA if mixed and not f32_attn else PEAK_FP32_MFMA
            achieved, unit, bound = flop / (ms * 1e-3), "TFLOP/s", "mfma"
            achieved, peak = achieved / 1e12, peak / 1e12
        else:
            achieved, peak, unit, bound = nbytes / (ms * 1e-3), PEAK_HBM, "GB/s", "hbm"
            achieved, peak = achieved / 1e9, peak / 1e9
        table.append({"launch": what, "ms": ms, "bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
                      "frac": achieved / peak, "flop": flop, "bytes": nbytes,
                      "kernel": kernels})
    table.sort(key=lambda r: -r["ms"])
    return table


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "dominant_launch_traffic.md")


def measured_traffic(launch):
    """HBM bytes per dispatch of `launch` from the committed rocprofv3 counter summary (FETCH_SIZE +
    WRITE_SIZE, each scaled by the counters' reading of a copy of known size), when it covers this
    launch; else None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("| traffic |"):
                    cells = [c.strip() for c in line.strip().strip("|").split("|")]
                    if cells[1].strip("`") == launch:
                        return float(cells[4])
    except (OSError, ValueError, IndexError):
        pass
    return None


def copy_once(ctx, mib):
    """One elementwise copy of `mib` MiB on the device (StopGradient: read n floats, write n)."""
    import numpy as np
    n = mib * (1 << 20) // 4
    prog = ctx.program(f'%0: Tensor<f32, [{n}]> = Input "x"\n%1: Tensor<f32, [{n}]> = StopGradient %0\noutput %1\n')
    try:
        prog.run({"x": np.zeros(n, np.float32)})
    finally:
        prog.close()


def quantile(xs, q):
    """The q-quantile of xs, linear between order statistics."""
    ys = sorted(xs)
    at = q * (len(ys) - 1)
    lo = int(at)
    hi = min(lo + 1, len(ys) - 1)
    return ys[lo] + (ys[hi] - ys[lo]) * (at - lo)


def _oracle_step_times(config, steps):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    return list(oracle_lib.Oracle().step_times(config, steps))


class CpuBaseline:
    """The CPU oracle (a single-threaded C++ restatement of the reference interpreter) on
    `workers` x `steps` training steps of the config, as `workers` processes of one thread each,
    started after the GPU run; the value is the median step. Spawned (not forked) processes, so no
    child inherits a GPU context."""

    def __init__(self, config, workers, steps):
        import multiprocessing as mp
        self.config, self.workers, self.steps = config, workers, steps
        self.t0 = time.time()
        self.pool = mp.get_context("spawn").Pool(workers)
        self.pending = [self.pool.apply_async(_oracle_step_times, (config, steps)) for _ in range(workers)]

    def result(self):
        times = [t for p in self.pending for t in p.get()]
        self.pool.close()
        self.pool.join()
        wall = time.time() - self.t0
        return {"value": statistics.median(times) * 1e3, "unit": "ms/step", "cores": 1, "kind": "port",
                "sample": f"median of {len(times)} training steps of {self.config} (b32 s128, V 30522, masked rows "
                          f"832) on the single-threaded C++ oracle, each step on one core: {self.workers} concurrent "
                          f"processes of {self.steps} steps, {sum(times):.1f} s of CPU work in {wall:.1f} s wall, "
                          f"inputs made before each step loop",
                "p10_ms": quantile(times, 0.1) * 1e3, "p90_ms": quantile(times, 0.9) * 1e3,
                "cpu": cpu_model(), "nproc": os.cpu_count()}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--config", choices=sorted(WORKLOADS), default="bert_tiny")
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--profile-reps", type=int, default=5)
    ap.add_argument("--cpu-steps", type=int, default=5, help="oracle steps per CPU worker")
    ap.add_argument("--cpu-workers", type=int, default=4, help="concurrent single-threaded oracle processes")
    ap.add_argument("--settle", type=int, default=64, metavar="N",
                    help="untimed steps before the timed region: at least N steps run in all (the W warmup "
                         "steps count toward it)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--fuse-ce-head", choices=("on", "off"), default=None,
                    help="force MSX_FUSE_CE_HEAD on or off (default: the library's default)")
    ap.add_argument("--step-times", action="store_true", help="print every timed step's ms to stderr")
    ap.add_argument("--launches", metavar="FILE", help="write every profiled launch (order, time, work, "
                    "kernels) to FILE as JSON lines")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after the bench, copy MIB MiB once with the elementwise kernel (a known-size "
                         "reference dispatch for the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    w = WORKLOADS[args.config]
    from modelspec_amd import api
    ctx = api.Context(0)
    if args.fuse_ce_head is not None:
        ctx.set_fusion(ce_head=args.fuse_ce_head == "on")
    # A fresh process's first ~25 steps hold stalls of 1.5-8 ms (measured on one MI355X, with and
    # without the hipGraph and the side stream); from 50 steps on there are none. The settle steps
    # run untimed after the W warmup steps' inputs, before the barrier that opens the timed region.
    untimed = max(args.warmup, args.settle)
    mean_ms, per_step, last_loss, rows = api.bench_config(ctx, args.config, untimed, args.steps,
                                                          profile_reps=args.profile_reps)
    median_ms = statistics.median(per_step)
    if args.step_times:
        print("step ms: " + " ".join(f"{x:.4f}" for x in per_step), file=sys.stderr, flush=True)
    table = roofline(rows, w["mixed"])
    top = table[0]
    if args.launches:
        with open(args.launches, "w") as f:
            for what, ms, flop, nbytes, kernels, runs in rows:
                f.write(json.dumps({"launch": what, "ms": ms, "flop": flop, "bytes": nbytes, "kernels": kernels,
                                    "runs": runs}) + "\n")
    # Where the dominant launch's dispatches sit in a profiled step (rocprofv3 counter runs).
    first = 0
    for what, _, _, _, kernels, runs in rows:
        if what == top["launch"]:
            break
        first += (len(kernels.split("+")) if kernels else 0) * runs
    dispatches = {"step_dispatches": sum((len(r[4].split("+")) if r[4] else 0) * r[5] for r in rows), "first": first,
                  "count": len(top["kernel"].split("+")) if top["kernel"] else 0}
    traffic = measured_traffic(top["launch"]) if args.config == "bert_tiny" else None
    stats = ctx.stats()
    ctx_scale = list(ctx.loss_scale()) if w["mixed"] else None
    if args.copy_calibration > 0:
        copy_once(ctx, args.copy_calibration)
    ctx.close()
    out = {
        "metric": w["metric"],
        "value": round(median_ms, 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "untimed_steps": untimed,
        "ms_per_step": round(median_ms, 4),
        "mean_ms_per_step": round(mean_ms, 4),
        "p10_ms": round(quantile(per_step, 0.1), 4),
        "p90_ms": round(quantile(per_step, 0.9), 4),
        "max_ms": round(max(per_step), 4),
        "tokens_per_s": round(w["tokens"] / (median_ms * 1e-3), 1),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w["dtype"],
        "data": "synthetic: Zipf(1.1) token ids, BERT 80/10/10 masking at 0.15, random-init (xavier) weights",
        "config": w["config"],
        "last_loss": last_loss,
        "kernels_per_step": stats["kernels_per_step"],
        "roofline": {"bound": top["bound"], "achieved": round(top["achieved"], 2), "peak": top["peak"],
                     "unit": top["unit"], "frac": round(top["frac"], 4), "traffic": traffic,
                     "dispatches": dispatches,
                     "kernel": top["kernel"], "launch": top["launch"], "launch_ms": round(top["ms"], 5),
                     "algorithmic": top["flop"] if top["bound"] == "mfma" else top["bytes"]},
        "top_kernels": [{k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()
                         if k in ("launch", "ms", "bound", "frac", "kernel")} for r in table[:12]],
        "profiled_step_ms": round(sum(r[1] for r in rows), 4),
    }
    if w["mixed"]:
        out["loss_scale"] = ctx_scale
    # The CPU baseline runs after the GPU run has finished (its processes start once the context is
    # closed), so neither competes with the other for host cores or memory.
    if not args.no_cpu and args.config == "bert_tiny":
        out["cpu_baseline"] = CpuBaseline(args.config, args.cpu_workers, args.cpu_steps).result()
        out["cpu_baseline"]["overlapped_gpu_run"] = False
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
