"""Benchmark of the BERT-tiny masked-LM training step on one MI355X.

One step = forward + backward + AdamW of BERT-tiny (2 layers, hidden 128, 2 heads, FFN 512,
V = 30522, batch 32, seq 128, dropout 0.1, the masked-row gather of 832 rows) on synthetic Zipf
tokens with BERT masking, captured once in a hipGraph and relaunched per step. The timed region
holds only device work: every step's host inputs (tokens, masks, dropout ids, AdamW scalars) are
made before it and staged per step through pinned memory.

Prints one JSON line: the median ms/step (the metric), tokens/s, the roofline fraction of the
dominant kernel (algorithmic FLOP or bytes per launch over its mean launch time, timed with HIP
events on the run's stream), and the CPU oracle (a single-threaded restatement of the reference
interpreter) timed on a bounded sample of the same step on this host.
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
CONFIG = "bert_tiny"
TOKENS = 32 * 128

# The HIP kernels each planned launch runs (the names rocprofv3 reports).
SYMBOLS = {
    "MatMul": "k_gemm", "MatMul+AddRows": "k_gemm", "EmbeddingGrad": "k_fill_zero+k_sort_ids+k_segment_sum",
    "CrossEntropy": "k_ce_stats+k_ce_loss", "CrossEntropyGrad": "k_ce_grad", "Attention": "k_attn_fwd_mfma",
    "AttentionGradQ": "k_attn_bwd_q_mfma+k_attn_bwd_kv_mfma", "AttentionGradK": "k_attn_bwd_q_mfma+k_attn_bwd_kv_mfma",
    "AttentionGradV": "k_attn_bwd_q_mfma+k_attn_bwd_kv_mfma", "LayerNorm": "k_layer_norm", "LayerNormGradX": "k_ln_grad_x",
    "LayerNormGradGamma": "k_column_partial+k_column_final", "SumRows": "k_column_partial+k_column_final",
    "Dropout": "k_dropout", "DropoutGrad": "k_dropout", "AdamW": "k_adamw", "Embedding": "k_embedding",
    "Transpose": "k_transpose", "AddRows": "k_add_rows",
}


def roofline(rows):
    """The launch with the largest mean time, and every launch's fraction of its roofline."""
    table = []
    for what, ms, flop, nbytes in rows:
        if ms <= 0:
            continue
        if flop > 0:
            achieved, peak, unit, bound = flop / (ms * 1e-3), PEAK_FP32_MFMA, "TFLOP/s", "mfma"
            achieved, peak = achieved / 1e12, peak / 1e12
        else:
            achieved, peak, unit, bound = nbytes / (ms * 1e-3), PEAK_HBM, "GB/s", "hbm"
            achieved, peak = achieved / 1e9, peak / 1e9
        table.append({"launch": what, "ms": ms, "bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
                      "frac": achieved / peak, "flop": flop, "bytes": nbytes,
                      "kernel": SYMBOLS.get(what.split()[0], "k_elementwise")})
    table.sort(key=lambda r: -r["ms"])
    return table


def cpu_baseline(steps):
    """The CPU oracle on `steps` steps of the same config, single-threaded."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib
    o = oracle_lib.Oracle()
    t0 = time.time()
    s = o.seconds_per_step(CONFIG, steps)
    wall = time.time() - t0
    return {"value": s * 1e3, "unit": "ms/step", "cores": 1, "kind": "port",
            "sample": f"{steps} training steps of {CONFIG} (b32 s128, V 30522, masked rows 832) on the "
                      f"single-threaded C++ oracle, {wall:.1f} s of CPU work, after input generation",
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
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--profile-reps", type=int, default=5)
    ap.add_argument("--cpu-steps", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    from modelspec_amd import api
    ctx = api.Context(0)
    mean_ms, per_step, last_loss, rows = api.bench_config(ctx, CONFIG, args.warmup, args.steps,
                                                          profile_reps=args.profile_reps)
    median_ms = statistics.median(per_step)
    table = roofline(rows)
    top = table[0]
    stats = ctx.stats()
    ctx.close()
    out = {
        "metric": "BERT-tiny b32 s128 train ms/step (median) + per-kernel % of MFMA/HBM roofline",
        "value": round(median_ms, 4),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(median_ms, 4),
        "mean_ms_per_step": round(mean_ms, 4),
        "tokens_per_s": round(TOKENS / (median_ms * 1e-3), 1),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: Zipf(1.1) token ids, BERT 80/10/10 masking at 0.15, random-init (xavier) weights",
        "config": {"workload": "bert_tiny masked-LM train step (fwd + bwd + AdamW), 2 layers, H 128, 2 heads, "
                               "FFN 512, V 30522, dropout 0.1, masked-row gather 832",
                   "global_batch": 32, "seq_len": 128, "parallelism": "single-gpu"},
        "last_loss": last_loss,
        "kernels_per_step": stats["kernels_per_step"],
        "roofline": {"bound": top["bound"], "achieved": round(top["achieved"], 2), "peak": top["peak"],
                     "unit": top["unit"], "frac": round(top["frac"], 4), "traffic": None,
                     "kernel": top["kernel"], "launch": top["launch"], "launch_ms": round(top["ms"], 5),
                     "algorithmic": top["flop"] if top["bound"] == "mfma" else top["bytes"]},
        "top_kernels": [{k: (round(v, 5) if isinstance(v, float) else v) for k, v in r.items()
                         if k in ("launch", "ms", "bound", "frac", "kernel")} for r in table[:12]],
        "profiled_step_ms": round(sum(r[1] for r in rows), 4),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_steps)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
