#!/usr/bin/env python3
"""Benchmark of the GPT semantic-token loop on one MI355X.

Workload (one "step"): the full-length sampled decode of the 24-layer d=1280 FP32 GPT at
batch 1 -- prefix of 32 conditioning latents ~N(0,1)*0.5 plus 120 text ids (155 prefix
rows), prefill, then 600 codes sampled with temperature 0.8, top_k 30, top_p 0.8,
repetition penalty 10, SplitMix64 seed 42; the KV cache grows to 754 rows.  Random-init
weights N(0, 0.02).  Codes 8192/8193 are suppressed so every step yields exactly 600
codes (suppress_stop; applied identically by the CPU oracle).

Prints one JSON line: tokens/s of whole generate() calls (prefill included) with inputs
resident on the device, the roofline of the dominant kernel (mlp.c_proj GEMV, 26 MB of
weights per launch) from HIP-event timing, and the CPU oracle timed on a bounded sample.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "index-tts-25-metal_amd"))

HBM_PEAK_GBS = 8000.0
WEIGHT_BYTES_PER_TOKEN = 1_931_051_016  # FP32 weights + biases + LayerNorm + mel_head + 2 embedding rows
KV_BYTES_PER_ROW = 245_760              # 24 layers x (K + V) x 1280 x 4 B


def decode_bytes(prefix_rows: int, tokens: int) -> float:
    """Algorithmic HBM bytes of the decode steps of one generate(): tokens-1 forwards."""
    total = 0.0
    for i in range(1, tokens):
        n = prefix_rows + i - 1  # cached rows before the forward
        total += WEIGHT_BYTES_PER_TOKEN + KV_BYTES_PER_ROW * (n + 1)
    return total


def cpu_baseline(weights, prefix, opts, sample_steps: int):
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or min(16, os.cpu_count() or 1)
    orc = oracle.OracleGpt(weights, kv_capacity=4096)
    o = oracle.options_from(opts)
    t0 = time.perf_counter()
    orc.prefill(prefix)
    t1 = time.perf_counter()
    lg = None
    code = 100
    for i in range(sample_steps):
        lg = orc.step(code, i + 2)
        code = int(np.argmax(lg[:8192]))
    t2 = time.perf_counter()
    del orc
    return {
        "value": round(sample_steps / (t2 - t1), 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle prefill of the 155-row prefix ({t1 - t0:.2f} s) + {sample_steps} decode steps of the same 24-layer FP32 model",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--tokens", type=int, default=600)
    ap.add_argument("--cpu-steps", type=int, default=24)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr)
        return 2

    import itts_gpt as it

    weights = it.make_synthetic_weights(layers=24, seed=0)
    cond, text = it.synthetic_prefix_inputs(120, seed=42)
    dec = it.GptDecoder(weights, kv_capacity=4096)
    prefix = dec.prepare_cond(cond, text, 0)
    rows = prefix.size // 1280
    opts = it.GenerationOptions(do_sample=True, seed=42, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0,
                                suppress_stop=True)
    for _ in range(args.warmup):
        dec.generate(prefix, opts, args.tokens)
    times, prefill_ms, decode_ms = [], [], []
    codes = None
    for _ in range(args.steps):
        t0 = time.perf_counter()
        r = dec.generate(prefix, opts, args.tokens)
        times.append(time.perf_counter() - t0)
        tm = dec.last_timing()
        prefill_ms.append(tm["prefill_ms"])
        decode_ms.append(tm["decode_ms"])
        assert len(r.codes) == args.tokens, len(r.codes)
        if codes is not None:
            assert r.codes == codes, "generate() is not deterministic"
        codes = r.codes
    total = sum(times)
    value = args.tokens * args.steps / total
    dmean = float(np.mean(decode_ms))
    step_bytes = decode_bytes(rows, args.tokens)
    step_gbs = step_bytes / (dmean * 1e-3) / 1e9

    kern = dec.bench_kernel("gemv_mlp_proj", iters=240)
    achieved = kern["bytes"] / (kern["avg_ms"] * 1e-3) / 1e9
    kernels = {k: dec.bench_kernel(k, iters=240 if k != "gemv_mel_head" else 48) for k in it.GptDecoder.KERNELS}
    extra = {k: {"avg_us": round(v["avg_ms"] * 1e3, 2), "GB/s": round(v["bytes"] / (v["avg_ms"] * 1e-3) / 1e9, 1)}
             for k, v in kernels.items()}

    traffic = None
    pmc = ROOT / "profiles" / "gemv_mlp_proj_traffic.json"
    if pmc.exists():
        traffic = json.loads(pmc.read_text()).get("bytes_per_launch")

    line = {
        "metric": "GPT decode tokens/s @bs1 FP32 + % of HBM roofline; beam-3 tokens/s",
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (random-init N(0,0.02) weights, seeded prefix)",
        "config": {
            "workload": "IndexTTS-2.5 GPT 24L d1280 FP32, batch 1, prefix 32 latents + 120 text ids (155 rows), "
                        "600 sampled codes (T0.8 k30 p0.8 rep10 seed42), KV to 754",
            "batch": 1, "prefix_rows": rows, "tokens": args.tokens,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_mlp_proj (mlp.c_proj 1280x5120 GEMV + residual)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "decode": {
            "prefill_ms": round(float(np.mean(prefill_ms)), 3),
            "decode_ms": round(dmean, 3),
            "decode_tokens_per_s": round((args.tokens - 1) / (dmean * 1e-3), 2),
            "step_algorithmic_GBps": round(step_gbs, 1),
            "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        },
        "kernels": extra,
    }
    del dec
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(weights, prefix, opts, args.cpu_steps)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
