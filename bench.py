#!/usr/bin/env python3
"""Benchmark of the GPT semantic-token loop on one MI355X.

Headline workload (one "step" of the contract = one whole generate() call): full-length
sampled decode of the 24-layer d=1280 FP32 GPT at batch 1 -- prefix of 32 conditioning
latents ~N(0,1)*0.5 plus 120 text ids (155 prefix rows), prefill, then 600 codes sampled
with temperature 0.8, top_k 30, top_p 0.8, repetition penalty 10, SplitMix64 seed 42; the
KV cache grows to 754 rows.  Random-init weights N(0, 0.02).  Codes 8192/8193 are
suppressed so every call yields exactly 600 codes (suppress_stop; the CPU oracle applies
the same rule).

Prints ONE JSON line: tokens/s of whole generate() calls (prefill included) with inputs
resident on the device; the roofline of the dominant decode kernel from HIP events; the
CPU oracle timed on a bounded sample; and, under "extras", the other workloads of the
same model: beam search with 3 beams, long-context greedy decode to a 2047-row cache
(attention GB/s reported separately), and 8 ragged sampled sequences with FP32 and BF16
weights.

    python bench.py                      # everything (a few minutes)
    python bench.py --no-extras --no-cpu # headline only
    python bench.py --kernel-only gemv_c_fc --iters 240   # one kernel kind, for profilers
"""
import argparse
import dataclasses
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "index-tts-25-metal_amd"))

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix-core peak
WEIGHT_BYTES_PER_TOKEN = 1_931_051_016  # FP32 weights + biases + LayerNorm + mel_head + 2 embedding rows
KV_BYTES_PER_ROW = 245_760              # 24 layers x (K + V) x 1280 x 4 B
METRIC = "GPT decode tokens/s @bs1 FP32 + % of HBM roofline; beam-3 tokens/s"


def decode_bytes(prefix_rows: int, tokens: int) -> float:
    """Algorithmic HBM bytes of the decode steps of one generate(): tokens-1 forwards."""
    total = 0.0
    for i in range(1, tokens):
        n = prefix_rows + i - 1  # cached rows before the forward
        total += WEIGHT_BYTES_PER_TOKEN + KV_BYTES_PER_ROW * (n + 1)
    return total


def prefill_flops(rows: int, layers: int = 24) -> float:
    """FLOPs of a P-row prefill: the four GEMMs per layer (2 P N K), causal attention
    (QK^T and PV over the lower triangle: 2 * 2 * 64 * P (P + 1) / 2 per head) and the head
    GEMV of the last row."""
    gemm = 2.0 * rows * (1280 * 3840 + 1280 * 1280 + 2 * 1280 * 5120)
    attn = 20 * 2.0 * 64 * rows * (rows + 1)
    return layers * (gemm + attn) + 2.0 * 8194 * 1280


def cpu_baseline(weights, prefix, sample_steps: int):
    """The FP32 CPU oracle (OpenMP over output rows) on a bounded sample of the same decode."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    cpu_model = "unknown"
    try:
        import subprocess

        for ln in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if ln.startswith("Model name:"):
                cpu_model = ln.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    orc = oracle.OracleGpt(weights, kv_capacity=4096)
    t0 = time.perf_counter()
    orc.prefill(prefix)
    t1 = time.perf_counter()
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
        "cpu_model": cpu_model,
        "host_cpus": os.cpu_count(),
        "sample": f"oracle prefill of the 155-row prefix ({t1 - t0:.2f} s) then {sample_steps} decode steps "
                  f"(KV 155..{155 + sample_steps}) of the same 24-layer FP32 model, {t2 - t1:.1f} s",
    }


def timed(fn, reps: int):
    out, times = None, []
    for _ in range(reps):
        t0 = time.perf_counter()
        out = fn()
        times.append(time.perf_counter() - t0)
    return out, times


def batch8_inputs(it, dec):
    """8 independent sequences: 32 latents + U[24, 200] text ids (lengths from seed 7, inputs seed
    100 + b), 300 sampled codes each with the default options and seed 1000 + b."""
    rng = np.random.default_rng(7)
    prefixes, opts = [], []
    for b in range(8):
        cond, text = it.synthetic_prefix_inputs(int(rng.integers(24, 201)), seed=100 + b)
        prefixes.append(dec.prepare_cond(cond, text, 0))
        opts.append(it.GenerationOptions(seed=1000 + b, suppress_stop=True))
    return prefixes, opts


QWEN_WEIGHT_BYTES = 28 * 15_728_640 * 4 + 151_936 * 1024 * 4 + (28 * 2304 + 1024) * 4  # slab, tied embedding, norms
QWEN_KV_BYTES_PER_ROW = 28 * 2 * 8 * 128 * 4                                        # K and V of one row, all layers


def qwen_step_bytes(rows: int) -> float:
    """Algorithmic HBM bytes of one Qwen decode step with `rows` cache rows after it: every
    weight byte once, the cache rows' K and V, the 151936 logits written."""
    return QWEN_WEIGHT_BYTES + QWEN_KV_BYTES_PER_ROW * rows + 151_936 * 4


def qwen_workload(it):
    """The Qwen3-0.6B emotion-text decoder (src/qwen.cpp), 28 layers, synthetic weights: a
    64-id prompt, greedy generation of 256 ids (random weights reach no EOS, so every call runs
    to the maximum), whole-call tokens/s; prefill time and the decode step's HIP-event time at
    64 + 128 cache rows."""
    q = it.QwenDecoder(it.make_synthetic_qwen_weights(seed=1))
    prompt = [int(x) for x in np.random.default_rng(12).integers(0, 151936, 64)]
    q.generate_tokens(prompt, 32)
    r, times = timed(lambda: q.generate_tokens(prompt, 256), 2)
    prefill_ms, step_us = q.bench(64, 64 + 128, 100)
    q.close()
    rows = 64 + 128 + 50  # the mean cache length over the 100 timed steps, plus the new row
    gbs = qwen_step_bytes(rows) / (step_us * 1e-6) / 1e9
    return {"prompt": 64, "generated": len(r[0]), "reached_eos": r[1], "seconds": round(min(times), 4),
            "tokens_per_s": round(len(r[0]) / min(times), 2), "prefill_ms_64": round(prefill_ms, 3),
            "step_us_at_192_rows": round(step_us, 2), "step_algorithmic_GBps": round(gbs, 1),
            "step_hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def extras(it, dec, weights):
    """Beam-3, long-context, 8-segment request and batch-8 (FP32, BF16) workloads of the same model."""
    res = {}
    # Beam search, 3 beams: 32 latents + 80 text ids, 400 codes, length penalty 0, repetition penalty 10.
    cond, text = it.synthetic_prefix_inputs(80, seed=3)
    prefix = dec.prepare_cond(cond, text, 0)
    o = it.GenerationOptions(num_beams=3, length_penalty=0.0, repetition_penalty=10.0, seed=7, suppress_stop=True)
    dec.generate(prefix, o, 32)
    r, times = timed(lambda: dec.generate(prefix, o, 400), 2)
    tm = dec.last_timing()
    steps = tm["decode_steps"]
    res["beam3"] = {
        "codes": len(r.codes), "seconds": round(min(times), 4),
        "beam_steps_per_s": round(steps / (tm["decode_ms"] * 1e-3), 2),
        "beam_tokens_per_s": round(3 * steps / (tm["decode_ms"] * 1e-3), 2),
        "prefix_rows": prefix.size // 1280,
    }
    # Long context: 32 latents + 200 text ids, greedy to the 1815 mel positions (KV -> 2047).
    cond, text = it.synthetic_prefix_inputs(200, seed=4)
    prefix = dec.prepare_cond(cond, text, 0)
    o = it.GenerationOptions(do_sample=False, repetition_penalty=1.0, suppress_stop=True)
    r, times = timed(lambda: dec.generate(prefix, o, 1813), 2)
    tm = dec.last_timing()
    rows = prefix.size // 1280
    res["long_context"] = {
        "codes": len(r.codes), "kv_rows": rows + len(r.codes) - 1,
        "decode_tokens_per_s": round((len(r.codes) - 1) / (tm["decode_ms"] * 1e-3), 2),
        "step_algorithmic_GBps": round(decode_bytes(rows, len(r.codes)) / (tm["decode_ms"] * 1e-3) / 1e9, 1),
    }
    if tm["decode_path"] == "step":
        # the path that ran: the persistent step's attention phase (tiles + merge) at the last
        # step (2046 cached rows + the new one), against its GEMV phases, from the kernel's stamps
        ph = dec.step_phases(cached_rows=2046, iters=20)
        att_us = ph["attention_tiles"] + ph["merge"]
        gemv_us = ph["c_attn"] + ph["attn_proj"] + ph["mlp_fc"] + ph["mlp_proj"]
        kv_layer = KV_BYTES_PER_ROW / 24 * 2047
        w_layer = (WEIGHT_BYTES_PER_TOKEN - 41_953_280 - 32_776 - 20_480 - 10_240) / 24
        res["long_context"]["persistent_step_at_2047_rows"] = {
            "layer_us": round(ph["layer"], 2),
            "attention_phase_us": round(att_us, 2), "attention_GBps": round(kv_layer / (att_us * 1e-6) / 1e9, 1),
            "gemv_phases_us": round(gemv_us, 2), "gemv_GBps": round(w_layer / (gemv_us * 1e-6) / 1e9, 1),
            "phases_us": {k: round(v, 2) for k, v in ph.items()},
        }
    att = dec.bench_kernel("attention", iters=240, cached_rows=2046)
    res["long_context"]["multikernel_attention_kernel_at_2047_rows"] = {
        "avg_us": round(att["avg_ms"] * 1e3, 2), "GBps": round(att["bytes"] / (att["avg_ms"] * 1e-3) / 1e9, 1)}
    prefixes, opts = batch8_inputs(it, dec)
    # One request's text segments (NativeRuntime's loop, native_runtime.cpp:98-99): 8 segments
    # of U[24, 120] text ids (seed 11), speaker/emotion conditioning, 300 sampled codes each.
    # generate_segments decodes them together; the reference's loop runs them one at a time.
    rng = np.random.default_rng(11)
    segs = [[int(x) for x in rng.integers(0, 12000, int(rng.integers(24, 121)))] for _ in range(8)]
    sp, em = it.synthetic_normal(192, 5), it.synthetic_normal(1280, 6)
    so = it.GenerationOptions(seed=500, suppress_stop=True)
    dec.generate_segments(sp, em, segs, 0, so, 16)
    r, times = timed(lambda: dec.generate_segments(sp, em, segs, 0, so, 300), 2)
    loop, ltimes = timed(lambda: [dec.generate(dec.prepare(sp, em, s, 0), dataclasses.replace(so, seed=so.seed + i), 300)
                                  for i, s in enumerate(segs)], 1)
    total = sum(len(x.codes) for x in r)
    res["segments8_f32"] = {
        "codes": total, "seconds": round(min(times), 4), "tokens_per_s": round(total / min(times), 2),
        "loop_seconds": round(min(ltimes), 4), "loop_tokens_per_s": round(total / min(ltimes), 2),
        "same_codes_as_loop": [x.codes for x in r] == [x.codes for x in loop],
    }
    # The consumer of the codes: EnhancedCodec::decode (codec.cpp:64-72) of 600 codes (config 2's
    # output) and of 47 (a short utterance), random-init codec weights; GEMM FLOPs over the
    # FP32 matrix-core peak.
    codec = it.EnhancedCodec(it.make_synthetic_codec_weights(seed=0))
    c600, c47 = codec.bench(600, 20), codec.bench(47, 20)
    codec.close()
    tf = c600["flops"] / (c600["avg_ms"] * 1e-3) / 1e12
    res["codec_decode"] = {"codes": 600, "avg_ms": round(c600["avg_ms"], 4), "TFLOPs": round(tf, 2),
                           "frac_fp32_mfma": round(tf / FP32_MFMA_PEAK_TFLOPS, 4), "codes_47_avg_ms": round(c47["avg_ms"], 4)}
    for dtype in ("f32", "bf16"):
        d = dec if dtype == "f32" else it.GptDecoder(weights, kv_capacity=4096, max_batch=8, weight_dtype="bf16")
        d.generate_batch(prefixes, opts, 16)
        r, times = timed(lambda: d.generate_batch(prefixes, opts, 300), 2)
        tm = d.last_timing()
        total = sum(len(x.codes) for x in r)
        res[f"batch8_{dtype}"] = {
            "codes": total, "seconds": round(min(times), 4),
            "tokens_per_s": round(total / min(times), 2),
            "decode_tokens_per_s": round(8 * (tm["decode_steps"] - 1) / (tm["decode_ms"] * 1e-3), 2),
        }
        if dtype == "bf16":
            ref = dec.prefill(prefixes[0])
            got = d.prefill(prefixes[0])
            res["batch8_bf16"]["prefill_logit_maxabs_vs_f32"] = float(np.max(np.abs(got - ref)))
            d.close()
    res["qwen3_emotion_decoder"] = qwen_workload(it)
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--tokens", type=int, default=600)
    ap.add_argument("--cpu-steps", type=int, default=599, help="oracle decode steps (599: KV 155..754, the whole workload)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--kernel-only", default=None, help="time one kernel kind only (for profiler runs); 'codec': a 600-code codec decode; 'beam3': the beam-3 workload; "
                         "'batch8' / 'batch8_bf16': the 8-sequence workload; "
                         "'prefill': the 155-row prefill; 'qwen': the Qwen3 emotion-text decoder")
    ap.add_argument("--iters", type=int, default=240)
    ap.add_argument("--kernel-batch", type=int, default=1, help="sequences per launch for --kernel-only")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})", file=sys.stderr)
        return 2

    import itts_gpt as it

    weights = it.make_synthetic_weights(layers=24, seed=0)
    dec = it.GptDecoder(weights, kv_capacity=4096, max_batch=8)
    if args.kernel_only == "beam3":
        # the extras' beam-3 workload alone: 32 latents + 80 text ids, 3 beams, 400 codes
        cond, text = it.synthetic_prefix_inputs(80, seed=3)
        prefix = dec.prepare_cond(cond, text, 0)
        o = it.GenerationOptions(num_beams=3, length_penalty=0.0, repetition_penalty=10.0, seed=7, suppress_stop=True)
        dec.generate(prefix, o, 32)
        r = dec.generate(prefix, o, 400)
        tm = dec.last_timing()
        print(json.dumps({"kernel": "beam3", "codes": len(r.codes), "beam_steps": tm["decode_steps"],
                          "beam_tokens_per_s": round(3 * tm["decode_steps"] / (tm["decode_ms"] * 1e-3), 2),
                          "ms_per_beam_step": round(tm["decode_ms"] / tm["decode_steps"], 4)}), flush=True)
        return 0
    if args.kernel_only == "prefill":
        # prefill of the headline's 155-row prefix, `iters` times (HIP-event time of each)
        cond, text = it.synthetic_prefix_inputs(120, seed=42)
        prefix = dec.prepare_cond(cond, text, 0)
        dec.prefill(prefix)
        ms = []
        for _ in range(args.iters):
            dec.prefill(prefix)
            ms.append(dec.last_timing()["prefill_ms"])
        rows = prefix.size // 1280
        flops = prefill_flops(rows)
        print(json.dumps({"kernel": "prefill", "rows": rows, "iters": args.iters, "avg_ms": round(float(np.mean(ms)), 4),
                          "min_ms": round(float(np.min(ms)), 4), "GFLOP": round(flops / 1e9, 2),
                          "TFLOPs": round(flops / (float(np.mean(ms)) * 1e-3) / 1e12, 2)}), flush=True)
        return 0
    if args.kernel_only in ("batch8", "batch8_bf16"):
        # the extras' batch-8 workload alone (8 ragged sequences x 300 sampled codes), for profilers
        d = dec if args.kernel_only == "batch8" else it.GptDecoder(weights, kv_capacity=4096, max_batch=8, weight_dtype="bf16")
        prefixes, opts = batch8_inputs(it, d)
        d.generate_batch(prefixes, opts, 16)
        r = d.generate_batch(prefixes, opts, 300)
        tm = d.last_timing()
        print(json.dumps({"kernel": args.kernel_only, "codes": sum(len(x.codes) for x in r), "decode_steps": tm["decode_steps"],
                          "decode_tokens_per_s": round(8 * (tm["decode_steps"] - 1) / (tm["decode_ms"] * 1e-3), 2),
                          "ms_per_step": round(tm["decode_ms"] / max(1, tm["decode_steps"] - 1), 4),
                          "prefill_ms": round(tm["prefill_ms"], 3)}), flush=True)
        return 0
    if args.kernel_only == "qwen":
        # the extras' Qwen workload alone (64-id prompt, 256 greedy ids, 28 layers), for profilers
        dec.close()
        print(json.dumps({"kernel": "qwen", **qwen_workload(it)}), flush=True)
        return 0
    if args.kernel_only == "codec":
        codec = it.EnhancedCodec(it.make_synthetic_codec_weights(seed=0))
        r = codec.bench(600, args.iters)
        print(json.dumps({"kernel": "codec_decode", "codes": 600, "iters": args.iters, "avg_ms": round(r["avg_ms"], 4),
                          "TFLOPs": round(r["flops"] / (r["avg_ms"] * 1e-3) / 1e12, 2)}), flush=True)
        return 0
    if args.kernel_only:
        k = dec.bench_kernel(args.kernel_only, iters=args.iters, batch=args.kernel_batch)
        print(json.dumps({"kernel": args.kernel_only, "batch": args.kernel_batch, "iters": args.iters,
                          "avg_us": round(k["avg_ms"] * 1e3, 3),
                          "bytes_per_launch": k["bytes"], "GBps": round(k["bytes"] / (k["avg_ms"] * 1e-3) / 1e9, 1)}),
              flush=True)
        return 0

    cond, text = it.synthetic_prefix_inputs(120, seed=42)
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
    path = dec.last_timing()["decode_path"]
    total = sum(times)
    value = args.tokens * args.steps / total
    dmean = float(np.mean(decode_ms))
    step_gbs = decode_bytes(rows, args.tokens) / (dmean * 1e-3) / 1e9

    # Dominant decode kernel: the whole-step kernel on the persistent path, else the
    # mlp.c_fc GEMV (the largest share of the multi-kernel step's time).
    dominant = "step" if path == "step" else "gemv_c_fc"
    kern = dec.bench_kernel(dominant, iters=args.iters if dominant != "step" else 60)
    achieved = kern["bytes"] / (kern["avg_ms"] * 1e-3) / 1e9
    names = [k for k in it.GptDecoder.KERNELS if k not in ("copy",) and (k != "step" or path == "step")]
    kernels = {k: dec.bench_kernel(k, iters=240 if k not in ("gemv_mel_head", "step") else 48) for k in names}
    per_kernel = {k: {"avg_us": round(v["avg_ms"] * 1e3, 2), "GBps": round(v["bytes"] / (v["avg_ms"] * 1e-3) / 1e9, 1)}
                  for k, v in kernels.items()}

    traffic = None
    pmc = ROOT / "profiles" / f"{dominant}_traffic.json"
    if pmc.exists():
        traffic = json.loads(pmc.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
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
            "batch": 1, "prefix_rows": rows, "tokens": args.tokens, "decode_path": path,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": kern["bytes"],
            "avg_us": round(kern["avg_ms"] * 1e3, 3),
        },
        "decode": {
            "prefill_ms": round(float(np.mean(prefill_ms)), 3),
            "decode_ms": round(dmean, 3),
            "decode_tokens_per_s": round((args.tokens - 1) / (dmean * 1e-3), 2),
            "step_algorithmic_GBps": round(step_gbs, 1),
            "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        },
        "kernels": per_kernel,
    }
    if path == "step":
        line["decode"]["step_phases_us_at_752_rows"] = {k: round(v, 2) for k, v in dec.step_phases(cached_rows=752, iters=20).items()}
    if not args.no_extras:
        line["extras"] = extras(it, dec, weights)
    del dec
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(weights, prefix, args.cpu_steps)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
