"""Writes tests/golden/full_configs.npz: the CPU oracle's codes and logits for the full-size
workloads of the 24-layer d=1280 FP32 GPT (synthetic weights N(0, 0.02), seed 0).

    python tests/golden/make_full_config_golden.py          # about 8 minutes on 8 cores
    python tests/golden/make_full_config_golden.py c3       # one workload, merged into the file

Workloads (the same inputs bench.py times):
  c2  32 latents + 120 text ids (seed 42; 155 prefix rows), 600 codes sampled with
      temperature 0.8, top_k 30, top_p 0.8, repetition penalty 10, seed 42; KV to 754 rows.
  c3  32 latents + 80 text ids (seed 3; 115 prefix rows), beam search with 3 beams, length
      penalty 0, repetition penalty 10, 400 codes: c3s sampled beams (temperature 0.8, top_k 30,
      top_p 0.8, seed 7), c3g greedy beams (do_sample false).  KV to 514 rows per beam.
  c4  32 latents + 200 text ids (seed 4; 235 rows), greedy (penalty 1) to 1813 codes; the
      KV cache reaches 2047 rows.
  c5  8 sequences, 32 latents + U[24, 200] text ids (lengths from default_rng(7), inputs
      seed 100 + b), 300 codes each sampled with the default options and seed 1000 + b.
All of them suppress codes 8192/8193 (fixed-length runs; the oracle and the HIP path apply the
same rule).  Stored: the codes, and the oracle's logits at chosen steps of the teacher-forced
replay of those codes (step 0 = the prefill logits; step t >= 1 = the logits of the forward
of code t-1 at mel position t+1, after which the cache holds prefix_rows + t rows).

The oracle is the checker here: these are its outputs, written once in the container and
compared with the HIP path on the GPU (tests/test_gpu_full_configs.py).
"""
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "index-tts-25-metal_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

import itts_gpt as it  # noqa: E402  (host-only helpers: synthetic weights and inputs)
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "full_configs.npz"

C2_STEPS = [0, 1, 300, 598, 599]
C3_STEPS = [0, 1, 200, 399]
C4_STEPS = [0, 789, 790, 1100, 1500, 1812]  # 235 + 789 = 1024 cached rows: attention beyond 16 splits of 64
C5_STEPS = [0, 299]


def c5_inputs():
    rng = np.random.default_rng(7)
    return [it.synthetic_prefix_inputs(int(rng.integers(24, 201)), seed=100 + b) for b in range(8)]


def replay(orc, prefix, codes, keep):
    """Teacher-forced oracle logits along `codes` at the steps in `keep`."""
    out = {}
    lg = orc.prefill(prefix)
    if 0 in keep:
        out[0] = lg
    last = max(keep)
    for t in range(1, last + 1):
        lg = orc.step(codes[t - 1], t + 1)
        if t in keep:
            out[t] = lg
    return np.stack([out[t] for t in keep])


def c2(orc, data):
    cond, text = it.synthetic_prefix_inputs(120, seed=42)
    prefix = orc.prepare_cond(cond, text, 0)
    o = oracle.options(do_sample=True, seed=42, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0,
                       suppress_stop=True)
    codes, stopped = orc.generate(prefix, o, 600)
    assert len(codes) == 600 and not stopped
    data["c2.codes"] = np.array(codes, np.uint32)
    data["c2.steps"] = np.array(C2_STEPS, np.int32)
    data["c2.logits"] = replay(orc, prefix, codes, C2_STEPS)


def c3_options(sampled: bool):
    """Config 3's beam options; the sampled run is the one bench.py times."""
    if sampled:
        return oracle.options(do_sample=True, seed=7, num_beams=3, length_penalty=0.0, repetition_penalty=10.0,
                              suppress_stop=True)
    return oracle.options(do_sample=False, num_beams=3, length_penalty=0.0, repetition_penalty=10.0, suppress_stop=True)


def c3(orc, data):
    cond, text = it.synthetic_prefix_inputs(80, seed=3)
    prefix = orc.prepare_cond(cond, text, 0)
    assert prefix.size // 1280 == 115
    for tag, sampled in (("c3s", True), ("c3g", False)):
        codes, stopped = orc.generate(prefix, c3_options(sampled), 400)
        assert len(codes) == 400 and not stopped
        data[f"{tag}.codes"] = np.array(codes, np.uint32)
        data[f"{tag}.steps"] = np.array(C3_STEPS, np.int32)
        data[f"{tag}.logits"] = replay(orc, prefix, codes, C3_STEPS)


def c4(orc, data):
    cond, text = it.synthetic_prefix_inputs(200, seed=4)
    prefix = orc.prepare_cond(cond, text, 0)
    assert prefix.size // 1280 == 235
    o = oracle.options(do_sample=False, repetition_penalty=1.0, suppress_stop=True)
    codes, stopped = orc.generate(prefix, o, 1813)
    assert len(codes) == 1813 and not stopped
    data["c4.codes"] = np.array(codes, np.uint32)
    data["c4.steps"] = np.array(C4_STEPS, np.int32)
    data["c4.logits"] = replay(orc, prefix, codes, C4_STEPS)


def c5(orc, data):
    rows, all_codes, logits = [], [], []
    for b, (cond, text) in enumerate(c5_inputs()):
        prefix = orc.prepare_cond(cond, text, 0)
        o = oracle.options(seed=1000 + b, suppress_stop=True)
        codes, stopped = orc.generate(prefix, o, 300)
        assert len(codes) == 300 and not stopped
        rows.append(prefix.size // 1280)
        all_codes.append(codes)
        logits.append(replay(orc, prefix, codes, C5_STEPS))
    data["c5.rows"] = np.array(rows, np.int32)
    data["c5.codes"] = np.array(all_codes, np.uint32)
    data["c5.steps"] = np.array(C5_STEPS, np.int32)
    data["c5.logits"] = np.stack(logits)


WORKLOADS = {"c2": c2, "c3": c3, "c4": c4, "c5": c5}


def main(names) -> None:
    """Writes every workload, or only `names`, merged over what the file already holds."""
    t0 = time.time()
    w = it.make_synthetic_weights(layers=24, seed=0)
    orc = oracle.OracleGpt(w, kv_capacity=4096)
    data = {}
    if names and OUT.exists():
        with np.load(OUT, allow_pickle=False) as old:
            data = {k: old[k] for k in old.files}
    for name in names or list(WORKLOADS):
        WORKLOADS[name](orc, data)
        print(f"{name} done {time.time() - t0:.0f} s", flush=True)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main(sys.argv[1:])
