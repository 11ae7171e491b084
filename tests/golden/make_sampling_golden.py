"""Writes tests/golden/sampling_golden.npz from the reference's own sampler.

oracle/_ref/ref_sampling is the reference's src/gpt_sampling.cpp compiled where it lies
(oracle/Makefile, target `ref`).  This script feeds it seeded logits/histories in the
schema of the reference's sampling fixture (main.cpp:147-158: `logits`, `history`,
`{case}.config = [temperature, top_k, top_p, repetition_penalty, num_beams]`,
`{case}.allowed`, `{case}.values`) plus sampled draws, and stores inputs and outputs.

    make -C oracle ref && python tests/golden/make_sampling_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "oracle"))
import oracle  # noqa: E402

CASES = {
    # name: (temperature, top_k, top_p, repetition_penalty, num_beams)
    "standard": (0.8, 30, 0.8, 10.0, 1),
    "beam": (0.8, 30, 0.8, 10.0, 3),
    "beam_edge": (1.0, 1, 0.05, 2.0, 3),
    "unfiltered": (1.0, 0, 1.0, 1.0, 1),
    "topp_only": (1.0, 0, 0.6, 1.0, 1),
    "wide_topk": (1.1, 2000, 0.97, 1.3, 1),
}


def main() -> None:
    if not oracle.ref_available():
        raise SystemExit("build oracle/_ref first: make -C oracle ref")
    ref = oracle.RefSampler()
    out = {}
    rng = np.random.default_rng(20261002)
    for variant in ("", "_ties"):
        logits = (rng.standard_normal(8194) * 3).astype(np.float32)
        if variant:
            logits = (np.round(logits * 2) / 2).astype(np.float32)
        history = np.concatenate([[1, 8192], rng.integers(0, 8194, 24)]).astype(np.uint32)
        for name, cfg in CASES.items():
            case = name + variant
            values = ref.processors(logits, history, *cfg)
            if isinstance(values, str):
                raise SystemExit(f"{case}: reference raised {values}")
            seed = int(rng.integers(0, 2**63))
            draws, state = ref.sample(values, seed, 16)
            out[case + ".logits"] = logits
            out[case + ".history"] = history
            out[case + ".config"] = np.array(cfg, np.float32)
            out[case + ".allowed"] = np.isfinite(values).astype(np.uint8)
            out[case + ".values"] = values
            out[case + ".draw_seed"] = np.array([seed], np.uint64)
            out[case + ".draws"] = np.array(draws, np.uint32)
            out[case + ".draw_state"] = np.array([state], np.uint64)
    # Signed zeros: the top-p comparator (gpt_sampling.cpp:78-83) finds -0 and +0 equal and
    # orders them by index.  "zeros_mixed": the top-p cut falls inside a run of alternating
    # +0/-0 scores; "zeros_only": every score is a zero and the kept top entry (the highest
    # index, a -0) decides the survivors.
    zeros = {}
    mixed = np.where(np.arange(8194) % 2 == 0, 0.0, -0.0).astype(np.float32)
    mixed[rng.choice(8194, 40, replace=False)] = 2.0
    mixed[:1500] = -4.0
    zeros["zeros_mixed"] = (mixed, [(1.0, 0, 0.5, 1.0, 1), (0.9, 0, 0.3, 1.0, 3), (1.0, 5000, 0.2, 1.0, 1)])
    only = np.where(np.arange(8194) % 2 == 0, 0.0, -0.0).astype(np.float32)
    zeros["zeros_only"] = (only, [(1.0, 0, 0.01, 1.0, 1), (1.0, 0, 0.5, 1.0, 3)])
    for name, (logits, cfgs) in zeros.items():
        history = np.array([1, 8192, 7, 8, 9], np.uint32)
        for c, cfg in enumerate(cfgs):
            case = f"{name}_{c}"
            values = ref.processors(logits, history, *cfg)
            if isinstance(values, str):
                raise SystemExit(f"{case}: reference raised {values}")
            allowed = np.isfinite(values)
            z = logits == 0
            if not (allowed[z].any() and not allowed[z].all()):
                raise SystemExit(f"{case}: the top-p cut does not split the zeros")
            seed = int(rng.integers(0, 2**63))
            draws, state = ref.sample(values, seed, 16)
            out[case + ".logits"] = logits
            out[case + ".history"] = history
            out[case + ".config"] = np.array(cfg, np.float32)
            out[case + ".allowed"] = allowed.astype(np.uint8)
            out[case + ".values"] = values
            out[case + ".draw_seed"] = np.array([seed], np.uint64)
            out[case + ".draws"] = np.array(draws, np.uint32)
            out[case + ".draw_state"] = np.array([state], np.uint64)
    ref.close()
    np.savez_compressed(HERE / "sampling_golden.npz", **out)
    print(f"wrote {len(out)} arrays to {HERE / 'sampling_golden.npz'}")


if __name__ == "__main__":
    main()
