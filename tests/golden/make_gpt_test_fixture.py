"""Writes tests/golden/gpt_test_fixture.mit2: a single-file MIT2 bundle in the schema the
reference's gpt_test reads (src/main.cpp:31-66), with the CPU oracle's outputs.

    python tests/golden/make_gpt_test_fixture.py        # about a minute on 8 cores

Model: the 24-layer d=1280 FP32 GPT at the real vocabularies (text 60510, lang 107, mel 8194,
speaker projection 1280 x 192: the shapes GptDecoder's constructor checks, src/gpt.cpp:12-21),
synthetic weights N(0, 0.02) with randomised LayerNorms (make_synthetic_weights(layers=24,
seed=MODEL_SEED, ln_random=True, text_vocab=60510)); the GPU test rebuilds it from the seed.
Tensors (names, dtypes and use as in gpt_test):
  speaker [192] f32, emotion [1280] f32
  prefix.{ZH,EN,JA,ES,AR}.tokens u32, .language u32 [1], .embeddings f32 = prepare(...)
  decode.prefill.logits [8194] f32       = prefill(prefix.ZH)
  decode.{1..4}.code u32 [1], .logits    = step(code, i) after that prefill (position i)
  generation.greedy.codes u32            = generate(prefix.ZH, do_sample false, penalty 1, 8)
  generation.beam.codes u32              = the same with num_beams 3
The token lists are synthetic ids; EN's holds a 0 and a 1, which prepare drops
(src/gpt.cpp:44-48).  The oracle is the checker: these are its outputs.
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "index-tts-25-metal_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

import itts_gpt as it  # noqa: E402  (host-only helpers: synthetic weights, the MIT2 writer)
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "gpt_test_fixture.mit2"
MODEL_SEED = 25
TEXT_VOCAB = 60510
LANGS = {"ZH": (3, 9), "EN": (1, 11), "JA": (5, 7), "ES": (8, 13), "AR": (2, 6)}  # language id, token count
CODES = [17, 8191, 4096, 0]  # decode.1..4.code


def model():
    return it.make_synthetic_weights(layers=24, seed=MODEL_SEED, ln_random=True, text_vocab=TEXT_VOCAB)


def inputs():
    """speaker, emotion and each language's token list (deterministic)."""
    speaker = it.synthetic_normal(192, 251, 0.0, 1.0)
    emotion = it.synthetic_normal(1280, 252, 0.0, 0.5)
    rng = np.random.default_rng(253)
    toks = {}
    for name, (_, n) in LANGS.items():
        t = rng.integers(2, TEXT_VOCAB, n).astype(np.uint32)
        if name == "EN":
            t[2], t[7] = 0, 1
        toks[name] = t
    return speaker, emotion, toks


def main() -> None:
    w = model()
    orc = oracle.OracleGpt(w, kv_capacity=4096)
    speaker, emotion, toks = inputs()
    fx = {"speaker": speaker, "emotion": emotion}
    for name, (lang, _) in LANGS.items():
        fx[f"prefix.{name}.tokens"] = toks[name]
        fx[f"prefix.{name}.language"] = np.array([lang], np.uint32)
        fx[f"prefix.{name}.embeddings"] = orc.prepare(speaker, emotion, toks[name], lang)
    zh = fx["prefix.ZH.embeddings"]
    fx["decode.prefill.logits"] = orc.prefill(zh)
    for i, code in enumerate(CODES, start=1):
        fx[f"decode.{i}.code"] = np.array([code], np.uint32)
        fx[f"decode.{i}.logits"] = orc.step(code, i)
    greedy = oracle.options(do_sample=False, repetition_penalty=1.0)
    codes, stopped = orc.generate(zh, greedy, 8)
    fx["generation.greedy.codes"] = np.array(codes + ([8193] if stopped else []), np.uint32)
    beam = oracle.options(do_sample=False, repetition_penalty=1.0, num_beams=3)
    codes, stopped = orc.generate(zh, beam, 8)
    fx["generation.beam.codes"] = np.array(codes + ([8193] if stopped else []), np.uint32)
    it.write_mit2_bundle(OUT, fx, single_file=True, alignment=64, target="gpt_test")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes); greedy {list(fx['generation.greedy.codes'])}, "
          f"beam {list(fx['generation.beam.codes'])}")


if __name__ == "__main__":
    main()
