"""The reference's gpt_test (src/main.cpp:31-66) run against this decoder, with a fixture in
that test's own schema (tests/golden/gpt_test_fixture.mit2, a single-file MIT2 bundle written
by tests/golden/make_gpt_test_fixture.py from the CPU oracle).

gpt_test's sequence and bars: prepare for ZH, EN, JA, ES, AR against prefix.*.embeddings
(compare's default bar: max-abs < 1e-4, RMSE < 1e-5, main.cpp:19); prefill(ZH) and
step(decode.i.code, i) for i = 1..4 against the stored logits (max-abs < 1e-4, RMSE < 2e-5,
argmax equal, main.cpp:40-47); generate(ZH) greedy (do_sample false, repetition penalty 1) and
with 3 beams, 8 codes each, equal to generation.*.codes with a trailing stop code dropped
(main.cpp:52-61).  The CPU test checks the fixture's schema (every name, dtype and shape
gpt_test reads) and its prepare outputs against the oracle; the GPU test runs the sequence on
the HIP path through the bundle reader.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "tests" / "golden"))
FIXTURE = ROOT / "tests" / "golden" / "gpt_test_fixture.mit2"
LANGS = ("ZH", "EN", "JA", "ES", "AR")


def compare(name, actual, expected, tolerance=1e-4, rms_tolerance=1e-5):
    """main.cpp:19-29: same size, all finite, max-abs < tolerance and RMSE < rms_tolerance."""
    actual = np.asarray(actual, np.float32)
    expected = np.asarray(expected, np.float32)
    assert actual.size == expected.size, f"Output shape mismatch: {name}"
    assert np.all(np.isfinite(actual)) and np.all(np.isfinite(expected)), f"Non-finite output: {name}"
    d = np.abs(actual.astype(np.float64) - expected.astype(np.float64))
    peak, rmse = float(d.max()), float(np.sqrt(np.mean(d * d)))
    print(f'{{"case":"{name}","max_abs_error":{peak:.3e},"rmse":{rmse:.3e}}}', flush=True)
    return peak < tolerance and rmse < rms_tolerance


def _codes(fx, name):
    c = [int(x) for x in fx.ids(name)]
    if c and c[-1] == 8193:
        c.pop()
    return c


def test_fixture_schema_and_prepare_match_oracle(itts, oracle):
    """Every tensor gpt_test reads is present with its dtype and shape; the prefixes equal the
    oracle's prepare (a 2-layer model with the fixture model's embedding tables: prepare reads
    no layer)."""
    import make_gpt_test_fixture as mk

    fx = itts.Bundle(FIXTURE, require_model=False)
    info = {t["name"]: t for t in fx.tensors()}
    assert info["speaker"]["shape"] == (192,) and info["emotion"]["shape"] == (1280,)
    for lang in LANGS:
        assert info[f"prefix.{lang}.tokens"]["dtype"] == "u32"
        assert info[f"prefix.{lang}.language"]["shape"] == (1,)
        n = sum(1 for t in fx.ids(f"prefix.{lang}.tokens") if t not in (0, 1))
        assert info[f"prefix.{lang}.embeddings"]["shape"] == ((3 + n + 2 + 1) * 1280,)
    for name in ["decode.prefill"] + [f"decode.{i}" for i in range(1, 5)]:
        assert info[name + ".logits"]["shape"] == (8194,) and info[name + ".logits"]["dtype"] == "f32"
    for i in range(1, 5):
        assert info[f"decode.{i}.code"]["dtype"] == "u32"
    assert info["generation.greedy.codes"]["dtype"] == info["generation.beam.codes"]["dtype"] == "u32"
    w = itts.make_synthetic_weights(layers=2, seed=mk.MODEL_SEED, ln_random=True, text_vocab=mk.TEXT_VOCAB)
    orc = oracle.OracleGpt(w, kv_capacity=256)
    for lang in LANGS:
        got = orc.prepare(fx.get("speaker"), fx.get("emotion"), fx.ids(f"prefix.{lang}.tokens"),
                          int(fx.ids(f"prefix.{lang}.language")[0]))
        assert np.array_equal(got, fx.get(f"prefix.{lang}.embeddings")), lang
    fx.close()


@pytest.mark.gpu
def test_gpt_test_sequence_on_the_hip_path(itts):
    import make_gpt_test_fixture as mk

    fx = itts.Bundle(FIXTURE, require_model=False)
    print("gpt_test: building the 24-layer model at the real vocabularies", flush=True)
    # max_batch 10: the KV slots the C++ drop-in's reference-form constructor creates, so that
    # num_beams up to the reference's limit of 10 runs on any decoder
    gpt = itts.GptDecoder(mk.model(), kv_capacity=4096, max_batch=10)
    ok = True
    chinese = None
    for lang in LANGS:
        name = f"prefix.{lang}"
        prefix = gpt.prepare(fx.get("speaker"), fx.get("emotion"), fx.ids(name + ".tokens"), int(fx.ids(name + ".language")[0]))
        ok = compare(name, prefix, fx.get(name + ".embeddings")) and ok
        if lang == "ZH":
            chinese = prefix

    def check_logits(name, logits):
        ref = fx.get(name + ".logits")
        match = int(np.argmax(logits)) == int(np.argmax(ref))
        print(f'{{"case":"{name}.argmax","exact_match":{str(match).lower()}}}', flush=True)
        return compare(name, logits, ref, 1e-4, 2e-5) and match

    ok = check_logits("decode.prefill", gpt.prefill(chinese)) and ok
    for i in range(1, 5):
        name = f"decode.{i}"
        ok = check_logits(name, gpt.step(int(fx.ids(name + ".code")[0]), i)) and ok
    config = itts.GenerationOptions(do_sample=False, repetition_penalty=1.0)
    generated = gpt.generate(chinese, config, 8)
    greedy_match = generated.codes == _codes(fx, "generation.greedy.codes")
    print(f'{{"case":"generation.greedy","exact_match":{str(greedy_match).lower()}}}', flush=True)
    config.num_beams = 3
    beam = gpt.generate(chinese, config, 8)
    beam_match = beam.codes == _codes(fx, "generation.beam.codes")
    print(f'{{"case":"generation.beam","exact_match":{str(beam_match).lower()}}}', flush=True)
    print(f'{{"stage":"gpt_2.5","cached_tokens":{gpt.cached_tokens()},"pass":{str(ok and greedy_match and beam_match).lower()}}}')
    assert ok and greedy_match and beam_match
    gpt.close()
    fx.close()


@pytest.mark.gpu
def test_gpt_test_through_the_cpp_dropin(itts, tmp_path):
    """The same sequence written as gpt_test writes it, in C++ against the drop-in
    (index-tts-25-metal_amd/cpp/gpt_shim_example.cpp, mode gpt_test): the model as a MIT2
    directory bundle (target index-tts2.5) and the fixture through BundleWeights."""
    import json
    import subprocess

    import make_gpt_test_fixture as mk

    exe = ROOT / "index-tts-25-metal_amd" / "cpp" / "gpt_shim_example"
    assert exe.exists(), "shim example not built"
    print("gpt_test (C++): writing the model bundle", flush=True)
    model = itts.write_mit2_bundle(tmp_path / "model", mk.model())
    out = subprocess.run([str(exe), "gpt_test", str(model), str(FIXTURE)], capture_output=True, text=True, timeout=600)
    print(out.stdout, flush=True)
    lines = [json.loads(l) for l in out.stdout.splitlines() if l.startswith("{")]
    assert out.returncode == 0, out.stdout + out.stderr
    assert lines[-1]["stage"] == "gpt_2.5" and lines[-1]["pass"] is True
    assert sum(1 for l in lines if "max_abs_error" in l) == 10 and all(l.get("pass", True) for l in lines)
