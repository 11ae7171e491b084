"""The C++17 drop-in GptDecoder (index-tts-25-metal_amd/cpp) links against the C ABI and,
on the GPU, runs prepare -> generate through the reference's constructor form."""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

EXE = Path(__file__).resolve().parent.parent / "index-tts-25-metal_amd" / "cpp" / "gpt_shim_example"


def test_shim_links():
    if not EXE.exists():
        pytest.skip("shim example not built (run __graft_entry__.build())")
    out = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "gpt shim linked" in out.stdout


@pytest.mark.gpu
def test_shim_runs_on_gpu():
    assert EXE.exists(), "shim example not built"
    out = subprocess.run([str(EXE), "run"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    lines = [json.loads(l) for l in out.stdout.splitlines() if l.startswith("{")]
    assert lines[0]["rows"] == 3 + 6 + 1  # 3 conditioning rows + [0, 5, 17, 300, 42, 1] + mel start
    assert lines[0]["codes"] + lines[0]["stopped"] >= 1
    assert lines[1]["beam_codes"] + lines[1]["beam_stopped"] >= 1
    assert lines[2]["processed"] == 8194
    assert lines[3] == {"segments": 3, "segments_equal_loop": 1}
    c = lines[4]
    assert c["codec_values"] == 2 * c["codec_codes"] * 1024 and c["codec_codes"] >= 1
    assert c["codec_finite"] == 1 and c["codec_refuses_8192"] == 1


@pytest.mark.gpu
def test_shim_bundle_matches_python_decoder(itts, small_weights, tmp_path):
    """Weights(path) + GptDecoder(weights, ctx) on a MIT2 bundle of the 2-layer model gives
    the codes the Python decoder gives from the same arrays."""
    assert EXE.exists(), "shim example not built"
    bundle = itts.write_mit2_bundle(tmp_path / "gpt2l", small_weights)
    outs = []
    for mode in ("bundle", "refbundle"):  # BundleWeights, and a reference-style Weights (bundle().root())
        out = subprocess.run([str(EXE), mode, str(bundle)], capture_output=True, text=True, timeout=300)
        assert out.returncode == 0, out.stdout + out.stderr
        outs.append([json.loads(l) for l in out.stdout.splitlines() if l.startswith("{")][0])
    got = outs[0]
    assert outs[1] == got
    dec = itts.GptDecoder(small_weights, kv_capacity=4096)
    prefix = dec.prepare(np.full(192, 0.1, np.float32), np.full(1280, 0.05, np.float32), [5, 17, 300, 1, 0, 42], 3)
    opt = itts.GenerationOptions(do_sample=False, repetition_penalty=1.0)
    r = dec.generate(prefix, opt, 8)
    dec.close()
    assert got["rows"] == prefix.size // 1280
    assert got["codes"] == list(r.codes) and bool(got["stopped"]) == bool(r.stopped)
    assert got["spk_shape"] == [1280, 192]


@pytest.mark.gpu
def test_shim_qwen_matches_python_decoder(itts, tmp_path):
    """QwenDecoder(weights) through the C++ drop-in (prefill, three steps, generate, as
    src/main.cpp:160-166 drives it), with weights from BundleWeights, from a reference-style
    Weights (bundle().root()) and from a plain info()/get() table, against the Python decoder on
    the same 28-layer synthetic weights.  EOS is made reachable by swapping a generated token's
    embedding row with EOS's (the head is tied, so the model only relabels the two tokens)."""
    assert EXE.exists(), "shim example not built"
    w = itts.make_synthetic_qwen_weights(seed=5)
    dec = itts.QwenDecoder(w)
    for seed in range(9, 40):  # a prompt whose greedy ids are not one repeated id
        prompt = [int(x) for x in np.random.default_rng(seed).integers(0, 151936, 17)]
        toks, _ = dec.generate_tokens(prompt, 12)
        ks = [i for i in range(1, len(toks)) if toks[i] not in toks[:i]]
        if ks:
            break
    dec.close()
    k, t = ks[0], toks[ks[0]]
    assert itts.QWEN_EOS not in prompt + toks
    # swap t and EOS everywhere: embedding rows (the tied head's too) and the prompt
    prompt = [itts.QWEN_EOS if x == t else x for x in prompt]
    e = w["qwen.model.embed_tokens.weight"].copy()
    e[[t, itts.QWEN_EOS]] = e[[itts.QWEN_EOS, t]]
    w["qwen.model.embed_tokens.weight"] = e
    bundle = itts.write_mit2_bundle(tmp_path / "qwen", w)
    dec = itts.QwenDecoder(w)
    logits = dec.prefill(prompt)
    steps = [int(np.argmax(dec.step(prompt[i % len(prompt)]))) for i in (1, 2, 3)]
    gen = dec.generate(prompt, 12)
    dec.close()
    del w, e
    assert gen == toks[:k] + [itts.QWEN_EOS]
    for mode in ("qwen", "qwenref", "qwentable"):
        out = subprocess.run([str(EXE), mode, str(bundle), *map(str, prompt)], capture_output=True, text=True, timeout=300)
        assert out.returncode == 0, out.stdout + out.stderr
        got = [json.loads(l) for l in out.stdout.splitlines() if l.startswith("{")][0]
        assert got["prefill_argmax"] == int(np.argmax(logits)), mode
        assert got["prefill_sum"] == pytest.approx(float(np.sum(logits, dtype=np.float64)), rel=1e-9, abs=1e-6), mode
        assert got["steps"] == steps and got["generated"] == gen, mode
        assert got["short_error"] == "Qwen did not reach EOS within 1024 generated tokens", mode
        assert got["submissions"] == 1 + 3 + len(gen) + (len(gen) - 1), mode
