"""The Qwen3-0.6B emotion-text decoder on the device (itts25::QwenDecoder, src/qwen.cpp) against
the CPU oracle (oracle/qwen_oracle.cpp, pinned by tests/test_qwen_oracle.py).

Bars: the reference's own qwen_test bar (src/main.cpp:159-169: logits max-abs < 5e-4 and
RMSE < 1e-4, argmax equal; generated ids exact) and the path's logit bar (max-abs 1e-3,
L2-relative 1e-4), at every compared prefill and step; the achieved worst case is printed.
Cases: 2 layers at the real widths (prompts past several 64-row attention splits, steps across
split boundaries, greedy generation, EOS through a vocabulary relabelling, errors, graph replay
against eager launches, MIT2 bundles), and the full 28-layer model the way qwen_test runs it
(prefill, 3 steps, greedy generation).
"""
import os

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

REF_ABS, REF_RMSE = 5e-4, 1e-4   # src/main.cpp:162 (compare(test, actual, expected, 5e-4, 1e-4))
PATH_ABS, PATH_REL = 1e-3, 1e-4
LAYERS = 2


class Worst:
    def __init__(self, what):
        self.what, self.abs, self.rmse, self.rel = what, 0.0, 0.0, 0.0

    def check(self, got, exp, where):
        d = np.abs(got.astype(np.float64) - exp)
        a, r, rel = float(d.max()), float(np.sqrt(np.mean(d * d))), rel_err(got, exp)
        self.abs, self.rmse, self.rel = max(self.abs, a), max(self.rmse, r), max(self.rel, rel)
        assert np.all(np.isfinite(got)), where
        assert a < REF_ABS and r < REF_RMSE, f"{self.what} {where}: max-abs {a:.3e} rmse {r:.3e}"
        assert a <= PATH_ABS and rel <= PATH_REL, f"{self.what} {where}: max-abs {a:.3e} rel {rel:.3e}"
        assert int(np.argmax(got)) == int(np.argmax(exp)), f"{self.what} {where}: argmax"

    def report(self):
        print(f"{self.what}: worst max-abs {self.abs:.3e}, rmse {self.rmse:.3e}, rel {self.rel:.3e}", flush=True)


@pytest.fixture(scope="module")
def qw(itts):
    return itts.make_synthetic_qwen_weights(layers=LAYERS, seed=7)


@pytest.fixture(scope="module")
def pair(itts, oracle, qw):
    dec = itts.QwenDecoder(qw, layers=LAYERS)
    orc = oracle.OracleQwen(qw, layers=LAYERS)
    yield dec, orc
    dec.close()


def ids_of(seed, n):
    return [int(x) for x in np.random.default_rng(seed).integers(0, 151936, n)]


@pytest.mark.parametrize("n_prompt", [1, 20, 63, 64, 65, 200])
def test_prefill_and_steps_match_oracle(pair, n_prompt):
    dec, orc = pair
    print(f"qwen prefill {n_prompt} + 5 steps", flush=True)
    w = Worst(f"qwen 2-layer, {n_prompt}-id prompt")
    p = ids_of(n_prompt, n_prompt + 5)
    w.check(dec.prefill(p[:n_prompt]), orc.prefill(p[:n_prompt]), "prefill")
    for i in range(5):
        w.check(dec.step(p[n_prompt + i]), orc.step(p[n_prompt + i]), f"step {i}")
    w.report()


def test_long_prompt_and_steps_across_splits(pair):
    """A 500-id prompt (8 attention splits) and 70 steps: the cache crosses row 512 and 576."""
    dec, orc = pair
    w = Worst("qwen 2-layer, 500-id prompt + 70 steps")
    p = ids_of(3, 570)
    w.check(dec.prefill(p[:500]), orc.prefill(p[:500]), "prefill")
    for i in range(500, 570):
        w.check(dec.step(p[i]), orc.step(p[i]), f"step at row {i}")
    w.report()


def test_steps_past_1024_rows(pair):
    """A 1010-id prompt (16 attention splits) and 30 steps: the cache crosses row 1024, and the
    split merge runs over 16 and then 17 splits."""
    dec, orc = pair
    w = Worst("qwen 2-layer, 1010-id prompt + 30 steps")
    p = ids_of(5, 1040)
    w.check(dec.prefill(p[:1010]), orc.prefill(p[:1010]), "prefill")
    for i in range(1010, 1040):
        w.check(dec.step(p[i]), orc.step(p[i]), f"step at row {i}")
    w.report()


def test_steps_past_2048_rows(itts, oracle):
    """One layer, a 2040-id prompt (32 attention splits) and 20 steps: the cache crosses row
    2048, where the split merge takes its widest form (33 and more splits; the reference's
    limits reach 3072 prompt ids + 1024 generated).  One layer keeps the oracle's prefill to
    seconds."""
    qw1 = itts.make_synthetic_qwen_weights(layers=1, seed=8)
    dec = itts.QwenDecoder(qw1, layers=1)
    orc = oracle.OracleQwen(qw1, layers=1)
    w = Worst("qwen 1-layer, 2040-id prompt + 20 steps")
    p = ids_of(6, 2060)
    print("qwen prefill 2040 ids (1 layer)", flush=True)
    w.check(dec.prefill(p[:2040]), orc.prefill(p[:2040]), "prefill")
    for i in range(2040, 2060):
        w.check(dec.step(p[i]), orc.step(p[i]), f"step at row {i}")
    w.report()
    dec.close()


def test_greedy_generate_matches_oracle(pair):
    dec, orc = pair
    for n, maximum in ((12, 40), (130, 16), (5, 1)):
        p = ids_of(n + 100, n)
        print(f"qwen generate: prompt {n}, maximum {maximum}", flush=True)
        before = dec.submissions()
        got = dec.generate_tokens(p, maximum)
        assert got == orc.generate(p, maximum)
        assert len(got[0]) == maximum and not got[1]
        assert dec.submissions() - before == maximum  # one prefill + maximum - 1 steps
        # the cache continues after generate (qwen.cpp:48): a step matches the oracle's
        w = Worst("qwen step after generate")
        w.check(dec.step(7), orc.step(7), "step")


def relabel(w, a, b):
    w = dict(w)
    e = w["qwen.model.embed_tokens.weight"].copy()
    e[[a, b]] = e[[b, a]]
    w["qwen.model.embed_tokens.weight"] = e
    return w


def test_generate_stops_at_eos(itts, oracle, qw, pair):
    dec, orc = pair
    for seed in range(11, 40):  # a prompt whose greedy ids are not one repeated id
        prompt = ids_of(seed, 12)
        toks, _ = orc.generate(prompt, 12)
        ks = [i for i in range(1, len(toks)) if toks[i] not in toks[:i]]
        if ks:
            break
    k, t = ks[0], toks[ks[0]]
    assert itts.QWEN_EOS not in prompt + toks
    prompt = [itts.QWEN_EOS if x == t else x for x in prompt]  # t and EOS swap names everywhere
    w2 = relabel(qw, t, itts.QWEN_EOS)
    d2 = itts.QwenDecoder(w2, layers=LAYERS)
    assert d2.generate(prompt, 12) == toks[:k] + [itts.QWEN_EOS]
    assert d2.generate_tokens(prompt, k + 1) == (toks[:k] + [itts.QWEN_EOS], True)
    with pytest.raises(itts.GptRuntimeError, match="Qwen did not reach EOS within 1024 generated tokens"):
        d2.generate(prompt, k)  # maximum reached one id before EOS
    d2.close()


def test_errors(itts, qw):
    d = itts.QwenDecoder(qw, layers=LAYERS)
    cases = [
        (lambda: d.step(5), itts.InvalidArgument, "Qwen cache capacity exceeded"),
        (lambda: d.prefill([]), itts.InvalidArgument, "Qwen prompt capacity is 3072 tokens"),
        (lambda: d.prefill([1] * 3073), itts.InvalidArgument, "Qwen prompt capacity is 3072 tokens"),
        (lambda: d.prefill([1, 151936]), itts.InvalidArgument, "Invalid Qwen token"),
        (lambda: d.generate([1], 0), itts.InvalidArgument, "Qwen generation capacity exceeded"),
        (lambda: d.generate([1], 1025), itts.InvalidArgument, "Qwen generation capacity exceeded"),
        (lambda: d.generate([1] * 3073, 1024), itts.InvalidArgument, "Qwen generation capacity exceeded"),
        (lambda: d.generate([], 5), itts.InvalidArgument, "Qwen prompt capacity is 3072 tokens"),
        (lambda: d.generate([3, 151936], 5), itts.InvalidArgument, "Invalid Qwen token"),
    ]
    for fn, kind, msg in cases:
        with pytest.raises(kind) as e:
            fn()
        assert str(e.value) == msg
    d.prefill([1, 2])
    with pytest.raises(itts.InvalidArgument, match="^Invalid Qwen token$"):
        d.step(151936)
    d.close()
    w = dict(qw)
    w["qwen.model.layers.1.mlp.up_proj.weight"] = w["qwen.model.layers.1.mlp.up_proj.weight"][:, :512]
    with pytest.raises(itts.InvalidArgument, match="^Unsupported Qwen shape: qwen.model.layers.1.mlp.up_proj.weight$"):
        itts.QwenDecoder(w, layers=LAYERS)
    w = dict(qw)
    del w["qwen.model.layers.0.self_attn.k_norm.weight"]
    with pytest.raises(itts.GptRuntimeError, match="^Missing tensor: qwen.model.layers.0.self_attn.k_norm.weight$"):
        itts.QwenDecoder(w, layers=LAYERS)


def test_graph_replay_equals_eager(itts, qw, pair):
    dec, _ = pair
    os.environ["ITTS_QWEN_GRAPHS"] = "0"
    try:
        eager = itts.QwenDecoder(qw, layers=LAYERS)
    finally:
        del os.environ["ITTS_QWEN_GRAPHS"]
    p = ids_of(21, 40)
    assert np.array_equal(dec.prefill(p[:30]), eager.prefill(p[:30]))
    for t in p[30:]:
        assert np.array_equal(dec.step(t), eager.step(t))
    assert dec.generate_tokens(p[:9], 20) == eager.generate_tokens(p[:9], 20)
    eager.close()


def test_decoder_from_bundle_bitwise_equals_arrays(itts, qw, pair, tmp_path):
    dec, _ = pair
    path = itts.write_mit2_bundle(tmp_path / "qwen.mit2", qw, single_file=True)
    b = itts.Bundle(path, require_model=False)
    d = itts.QwenDecoder.from_bundle(b, layers=LAYERS)
    b.close()
    p = ids_of(31, 24)
    assert np.array_equal(dec.prefill(p[:20]), d.prefill(p[:20]))
    assert np.array_equal(dec.step(p[20]), d.step(p[20]))
    d.close()


def test_full_28_layers_like_qwen_test(itts, oracle):
    """The reference's qwen_test sequence (main.cpp:159-169) on the 28-layer model with synthetic
    weights: prefill, three steps, then greedy generation (32 ids; random weights reach no EOS,
    so both sides stop at the maximum)."""
    w = itts.make_synthetic_qwen_weights(layers=28, seed=3)
    dec = itts.QwenDecoder(w)
    orc = oracle.OracleQwen(w, layers=28)
    del w
    worst = Worst("qwen 28-layer")
    for label, seed in (("happy", 1), ("sad", 2)):
        p = ids_of(seed, 43)
        print(f"qwen 28 layers: {label}", flush=True)
        worst.check(dec.prefill(p[:40]), orc.prefill(p[:40]), f"{label}.prefill")
        for i in range(3):
            worst.check(dec.step(p[40 + i]), orc.step(p[40 + i]), f"{label}.step.{i + 1}")
        got = dec.generate_tokens(p[:40], 32)
        assert got == orc.generate(p[:40], 32), label
    worst.report()
    dec.close()
