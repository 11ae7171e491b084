"""Pins the Qwen3 oracle (oracle/qwen_oracle.cpp, a restatement of src/qwen.cpp:5-49) on the CPU.

* Hugging Face transformers' Qwen3ForCausalLM, an independent implementation of the same
  architecture (RMSNorm eps 1e-6, per-head q/k RMSNorm, rotate-half RoPE with theta 1e6,
  16 query heads over 8 KV heads, SiLU-gated MLP, tied embedding head), run in float64 on the
  same weights (2 layers at the real widths): the oracle's prefill logits, teacher-forced step
  logits and cached K/V rows must agree with it.  Achieved: max-abs about 7e-6 on logits of
  magnitude about 3.
* Planted mistakes (orc_qwen_set_mutation: GQA head mapping, RoPE sign, skipped q/k norm, RoPE
  without the cache offset, SiLU on the wrong half) must each fail that comparison.
* Greedy generation is the argmax of the teacher-forced logits; EOS handling through a
  vocabulary relabelling (tied head: swapping two tokens' embedding rows swaps their logits);
  the reference's error kinds and messages.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

LAYERS = 2
LOGIT_ABS, LOGIT_RMSE = 1e-4, 2e-5  # against float64; the planted mistakes move logits by > 1


@pytest.fixture(scope="module")
def qw(itts):
    return itts.make_synthetic_qwen_weights(layers=LAYERS, seed=7)


@pytest.fixture(scope="module")
def hf(qw):
    cfg = transformers.Qwen3Config(vocab_size=151936, hidden_size=1024, intermediate_size=3072, num_hidden_layers=LAYERS,
                                   num_attention_heads=16, num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6,
                                   rope_theta=1e6, max_position_embeddings=4096, tie_word_embeddings=True,
                                   attention_bias=False)
    cfg._attn_implementation = "eager"
    m = transformers.Qwen3ForCausalLM(cfg).double().eval()
    sd = {k[len("qwen."):]: torch.from_numpy(v.astype(np.float64)) for k, v in qw.items()}
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert missing == ["lm_head.weight"] and not unexpected  # lm_head is the tied embedding
    return m


@pytest.fixture(scope="module")
def orc(oracle, qw):
    o = oracle.OracleQwen(qw, layers=LAYERS)
    yield o
    o.set_mutation(0)


def hf_forward(hf, ids):
    with torch.no_grad():
        out = hf(torch.tensor([list(ids)]), use_cache=True)
    return out.logits[0].numpy(), out.past_key_values


def hf_kv(cache, layer):
    """(keys, values) of one layer, [8 heads][rows][128], after q/k norm and RoPE."""
    if hasattr(cache, "layers"):
        return cache.layers[layer].keys[0].numpy(), cache.layers[layer].values[0].numpy()
    return cache.key_cache[layer][0].numpy(), cache.value_cache[layer][0].numpy()


def errors(a, b):
    d = np.abs(np.asarray(a, np.float64) - b)
    return float(d.max()), float(np.sqrt(np.mean(d * d)))


IDS = [int(x) for x in np.random.default_rng(3).integers(0, 151936, 24)]


def test_prefill_steps_and_cache_match_hf_float64(orc, hf):
    ref, cache = hf_forward(hf, IDS)
    o = orc
    e = errors(o.prefill(IDS[:20]), ref[19])
    assert o.cached == 20
    for j in range(20, 24):
        e2 = errors(o.step(IDS[j]), ref[j])
        e = (max(e[0], e2[0]), max(e[1], e2[1]))
    print(f"oracle vs float64 transformers: max-abs {e[0]:.3e}, rmse {e[1]:.3e}")
    assert e[0] < LOGIT_ABS and e[1] < LOGIT_RMSE
    assert o.cached == 24
    for layer in range(LAYERS):
        keys, values = hf_kv(cache, layer)
        for pos in (0, 19, 23):
            assert np.allclose(o.kv_row(layer, False, pos), keys[:, pos, :].reshape(-1), atol=2e-5)
            assert np.allclose(o.kv_row(layer, True, pos), values[:, pos, :].reshape(-1), atol=2e-5)


@pytest.mark.parametrize("mutation", [1, 2, 3, 4, 5])
def test_planted_mistakes_fail_the_comparison(orc, hf, mutation):
    ref, _ = hf_forward(hf, IDS[:22])
    orc.set_mutation(mutation)
    try:
        a = errors(orc.prefill(IDS[:20]), ref[19])
        b = errors(orc.step(IDS[20]), ref[20])
    finally:
        orc.set_mutation(0)
    assert max(a[0], b[0]) > 100 * LOGIT_ABS


def test_step_equals_prefill_of_the_longer_prompt(orc):
    o = orc
    o.prefill(IDS[:9])
    a = o.step(IDS[9])
    b = o.prefill(IDS[:10])
    assert np.allclose(a, b, atol=1e-6, rtol=0)


def test_greedy_generate_is_argmax_of_teacher_forced_logits(orc, hf):
    o = orc
    toks, eos = o.generate(IDS[:12], 6)
    assert not eos and len(toks) == 6 and o.cached == 12 + 5
    ref, _ = hf_forward(hf, IDS[:12] + toks)
    assert toks == [int(np.argmax(ref[11 + i])) for i in range(6)]


def relabel(w, a, b):
    """Swap tokens a and b: their embedding rows (the tied head's rows too)."""
    w = dict(w)
    e = w["qwen.model.embed_tokens.weight"].copy()
    e[[a, b]] = e[[b, a]]
    w["qwen.model.embed_tokens.weight"] = e
    return w


def test_generate_stops_at_eos(oracle, qw, orc):
    for start in range(0, 12):  # a prompt whose greedy ids are not one repeated id
        prompt = IDS[start:start + 12]
        toks, _ = orc.generate(prompt, 8)
        ks = [i for i in range(1, len(toks)) if toks[i] not in toks[:i]]
        if ks:
            break
    k, t = ks[0], toks[ks[0]]
    assert oracle.QWEN_EOS not in prompt + toks
    prompt = [oracle.QWEN_EOS if x == t else x for x in prompt]  # t and EOS swap names everywhere
    o = oracle.OracleQwen(relabel(qw, t, oracle.QWEN_EOS), layers=LAYERS)
    got, eos = o.generate(prompt, 8)
    assert eos and got == toks[:k] + [oracle.QWEN_EOS]
    assert o.cached == len(prompt) + k  # the EOS token is not run (qwen.cpp:48)


def test_errors(oracle, qw):
    o = oracle.OracleQwen({k: v for k, v in qw.items()}, layers=LAYERS)
    cases = [
        (lambda: o.step(5), -1, "Qwen cache capacity exceeded"),
        (lambda: o.prefill([]), -1, "Qwen prompt capacity is 3072 tokens"),
        (lambda: o.prefill([1] * 3073), -1, "Qwen prompt capacity is 3072 tokens"),
        (lambda: o.prefill([1, 151936]), -1, "Invalid Qwen token"),
        (lambda: o.generate([1], 0), -1, "Qwen generation capacity exceeded"),
        (lambda: o.generate([1], 1025), -1, "Qwen generation capacity exceeded"),
        (lambda: o.generate([1] * 3073, 1024), -1, "Qwen generation capacity exceeded"),  # checked first (qwen.cpp:47)
        (lambda: o.generate([], 5), -1, "Qwen prompt capacity is 3072 tokens"),
    ]
    for fn, status, msg in cases:
        with pytest.raises(oracle.OracleError) as e:
            fn()
        assert str(e.value) == msg and e.value.status == status, (msg, str(e.value))
    o.prefill([1, 2])
    with pytest.raises(oracle.OracleError, match="Invalid Qwen token"):
        o.step(151936)
    w = dict(qw)
    w["qwen.model.layers.1.mlp.up_proj.weight"] = w["qwen.model.layers.1.mlp.up_proj.weight"][:, :512]
    with pytest.raises(oracle.OracleError, match="Unsupported Qwen shape: qwen.model.layers.1.mlp.up_proj.weight"):
        oracle.OracleQwen(w, layers=LAYERS)
    w = dict(qw)
    del w["qwen.model.layers.0.self_attn.k_norm.weight"]
    with pytest.raises(oracle.OracleError, match="Missing tensor: qwen.model.layers.0.self_attn.k_norm.weight"):
        oracle.OracleQwen(w, layers=LAYERS)
