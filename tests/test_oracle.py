"""Pins the CPU oracle (CPU only).

Forward math is checked against an independent float64 numpy GPT-2 block on tiny
shapes and against KV-cache invariants; the sampler against the reference's own
gpt_sampling.cpp compiled from its sources (oracle/_ref) and the committed fixtures
it produced (tests/golden/sampling_golden.npz); SplitMix64 against published vectors.
"""
import math
from pathlib import Path

import numpy as np
import pytest

from conftest import same_bits

GOLDEN = Path(__file__).resolve().parent / "golden"

# ---------------------------------------------------------------------------- tiny model

W_T, F_T, L_T, MEL = 128, 256, 2, 8194


def tiny_weights(seed=3):
    rng = np.random.default_rng(seed)
    n = lambda *s, sd=0.05: (rng.standard_normal(s) * sd).astype(np.float32)
    w = {
        "gpt.spk_emb_proj.weight": n(W_T, 192),
        "gpt.spk_emb_proj.bias": n(W_T),
        "gpt.text_embedding.weight": n(50, W_T, sd=0.3),
        "gpt.text_pos_embedding.emb.weight": n(40, W_T, sd=0.3),
        "gpt.lang_embedding.weight": n(3, W_T, sd=0.3),
        "gpt.mel_embedding.weight": n(MEL, W_T, sd=0.3),
        "gpt.mel_pos_embedding.emb.weight": n(64, W_T, sd=0.3),
        "gpt.gpt.ln_f.weight": 1 + n(W_T, sd=0.1),
        "gpt.gpt.ln_f.bias": n(W_T, sd=0.1),
        "gpt.final_norm.weight": 1 + n(W_T, sd=0.1),
        "gpt.final_norm.bias": n(W_T, sd=0.1),
        "gpt.mel_head.weight": n(MEL, W_T, sd=0.2),
        "gpt.mel_head.bias": n(MEL),
    }
    for l in range(L_T):
        p = f"gpt.gpt.h.{l}"
        w[p + ".ln_1.weight"] = 1 + n(W_T, sd=0.1)
        w[p + ".ln_1.bias"] = n(W_T, sd=0.1)
        w[p + ".attn.c_attn.weight"] = n(W_T, 3 * W_T, sd=0.15)
        w[p + ".attn.c_attn.bias"] = n(3 * W_T)
        w[p + ".attn.c_proj.weight"] = n(W_T, W_T)
        w[p + ".attn.c_proj.bias"] = n(W_T)
        w[p + ".ln_2.weight"] = 1 + n(W_T, sd=0.1)
        w[p + ".ln_2.bias"] = n(W_T, sd=0.1)
        w[p + ".mlp.c_fc.weight"] = n(W_T, F_T, sd=0.1)
        w[p + ".mlp.c_fc.bias"] = n(F_T)
        w[p + ".mlp.c_proj.weight"] = n(F_T, W_T)
        w[p + ".mlp.c_proj.bias"] = n(W_T)
    return w


def np_gpt(w, rows):
    """Independent float64 GPT-2 pre-LN forward (HF GPT2Block with Conv1D weights)."""
    W = w["gpt.mel_embedding.weight"].shape[1]
    H = W // 64
    f = {k: v.astype(np.float64) for k, v in w.items()}

    def ln(x, g, b):
        mu = x.mean(-1, keepdims=True)
        var = ((x - mu) ** 2).mean(-1, keepdims=True)
        return (x - mu) / np.sqrt(var + 1e-5) * g + b

    def gelu(v):
        out = 0.5 * v * (1 + np.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
        return np.where(v > 10, v, np.where(v < -10, 0.0, out))

    h = rows.astype(np.float64)
    T = h.shape[0]
    ks, vs = [], []
    mask = np.tril(np.ones((T, T), bool))
    for l in range(L_T):
        p = f"gpt.gpt.h.{l}"
        qkv = ln(h, f[p + ".ln_1.weight"], f[p + ".ln_1.bias"]) @ f[p + ".attn.c_attn.weight"] + f[p + ".attn.c_attn.bias"]
        q, k, v = qkv[:, :W], qkv[:, W:2 * W], qkv[:, 2 * W:]
        ks.append(k)
        vs.append(v)
        att = np.zeros_like(q)
        for hh in range(H):
            sl = slice(hh * 64, hh * 64 + 64)
            s = q[:, sl] @ k[:, sl].T / 8.0
            s = np.where(mask, s, -np.inf)
            s = np.exp(s - s.max(-1, keepdims=True))
            att[:, sl] = (s / s.sum(-1, keepdims=True)) @ v[:, sl]
        h = h + att @ f[p + ".attn.c_proj.weight"] + f[p + ".attn.c_proj.bias"]
        ff = gelu(ln(h, f[p + ".ln_2.weight"], f[p + ".ln_2.bias"]) @ f[p + ".mlp.c_fc.weight"] + f[p + ".mlp.c_fc.bias"])
        h = h + ff @ f[p + ".mlp.c_proj.weight"] + f[p + ".mlp.c_proj.bias"]
    last = ln(ln(h[-1], f["gpt.gpt.ln_f.weight"], f["gpt.gpt.ln_f.bias"]), f["gpt.final_norm.weight"], f["gpt.final_norm.bias"])
    return f["gpt.mel_head.weight"] @ last + f["gpt.mel_head.bias"], ks, vs


@pytest.fixture(scope="module")
def tiny(oracle):
    w = tiny_weights()
    return w, oracle.OracleGpt(w, kv_capacity=128)


def test_forward_matches_float64_restatement(tiny):
    w, m = tiny
    rows = np.random.default_rng(5).standard_normal((9, W_T)).astype(np.float32)
    got = m.prefill(rows)
    ref, ks, vs = np_gpt(w, rows)
    assert np.max(np.abs(got - ref)) < 2e-4 * max(1.0, np.max(np.abs(ref)))
    for l in range(L_T):
        for t in (0, 8):
            assert np.allclose(m.kv_row(l, False, t), ks[l][t], atol=1e-4)
            assert np.allclose(m.kv_row(l, True, t), vs[l][t], atol=1e-4)


def test_mutation_is_caught_by_float64_restatement(tiny):
    """A dropped final_norm (a plausible slip) must fail the check above."""
    w, _ = tiny
    rows = np.random.default_rng(5).standard_normal((9, W_T)).astype(np.float32)
    ref, _, _ = np_gpt(w, rows)
    w2 = dict(w)
    w2["gpt.final_norm.weight"] = np.ones(W_T, np.float32)
    w2["gpt.final_norm.bias"] = np.zeros(W_T, np.float32)
    bad, _, _ = np_gpt(w2, rows)
    assert np.max(np.abs(bad - ref)) > 1e-2


def test_step_equals_prefill_of_extended_prefix(tiny, oracle):
    """KV invariant: prefill(P rows) + step(code, pos) == prefill(P+1 rows) whose last row is mel_emb[code]+mel_pos[pos]."""
    w, m = tiny
    rows = np.random.default_rng(6).standard_normal((7, W_T)).astype(np.float32)
    code, pos = 1234, 5
    extra = (w["gpt.mel_embedding.weight"][code] + w["gpt.mel_pos_embedding.emb.weight"][pos]).astype(np.float32)
    m.prefill(rows)
    a = m.step(code, pos)
    assert m.cached_tokens() == 8
    b = m.prefill(np.vstack([rows, extra[None]]))
    assert np.max(np.abs(a - b)) < 1e-5
    # Full recompute of a two-step chain.
    m.prefill(rows)
    m.step(code, pos)
    c = m.step(77, 6)
    extra2 = (w["gpt.mel_embedding.weight"][77] + w["gpt.mel_pos_embedding.emb.weight"][6]).astype(np.float32)
    d = m.prefill(np.vstack([rows, extra[None], extra2[None]]))
    assert np.max(np.abs(c - d)) < 1e-5


def test_prepare_identities(tiny, oracle):
    w, m = tiny
    cond = np.random.default_rng(7).standard_normal((4, W_T)).astype(np.float32)
    text = [5, 0, 9, 1, 12]
    p = m.prepare_cond(cond, text, 2).reshape(-1, W_T)
    ids = [0, 5, 9, 12, 1]  # 0/1 dropped, wrapped in 0 ... 1 (gpt.cpp:44-49)
    assert p.shape[0] == 4 + len(ids) + 1
    assert np.array_equal(p[:4], cond)
    for r, i in enumerate(ids):
        exp = (w["gpt.text_embedding.weight"][i] + w["gpt.text_pos_embedding.emb.weight"][r]) + w["gpt.lang_embedding.weight"][2]
        assert np.array_equal(p[4 + r], exp.astype(np.float32))
    start = w["gpt.mel_embedding.weight"][8192] + w["gpt.mel_pos_embedding.emb.weight"][0]
    assert np.array_equal(p[-1], start)
    sp = np.random.default_rng(8).standard_normal(192).astype(np.float32)
    em = np.random.default_rng(9).standard_normal(W_T).astype(np.float32)
    q = m.prepare(sp, em, text, 2).reshape(-1, W_T)
    row0 = w["gpt.spk_emb_proj.weight"].astype(np.float64) @ sp + w["gpt.spk_emb_proj.bias"] + em
    assert np.allclose(q[0], row0, atol=1e-5)
    assert not q[1:3].any()
    assert np.array_equal(q[3:], p[4:])


def test_prepare_errors(tiny, oracle):
    _, m = tiny
    with pytest.raises(oracle.OracleError, match="outside 2.5 vocabulary"):
        m.prepare_cond(np.zeros((1, W_T), np.float32), [50], 0)
    with pytest.raises(oracle.OracleError, match="position capacity"):
        m.prepare_cond(np.zeros((1, W_T), np.float32), list(range(2, 42)), 0)
    with pytest.raises(oracle.OracleError, match="conditioning"):
        m.prepare_cond(np.zeros((1, W_T), np.float32), [3], 3)


def test_step_errors(tiny, oracle):
    _, m = tiny
    m.prefill(np.zeros((3, W_T), np.float32))
    for code, pos in ((8194, 2), (5, 64)):
        with pytest.raises(oracle.OracleError, match="valid cache, code and position") as e:
            m.step(code, pos)
        assert e.value.status == -1


def test_greedy_generate_is_teacher_forced_argmax(tiny, oracle):
    w, m = tiny
    rows = np.random.default_rng(10).standard_normal((6, W_T)).astype(np.float32)
    opt = oracle.options(do_sample=False, repetition_penalty=1.0, suppress_stop=True)
    codes, stopped = m.generate(rows, opt, 12)
    assert len(codes) == 12 and not stopped
    lg = m.prefill(rows)
    for i, c in enumerate(codes):
        lg[8192:] = -np.inf
        assert c == int(np.argmax(lg))
        if i + 1 < len(codes):
            lg = m.step(c, i + 2)  # first generated code is at mel position 2 (gpt_sampling.cpp:184-186)


def test_generate_capacity_errors(tiny, oracle):
    _, m = tiny
    rows = np.zeros((6, W_T), np.float32)
    with pytest.raises(oracle.OracleError, match="capacity exceeded"):
        m.generate(rows, oracle.options(), 63)  # max+1 >= 64 mel positions
    with pytest.raises(oracle.OracleError, match="Invalid GPT generation parameters"):
        m.generate(rows, oracle.options(temperature=0.0), 4)
    with pytest.raises(oracle.OracleError, match="Invalid beam search configuration"):
        m.generate(rows, oracle.options(num_beams=11), 4)


# ---------------------------------------------------------------------------- elementwise pieces

def test_gelu_closed_forms(oracle):
    assert oracle.gelu(0.0) == 0.0
    assert oracle.gelu(10.5) == 10.5
    assert oracle.gelu(-10.5) == 0.0
    for v in np.linspace(-9.9, 9.9, 97):
        exact = 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
        assert abs(oracle.gelu(float(np.float32(v))) - exact) < 2e-6 * max(1, abs(exact))


def test_layernorm_matches_float64(oracle):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(1280) * 3 + 1).astype(np.float32)
    g = rng.standard_normal(1280).astype(np.float32)
    b = rng.standard_normal(1280).astype(np.float32)
    y = oracle.layernorm(x, g, b)
    x64 = x.astype(np.float64)
    ref = (x64 - x64.mean()) / np.sqrt(x64.var() + 1e-5) * g + b
    assert np.max(np.abs(y - ref)) < 1e-5


# ---------------------------------------------------------------------------- SplitMix64 / sampler

def test_splitmix64_published_vectors(oracle):
    # Vigna's splitmix64.c seeded with 1234567 (the reference test vectors of the generator).
    assert oracle.splitmix_sequence(1234567, 5) == [
        6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431, 16408922859458223821,
    ]


def test_splitmix_counter_form(oracle):
    """k-th output == mix(seed + (k+1) * gamma): the counter form the device uses."""
    gamma = 0x9E3779B97F4A7C15
    M = 2**64 - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        return z ^ (z >> 31)

    seq = oracle.splitmix_sequence(42, 8)
    assert seq == [mix((42 + (k + 1) * gamma) & M) for k in range(8)]


def _golden():
    path = GOLDEN / "sampling_golden.npz"
    if not path.exists():
        pytest.skip("sampling golden fixture not generated")
    return np.load(path, allow_pickle=False)


def test_oracle_processors_match_reference_golden(oracle):
    g = _golden()
    for case in [k[: -len(".config")] for k in g.files if k.endswith(".config")]:
        cfg = g[case + ".config"]
        opt = oracle.options(temperature=float(cfg[0]), top_k=int(cfg[1]), top_p=float(cfg[2]), repetition_penalty=float(cfg[3]),
                             num_beams=int(cfg[4]))
        out = oracle.processors(g[case + ".logits"], g[case + ".history"], opt)
        exp = g[case + ".values"]
        assert np.array_equal(np.isfinite(out), g[case + ".allowed"].astype(bool)), case
        assert same_bits(out, exp), case


def test_oracle_sampler_matches_reference_golden(oracle):
    g = _golden()
    for case in [k[: -len(".draw_seed")] for k in g.files if k.endswith(".draw_seed")]:
        seed = int(g[case + ".draw_seed"][0])
        toks, state = oracle.sample(g[case + ".values"], seed, len(g[case + ".draws"]))
        assert toks == [int(t) for t in g[case + ".draws"]], case
        assert state == int(g[case + ".draw_state"][0]), case


def _tie_logits(rng, n=8194):
    base = rng.standard_normal(n).astype(np.float32)
    return np.round(base * 4) / 4  # heavy ties


@pytest.mark.parametrize("seed", range(6))
def test_oracle_processors_match_reference_live(oracle, seed):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(100 + seed)
    ref = oracle.RefSampler()
    try:
        for logits in (rng.standard_normal(8194).astype(np.float32) * 3, _tie_logits(rng)):
            hist = [1, 8192] + list(rng.integers(0, 8194, 20))
            for (T, k, p, pen, beams) in [(0.8, 30, 0.8, 10.0, 1), (1.0, 0, 0.5, 1.0, 1), (0.7, 1, 0.9, 2.0, 3),
                                          (1.3, 500, 0.95, 1.0, 2), (1.0, 0, 1.0, 1.0, 1), (0.5, 30, 0.01, 10.0, 3)]:
                exp = ref.processors(logits, hist, T, k, p, pen, beams)
                got = oracle.processors(logits, hist, oracle.options(temperature=T, top_k=k, top_p=p, repetition_penalty=pen,
                                                                     num_beams=beams))
                assert same_bits(got, exp)
                s = int(rng.integers(0, 2**63))
                assert oracle.sample(got, s, 5) == ref.sample(got, s, 5)
    finally:
        ref.close()
