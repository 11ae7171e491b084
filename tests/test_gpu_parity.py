"""HIP path vs the CPU oracle and the reference-sampler fixtures (MI355X).

Tolerances (north star): teacher-forced logits max-abs <= 1e-3 and relative (L2) <= 1e-4;
greedy codes exact; processors (mask and values) and sampled tokens bit-exact given the
same logits and RNG state.
"""
import numpy as np
import pytest

from conftest import rel_err, same_bits

pytestmark = pytest.mark.gpu

GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden" / "sampling_golden.npz"
LOGIT_ABS = 1e-3
LOGIT_REL = 1e-4


def assert_logits_close(got, ref, what=""):
    err = float(np.max(np.abs(got - ref)))
    rel = rel_err(got, ref)
    assert err <= LOGIT_ABS and rel <= LOGIT_REL, f"{what}: max-abs {err:.3e} rel {rel:.3e}"
    assert int(np.argmax(got)) == int(np.argmax(ref)), what


# ---------------------------------------------------------------------------- sampler

def _opts(itts, cfg):
    return itts.GenerationOptions(temperature=float(cfg[0]), top_k=int(cfg[1]), top_p=float(cfg[2]),
                                  repetition_penalty=float(cfg[3]), num_beams=int(cfg[4]))


def test_processors_match_reference_golden(itts):
    g = np.load(GOLDEN, allow_pickle=False)
    cases = [k[: -len(".config")] for k in g.files if k.endswith(".config")]
    assert cases
    for case in cases:
        out = itts.apply_gpt_sampling_processors(g[case + ".logits"], g[case + ".history"], _opts(itts, g[case + ".config"]))
        assert np.array_equal(np.isfinite(out), g[case + ".allowed"].astype(bool)), case
        assert same_bits(out, g[case + ".values"]), case


def test_sampler_draws_match_reference_golden(itts):
    g = np.load(GOLDEN, allow_pickle=False)
    for case in [k[: -len(".draw_seed")] for k in g.files if k.endswith(".draw_seed")]:
        toks, state = itts.sample_gpt_token(g[case + ".values"], int(g[case + ".draw_seed"][0]), len(g[case + ".draws"]))
        assert toks == [int(t) for t in g[case + ".draws"]], case
        assert state == int(g[case + ".draw_state"][0]), case


@pytest.mark.parametrize("seed", range(4))
def test_processors_and_draws_match_oracle_random(itts, oracle, seed):
    rng = np.random.default_rng(seed)
    configs = [(0.8, 30, 0.8, 10.0, 1), (1.0, 0, 0.5, 1.0, 1), (0.7, 1, 0.9, 2.0, 3), (1.3, 700, 0.95, 1.0, 2),
               (1.0, 0, 1.0, 1.0, 1), (0.5, 30, 0.01, 10.0, 3), (1.0, 8193, 0.3, 1.5, 1), (0.9, 1500, 1.0, 3.0, 1)]
    for logits in ((rng.standard_normal(8194) * 3).astype(np.float32),
                   (np.round(rng.standard_normal(8194) * 3) / 3).astype(np.float32)):
        hist = [1, 8192] + [int(x) for x in rng.integers(0, 8194, 30)]
        for T, k, p, pen, beams in configs:
            o = itts.GenerationOptions(temperature=T, top_k=k, top_p=p, repetition_penalty=pen, num_beams=beams)
            got = itts.apply_gpt_sampling_processors(logits, hist, o)
            exp = oracle.processors(logits, hist, oracle.options_from(o))
            assert same_bits(got, exp), (T, k, p, pen, beams)
            s = int(rng.integers(0, 2**63))
            assert itts.sample_gpt_token(got, s, 8) == oracle.sample(got, s, 8)


def test_processor_errors(itts):
    lg = np.zeros(8194, np.float32)
    with pytest.raises(itts.GptRuntimeError, match="temperature must be positive"):
        itts.apply_gpt_sampling_processors(lg, [], itts.GenerationOptions(temperature=0.0))
    with pytest.raises(itts.GptRuntimeError, match="repetition penalty must be positive"):
        itts.apply_gpt_sampling_processors(lg, [], itts.GenerationOptions(repetition_penalty=-1.0))
    with pytest.raises(itts.GptRuntimeError, match="received no finite logits"):
        itts.sample_gpt_token(np.full(8194, -np.inf, np.float32), 1)


# ---------------------------------------------------------------------------- small model (2 layers, real widths)

@pytest.fixture(scope="module")
def small(itts, oracle, small_weights):
    dec = itts.GptDecoder(small_weights, kv_capacity=1024, max_batch=4)
    orc = oracle.OracleGpt(small_weights, kv_capacity=1024)
    cond, text = itts.synthetic_prefix_inputs(40, seed=1)
    return dec, orc, cond, text


def test_prepare_matches_oracle(small, itts):
    dec, orc, cond, text = small
    a = dec.prepare_cond(cond, text, 5)
    b = orc.prepare_cond(cond, text, 5)
    assert np.array_equal(a, b)
    sp = itts.synthetic_normal(192, 3)
    em = itts.synthetic_normal(1280, 4)
    pa = dec.prepare(sp, em, text, 5)
    pb = orc.prepare(sp, em, text, 5)
    assert pa.shape == pb.shape
    assert np.max(np.abs(pa - pb)) < 1e-5


def test_prefill_and_steps_small(small):
    dec, orc, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    assert_logits_close(dec.prefill(prefix), orc.prefill(prefix), "prefill")
    assert dec.cached_tokens() == orc.cached_tokens() == prefix.size // 1280
    for i, code in enumerate([17, 4000, 8191, 2]):
        assert_logits_close(dec.step(code, i + 2), orc.step(code, i + 2), f"step {i}")
    assert dec.cached_tokens() == orc.cached_tokens()


@pytest.mark.parametrize("n_text", [1, 13, 29, 61, 93, 125, 157, 253, 480])
def test_prefill_row_counts_match_oracle(small, itts, n_text):
    """Prefill logits and the next step against the oracle for prefixes of 36..515 rows: the
    prefill GEMM picks its row blocking (16..192 rows per block) and K split from the row
    count, the last row block holds clamped rows past the prefix, and the causal attention
    walks one to nine 64-key chunks.  The step after it reads the K/V rows the prefill wrote."""
    dec, orc, cond, _ = small
    _, text = itts.synthetic_prefix_inputs(n_text, seed=100 + n_text)
    prefix = dec.prepare_cond(cond, text, 0)
    rows = prefix.size // 1280
    print(f"prefill rows {rows}", flush=True)
    assert_logits_close(dec.prefill(prefix), orc.prefill(prefix), f"prefill {rows} rows")
    assert_logits_close(dec.step(17, 2), orc.step(17, 2), f"step after {rows} rows")


def test_step_errors(small, itts):
    dec, orc, cond, text = small
    dec.prefill(dec.prepare_cond(cond, text, 0))
    with pytest.raises(itts.InvalidArgument, match="valid cache, code and position"):
        dec.step(8194, 2)
    with pytest.raises(itts.InvalidArgument, match="valid cache, code and position"):
        dec.step(3, 1815)
    with pytest.raises(itts.InvalidArgument, match="Invalid GPT prefill dimensions"):
        dec.prefill(np.zeros(1280 * 1025, np.float32))


def test_checkpoint_restore(small):
    """checkpoint / restore (gpt.cpp:86-87) on the device and in the oracle: after a restore, steps
    continue from the snapshot's cache (logits against the oracle's restore + step, and bitwise
    against the device's own steps before the restore)."""
    dec, orc, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    dec.prefill(prefix)
    orc.prefill(prefix)
    for i, c in enumerate([10, 20]):
        dec.step(c, i + 2)
        orc.step(c, i + 2)
    st, so = dec.checkpoint(), orc.checkpoint()
    assert st.tokens == dec.cached_tokens() == orc.cached_tokens()
    a = dec.step(11, 4)
    assert_logits_close(a, orc.step(11, 4), "before restore")
    for i, c in enumerate([12, 13, 14]):
        dec.step(c, i + 5)
        orc.step(c, i + 5)
    dec.restore(st)
    orc.restore(so)
    assert dec.cached_tokens() == orc.cached_tokens() == st.tokens
    b = dec.step(11, 4)
    assert np.array_equal(a, b)
    assert_logits_close(b, orc.step(11, 4), "after restore")
    for i, c in enumerate([900, 8000]):
        assert_logits_close(dec.step(c, i + 5), orc.step(c, i + 5), f"after restore, step {i}")
    # a snapshot outlives later snapshots and can be restored again
    dec.checkpoint()
    dec.restore(st)
    orc.restore(so)
    assert_logits_close(dec.step(7, 4), orc.step(7, 4), "second restore")


def test_step_is_deterministic(small):
    dec, _, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    runs = []
    for _ in range(2):
        dec.prefill(prefix)
        runs.append(dec.step(99, 2))
    assert np.array_equal(runs[0], runs[1])


def test_greedy_generate_small(small, itts, oracle):
    dec, orc, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    o = itts.GenerationOptions(do_sample=False, repetition_penalty=1.0)
    r = dec.generate(prefix, o, 48)
    codes, stopped = orc.generate(prefix, oracle.options_from(o), 48)
    assert r.codes == codes and r.stopped == stopped
    assert dec.cached_tokens() == orc.cached_tokens()


def test_sampled_generate_small(small, itts, oracle):
    dec, orc, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    o = itts.GenerationOptions(do_sample=True, seed=42, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0)
    r = dec.generate(prefix, o, 64)
    codes, stopped = orc.generate(prefix, oracle.options_from(o), 64)
    assert r.codes == codes and r.stopped == stopped


@pytest.mark.parametrize("opts", [
    # no processor at all: plain softmax draws
    dict(do_sample=True, seed=1, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0),
    # top-k of one: every draw has a single survivor
    dict(do_sample=True, seed=2, temperature=0.3, top_k=1, top_p=1.0, repetition_penalty=1.0),
    # top-k at and past the vocabulary (gpt_sampling.cpp:58: no filter), top-p 0.5, mild penalty
    dict(do_sample=True, seed=3, temperature=1.5, top_k=8194, top_p=0.5, repetition_penalty=2.0),
    dict(do_sample=True, seed=4, temperature=1.0, top_k=10000, top_p=0.9, repetition_penalty=1.0),
    # a tiny top-p (only the best survives) under the headline's other processors
    dict(do_sample=True, seed=5, temperature=0.8, top_k=30, top_p=0.01, repetition_penalty=10.0),
    # a penalty below one favours the codes in the history, the start code 8192 included
    # (history {1, 8192}, gpt_sampling.cpp:174), so a draw of 8192 ends the call with the
    # reference's "GPT generated invalid semantic code" (:180)
    dict(do_sample=True, seed=6, temperature=1.0, top_k=5, top_p=0.99, repetition_penalty=0.7),
    # greedy after the processors
    dict(do_sample=False, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=3.0),
    # a seed above 2^63 and a high temperature
    dict(do_sample=True, seed=2**63 + 5, temperature=2.0, top_k=100, top_p=0.95, repetition_penalty=1.2),
    dict(do_sample=True, seed=0, temperature=0.05, top_k=50, top_p=0.8, repetition_penalty=10.0, suppress_stop=True),
])
def test_generate_option_sweep_matches_oracle(small, itts, oracle, opts):
    """generate() on the device (processors, draw and SplitMix64 state, the history that the
    repetition penalty reads, the stop rule, the invalid-code error) equals the oracle's
    gpt_sampling.cpp:168-189 loop over option edge cases, at 2 layers: the same codes and stop
    flag, or the same error message."""
    dec, orc, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    o = itts.GenerationOptions(**opts)
    print(f"option sweep {opts}", flush=True)
    try:
        r = dec.generate(prefix, o, 48)
        got = ("codes", r.codes, r.stopped)
    except itts.GptRuntimeError as e:
        got = ("error", str(e))
    try:
        codes, stopped = orc.generate(prefix, oracle.options_from(o), 48)
        want = ("codes", codes, stopped)
    except oracle.OracleError as e:
        want = ("error", str(e))
    assert got == want
    if got[0] == "codes":
        assert dec.cached_tokens() == orc.cached_tokens()


def test_batch_generate_matches_single_and_oracle(small, itts, oracle):
    dec, orc, cond, _ = small
    rng = np.random.default_rng(7)
    prefixes, opts = [], []
    for b in range(3):
        t = rng.integers(0, 12000, int(rng.integers(24, 60))).astype(np.uint32)
        prefixes.append(dec.prepare_cond(cond, t, 0))
        opts.append(itts.GenerationOptions(seed=100 + b, suppress_stop=True))
    batch = dec.generate_batch(prefixes, opts, 40)
    for b in range(3):
        single = dec.generate(prefixes[b], opts[b], 40)
        assert batch[b].codes == single.codes and batch[b].stopped == single.stopped
        codes, stopped = orc.generate(prefixes[b], oracle.options_from(opts[b]), 40)
        assert batch[b].codes == codes


@pytest.mark.parametrize("maximum", [1, 2, 3])
def test_generate_shortest_runs_match_oracle(small, itts, oracle, maximum):
    """generate() for 1-3 codes (gpt_sampling.cpp:176-185: no step after the last code), single
    and batched, greedy and sampled, against the oracle; the cache then holds the prefix and
    maximum - 1 steps."""
    dec, orc, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    opts = [itts.GenerationOptions(do_sample=False, repetition_penalty=1.0, suppress_stop=True),
            itts.GenerationOptions(seed=31, suppress_stop=True)]
    for o in opts:
        r = dec.generate(prefix, o, maximum)
        codes, stopped = orc.generate(prefix, oracle.options_from(o), maximum)
        assert (r.codes, r.stopped) == (codes, stopped) and len(codes) == maximum
        assert dec.cached_tokens() == orc.cached_tokens() == prefix.size // 1280 + maximum - 1
    batch = dec.generate_batch([prefix, prefix], opts, maximum)
    for b, o in enumerate(opts):
        codes, _ = orc.generate(prefix, oracle.options_from(o), maximum)
        assert batch[b].codes == codes, b


def test_bf16_batch_equals_single(small_weights, itts):
    """BF16-stored weights: a batch of ragged sequences gives each sequence the codes of its own
    batch-1 generate(), bit for bit (the batched GEMVs keep batch 1's per-row FMA order and
    reduction pairings)."""
    d16 = itts.GptDecoder(small_weights, kv_capacity=1024, max_batch=4, weight_dtype="bf16")
    cond, _ = itts.synthetic_prefix_inputs(30, seed=3)
    rng = np.random.default_rng(17)
    prefixes = [d16.prepare_cond(cond, rng.integers(0, 12000, int(rng.integers(5, 90))).astype(np.uint32), 0)
                for _ in range(4)]
    opts = [itts.GenerationOptions(seed=40 + b, suppress_stop=True) for b in range(4)]
    batch = d16.generate_batch(prefixes, opts, 32)
    for b in range(4):
        single = d16.generate(prefixes[b], opts[b], 32)
        assert (batch[b].codes, batch[b].stopped) == (single.codes, single.stopped), b
    d16.close()


def test_batch_generate_mixed_options_match_oracle(small, itts, oracle):
    """One batch whose sequences each carry different sampling options (greedy after the
    processors, top-k 1, no processor at all, the stop code allowed) and ragged prefixes: each
    sequence's codes and stop flag equal the oracle's single-sequence loop
    (gpt_sampling.cpp:168-189) with its own options."""
    dec, orc, cond, _ = small
    rng = np.random.default_rng(11)
    opts = [itts.GenerationOptions(do_sample=False, top_k=30, top_p=0.8, repetition_penalty=3.0),
            itts.GenerationOptions(seed=21, temperature=0.3, top_k=1, top_p=1.0, repetition_penalty=1.0),
            itts.GenerationOptions(seed=22, temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0),
            itts.GenerationOptions(seed=23, temperature=1.2, top_k=200, top_p=0.95, repetition_penalty=1.5)]
    prefixes = []
    for b in range(len(opts)):
        t = rng.integers(0, 12000, int(rng.integers(5, 120))).astype(np.uint32)
        prefixes.append(dec.prepare_cond(cond, t, 0))
    print("mixed-option batch, prefix rows", [p.size // 1280 for p in prefixes], flush=True)
    batch = dec.generate_batch(prefixes, opts, 40)
    for b in range(len(opts)):
        codes, stopped = orc.generate(prefixes[b], oracle.options_from(opts[b]), 40)
        assert (batch[b].codes, batch[b].stopped) == (codes, stopped), b


def _segment_case(itts, n, seed):
    rng = np.random.default_rng(seed)
    segments = [[int(x) for x in rng.integers(0, 12000, int(rng.integers(1, 40)))] for _ in range(n)]
    segments[min(2, n - 1)] = [0, 1, 5]  # prepare drops ids 0 and 1
    return segments


@pytest.mark.parametrize("opts", [
    dict(seed=77),
    dict(do_sample=False, repetition_penalty=1.0),
    dict(seed=5, num_beams=3),
])
def test_generate_segments_equal_loop_and_oracle(small_weights, itts, oracle, opts):
    """NativeRuntime::synthesize's segment loop (native_runtime.cpp:98-99): segment i's codes
    are those of prepare(speaker, emotion, ids_i) + generate(options with seed + i), both on
    the GPU and in the oracle.  Five segments on a max_batch 2 decoder: groups of 2, 2, 1
    (beam search: one segment at a time)."""
    import dataclasses

    dec = itts.GptDecoder(small_weights, kv_capacity=1024, max_batch=3 if opts.get("num_beams") else 2)
    orc = oracle.OracleGpt(small_weights, kv_capacity=1024)
    sp, em = itts.synthetic_normal(192, 31), itts.synthetic_normal(1280, 32)
    segments = _segment_case(itts, 5, 21)
    o = itts.GenerationOptions(**opts)
    print(f"segments: {opts}", flush=True)
    got = dec.generate_segments(sp, em, segments, 3, o, 24)
    assert len(got) == 5
    for i, seg in enumerate(segments):
        oi = dataclasses.replace(o, seed=o.seed + i)
        single = dec.generate(dec.prepare(sp, em, seg, 3), oi, 24)
        assert (got[i].codes, got[i].stopped) == (single.codes, single.stopped), i
        codes, stopped = orc.generate(orc.prepare(sp, em, seg, 3), oracle.options_from(oi), 24)
        assert (got[i].codes, got[i].stopped) == (codes, stopped), i
    dec.close()


def test_generate_segments_cond_and_errors(small_weights, itts):
    """The raw-conditioning form equals prepare_cond + generate per segment; argument errors
    carry prepare's and generate's messages, checked for every segment before any work."""
    import dataclasses

    dec = itts.GptDecoder(small_weights, kv_capacity=1024, max_batch=4)
    cond, _ = itts.synthetic_prefix_inputs(4, seed=8)
    segments = _segment_case(itts, 3, 9)
    o = itts.GenerationOptions(seed=123, suppress_stop=True)
    got = dec.generate_segments_cond(cond, segments, 0, o, 30)
    for i, seg in enumerate(segments):
        single = dec.generate(dec.prepare_cond(cond, seg, 0), dataclasses.replace(o, seed=o.seed + i), 30)
        assert (got[i].codes, got[i].stopped) == (single.codes, single.stopped), i
        assert len(got[i].codes) == 30
    sp, em = itts.synthetic_normal(192, 1), itts.synthetic_normal(1280, 2)
    with pytest.raises(itts.InvalidArgument, match="Invalid segment count"):
        dec.generate_segments(sp, em, [], 0, o, 8)
    with pytest.raises(itts.InvalidArgument, match="Text token is outside 2.5 vocabulary"):
        dec.generate_segments(sp, em, [[5, 6], [12000]], 0, o, 8)
    with pytest.raises(itts.InvalidArgument, match="GPT generation capacity exceeded"):
        dec.generate_segments(sp, em, [[5, 6], [7]], 0, o, 1020)  # 8 + 1020 rows >= capacity 1024
    with pytest.raises(itts.InvalidArgument, match="Invalid GPT conditioning dimensions"):
        dec.generate_segments(sp[:10], em, [[5]], 0, o, 8)
    dec.close()


def test_generate_argument_errors(small, itts):
    dec, _, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    with pytest.raises(itts.InvalidArgument, match="capacity exceeded"):
        dec.generate(prefix, itts.GenerationOptions(), 1814)
    with pytest.raises(itts.InvalidArgument, match="Invalid GPT generation parameters"):
        dec.generate(prefix, itts.GenerationOptions(top_p=0.0), 8)
    with pytest.raises(itts.InvalidArgument, match="Invalid beam search configuration"):
        dec.generate(prefix, itts.GenerationOptions(num_beams=0), 8)


def test_bf16_weights_logit_tolerance(small_weights, small, itts):
    """BF16-stored weights, FP32 accumulate: logits within 5e-2 max-abs of the FP32 path."""
    dec, _, cond, text = small
    prefix = dec.prepare_cond(cond, text, 0)
    ref = dec.prefill(prefix)
    d16 = itts.GptDecoder(small_weights, kv_capacity=1024, weight_dtype="bf16")
    got = d16.prefill(prefix)
    assert float(np.max(np.abs(got - ref))) < 5e-2
    s16 = d16.step(5, 2)
    s32 = dec.step(5, 2)
    assert float(np.max(np.abs(s16 - s32))) < 5e-2
    d16.close()


# ---------------------------------------------------------------------------- full model, config 1

@pytest.fixture(scope="module")
def full(itts, oracle, full_weights):
    dec = itts.GptDecoder(full_weights, kv_capacity=4096)
    orc = oracle.OracleGpt(full_weights, kv_capacity=4096)
    cond, text = itts.synthetic_prefix_inputs(48, seed=0)
    prefix = orc.prepare_cond(cond, text, 0)
    return dec, orc, prefix


def test_full_teacher_forced_logits(full):
    """Prefill and four steps of the 24-layer model (config 1 shape): the path's bar, and the
    reference gpt_test's own bar (max-abs < 1e-4, RMSE < 2e-5, argmax equal; src/main.cpp:44-51)."""
    dec, orc, prefix = full
    assert prefix.size // 1280 == 83
    pairs = [("prefill", dec.prefill(prefix), orc.prefill(prefix))]
    for i, code in enumerate([100, 2000, 3000, 8000]):
        pairs.append((f"decode.{i + 1}", dec.step(code, i + 2), orc.step(code, i + 2)))
    for name, got, ref in pairs:
        d = np.abs(got.astype(np.float64) - ref)
        print(f"{name}: max-abs {d.max():.3e} rmse {np.sqrt(np.mean(d * d)):.3e}", flush=True)
        assert_logits_close(got, ref, name)
        assert d.max() < 1e-4 and np.sqrt(np.mean(d * d)) < 2e-5, name


def test_full_greedy_128(full, itts, oracle):
    """Greedy decode of 128 codes on the 24-layer model (config 1 shape): the codes equal the
    oracle's, and the oracle's own run produces all 128 (no stop, no error)."""
    dec, orc, prefix = full
    o = itts.GenerationOptions(do_sample=False, repetition_penalty=1.0)
    exp = orc.generate(prefix, oracle.options_from(o), 128)
    assert len(exp[0]) == 128 and not exp[1]
    r = dec.generate(prefix, o, 128)
    assert (r.codes, r.stopped) == exp


# ---------------------------------------------------------------------------- beam search (gpt_sampling.cpp:190-245)

@pytest.fixture(scope="module")
def beam_small(itts, oracle, small_weights):
    dec = itts.GptDecoder(small_weights, kv_capacity=1024, max_batch=4)
    orc = oracle.OracleGpt(small_weights, kv_capacity=1024)
    cond, text = itts.synthetic_prefix_inputs(30, seed=2)
    return dec, orc, dec.prepare_cond(cond, text, 0)


@pytest.mark.parametrize("opts", [
    dict(do_sample=False, repetition_penalty=1.0, num_beams=3),
    dict(do_sample=False, repetition_penalty=10.0, num_beams=3),
    dict(do_sample=True, seed=7, num_beams=3),
    dict(do_sample=True, seed=9, num_beams=2, top_k=0, top_p=0.9, temperature=1.2),
    dict(do_sample=False, num_beams=4, length_penalty=1.0, top_k=5),
    # every score but the two suppressed codes finite (8192 per parent): the selection keeps
    # its 24576 candidates in global memory instead of LDS
    dict(do_sample=True, seed=11, num_beams=3, top_k=0, top_p=1.0, temperature=1.0, repetition_penalty=1.0, suppress_stop=True),
])
def test_beam_search_matches_oracle(beam_small, itts, oracle, opts):
    dec, orc, prefix = beam_small
    o = itts.GenerationOptions(**opts)
    r = dec.generate(prefix, o, 24)
    codes, stopped = orc.generate(prefix, oracle.options_from(o), 24)
    assert (r.codes, r.stopped) == (codes, stopped)
    assert dec.cached_tokens() == orc.cached_tokens()


@pytest.mark.parametrize("opts", [
    # a penalty below one favours every code in the history, the start code 8192 included
    # (gpt_sampling.cpp:211), so a candidate 8192 ends the search with the reference's error (:233)
    dict(do_sample=False, repetition_penalty=0.5, num_beams=3),
    dict(do_sample=True, seed=12, num_beams=2, top_k=4, top_p=1.0, temperature=1.0, repetition_penalty=0.8),
    # a tiny top-p: one survivor per parent beyond the two that beams keep (:62)
    dict(do_sample=True, seed=13, num_beams=3, top_k=0, top_p=0.01, temperature=0.7, repetition_penalty=1.0),
])
def test_beam_search_edge_options_match_oracle(beam_small, itts, oracle, opts):
    """Beam search over option edge cases: the device and the oracle (gpt_sampling.cpp:190-245)
    give the same codes and stop flag, or the same error message."""
    dec, orc, prefix = beam_small
    o = itts.GenerationOptions(**opts)
    print(f"beam edge options {opts}", flush=True)
    try:
        r = dec.generate(prefix, o, 24)
        got = ("codes", r.codes, r.stopped)
    except itts.GptRuntimeError as e:
        got = ("error", str(e))
    try:
        codes, stopped = orc.generate(prefix, oracle.options_from(o), 24)
        want = ("codes", codes, stopped)
    except oracle.OracleError as e:
        want = ("error", str(e))
    assert got == want


def test_beam_search_needs_capacity(beam_small, itts):
    dec, _, prefix = beam_small
    with pytest.raises(itts.InvalidArgument, match="max_batch"):
        dec.generate(prefix, itts.GenerationOptions(num_beams=5), 4)


def test_full_beam3_config3_shape(itts, oracle, full_weights):
    """Config 3 shape: 32 latents + 80 text ids, 3 beams, repetition penalty 10 (40 codes here)."""
    dec = itts.GptDecoder(full_weights, kv_capacity=4096, max_batch=3)
    orc = oracle.OracleGpt(full_weights, kv_capacity=4096)
    cond, text = itts.synthetic_prefix_inputs(80, seed=3)
    prefix = orc.prepare_cond(cond, text, 0)
    assert prefix.size // 1280 == 115
    o = itts.GenerationOptions(do_sample=False, num_beams=3, length_penalty=0.0, repetition_penalty=10.0, suppress_stop=True)
    r = dec.generate(prefix, o, 40)
    codes, stopped = orc.generate(prefix, oracle.options_from(o), 40)
    assert (r.codes, r.stopped) == (codes, stopped)


# ---------------------------------------------------------------------------- persistent step kernel (step.hip)

@pytest.fixture(scope="module")
def both_paths(itts, small_weights):
    """The same 2-layer model on the persistent step kernel and on the multi-kernel path."""
    import os

    old = os.environ.get("ITTS_GPT_PERSISTENT")
    try:
        os.environ["ITTS_GPT_PERSISTENT"] = "0"
        multi = itts.GptDecoder(small_weights, kv_capacity=1024)
        os.environ["ITTS_GPT_PERSISTENT"] = "1"
        step = itts.GptDecoder(small_weights, kv_capacity=1024)
    finally:
        if old is None:
            del os.environ["ITTS_GPT_PERSISTENT"]
        else:
            os.environ["ITTS_GPT_PERSISTENT"] = old
    return step, multi


@pytest.mark.parametrize("n_text", [10, 40, 300, -900])
def test_persistent_step_bitwise_equals_multikernel(both_paths, itts, n_text):
    """Same FMA orders, LayerNorm reduction, attention tiles and merge: logits equal bit for bit
    (KV lengths spanning 1 to 12 attention splits; -900 = a raw 900-row random prefix, whose
    12 splits of 76 rows use the attention's eight arithmetic slots)."""
    step, multi = both_paths
    if n_text > 0:
        cond, text = itts.synthetic_prefix_inputs(n_text, seed=n_text)
        prefix = step.prepare_cond(cond, text, 0)
    else:
        prefix = itts.synthetic_normal(-n_text * 1280, 77, 0.0, 0.5)
    assert np.array_equal(step.prefill(prefix), multi.prefill(prefix))
    for i, code in enumerate([5, 8191, 0, 4096, 17, 300]):
        a = step.step(code, i + 2)
        assert step.last_timing()["decode_path"] == "step"
        b = multi.step(code, i + 2)
        assert multi.last_timing()["decode_path"] == "multi"
        assert np.array_equal(a, b), f"step {i}: max diff {np.max(np.abs(a - b))}"


def test_persistent_step_past_2048_rows_bitwise_equals_multikernel(itts, small_weights):
    """Caches past 2048 rows take 17 or more attention splits of up to 128 rows, so the split
    merge gathers its records through LDS (one step kernel path, one merge kernel path): a
    raw 1000-row prefix then 1100 steps to a 2101-row cache, logits equal bit for bit at
    every step."""
    import os

    old = os.environ.get("ITTS_GPT_PERSISTENT")
    try:
        os.environ["ITTS_GPT_PERSISTENT"] = "0"
        multi = itts.GptDecoder(small_weights, kv_capacity=4096)
        os.environ["ITTS_GPT_PERSISTENT"] = "1"
        step = itts.GptDecoder(small_weights, kv_capacity=4096)
    finally:
        if old is None:
            del os.environ["ITTS_GPT_PERSISTENT"]
        else:
            os.environ["ITTS_GPT_PERSISTENT"] = old
    prefix = itts.synthetic_normal(1000 * 1280, 55, 0.0, 0.5)
    assert np.array_equal(step.prefill(prefix), multi.prefill(prefix))
    codes = np.random.default_rng(3).integers(0, 8192, 1100)
    for i, code in enumerate(codes):
        a = step.step(int(code), 2 + i % 1800)
        b = multi.step(int(code), 2 + i % 1800)
        assert np.array_equal(a, b), f"step {i} ({1000 + i} cached rows): max diff {np.max(np.abs(a - b))}"
    assert step.last_timing()["decode_path"] == "step" and multi.last_timing()["decode_path"] == "multi"
    assert step.cached_tokens() == multi.cached_tokens() == 2100
    step.close()
    multi.close()


def _step_paths(itts, weights, var, **kw):
    """Two decoders over the same weights: `var`=0 (multi-kernel path) and `var`=1 (persistent)."""
    import os

    old = os.environ.get(var)
    try:
        os.environ[var] = "0"
        multi = itts.GptDecoder(weights, kv_capacity=4096, **kw)
        os.environ[var] = "1"
        step = itts.GptDecoder(weights, kv_capacity=4096, **kw)
    finally:
        if old is None:
            del os.environ[var]
        else:
            os.environ[var] = old
    return step, multi


def test_past_2048_rows_to_the_reference_limit_match_oracle(itts, oracle, small_weights):
    """The longest cache the reference admits: a 1024-row prefix (src/gpt.cpp:73) and 1813
    teacher-forced steps at mel positions 2..1814 (src/gpt_sampling.cpp:169), so the last step
    attends over 2837 rows.  From 2049 rows on, every step takes 17-23 attention splits and the
    split merge gathers its records through LDS.  Both the persistent step and the multi-kernel
    path are compared with the CPU oracle (not only with each other) at every step from 2040
    cached rows on, at the path's bar and at the reference's gpt_test bar (src/main.cpp:47)."""
    step, multi = _step_paths(itts, small_weights, "ITTS_GPT_PERSISTENT")
    orc = oracle.OracleGpt(small_weights, kv_capacity=4096)
    prefix = itts.synthetic_normal(1024 * 1280, 56, 0.0, 0.5)
    print("past 2048 rows vs oracle: 1024-row prefix, 1813 steps", flush=True)
    ref = orc.prefill(prefix)
    assert_logits_close(step.prefill(prefix), ref, "persistent prefill")
    assert_logits_close(multi.prefill(prefix), ref, "multi-kernel prefill")
    codes = np.random.default_rng(4).integers(0, 8192, 1813)
    worst_abs, worst_rmse, compared = 0.0, 0.0, 0
    for i, code in enumerate(codes):
        rows = 1024 + i + 1  # cache length after this step
        ref = orc.step(int(code), i + 2)
        a = step.step(int(code), i + 2)
        b = multi.step(int(code), i + 2)
        if rows < 2040:
            continue
        for got, what in ((a, "persistent"), (b, "multi-kernel")):
            assert_logits_close(got, ref, f"{what} step {i} ({rows} cached rows)")
            d = np.abs(got.astype(np.float64) - ref)
            worst_abs, worst_rmse = max(worst_abs, float(d.max())), max(worst_rmse, float(np.sqrt(np.mean(d * d))))
        compared += 1
    assert step.last_timing()["decode_path"] == "step" and multi.last_timing()["decode_path"] == "multi"
    assert step.cached_tokens() == multi.cached_tokens() == orc.cached_tokens() == 2837
    print(f"{compared} steps at 2040-2837 rows: worst max-abs {worst_abs:.3e}, rmse {worst_rmse:.3e}", flush=True)
    assert worst_abs < 1e-4 and worst_rmse < 2e-5
    step.close()
    multi.close()


def test_batch_past_2048_rows_to_the_reference_limit_match_oracle(itts, oracle, small_weights):
    """Three sequences of 1024-row prefixes, 1813 sampled codes each (caches to 2837 rows, up
    to 23 attention splits per (sequence, head)): the codes of the persistent batch step and of
    the multi-kernel batch path both equal the CPU oracle's generate for every sequence."""
    step, multi = _step_paths(itts, small_weights, "ITTS_GPT_PERSISTENT_BATCH", max_batch=3)
    orc = oracle.OracleGpt(small_weights, kv_capacity=4096)
    prefixes = [itts.synthetic_normal(1024 * 1280, 160 + b, 0.0, 0.5) for b in range(3)]
    opts = [itts.GenerationOptions(seed=170 + b, top_k=0, top_p=1.0, temperature=1.0, repetition_penalty=1.0,
                                   suppress_stop=True) for b in range(3)]
    print("batch past 2048 rows vs oracle: 3 x (1024-row prefix, 1813 codes)", flush=True)
    a = step.generate_batch(prefixes, opts, 1813)
    assert step.last_timing()["decode_path"] == "step"
    b = multi.generate_batch(prefixes, opts, 1813)
    assert multi.last_timing()["decode_path"] == "multi"
    for q in range(3):
        exp = orc.generate(prefixes[q], oracle.options_from(opts[q]), 1813)
        assert len(exp[0]) == 1813
        assert (a[q].codes, a[q].stopped) == exp, f"persistent batch, sequence {q}"
        assert (b[q].codes, b[q].stopped) == exp, f"multi-kernel batch, sequence {q}"
    step.close()
    multi.close()


def test_persistent_generate_equals_multikernel(both_paths, itts):
    step, multi = both_paths
    cond, text = itts.synthetic_prefix_inputs(60, seed=5)
    prefix = step.prepare_cond(cond, text, 0)
    o = itts.GenerationOptions(do_sample=True, seed=11, suppress_stop=True)
    a = step.generate(prefix, o, 96)
    assert step.last_timing()["decode_path"] == "step"
    b = multi.generate(prefix, o, 96)
    assert (a.codes, a.stopped) == (b.codes, b.stopped)
    assert step.cached_tokens() == multi.cached_tokens()


def test_fused_sampling_tail_equals_separate_sampler(itts, small_weights):
    """ITTS_GPT_FUSED_SAMPLER=1: the step kernel's last workgroup samples the next token from the
    tagged logits (512 threads) instead of a sampler launch (1024 threads): same codes, sampled
    (top-k/top-p, penalty, temperature), greedy, and with a stop token allowed."""
    import os

    old = os.environ.get("ITTS_GPT_FUSED_SAMPLER")
    try:
        os.environ["ITTS_GPT_FUSED_SAMPLER"] = "1"
        fused = itts.GptDecoder(small_weights, kv_capacity=1024)
    finally:
        if old is None:
            del os.environ["ITTS_GPT_FUSED_SAMPLER"]
        else:
            os.environ["ITTS_GPT_FUSED_SAMPLER"] = old
    plain = itts.GptDecoder(small_weights, kv_capacity=1024)
    cond, text = itts.synthetic_prefix_inputs(60, seed=7)
    prefix = fused.prepare_cond(cond, text, 0)
    for o in (itts.GenerationOptions(do_sample=True, seed=11, suppress_stop=True),
              itts.GenerationOptions(do_sample=True, seed=12, top_k=0, top_p=0.9, temperature=1.1, repetition_penalty=2.0),
              itts.GenerationOptions(do_sample=False, repetition_penalty=1.0, suppress_stop=True)):
        a = fused.generate(prefix, o, 80)
        assert fused.last_timing()["decode_path"] == "step"
        b = plain.generate(prefix, o, 80)
        assert (a.codes, a.stopped) == (b.codes, b.stopped), o
        assert fused.cached_tokens() == plain.cached_tokens()
    fused.close()
    plain.close()


def test_two_decoders_concurrently_on_one_gpu(itts, small_weights):
    """Two decoders of one process on one GPU, each driven from its own thread, both on the
    persistent step (batch 1 and batch 2): their grids are chained, never resident together,
    so each gets the codes it gets alone and no hand-off times out."""
    import dataclasses
    import threading

    import os

    a = itts.GptDecoder(small_weights, kv_capacity=1024)
    old = os.environ.get("ITTS_GPT_PERSISTENT_BATCH")
    os.environ["ITTS_GPT_PERSISTENT_BATCH"] = "1"  # the batch step is opt-in
    try:
        b = itts.GptDecoder(small_weights, kv_capacity=1024, max_batch=2)
    finally:
        if old is None:
            del os.environ["ITTS_GPT_PERSISTENT_BATCH"]
        else:
            os.environ["ITTS_GPT_PERSISTENT_BATCH"] = old
    cond, text = itts.synthetic_prefix_inputs(30, seed=12)
    prefix = a.prepare_cond(cond, text, 0)
    o = itts.GenerationOptions(seed=3, suppress_stop=True)
    opts = [o, dataclasses.replace(o, seed=4)]
    ref_a = a.generate(prefix, o, 64)
    ref_b = b.generate_batch([prefix, prefix], opts, 64)
    assert a.last_timing()["decode_path"] == b.last_timing()["decode_path"] == "step"
    out, errors = {}, []

    def run(name, fn):
        try:
            out[name] = [fn() for _ in range(3)]
        except Exception as e:  # reported below: a thread's exception is not raised by join()
            errors.append(e)

    threads = [threading.Thread(target=run, args=("a", lambda: a.generate(prefix, o, 64))),
               threading.Thread(target=run, args=("b", lambda: b.generate_batch([prefix, prefix], opts, 64)))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(120)
    assert not errors, errors
    assert all(r.codes == ref_a.codes for r in out["a"])
    assert all([x.codes for x in r] == [x.codes for x in ref_b] for r in out["b"])
    a.close()
    b.close()


@pytest.fixture(scope="module")
def batch_paths(itts, small_weights):
    """The 2-layer model with its stop token made likely (mel_head bias + 2.5), on the persistent
    batch step (groups of up to 4 sequences per launch) and on the multi-kernel batch path."""
    import os

    w = dict(small_weights)
    hb = w["gpt.mel_head.bias"].copy()
    hb[8193] += 2.5
    w["gpt.mel_head.bias"] = hb
    old = os.environ.get("ITTS_GPT_PERSISTENT_BATCH")
    try:
        os.environ["ITTS_GPT_PERSISTENT_BATCH"] = "0"
        multi = itts.GptDecoder(w, kv_capacity=1024, max_batch=8)
        os.environ["ITTS_GPT_PERSISTENT_BATCH"] = "1"
        step = itts.GptDecoder(w, kv_capacity=1024, max_batch=8)
    finally:
        if old is None:
            del os.environ["ITTS_GPT_PERSISTENT_BATCH"]
        else:
            os.environ["ITTS_GPT_PERSISTENT_BATCH"] = old
    return step, multi


@pytest.mark.parametrize("nseq", [2, 3, 4, 5, 7])
def test_persistent_batch_generate_equals_multikernel(batch_paths, itts, nseq):
    """Ragged prefixes (8..300 text ids: 1..6 attention splits per sequence), sampled codes, some
    sequences stopping early (then inactive inside the launch): the persistent batch step (up to
    4 sequences; more stay on the multi-kernel path) and the multi-kernel path give the same
    codes, and each equals its batch-1 generate."""
    step, multi = batch_paths
    rng = np.random.default_rng(nseq)
    prefixes, opts = [], []
    for b in range(nseq):
        cond, text = itts.synthetic_prefix_inputs(int(rng.integers(8, 300)), seed=200 + b)
        prefixes.append(step.prepare_cond(cond, text, 0))
        opts.append(itts.GenerationOptions(seed=300 + b, suppress_stop=b % 3 == 0))
    print(f"persistent batch: nseq {nseq}", flush=True)
    a = step.generate_batch(prefixes, opts, 40)
    assert step.last_timing()["decode_path"] == ("step" if nseq <= 4 else "multi")
    b = multi.generate_batch(prefixes, opts, 40)
    assert multi.last_timing()["decode_path"] == "multi"
    assert [(r.codes, r.stopped) for r in a] == [(r.codes, r.stopped) for r in b]
    for q in (0, nseq - 1):
        single = step.generate(prefixes[q], opts[q], 40)
        assert (single.codes, single.stopped) == (a[q].codes, a[q].stopped)


def test_persistent_batch_long_caches_equal_multikernel(batch_paths, itts):
    """Caches of 780-1014 rows: 12 attention splits of 65-85 rows, so the tiles use the
    attention's eight arithmetic slots (slots 4-7 loaded once 0-3 are used), three tile
    rounds for three sequences.  Sampled over every code (top_k 0, top_p 1): the persistent
    batch step, the multi-kernel path and each sequence's batch-1 generate agree."""
    step, multi = batch_paths
    prefixes = [itts.synthetic_normal(rows * 1280, 90 + rows, 0.0, 0.5) for rows in (780, 900, 990)]
    opts = [itts.GenerationOptions(seed=40 + b, top_k=0, top_p=1.0, temperature=1.0, repetition_penalty=1.0, suppress_stop=True)
            for b in range(3)]
    print("persistent batch: long caches", flush=True)
    a = step.generate_batch(prefixes, opts, 24)
    assert step.last_timing()["decode_path"] == "step"
    b = multi.generate_batch(prefixes, opts, 24)
    assert multi.last_timing()["decode_path"] == "multi"
    assert [(r.codes, r.stopped) for r in a] == [(r.codes, r.stopped) for r in b]
    for q in range(3):
        single = step.generate(prefixes[q], opts[q], 24)
        assert (single.codes, single.stopped) == (a[q].codes, a[q].stopped)


def test_persistent_batch_past_2048_rows_equals_multikernel(itts, small_weights):
    """Three sequences from raw 1000-row prefixes to 2100-row caches: past 2048 rows 17
    attention splits per (sequence, head), merged through LDS.  Sampled over every code:
    the persistent batch step, the multi-kernel path and the first sequence's batch-1
    generate agree."""
    import os

    old = os.environ.get("ITTS_GPT_PERSISTENT_BATCH")
    try:
        os.environ["ITTS_GPT_PERSISTENT_BATCH"] = "0"
        multi = itts.GptDecoder(small_weights, kv_capacity=4096, max_batch=3)
        os.environ["ITTS_GPT_PERSISTENT_BATCH"] = "1"
        step = itts.GptDecoder(small_weights, kv_capacity=4096, max_batch=3)
    finally:
        if old is None:
            del os.environ["ITTS_GPT_PERSISTENT_BATCH"]
        else:
            os.environ["ITTS_GPT_PERSISTENT_BATCH"] = old
    prefixes = [itts.synthetic_normal(1000 * 1280, 60 + b, 0.0, 0.5) for b in range(3)]
    opts = [itts.GenerationOptions(seed=70 + b, top_k=0, top_p=1.0, temperature=1.0, repetition_penalty=1.0, suppress_stop=True)
            for b in range(3)]
    print("persistent batch: caches past 2048 rows", flush=True)
    a = step.generate_batch(prefixes, opts, 1100)
    assert step.last_timing()["decode_path"] == "step"
    b = multi.generate_batch(prefixes, opts, 1100)
    assert multi.last_timing()["decode_path"] == "multi"
    assert [(r.codes, r.stopped) for r in a] == [(r.codes, r.stopped) for r in b]
    single = step.generate(prefixes[0], opts[0], 1100)
    assert (single.codes, single.stopped) == (a[0].codes, a[0].stopped)
    step.close()
    multi.close()


@pytest.mark.parametrize("opts", [
    dict(do_sample=False, num_beams=3, repetition_penalty=10.0, suppress_stop=True),
    dict(do_sample=False, num_beams=4, length_penalty=1.0),
    dict(do_sample=True, seed=5, num_beams=3),
    dict(do_sample=True, seed=6, num_beams=2, top_k=0, top_p=0.9, temperature=1.2),
])
def test_persistent_beam_search_equals_multikernel(batch_paths, itts, opts):
    """Beam search on the persistent batch step, children reading their parents' cached rows
    through the row-owner table, gives the multi-kernel path's codes (the stop bias ends
    beams, so the number of children per step varies)."""
    step, multi = batch_paths
    cond, text = itts.synthetic_prefix_inputs(50, seed=9)
    prefix = step.prepare_cond(cond, text, 0)
    o = itts.GenerationOptions(**opts)
    print(f"persistent beams: {opts}", flush=True)
    a = step.generate(prefix, o, 32)
    if o.suppress_stop:
        assert step.last_timing()["decode_path"] == "step"
    b = multi.generate(prefix, o, 32)
    assert multi.last_timing()["decode_path"] == "multi"
    assert (a.codes, a.stopped) == (b.codes, b.stopped)
    assert step.cached_tokens() == multi.cached_tokens()


def test_step_phase_stamps(batch_paths, itts):
    """The phase stamps of the step kernel (1 sequence) and the batch step kernel (3): every
    phase takes a positive time, the six layer phases add up to the layer, and requests the
    kernels cannot serve are errors.  A generate afterwards is unaffected."""
    step, multi = batch_paths
    for nseq in (1, 3):
        print(f"phase stamps: nseq {nseq}", flush=True)
        ph = step.step_phases(cached_rows=200, iters=2, nseq=nseq)
        assert list(ph) == list(step.STEP_PHASES)
        assert all(np.isfinite(v) and v > 0 for v in ph.values()), ph
        parts = sum(ph[k] for k in step.STEP_PHASES[1:7])
        assert abs(parts - ph["layer"]) <= 1e-3 * ph["layer"] + 1e-3, ph
    for nseq in (0, 5):
        with pytest.raises(itts.InvalidArgument):
            step.step_phases(cached_rows=200, iters=1, nseq=nseq)
    with pytest.raises(itts.InvalidArgument):
        step.step_phases(cached_rows=1023, iters=1, nseq=3)
    cond, text = itts.synthetic_prefix_inputs(30, seed=4)
    prefix = step.prepare_cond(cond, text, 0)
    o = itts.GenerationOptions(seed=8)
    a, b = step.generate(prefix, o, 16), multi.generate(prefix, o, 16)
    assert (a.codes, a.stopped) == (b.codes, b.stopped)


@pytest.mark.gpu
def test_decoder_from_bundle_bitwise_equals_arrays(itts, small_weights, tmp_path):
    """GptDecoder.from_bundle (zero-copy from the mapping) and GptDecoder(arrays) upload the
    same weights: identical prefill logits, steps and sampled codes."""
    for single in (False, True):
        path = itts.write_mit2_bundle(tmp_path / ("one.mit2" if single else "dir"), small_weights, single_file=single)
        b = itts.Bundle(path, require_model=not single)
        a = itts.GptDecoder(small_weights, kv_capacity=1024)
        d = itts.GptDecoder.from_bundle(b, kv_capacity=1024)
        b.close()  # the decoder holds device copies; the mapping is no longer needed
        cond, ids = itts.synthetic_prefix_inputs(40, seed=5)
        prefix = a.prepare_cond(cond, ids, 3)
        la, ld = a.prefill(prefix), d.prefill(prefix)
        assert np.array_equal(la, ld)
        assert np.array_equal(a.step(17, 2), d.step(17, 2))
        opt = itts.GenerationOptions(seed=9, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0)
        ra, rd = a.generate(prefix, opt, 24), d.generate(prefix, opt, 24)
        assert list(ra.codes) == list(rd.codes) and ra.stopped == rd.stopped
        a.close()
        d.close()


def test_beam_error_with_queued_steps(itts, small_weights):
    """A beam search that raises (its best candidate is code 8192, gpt_sampling.cpp:234) while
    later steps are already queued: the queued steps stay in bounds (all children inactive),
    the decoder closes cleanly, and a new search works."""
    w = dict(small_weights)
    hb = w["gpt.mel_head.bias"].copy()
    hb[8192] += 6.0
    w["gpt.mel_head.bias"] = hb
    dec = itts.GptDecoder(w, kv_capacity=1024, max_batch=4)
    cond, text = itts.synthetic_prefix_inputs(20, seed=4)
    prefix = dec.prepare_cond(cond, text, 0)
    with pytest.raises(itts.GptRuntimeError, match="Beam generated invalid semantic code"):
        # penalty 1: 8192 is in every history ({1, 8192}, gpt_sampling.cpp:176), which a penalty would push down
        dec.generate(prefix, itts.GenerationOptions(do_sample=False, num_beams=3, repetition_penalty=1.0), 32)
    dec.close()
    ok = itts.GptDecoder(small_weights, kv_capacity=1024, max_batch=4)
    r = ok.generate(ok.prepare_cond(cond, text, 0), itts.GenerationOptions(num_beams=3, seed=1, suppress_stop=True), 8)
    assert len(r.codes) == 8
    ok.close()
