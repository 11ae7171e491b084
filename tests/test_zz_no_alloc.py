"""itts_gpt_generate_noalloc (include/itts_gpt.h): generate() for callers that cannot allocate.

Its prefill activations live in the library's device scratch array instead of buffers grown
per call.  Through the C ABI, on two calls in a row (the second with a shorter prefix and
fewer codes), its codes must equal itts_gpt_generate's on the same decoder: on the persistent
step path (FP32) and on the multi-kernel path (BF16 weights: eager launches while the decode
graph is not captured yet, graph replays once generate() has captured it).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(itts, n_text, seed):
    cond, text = itts.synthetic_prefix_inputs(n_text, seed=seed)
    return cond, text


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_noalloc_codes_equal_generate(itts, small_weights, dtype):
    dec = itts.GptDecoder(small_weights, kv_capacity=1024, weight_dtype=dtype)
    calls = [(200, 5, 48, dict(seed=42, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0)),
             (40, 6, 24, dict(do_sample=False, repetition_penalty=1.0, suppress_stop=True))]
    for i, (n_text, seed, max_tokens, opts) in enumerate(calls):
        cond, text = _case(itts, n_text, seed)
        prefix = dec.prepare_cond(cond, text, 0)
        o = itts.GenerationOptions(**opts)
        print(f"noalloc {dtype} call {i}: {prefix.size // 1280} prefix rows, {max_tokens} codes", flush=True)
        if dtype == "bf16" and i == 0:
            # no decode graph captured yet: the no-alloc call launches the kernels eagerly
            a = dec.generate_noalloc(prefix, o, max_tokens)
            cached_a = dec.cached_tokens()
            b = dec.generate(prefix, o, max_tokens)
        else:
            b = dec.generate(prefix, o, max_tokens)
            a = dec.generate_noalloc(prefix, o, max_tokens)
            cached_a = dec.cached_tokens()
        assert dec.last_timing()["decode_path"] == ("step" if dtype == "f32" else "multi")
        assert (a.codes, a.stopped) == (b.codes, b.stopped), i
        assert cached_a == dec.cached_tokens()
        assert len(a.codes) == max_tokens or a.stopped
    dec.close()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_noalloc_allocates_nothing(itts, small_weights, dtype):
    """itts_gpt_alloc_events counts every device and pinned allocation and every graph
    instantiation the decoders make.  On a fresh decoder (no prefill yet, so generate() would
    grow its prefill buffers to the prefix; for BF16 no decode graph captured yet), a no-alloc
    call leaves the count unchanged.  generate() on the same input then moves it, which shows
    the count sees those allocations; the codes are equal."""
    dec = itts.GptDecoder(small_weights, kv_capacity=1024, weight_dtype=dtype)
    prefix = itts.synthetic_normal(480 * 1280, 21, 0.0, 0.5)
    o = itts.GenerationOptions(seed=5, suppress_stop=True)
    before = itts.alloc_events()
    a = dec.generate_noalloc(prefix, o, 40)
    a2 = dec.generate_noalloc(prefix[: 300 * 1280], o, 20)
    assert itts.alloc_events() == before, "a no-alloc call allocated"
    b = dec.generate(prefix, o, 40)
    assert itts.alloc_events() > before, "generate() grew nothing: the count does not see allocations"
    assert (a.codes, a.stopped) == (b.codes, b.stopped)
    assert a2.codes == dec.generate(prefix[: 300 * 1280], o, 20).codes
    dec.close()


def test_noalloc_prefill_state_continues_like_generate(itts, small_weights):
    """After generate_noalloc, step() continues from the same KV cache as after generate()."""
    dec = itts.GptDecoder(small_weights, kv_capacity=1024)
    cond, text = _case(itts, 60, 9)
    prefix = dec.prepare_cond(cond, text, 0)
    o = itts.GenerationOptions(do_sample=False, repetition_penalty=1.0, suppress_stop=True)
    r1 = dec.generate(prefix, o, 16)
    s1 = dec.step(11, 18)
    r2 = dec.generate_noalloc(prefix, o, 16)
    s2 = dec.step(11, 18)
    assert r1.codes == r2.codes
    assert np.array_equal(s1, s2)
    dec.close()


def test_noalloc_limits(itts, small_weights):
    dec = itts.GptDecoder(small_weights, kv_capacity=1024, max_batch=2)
    big = itts.synthetic_normal(513 * 1280, 3, 0.0, 0.5)
    with pytest.raises(itts.InvalidArgument, match="512-row scratch"):
        dec.generate_noalloc(big, itts.GenerationOptions(), 4)
    cond, text = _case(itts, 20, 4)
    prefix = dec.prepare_cond(cond, text, 0)
    with pytest.raises(itts.InvalidArgument, match="num_beams 1"):
        dec.generate_noalloc(prefix, itts.GenerationOptions(num_beams=2), 4)
    with pytest.raises(itts.InvalidArgument, match="capacity exceeded"):
        dec.generate_noalloc(prefix, itts.GenerationOptions(), 1814)
    # 512 rows is within the limit
    ok = itts.synthetic_normal(512 * 1280, 3, 0.0, 0.5)
    o = itts.GenerationOptions(do_sample=False, repetition_penalty=1.0, suppress_stop=True)
    assert dec.generate_noalloc(ok, o, 8).codes == dec.generate(ok, o, 8).codes
    dec.close()
