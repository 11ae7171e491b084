"""Beam search on the device (gpt_sampling.cpp:190-245) against exhaustive search and the oracle.

* On a history-independent head (mel_head.weight = 0, a designed bias; tests/beam_brute.py)
  the device's search returns the exhaustive best hypothesis, the same as the oracle's.
* Tie-heavy heads at 9 and 10 beams (20 candidates per step, many with equal scores): the
  device's codes equal the oracle's.  The reference's candidate sort (std::sort, :228, built
  with libc++) keeps equal candidates in order below 24 elements; the oracle and the device
  sort stably (tests/test_beam_oracle.py).
"""
import numpy as np
import pytest

import beam_brute as bb

pytestmark = pytest.mark.gpu


def _bias_only(weights, bias):
    w = dict(weights)
    w["gpt.mel_head.weight"] = np.zeros_like(w["gpt.mel_head.weight"])
    w["gpt.mel_head.bias"] = bias
    return w


@pytest.fixture(scope="module")
def prefix(itts):
    cond, text = itts.synthetic_prefix_inputs(12, seed=21)
    return cond, text


@pytest.mark.parametrize("case", range(len(bb.CASES)))
def test_device_beam_search_returns_exhaustive_best(itts, oracle, small_weights, prefix, case):
    good, opts, beams, steps = bb.CASES[case]
    tokens, _, _ = bb.case_tokens(good)
    w = _bias_only(small_weights, bb.head_bias(good))
    dec = itts.GptDecoder(w, kv_capacity=256, max_batch=10)
    orc = oracle.OracleGpt(w, kv_capacity=256)
    p = dec.prepare_cond(*prefix, 0)
    o = orc_opts = oracle.options(num_beams=beams, **opts)
    if not o.do_sample:
        o2 = oracle.options(num_beams=beams, **opts)
        o2.temperature, o2.top_k, o2.top_p = 1.0, 0, 1.0
        proc = lambda lp, h: oracle.processors(lp, h, o2)
    else:
        proc = lambda lp, h: oracle.processors(lp, h, orc_opts)
    (_, codes, eos), _ = bb.best(bb.head_bias(good), proc, opts["length_penalty"], steps, tokens)
    print(f"beam case {case}: {beams} beams, {steps} steps, expect {list(codes)} eos={eos}", flush=True)
    r = dec.generate(p, itts.GenerationOptions(num_beams=beams, **opts), steps)
    assert (r.codes, r.stopped) == (list(codes), eos)
    assert orc.generate(p, o, steps) == (list(codes), eos)
    dec.close()


TIE_HEADS = {
    # six tokens with one bias value, the stop token just below
    "six_equal": {**{t: 1.0 for t in (3, 500, 501, 2048, 6000, 8191)}, bb.STOP: 0.5},
    # pairs of equal values
    "pairs": {3: 1.25, 9: 1.25, 77: 0.75, 78: 0.75, 4000: 0.5, 4001: 0.5, bb.STOP: 0.25},
}


@pytest.mark.parametrize("head", sorted(TIE_HEADS))
@pytest.mark.parametrize("opts", [
    dict(do_sample=False, num_beams=10, repetition_penalty=1.0, length_penalty=0.0),
    dict(do_sample=False, num_beams=9, repetition_penalty=10.0, length_penalty=1.0),
    dict(do_sample=True, seed=3, num_beams=10, top_k=8, top_p=1.0, temperature=1.0, repetition_penalty=1.0),
    dict(do_sample=True, seed=4, num_beams=9, top_k=0, top_p=0.99, temperature=0.9, repetition_penalty=2.0),
])
def test_tie_heavy_nine_and_ten_beams_equal_oracle(itts, oracle, small_weights, prefix, head, opts):
    w = _bias_only(small_weights, bb.head_bias(TIE_HEADS[head]))
    dec = itts.GptDecoder(w, kv_capacity=256, max_batch=10)
    orc = oracle.OracleGpt(w, kv_capacity=256)
    p = dec.prepare_cond(*prefix, 0)
    print(f"tie-heavy beams: {head} {opts}", flush=True)
    r = dec.generate(p, itts.GenerationOptions(**opts), 6)
    assert (r.codes, r.stopped) == orc.generate(p, oracle.options(**opts), 6)
    dec.close()
