"""Pins the oracle's beam search (orc_generate with num_beams > 1; src/gpt_sampling.cpp:190-245).

CPU only.  On a history-independent head (mel_head.weight = 0) the search must return the
exhaustive best hypothesis (tests/beam_brute.py explains why); a hand-derived case shows the
-1e9 initial scores of beams 1.. decide the answer; and the candidate order the search relies
on is the one the reference's toolchain gives.
"""
import numpy as np
import pytest

import beam_brute as bb
from test_oracle import tiny_weights


def _model(oracle, good):
    w = tiny_weights(seed=4)
    w["gpt.mel_head.weight"] = np.zeros_like(w["gpt.mel_head.weight"])
    w["gpt.mel_head.bias"] = bb.head_bias(good)
    return oracle.OracleGpt(w, kv_capacity=128)


def _processors(oracle, opts):
    o = oracle.options(**opts)
    if not o.do_sample:  # generate() (gpt_sampling.cpp:171)
        o.temperature, o.top_k, o.top_p = 1.0, 0, 1.0
    return lambda lp, hist: oracle.processors(lp, hist, o)


@pytest.mark.parametrize("case", range(len(bb.CASES)))
def test_beam_search_returns_exhaustive_best(oracle, case):
    good, opts, beams, steps = bb.CASES[case]
    tokens, n_good, n_nonstop = bb.case_tokens(good)
    assert bb.good_counts_ok(n_good, n_nonstop, beams, steps, bb.STOP in good)
    m = _model(oracle, good)
    rows = np.random.default_rng(case).standard_normal((5, 128)).astype(np.float32)
    assert np.array_equal(m.prefill(rows), bb.head_bias(good))  # the head is bias only
    (score, codes, eos), runner_up = bb.best(bb.head_bias(good), _processors(oracle, opts), opts["length_penalty"], steps, tokens)
    assert score > runner_up  # the best hypothesis is unique: no tie rule involved
    got = m.generate(rows, oracle.options(num_beams=beams, **opts), steps)
    assert got == (list(codes), eos), (got, codes, eos)


def test_planted_mistakes_change_the_exhaustive_answer(oracle):
    """The enumeration is discriminating: with a planted mistake (the length penalty dropped, or
    the processors run without the hypothesis' own history) its best hypothesis differs from the
    correct one in some cases, and in each of them the oracle's search returns the correct one,
    not the mistaken one."""
    mistakes = {
        "no length penalty": lambda proc, lpen: (proc, 0.0),
        "processors without history": lambda proc, lpen: (lambda lp, h: proc(lp, [1, 8192]), lpen),
    }
    for name, plant in mistakes.items():
        caught = 0
        for case, (good, opts, beams, steps) in enumerate(bb.CASES):
            tokens, _, _ = bb.case_tokens(good)
            proc = _processors(oracle, opts)
            (_, codes, eos), _ = bb.best(bb.head_bias(good), proc, opts["length_penalty"], steps, tokens)
            wrong_proc, wrong_lpen = plant(proc, opts["length_penalty"])
            (_, wcodes, weos), _ = bb.best(bb.head_bias(good), wrong_proc, wrong_lpen, steps, tokens)
            if (wcodes, weos) == (codes, eos):
                continue
            got = _model(oracle, good).generate(np.zeros((3, 128), np.float32), oracle.options(num_beams=beams, **opts), steps)
            assert got == (list(codes), eos) and got != (list(wcodes), weos), (name, case)
            caught += 1
        assert caught > 0, name


def test_initial_beam_scores_minus_1e9_closed_form(oracle):
    """Three beams, two steps, penalty 10, length penalty 0; the head leaves token a = 17 and the
    stop token as the only good candidates, with log-probabilities la > le (about -0.43 and
    -1.05) and every other token near -200.

    Step 0, with beams 1 and 2 at -1e9 (gpt_sampling.cpp:198): the ranked candidates start
    [a (la), stop (le), then tokens of beam 0 near -200]; stop has rank 1 < 3, so the empty
    hypothesis finishes with score le.  Step 1 from [a]: [a, stop] scores la + le and
    [a, a] la + 10 la (penalised repeat).  Best finished: the empty one (le > la + le), so
    generate returns no codes, stopped.

    Had beams 1 and 2 started at 0 like beam 0, step 0 would rank [a, a, a, stop, ...]: the
    three children fill the beams before the stop token is reached, and the answer would be [a]
    (stopped at step 1) instead."""
    good = {17: 1.0, bb.STOP: 0.37}
    lp = bb.log_softmax(bb.head_bias(good))
    la, le = float(lp[17]), float(lp[bb.STOP])
    assert la > le and le > la + le > la + 10 * la
    m = _model(oracle, good)
    rows = np.random.default_rng(1).standard_normal((4, 128)).astype(np.float32)
    got = m.generate(rows, oracle.options(do_sample=False, num_beams=3, repetition_penalty=10.0, length_penalty=0.0), 2)
    assert got == ([], True)


def test_candidate_sort_is_stable_in_the_reference_toolchain():
    """The reference sorts its 2*num_beams candidates with std::sort (gpt_sampling.cpp:228), which
    is not stable in general.  Its recorded build uses AppleClang 17 (docs/standalone-build.txt:1),
    i.e. libc++, whose std::sort handles ranges below 24 elements with the 2..5-element sorting
    networks (__sort2.. __sort5, which swap only on a strict comparison) and a plain insertion
    sort.  Both keep equal elements in their order, so for take = 2*num_beams <= 20 the
    reference's candidate order is the stable one, which the oracle (std::stable_sort) and the
    device (insertion sort) use.  Checked here on the published algorithm: the networks and the
    insertion sort, restated, equal a stable sort on every tie pattern of 3..5 elements and on
    random tie-heavy arrays up to 20."""
    import itertools

    def sort3(a, x, y, z, less):
        if not less(a[y], a[x]):
            if not less(a[z], a[y]):
                return
            a[y], a[z] = a[z], a[y]
            if less(a[y], a[x]):
                a[x], a[y] = a[y], a[x]
            return
        if less(a[z], a[y]):
            a[x], a[z] = a[z], a[x]
            return
        a[x], a[y] = a[y], a[x]
        if less(a[z], a[y]):
            a[y], a[z] = a[z], a[y]

    def insert_last(a, lo, hi, less):  # a[lo..hi-1] sorted; insert a[hi] with strict comparisons
        j = hi
        while j > lo and less(a[j], a[j - 1]):
            a[j], a[j - 1] = a[j - 1], a[j]
            j -= 1

    def libcxx_small_sort(a, less):
        n = len(a)
        if n == 2:
            if less(a[1], a[0]):
                a[0], a[1] = a[1], a[0]
        elif 3 <= n <= 5:
            sort3(a, 0, 1, 2, less)
            for k in range(3, n):
                insert_last(a, 0, k, less)
        elif n >= 6:
            for k in range(1, n):
                insert_last(a, 0, k, less)
        return a

    less = lambda p, q: p[0] > q[0]  # candidates by score, descending (gpt_sampling.cpp:228)
    for n in range(1, 6):
        for scores in itertools.product(range(3), repeat=n):
            items = [(s, i) for i, s in enumerate(scores)]
            assert libcxx_small_sort(list(items), less) == sorted(items, key=lambda p: -p[0])
    rng = np.random.default_rng(0)
    for _ in range(2000):
        n = int(rng.integers(6, 21))
        items = [(int(s), i) for i, s in enumerate(rng.integers(0, 4, n))]
        assert libcxx_small_sort(list(items), less) == sorted(items, key=lambda p: -p[0])
