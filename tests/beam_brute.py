"""Exhaustive search for beam search on a history-independent head (shared by the CPU and GPU tests).

With mel_head.weight = 0 the logits are mel_head.bias at every step, whatever the history, so
the per-step log-probabilities are one fixed vector and the only history dependence left is
the repetition penalty (a pinned processor).  Take a bias with a few "good" tokens near zero
and every other entry at -200, and a num_beams no smaller than the number of good
candidates at any step, and larger than the number of good hypotheses that end in the stop
token: beam search then never prunes a good hypothesis, never stops early (:240 needs
num_beams finished hypotheses all at least as good as the best candidate, and only good ones
can be), the -1e9 initial scores of beams 1.. keep their candidates behind every good one,
and the reference's search
(src/gpt_sampling.cpp:190-245) must return the best of all good hypotheses under its scoring:
  * a step adds the processed log-probability to the parent's float score (:207-214);
  * a stop token (8193) at step i finishes the parent's codes with length i + 1 (:232);
  * after the last step the survivors finish with length = their code count (:242);
  * finished score = score / length^length_penalty in double (:200), best first (:244).
The enumeration below follows those rules with the same float32 arithmetic; it shares none of
the search's machinery (candidate ranking, sorting, children, finished-list trimming).
"""
import ctypes

import numpy as np

MEL = 8194
STOP = 8193
BAD = -200.0

_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]
_libm.logf.restype = ctypes.c_float
_libm.logf.argtypes = [ctypes.c_float]


def head_bias(good):
    """mel_head.bias: -200 everywhere except the good tokens ({token: value})."""
    b = np.full(MEL, BAD, np.float32)
    for t, v in good.items():
        b[t] = np.float32(v)
    return b


def log_softmax(logits):
    """gpt_sampling.cpp:207-210 in float32: peak, sequential sum of expf in index order, logf."""
    x = np.asarray(logits, np.float32)
    peak = np.float32(x.max())
    s = np.float32(0.0)
    for v in x:
        s = np.float32(s + np.float32(_libm.expf(np.float32(v - peak))))
    log_sum = np.float32(peak + np.float32(_libm.logf(s)))
    return (x - log_sum).astype(np.float32)


def good_counts_ok(n_good, n_good_nonstop, beams, steps, has_stop):
    """True when no step has more good candidates than beams (nothing good is pruned) and fewer
    good hypotheses can end in the stop token than there are beams (no early stop)."""
    unpruned = all(n_good_nonstop ** i * n_good <= beams for i in range(steps))
    stops = sum(n_good_nonstop ** i for i in range(steps)) if has_stop else 0
    return unpruned and stops < beams


def best(bias, processors, length_penalty, steps, good_tokens):
    """Best finished hypothesis (codes, eos, score) over every sequence of good tokens, and the
    runner-up's score.  processors(log_probs, history) -> processed float32 scores."""
    lp = log_softmax(bias)
    lpen = float(np.float32(length_penalty))
    out = []

    def rec(codes, score):
        i = len(codes)
        proc = processors(lp, [1, 8192] + codes).astype(np.float32) + np.float32(score)
        for tok in good_tokens:
            s = np.float32(proc[tok])
            if not np.isfinite(s):
                continue
            if tok == STOP:
                out.append((float(s) / float(i + 1) ** lpen, tuple(codes), True))
            elif i + 1 == steps:
                out.append((float(s) / float(i + 1) ** lpen, tuple(codes + [tok]), False))
            else:
                rec(codes + [tok], s)

    rec([], np.float32(0.0))
    out.sort(key=lambda r: -r[0])
    return out[0], (out[1][0] if len(out) > 1 else -np.inf)


CASES = [
    # (good {token: bias}, options, num_beams, max_tokens); every case meets good_counts_ok.
    # Two tokens, three steps: the winner is decided by the float rounding of sums that are
    # equal in exact arithmetic (the search and the enumeration add in the same order).
    ({17: -0.0904, 4001: 0.3605}, dict(do_sample=False, repetition_penalty=10.0, length_penalty=0.0), 10, 3),
    ({17: 0.8611, 4001: 0.5135}, dict(do_sample=True, seed=5, top_k=2, top_p=1.0, temperature=1.0, repetition_penalty=10.0,
                                      length_penalty=0.5), 8, 3),
    # The stop token among the good ones; the best hypothesis is not the one-beam greedy path.
    ({17: -0.4228, 4001: 1.0761, STOP: -0.3982}, dict(do_sample=False, repetition_penalty=10.0, length_penalty=-1.0), 7, 2),
    ({17: -0.2417, 4001: -0.2543, STOP: -0.4375}, dict(do_sample=False, repetition_penalty=1.5, length_penalty=-1.0), 6, 2),
    ({17: 1.7275, 4001: -0.5468, STOP: 1.8003}, dict(do_sample=True, seed=52, top_k=3, top_p=1.0, temperature=1.0,
                                                     repetition_penalty=1.5, length_penalty=2.0), 10, 2),
    ({17: 0.742, 4001: 0.2799, STOP: 1.6346}, dict(do_sample=True, seed=89, top_k=3, top_p=1.0, temperature=1.3,
                                                   repetition_penalty=3.0, length_penalty=2.0), 10, 2),
    # One token and the stop token over five steps: where to stop, under penalty and length penalty.
    ({17: 0.7555, STOP: 0.4139}, dict(do_sample=False, repetition_penalty=1.2, length_penalty=0.5), 10, 5),
    ({17: 1.1209, STOP: 0.1227}, dict(do_sample=False, repetition_penalty=3.0, length_penalty=1.0), 6, 5),
    ({17: 1.0484, STOP: 1.4602}, dict(do_sample=False, repetition_penalty=3.0, length_penalty=3.0), 9, 5),
    ({17: 1.3611, STOP: 1.3698}, dict(do_sample=True, seed=61, top_k=2, top_p=1.0, temperature=1.0, repetition_penalty=2.0,
                                      length_penalty=3.0), 10, 5),
]


def case_tokens(good):
    """(sorted good tokens, how many, how many of them are not the stop token)"""
    n_good = len(good)
    return sorted(good), n_good, n_good - (1 if STOP in good else 0)

