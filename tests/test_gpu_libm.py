"""The device expf / exp / logf of the sampler and beam kernels against glibc (MI355X).

The reference's sampler feeds libm results straight into its decisions (gpt_sampling.cpp:96,
:144, :207-210); the device restates glibc 2.35's routines (csrc/glibc_math.h).  Here every
float input the sampler can give them is run through the device (itts_libm_eval, the same
inline functions the kernels call) and compared bit for bit with glibc on the host
(oracle.libm_eval): expf and exp on every negative float (exp(x - max) with x <= max, including
the range where the result underflows to 0), logf on every float in [1, 8194] (the beam softmax
sum), plus a strided sweep of all float bit patterns for each.  Mismatches found: printed, and
must be 0.
"""
import ctypes
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CHUNK = 1 << 26


def _bits(f):
    return struct.unpack("<I", struct.pack("<f", f))[0]


def _device(itts, fn, first, stride, count):
    out = np.empty(count, np.float64 if fn == 1 else np.float32)
    st = itts._lib.itts_libm_eval(fn, first, stride, count, out.ctypes.data_as(ctypes.c_void_p))
    assert st == 0
    return out


def _compare(itts, oracle, fn, first, stride, total):
    bad = checked = 0
    for c0 in range(0, total, CHUNK):
        n = min(CHUNK, total - c0)
        start = first + c0 * stride
        d = _device(itts, fn, start, stride, n)
        h = oracle.libm_eval(fn, start, stride, n)
        iv = np.uint64 if fn == 1 else np.uint32
        differ = d.view(iv) != h.view(iv)
        differ &= ~(np.isnan(d) & np.isnan(h))  # NaN results agree whatever their bits
        bad += int(np.count_nonzero(differ))
        checked += n
    return checked, bad


@pytest.mark.parametrize("fn,name", [(0, "expf"), (1, "exp")])
def test_every_negative_float(itts, oracle, fn, name):
    first = 0x80000000
    total = 0xff800000 - first + 1  # -0 .. -inf
    checked, bad = _compare(itts, oracle, fn, first, 1, total)
    print(f"{name}: {bad} of {checked} negative floats differ from glibc", flush=True)
    assert bad == 0


def test_logf_sum_range(itts, oracle):
    first = _bits(1.0)
    total = _bits(8194.0) - first + 1
    checked, bad = _compare(itts, oracle, 2, first, 1, total)
    print(f"logf: {bad} of {checked} floats in [1, 8194] differ from glibc", flush=True)
    assert bad == 0


@pytest.mark.parametrize("fn,name", [(0, "expf"), (1, "exp"), (2, "logf")])
def test_strided_all_bit_patterns(itts, oracle, fn, name):
    checked, bad = _compare(itts, oracle, fn, 0, 61, (1 << 32) // 61)
    print(f"{name}: {bad} of {checked} strided bit patterns differ from glibc", flush=True)
    assert bad == 0


def _chain_rows(seed):
    """Rows of 8194 non-negative floats: exp(x - max) of logit rows of several spreads, masked
    and tied logits, all-equal rows, sums that start subnormal, tie-heavy sequences of
    short-mantissa powers of two (which put exact halves of the running sum's unit in play),
    and rows holding NaN or +inf (the chain then ends NaN, or +inf with no NaN after it)."""
    rng = np.random.default_rng(seed)
    rows = []
    for sd in (0.5, 1.0, 3.0, 10.0, 40.0):
        x = rng.standard_normal(8194) * sd
        rows.append(x)
        rows.append(np.round(x * 4) / 4)
        m = x.copy()
        m[rng.random(8194) < 0.4] = -np.inf
        rows.append(m)
    rows.append(np.zeros(8194))
    rows.append(-100.0 + rng.standard_normal(8194))
    out = []
    for x in rows:
        x = x.astype(np.float32)
        out.append(np.exp(x - x.max()).astype(np.float32))
    tiny = out[-1].copy()
    tiny[4000] = 1.0
    out.append(tiny)
    # subnormal exponentials: a running sum that stays below 2^-126 for 8000 values
    for lo in (-95.0, -101.0):
        x = (lo + rng.standard_normal(8194) * 0.5).astype(np.float32)
        x[8000] = 0.0
        e = np.exp(x.astype(np.float64)).astype(np.float32)
        assert np.count_nonzero((e > 0) & (e < np.finfo(np.float32).tiny)) > 4000
        out.append(e)
    for _ in range(12):
        ex = -rng.integers(0, 40, 8194)
        v = np.ldexp(1.0 + rng.integers(0, 4, 8194) * 0.25, ex).astype(np.float32)
        v[rng.random(8194) < 0.2] = 0.0
        out.append(v)
    # a NaN in the first, a middle and the last chunk; +inf alone, and +inf then a later NaN
    base = out[3]
    for idx in (5, 4100, 8193):
        v = base.copy()
        v[idx] = np.nan
        out.append(v)
    v = base.copy()
    v[3000] = np.inf
    out.append(v)
    v = v.copy()
    v[7000] = np.nan
    out.append(v)
    return np.stack(out)


def test_beam_softmax_sum_is_the_index_order_chain(itts):
    """The beam scores' log-softmax denominator (gpt_sampling.cpp:208: sum += exp(value - peak)
    in index order, float) is formed on the device without 8194 dependent additions
    (csrc/chain_sum.h).  It must equal the one-at-a-time float chain bit for bit; the chain is
    numpy's sequential float32 accumulate, itself checked against a Python loop on one row."""
    vals = _chain_rows(5)
    exp = np.add.accumulate(vals, axis=1, dtype=np.float32)[:, -1]
    s = np.float32(0.0)
    for v in vals[7]:
        s = np.float32(s + v)
    assert s.view(np.uint32) == exp[7].view(np.uint32)
    got = np.empty(len(vals), np.float32)
    v = np.ascontiguousarray(vals)
    st = itts._lib.itts_chain_sum_eval(v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(vals),
                                       got.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    assert st == 0
    nan = np.isnan(exp)
    assert nan.sum() == 4 and np.array_equal(np.isnan(got), nan), "NaN rows: the chain stays NaN"
    got[nan] = exp[nan] = 0.0
    bad = np.nonzero(got.view(np.uint32) != exp.view(np.uint32))[0]
    print(f"chain sum: {len(bad)} of {len(vals)} rows differ", flush=True)
    assert len(bad) == 0, [(int(i), float(got[i]), float(exp[i])) for i in bad[:5]]
