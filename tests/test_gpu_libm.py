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
