"""The sampler's libm, restated in index-tts-25-metal_amd/csrc/glibc_math.h, against glibc (CPU).

The reference's sampler (src/gpt_sampling.cpp) calls expf and logf in the beam log-softmax
(:207-210) and exp on float-valued doubles for the top-p and draw probabilities (:96, :144).
Built for x86-64 (the oracle, oracle/_ref) these are glibc 2.35's.  The device copies must give
the same bits, so they are compared with glibc here on strided sweeps of all 2^32 float bit
patterns and on every float of the ranges the sampler feeds them: expf and exp on every
negative float above -104 (exp(x - max) with x <= max), logf on every float in [1, 8194]
(the beam softmax sum: 1 <= sum <= 8194).  tests/test_gpu_libm.py runs the same inputs through
the device.  The tables are also recomputed from the mathematics.
"""
import shutil
import struct
import subprocess
from decimal import Decimal, getcontext
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HDR = ROOT / "index-tts-25-metal_amd" / "csrc" / "glibc_math.h"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("libm") / "libm_repro_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fopenmp", f"-I{HDR.parent}",
                    str(Path(__file__).with_name("libm_repro_check.cpp")), "-o", str(exe), "-lm"], check=True)

    def run(fn, first, stride, count):
        out = subprocess.run([str(exe), str(fn), str(first), str(stride), str(count)], check=True, capture_output=True,
                             text=True).stdout.split()
        return int(out[0]), int(out[1])

    return run


def _bits(f):
    return struct.unpack("<I", struct.pack("<f", f))[0]


@pytest.mark.parametrize("fn", [0, 1, 2], ids=["expf", "exp", "logf"])
def test_strided_sweep_of_all_floats(checker, fn):
    checked, bad = checker(fn, 0, 97, (1 << 32) // 97)
    assert checked > 40_000_000 and bad == 0


@pytest.mark.parametrize("fn", [0, 1], ids=["expf", "exp"])
def test_every_negative_float_above_minus_104(checker, fn):
    first = 0x80000000
    count = _bits(-104.0) - first + 1
    checked, bad = checker(fn, first, 1, count)
    assert checked == count and bad == 0


def test_logf_every_float_in_1_to_8194(checker):
    first = _bits(1.0)
    count = _bits(8194.0) - first + 1
    checked, bad = checker(2, first, 1, count)
    assert checked == count and bad == 0


def test_exp_tables_are_the_correctly_rounded_powers_of_two():
    """kExpfTab[i] = bits(2^(i/32)) - (i << 47); kExpTab = {bits(tail), bits(scale) - (i << 45)}
    with scale = 2^(i/128) rounded to double and tail = (2^(i/128) - scale) / scale rounded."""
    import re

    text = HDR.read_text()
    getcontext().prec = 80

    def table(name):
        body = re.search(name + r"\[[^\]]*\] = \{(.*?)\};", text, re.S).group(1)
        return [int(x, 16) for x in re.findall(r"0x[0-9a-f]{16}", body)]

    dbits = lambda x: struct.unpack("<Q", struct.pack("<d", x))[0]
    t32 = table("kExpfTab")
    assert len(t32) == 32
    for i, v in enumerate(t32):
        assert v == dbits(float(Decimal(2) ** (Decimal(i) / 32))) - (i << 47)
    t128 = table("kExpTab")
    assert len(t128) == 256
    for i in range(128):
        exact = Decimal(2) ** (Decimal(i) / 128)
        scale = float(exact)
        assert t128[2 * i + 1] == (dbits(scale) - (i << 45)) % (1 << 64)
        assert t128[2 * i] == dbits(float((exact - Decimal(scale)) / Decimal(scale)))
