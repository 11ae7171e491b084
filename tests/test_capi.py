"""The C-ABI library loads and exports every entry point include/*.h declares (CPU only:
no compute call is made)."""
import ctypes
import re
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = "".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    return sorted(set(re.findall(r"\b(itts_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(itts):
    lib = ctypes.CDLL(str(itts.LIB_PATH))
    names = declared_symbols()
    assert len(names) >= 19
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_options_defaults_match_reference(itts):
    # GenerationOptions defaults (include/itts25/gpt.hpp:7-16).
    o = itts._Options()
    itts._lib.itts_gen_options_default(ctypes.byref(o))
    assert (o.do_sample, o.seed, o.top_k, o.num_beams) == (1, 20261002, 30, 1)
    assert (o.temperature, o.top_p, o.repetition_penalty, o.length_penalty) == (np.float32(0.8), np.float32(0.8), 10.0, 0.0)
    d = itts.GenerationOptions()
    assert (d.do_sample, d.seed, d.top_k, d.num_beams) == (True, 20261002, 30, 1)


def test_synthetic_normal_is_deterministic_and_normal(itts):
    a = itts.synthetic_normal(200_000, 7)
    b = itts.synthetic_normal(200_000, 7)
    assert np.array_equal(a, b)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    c = itts.synthetic_normal(1000, 8, mean=2.0, std=0.5)
    assert abs(c.mean() - 2.0) < 0.1


def test_c_abi_struct_layouts(itts):
    assert ctypes.sizeof(itts._Options) == 48
    assert ctypes.sizeof(itts._Tensor) == 56
    assert ctypes.sizeof(itts._Config) == 16
