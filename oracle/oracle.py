"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of the reference's own
sampler compiled from its sources (oracle/_ref/ref_sampling).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the CPU
baseline leg of bench.py, which compare the HIP path against it.  See gpt_oracle.h for
what each function restates and what pins it.
"""
from __future__ import annotations

import ctypes as C
import struct
import subprocess
from pathlib import Path
from typing import Dict, List, Sequence, Tuple

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_SAMPLING = HERE / "_ref" / "ref_sampling"
WIDTH = 1280
MEL_VOCAB = 8194


class _T(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.c_void_p), ("shape", C.c_int64 * 4), ("ndim", C.c_int32), ("_pad", C.c_int32)]


class _O(C.Structure):
    _fields_ = [
        ("do_sample", C.c_int32), ("_pad0", C.c_uint32), ("seed", C.c_uint64), ("temperature", C.c_float),
        ("top_k", C.c_uint32), ("top_p", C.c_float), ("repetition_penalty", C.c_float), ("num_beams", C.c_uint32),
        ("length_penalty", C.c_float), ("suppress_stop", C.c_uint32), ("_pad1", C.c_uint32),
    ]


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        build()
    lib = C.CDLL(str(LIB_PATH))
    P, u32, f32p, u32p = C.c_void_p, C.c_uint32, C.POINTER(C.c_float), C.POINTER(C.c_uint32)
    sig = {
        "orc_create": (P, [C.POINTER(_T), C.c_int32, u32, C.c_char_p, C.c_size_t]),
        "orc_destroy": (None, [P]),
        "orc_width": (u32, [P]),
        "orc_cached_tokens": (u32, [P]),
        "orc_prepare_ref": (C.c_int, [P, f32p, f32p, u32p, u32, u32, f32p, u32p]),
        "orc_prepare_cond": (C.c_int, [P, f32p, u32, u32p, u32, u32, f32p, u32p]),
        "orc_prefill": (C.c_int, [P, f32p, u32, f32p]),
        "orc_step": (C.c_int, [P, u32, u32, f32p]),
        "orc_kv_row": (C.c_int, [P, u32, C.c_int32, u32, f32p]),
        "orc_checkpoint": (P, [P]),
        "orc_restore": (C.c_int, [P, P]),
        "orc_state_free": (None, [P]),
        "orc_processors": (C.c_int, [f32p, u32, u32p, u32, C.POINTER(_O), f32p]),
        "orc_sample": (C.c_int, [f32p, u32, C.POINTER(C.c_uint64), u32p]),
        "orc_splitmix_next": (C.c_uint64, [C.POINTER(C.c_uint64)]),
        "orc_splitmix_unit": (C.c_double, [C.POINTER(C.c_uint64)]),
        "orc_generate": (C.c_int, [P, f32p, u32, C.POINTER(_O), u32, u32p, u32p, C.POINTER(C.c_int32)]),
        "orc_gelu": (C.c_float, [C.c_float]),
        "orc_libm_eval": (None, [C.c_int32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p]),
        "orc_layernorm": (None, [f32p, f32p, f32p, u32, C.c_float, f32p]),
        "orc_last_error": (C.c_char_p, []),
        "orc_qwen_create": (P, [C.POINTER(_T), C.c_int32, u32, C.c_char_p, C.c_size_t]),
        "orc_qwen_destroy": (None, [P]),
        "orc_qwen_cached": (u32, [P]),
        "orc_qwen_prefill": (C.c_int, [P, u32p, u32, f32p]),
        "orc_qwen_step": (C.c_int, [P, u32, f32p]),
        "orc_qwen_generate": (C.c_int, [P, u32p, u32, u32, u32p, u32p]),
        "orc_qwen_kv_row": (C.c_int, [P, u32, C.c_int32, u32, f32p]),
        "orc_qwen_set_mutation": (None, [P, C.c_int32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _up(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


class OracleError(Exception):
    def __init__(self, status: int, msg: str):
        super().__init__(msg)
        self.status = status  # -1 invalid_argument, -2 runtime_error, -3 other


def _check(st: int) -> None:
    if st != 0:
        raise OracleError(st, _lib.orc_last_error().decode())


def options(do_sample=True, seed=20261002, temperature=0.8, top_k=30, top_p=0.8, repetition_penalty=10.0, num_beams=1,
            length_penalty=0.0, suppress_stop=False) -> _O:
    return _O(int(bool(do_sample)), 0, int(seed) & (2**64 - 1), temperature, int(top_k), top_p, repetition_penalty,
              int(num_beams), length_penalty, int(bool(suppress_stop)), 0)


def options_from(o) -> _O:
    """Convert an itts_gpt.GenerationOptions (same fields) to the oracle struct."""
    return options(o.do_sample, o.seed, o.temperature, o.top_k, o.top_p, o.repetition_penalty, o.num_beams,
                   o.length_penalty, o.suppress_stop)


class OracleState:
    """A KV snapshot (gpt.cpp:86-87) of an OracleGpt."""

    def __init__(self, h):
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None):
            _lib.orc_state_free(self._h)
            self._h = None


class OracleGpt:
    def __init__(self, weights: Dict[str, np.ndarray], kv_capacity: int = 4096):
        self._keep = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}
        ts = []
        for name, a in self._keep.items():
            shape = (C.c_int64 * 4)(*(list(a.shape) + [0] * (4 - a.ndim)))
            ts.append(_T(name.encode(), a.ctypes.data, shape, a.ndim, 0))
        arr = (_T * len(ts))(*ts)
        err = C.create_string_buffer(512)
        self._h = _lib.orc_create(arr, len(ts), kv_capacity, err, 512)
        if not self._h:
            raise OracleError(-2, err.value.decode())
        self.width = int(_lib.orc_width(self._h))

    def __del__(self):
        if getattr(self, "_h", None):
            _lib.orc_destroy(self._h)
            self._h = None

    def cached_tokens(self) -> int:
        return int(_lib.orc_cached_tokens(self._h))

    def prepare_cond(self, cond: np.ndarray, text: Sequence[int], language: int) -> np.ndarray:
        cd = np.ascontiguousarray(cond, dtype=np.float32).reshape(-1, self.width)
        ids = np.ascontiguousarray(np.asarray(text, dtype=np.uint32))
        out = np.zeros((cd.shape[0] + len(ids) + 3, self.width), np.float32)
        rows = C.c_uint32()
        _check(_lib.orc_prepare_cond(self._h, _fp(cd), cd.shape[0], _up(ids), len(ids), language, _fp(out), C.byref(rows)))
        return out[: rows.value].reshape(-1)

    def prepare(self, speaker, emotion, text, language) -> np.ndarray:
        sp = np.ascontiguousarray(speaker, dtype=np.float32)
        em = np.ascontiguousarray(emotion, dtype=np.float32)
        ids = np.ascontiguousarray(np.asarray(text, dtype=np.uint32))
        out = np.zeros((3 + len(ids) + 3, self.width), np.float32)
        rows = C.c_uint32()
        _check(_lib.orc_prepare_ref(self._h, _fp(sp), _fp(em), _up(ids), len(ids), language, _fp(out), C.byref(rows)))
        return out[: rows.value].reshape(-1)

    def prefill(self, prefix: np.ndarray) -> np.ndarray:
        p = np.ascontiguousarray(prefix, dtype=np.float32).reshape(-1)
        out = np.empty(MEL_VOCAB, np.float32)
        _check(_lib.orc_prefill(self._h, _fp(p), p.size // self.width, _fp(out)))
        return out

    def step(self, code: int, position: int) -> np.ndarray:
        out = np.empty(MEL_VOCAB, np.float32)
        _check(_lib.orc_step(self._h, int(code) & 0xFFFFFFFF, int(position) & 0xFFFFFFFF, _fp(out)))
        return out

    def checkpoint(self) -> "OracleState":
        h = _lib.orc_checkpoint(self._h)
        if not h:
            raise OracleError(-1, _lib.orc_last_error().decode())
        return OracleState(h)

    def restore(self, state: "OracleState") -> None:
        _check(_lib.orc_restore(self._h, state._h))

    def kv_row(self, layer: int, is_v: bool, pos: int) -> np.ndarray:
        out = np.empty(self.width, np.float32)
        _check(_lib.orc_kv_row(self._h, layer, int(is_v), pos, _fp(out)))
        return out

    def generate(self, prefix: np.ndarray, opt: _O, max_tokens: int) -> Tuple[List[int], bool]:
        p = np.ascontiguousarray(prefix, dtype=np.float32).reshape(-1)
        codes = np.zeros(max(1, max_tokens), np.uint32)
        n = C.c_uint32()
        stopped = C.c_int32()
        _check(_lib.orc_generate(self._h, _fp(p), p.size // self.width, C.byref(opt), max_tokens, _up(codes), C.byref(n),
                                 C.byref(stopped)))
        return [int(c) for c in codes[: n.value]], bool(stopped.value)


QWEN_VOCAB = 151936
QWEN_EOS = 151643


class OracleQwen:
    """FP32 CPU restatement of itts25::QwenDecoder (src/qwen.cpp:5-49); see qwen_oracle.h."""

    def __init__(self, weights: Dict[str, np.ndarray], layers: int = 28):
        ts = []
        for name, a in weights.items():
            a = np.ascontiguousarray(a, dtype=np.float32)
            shape = (C.c_int64 * 4)(*(list(a.shape) + [0] * (4 - a.ndim)))
            ts.append((_T(name.encode(), a.ctypes.data, shape, a.ndim, 0), a))
        arr = (_T * len(ts))(*[t for t, _ in ts])
        err = C.create_string_buffer(512)
        self._h = _lib.orc_qwen_create(arr, len(ts), layers, err, 512)  # copies the tensors
        if not self._h:
            raise OracleError(-2, err.value.decode())

    def __del__(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.orc_qwen_destroy(self._h)
            self._h = None

    @property
    def cached(self) -> int:
        return int(_lib.orc_qwen_cached(self._h))

    def set_mutation(self, mutation: int) -> None:
        _lib.orc_qwen_set_mutation(self._h, int(mutation))

    def prefill(self, ids: Sequence[int]) -> np.ndarray:
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(QWEN_VOCAB, np.float32)
        _check(_lib.orc_qwen_prefill(self._h, _up(a), a.size, _fp(out)))
        return out

    def step(self, token: int) -> np.ndarray:
        out = np.empty(QWEN_VOCAB, np.float32)
        _check(_lib.orc_qwen_step(self._h, int(token) & 0xFFFFFFFF, _fp(out)))
        return out

    def generate(self, ids: Sequence[int], maximum: int = 1024) -> Tuple[List[int], bool]:
        """(tokens, reached EOS): the tokens produced also when the reference would throw
        "Qwen did not reach EOS within 1024 generated tokens"."""
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros(max(1, maximum), np.uint32)
        n = C.c_uint32(0)
        st = _lib.orc_qwen_generate(self._h, _up(a), a.size, int(maximum) & 0xFFFFFFFF, _up(out), C.byref(n))
        toks = [int(x) for x in out[: n.value]]
        if st == -2 and _lib.orc_last_error().decode() == "Qwen did not reach EOS within 1024 generated tokens":
            return toks, False
        _check(st)
        return toks, True

    def kv_row(self, layer: int, is_v: bool, pos: int) -> np.ndarray:
        out = np.empty(1024, np.float32)
        _check(_lib.orc_qwen_kv_row(self._h, layer, int(is_v), pos, _fp(out)))
        return out


def processors(logits: np.ndarray, history: Sequence[int], opt: _O) -> np.ndarray:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(np.asarray(history, dtype=np.uint32))
    out = np.empty_like(lg)
    _check(_lib.orc_processors(_fp(lg), lg.size, _up(h), h.size, C.byref(opt), _fp(out)))
    return out


def sample(processed: np.ndarray, rng_state: int, draws: int = 1) -> Tuple[List[int], int]:
    p = np.ascontiguousarray(processed, dtype=np.float32)
    st = C.c_uint64(rng_state & (2**64 - 1))
    toks = []
    tok = C.c_uint32()
    for _ in range(draws):
        _check(_lib.orc_sample(_fp(p), p.size, C.byref(st), C.byref(tok)))
        toks.append(int(tok.value))
    return toks, int(st.value)


def splitmix_sequence(seed: int, n: int) -> List[int]:
    st = C.c_uint64(seed & (2**64 - 1))
    return [int(_lib.orc_splitmix_next(C.byref(st))) for _ in range(n)]


def libm_eval(fn: int, first: int, stride: int, count: int) -> np.ndarray:
    """glibc's expf (0), exp of the float widened (1) or logf (2) on the floats with bit patterns
    first + i * stride."""
    out = np.empty(count, np.float64 if fn == 1 else np.float32)
    _lib.orc_libm_eval(fn, first, stride, count, out.ctypes.data)
    return out


def gelu(v: float) -> float:
    return float(_lib.orc_gelu(v))


def layernorm(x: np.ndarray, g: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    _lib.orc_layernorm(_fp(x), _fp(np.ascontiguousarray(g, np.float32)), _fp(np.ascontiguousarray(b, np.float32)), x.size, eps,
                       _fp(out))
    return out


# ---------------------------------------------------------------- reference sampler (oracle/_ref)

def ref_available() -> bool:
    return REF_SAMPLING.exists()


class RefSampler:
    """Pipe to the reference's own apply_gpt_sampling_processors / sample_gpt_token_from_logits."""

    def __init__(self):
        self.p = subprocess.Popen([str(REF_SAMPLING)], stdin=subprocess.PIPE, stdout=subprocess.PIPE)

    def close(self):
        if self.p:
            self.p.stdin.close()
            self.p.wait(timeout=10)
            self.p = None

    def _read(self, n: int) -> bytes:
        b = self.p.stdout.read(n)
        if len(b) != n:
            raise RuntimeError("reference sampler pipe closed")
        return b

    def _status(self):
        st = struct.unpack("<i", self._read(4))[0]
        if st != 0:
            ln = struct.unpack("<I", self._read(4))[0]
            return self._read(ln).decode()
        return None

    def processors(self, logits, history, temperature, top_k, top_p, penalty, beams):
        lg = np.ascontiguousarray(logits, np.float32)
        h = np.ascontiguousarray(np.asarray(history, np.uint32))
        self.p.stdin.write(struct.pack("<IIIfIffI", 1, lg.size, h.size, temperature, top_k, top_p, penalty, beams))
        self.p.stdin.write(lg.tobytes())
        self.p.stdin.write(h.tobytes())
        self.p.stdin.flush()
        err = self._status()
        if err is not None:
            return err
        return np.frombuffer(self._read(4 * lg.size), np.float32).copy()

    def sample(self, processed, seed: int, draws: int):
        p = np.ascontiguousarray(processed, np.float32)
        self.p.stdin.write(struct.pack("<IIQI", 2, p.size, seed & (2**64 - 1), draws))
        self.p.stdin.write(p.tobytes())
        self.p.stdin.flush()
        err = self._status()
        if err is not None:
            return err
        toks = list(np.frombuffer(self._read(4 * draws), np.uint32))
        state = struct.unpack("<Q", self._read(8))[0]
        return [int(t) for t in toks], state
