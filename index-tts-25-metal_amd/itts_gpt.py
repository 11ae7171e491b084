"""Python binding of the MI355X-native IndexTTS 2.5 GPT semantic-token loop.

Mirrors the reference's C++ interface (include/itts25/gpt.hpp:7-43):

    GenerationOptions, GenerationResult, GptState, GptDecoder
        .prepare(speaker, emotion, text, language)    gpt.cpp:42-71
        .prefill(prefix)                              gpt.cpp:72-78
        .step(code, position)                         gpt.cpp:79-85
        .generate(prefix, options, max_tokens=1500)   gpt_sampling.cpp:168-245
        .checkpoint() / .restore(state)               gpt.cpp:86-87
        .cached_tokens()
    apply_gpt_sampling_processors(logits, history, options)   gpt_sampling.cpp:28-128

Everything runs through the C ABI of libitts_gpt.so (include/itts_gpt.h); there is
no CPU path.  The reference's exception kinds map to InvalidArgument (a ValueError,
std::invalid_argument), GptRuntimeError (a RuntimeError, std::runtime_error) and
LogicError (std::logic_error), with the reference's messages.
"""
from __future__ import annotations

import ctypes as C
import os
import zlib
from dataclasses import dataclass, field
from pathlib import Path
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libitts_gpt.so"

WIDTH = 1280
HEADS = 20
FFN = 5120
MEL_VOCAB = 8194
MEL_START = 8192
MEL_STOP = 8193


class InvalidArgument(ValueError):
    """std::invalid_argument in the reference."""


class GptRuntimeError(RuntimeError):
    """std::runtime_error in the reference."""


class LogicError(Exception):
    """std::logic_error in the reference."""


class _Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.c_void_p), ("shape", C.c_int64 * 4), ("ndim", C.c_int32), ("_pad", C.c_int32)]


class _Config(C.Structure):
    _fields_ = [("kv_capacity", C.c_uint32), ("max_batch", C.c_uint32), ("weight_dtype", C.c_uint32), ("flags", C.c_uint32)]


class _Options(C.Structure):
    _fields_ = [
        ("do_sample", C.c_int32), ("_pad0", C.c_uint32), ("seed", C.c_uint64), ("temperature", C.c_float),
        ("top_k", C.c_uint32), ("top_p", C.c_float), ("repetition_penalty", C.c_float), ("num_beams", C.c_uint32),
        ("length_penalty", C.c_float), ("suppress_stop", C.c_uint32), ("_pad1", C.c_uint32),
    ]


class _BundleTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.c_void_p), ("shape", C.c_int64 * 8), ("ndim", C.c_int32), ("dtype", C.c_uint32),
                ("offset", C.c_uint64), ("nbytes", C.c_uint64)]


class _Timing(C.Structure):
    _fields_ = [("prefill_ms", C.c_float), ("decode_ms", C.c_float), ("decode_steps", C.c_uint32), ("decode_path", C.c_uint32)]


class _QwenConfig(C.Structure):
    _fields_ = [("layers", C.c_uint32), ("flags", C.c_uint32)]


def _load() -> C.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"HIP extension not built: {LIB_PATH} is missing (run index-tts-25-metal_amd/build.py)")
    lib = C.CDLL(str(LIB_PATH))
    P = C.c_void_p
    u32, i32, f32p, u32p = C.c_uint32, C.c_int32, C.POINTER(C.c_float), C.POINTER(C.c_uint32)
    sig = {
        "itts_gen_options_default": (None, [C.POINTER(_Options)]),
        "itts_gpt_create": (C.c_int, [C.POINTER(_Tensor), i32, C.POINTER(_Config), C.POINTER(P)]),
        "itts_gpt_destroy": (None, [P]),
        "itts_gpt_last_error": (C.c_char_p, [P]),
        "itts_gpt_prepare": (C.c_int, [P, f32p, f32p, u32p, u32, u32, f32p, u32, u32p]),
        "itts_gpt_prepare_cond": (C.c_int, [P, f32p, u32, u32p, u32, u32, f32p, u32, u32p]),
        "itts_gpt_prefill": (C.c_int, [P, f32p, u32, f32p]),
        "itts_gpt_step": (C.c_int, [P, u32, u32, f32p]),
        "itts_gpt_cached_tokens": (u32, [P]),
        "itts_gpt_checkpoint": (C.c_int, [P, C.POINTER(P)]),
        "itts_gpt_restore": (C.c_int, [P, P]),
        "itts_gpt_state_tokens": (u32, [P]),
        "itts_gpt_state_release": (None, [P]),
        "itts_gpt_generate": (C.c_int, [P, f32p, u32, C.POINTER(_Options), u32, u32p, u32p, C.POINTER(i32)]),
        "itts_gpt_generate_noalloc": (C.c_int, [P, f32p, u32, C.POINTER(_Options), u32, u32p, u32p, C.POINTER(i32)]),
        "itts_gpt_alloc_events": (C.c_uint64, []),
        "itts_gpt_generate_batch": (C.c_int, [P, u32, C.POINTER(f32p), u32p, C.POINTER(_Options), u32, u32p, u32p, C.POINTER(i32)]),
        "itts_gpt_generate_segments": (C.c_int, [P, f32p, f32p, u32p, u32p, u32, u32, C.POINTER(_Options), u32, u32p, u32p,
                                                 C.POINTER(i32)]),
        "itts_gpt_generate_segments_cond": (C.c_int, [P, f32p, u32, u32p, u32p, u32, u32, C.POINTER(_Options), u32, u32p, u32p,
                                                      C.POINTER(i32)]),
        "itts_gpt_apply_processors": (C.c_int, [P, f32p, u32, u32p, u32, C.POINTER(_Options), f32p]),
        "itts_gpt_sample": (C.c_int, [P, f32p, u32, C.POINTER(C.c_uint64), u32, u32p]),
        "itts_gpt_last_timing": (C.c_int, [P, C.POINTER(_Timing)]),
        "itts_gpt_bench_kernel": (C.c_int, [P, i32, u32, u32, u32, C.POINTER(C.c_float), C.POINTER(C.c_double)]),
        "itts_gpt_step_phases": (C.c_int, [P, u32, u32, C.POINTER(C.c_float)]),
        "itts_gpt_step_phases_batch": (C.c_int, [P, u32, u32, u32, C.POINTER(C.c_float)]),
        "itts_synthetic_normal": (None, [f32p, C.c_size_t, C.c_uint64, C.c_float, C.c_float]),
        "itts_bundle_open": (C.c_int, [C.c_char_p, i32, C.POINTER(P)]),
        "itts_bundle_close": (None, [P]),
        "itts_bundle_last_error": (C.c_char_p, []),
        "itts_bundle_count": (i32, [P]),
        "itts_bundle_tensor_at": (C.c_int, [P, i32, C.POINTER(_BundleTensor)]),
        "itts_bundle_find": (C.c_int, [P, C.c_char_p, C.POINTER(_BundleTensor)]),
        "itts_gpt_create_from_bundle": (C.c_int, [P, C.POINTER(_Config), C.POINTER(P)]),
        "itts_codec_create": (C.c_int, [C.POINTER(_Tensor), i32, C.POINTER(P)]),
        "itts_codec_create_from_bundle": (C.c_int, [P, C.POINTER(P)]),
        "itts_codec_destroy": (None, [P]),
        "itts_codec_last_error": (C.c_char_p, [P]),
        "itts_codec_decode": (C.c_int, [P, u32p, u32, f32p]),
        "itts_codec_bench": (C.c_int, [P, u32, u32, C.POINTER(C.c_float), C.POINTER(C.c_double)]),
        "itts_libm_eval": (C.c_int, [i32, C.c_uint64, C.c_uint64, C.c_uint64, C.c_void_p]),
        "itts_chain_sum_eval": (C.c_int, [C.POINTER(C.c_float), u32, C.POINTER(C.c_float)]),
        "itts_qwen_create": (C.c_int, [C.POINTER(_Tensor), i32, C.POINTER(_QwenConfig), C.POINTER(P)]),
        "itts_qwen_create_from_bundle": (C.c_int, [P, C.POINTER(_QwenConfig), C.POINTER(P)]),
        "itts_qwen_destroy": (None, [P]),
        "itts_qwen_last_error": (C.c_char_p, [P]),
        "itts_qwen_prefill": (C.c_int, [P, u32p, u32, f32p]),
        "itts_qwen_step": (C.c_int, [P, u32, f32p]),
        "itts_qwen_generate": (C.c_int, [P, u32p, u32, u32, u32p, u32p]),
        "itts_qwen_submissions": (C.c_uint64, [P]),
        "itts_qwen_bench": (C.c_int, [P, u32, u32, u32, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()


def exported_symbols() -> List[str]:
    """Names of the C ABI entry points bound here (all declared in include/itts_gpt.h)."""
    return [n for n in dir(_lib) if n.startswith("itts_")]


def _fp(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _up(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


@dataclass
class GenerationOptions:
    """itts25::GenerationOptions (gpt.hpp:7-16) plus suppress_stop (fixed-length runs)."""

    do_sample: bool = True
    seed: int = 20261002
    temperature: float = 0.8
    top_k: int = 30
    top_p: float = 0.8
    repetition_penalty: float = 10.0
    num_beams: int = 1
    length_penalty: float = 0.0
    suppress_stop: bool = False

    def _c(self) -> _Options:
        return _Options(int(bool(self.do_sample)), 0, int(self.seed) & (2**64 - 1), float(self.temperature), int(self.top_k),
                        float(self.top_p), float(self.repetition_penalty), int(self.num_beams), float(self.length_penalty),
                        int(bool(self.suppress_stop)), 0)


@dataclass
class GenerationResult:
    codes: List[int] = field(default_factory=list)
    stopped: bool = False


class GptState:
    """Device snapshot of the cached KV rows (gpt.hpp:18)."""

    def __init__(self, ptr: int):
        self._ptr = C.c_void_p(ptr)
        self.tokens = int(_lib.itts_gpt_state_tokens(self._ptr))

    def __del__(self):
        if getattr(self, "_ptr", None) and self._ptr.value:
            _lib.itts_gpt_state_release(self._ptr)
            self._ptr = C.c_void_p()


def _raise(status: int, msg: str) -> None:
    if status == -1:
        raise InvalidArgument(msg)
    if status == -2:
        raise GptRuntimeError(msg)
    raise LogicError(msg)


_DTYPES = {0: ("f32", np.float32), 1: ("u32", np.uint32)}


class Bundle:
    """A MIT2 weight bundle (directory or single file), memory-mapped: the reference's
    mit2::Bundle (vendor/metal-runtime/bundle.cpp:150-293) with the checks of
    itts25::Weights (src/weights.cpp:9-49).  get/ids/info mirror Weights."""

    def __init__(self, path, require_model: bool = True):
        self._b = C.c_void_p()
        st = _lib.itts_bundle_open(str(path).encode(), 1 if require_model else 0, C.byref(self._b))
        if st != 0:
            _raise(st, _lib.itts_bundle_last_error().decode())
        self.path = str(path)

    def close(self) -> None:
        if self._b.value:
            _lib.itts_bundle_close(self._b)
            self._b = C.c_void_p()

    def __del__(self):
        self.close()

    def __len__(self) -> int:
        return int(_lib.itts_bundle_count(self._b))

    @staticmethod
    def _describe(t: "_BundleTensor") -> dict:
        return {"name": t.name.decode(), "shape": tuple(int(t.shape[i]) for i in range(t.ndim)), "dtype": _DTYPES[t.dtype][0],
                "offset": int(t.offset), "nbytes": int(t.nbytes)}

    def tensors(self) -> List[dict]:
        out = []
        for i in range(len(self)):
            t = _BundleTensor()
            st = _lib.itts_bundle_tensor_at(self._b, i, C.byref(t))
            if st != 0:
                _raise(st, _lib.itts_bundle_last_error().decode())
            out.append(self._describe(t))
        return out

    def _find(self, name: str) -> "_BundleTensor":
        t = _BundleTensor()
        st = _lib.itts_bundle_find(self._b, name.encode(), C.byref(t))
        if st != 0:
            _raise(st, _lib.itts_bundle_last_error().decode())
        return t

    def info(self, name: str) -> dict:
        return self._describe(self._find(name))

    def _array(self, name: str, want: int, what: str) -> np.ndarray:
        t = self._find(name)
        if t.dtype != want:
            raise GptRuntimeError(f"Expected {what}: {name}")
        dt = _DTYPES[t.dtype][1]
        buf = (C.c_char * int(t.nbytes)).from_address(t.data)
        a = np.frombuffer(buf, dtype=dt).copy()  # the mapping closes with the bundle
        return a.reshape(tuple(int(t.shape[i]) for i in range(t.ndim)))

    def get(self, name: str) -> np.ndarray:
        """Weights::get (weights.cpp:34-42): a float32 tensor."""
        return self._array(name, 0, "float32")

    def ids(self, name: str) -> np.ndarray:
        """Weights::ids (weights.cpp:43-48): a uint32 tensor."""
        return self._array(name, 1, "uint32")


def write_mit2_bundle(path, tensors: Dict[str, np.ndarray], single_file: bool = False, alignment: int = 4096,
                      target: str = "index-tts2.5", weights_file: str = "weights.bin") -> Path:
    """Writes tensors (float32 or uint32 arrays) as a MIT2 bundle: a directory with
    manifest.json + weights_file, or one file with the manifest and the "MIT2VOIC" footer
    appended.  Offsets are multiples of `alignment`; the stream starts with the 12-byte
    header "MIT2", version 1, alignment."""
    import hashlib
    import json
    import struct

    path = Path(path)
    records, blobs, pos = [], [], 12
    for name, arr in tensors.items():
        a = np.ascontiguousarray(arr)
        if a.dtype == np.float32:
            dtype = "f32"
        elif a.dtype == np.uint32:
            dtype = "u32"
        else:
            raise InvalidArgument(f"Unsupported bundle dtype {a.dtype}: {name}")
        pos = (pos + alignment - 1) // alignment * alignment
        data = a.tobytes()
        records.append({"name": name, "shape": list(a.shape), "dtype": dtype, "offset": pos, "nbytes": len(data),
                        "sha256": hashlib.sha256(data).hexdigest(), "layout": "row_major", "component": "gpt"})
        blobs.append((pos, data))
        pos += len(data)
    manifest = {"format": "MIT2", "version": 1, "alignment": alignment, "endianness": "little", "weights_file": weights_file,
                "metadata": {"target": target, "kind": "model"}, "tensors": records}
    text = json.dumps(manifest).encode()

    def write_stream(f) -> int:
        f.write(b"MIT2" + struct.pack("<II", 1, alignment))
        for off, data in blobs:
            f.seek(off)
            f.write(data)
        return max([12] + [off + len(d) for off, d in blobs])

    if single_file:
        with open(path, "wb") as f:
            end = write_stream(f)
            f.seek(end)
            f.write(text)
            f.write(struct.pack("<QQ", end, len(text)) + b"MIT2VOIC")
    else:
        path.mkdir(parents=True, exist_ok=True)
        with open(path / weights_file, "wb") as f:
            write_stream(f)
        (path / "manifest.json").write_bytes(text)
    return path


class GptDecoder:
    """itts25::GptDecoder on one MI355X (gpt.hpp:22-43)."""

    @classmethod
    def from_bundle(cls, bundle: "Bundle", kv_capacity: int = 4096, max_batch: int = 1, weight_dtype: str = "f32") -> "GptDecoder":
        """GptDecoder(Weights&, ...) on a MIT2 bundle: the GPT tensors go to the device
        straight from the bundle's mapping."""
        self = cls.__new__(cls)
        self._h = C.c_void_p()
        self._keep = []
        cfg = _Config(int(kv_capacity), int(max_batch), 1 if weight_dtype == "bf16" else 0, 0)
        st = _lib.itts_gpt_create_from_bundle(bundle._b, C.byref(cfg), C.byref(self._h))
        if st != 0:
            _raise(st, _lib.itts_gpt_last_error(None).decode())
        self.kv_capacity = int(kv_capacity)
        self.max_batch = int(max_batch)
        return self

    def __init__(self, weights: Optional[Dict[str, np.ndarray]], kv_capacity: int = 4096, max_batch: int = 1,
                 weight_dtype: str = "f32"):
        self._h = C.c_void_p()
        self._keep = []
        tensors = []
        for name, arr in (weights or {}).items():
            a = np.ascontiguousarray(arr, dtype=np.float32)
            self._keep.append(a)
            shape = (C.c_int64 * 4)(*(list(a.shape) + [0] * (4 - a.ndim)))
            tensors.append(_Tensor(name.encode(), a.ctypes.data, shape, a.ndim, 0))
        arr_t = (_Tensor * max(1, len(tensors)))(*tensors)
        cfg = _Config(int(kv_capacity), int(max_batch), 1 if weight_dtype == "bf16" else 0, 0)
        st = _lib.itts_gpt_create(arr_t, len(tensors), C.byref(cfg), C.byref(self._h))
        self._keep = []  # weights live on the device now
        if st != 0:
            _raise(st, _lib.itts_gpt_last_error(None).decode())
        self.kv_capacity = int(kv_capacity)
        self.max_batch = int(max_batch)

    def close(self) -> None:
        if self._h.value:
            _lib.itts_gpt_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        self.close()

    def _check(self, st: int) -> None:
        if st != 0:
            _raise(st, _lib.itts_gpt_last_error(self._h).decode())

    # gpt.cpp:42-71
    def prepare(self, speaker: np.ndarray, emotion: np.ndarray, text: Sequence[int], language: int) -> np.ndarray:
        sp = np.ascontiguousarray(speaker, dtype=np.float32)
        em = np.ascontiguousarray(emotion, dtype=np.float32)
        if sp.size != 192 or em.size != WIDTH:
            raise InvalidArgument("Invalid GPT conditioning dimensions")
        ids = np.ascontiguousarray(np.asarray(text, dtype=np.uint32))
        cap = 3 + len(ids) + 3
        out = np.zeros((cap, WIDTH), np.float32)
        rows = C.c_uint32()
        self._check(_lib.itts_gpt_prepare(self._h, _fp(sp), _fp(em), _up(ids), len(ids), int(language), _fp(out), cap, C.byref(rows)))
        return out[: rows.value].reshape(-1)

    def prepare_cond(self, cond: np.ndarray, text: Sequence[int], language: int) -> np.ndarray:
        """prepare() with the conditioning rows given directly (e.g. synthetic latents)."""
        cd = np.ascontiguousarray(cond, dtype=np.float32).reshape(-1, WIDTH)
        ids = np.ascontiguousarray(np.asarray(text, dtype=np.uint32))
        cap = cd.shape[0] + len(ids) + 3
        out = np.zeros((cap, WIDTH), np.float32)
        rows = C.c_uint32()
        self._check(_lib.itts_gpt_prepare_cond(self._h, _fp(cd), cd.shape[0], _up(ids), len(ids), int(language), _fp(out), cap,
                                               C.byref(rows)))
        return out[: rows.value].reshape(-1)

    @staticmethod
    def _prefix(prefix: np.ndarray) -> np.ndarray:
        p = np.ascontiguousarray(prefix, dtype=np.float32).reshape(-1)
        if p.size == 0 or p.size % WIDTH:
            raise InvalidArgument("Invalid GPT prefill dimensions")
        return p

    def prefill(self, prefix: np.ndarray) -> np.ndarray:
        p = self._prefix(prefix)
        out = np.empty(MEL_VOCAB, np.float32)
        self._check(_lib.itts_gpt_prefill(self._h, _fp(p), p.size // WIDTH, _fp(out)))
        return out

    def step(self, code: int, position: int) -> np.ndarray:
        out = np.empty(MEL_VOCAB, np.float32)
        self._check(_lib.itts_gpt_step(self._h, int(code) & 0xFFFFFFFF, int(position) & 0xFFFFFFFF, _fp(out)))
        return out

    def generate(self, prefix: np.ndarray, options: GenerationOptions, max_tokens: int = 1500) -> GenerationResult:
        p = self._prefix(prefix)
        codes = np.zeros(max(1, int(max_tokens)), np.uint32)
        n = C.c_uint32()
        stopped = C.c_int32()
        o = options._c()
        self._check(_lib.itts_gpt_generate(self._h, _fp(p), p.size // WIDTH, C.byref(o), int(max_tokens), _up(codes), C.byref(n),
                                           C.byref(stopped)))
        return GenerationResult([int(c) for c in codes[: n.value]], bool(stopped.value))

    def generate_noalloc(self, prefix: np.ndarray, options: GenerationOptions, max_tokens: int = 1500) -> GenerationResult:
        """generate() through itts_gpt_generate_noalloc: no device allocation (prefix <= 512 rows, num_beams 1)."""
        p = self._prefix(prefix)
        codes = np.zeros(max(1, int(max_tokens)), np.uint32)
        n = C.c_uint32()
        stopped = C.c_int32()
        o = options._c()
        self._check(_lib.itts_gpt_generate_noalloc(self._h, _fp(p), p.size // WIDTH, C.byref(o), int(max_tokens), _up(codes),
                                                   C.byref(n), C.byref(stopped)))
        return GenerationResult([int(c) for c in codes[: n.value]], bool(stopped.value))

    def generate_batch(self, prefixes: Sequence[np.ndarray], options, max_tokens: int) -> List[GenerationResult]:
        ps = [self._prefix(p) for p in prefixes]
        B = len(ps)
        opts = list(options) if isinstance(options, (list, tuple)) else [options] * B
        ptrs = (C.POINTER(C.c_float) * B)(*[_fp(p) for p in ps])
        rows = np.array([p.size // WIDTH for p in ps], np.uint32)
        copts = (_Options * B)(*[o._c() for o in opts])
        codes = np.zeros((B, max(1, int(max_tokens))), np.uint32)
        n = np.zeros(B, np.uint32)
        stopped = np.zeros(B, np.int32)
        self._check(_lib.itts_gpt_generate_batch(self._h, B, ptrs, _up(rows), copts, int(max_tokens), _up(codes), _up(n),
                                                 stopped.ctypes.data_as(C.POINTER(C.c_int32))))
        return [GenerationResult([int(c) for c in codes[b, : n[b]]], bool(stopped[b])) for b in range(B)]

    @staticmethod
    def _segments(segments: Sequence[Sequence[int]]):
        counts = np.array([len(x) for x in segments], np.uint32)
        flat = np.concatenate([np.asarray(x, dtype=np.uint32).reshape(-1) for x in segments]) if len(segments) else \
            np.zeros(0, np.uint32)
        return np.ascontiguousarray(flat, dtype=np.uint32), counts

    def _segment_results(self, fn, args, nseg: int, options, max_tokens: int) -> List[GenerationResult]:
        codes = np.zeros((max(1, nseg), max(1, int(max_tokens))), np.uint32)
        n = np.zeros(max(1, nseg), np.uint32)
        stopped = np.zeros(max(1, nseg), np.int32)
        o = options._c()
        self._check(fn(self._h, *args, C.byref(o), int(max_tokens), _up(codes), _up(n), stopped.ctypes.data_as(C.POINTER(C.c_int32))))
        return [GenerationResult([int(c) for c in codes[i, : n[i]]], bool(stopped[i])) for i in range(nseg)]

    def generate_segments(self, speaker: np.ndarray, emotion: np.ndarray, segments: Sequence[Sequence[int]], language: int,
                          options: "GenerationOptions", max_tokens: int = 1500) -> List[GenerationResult]:
        """NativeRuntime::synthesize's GPT loop (native_runtime.cpp:98-99) for a request's text
        segments: segment i is prepare(speaker, emotion, segments[i], language) then generate()
        with options.seed + i; all segments are decoded together on the device."""
        sp = np.ascontiguousarray(speaker, dtype=np.float32)
        em = np.ascontiguousarray(emotion, dtype=np.float32)
        if sp.size != 192 or em.size != WIDTH:
            raise InvalidArgument("Invalid GPT conditioning dimensions")
        flat, counts = self._segments(segments)
        return self._segment_results(_lib.itts_gpt_generate_segments,
                                     (_fp(sp), _fp(em), _up(flat), _up(counts), len(counts), int(language)), len(counts), options,
                                     max_tokens)

    def generate_segments_cond(self, cond: np.ndarray, segments: Sequence[Sequence[int]], language: int,
                               options: "GenerationOptions", max_tokens: int = 1500) -> List[GenerationResult]:
        """generate_segments() with the conditioning rows given directly (as prepare_cond)."""
        cd = np.ascontiguousarray(cond, dtype=np.float32).reshape(-1, WIDTH)
        flat, counts = self._segments(segments)
        return self._segment_results(_lib.itts_gpt_generate_segments_cond,
                                     (_fp(cd), cd.shape[0], _up(flat), _up(counts), len(counts), int(language)), len(counts),
                                     options, max_tokens)

    def checkpoint(self) -> GptState:
        ptr = C.c_void_p()
        self._check(_lib.itts_gpt_checkpoint(self._h, C.byref(ptr)))
        return GptState(ptr.value)

    def restore(self, state: GptState) -> None:
        self._check(_lib.itts_gpt_restore(self._h, state._ptr))

    def cached_tokens(self) -> int:
        return int(_lib.itts_gpt_cached_tokens(self._h))

    def last_timing(self) -> dict:
        t = _Timing()
        self._check(_lib.itts_gpt_last_timing(self._h, C.byref(t)))
        return {"prefill_ms": t.prefill_ms, "decode_ms": t.decode_ms, "decode_steps": t.decode_steps,
                "decode_path": "step" if t.decode_path == 1 else "multi"}

    KERNELS = ("gemv_c_attn", "gemv_attn_proj", "gemv_c_fc", "gemv_mlp_proj", "gemv_mel_head", "attention", "step", "copy")

    def bench_kernel(self, which: str, iters: int = 240, batch: int = 1, cached_rows: int = 0, one_layer: bool = False) -> dict:
        """Mean duration (HIP events, back-to-back launches) and algorithmic bytes of one decode
        kernel kind; attention and "step" run with `cached_rows` cached rows (0 -> 752).
        one_layer: every launch on layer 0's weights (served from the memory-side cache)."""
        ms = C.c_float()
        by = C.c_double()
        kind = self.KERNELS.index(which) | (0x100 if one_layer else 0)
        self._check(_lib.itts_gpt_bench_kernel(self._h, kind, int(batch), int(cached_rows), int(iters),
                                               C.byref(ms), C.byref(by)))
        return {"avg_ms": float(ms.value), "bytes": float(by.value)}

    # Processors / sampler on this handle's stream.
    STEP_PHASES = ("layer", "c_attn", "attention_tiles", "merge", "attn_proj", "mlp_fc", "mlp_proj", "head")

    def step_phases(self, cached_rows: int = 0, iters: int = 20, nseq: int = 1) -> dict:
        """Per-phase time (us) of the persistent step kernel (nseq 1) or batch step kernel
        (nseq 2-4 sequences, each at cached_rows) from its own clock stamps."""
        out = (C.c_float * 8)()
        if nseq == 1:
            self._check(_lib.itts_gpt_step_phases(self._h, int(cached_rows), int(iters), out))
        else:
            self._check(_lib.itts_gpt_step_phases_batch(self._h, int(nseq), int(cached_rows), int(iters), out))
        return {k: float(v) for k, v in zip(self.STEP_PHASES, out)}

    def apply_processors(self, logits: np.ndarray, history: Sequence[int], options: GenerationOptions) -> np.ndarray:
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        hist = np.ascontiguousarray(np.asarray(history, dtype=np.uint32))
        out = np.empty_like(lg)
        o = options._c()
        self._check(_lib.itts_gpt_apply_processors(self._h, _fp(lg), lg.size, _up(hist), hist.size, C.byref(o), _fp(out)))
        return out

    def sample(self, processed: np.ndarray, rng_state: int, draws: int = 1):
        pr = np.ascontiguousarray(processed, dtype=np.float32)
        st = C.c_uint64(int(rng_state) & (2**64 - 1))
        toks = np.zeros(int(draws), np.uint32)
        self._check(_lib.itts_gpt_sample(self._h, _fp(pr), pr.size, C.byref(st), int(draws), _up(toks)))
        return [int(t) for t in toks], int(st.value)


_sampler_handle: Optional[GptDecoder] = None


def _sampler() -> GptDecoder:
    global _sampler_handle
    if _sampler_handle is None:
        _sampler_handle = GptDecoder(None)
    return _sampler_handle


def apply_gpt_sampling_processors(logits: np.ndarray, history: Sequence[int], options: GenerationOptions) -> np.ndarray:
    """gpt_sampling.cpp:28-128, on the device (process-wide sampler-only handle)."""
    return _sampler().apply_processors(logits, history, options)


def sample_gpt_token(processed: np.ndarray, rng_state: int, draws: int = 1):
    """gpt_sampling.cpp:130-165 `draws` times with SplitMix64 state rng_state; returns (tokens, new_state)."""
    return _sampler().sample(processed, rng_state, draws)


# ---------------------------------------------------------------------- synthetic inputs

def alloc_events() -> int:
    """itts_gpt_alloc_events: device/pinned allocations and graph instantiations made so far."""
    return int(_lib.itts_gpt_alloc_events())


def synthetic_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """Deterministic N(mean, std^2) values (Box-Muller over SplitMix64 keyed by (seed, index))."""
    out = np.empty(int(n), np.float32)
    _lib.itts_synthetic_normal(_fp(out), out.size, int(seed) & (2**64 - 1), float(mean), float(std))
    return out


def _tensor_seed(seed: int, name: str) -> int:
    return (int(seed) * 0x9E3779B97F4A7C15 + zlib.crc32(name.encode())) & (2**64 - 1)


def synthetic_weight_shapes(layers: int = 24, text_vocab: int = 12000, text_pos: int = 602, mel_pos: int = 1815,
                            lang_vocab: int = 107, speaker: bool = True) -> Dict[str, tuple]:
    """Tensor names and HF layouts of the IndexTTS 2.5 GPT (gpt.cpp:12-21)."""
    s: Dict[str, tuple] = {}
    if speaker:
        s["gpt.spk_emb_proj.weight"] = (WIDTH, 192)
        s["gpt.spk_emb_proj.bias"] = (WIDTH,)
    s["gpt.text_embedding.weight"] = (text_vocab, WIDTH)
    s["gpt.text_pos_embedding.emb.weight"] = (text_pos, WIDTH)
    s["gpt.lang_embedding.weight"] = (lang_vocab, WIDTH)
    s["gpt.mel_embedding.weight"] = (MEL_VOCAB, WIDTH)
    s["gpt.mel_pos_embedding.emb.weight"] = (mel_pos, WIDTH)
    for i in range(layers):
        p = f"gpt.gpt.h.{i}"
        s[p + ".ln_1.weight"] = (WIDTH,)
        s[p + ".ln_1.bias"] = (WIDTH,)
        s[p + ".attn.c_attn.weight"] = (WIDTH, 3 * WIDTH)
        s[p + ".attn.c_attn.bias"] = (3 * WIDTH,)
        s[p + ".attn.c_proj.weight"] = (WIDTH, WIDTH)
        s[p + ".attn.c_proj.bias"] = (WIDTH,)
        s[p + ".ln_2.weight"] = (WIDTH,)
        s[p + ".ln_2.bias"] = (WIDTH,)
        s[p + ".mlp.c_fc.weight"] = (WIDTH, FFN)
        s[p + ".mlp.c_fc.bias"] = (FFN,)
        s[p + ".mlp.c_proj.weight"] = (FFN, WIDTH)
        s[p + ".mlp.c_proj.bias"] = (WIDTH,)
    s["gpt.gpt.ln_f.weight"] = (WIDTH,)
    s["gpt.gpt.ln_f.bias"] = (WIDTH,)
    s["gpt.final_norm.weight"] = (WIDTH,)
    s["gpt.final_norm.bias"] = (WIDTH,)
    s["gpt.mel_head.weight"] = (MEL_VOCAB, WIDTH)
    s["gpt.mel_head.bias"] = (MEL_VOCAB,)
    return s


def make_synthetic_weights(layers: int = 24, seed: int = 0, std: float = 0.02, ln_random: bool = False,
                           **shape_kw) -> Dict[str, np.ndarray]:
    """Random-init FP32 weights N(0, std^2); LayerNorm gamma=1, beta=0 unless ln_random."""
    out: Dict[str, np.ndarray] = {}
    for name, shape in synthetic_weight_shapes(layers, **shape_kw).items():
        n = int(np.prod(shape))
        is_ln = (".ln_" in name or "ln_f" in name or "final_norm" in name)
        if is_ln and not ln_random:
            out[name] = np.ones(shape, np.float32) if name.endswith("weight") else np.zeros(shape, np.float32)
        elif is_ln:
            mean = 1.0 if name.endswith("weight") else 0.0
            out[name] = synthetic_normal(n, _tensor_seed(seed, name), mean, 0.1).reshape(shape)
        else:
            out[name] = synthetic_normal(n, _tensor_seed(seed, name), 0.0, std).reshape(shape)
    return out


CODEC_WIDTH, CODEC_HIDDEN, CODEC_FFN, CODEC_BLOCKS, CODEBOOK = 1024, 384, 2048, 12, 8192


def codec_weight_shapes() -> Dict[str, tuple]:
    """The tensors EnhancedCodec::decode reads (src/codec.cpp:5-20, 36-72), reference names."""
    q, d = "codec.quantizer.quantizers.0", "codec.decoder.0"
    s = {f"{q}.codebook.weight": (CODEBOOK, 8), f"{q}.out_project.weight": (CODEC_WIDTH, 8), f"{q}.out_project.bias": (CODEC_WIDTH,),
         f"{d}.embed.weight": (CODEC_HIDDEN, CODEC_WIDTH, 7), f"{d}.embed.bias": (CODEC_HIDDEN,),
         f"{d}.norm.weight": (CODEC_HIDDEN,), f"{d}.norm.bias": (CODEC_HIDDEN,)}
    for i in range(CODEC_BLOCKS):
        l = f"{d}.convnext.{i}"
        s.update({f"{l}.dwconv.weight": (CODEC_HIDDEN, 1, 7), f"{l}.dwconv.bias": (CODEC_HIDDEN,),
                  f"{l}.norm.weight": (CODEC_HIDDEN,), f"{l}.norm.bias": (CODEC_HIDDEN,),
                  f"{l}.pwconv1.weight": (CODEC_FFN, CODEC_HIDDEN), f"{l}.pwconv1.bias": (CODEC_FFN,),
                  f"{l}.pwconv2.weight": (CODEC_HIDDEN, CODEC_FFN), f"{l}.pwconv2.bias": (CODEC_HIDDEN,),
                  f"{l}.gamma": (CODEC_HIDDEN,)})
    s.update({f"{d}.final_layer_norm.weight": (CODEC_HIDDEN,), f"{d}.final_layer_norm.bias": (CODEC_HIDDEN,),
              "codec.decoder.1.weight": (CODEC_WIDTH, CODEC_HIDDEN), "codec.decoder.1.bias": (CODEC_WIDTH,),
              "codec.up.weight": (CODEC_WIDTH, CODEC_WIDTH, 3), "codec.up.bias": (CODEC_WIDTH,)})
    return s


def make_synthetic_codec_weights(seed: int = 0, std: float = 0.02) -> Dict[str, np.ndarray]:
    """Random-init codec decode weights: convolutions, linears and biases N(0, std^2); codebook
    N(0, 1); LayerNorm gamma N(1, 0.1^2), beta N(0, 0.1^2); layer scales N(0.5, 0.1^2)."""
    out: Dict[str, np.ndarray] = {}
    for name, shape in codec_weight_shapes().items():
        n, key = int(np.prod(shape)), _tensor_seed(seed, name)
        if "codebook" in name:
            v = synthetic_normal(n, key, 0.0, 1.0)
        elif ".norm." in name or "final_layer_norm" in name:
            v = synthetic_normal(n, key, 1.0 if name.endswith("weight") else 0.0, 0.1)
        elif name.endswith(".gamma"):
            v = synthetic_normal(n, key, 0.5, 0.1)
        else:
            v = synthetic_normal(n, key, 0.0, std)
        out[name] = v.reshape(shape)
    return out


QWEN_VOCAB, QWEN_WIDTH, QWEN_Q, QWEN_KV, QWEN_FFN, QWEN_LAYERS, QWEN_EOS = 151936, 1024, 2048, 1024, 3072, 28, 151643


def qwen_weight_shapes(layers: int = QWEN_LAYERS) -> Dict[str, tuple]:
    """The tensors QwenDecoder reads (src/qwen.cpp:5-15, 23-45), reference names."""
    s = {"qwen.model.embed_tokens.weight": (QWEN_VOCAB, QWEN_WIDTH), "qwen.model.norm.weight": (QWEN_WIDTH,)}
    for i in range(layers):
        p = f"qwen.model.layers.{i}"
        s.update({f"{p}.self_attn.q_proj.weight": (QWEN_Q, QWEN_WIDTH), f"{p}.self_attn.k_proj.weight": (QWEN_KV, QWEN_WIDTH),
                  f"{p}.self_attn.v_proj.weight": (QWEN_KV, QWEN_WIDTH), f"{p}.self_attn.o_proj.weight": (QWEN_WIDTH, QWEN_Q),
                  f"{p}.self_attn.q_norm.weight": (128,), f"{p}.self_attn.k_norm.weight": (128,),
                  f"{p}.mlp.gate_proj.weight": (QWEN_FFN, QWEN_WIDTH), f"{p}.mlp.up_proj.weight": (QWEN_FFN, QWEN_WIDTH),
                  f"{p}.mlp.down_proj.weight": (QWEN_WIDTH, QWEN_FFN), f"{p}.input_layernorm.weight": (QWEN_WIDTH,),
                  f"{p}.post_attention_layernorm.weight": (QWEN_WIDTH,)})
    return s


def make_synthetic_qwen_weights(layers: int = QWEN_LAYERS, seed: int = 0, std: float = 0.02) -> Dict[str, np.ndarray]:
    """Random-init Qwen3-0.6B decoder weights: matrices and the embedding N(0, std^2), RMSNorm
    weights N(1, 0.1^2)."""
    out: Dict[str, np.ndarray] = {}
    for name, shape in qwen_weight_shapes(layers).items():
        n, key = int(np.prod(shape)), _tensor_seed(seed, name)
        v = synthetic_normal(n, key, 1.0, 0.1) if len(shape) == 1 else synthetic_normal(n, key, 0.0, std)
        out[name] = v.reshape(shape)
    return out


class EnhancedCodec:
    """The decode path of itts25::EnhancedCodec (include/itts25/codec.hpp:11-17) on the MI355X."""

    def __init__(self, weights: Optional[Dict[str, np.ndarray]]):
        self._c = C.c_void_p()
        keep, tensors = [], []
        for name, arr in (weights or {}).items():
            a = np.ascontiguousarray(arr, dtype=np.float32)
            keep.append(a)
            shape = (C.c_int64 * 4)(*(list(a.shape) + [0] * (4 - a.ndim)))
            tensors.append(_Tensor(name.encode(), a.ctypes.data, shape, a.ndim, 0))
        arr_t = (_Tensor * max(1, len(tensors)))(*tensors)
        st = _lib.itts_codec_create(arr_t, len(tensors), C.byref(self._c))
        if st != 0:
            _raise(st, _lib.itts_codec_last_error(None).decode())

    @classmethod
    def from_bundle(cls, bundle: "Bundle") -> "EnhancedCodec":
        self = cls.__new__(cls)
        self._c = C.c_void_p()
        st = _lib.itts_codec_create_from_bundle(bundle._b, C.byref(self._c))
        if st != 0:
            _raise(st, _lib.itts_codec_last_error(None).decode())
        return self

    def close(self) -> None:
        if self._c.value:
            _lib.itts_codec_destroy(self._c)
            self._c = C.c_void_p()

    def __del__(self):
        self.close()

    def decode(self, codes: Sequence[int]) -> np.ndarray:
        """EnhancedCodec::decode (codec.cpp:64-72): [2T, 1024] features, time-major."""
        ids = np.ascontiguousarray(np.asarray(codes, dtype=np.int64))
        if ids.size and (ids.min() < 0 or ids.max() > 0xFFFFFFFF):
            raise InvalidArgument("Codec expects 1..5000 code IDs in [0,8192)")
        ids = ids.astype(np.uint32)
        out = np.empty((2 * max(1, ids.size), CODEC_WIDTH), np.float32)
        st = _lib.itts_codec_decode(self._c, _up(ids), ids.size, _fp(out))
        if st != 0:
            _raise(st, _lib.itts_codec_last_error(self._c).decode())
        return out[: 2 * ids.size]

    def bench(self, n: int, iters: int = 20) -> dict:
        ms, fl = C.c_float(), C.c_double()
        st = _lib.itts_codec_bench(self._c, int(n), int(iters), C.byref(ms), C.byref(fl))
        if st != 0:
            _raise(st, _lib.itts_codec_last_error(self._c).decode())
        return {"avg_ms": float(ms.value), "flops": float(fl.value)}


def synthetic_prefix_inputs(n_text: int, seed: int, n_cond: int = 32, text_vocab: int = 12000):
    """32 conditioning latents ~N(0,1)*0.5 and n_text ids uniform in [0, text_vocab)."""
    cond = synthetic_normal(n_cond * WIDTH, _tensor_seed(seed, "cond"), 0.0, 0.5).reshape(n_cond, WIDTH)
    rng = np.random.default_rng(seed)
    text = rng.integers(0, text_vocab, size=n_text, dtype=np.int64).astype(np.uint32)
    return cond, text


QWEN_DID_NOT_STOP = "Qwen did not reach EOS within 1024 generated tokens"


class QwenDecoder:
    """itts25::QwenDecoder (include/itts25/qwen.hpp:5-18, src/qwen.cpp:5-49) on the MI355X."""

    def __init__(self, weights: Dict[str, np.ndarray], layers: int = QWEN_LAYERS):
        keep, table = {}, []
        for name, v in weights.items():
            a = keep[name] = np.ascontiguousarray(v, dtype=np.float32)
            shape = (C.c_int64 * 4)(*(list(a.shape) + [0] * (4 - a.ndim)))
            table.append(_Tensor(name.encode(), a.ctypes.data, shape, a.ndim, 0))
        arr = (_Tensor * max(1, len(table)))(*table)
        self._q = C.c_void_p()
        st = _lib.itts_qwen_create(arr, len(table), C.byref(_QwenConfig(layers, 0)), C.byref(self._q))
        if st != 0:
            _raise(st, _lib.itts_qwen_last_error(None).decode())

    @classmethod
    def from_bundle(cls, bundle: "Bundle", layers: int = QWEN_LAYERS) -> "QwenDecoder":
        self = cls.__new__(cls)
        self._q = C.c_void_p()
        st = _lib.itts_qwen_create_from_bundle(bundle._b, C.byref(_QwenConfig(layers, 0)), C.byref(self._q))
        if st != 0:
            _raise(st, _lib.itts_qwen_last_error(None).decode())
        return self

    def close(self) -> None:
        if getattr(self, "_q", None):
            _lib.itts_qwen_destroy(self._q)
            self._q = None

    def __del__(self):
        if _lib is not None:
            self.close()

    def _check(self, st: int) -> None:
        if st != 0:
            _raise(st, _lib.itts_qwen_last_error(self._q).decode())

    def prefill(self, ids: Sequence[int]) -> np.ndarray:
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(QWEN_VOCAB, np.float32)
        self._check(_lib.itts_qwen_prefill(self._q, _up(a), a.size, _fp(out)))
        return out

    def step(self, token: int) -> np.ndarray:
        out = np.empty(QWEN_VOCAB, np.float32)
        self._check(_lib.itts_qwen_step(self._q, int(token) & 0xFFFFFFFF, _fp(out)))
        return out

    def generate_tokens(self, ids: Sequence[int], maximum: int = 1024) -> Tuple[List[int], bool]:
        """(ids, reached EOS): the ids produced also when generate() raises at `maximum`."""
        a = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros(max(1, int(maximum)), np.uint32)
        n = C.c_uint32(0)
        st = _lib.itts_qwen_generate(self._q, _up(a), a.size, int(maximum) & 0xFFFFFFFF, _up(out), C.byref(n))
        toks = [int(x) for x in out[: n.value]]
        if st == -2 and _lib.itts_qwen_last_error(self._q).decode() == QWEN_DID_NOT_STOP:
            return toks, False
        self._check(st)
        return toks, True

    def generate(self, ids: Sequence[int], maximum: int = 1024) -> List[int]:
        """QwenDecoder::generate (qwen.cpp:46-49): greedy ids up to and including EOS."""
        toks, eos = self.generate_tokens(ids, maximum)
        if not eos:
            raise GptRuntimeError(QWEN_DID_NOT_STOP)
        return toks

    def submissions(self) -> int:
        return int(_lib.itts_qwen_submissions(self._q))

    def bench(self, prompt: int, cached_rows: int, iters: int) -> Tuple[float, float]:
        """(prefill ms of `prompt` ids, mean µs per decode step from `cached_rows` rows)."""
        pm, su = C.c_float(0), C.c_float(0)
        self._check(_lib.itts_qwen_bench(self._q, prompt, cached_rows, iters, C.byref(pm), C.byref(su)))
        return pm.value, su.value
