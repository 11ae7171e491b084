"""The C++ drop-in stays a drop-in: the reference's own callers of itts25::GptDecoder,
itts25::EnhancedCodec and itts25::QwenDecoder compile against index-tts-25-metal_amd/cpp (CPU
only).

Callers (src/pipeline.cpp:12-25, src/native_runtime.cpp:50-53, 98-100, src/server.cpp:33-47,
src/main.cpp:31-66, 159-169) are syntax-checked with g++ -std=c++17 -fsyntax-only, with this
repository's cpp/ ahead of the reference's include/ on the search path, so "itts25/gpt.hpp",
"itts25/codec.hpp" and "itts25/qwen.hpp" resolve to the drop-in and every other header to the
reference's own.
Runs only where the reference tree is present (it is read, not built or copied).
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference")
CPP = ROOT / "index-tts-25-metal_amd" / "cpp"

pytestmark = pytest.mark.skipif(not (REF / "src" / "pipeline.cpp").exists() or shutil.which("g++") is None,
                                reason="needs the reference tree and g++")


def _flags():
    return ["-std=c++17", "-fsyntax-only", f"-I{CPP}", f"-I{ROOT / 'include'}", f"-I{REF / 'include'}",
            f"-I{REF / 'vendor' / 'metal-runtime' / 'include'}", f"-I{REF / 'vendor' / 'headers'}"]


@pytest.mark.parametrize("caller", ["pipeline", "native_runtime", "server", "main"])
def test_reference_caller_compiles_against_dropin(caller):
    src = REF / "src" / f"{caller}.cpp"
    p = subprocess.run(["g++", *_flags(), "-H", str(src)], capture_output=True, text=True)
    assert p.returncode == 0, p.stderr[-3000:]
    included = [ln.lstrip(". ").strip() for ln in p.stderr.splitlines() if ln.startswith(".")]
    gpt = [h for h in included if h.endswith("itts25/gpt.hpp")]
    assert gpt and all(Path(h).resolve().is_relative_to(CPP) for h in gpt), gpt
    for name in ("itts25/codec.hpp", "itts25/qwen.hpp"):
        hs = [h for h in included if h.endswith(name)]
        assert all(Path(h).resolve().is_relative_to(CPP) for h in hs), hs
    if caller in ("main", "native_runtime", "server"):  # the QwenDecoder callers
        assert any(h.endswith("itts25/qwen.hpp") for h in included), caller
