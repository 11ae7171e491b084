"""Build recipe for libitts_gpt.so (the HIP path + C ABI) and the C++17 drop-in shim.

    python index-tts-25-metal_amd/build.py            # library + shim example
    python index-tts-25-metal_amd/build.py --lib-only

Every .hip file is compiled for gfx950 with hipcc, in parallel, into _build/, then
linked into index-tts-25-metal_amd/libitts_gpt.so next to this file (in-tree, so it
travels with the source tree).  Packed-FP32 instruction selection is disabled on
every device compile (-packed-fp32-ops).
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
INCLUDE = ROOT / "include"
LIB = PKG / "libitts_gpt.so"
SHIM_EXE = PKG / "cpp" / "gpt_shim_example"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
SOURCES = ["decode.hip", "step.hip", "step_batch.hip", "sampler.hip", "beam.hip", "prefill.hip", "util.hip", "runtime.hip",
           "codec.hip", "libm_check.hip", "qwen.hip"]
# Per-file device flags.  step.hip: the persistent step kernel is scheduled with LLVM's max-ILP
# strategy, 578.4 -> 567.9 us per step at 752 cached rows (one box, three alternating runs); the
# same strategy made the batched GEMVs of decode.hip 9% slower, so it is not applied there.
# codec.hip: the same strategy, 47-code decode 0.367 -> 0.356 ms, 600 codes 0.707 -> 0.705 ms
# (one box, alternating).  Measured and not applied: max-ILP for prefill.hip (155-row prefill
# 3.23 -> 3.29 ms) and qwen.hip (step 835 -> 846 us), no change for sampler.hip and beam.hip.
_MAX_ILP = ["-mllvm", "--amdgpu-sched-strategy=max-ilp"]
SOURCE_FLAGS = {"step.hip": _MAX_ILP, "codec.hip": _MAX_ILP}
HOST_SOURCES = ["bundle.cpp"]  # host-only C++ (g++)
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}", f"-I{CSRC}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def build_library(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = []

    def compile_one(src: str) -> Path:
        obj = BUILD / (Path(src).stem + ".o")
        _run([HIPCC, *DEVICE_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    def compile_host(src: str) -> Path:
        obj = BUILD / (Path(src).stem + ".host.o")
        _run(["g++", *HOST_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(SOURCES) + len(HOST_SOURCES)))) as ex:
        dev = ex.map(compile_one, SOURCES)
        host = ex.map(compile_host, HOST_SOURCES)
        objs = list(dev) + list(host)
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_shim() -> Path:
    """Compile the C++17 GptDecoder shim and its example against the C ABI (host g++)."""
    cpp = PKG / "cpp"
    tmp = SHIM_EXE.with_suffix(".tmp")
    _run([
        "g++", "-O2", "-std=c++17", "-Wall",
        f"-I{cpp}", f"-I{INCLUDE}",
        str(cpp / "gpt.cpp"), str(cpp / "codec.cpp"), str(cpp / "qwen.cpp"), str(cpp / "gpt_shim_example.cpp"),
        f"-L{PKG}", "-litts_gpt", f"-Wl,-rpath,{PKG}",
        "-o", str(tmp),
    ])
    os.replace(tmp, SHIM_EXE)
    return SHIM_EXE


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-j", type=int, default=8)
    args = ap.parse_args()
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        print(f"hipcc not found at {HIPCC}", file=sys.stderr)
        return 1
    print(build_library(args.j))
    if not args.lib_only and (PKG / "cpp" / "gpt.cpp").exists():
        print(build_shim())
    return 0


if __name__ == "__main__":
    sys.exit(main())
