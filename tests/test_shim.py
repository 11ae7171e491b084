"""The C++17 drop-in GptDecoder (index-tts-25-metal_amd/cpp) links against the C ABI and,
on the GPU, runs prepare -> generate through the reference's constructor form."""
import json
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent.parent / "index-tts-25-metal_amd" / "cpp" / "gpt_shim_example"


def test_shim_links():
    if not EXE.exists():
        pytest.skip("shim example not built (run __graft_entry__.build())")
    out = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "gpt shim linked" in out.stdout


@pytest.mark.gpu
def test_shim_runs_on_gpu():
    assert EXE.exists(), "shim example not built"
    out = subprocess.run([str(EXE), "run"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    lines = [json.loads(l) for l in out.stdout.splitlines() if l.startswith("{")]
    assert lines[0]["rows"] == 3 + 6 + 1  # 3 conditioning rows + [0, 5, 17, 300, 42, 1] + mel start
    assert lines[0]["codes"] + lines[0]["stopped"] >= 1
    assert lines[1]["beam_codes"] + lines[1]["beam_stopped"] >= 1
    assert lines[2]["processed"] == 8194
