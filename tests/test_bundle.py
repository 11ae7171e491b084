"""MIT2 bundle reader (csrc/bundle.cpp) against the format and checks of the reference's
mit2::Bundle (vendor/metal-runtime/bundle.cpp:150-266) and itts25::Weights
(src/weights.cpp:9-49).  CPU only: opening a bundle touches no GPU.

Every check of the reference reader has a case that breaks exactly that rule and expects
the reference's message; round trips write bundles with itts_gpt.write_mit2_bundle (the
manifest fields of the reference's tools/validate_flow_cache.py:15) and compare every
byte read back.
"""
import json
import struct

import numpy as np
import pytest


def _tensors():
    rng = np.random.default_rng(3)
    return {
        "gpt.a.weight": rng.standard_normal((3, 5)).astype(np.float32),
        "gpt.a.bias": rng.standard_normal(5).astype(np.float32),
        "tokens.ids": np.arange(7, dtype=np.uint32) * 1000003,
        "name with é and \"quotes\"": rng.standard_normal((2, 2, 2)).astype(np.float32),
    }


def _rewrite_manifest(path, fn):
    m = json.loads((path / "manifest.json").read_text())
    fn(m)
    (path / "manifest.json").write_text(json.dumps(m))


def test_directory_bundle_round_trip(itts, tmp_path):
    t = _tensors()
    p = itts.write_mit2_bundle(tmp_path / "b", t, alignment=256)
    b = itts.Bundle(p)
    lst = b.tensors()
    assert len(b) == len(t) == len(lst)
    assert [r["name"] for r in lst] == list(t)
    for r, (name, a) in zip(lst, t.items()):
        assert r["shape"] == a.shape
        assert r["dtype"] == ("u32" if a.dtype == np.uint32 else "f32")
        assert r["offset"] % 256 == 0 and r["offset"] >= 12
        assert r["nbytes"] == a.nbytes
        got = b.ids(name) if a.dtype == np.uint32 else b.get(name)
        assert got.dtype == a.dtype and got.shape == a.shape
        assert got.tobytes() == a.tobytes()
    assert b.info("gpt.a.weight")["shape"] == (3, 5)
    with pytest.raises(itts.GptRuntimeError, match="^Missing tensor: nope$"):
        b.info("nope")
    with pytest.raises(itts.GptRuntimeError, match="^Expected float32: tokens.ids$"):
        b.get("tokens.ids")
    with pytest.raises(itts.GptRuntimeError, match="^Expected uint32: gpt.a.bias$"):
        b.ids("gpt.a.bias")


def test_single_file_bundle(itts, tmp_path):
    t = _tensors()
    p = itts.write_mit2_bundle(tmp_path / "one.mit2", t, single_file=True, alignment=64)
    raw = p.read_bytes()
    assert raw[:4] == b"MIT2" and raw[-8:] == b"MIT2VOIC"
    b = itts.Bundle(p, require_model=False)
    for name, a in t.items():
        got = b.ids(name) if a.dtype == np.uint32 else b.get(name)
        assert got.tobytes() == a.tobytes()
    # Weights(path, true) reads <path>/manifest.json (weights.cpp:10-13): a single-file
    # bundle has none, so the model check fails as in the reference
    with pytest.raises(itts.GptRuntimeError, match="^Expected an IndexTTS 2.5 model bundle$"):
        itts.Bundle(p, require_model=True)


def test_model_target_required(itts, tmp_path):
    p = itts.write_mit2_bundle(tmp_path / "b", _tensors(), target="something-else")
    with pytest.raises(itts.GptRuntimeError, match="^Expected an IndexTTS 2.5 model bundle$"):
        itts.Bundle(p)
    assert len(itts.Bundle(p, require_model=False)) == 4


def test_missing_bundle(itts, tmp_path):
    with pytest.raises(itts.GptRuntimeError, match="^failed to open .*/manifest.json$"):
        itts.Bundle(tmp_path / "none")


MANIFEST_CASES = [
    (lambda m: m.update(format="MIT3"), "unsupported bundle format: MIT3"),
    (lambda m: m.update(version=2), "unsupported bundle version: 2"),
    (lambda m: m.pop("version"), "missing numeric key version"),
    (lambda m: m.update(alignment=0), "bundle alignment must be non-zero"),
    (lambda m: m.update(endianness="big"), "unsupported bundle endianness: big"),
    (lambda m: m.pop("tensors"), "manifest missing tensors"),
    (lambda m: m["tensors"][0].update(name=""), "tensor record has empty name"),
    (lambda m: m["tensors"][1].update(name=m["tensors"][0]["name"]), "duplicate tensor in manifest: gpt.a.weight"),
    (lambda m: m["tensors"][0].update(offset=m["tensors"][0]["offset"] + 4), "tensor offset is not bundle-aligned: gpt.a.weight"),
    (lambda m: m["tensors"][0].update(nbytes=0), "tensor has zero bytes: gpt.a.weight"),
    (lambda m: m["tensors"][0].update(nbytes=1 << 40), "tensor extends beyond weights file: gpt.a.weight"),
    (lambda m: m["tensors"][0].pop("offset"), "missing numeric key offset"),
    (lambda m: m["tensors"][0].pop("shape"), "missing tensor shape"),
    (lambda m: m["tensors"][0].update(dtype="f16"), "Initial native backend requires f32/u32: gpt.a.weight"),
    (lambda m: m["tensors"][0].update(shape=[3, 0]), "Invalid shape: gpt.a.weight"),
    (lambda m: m["tensors"][0].update(shape=[3, 4]), "Tensor size does not match shape: gpt.a.weight"),
    (lambda m: m["tensors"][0].update(nbytes=m["tensors"][0]["nbytes"] - 4), "Tensor size does not match shape: gpt.a.weight"),
]


@pytest.mark.parametrize("case", range(len(MANIFEST_CASES)))
def test_manifest_checks(itts, tmp_path, case):
    fn, msg = MANIFEST_CASES[case]
    p = itts.write_mit2_bundle(tmp_path / "b", _tensors(), alignment=256)
    _rewrite_manifest(p, fn)
    with pytest.raises(itts.GptRuntimeError) as e:
        itts.Bundle(p)
    assert str(e.value) == msg


@pytest.mark.parametrize("edit,msg", [
    (lambda raw: b"MIT3" + raw[4:], "weights file has invalid MIT2 magic"),
    (lambda raw: raw[:4] + struct.pack("<I", 2) + raw[8:], "weights header version mismatch"),
    (lambda raw: raw[:8] + struct.pack("<I", 128) + raw[12:], "weights header alignment mismatch"),
    (lambda raw: raw[:10], "weights file is too small for MIT2 header"),
])
def test_weights_header_checks(itts, tmp_path, edit, msg):
    p = itts.write_mit2_bundle(tmp_path / "b", _tensors(), alignment=256)
    w = p / "weights.bin"
    w.write_bytes(edit(w.read_bytes()))
    with pytest.raises(itts.GptRuntimeError) as e:
        itts.Bundle(p)
    assert str(e.value) == msg


def test_single_file_footer_checks(itts, tmp_path):
    p = itts.write_mit2_bundle(tmp_path / "one", _tensors(), single_file=True)
    raw = p.read_bytes()
    bad = tmp_path / "bad"
    bad.write_bytes(raw[:-8] + b"MIT2XXXX")
    with pytest.raises(itts.GptRuntimeError, match="^single-file bundle footer magic missing: "):
        itts.Bundle(bad, require_model=False)
    small = tmp_path / "small"
    small.write_bytes(raw[:30])
    with pytest.raises(itts.GptRuntimeError, match="^single-file bundle is too small: "):
        itts.Bundle(small, require_model=False)
    over = tmp_path / "over"
    off, n = struct.unpack("<QQ", raw[-24:-8])
    over.write_bytes(raw[:-24] + struct.pack("<QQ", off, n + 100) + b"MIT2VOIC")
    with pytest.raises(itts.GptRuntimeError, match="^single-file bundle manifest exceeds file: "):
        itts.Bundle(over, require_model=False)


def test_custom_weights_file_and_whitespace(itts, tmp_path):
    t = _tensors()
    p = itts.write_mit2_bundle(tmp_path / "b", t, weights_file="w.dat")
    # the same manifest re-serialised with indentation and unicode escapes
    m = json.loads((p / "manifest.json").read_text())
    (p / "manifest.json").write_text(json.dumps(m, indent=3, ensure_ascii=True))
    b = itts.Bundle(p)
    assert [r["name"] for r in b.tensors()] == list(t)
    assert b.get("name with é and \"quotes\"").tobytes() == t["name with é and \"quotes\""].tobytes()


def test_gpt_from_bundle_reports_missing_tensor(itts, tmp_path):
    # the GPT tensor list is checked before anything is uploaded (no GPU needed to fail)
    p = itts.write_mit2_bundle(tmp_path / "b", _tensors())
    with pytest.raises(itts.GptRuntimeError, match="^Missing tensor: gpt.spk_emb_proj.weight$"):
        itts.GptDecoder.from_bundle(itts.Bundle(p))
