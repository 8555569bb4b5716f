"""The on-disk stores on the host (no GPU): the library's manifest and
index parsers (store.c) against the reference's formats.

The fixtures come from sepia_amd/store_synth.py. Its smoke fixture is
accepted by the reference's own loader (the reference engine's
`--smoke DIR`: index_load, manifest_load, the expert slices' bytes and a
bitwise qlinear, reference src/sepia.c:4312-4446), which pins the writer
to the reference's formats; the library's parser must then read every
field of the same files as the JSON holds them, and reject what the
reference's loader dies on (src/sepia.c:1876-1910, :2010-2080).
"""
import ctypes
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from sepia_amd import hip, store_synth

REF_BIN = os.path.join(ROOT, "oracle", "_ref", "sepia_hip")


@pytest.fixture(scope="module")
def L():
    return hip.load()


@pytest.fixture
def smoke(tmp_path):
    d = str(tmp_path / "smoke")
    info = store_synth.write_smoke_fixture(d)
    info["dir"] = d
    return info


@pytest.fixture
def layer_store(tmp_path):
    d = str(tmp_path / "layer")
    paths, host = store_synth.write_layer_store(d, np.random.default_rng(5), layer=3, hidden=512, inter=256,
                                                n_routed=4, n_shared=2, types=(17, 18, 13, 14), n_parts=2,
                                                extra_layers=(7,))
    paths["dir"] = d
    return paths, host


@pytest.mark.skipif(not os.path.exists(REF_BIN), reason="oracle/_ref/sepia_hip not built")
def test_reference_loader_accepts_the_fixture(smoke):
    r = subprocess.run([REF_BIN, "--smoke", smoke["dir"]], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "smoke ok" in r.stdout, (r.stdout, r.stderr)


@pytest.mark.skipif(not os.path.exists(REF_BIN), reason="oracle/_ref/sepia_hip not built")
def test_reference_loader_rejects_a_wrong_slice(smoke):
    """The same gate fails when an expert slice's recorded offset is off by
    one block, so passing it means the offsets are right."""
    p = os.path.join(smoke["dir"], "smoke_expected.json")
    with open(p) as f:
        exp = json.load(f)
    exp["experts"][1]["up"]["abs_offset"] += 34
    with open(p, "w") as f:
        json.dump(exp, f)
    r = subprocess.run([REF_BIN, "--smoke", smoke["dir"]], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0


def manifest_entries(L, t):
    out = []
    for i in range(L.sepia_hip_manifest_count(t)):
        e = L.sepia_hip_manifest_tensor(t, i).contents
        out.append({"name": e.name.decode(), "ggml_type": e.ggml_type, "shape": list(e.shape[:e.n_dims]),
                    "offset": e.offset, "nbytes": e.nbytes})
    return out


@pytest.mark.parametrize("which", ["smoke", "layer"])
def test_manifest_parse(L, smoke, layer_store, which):
    paths = smoke if which == "smoke" else layer_store[0]
    t = L.sepia_hip_manifest_load(paths["manifest"].encode(), paths["bin"].encode())
    assert t
    try:
        with open(paths["manifest"]) as f:
            want = [{k: e[k] for k in ("name", "ggml_type", "shape", "offset", "nbytes")}
                    for e in json.load(f)["tensors"]]
        assert manifest_entries(L, t) == want
        for e in want:
            got = L.sepia_hip_manifest_find(t, e["name"].encode())
            assert got and got.contents.offset == e["offset"]
        assert not L.sepia_hip_manifest_find(t, b"no.such.tensor")
        # resident.bin holds what the GGUF parts hold for each tensor
        with open(paths["manifest"]) as f:
            man = json.load(f)
        with open(paths["bin"], "rb") as fb:
            blob = fb.read()
        gg = os.path.join(os.path.dirname(paths["manifest"]), store_synth.GGUF_DIR)
        for e in man["tensors"]:
            with open(os.path.join(gg, e["source_part_file"]), "rb") as fp:
                fp.seek(e["source_abs_offset"])
                assert fp.read(e["nbytes"]) == blob[e["offset"]:e["offset"] + e["nbytes"]], e["name"]
    finally:
        L.sepia_hip_manifest_free(t)


def test_index_parse(L, layer_store):
    paths, host = layer_store
    idx = L.sepia_hip_index_load(paths["index"].encode())
    assert idx
    try:
        with open(paths["index"]) as f:
            doc = json.load(f)
        assert L.sepia_hip_index_n_experts(idx) == doc["n_experts_per_layer"] == 4
        parts = [L.sepia_hip_index_part(idx, i).decode() for i in range(L.sepia_hip_index_n_parts(idx))]
        assert parts == [p["part_file"] for p in doc["parts"]] and len(parts) == 2
        assert [L.sepia_hip_index_has_layer(idx, l) for l in range(9)] == [int(l in (3, 7)) for l in range(9)]
        s = hip.ExpertSlot()
        for layer, kinds in doc["moe_layers"].items():
            for k, kind in enumerate(("gate", "up", "down")):
                for e, ent in enumerate(kinds[kind]["experts"]):
                    assert L.sepia_hip_index_slot(idx, int(layer), k, e, ctypes.byref(s)) == 1
                    assert (parts[s.part_idx], s.abs_offset, s.nbytes, s.ggml_type) == \
                        (ent["part_file"], ent["abs_offset"], ent["nbytes"], ent["ggml_type"])
        assert L.sepia_hip_index_slot(idx, 3, 3, 0, ctypes.byref(s)) == 0
        assert L.sepia_hip_index_slot(idx, 3, 0, 4, ctypes.byref(s)) == 0
        assert L.sepia_hip_index_slot(idx, 4, 0, 0, ctypes.byref(s)) == 0
        # each slice is the expert's matrix, byte for byte, in its part
        gg = os.path.join(paths["dir"], store_synth.GGUF_DIR)
        for k, kind in enumerate(("gate", "up", "down")):
            for e in range(4):
                L.sepia_hip_index_slot(idx, 3, k, e, ctypes.byref(s))
                with open(os.path.join(gg, parts[s.part_idx]), "rb") as f:
                    f.seek(s.abs_offset)
                    assert f.read(s.nbytes) == host[3][kind][e].tobytes()
    finally:
        L.sepia_hip_index_free(idx)


def edit_json(path, fn):
    with open(path) as f:
        doc = json.load(f)
    fn(doc)
    with open(path, "w") as f:
        json.dump(doc, f)


MANIFEST_BREAKS = {
    "no_tensors": lambda d: d.pop("tensors"),
    "past_end": lambda d: d["tensors"][0].update(nbytes=1 << 40),
    "negative": lambda d: d["tensors"][1].update(offset=-64),
    "shape_5d": lambda d: d["tensors"][0].update(shape=[1, 1, 1, 1, 4]),
    "shape_empty": lambda d: d["tensors"][0].update(shape=[]),
    "no_name": lambda d: d["tensors"][2].pop("name"),
    "float_offset": lambda d: d["tensors"][0].update(offset=1.5),
}


@pytest.mark.parametrize("brk", sorted(MANIFEST_BREAKS))
def test_manifest_rejects(L, smoke, brk):
    edit_json(smoke["manifest"], MANIFEST_BREAKS[brk])
    assert not L.sepia_hip_manifest_load(smoke["manifest"].encode(), smoke["bin"].encode())


def test_manifest_rejects_unparsable_and_missing(L, smoke, tmp_path):
    bad = tmp_path / "bad.json"
    for text in ('{"tensors": [', '{"tensors": []} x', '{"a": "\\ud800"}', "[1, 2,]", ""):
        bad.write_text(text)
        assert not L.sepia_hip_manifest_load(str(bad).encode(), smoke["bin"].encode()), text
    assert not L.sepia_hip_manifest_load(smoke["manifest"].encode(), b"/nonexistent/resident.bin")


def test_json_strings_and_numbers(L, smoke):
    """Escapes, non-ASCII names and big integer offsets read exactly."""
    names = ["blk.0.é中\U0001f600", 'quote"and\\back/slash\ttab']

    def fn(d):
        d["tensors"][0]["name"] = names[0]
        d["tensors"][1]["name"] = names[1]
    edit_json(smoke["manifest"], fn)
    t = L.sepia_hip_manifest_load(smoke["manifest"].encode(), smoke["bin"].encode())
    assert t
    try:
        got = [e["name"] for e in manifest_entries(L, t)[:2]]
        assert got == names
        assert L.sepia_hip_manifest_find(t, names[0].encode("utf-8"))
    finally:
        L.sepia_hip_manifest_free(t)


INDEX_BREAKS = {
    "count": lambda d: d["moe_layers"]["3"]["up"]["experts"].pop(),
    "unknown_part": lambda d: d["moe_layers"]["7"]["down"]["experts"][2].update(part_file="nope.gguf"),
    "missing_down": lambda d: d["moe_layers"]["3"].pop("down"),
    "negative": lambda d: d["moe_layers"]["3"]["gate"]["experts"][0].update(abs_offset=-1),
    "layer_key": lambda d: d["moe_layers"].update({"3x": d["moe_layers"]["3"]}),
    "zero_experts": lambda d: d.update(n_experts_per_layer=0),
    "no_parts": lambda d: d.update(parts=[]),
    "no_layers": lambda d: d.pop("moe_layers"),
}


@pytest.mark.parametrize("brk", sorted(INDEX_BREAKS))
def test_index_rejects(L, layer_store, brk):
    edit_json(layer_store[0]["index"], INDEX_BREAKS[brk])
    assert not L.sepia_hip_index_load(layer_store[0]["index"].encode())


def test_store_calls_without_gpu_fail_cleanly(L, smoke):
    """Uploads need an initialized device; without one they return NULL."""
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK):
        pytest.skip("a GPU is present")
    t = L.sepia_hip_manifest_load(smoke["manifest"].encode(), smoke["bin"].encode())
    idx = L.sepia_hip_index_load(smoke["index"].encode())
    try:
        assert t and idx
        assert not L.sepia_hip_manifest_upload(t)
        out = (hip.ExpertTensor * 3)()
        assert not L.sepia_hip_index_upload_layer(idx, None, 0, out)
    finally:
        L.sepia_hip_manifest_free(t)
        L.sepia_hip_index_free(idx)
