"""The sidecar parsers (store.c, json.c) on damaged files, on the host (no
GPU): seeded truncations, byte flips, insertions and deep nesting of a valid
resident-manifest.json and index.json. Every call must either refuse the
file (NULL, one log line) or return a table that frees cleanly; none may
crash. The reference's loaders exit on such files (src/sepia.c:1876-1910,
:2010-2080); this library returns NULL instead.

The mutated files are parsed in a child process, so a crash is reported as
this test's failure rather than ending the test run."""
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import ROOT
from sepia_amd import store_synth

CHILD = r"""
import sys
sys.path.insert(0, sys.argv[1])
from sepia_amd import hip
L = hip.load()
kind, bin_path = sys.argv[2], sys.argv[3]
ok = bad = 0
for path in sys.argv[4:]:
    if kind == "manifest":
        t = L.sepia_hip_manifest_load(path.encode(), bin_path.encode())
        if t:
            L.sepia_hip_manifest_free(t)
    else:
        t = L.sepia_hip_index_load(path.encode())
        if t:
            L.sepia_hip_index_free(t)
    ok += bool(t)
    bad += not t
print("parsed", ok, "refused", bad)
"""


def mutations(text, rng, n):
    """n damaged copies of text: cut short, bytes flipped, bytes inserted,
    a run deleted, or a value replaced by deep nesting."""
    raw = text.encode("utf-8")
    out = []
    for i in range(n):
        b = bytearray(raw)
        kind = i % 5
        if kind == 0:
            b = b[:int(rng.integers(0, len(b)))]
        elif kind == 1:
            for _ in range(int(rng.integers(1, 8))):
                b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        elif kind == 2:
            at = int(rng.integers(0, len(b)))
            b[at:at] = bytes(rng.choice(list(b'{}[]",:\\0123456789-.eE truefalsenull'), int(rng.integers(1, 6))))
        elif kind == 3:
            at = int(rng.integers(0, len(b)))
            del b[at:at + int(rng.integers(1, 64))]
        else:
            depth = int(rng.integers(50, 5000))
            at = b.find(b":", int(rng.integers(0, len(b))))
            at = at if at >= 0 else b.find(b":")
            b[at + 1:at + 1] = b"[" * depth + b"1" + b"]" * (depth if i % 2 else depth // 2)
        out.append(bytes(b))
    return out


def run_child(kind, bin_path, paths):
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT, kind, bin_path, *paths], capture_output=True,
                       timeout=300)
    # the log lines may quote the damaged bytes
    err = r.stderr.decode("utf-8", "replace")
    assert r.returncode == 0, (r.returncode, err[-2000:])
    return r.stdout.decode()


@pytest.mark.parametrize("kind", ["manifest", "index"])
def test_damaged_sidecars_refused_without_crash(tmp_path, kind):
    paths, _host = store_synth.write_layer_store(str(tmp_path / "store"), np.random.default_rng(31), layer=3,
                                                 hidden=512, inter=256, n_routed=4, n_shared=2,
                                                 types=(17, 18, 13, 14), n_parts=2, extra_layers=(7,))
    src = paths["manifest"] if kind == "manifest" else paths["index"]
    with open(src, encoding="utf-8") as f:
        text = f.read()
    rng = np.random.default_rng(4242 if kind == "manifest" else 4243)
    files = []
    for i, data in enumerate(mutations(text, rng, 400)):
        p = str(tmp_path / ("m%03d.json" % i))
        with open(p, "wb") as f:
            f.write(data)
        files.append(p)
    out = run_child(kind, paths["bin"], [src] + files)
    parsed, refused = (int(v) for v in out.split()[1::2])
    assert parsed >= 1 and parsed + refused == len(files) + 1, out
    # most damage must be caught; the untouched original parses
    assert refused >= len(files) // 2, out
