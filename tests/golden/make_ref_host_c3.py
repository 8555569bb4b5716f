#!/usr/bin/env python3
"""Writes tests/golden/ref_host_c3_real.json: what the reference's own CPU
engine (oracle/_ref/sepia_hip, its unmodified src/sepia.c built by
oracle/Makefile) computes on a synthetic model whose MoE layer has the C3
shape in the real checkpoint's formats -- hidden 6144, moe_intermediate
3072, 256 routed experts (IQ2_XS gate/up, IQ3_XXS down) and 2 shared
(Q5_K gate/up, Q6_K down), top-6; layer 0 dense, layer 1 MoE
(sepia_amd/store_synth.py write_tiny_model, seed 2024, 4.6 GB of GGUF parts).

Recorded: the top-10 first-token logits of the prompt (`--real
--logits-only`, src/sepia.c:4158-4212) and the greedy tokens of `--real
--n-gen 8` (real_generate). tests/test_reference_real.py runs the same
binary's `--metal --real` path on this library against them, so the CPU
engine (about a minute at this size) need not run on the GPU box.

Run from the repository root after oracle/_ref is built:
    python tests/golden/make_ref_host_c3.py [scratch_dir]
With --models-only DIR it only writes the model to DIR/moe and its twin
with a dense FFN in layer 1 to DIR/dense (for profiling the GPU path).
"""
import json
import os
import re
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from sepia_amd import store_synth  # noqa: E402

BIN = os.path.join(ROOT, "oracle", "_ref", "sepia_hip")
TOKENIZER = os.path.join(ROOT, "tests", "golden", "tokenizer", "mini.bin")
OUT = os.path.join(ROOT, "tests", "golden", "ref_host_c3_real.json")
SPEC = dict(seed=2024, n_layers=2, hidden=6144, moe_inter=3072, n_routed=256, expert_types=[17, 18, 13, 14],
            prompt="hello the thing in the end, hello", n_gen=8)


def write_model(out_dir, sparse=True):
    return store_synth.write_tiny_model(out_dir, np.random.default_rng(SPEC["seed"]), TOKENIZER,
                                        n_layers=SPEC["n_layers"], hidden=SPEC["hidden"],
                                        moe_inter=SPEC["moe_inter"], n_routed=SPEC["n_routed"], sparse=sparse,
                                        expert_types=tuple(SPEC["expert_types"]))


def env_for(paths):
    return dict(os.environ, SEPIA_REAL_CONFIG_PATH=paths["config"], SEPIA_REAL_MANIFEST_PATH=paths["manifest"],
                SEPIA_REAL_INDEX_PATH=paths["index"], SEPIA_REAL_TOKENIZER_PATH=paths["tokenizer"])


def run(env, *args):
    """stdout of the binary (token pieces need not be whole UTF-8)."""
    r = subprocess.run([BIN, *args, "--prompt", SPEC["prompt"]], env=env, check=True, capture_output=True)
    return r.stdout.decode("utf-8", "replace")


def main():
    if len(sys.argv) == 3 and sys.argv[1] == "--models-only":
        write_model(os.path.join(sys.argv[2], "moe"))
        write_model(os.path.join(sys.argv[2], "dense"), sparse=False)
        return
    scratch = sys.argv[1] if len(sys.argv) > 1 else tempfile.mkdtemp(prefix="ref-host-c3-")
    paths = write_model(os.path.join(scratch, "model"))
    env = env_for(paths)
    top = run(env, "--real", "--logits-only")
    rows = re.findall(r"\[(\d)\] id=(\d+) logit=(-?[\d.]+(?:e-?\d+)?)", top)
    assert len(rows) == 10, top
    gen = run(env, "--real", "--n-gen", str(SPEC["n_gen"]))
    tokens = [int(t) for t in re.findall(r"^(\d+)\t", gen, flags=re.M)]
    assert tokens, gen
    out = dict(SPEC, top10_ids=[int(i) for _, i, _ in rows], top10_logits=[float(v) for _, _, v in rows],
               tokens=tokens)
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print("wrote", OUT, out["top10_ids"], tokens)


if __name__ == "__main__":
    main()
