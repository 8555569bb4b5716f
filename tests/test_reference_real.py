"""The reference's own real-model host path driving this library.

oracle/_ref/sepia_hip is the reference's unmodified src/sepia.c linked
against libsepia_hip.so (oracle/Makefile, target ref). Pointed at a complete
synthetic model in the real checkpoint's formats (sepia_amd/store_synth.py
write_tiny_model: config.json, tokenizer.bin, GGUF parts, the sepia-index
sidecar, resident.bin and its manifest) through its
SEPIA_REAL_{CONFIG,MANIFEST,INDEX,TOKENIZER}_PATH overrides
(src/sepia.c:6214-6217), it runs:

  --real --logits-only          the CPU engine: real_forward_chunk with
                                qlinear (double accumulate) and the streamed
                                routed experts of real_expert_ffn
                                (src/sepia.c:4158-4212, :2993-3017);
  --metal --real --logits-only  the same prompt through real_forward_chunk_gpu
                                (src/sepia.c:3387-4120): every resident
                                weight read from the wrapped resident.bin,
                                attention on rel_project_off / banded_attn,
                                and real_mlp_moe_forward_gpu (:3831-3974) per
                                token -- router matvec_off, host routing,
                                the GPU-resident expert cache filled by the
                                loader threads, matvec_q x 3 + silu_mul per
                                expert, host combine;
  --metal --real --n-gen N      greedy decode on the GPU path, which prints
                                each token's wall time.

The GPU run's top-10 first-token logits must match the CPU run's within
the reference's op gate (2e-4 of the largest logit), ids included except
where two CPU logits are that close; the greedy tokens must match too.
"""
import json
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, ROOT
from sepia_amd import store_synth

BIN = os.path.join(ROOT, "oracle", "_ref", "sepia_hip")
TOKENIZER = os.path.join(GOLDEN, "tokenizer", "mini.bin")
PROMPT = "hello the thing in the end, hello"
TOL = 2e-4

needs_bin = pytest.mark.skipif(not os.path.exists(BIN),
                               reason="oracle/_ref/sepia_hip not built (the reference checkout was absent at build)")


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("tiny_model"))
    paths = store_synth.write_tiny_model(d, np.random.default_rng(2024), TOKENIZER)
    env = dict(os.environ, SEPIA_REAL_CONFIG_PATH=paths["config"], SEPIA_REAL_MANIFEST_PATH=paths["manifest"],
               SEPIA_REAL_INDEX_PATH=paths["index"], SEPIA_REAL_TOKENIZER_PATH=paths["tokenizer"])
    return paths, env


def run(env, *args, timeout=300):
    r = subprocess.run([BIN, *args, "--prompt", PROMPT], capture_output=True, env=env, timeout=timeout)
    return r.returncode, r.stdout.decode("utf-8", "replace"), r.stderr.decode("utf-8", "replace")


def top10(out):
    rows = re.findall(r"\[(\d)\] id=(\d+) logit=(-?[\d.]+(?:e-?\d+)?)", out)
    assert len(rows) == 10, out
    return [int(i) for _, i, _ in rows], np.array([float(v) for _, _, v in rows])


def generated(out):
    """(token id, wall ms) per generated token of real_generate(_gpu)."""
    rows = re.findall(r"^(\d+)\t.*\t([\d.]+) ms$", out, flags=re.M)
    return [int(t) for t, _ in rows], [float(ms) for _, ms in rows]


def compare_top10(cpu, gpu):
    (ci, cv), (gi, gv) = cpu, gpu
    scale = float(np.max(np.abs(cv)))
    print("top-10 logits: max|gpu - cpu| %.3e (bar %.3e)" % (float(np.max(np.abs(gv - cv))), TOL * scale))
    assert np.max(np.abs(gv - cv)) <= TOL * scale, (cv, gv)
    for k in range(10):
        if gi[k] == ci[k]:
            continue
        # a swap is allowed only across a near-tie of the CPU's own logits
        j = ci.index(gi[k]) if gi[k] in ci else None
        assert j is not None and abs(cv[j] - cv[k]) <= 2 * TOL * scale, (k, ci, gi, cv, gv)


@needs_bin
def test_reference_cpu_real_path_runs_on_the_synthetic_model(tiny):
    """The reference's own loader (real_load: config, tokenizer, manifest,
    index and GGUF parts, every shape/size check) accepts the synthetic
    model, and its CPU engine produces finite, distinct top logits."""
    _paths, env = tiny
    rc, out, err = run(env, "--real", "--logits-only")
    assert rc == 0, err
    ids, vals = top10(out)
    assert np.all(np.isfinite(vals)) and len(set(ids)) == 10 and vals[0] > vals[9], out


@needs_bin
@pytest.mark.gpu
def test_reference_real_gpu_path_matches_its_cpu_path(tiny):
    _paths, env = tiny
    rc, cpu_out, err = run(env, "--real", "--logits-only")
    assert rc == 0, err
    rc, gpu_out, gerr = run(env, "--metal", "--real", "--logits-only")
    assert rc == 0, gerr
    assert "sepia: metal: resident.bin wrapped" in gerr and "expert-cache" in gerr, gerr
    print(gpu_out)
    compare_top10(top10(cpu_out), top10(gpu_out))


@needs_bin
@pytest.mark.gpu
def test_reference_real_gpu_decode_matches_its_cpu_decode(tiny):
    """Greedy decode through the prompt's prefill and 6 further tokens (the
    GPU path's KV cache, short-conv histories and expert cache carried across
    calls): the same tokens as the CPU engine, and each decode step's wall
    time as the reference prints it."""
    _paths, env = tiny
    rc, cpu_out, err = run(env, "--real", "--n-gen", "6")
    assert rc == 0, err
    rc, gpu_out, gerr = run(env, "--metal", "--real", "--n-gen", "6")
    assert rc == 0, gerr
    ct, _ = generated(cpu_out)
    gt, gms = generated(gpu_out)
    assert len(ct) == len(gt) >= 1 and ct == gt, (cpu_out, gpu_out)
    print("reference host path on this library: first token (prefill) %.1f ms, decode tokens %s ms"
          % (gms[0], gms[1:]))


# ---------------------------------------------------------- the C3 shape --
# The same host path on a model whose MoE layer is C3 in the real
# checkpoint's formats (hidden 6144, moe_intermediate 3072, 256 routed
# IQ2_XS/IQ3_XXS experts, 2 shared Q5_K/Q6_K, top-6; layer 0 dense, layer 1
# MoE), against what the same binary's CPU engine computed on it
# (tests/golden/make_ref_host_c3.py, ref_host_c3_real.json).
C3_GOLDEN = os.path.join(GOLDEN, "ref_host_c3_real.json")


def write_c3_model(out_dir, golden, sparse=True):
    g = golden
    return store_synth.write_tiny_model(out_dir, np.random.default_rng(g["seed"]), TOKENIZER,
                                        n_layers=g["n_layers"], hidden=g["hidden"], moe_inter=g["moe_inter"],
                                        n_routed=g["n_routed"], sparse=sparse,
                                        expert_types=tuple(g["expert_types"]))


def env_of(paths):
    return dict(os.environ, SEPIA_REAL_CONFIG_PATH=paths["config"], SEPIA_REAL_MANIFEST_PATH=paths["manifest"],
                SEPIA_REAL_INDEX_PATH=paths["index"], SEPIA_REAL_TOKENIZER_PATH=paths["tokenizer"])


@pytest.fixture(scope="module")
def c3model(tmp_path_factory):
    with open(C3_GOLDEN) as f:
        golden = json.load(f)
    d = tmp_path_factory.mktemp("c3_model")
    if shutil.disk_usage(str(d)).free < (12 << 30):
        pytest.skip("the C3-shaped model needs 4.6 GB of scratch space (12 GB free asked)")
    paths = write_c3_model(str(d / "moe"), golden)
    dense = write_c3_model(str(d / "dense"), golden, sparse=False)
    return golden, paths, env_of(paths), env_of(dense)


def warm_decode_ms(env, n_gen, *extra):
    """Greedy tokens of both runs of --repeat 2 and the second (warm) run's
    decode-step wall times (its first line carries the prefill's)."""
    rc, out, err = run(env, "--metal", "--real", "--n-gen", str(n_gen), "--repeat", "2", *extra)
    assert rc == 0, err
    toks, ms = generated(out)
    half = len(toks) // 2
    assert len(toks) == 2 * half and half >= 2, out
    return toks[:half], toks[half:], ms[half + 1:]


@needs_bin
@pytest.mark.gpu
def test_reference_host_path_at_c3_shape(c3model):
    """real_forward_chunk_gpu / real_mlp_moe_forward_gpu (src/sepia.c:3387-4120,
    :3831-3974) through this library at the C3 shape: the prompt's top-10
    logits within the reference's op gate of its CPU engine's, and its greedy
    tokens equal to the CPU engine's on a cold and a warm expert cache. The
    warm decode-step wall time is printed beside the same binary's on the
    model with a dense FFN in place of the MoE layer."""
    golden, _paths, env, env_dense = c3model
    rc, out, err = run(env, "--metal", "--real", "--logits-only", "--expert-cache-gb", "6")
    assert rc == 0, err
    ref = (golden["top10_ids"], np.array(golden["top10_logits"]))
    compare_top10(ref, top10(out))
    cold, warm, ms = warm_decode_ms(env, golden["n_gen"], "--expert-cache-gb", "6")
    assert cold == golden["tokens"] and warm == golden["tokens"], (cold, warm, golden["tokens"])
    _c, _w, ms_dense = warm_decode_ms(env_dense, golden["n_gen"])
    print("reference host path, C3-shaped MoE model, warm decode step ms: %s (median %.3f); "
          "the same model with a dense FFN in layer 1: %s (median %.3f)"
          % (ms, float(np.median(ms)), ms_dense, float(np.median(ms_dense))))


@pytest.mark.gpu
def test_fused_decode_on_the_c3_model(c3model):
    """The C3-shaped model's MoE layer taken from its own stores by this
    library (sepia_hip_manifest_upload, sepia_hip_index_upload_layer,
    sepia_hip_moe_layer_from_stores) and run by sepia_gpu_moe_decode: the
    eager per-call time through the C ABI, for comparison with the
    reference's host path on the same bytes."""
    import ctypes
    import time

    from sepia_amd import hip

    golden, paths, _env, _env_dense = c3model
    dev = hip.Device()
    L, H = dev.L, golden["hidden"]
    t = L.sepia_hip_manifest_load(paths["manifest"].encode(), os.path.join(os.path.dirname(paths["manifest"]),
                                                                            "resident.bin").encode())
    idx = L.sepia_hip_index_load(paths["index"].encode())
    assert t and idx
    rbuf = L.sepia_hip_manifest_upload(t)
    ex = (hip.ExpertTensor * 3)()
    ebuf = L.sepia_hip_index_upload_layer(idx, None, 1, ex)
    assert rbuf and ebuf
    desc = hip.MoeLayerDesc()
    bufs = [rbuf, ebuf]
    try:
        cfg = paths["cfg"]["text_config"]
        assert L.sepia_hip_moe_layer_from_stores(t, rbuf, 1, ex, golden["n_routed"], 6, cfg["route_scale"],
                                                 ctypes.byref(desc)) == 1
        xs = [dev.shared_from(np.random.default_rng(k).standard_normal(H).astype(np.float32)) for k in range(8)]
        yb, rb = dev.alloc(H * 4), dev.alloc(64 * 4)
        bufs += xs + [yb, rb]
        for b in xs:
            dev.run(L.sepia_gpu_moe_decode, ctypes.byref(desc), b, yb, rb)
        y = dev.download(yb, H)
        assert np.all(np.isfinite(y)) and np.max(np.abs(y)) > 0
        n = 400
        dev.begin()
        t0 = time.perf_counter()
        for i in range(n):
            assert L.sepia_gpu_moe_decode(ctypes.byref(desc), xs[i % len(xs)], yb, rb)
        dev.end()
        us = (time.perf_counter() - t0) / n * 1e6
        print("sepia_gpu_moe_decode on the C3-shaped model's MoE layer: %.1f us per call "
              "(eager through the C ABI, %d calls in one batch)" % (us, n))
    finally:
        for b in bufs:
            dev.free(b)
        L.sepia_hip_manifest_free(t)
        L.sepia_hip_index_free(idx)
