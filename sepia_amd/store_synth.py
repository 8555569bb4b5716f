"""Synthetic on-disk stores in the reference's formats, for tests and the
benchmark (host side, numpy + stdlib).

Writes what the reference's tools produce from a real checkpoint, from
their documented layouts (reference docs/container.md:123-257):

* GGUF v3 parts (the public GGUF layout: magic, version, tensor and
  metadata counts, metadata key/values, tensor infos with dims fastest
  first, then the data section at the general.alignment boundary, each
  tensor at an aligned offset);
* the sepia-index sidecar (tools/make_index.py:282-323): parts[], and per
  MoE layer gate/up/down blocks with the per-expert
  {part_file, abs_offset, nbytes, ggml_type} entries, abs_offset =
  data_start + tensor offset + e * bytes_per_expert;
* resident.bin + resident-manifest.json (tools/extract_resident.py:
  131-230): every non-expert tensor appended at 64-byte alignment, the
  manifest listing {name, ggml_type, shape, offset, nbytes, sha256, ...};
* the smoke fixture of tools/make_smoke_fixture.py (2 Q8_0 experts with
  byte-tagged blocks, 3 resident tensors, a Q8_0 qlinear case) and its
  smoke_expected.json, which the reference's `sepia --smoke DIR` checks.
"""
import hashlib
import json
import os
import struct

import numpy as np

from . import synth

GGUF_TYPE_UINT32, GGUF_TYPE_STRING = 4, 8
TYPE_NAMES = {0: "F32", 1: "F16", 8: "Q8_0", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K",
              16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS", 23: "IQ4_XS"}
RESIDENT_ALIGNMENT = 64
GGUF_DIR = "inkling-gguf"


def tensor_nbytes(t, dims):
    """Bytes of a GGUF tensor of ggml type t and dims (fastest first)."""
    be, bb = synth.GEOM[t]
    n = int(np.prod(dims))
    if dims[0] % be:
        raise ValueError("row of %d is not a whole number of %d-element blocks" % (dims[0], be))
    return n // be * bb


def _s(x):
    raw = x.encode("utf-8")
    return struct.pack("<Q", len(raw)) + raw


def _align(n, a):
    return (n + a - 1) // a * a


def write_gguf(path, tensors, alignment=32):
    """tensors: [(name, dims, ggml_type, bytes)]. Returns (data_start, {name: offset})."""
    offsets, pos = {}, 0
    for name, _dims, _t, data in tensors:
        pos = _align(pos, alignment)
        offsets[name] = pos
        pos += len(data)
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 2))
    head += _s("general.architecture") + struct.pack("<I", GGUF_TYPE_STRING) + _s("sepia-synthetic")
    head += _s("general.alignment") + struct.pack("<II", GGUF_TYPE_UINT32, alignment)
    for name, dims, t, _data in tensors:
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, offsets[name])
    data_start = _align(len(head), alignment)
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "wb") as f:
        f.write(bytes(head) + b"\0" * (data_start - len(head)))
        for name, _dims, _t, data in tensors:
            f.write(b"\0" * (data_start + offsets[name] - f.tell()))
            f.write(data)
    return data_start, offsets


class Store:
    """Accumulates GGUF parts, then writes index.json, resident.bin and
    resident-manifest.json beside them (out_dir/inkling-gguf/<part>)."""

    def __init__(self, out_dir, n_experts):
        self.out = out_dir
        self.n_experts = n_experts
        self.parts = []          # index parts[] entries
        self.moe = {}            # layer -> kind -> block
        self.resident = []       # (name, t, dims, abs_offset, nbytes, part_file)

    def add_part(self, part_file, tensors, alignment=32):
        """tensors: [(name, dims, ggml_type, bytes)]; expert tensors are named
        blk.<L>.ffn_{gate,up,down}_exps.weight with dims [.., .., n_experts]."""
        path = os.path.join(self.out, GGUF_DIR, part_file)
        data_start, offsets = write_gguf(path, tensors, alignment)
        size = os.path.getsize(path)
        self.parts.append({"part_file": part_file, "source": "local", "expected_size_bytes": size,
                           "local_size_bytes": size, "data_start": data_start, "alignment": alignment})
        for name, dims, t, data in tensors:
            off = offsets[name]
            assert len(data) == tensor_nbytes(t, dims), name
            fields = name.split(".")
            if len(fields) == 4 and fields[0] == "blk" and fields[2] in ("ffn_gate_exps", "ffn_up_exps",
                                                                          "ffn_down_exps"):
                layer, kind = int(fields[1]), fields[2][4:-5]
                assert dims[-1] == self.n_experts and len(data) % self.n_experts == 0
                bpe = len(data) // self.n_experts
                self.moe.setdefault(layer, {})[kind] = {
                    "tensor_name": name, "part_file": part_file, "source": "local", "ggml_type": t,
                    "ggml_type_name": TYPE_NAMES[t], "data_start": data_start, "tensor_offset": off,
                    "n_bytes_total": len(data), "n_expert": self.n_experts, "bytes_per_expert": bpe,
                    "experts": [{"part_file": part_file, "abs_offset": data_start + off + e * bpe, "nbytes": bpe,
                                 "ggml_type": t} for e in range(self.n_experts)]}
            else:
                self.resident.append((name, t, list(dims), data_start + off, len(data), part_file))

    def write(self):
        """index.json, resident.bin and resident-manifest.json; returns their paths."""
        index = {"generated_at": "synthetic", "source_repo": "sepia/synthetic", "quant": "SYNTH",
                 "alignment": self.parts[0]["alignment"], "n_experts_per_layer": self.n_experts,
                 "n_moe_layers_indexed": len(self.moe),
                 "n_expert_tensor_entries": 3 * self.n_experts * len(self.moe),
                 "parts": self.parts,
                 "resident_tensors": [{"name": n, "part_file": pf, "source": "local", "abs_offset": ao,
                                       "nbytes": nb, "ggml_type": t, "ggml_type_name": TYPE_NAMES[t], "shape": d}
                                      for n, t, d, ao, nb, pf in self.resident],
                 "moe_layers": {str(layer): kinds for layer, kinds in sorted(self.moe.items())}}
        index_path = os.path.join(self.out, "index.json")
        with open(index_path, "w") as f:
            json.dump(index, f, indent=2)
            f.write("\n")
        bin_path = os.path.join(self.out, "resident.bin")
        tensors = []
        with open(bin_path, "wb") as dst:
            for name, t, dims, abs_off, nbytes, pf in self.resident:
                with open(os.path.join(self.out, GGUF_DIR, pf), "rb") as src:
                    src.seek(abs_off)
                    data = src.read(nbytes)
                start = _align(dst.tell(), RESIDENT_ALIGNMENT)
                dst.write(b"\0" * (start - dst.tell()))
                dst.write(data)
                tensors.append({"name": name, "ggml_type": t, "ggml_type_name": TYPE_NAMES[t], "shape": dims,
                                "offset": start, "nbytes": nbytes, "sha256": hashlib.sha256(data).hexdigest(),
                                "source_part_file": pf, "source_abs_offset": abs_off})
        manifest = {"generated_at": "synthetic", "resident_bin_path": bin_path,
                    "resident_bin_size": os.path.getsize(bin_path), "alignment": RESIDENT_ALIGNMENT,
                    "n_resident_tensors_total": len(tensors), "n_tensors_extracted": len(tensors),
                    "tensors": tensors, "pending_parts": []}
        manifest_path = os.path.join(self.out, "resident-manifest.json")
        with open(manifest_path, "w") as f:
            json.dump(manifest, f, indent=2)
            f.write("\n")
        return index_path, bin_path, manifest_path


# ------------------------------------------------------------ smoke fixture --
def _q8_0_matrix(out_dim, in_dim, scale):
    """Q8_0 rows with a distinct int8 pattern each (small integers, a
    power-of-two scale: every product and partial sum is exact in f32)."""
    raw, rows = bytearray(), []
    for r in range(out_dim):
        vals = []
        for b in range(in_dim // 32):
            ints = [((j + 7 * r + 3 * b) % 32) - 16 for j in range(32)]
            raw += struct.pack("<e", scale) + struct.pack("<32b", *ints)
            vals += [scale * v for v in ints]
        rows.append(vals)
    return bytes(raw), rows


def write_smoke_fixture(out_dir):
    """The fixture `sepia --smoke DIR` checks (reference src/sepia.c:4312-4446):
    layer 0 with 2 routed Q8_0 experts of one block each, byte-tagged per
    expert; F32 token_embd_norm / output_norm and a Q8_0 blk.0.attn_r.weight
    [32 -> 3]; smoke_expected.json with each expert slice's offset, size and
    first 8 bytes, the resident offsets, and the qlinear x and y (y summed in
    double and rounded to f32, exact here)."""
    n_exp = 2
    store = Store(out_dir, n_exp)
    tag = lambda base: b"".join(bytes([(base + e) % 256]) * 34 for e in range(n_exp))
    q8, rows = _q8_0_matrix(3, 32, 0.5)
    x = [float(i + 1) for i in range(32)]
    y = [float(np.float32(sum(a * b for a, b in zip(row, x)))) for row in rows]
    part = "SMOKE/smoke-00001-of-00001.gguf"
    store.add_part(part, [
        ("token_embd_norm.weight", [4], 0, struct.pack("<4f", 1, 2, 3, 4)),
        ("output_norm.weight", [4], 0, struct.pack("<4f", 5, 6, 7, 8)),
        ("blk.0.attn_r.weight", [32, 3], 8, q8),
        ("blk.0.ffn_gate_exps.weight", [32, 1, n_exp], 8, tag(0)),
        ("blk.0.ffn_up_exps.weight", [32, 1, n_exp], 8, tag(50)),
        ("blk.0.ffn_down_exps.weight", [32, 1, n_exp], 8, tag(100)),
    ])
    index_path, bin_path, manifest_path = store.write()
    layer0 = store.moe[0]
    experts = []
    with open(os.path.join(out_dir, GGUF_DIR, part), "rb") as f:
        for e in range(n_exp):
            ent = {"expert": e}
            for kind in ("gate", "up", "down"):
                s = layer0[kind]["experts"][e]
                f.seek(s["abs_offset"])
                ent[kind] = {"abs_offset": s["abs_offset"], "nbytes": s["nbytes"], "first8_hex": f.read(8).hex()}
            experts.append(ent)
    with open(manifest_path) as f:
        by_name = {t["name"]: t for t in json.load(f)["tensors"]}
    expected = {"layer": 0, "n_experts": n_exp, "experts": experts,
                "resident": [{"name": n, "offset": by_name[n]["offset"], "nbytes": by_name[n]["nbytes"]}
                             for n in ("token_embd_norm.weight", "output_norm.weight", "blk.0.attn_r.weight")],
                "qlinear": {"tensor_name": "blk.0.attn_r.weight", "x": x, "y": y}}
    with open(os.path.join(out_dir, "smoke_expected.json"), "w") as f:
        json.dump(expected, f, indent=2)
        f.write("\n")
    return {"index": index_path, "bin": bin_path, "manifest": manifest_path, "q8": q8, "x": x, "y": y}


# ------------------------------------------------------------- layer stores --
def write_layer_store(out_dir, rng, layer, hidden, inter, n_routed, n_shared, types, n_parts=1,
                      extra_layers=()):
    """A MoE layer in the reference's formats, with random block contents
    (synth.random_matrix: f16 scales in [2^-10, 2^-6]): routed experts'
    gate/up/down as 3-D tensors (types[0] gate/up, types[1] down) spread over
    n_parts GGUF parts (gate/up/down of a layer in different parts when
    n_parts > 1); resident router ffn_gate_inp.weight (f32, N(0, 0.02)),
    exp_probs_b.bias (U(-0.1, 0.1)), ffn_gscale.weight (1.0) and the shared
    stacks ffn_{gate,up,down}_shexp.weight (types[2] gate/up, types[3] down).
    extra_layers: other layer numbers with the same shapes (more tensors in
    the parts). Returns (paths, host arrays for the oracle)."""
    tg, td, tsg, tsd = types
    store = Store(out_dir, n_routed)
    parts = [[] for _ in range(n_parts)]
    host = {}
    for li, L in enumerate((layer,) + tuple(extra_layers)):
        gate = [synth.random_matrix(tg, inter, hidden, rng) for _ in range(n_routed)]
        up = [synth.random_matrix(tg, inter, hidden, rng) for _ in range(n_routed)]
        down = [synth.random_matrix(td, hidden, inter, rng) for _ in range(n_routed)]
        rw = (rng.standard_normal((n_routed + n_shared, hidden)) * 0.02).astype(np.float32)
        rb = rng.uniform(-0.1, 0.1, n_routed).astype(np.float32)
        sg = [synth.random_matrix(tsg, inter, hidden, rng) for _ in range(n_shared)]
        su = [synth.random_matrix(tsg, inter, hidden, rng) for _ in range(n_shared)]
        sd = [synth.random_matrix(tsd, hidden, inter, rng) for _ in range(n_shared)]
        exp = [("blk.%d.ffn_gate_exps.weight" % L, [hidden, inter, n_routed], tg, b"".join(m.tobytes() for m in gate)),
               ("blk.%d.ffn_up_exps.weight" % L, [hidden, inter, n_routed], tg, b"".join(m.tobytes() for m in up)),
               ("blk.%d.ffn_down_exps.weight" % L, [inter, hidden, n_routed], td, b"".join(m.tobytes() for m in down))]
        for k, ten in enumerate(exp):
            parts[(k + li) % n_parts].append(ten)
        res = [("blk.%d.ffn_gate_inp.weight" % L, [hidden, n_routed + n_shared], 0, rw.tobytes()),
               ("blk.%d.exp_probs_b.bias" % L, [n_routed], 0, rb.tobytes()),
               ("blk.%d.ffn_gscale.weight" % L, [1], 0, np.float32(1.0).tobytes())]
        if n_shared:
            res += [("blk.%d.ffn_gate_shexp.weight" % L, [hidden, inter, n_shared], tsg, b"".join(m.tobytes() for m in sg)),
                    ("blk.%d.ffn_up_shexp.weight" % L, [hidden, inter, n_shared], tsg, b"".join(m.tobytes() for m in su)),
                    ("blk.%d.ffn_down_shexp.weight" % L, [inter, hidden, n_shared], tsd,
                     b"".join(m.tobytes() for m in sd))]
        parts[0].extend(res)
        host[L] = dict(hidden=hidden, inter=inter, n_routed=n_routed, n_shared=n_shared, router_w=rw, router_bias=rb,
                       t_gate=tg, t_up=tg, t_down=td, ts_gate=tsg, ts_up=tsg, ts_down=tsd, gate=gate, up=up, down=down,
                       s_gate=sg, s_up=su, s_down=sd)
    for p in range(n_parts):
        store.add_part("SYNTH/synth-%05d-of-%05d.gguf" % (p + 1, n_parts), parts[p])
    index_path, bin_path, manifest_path = store.write()
    return {"index": index_path, "bin": bin_path, "manifest": manifest_path, "store": store}, host


# -------------------------------------------------------------- tiny model --
def tiny_config(n_layers=4, hidden=512, vocab=272, unpadded=266, moe_inter=256, n_routed=16, sparse=True):
    """A small model config in the reference's config.json layout
    (docs/inkling-config.json; read by src/sepia.c:455-560): sliding and
    global attention layers of different head geometries, one dense FFN
    layer then MoE layers (every layer dense if not sparse), top-6 of
    n_routed routed experts plus 2 shared. The log-scaling floor is low
    enough that the attention temperature tau changes within a short
    prompt."""
    layer_types = ["hybrid_sliding" if (i % 3) != 2 else "hybrid" for i in range(n_layers)]
    return {"architectures": ["InklingForConditionalGeneration"], "model_type": "inkling_mm_model",
            "text_config": {
                "hidden_size": hidden, "num_hidden_layers": n_layers, "vocab_size": vocab,
                "unpadded_vocab_size": unpadded,
                "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 64,
                "swa_num_attention_heads": 4, "swa_num_key_value_heads": 4, "swa_head_dim": 32,
                "sliding_window_size": 8, "layer_types": layer_types,
                "mlp_layer_types": ["dense"] + ["sparse" if sparse else "dense"] * (n_layers - 1),
                "d_rel": 16, "rel_extent": 32, "conv_kernel_size": 4,
                "intermediate_size": 512, "moe_intermediate_size": moe_inter,
                "n_routed_experts": n_routed, "num_experts_per_tok": 6, "n_shared_experts": 2,
                "route_scale": 8.0, "logits_mup_width_multiplier": 24.0, "rms_norm_eps": 1e-6,
                "log_scaling_alpha": 0.1, "log_scaling_n_floor": 4}}


# The real checkpoint's per-layer expert formats (reference
# docs/gguf-inventory-ud-q2_k_xl.md:72-111, :214-235): routed gate/up IQ2_XS
# with IQ3_XXS or IQ4_XS down, shared gate/up Q5_K with Q6_K down; the
# attention projections Q8_0, token_embd Q5_K and output Q4_K.
TINY_EXPERT_TYPES = ((17, 18, 13, 14), (17, 23, 13, 14), (18, 18, 13, 14))


def _f32(name, dims, arr):
    return (name, list(dims), 0, np.asarray(arr, dtype=np.float32).tobytes())


def _q(name, t, in_dim, out_dim, rng, stack=None):
    n = 1 if stack is None else stack
    data = b"".join(synth.random_matrix(t, out_dim, in_dim, rng).tobytes() for _ in range(n))
    dims = [in_dim, out_dim] + ([] if stack is None else [stack])
    return (name, dims, t, data)


def write_tiny_model(out_dir, rng, tokenizer_src, n_layers=4, n_parts=2, hidden=512, moe_inter=256, n_routed=16,
                     sparse=True, expert_types=None):
    """A complete model in the reference's real-checkpoint formats, by
    default small enough to build in seconds (hidden, moe_inter and n_routed
    set the MoE layers' shape; expert_types, a (gate/up, down, shared
    gate/up, shared down) type tuple, replaces the per-layer rotation of
    TINY_EXPERT_TYPES; sparse=False makes every layer dense): config.json,
    tokenizer.bin (copied from
    tokenizer_src, an SPTK v1 sidecar), GGUF parts under inkling-gguf/, the
    sepia-index sidecar (index.json) and resident.bin + its manifest. Every
    tensor real_load resolves (reference src/sepia.c:2647-2861) is present:
    token_embd / output / their norms, per layer the attention norms,
    projections, relative-position projection and short-conv weights, the
    dense FFN of layer 0, and for each MoE layer the router, its bias, the
    global scale and the shared-expert stacks, with the routed experts as
    3-D GGUF tensors reached through the index. Block contents are random
    (f16 scales in [2^-10, 2^-6]); f32 norms ~ 1 + N(0, 0.1), short-conv taps
    and relative projections ~ N(0, 0.3). Returns the four paths the
    reference reads through SEPIA_REAL_{CONFIG,MANIFEST,INDEX,TOKENIZER}_PATH."""
    cfg = tiny_config(n_layers, hidden=hidden, moe_inter=moe_inter, n_routed=n_routed, sparse=sparse)
    tc = cfg["text_config"]
    H, V = tc["hidden_size"], tc["vocab_size"]
    K, d_rel, inter = tc["conv_kernel_size"], tc["d_rel"], tc["moe_intermediate_size"]
    n_r, n_s = tc["n_routed_experts"], tc["n_shared_experts"]
    norm = lambda n: 1.0 + 0.1 * rng.standard_normal(n)
    small = lambda n: 0.3 * rng.standard_normal(n)
    store = Store(out_dir, n_r)
    parts = [[] for _ in range(n_parts)]
    parts[0] += [_q("token_embd.weight", 13, H, V, rng), _q("output.weight", 12, H, V, rng),
                 _f32("token_embd_norm.weight", [H], norm(H)), _f32("output_norm.weight", [H], norm(H))]
    for L in range(n_layers):
        sliding = tc["layer_types"][L] == "hybrid_sliding"
        nh = tc["swa_num_attention_heads"] if sliding else tc["num_attention_heads"]
        nkv = tc["swa_num_key_value_heads"] if sliding else tc["num_key_value_heads"]
        dh = tc["swa_head_dim"] if sliding else tc["head_dim"]
        ext = tc["sliding_window_size"] if sliding else tc["rel_extent"]
        q_dim, kv_dim = nh * dh, nkv * dh
        p = "blk.%d." % L
        res = [_f32(p + "attn_norm.weight", [H], norm(H)), _f32(p + "ffn_norm.weight", [H], norm(H)),
               _f32(p + "attn_q_norm.weight", [dh], norm(dh)), _f32(p + "attn_k_norm.weight", [dh], norm(dh)),
               _f32(p + "attn_rel_proj.weight", [d_rel, ext], small(d_rel * ext)),
               _f32(p + "shortconv_k.weight", [K, kv_dim], small(K * kv_dim)),
               _f32(p + "shortconv_v.weight", [K, kv_dim], small(K * kv_dim)),
               _f32(p + "shortconv_attn.weight", [K, H], small(K * H)),
               _f32(p + "shortconv_mlp.weight", [K, H], small(K * H)),
               _q(p + "attn_q.weight", 8, H, q_dim, rng), _q(p + "attn_k.weight", 8, H, kv_dim, rng),
               _q(p + "attn_v.weight", 8, H, kv_dim, rng), _q(p + "attn_r.weight", 8, H, nh * d_rel, rng),
               _q(p + "attn_output.weight", 8, q_dim, H, rng)]
        if tc["mlp_layer_types"][L] == "dense":
            di = tc["intermediate_size"]
            res += [_q(p + "ffn_gate.weight", 12, H, di, rng), _q(p + "ffn_up.weight", 12, H, di, rng),
                    _q(p + "ffn_down.weight", 14, di, H, rng), _f32(p + "ffn_gscale.weight", [1], [1.25])]
        else:
            tg, td, tsg, tsd = expert_types or TINY_EXPERT_TYPES[L % len(TINY_EXPERT_TYPES)]
            res += [_f32(p + "ffn_gate_inp.weight", [H, n_r + n_s], 0.02 * rng.standard_normal((n_r + n_s) * H)),
                    _f32(p + "exp_probs_b.bias", [n_r], rng.uniform(-0.1, 0.1, n_r)),
                    _f32(p + "ffn_gscale.weight", [1], [0.75]),
                    _q(p + "ffn_gate_shexp.weight", tsg, H, inter, rng, stack=n_s),
                    _q(p + "ffn_up_shexp.weight", tsg, H, inter, rng, stack=n_s),
                    _q(p + "ffn_down_shexp.weight", tsd, inter, H, rng, stack=n_s)]
            exps = [_q(p + "ffn_gate_exps.weight", tg, H, inter, rng, stack=n_r),
                    _q(p + "ffn_up_exps.weight", tg, H, inter, rng, stack=n_r),
                    _q(p + "ffn_down_exps.weight", td, inter, H, rng, stack=n_r)]
            for k, ten in enumerate(exps):
                parts[(k + L) % n_parts].append(ten)
        parts[L % n_parts] += res
    for i in range(n_parts):
        store.add_part("TINY/tiny-%05d-of-%05d.gguf" % (i + 1, n_parts), parts[i])
    index_path, _bin_path, manifest_path = store.write()
    config_path = os.path.join(out_dir, "config.json")
    with open(config_path, "w") as f:
        json.dump(cfg, f, indent=2)
        f.write("\n")
    tok_path = os.path.join(out_dir, "tokenizer.bin")
    with open(tokenizer_src, "rb") as src, open(tok_path, "wb") as dst:
        dst.write(src.read())
    return {"config": config_path, "manifest": manifest_path, "index": index_path, "tokenizer": tok_path,
            "cfg": cfg}
