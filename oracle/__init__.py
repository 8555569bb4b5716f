"""ctypes bindings for the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg, as the checker. The product (sepia_amd/) never
imports this package.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_quants.so")

# GGUF type ids (reference src/quants.h:6-10; tools/gguf_inspect.py:62-84).
F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ4_XS = (
    0, 1, 8, 10, 11, 12, 13, 14, 16, 17, 18, 23)
TYPE_NAMES = {F32: "f32", F16: "f16", Q8_0: "q8_0", Q2_K: "q2_k", Q3_K: "q3_k", Q4_K: "q4_k",
              Q5_K: "q5_k", Q6_K: "q6_k", IQ2_XXS: "iq2_xxs", IQ2_XS: "iq2_xs",
              IQ3_XXS: "iq3_xxs", IQ4_XS: "iq4_xs"}
# (elements per block, bytes per block)
GEOM = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110),
        Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), IQ2_XXS: (256, 66),
        IQ2_XS: (256, 74), IQ3_XXS: (256, 98), IQ4_XS: (256, 136)}
# Byte offsets of the f16 scale fields inside one block.
F16_FIELDS = {Q8_0: (0,), Q2_K: (80, 82), Q3_K: (108,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,),
              IQ2_XXS: (0,), IQ2_XS: (0,), IQ3_XXS: (0,), IQ4_XS: (0,)}
# Types the reference's src/quants.c decodes (src/quants.c:28-56).
REF_TYPES = (F16, Q8_0, Q4_K, Q5_K, Q6_K, IQ2_XS, IQ3_XXS, IQ4_XS)

_lib = None


def build(force=False):
    """Compile liboracle.so (and oracle/_ref when the reference is present)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def build_ref():
    if os.path.isdir("/root/reference/src"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        c_p, c_i64, c_sz, c_f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float
        L.orc_supported.argtypes = [ctypes.c_int]
        L.orc_row_bytes.argtypes = [ctypes.c_int, c_i64]
        L.orc_row_bytes.restype = c_sz
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = c_f
        L.orc_set_iq2xxs_grid.argtypes = [c_p]
        L.orc_dequantize_row.argtypes = [ctypes.c_int, c_p, c_p, c_i64]
        L.orc_qlinear.argtypes = [ctypes.c_int, c_p, c_i64, c_i64, c_p, c_p, ctypes.c_int]
        L.orc_linear_f32.argtypes = [c_p, c_i64, c_i64, c_p, c_p]
        for fn in ("orc_sigmoid", "orc_silu", "orc_logsigmoid"):
            getattr(L, fn).argtypes = [c_f]
            getattr(L, fn).restype = c_f
        L.orc_silu_mul.argtypes = [c_p, c_p, c_p, c_i64]
        L.orc_route_topk.argtypes = [c_p, c_p, ctypes.c_int, ctypes.c_int, c_p]
        L.orc_route_weights.argtypes = [c_p, ctypes.c_int, ctypes.c_int, c_p, ctypes.c_int,
                                        ctypes.c_double, ctypes.c_double, c_p]
        L.orc_route_select.argtypes = [c_p, c_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_double, ctypes.c_double, c_p, c_p]
        L.orc_expert_ffn.argtypes = [ctypes.c_int, c_p, ctypes.c_int, c_p, ctypes.c_int, c_p,
                                     c_i64, c_i64, c_p, c_p, ctypes.c_int]
        L.orc_moe_layer.argtypes = [c_p, c_p, c_p, c_p, c_p, c_p, c_p, ctypes.c_int]
        L.orc_rel_project.argtypes = [c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64]
        L.orc_rel_project.restype = None
        L.orc_banded_attn.argtypes = [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i64, c_i64, c_i64,
                                      c_i64, c_i64, c_f]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(t, n):
    be, bb = GEOM[t]
    assert n % be == 0
    return n // be * bb


def set_iq2xxs_grid(grid):
    """Install an IQ2_XXS codebook (256 x u64) or None to remove it."""
    if grid is None:
        lib().orc_set_iq2xxs_grid(None)
        return
    g = np.ascontiguousarray(grid, dtype=np.uint64)
    assert g.shape == (256,)
    lib().orc_set_iq2xxs_grid(_ptr(g))


def dequantize(t, raw, n):
    raw = np.ascontiguousarray(np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw)
    out = np.empty(n, dtype=np.float32)
    if not lib().orc_dequantize_row(t, _ptr(raw), _ptr(out), n):
        raise ValueError("oracle: cannot dequantize type %d n=%d" % (t, n))
    return out


def qlinear(t, w, out_dim, in_dim, x, threads=1):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert w.nbytes >= out_dim * row_bytes(t, in_dim) and x.size == in_dim
    y = np.empty(out_dim, dtype=np.float32)
    if not lib().orc_qlinear(t, _ptr(w), out_dim, in_dim, _ptr(x), _ptr(y), threads):
        raise ValueError("oracle: qlinear failed")
    return y


def linear_f32(w, x):
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(w.shape[0], dtype=np.float32)
    lib().orc_linear_f32(_ptr(w), w.shape[0], w.shape[1], _ptr(x), _ptr(y))
    return y


def silu_mul(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    z = np.empty_like(g)
    lib().orc_silu_mul(_ptr(g), _ptr(u), _ptr(z), g.size)
    return z


def route_select(logits, bias, n_routed, n_shared, topk, route_scale, global_scale):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    idx = np.empty(topk, dtype=np.int32)
    w = np.empty(topk + n_shared, dtype=np.float32)
    lib().orc_route_select(_ptr(logits), _ptr(bias), n_routed, n_shared, topk,
                           route_scale, global_scale, _ptr(idx), _ptr(w))
    return idx, w


def route_weights(logits, n_routed, n_shared, idx, route_scale, global_scale):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    w = np.empty(idx.size + n_shared, dtype=np.float32)
    lib().orc_route_weights(_ptr(logits), n_routed, n_shared, _ptr(idx), idx.size,
                            route_scale, global_scale, _ptr(w))
    return w


def expert_ffn(tg, gate, tu, up, td, down, hidden, inter, x, threads=1):
    arrs = [np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down)]
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(hidden, dtype=np.float32)
    ok = lib().orc_expert_ffn(tg, _ptr(arrs[0]), tu, _ptr(arrs[1]), td, _ptr(arrs[2]),
                              hidden, inter, _ptr(x), _ptr(y), threads)
    if not ok:
        raise ValueError("oracle: expert_ffn failed")
    return y


class _MoeLayer(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int64), ("inter", ctypes.c_int64),
                ("n_routed", ctypes.c_int), ("n_shared", ctypes.c_int), ("topk", ctypes.c_int),
                ("route_scale", ctypes.c_double), ("global_scale", ctypes.c_double),
                ("router_w", ctypes.c_void_p), ("router_bias", ctypes.c_void_p),
                ("t_gate", ctypes.c_int), ("t_up", ctypes.c_int), ("t_down", ctypes.c_int),
                ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
                ("ts_gate", ctypes.c_int), ("ts_up", ctypes.c_int), ("ts_down", ctypes.c_int),
                ("s_gate", ctypes.c_void_p), ("s_up", ctypes.c_void_p), ("s_down", ctypes.c_void_p)]


def moe_layer(spec, x, force_idx=None, threads=1):
    """spec: dict with hidden, inter, n_routed, n_shared, topk, route_scale, global_scale,
    router_w [n_tot, hidden] f32, router_bias [n_routed] f32, types (t_gate, t_up, t_down,
    ts_gate, ts_up, ts_down) and byte arrays gate/up/down (lists, indexable by expert;
    None allowed for experts never selected) and s_gate/s_up/s_down (lists).
    Returns (y, logits, idx, weights)."""
    keep = []

    def ptr_table(arrs):
        tab = (ctypes.c_void_p * len(arrs))()
        for i, a in enumerate(arrs):
            if a is None:
                tab[i] = None
                continue
            a = np.ascontiguousarray(a, dtype=np.uint8)
            keep.append(a)
            tab[i] = a.ctypes.data
        keep.append(tab)
        return ctypes.cast(tab, ctypes.c_void_p)

    rw = np.ascontiguousarray(spec["router_w"], dtype=np.float32)
    rb = np.ascontiguousarray(spec["router_bias"], dtype=np.float32)
    L = _MoeLayer(spec["hidden"], spec["inter"], spec["n_routed"], spec["n_shared"], spec["topk"],
                  spec["route_scale"], spec["global_scale"], rw.ctypes.data, rb.ctypes.data,
                  spec["t_gate"], spec["t_up"], spec["t_down"],
                  ptr_table(spec["gate"]), ptr_table(spec["up"]), ptr_table(spec["down"]),
                  spec["ts_gate"], spec["ts_up"], spec["ts_down"],
                  ptr_table(spec["s_gate"]), ptr_table(spec["s_up"]), ptr_table(spec["s_down"]))
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_tot = spec["n_routed"] + spec["n_shared"]
    y = np.empty(spec["hidden"], dtype=np.float32)
    logits = np.empty(n_tot, dtype=np.float32)
    idx = np.empty(spec["topk"], dtype=np.int32)
    w = np.empty(spec["topk"] + spec["n_shared"], dtype=np.float32)
    fi = None
    if force_idx is not None:
        fi = np.ascontiguousarray(force_idx, dtype=np.int32)
        keep.append(fi)
    ok = lib().orc_moe_layer(ctypes.byref(L), _ptr(x), _ptr(y), _ptr(fi) if fi is not None else None,
                             _ptr(logits), _ptr(idx), _ptr(w), threads)
    if not ok:
        raise ValueError("oracle: moe_layer failed")
    return y, logits, idx, w


def rel_project(r_vec, rel_proj, T, H, d_rel, rel_extent):
    r_vec = np.ascontiguousarray(r_vec, dtype=np.float32)
    rel_proj = np.ascontiguousarray(rel_proj, dtype=np.float32)
    out = np.empty(T * H * rel_extent, dtype=np.float32)
    lib().orc_rel_project(_ptr(r_vec), _ptr(rel_proj), _ptr(out), T, H, d_rel, rel_extent)
    return out


def banded_attn(q, k, v, rel_logits, kv_lo, kv_hi, tau, T, H, Hkv, Dh, rel_extent, q_pos_base, kv_dim,
                inv_head_dim):
    arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, rel_logits, tau)]
    lo = np.ascontiguousarray(kv_lo, dtype=np.int64)
    hi = np.ascontiguousarray(kv_hi, dtype=np.int64)
    out = np.empty(T * H * Dh, dtype=np.float32)
    ok = lib().orc_banded_attn(_ptr(arrs[0]), _ptr(arrs[1]), _ptr(arrs[2]), _ptr(arrs[3]), _ptr(out), _ptr(lo),
                               _ptr(hi), _ptr(arrs[4]), T, H, Hkv, Dh, rel_extent, q_pos_base, kv_dim,
                               ctypes.c_float(inv_head_dim))
    if not ok:
        raise ValueError("oracle: banded_attn rejected its arguments")
    return out


# ---------------------------------------------------------------- reference
_ref = None


def ref_lib():
    """The reference's own src/quants.c, compiled into oracle/_ref (None if absent)."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB_PATH):
        R = ctypes.CDLL(REF_LIB_PATH)
        R.dequantize_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        R.dequantize_row.restype = None
        R.quants_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int64]
        R.quants_row_bytes.restype = ctypes.c_size_t
        _ref = R
    return _ref


def ref_dequantize(t, raw, n):
    """Decode with the reference's own dequantize_row (types in REF_TYPES only:
    the reference exits the process on any other type)."""
    assert t in REF_TYPES or t == F32
    R = ref_lib()
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    R.dequantize_row(t, _ptr(raw), _ptr(out), n)
    return out
