"""ctypes bindings to libsepia_hip.so: the C ABI of include/sepia_gpu.h
(the reference's src/sepia_gpu.h) plus include/sepia_hip_ext.h.

Python is plumbing here: every call goes straight through the C ABI, the way
the reference engine (src/sepia.c) would call it. There is no fallback: if
the library or its code object is missing, or the device cannot be
initialised, these helpers raise.
"""
import ctypes
import os
import re

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libsepia_hip.so")
HSACO_PATH = os.path.join(LIB_DIR, "sepia_kernels.hsaco")
INCLUDE_DIR = os.path.join(os.path.dirname(PKG), "include")


class SepiaHipError(RuntimeError):
    pass


class ExpertTensor(ctypes.Structure):
    _fields_ = [("buf", ctypes.c_void_p), ("off", ctypes.c_size_t), ("stride", ctypes.c_size_t),
                ("ggml_type", ctypes.c_int)]


class MoeLayerDesc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int64), ("inter", ctypes.c_int64),
                ("n_routed", ctypes.c_int), ("n_shared", ctypes.c_int), ("topk", ctypes.c_int),
                ("route_scale", ctypes.c_float), ("global_scale", ctypes.c_float),
                ("router_w", ctypes.c_void_p), ("router_w_off", ctypes.c_size_t),
                ("router_bias", ctypes.c_void_p), ("router_bias_off", ctypes.c_size_t),
                ("gate", ExpertTensor), ("up", ExpertTensor), ("down", ExpertTensor),
                ("s_gate", ExpertTensor), ("s_up", ExpertTensor), ("s_down", ExpertTensor)]


class ResidentTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("ggml_type", ctypes.c_int), ("n_dims", ctypes.c_int),
                ("shape", ctypes.c_int64 * 4), ("offset", ctypes.c_int64), ("nbytes", ctypes.c_int64)]


class ExpertSlot(ctypes.Structure):
    _fields_ = [("part_idx", ctypes.c_int), ("abs_offset", ctypes.c_int64), ("nbytes", ctypes.c_int64),
                ("ggml_type", ctypes.c_int)]


_P, _SZ, _I64, _F, _I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int64, ctypes.c_float, ctypes.c_int
_RT = ctypes.POINTER(ResidentTensor)
PROTOTYPES = {
    # name: (restype, argtypes)
    "sepia_gpu_available": (_I, []),
    "sepia_gpu_init": (_I, [ctypes.c_char_p]),
    "sepia_gpu_shutdown": (None, []),
    "sepia_gpu_device_name": (ctypes.c_char_p, []),
    "sepia_gpu_wrap_mmap": (_P, [_P, _SZ]),
    "sepia_gpu_alloc": (_P, [_SZ, _I]),
    "sepia_gpu_free": (None, [_P]),
    "sepia_gpu_host_ptr": (_P, [_P]),
    "sepia_gpu_gpu_addr": (ctypes.c_uint64, [_P]),
    "sepia_gpu_selftest_touch": (_I, [_P, _SZ]),
    "sepia_gpu_begin": (_I, []),
    "sepia_gpu_flush": (_I, []),
    "sepia_gpu_end": (_I, []),
    "sepia_gpu_rmsnorm": (_I, [_P, _P, _P, _I64, _I64, _F]),
    "sepia_gpu_matvec": (_I, [_P, _P, _P, _I64, _I64]),
    "sepia_gpu_silu_mul": (_I, [_P, _P, _P, _I64]),
    "sepia_gpu_add": (_I, [_P, _P, _P, _I64]),
    "sepia_gpu_softmax": (_I, [_P, _P, _I64, _I64]),
    "sepia_gpu_sconv": (_I, [_P, _P, _P, _P, _I64, _I64, _I64]),
    "sepia_gpu_matvec_q": (_I, [_I, _P, _SZ, _P, _P, _I64, _I64]),
    "sepia_gpu_dequant_rows": (_I, [_I, _P, _SZ, _P, _I64]),
    "sepia_gpu_rel_project": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64]),
    "sepia_gpu_banded_attn": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                   _I64, _F]),
    "sepia_gpu_matvec_off": (_I, [_P, _SZ, _P, _P, _I64, _I64]),
    "sepia_gpu_rmsnorm_off": (_I, [_P, _SZ, _P, _P, _I64, _I64, _F]),
    "sepia_gpu_sconv_off": (_I, [_P, _SZ, _P, _P, _P, _I64, _I64, _I64]),
    "sepia_gpu_rel_project_off": (_I, [_P, _P, _SZ, _P, _I64, _I64, _I64, _I64]),
    "sepia_gpu_copy": (_I, [_P, _SZ, _P, _SZ, _I64]),
    "sepia_gpu_scale": (_I, [_F, _P, _P, _I64]),
    "sepia_gpu_sconv_hist_roll": (_I, [_P, _P, _I64, _I64, _I64]),
    "sepia_gpu_moe_decode": (_I, [ctypes.POINTER(MoeLayerDesc), _P, _P, _P]),
    "sepia_gpu_moe_prefill": (_I, [ctypes.POINTER(MoeLayerDesc), ctypes.c_int64, _P, _P, _P]),
    "sepia_hip_moe_decode_noalloc": (_I, [ctypes.POINTER(MoeLayerDesc), _P, _P, _P]),
    "sepia_gpu_expert_ffn": (_I, [ctypes.POINTER(ExpertTensor), ctypes.POINTER(ExpertTensor),
                                  ctypes.POINTER(ExpertTensor), _I, _I, _I64, _I64, _P, _P]),
    "sepia_hip_profile_start": (_I, []),
    "sepia_hip_profile_stop": (_I, []),
    "sepia_hip_profile_query": (_I, [ctypes.c_char_p, ctypes.POINTER(_I64), ctypes.POINTER(ctypes.c_double)]),
    "sepia_hip_profile_reset": (None, []),
    "sepia_hip_synth_blocks": (_I, [_I, _P, _SZ, _I64, ctypes.c_uint64, _F, _F]),
    "sepia_hip_set_iq2xxs_grid": (_I, [_P]),
    "sepia_hip_reserve_scratch": (_I, [_SZ]),
    "sepia_hip_uploaded_bytes": (ctypes.c_uint64, []),
    "sepia_hip_take_device_error": (ctypes.c_uint, []),
    "sepia_hip_scratch_bytes": (ctypes.c_size_t, []),
    "sepia_hip_alloc_count": (ctypes.c_uint64, []),
    "sepia_hip_read_probe": (_I, [_P, _SZ, _SZ, ctypes.c_uint]),
    "sepia_hip_read_probe_dma": (_I, [_P, _SZ, _SZ, ctypes.c_uint, ctypes.c_uint, _I, _I]),
    "sepia_hip_stream": (_P, []),
    "sepia_hip_set_option": (_I, [ctypes.c_char_p, _I]),
    # the on-disk stores (store.c)
    "sepia_hip_manifest_load": (_P, [ctypes.c_char_p, ctypes.c_char_p]),
    "sepia_hip_manifest_count": (_SZ, [_P]),
    "sepia_hip_manifest_tensor": (_RT, [_P, _SZ]),
    "sepia_hip_manifest_find": (_RT, [_P, ctypes.c_char_p]),
    "sepia_hip_manifest_upload": (_P, [_P]),
    "sepia_hip_manifest_free": (None, [_P]),
    "sepia_hip_index_load": (_P, [ctypes.c_char_p]),
    "sepia_hip_index_n_experts": (_I, [_P]),
    "sepia_hip_index_n_parts": (_I, [_P]),
    "sepia_hip_index_part": (ctypes.c_char_p, [_P, _I]),
    "sepia_hip_index_has_layer": (_I, [_P, _I]),
    "sepia_hip_index_slot": (_I, [_P, _I, _I, _I, ctypes.POINTER(ExpertSlot)]),
    "sepia_hip_index_upload_layer": (_P, [_P, ctypes.c_char_p, _I, ctypes.POINTER(ExpertTensor)]),
    "sepia_hip_index_free": (None, [_P]),
    "sepia_hip_moe_layer_from_stores": (_I, [_P, _P, _I, ctypes.POINTER(ExpertTensor), _I, _I, _F,
                                             ctypes.POINTER(MoeLayerDesc)]),
}

_lib = None


def load():
    """Load libsepia_hip.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH) or not os.path.exists(HSACO_PATH):
            raise SepiaHipError("libsepia_hip.so / sepia_kernels.hsaco not built under %s "
                                "(run __graft_entry__.build())" % LIB_DIR)
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def declared_symbols():
    """Every function name declared in include/*.h."""
    names = set()
    for fn in sorted(os.listdir(INCLUDE_DIR)):
        if fn.endswith(".h"):
            text = open(os.path.join(INCLUDE_DIR, fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names.update(re.findall(r"\b(sepia_\w+)\s*\(", text))
    return names


class Device:
    """The library's one device, through the C ABI."""

    def __init__(self):
        self.L = load()
        # the kernel directory handed to sepia_gpu_init (the reference passes
        # its metal/ directory, src/sepia.c:6181): the built code object, or
        # another build of it named by SEPIA_KERNEL_DIR
        kdir = os.environ.get("SEPIA_KERNEL_DIR", LIB_DIR)
        if not self.L.sepia_gpu_init(kdir.encode()):
            raise SepiaHipError("sepia_gpu_init failed (no MI355X, or the code object did not load)")
        self.name = self.L.sepia_gpu_device_name().decode()

    def check(self, ok, what):
        if not ok:
            raise SepiaHipError("%s failed (see the sepia: hip: log line)" % what)

    # buffers ------------------------------------------------------------
    def alloc(self, nbytes, private=False):
        b = self.L.sepia_gpu_alloc(int(nbytes), 1 if private else 0)
        self.check(b, "alloc(%d)" % nbytes)
        return b

    def free(self, b):
        self.L.sepia_gpu_free(b)

    def upload(self, b, arr, offset=0):
        """Write arr's bytes into a shared buffer's host copy."""
        a = np.ascontiguousarray(arr)
        hp = self.L.sepia_gpu_host_ptr(b)
        self.check(hp, "host_ptr")
        ctypes.memmove(hp + offset, a.ctypes.data, a.nbytes)

    def download(self, b, count, dtype=np.float32, offset=0):
        hp = self.L.sepia_gpu_host_ptr(b)
        self.check(hp, "host_ptr")
        out = np.empty(count, dtype=dtype)
        ctypes.memmove(out.ctypes.data, hp + offset, out.nbytes)
        return out

    def shared_from(self, arr, extra=0):
        a = np.ascontiguousarray(arr)
        b = self.alloc(a.nbytes + extra)
        self.upload(b, a)
        return b

    # batching -------------------------------------------------------------
    def begin(self):
        self.check(self.L.sepia_gpu_begin(), "begin")

    def end(self):
        self.check(self.L.sepia_gpu_end(), "end")

    def run(self, fn, *args):
        """One op in its own batch; raises if it is rejected or the batch fails."""
        self.begin()
        try:
            ok = fn(*args)
        finally:
            end_ok = self.L.sepia_gpu_end()
        self.check(ok, fn.__name__)
        self.check(end_ok, "end")

    def stream(self):
        return self.L.sepia_hip_stream()
