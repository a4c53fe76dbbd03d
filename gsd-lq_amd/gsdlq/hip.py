"""ctypes binding of libgsdhip.so (C ABI in include/gsdhip.h).

There is no CPU fallback: loading fails with RuntimeError when the library is
not built, and every call raises RuntimeError with the library's error text
when it returns a nonzero status (the reference raised RuntimeError on OpenCL
buffer/launch failures, gsd_lq_v2/run_gpu_native_chat.py:606-607,648-649).
"""
from __future__ import annotations

import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# GSD_HIP_LIB: another build of the engine library (e.g. to compare two
# builds on one machine); the in-tree build otherwise
LIB_PATH = os.environ.get("GSD_HIP_LIB") or os.path.join(_PKG_DIR, "libgsdhip.so")

vp, i32, i64, u64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float

# name -> argtypes (restype int unless noted)
SIGNATURES = {
    "gsdh_device_info": [ctypes.c_char_p, i32, ctypes.POINTER(u64), ctypes.POINTER(i32)],
    "gsdh_malloc": [ctypes.POINTER(vp), u64],
    "gsdh_free": [vp],
    "gsdh_memcpy_h2d": [vp, vp, u64, vp],
    "gsdh_memcpy_d2h": [vp, vp, u64, vp],
    "gsdh_stream_sync": [vp],
    "gsdh_stream_create": [ctypes.POINTER(vp)],
    "gsdh_stream_destroy": [vp],
    "gsdh_stream_begin_capture": [vp],
    "gsdh_stream_end_capture": [vp, ctypes.POINTER(vp)],
    "gsdh_graph_replay": [vp, vp],
    "gsdh_attention_workspace_create": [vp, i32, i32, i32, i32],
    "gsdh_attention_workspace_destroy": [vp],
    "gsdh_stream_copy": [vp, vp, vp, u64],
    "gsdh_rmsnorm": [vp, vp, vp, vp, i32, f32],
    "gsdh_vec_add": [vp, vp, vp, vp, i32],
    "gsdh_swiglu": [vp, vp, vp, vp, i32],
    "gsdh_lowrank_proj": [vp, vp, vp, vp, vp, i32, i32],
    "gsdh_hex2d_matvec": [vp] + [vp] * 10 + [i32] * 4,
    "gsdh_rope_and_store_kv": [vp] + [vp] * 5 + [i32] * 6 + [f32, i32],
    "gsdh_gqa_attention": [vp] + [vp] * 4 + [i32] * 6 + [f32],
    "gsdh_rope_store_gqa_attention": [vp] + [vp] * 6 + [i32] * 6 + [f32, i32, f32],
    "gsdh_gqa_attention_noalloc": [vp] + [vp] * 4 + [i32] * 6 + [f32],
    "gsdh_prefill_attention": [vp] + [vp] * 4 + [i32] * 7 + [f32],
    "gsdh_unpack_codes": [vp, vp, i64, i32, vp, vp],
    "gsdh_model_create": [vp, ctypes.POINTER(vp)],
    "gsdh_model_destroy": [vp],
    "gsdh_model_set_embedding": [vp, vp],
    "gsdh_model_set_norm": [vp, i32, i32, vp],
    "gsdh_model_set_hex": [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, i64, vp, vp, vp],
    "gsdh_model_finalize": [vp],
    "gsdh_forward_token": [vp, i32, i32, i32, vp, ctypes.POINTER(i32)],
    "gsdh_generate_greedy": [vp, vp, i32, i32, i32, vp, vp],
    "gsdh_model_run_linear": [vp, i32, i32],
    "gsdh_model_matmul": [vp, i32, i32, vp, i32, vp],
    "gsdh_model_matmul_shared": [vp, i32, ctypes.POINTER(i32), i32, vp, i32, ctypes.POINTER(vp)],
    "gsdh_matmul_plan": [i32, i32, i32, ctypes.POINTER(i32), ctypes.POINTER(i32), ctypes.POINTER(i32)],
    "gsdh_model_read_codes": [vp, i32, i32, vp],
    "gsdh_model_capture_begin": [vp],
    "gsdh_model_capture_end": [vp, ctypes.POINTER(vp)],
    "gsdh_graph_launch": [vp, vp, i32],
    "gsdh_graph_destroy": [vp],
    "gsdh_graph_time": [vp, vp, i32, ctypes.POINTER(f32)],
    "gsdh_greedy_argmax": [vp, vp, i32, vp, vp],
    "gsdh_greedy_argmax_split": [vp, vp, i32, vp, vp, vp, vp],
    "gsdh_model_vector": [vp, i32, i32, vp, u64],
    "gsdh_model_set_step": [vp, i32, i32],
    "gsdh_model_read_kv": [vp, i32, i32, vp, vp],
    "gsdh_model_prefill": [vp, vp, i32, i32, i32, vp, ctypes.POINTER(i32)],
    "gsdh_model_set_prefill": [vp, i32],
}
RESTYPES = {"gsdh_model_device_bytes": (u64, [vp]), "gsdh_model_stream": (vp, [vp]),
            "gsdh_attention_workspace_bytes": (u64, [i32, i32, i32, i32]),
            "gsdh_model_fused_ffn": (i32, [vp, i32]),
            "gsdh_last_error": (ctypes.c_char_p, [])}


class GsdModelConfig(ctypes.Structure):
    _fields_ = [("n_layers", i32), ("hidden", i32), ("ffn", i32), ("n_heads", i32),
                ("n_kv_heads", i32), ("head_dim", i32), ("vocab", i32), ("max_seq_len", i32),
                ("rope_interleaved", i32), ("rms_eps", f32), ("rope_theta", f32)]


VECTORS = {"x": 0, "q": 1, "k": 2, "v": 3, "attn": 4, "h": 5, "logits": 6}

SLOTS = {"attn_q": 0, "attn_k": 1, "attn_v": 2, "attn_output": 3, "ffn_gate": 4, "ffn_up": 5,
         "ffn_down": 6, "output": 7}


class HipError(RuntimeError):
    pass


class _Lib:
    def __init__(self, path: str = LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"HIP engine library {path} is not built (run __graft_entry__.build()); "
                               "there is no CPU fallback")
        self.path = path
        self.cdll = ctypes.CDLL(path)
        for name, args in SIGNATURES.items():
            fn = getattr(self.cdll, name)
            fn.argtypes = args
            fn.restype = i32
        for name, (rt, args) in RESTYPES.items():
            fn = getattr(self.cdll, name)
            fn.argtypes = args
            fn.restype = rt

    def last_error(self) -> str:
        e = self.cdll.gsdh_last_error()
        return e.decode() if e else ""

    def __getattr__(self, name):
        fn = getattr(self.cdll, name)
        if name in SIGNATURES:
            def call(*args):
                rc = fn(*args)
                if rc != 0:
                    raise HipError(f"{name} failed ({rc}): {self.last_error()}")
                return rc
            return call
        return fn


_lib = None


def lib() -> _Lib:
    global _lib
    if _lib is None:
        _lib = _Lib()
    return _lib


def device_info():
    name = ctypes.create_string_buffer(256)
    total = u64(0)
    ncu = i32(0)
    lib().gsdh_device_info(name, 256, ctypes.byref(total), ctypes.byref(ncu))
    return name.value.decode(errors="replace"), int(total.value), int(ncu.value)


def ptr(a):
    """Device pointer of a torch tensor, host pointer of a numpy array, or None."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return ctypes.c_void_p(a.data_ptr())
    return a.ctypes.data_as(ctypes.c_void_p)
