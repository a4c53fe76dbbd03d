"""ctypes binding of the native encoder (csrc/gsdpack.cpp -> libgsdpack.so).

The reference ships no packer (its loaders only read the format), so the
encoder policy is this project's own; see csrc/gsdpack.cpp for the algorithm.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import codebook

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libgsdpack.so")

_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, u64, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float
    lib.gsdp_codebook.argtypes = [i32, vp, vp]
    lib.gsdp_codebook.restype = i32
    lib.gsdp_synth_bf16.argtypes = [u64, u64, i64, i64, f32, vp]
    lib.gsdp_synth_bf16.restype = None
    lib.gsdp_synth_f16.argtypes = [u64, u64, i64, i64, f32, vp]
    lib.gsdp_synth_f16.restype = None
    lib.gsdp_pack.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.gsdp_pack.restype = i64
    _lib = lib
    return lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def synth_bf16(seed: int, stream: int, n: int, sigma: float = 0.02, offset: int = 0) -> np.ndarray:
    """n float32 values, each exactly representable in bf16, ~N(0, sigma)."""
    out = np.empty(n, dtype=np.float32)
    _load().gsdp_synth_bf16(seed, stream, offset, n, sigma, _p(out))
    return out


def synth_f16(seed: int, stream: int, n: int, sigma: float = 0.02, offset: int = 0) -> np.ndarray:
    """n fp16 bit patterns (uint16), ~N(0, sigma)."""
    out = np.empty(n, dtype=np.uint16)
    _load().gsdp_synth_f16(seed, stream, offset, n, sigma, _p(out))
    return out


_ERRORS = {-1: "unsupported radius", -2: "cols must be a positive multiple of 64",
           -3: "k_dim must be in 0..16", -4: "cols > 65536 (kink columns are u16)"}


def pack_tensor(W: np.ndarray, radius: int, k_dim: int = 0, kinks_per_row: int = 0,
                lr_iters: int = 2) -> dict:
    """Encode W [rows, cols] into the .gsd2 packed-tensor fields."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    rows, cols = W.shape
    cap = rows * max(kinks_per_row, 0)
    f = {
        "codes": np.empty(rows * cols // 2, dtype=np.uint8),
        "scales": np.empty(rows * cols // 64, dtype=np.uint16),
        "row_ptr": np.empty(rows + 1, dtype=np.uint32),
        "kink_cols": np.empty(max(cap, 1), dtype=np.uint16),
        "kink_deltas": np.empty(max(cap, 1), dtype=np.float32),
        "U": np.empty(max(rows * k_dim, 1), dtype=np.uint16),
        "S": np.empty(max(k_dim, 1), dtype=np.float32),
        "Vt": np.empty(max(k_dim * cols, 1), dtype=np.uint16),
    }
    nk = _load().gsdp_pack(_p(W), rows, cols, radius, k_dim, kinks_per_row, lr_iters,
                           _p(f["codes"]), _p(f["scales"]), _p(f["row_ptr"]), _p(f["kink_cols"]),
                           _p(f["kink_deltas"]), _p(f["U"]), _p(f["S"]), _p(f["Vt"]))
    if nk < 0:
        raise ValueError(f"pack_tensor: {_ERRORS.get(nk, nk)} (shape {rows}x{cols}, radius {radius}, k {k_dim})")
    f["kink_cols"] = f["kink_cols"][:nk].copy()
    f["kink_deltas"] = f["kink_deltas"][:nk].copy()
    if k_dim == 0:
        for key in ("U", "S", "Vt"):
            f[key] = f[key][:0]
    f.update({"radius": radius, "rows": rows, "cols": cols, "k_dim": k_dim, "nk": int(nk)})
    return f


def dequantize(f: dict, include_lowrank: bool = True) -> np.ndarray:
    """float64 dense view of a packed tensor (codebook point x fp16 scale, plus
    kinks and the rank-k term); used to measure encoder error."""
    rows, cols, R = f["rows"], f["cols"], f["radius"]
    t = codebook.xy_table(R).astype(np.float64)
    pts = t[f["codes"].astype(np.int64)].reshape(rows, cols)
    s = f["scales"].view(np.float16).astype(np.float64).reshape(rows, cols // 64)
    W = pts * np.repeat(s, 64, axis=1)
    rp = f["row_ptr"].astype(np.int64)
    for r in range(rows):
        for i in range(rp[r], rp[r + 1]):
            W[r, int(f["kink_cols"][i])] += float(f["kink_deltas"][i])
    if include_lowrank and f["k_dim"] > 0:
        k = f["k_dim"]
        U = f["U"].view(np.float16).astype(np.float64).reshape(rows, k)
        Vt = f["Vt"].view(np.float16).astype(np.float64).reshape(k, cols)
        W += U @ (f["S"].astype(np.float64)[:, None] * Vt)
    return W


def packed_nbytes(f: dict) -> int:
    return sum(int(np.asarray(f[k]).nbytes) for k in ("codes", "scales", "row_ptr", "kink_cols",
                                                        "kink_deltas", "U", "S", "Vt"))
