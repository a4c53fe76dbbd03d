"""CPU oracle driver -- TEST INFRASTRUCTURE ONLY.

Loads either this repository's C restatement (oracle/libgsdref.so, kind
"port") or the reference engine compiled from its own source
(oracle/_ref/libgsd_cpu.so, kind "reference"), binds the seven gsd_cpu_*
functions exactly as gsd_lq_v2/gsd_lq_cpu_runtime.py:91-108 does, and runs the
per-token forward in the order of gsd_lq_v2/gsd_lq_cpu_runtime.py:302-420.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  The product (gsd-lq_amd/) never does.
"""
from __future__ import annotations

import ctypes
import json
import os
import struct
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
PORT_LIB = os.path.join(ORACLE_DIR, "libgsdref.so")
REF_LIB = os.path.join(ORACLE_DIR, "_ref", "libgsd_cpu.so")
MAX_SEQ_LEN = 2048   # gsd_lq_cpu_runtime.py:22


def build(quiet: bool = True) -> None:
    """Compile the oracle (and the reference engine when its source exists)."""
    r = subprocess.run(["make", "-C", ORACLE_DIR, "all"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    if not quiet:
        print(r.stdout)


def have_reference() -> bool:
    return os.path.exists(REF_LIB)


_libs = {}


def load(kind: str = "port"):
    """kind = "port" (restatement) or "reference" (engine.c built from source)."""
    if kind in _libs:
        return _libs[kind]
    path = PORT_LIB if kind == "port" else REF_LIB
    if not os.path.exists(path):
        if kind == "port":
            build()
        else:
            raise FileNotFoundError(path)
    lib = ctypes.CDLL(path)
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    lib.gsd_cpu_rmsnorm.argtypes = [vp, vp, vp, i32, f32]
    lib.gsd_cpu_vec_add.argtypes = [vp, vp, vp, i32]
    lib.gsd_cpu_swiglu.argtypes = [vp, vp, vp, i32]
    lib.gsd_cpu_lowrank_proj.argtypes = [vp, vp, vp, vp, i32, i32]
    lib.gsd_cpu_hex2d_matvec.argtypes = [vp] * 10 + [i32] * 4
    lib.gsd_cpu_rope_and_store_kv.argtypes = [vp] * 5 + [i32] * 6 + [f32, i32]
    lib.gsd_cpu_gqa_attention.argtypes = [vp] * 4 + [i32] * 6 + [f32]
    for fn in ("gsd_cpu_rmsnorm", "gsd_cpu_vec_add", "gsd_cpu_swiglu", "gsd_cpu_lowrank_proj",
               "gsd_cpu_hex2d_matvec", "gsd_cpu_rope_and_store_kv", "gsd_cpu_gqa_attention"):
        getattr(lib, fn).restype = None
    if kind == "port":
        lib.gsdref_f16_to_f32.argtypes = [vp, vp, ctypes.c_long]
        lib.gsdref_f32_to_f16.argtypes = [vp, vp, ctypes.c_long]
        lib.gsdref_codebook.argtypes = [i32, vp, vp]
        lib.gsdref_codebook.restype = i32
        lib.gsdref_dequant.argtypes = [vp] * 7 + [i32, i32]
    _libs[kind] = lib
    return lib


def P(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# --------------------------------------------------------------------------
# The reference's codebook (gsd_lq_cpu_runtime.py:111-118), restated.
# --------------------------------------------------------------------------
def codebook(radius: int):
    s32 = float(np.sqrt(3.0) / 2.0)
    pts = [[r0 + 0.5 * r1, r1 * s32]
           for r0 in range(-radius, radius + 1)
           for r1 in range(-radius, radius + 1) if abs(r0 + r1) <= radius]
    return np.array(pts, dtype=np.float32), len(pts)


# --------------------------------------------------------------------------
# Thin wrappers with the reference argument order.
# --------------------------------------------------------------------------
def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    load("port").gsdref_f16_to_f32(P(h), P(out), h.size)
    return out


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, dtype=np.uint16)
    load("port").gsdref_f32_to_f16(P(f), P(out), f.size)
    return out


def hex2d_matvec(x, t: dict, tmp_k=None, kind: str = "port") -> np.ndarray:
    """y = fused matvec of packed tensor t (fields as in the .gsd2 file)."""
    lib = load(kind)
    xy, n_pts = codebook(t["radius"])
    rows, cols, k = t["rows"], t["cols"], t["k_dim"]
    y = np.zeros(rows, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    dummy16 = np.zeros(2, dtype=np.uint16)
    tk = np.zeros(16, dtype=np.float32)
    if k > 0:
        if tmp_k is None:
            lib.gsd_cpu_lowrank_proj(P(x), P(t["Vt"]), P(t["S"]), P(tk), k, cols)
        else:
            tk[:k] = tmp_k
    kc = t["kink_cols"] if t["kink_cols"].size else dummy16
    kd = t["kink_deltas"] if t["kink_deltas"].size else np.zeros(1, np.float32)
    lib.gsd_cpu_hex2d_matvec(P(x), P(t["codes"]), P(t["scales"]), P(xy),
                             P(t["U"] if k > 0 else dummy16), P(tk), P(t["row_ptr"]), P(kc), P(kd),
                             P(y), rows, cols, k, n_pts)
    return y


# --------------------------------------------------------------------------
# Minimal .gsd2 reader (gsd_lq_cpu_runtime.py:128-217), independent of the
# product's loader.
# --------------------------------------------------------------------------
class FileSource:
    def __init__(self, path: str):
        with open(path, "rb") as f:
            magic = f.read(4)
            if magic != b"GSD2":
                raise ValueError(f"Invalid GSD2 magic: {magic}")
            hlen = struct.unpack("<Q", f.read(8))[0]
            self.header = json.loads(f.read(hlen).decode("utf-8"))
        self.base = 12 + hlen
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        self.config = self.header["config"]
        self.tensors = self.header["tensors"]

    def _blob(self, meta, dtype):
        o, n = self.base + meta["offset"], meta["nbytes"]
        return np.frombuffer(self.mm[o:o + n], dtype=dtype)

    def dense(self, name, dtype):
        meta = self.tensors[name]["data"]
        a = self._blob(meta, dtype)
        return a.reshape(meta["shape"]) if "shape" in meta else a

    def hex_field(self, name, field):
        dt = {"codes": np.uint8, "scales": np.uint16, "row_ptr": np.uint32, "kink_cols": np.uint16,
              "kink_deltas": np.float32, "U": np.uint16, "S": np.float32, "Vt": np.uint16}[field]
        meta = self.tensors[name]
        if field == "codes" and meta.get("code_bits", 8) == 7:
            # 7-bit stream (this build's extension of the format): code i at
            # bits 7i .. 7i+6, little-endian; decoded bit by bit
            n = meta["rows"] * meta["cols"] // 2
            bits = np.unpackbits(self._blob(meta["codes"], np.uint8), bitorder="little")[:7 * n]
            return (bits.reshape(n, 7).astype(np.uint16) << np.arange(7, dtype=np.uint16)).sum(1).astype(np.uint8)
        return self._blob(meta[field], dt)


class OracleModel:
    """The reference CPU forward (gsd_lq_cpu_runtime.py:302-420) over the
    oracle library.  `source` provides config / tensors / dense() /
    hex_field() (a FileSource, or any object with that surface)."""

    def __init__(self, source, kind: str = "port", max_seq_len: int = MAX_SEQ_LEN,
                 rope_interleaved: int = 1):
        self.lib = load(kind)
        self.kind = kind
        cfg = source.config
        self.cfg = cfg
        self.n_layers, self.hidden = cfg["n_layers"], cfg["hidden_size"]
        self.n_heads, self.n_kv_heads = cfg["n_heads"], cfg["n_kv_heads"]
        self.head_dim, self.ffn_size = cfg["head_dim"], cfg["ffn_size"]
        self.rms_eps, self.rope_theta = cfg["rms_eps"], cfg["rope_theta"]
        self.vocab_size = cfg["vocab_size"]
        self.max_seq_len = max_seq_len
        self.rope_interleaved = rope_interleaved
        self.embed = np.asarray(source.dense("token_embd.weight", np.float16)).astype(np.float32)
        self.tables = {r: codebook(r) for r in range(1, 9)}
        self.d16 = np.zeros(2, dtype=np.uint16)
        self.d32 = np.zeros(1, dtype=np.float32)

        def hexw(name):
            m = source.tensors[name]
            k = m["k_dim"]
            g = lambda f: np.ascontiguousarray(source.hex_field(name, f))
            xy, n_pts = self.tables[m["radius"]]
            d = {"rows": m["rows"], "cols": m["cols"], "k_dim": k, "n_pts": n_pts, "xy": xy,
                 "codes": g("codes"), "scales": g("scales"), "row_ptr": g("row_ptr"),
                 "kink_cols": g("kink_cols"), "kink_deltas": g("kink_deltas")}
            if d["kink_cols"].size == 0:
                d["kink_cols"], d["kink_deltas"] = self.d16, self.d32
            if k > 0:
                d.update(U=g("U"), S=g("S"), Vt=g("Vt"))
            else:
                d.update(U=self.d16, S=self.d32, Vt=self.d16)
            return d

        self.layers = []
        for l in range(self.n_layers):
            p = f"blk.{l}."
            self.layers.append({
                "attn_norm": np.ascontiguousarray(source.dense(p + "attn_norm.weight", np.float32)),
                "ffn_norm": np.ascontiguousarray(source.dense(p + "ffn_norm.weight", np.float32)),
                "q": hexw(p + "attn_q.weight"), "k": hexw(p + "attn_k.weight"),
                "v": hexw(p + "attn_v.weight"), "o": hexw(p + "attn_output.weight"),
                "gate": hexw(p + "ffn_gate.weight"), "up": hexw(p + "ffn_up.weight"),
                "down": hexw(p + "ffn_down.weight")})
        self.final_norm = np.ascontiguousarray(source.dense("output_norm.weight", np.float32))
        self.lm_head = hexw("output.weight")
        kvshape = (self.n_layers, max_seq_len, self.n_kv_heads, self.head_dim)
        self.k_cache = np.zeros(kvshape, dtype=np.uint16)
        self.v_cache = np.zeros(kvshape, dtype=np.uint16)
        kvd = self.n_kv_heads * self.head_dim
        self.x = np.zeros(self.hidden, np.float32)
        self.xb = np.zeros(self.hidden, np.float32)
        self.q = np.zeros(self.n_heads * self.head_dim, np.float32)
        self.k = np.zeros(kvd, np.float32)
        self.v = np.zeros(kvd, np.float32)
        self.attn = np.zeros(self.n_heads * self.head_dim, np.float32)
        self.gate = np.zeros(self.ffn_size, np.float32)
        self.up = np.zeros(self.ffn_size, np.float32)
        self.tmp_k = np.zeros(16, np.float32)
        self.logits = np.zeros(self.vocab_size, np.float32)

    def matvec(self, x, t, out):
        c = self.lib
        if t["k_dim"] > 0:
            c.gsd_cpu_lowrank_proj(P(x), P(t["Vt"]), P(t["S"]), P(self.tmp_k), t["k_dim"], t["cols"])
        c.gsd_cpu_hex2d_matvec(P(x), P(t["codes"]), P(t["scales"]), P(t["xy"]), P(t["U"]),
                               P(self.tmp_k), P(t["row_ptr"]), P(t["kink_cols"]),
                               P(t["kink_deltas"]), P(out), t["rows"], t["cols"], t["k_dim"],
                               t["n_pts"])

    def forward_token(self, token_id: int, pos: int, return_logits: bool = True):
        c = self.lib
        self.x[:] = self.embed[token_id]
        for l, ly in enumerate(self.layers):
            c.gsd_cpu_rmsnorm(P(self.x), P(ly["attn_norm"]), P(self.xb), self.hidden, float(self.rms_eps))
            self.matvec(self.xb, ly["q"], self.q)
            self.matvec(self.xb, ly["k"], self.k)
            self.matvec(self.xb, ly["v"], self.v)
            c.gsd_cpu_rope_and_store_kv(P(self.q), P(self.k), P(self.v), P(self.k_cache),
                                        P(self.v_cache), l, pos, self.n_heads, self.n_kv_heads,
                                        self.head_dim, self.max_seq_len, float(self.rope_theta),
                                        self.rope_interleaved)
            sm_scale = 1.0 / float(np.sqrt(self.head_dim))
            c.gsd_cpu_gqa_attention(P(self.q), P(self.k_cache), P(self.v_cache), P(self.attn), l,
                                    pos, self.n_heads, self.n_kv_heads, self.head_dim,
                                    self.max_seq_len, sm_scale)
            self.matvec(self.attn, ly["o"], self.xb)
            self.x += self.xb
            c.gsd_cpu_rmsnorm(P(self.x), P(ly["ffn_norm"]), P(self.xb), self.hidden, float(self.rms_eps))
            self.matvec(self.xb, ly["gate"], self.gate)
            self.matvec(self.xb, ly["up"], self.up)
            c.gsd_cpu_swiglu(P(self.gate), P(self.up), P(self.gate), self.ffn_size)
            self.matvec(self.gate, ly["down"], self.xb)
            self.x += self.xb
        if not return_logits:
            return None
        c.gsd_cpu_rmsnorm(P(self.x), P(self.final_norm), P(self.xb), self.hidden, float(self.rms_eps))
        self.matvec(self.xb, self.lm_head, self.logits)
        return self.logits.copy()

    @staticmethod
    def greedy(logits) -> int:
        """gsd_lq_cpu_runtime.py:422-425: nan_to_num, then first argmax."""
        lg = np.nan_to_num(logits, nan=-1e4, posinf=100.0, neginf=-1e4)
        return int(np.argmax(lg))

    def generate_greedy(self, prompt, n_new: int):
        """Prefill prompt token by token, then n_new greedy steps.  Returns
        (tokens, margins) where margin = top1 - top2 logit at each step."""
        logits = None
        for pos, tid in enumerate(prompt):
            logits = self.forward_token(int(tid), pos, return_logits=(pos == len(prompt) - 1))
        out, margins = [], []
        pos = len(prompt)
        for _ in range(n_new):
            nxt = self.greedy(logits)
            top2 = np.partition(logits, -2)[-2:]
            margins.append(float(abs(top2[1] - top2[0])))
            out.append(nxt)
            logits = self.forward_token(nxt, pos, return_logits=True)
            pos += 1
        return out, margins
