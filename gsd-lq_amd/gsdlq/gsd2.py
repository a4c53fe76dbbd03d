"""The .gsd2 packed-model container: reader and writer.

Layout (the contract both reference loaders read,
gsd_lq_v2/run_gpu_native_chat.py:741-832 and
gsd_lq_v2/gsd_lq_cpu_runtime.py:128-217):

    offset 0       b"GSD2"
    offset 4       u64 little-endian header length hlen
    offset 12      UTF-8 JSON header (hlen bytes)
    offset 12+hlen data region; every blob is {"offset", "nbytes"[, "shape"]}
                   with offset relative to the start of the data region.

Header keys: "config" (model hyper-parameters and the tokenizer vocabulary),
"avg_bpw", "tensors".  Dense tensors carry {"data": blob}; packed ("hex")
tensors carry radius, rows, cols, k_dim and the blobs codes (u8, one per
weight pair), scales (fp16 bits, one per 64 weights), row_ptr (u32, rows+1),
kink_cols (u16), kink_deltas (f32) and, when k_dim > 0, U (fp16 [rows,k]),
S (f32 [k]), Vt (fp16 [k,cols]).

Extension (this build's writer only; the reference's loaders read u8 codes):
a packed tensor whose codebook has at most 128 points (radius <= 6, the
Precision mode) may carry "code_bits": 7, and then its codes blob holds the
rows * cols / 2 codes as one little-endian bit stream of 7 bits each (code
i at bits 7i .. 7i + 6, ceil(7n / 8) bytes): 3.76 instead of 4.26 bits per
weight on disk for a rank-2 Precision model.  Readers return u8 codes either
way.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from typing import Callable, Dict, Iterable, Optional

import numpy as np

MAGIC = b"GSD2"
HEX_FIELDS = ("codes", "scales", "row_ptr", "kink_cols", "kink_deltas")
LOWRANK_FIELDS = ("U", "S", "Vt")
FIELD_DTYPES = {
    "codes": np.uint8,
    "scales": np.uint16,
    "row_ptr": np.uint32,
    "kink_cols": np.uint16,
    "kink_deltas": np.float32,
    "U": np.uint16,
    "S": np.float32,
    "Vt": np.uint16,
}
LAYER_HEX = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
def pack_codes7(codes: np.ndarray) -> np.ndarray:
    """u8 codes (each < 128) as a 7-bit little-endian stream: code i at bits
    7i .. 7i + 6; ceil(7 n / 8) bytes."""
    c = np.ascontiguousarray(codes, dtype=np.uint8).reshape(-1)
    n = c.size
    if n and int(c.max()) >= 128:
        raise ValueError("7-bit codes: a code is >= 128")
    g = np.zeros((n + 7) // 8 * 8, dtype=np.uint64)
    g[:n] = c
    g = g.reshape(-1, 8)
    word = np.zeros(g.shape[0], dtype=np.uint64)
    for j in range(8):               # 8 codes -> one 56-bit group (7 bytes)
        word |= g[:, j] << np.uint64(7 * j)
    out = word.view(np.uint8).reshape(-1, 8)[:, :7].reshape(-1)
    return np.ascontiguousarray(out[:(7 * n + 7) // 8])


def unpack_codes7(blob: np.ndarray, n: int) -> np.ndarray:
    """Inverse of pack_codes7: n u8 codes from the 7-bit stream."""
    b = np.asarray(blob, dtype=np.uint8).reshape(-1)
    if b.size != (7 * n + 7) // 8:
        raise ValueError(f"7-bit codes: {b.size} bytes for {n} codes")
    ng = (n + 7) // 8
    g7 = np.zeros(ng * 7, dtype=np.uint8)
    g7[:b.size] = b
    pad = np.zeros((ng, 8), dtype=np.uint8)
    pad[:, :7] = g7.reshape(ng, 7)
    word = pad.reshape(-1).view(np.uint64)
    out = np.empty((ng, 8), dtype=np.uint8)
    for j in range(8):
        out[:, j] = ((word >> np.uint64(7 * j)) & np.uint64(0x7F)).astype(np.uint8)
    return out.reshape(-1)[:n]


CONFIG_KEYS = ("n_layers", "hidden_size", "n_heads", "n_kv_heads", "head_dim", "ffn_size",
               "rms_eps", "rope_theta", "vocab_size", "tokens", "scores", "token_types",
               "bos_id", "eos_id")


class Gsd2File:
    """Read-only view of a .gsd2 file; blobs are zero-copy numpy views of an mmap."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        magic = self._f.read(4)
        if magic != MAGIC:
            self._f.close()
            raise ValueError(f"Invalid GSD2 magic: {magic}")
        raw = self._f.read(8)
        if len(raw) != 8:
            self._f.close()
            raise ValueError("Truncated GSD2 header length")
        hlen = struct.unpack("<Q", raw)[0]
        hbytes = self._f.read(hlen)
        if len(hbytes) != hlen:
            self._f.close()
            raise ValueError("Truncated GSD2 header")
        self.header = json.loads(hbytes.decode("utf-8"))
        self.data_base = 12 + hlen
        size = os.fstat(self._f.fileno()).st_size
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ) if size > 0 else None
        self.file_size = size

    @property
    def config(self) -> dict:
        return self.header["config"]

    @property
    def tensors(self) -> dict:
        return self.header["tensors"]

    def blob(self, meta: dict, dtype=np.uint8) -> np.ndarray:
        off = self.data_base + int(meta["offset"])
        n = int(meta["nbytes"])
        if off + n > self.file_size:
            raise ValueError(f"GSD2 blob [{off}, {off + n}) beyond end of file ({self.file_size})")
        itemsize = np.dtype(dtype).itemsize
        if n % itemsize:
            raise ValueError(f"GSD2 blob of {n} bytes is not a whole number of {np.dtype(dtype)}")
        if n == 0:
            return np.zeros(0, dtype=dtype)
        return np.frombuffer(self._mm, dtype=dtype, count=n // itemsize, offset=off)

    def hex_field(self, name: str, field: str) -> np.ndarray:
        meta = self.tensors[name]
        bits = int(meta.get("code_bits", 8))
        if field == "codes" and bits != 8:
            if bits != 7 or int(meta["radius"]) > 6:
                raise ValueError(f"{name}: code_bits {bits} with radius {meta['radius']} is not a valid encoding")
            return unpack_codes7(self.blob(meta["codes"], np.uint8), int(meta["rows"]) * int(meta["cols"]) // 2)
        return self.blob(meta[field], FIELD_DTYPES[field])

    def dense(self, name: str, dtype) -> np.ndarray:
        meta = self.tensors[name]["data"]
        arr = self.blob(meta, dtype)
        if "shape" in meta:
            arr = arr.reshape(meta["shape"])
        return arr

    def close(self):
        if self._mm is not None:
            self._mm = None
        if not self._f.closed:
            self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Gsd2Writer:
    """Streams a .gsd2 file.  Blobs are registered with their byte size first
    (optionally as callables producing the bytes later), so that the header,
    which precedes the data, can be written before any blob is produced."""

    ALIGN = 256

    def __init__(self, config: dict, avg_bpw: float):
        missing = [k for k in CONFIG_KEYS if k not in config]
        if missing:
            raise ValueError(f"config lacks keys {missing}")
        self.config = config
        self.avg_bpw = float(avg_bpw)
        self.tensors: Dict[str, dict] = {}
        self._blobs = []          # (offset, nbytes, producer)
        self._cursor = 0

    def _add_blob(self, nbytes: int, producer, shape=None) -> dict:
        off = self._cursor
        meta = {"offset": off, "nbytes": int(nbytes)}
        if shape is not None:
            meta["shape"] = [int(s) for s in shape]
        self._blobs.append((off, int(nbytes), producer))
        self._cursor = off + ((int(nbytes) + self.ALIGN - 1) // self.ALIGN) * self.ALIGN
        return meta

    def add_dense(self, name: str, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        self.tensors[name] = {"data": self._add_blob(arr.nbytes, arr, arr.shape)}

    def add_hex(self, name: str, radius: int, rows: int, cols: int, k_dim: int,
                fields: Optional[dict] = None, nbytes: Optional[dict] = None,
                producer: Optional[Callable[[str], np.ndarray]] = None, code_bits: int = 8):
        """Register a packed tensor.  Either give the arrays (fields) or their
        byte sizes (nbytes) plus producer(field) -> array, called at write time.
        code_bits = 7 stores the codes as a 7-bit stream (radius <= 6; fields only)."""
        meta = {"radius": int(radius), "rows": int(rows), "cols": int(cols), "k_dim": int(k_dim)}
        if code_bits not in (7, 8):
            raise ValueError(f"code_bits {code_bits}: 7 or 8")
        if code_bits == 7:
            if radius > 6:
                raise ValueError(f"{name}: 7-bit codes need a codebook of at most 128 points (radius <= 6)")
            if fields is None:
                raise ValueError("7-bit codes are written from arrays")
            meta["code_bits"] = 7
        names = HEX_FIELDS + (LOWRANK_FIELDS if k_dim > 0 else ())
        for fld in names:
            if fields is not None:
                arr = np.ascontiguousarray(fields[fld], dtype=FIELD_DTYPES[fld])
                if fld == "codes" and code_bits == 7:
                    arr = pack_codes7(arr)
                meta[fld] = self._add_blob(arr.nbytes, arr)
            else:
                meta[fld] = self._add_blob(nbytes[fld], (producer, fld))
        self.tensors[name] = meta

    def write(self, path: str):
        header = {"config": self.config, "avg_bpw": self.avg_bpw, "tensors": self.tensors}
        hbytes = json.dumps(header).encode("utf-8")
        with open(path, "wb") as f:
            f.write(MAGIC)
            f.write(struct.pack("<Q", len(hbytes)))
            f.write(hbytes)
            base = f.tell()
            for off, n, prod in self._blobs:
                if isinstance(prod, tuple):
                    fn, fld = prod
                    arr = np.ascontiguousarray(fn(fld), dtype=FIELD_DTYPES[fld])
                else:
                    arr = prod
                data = memoryview(arr).cast("B") if arr.nbytes else b""
                if len(data) != n:
                    raise ValueError(f"blob produced {len(data)} bytes, registered {n}")
                f.seek(base + off)
                f.write(data)
            end = base + self._cursor
            f.truncate(max(end, f.tell()))


def hex_nbytes(rows: int, cols: int, k_dim: int, nk: int, code_bits: int = 8) -> dict:
    """Byte size of every blob of a packed tensor with nk kinks."""
    d = {
        "codes": rows * cols // 2 if code_bits == 8 else (7 * (rows * cols // 2) + 7) // 8,
        "scales": rows * cols // 64 * 2,
        "row_ptr": (rows + 1) * 4,
        "kink_cols": nk * 2,
        "kink_deltas": nk * 4,
    }
    if k_dim > 0:
        d.update({"U": rows * k_dim * 2, "S": k_dim * 4, "Vt": k_dim * cols * 2})
    return d


def layer_tensor_names(n_layers: int) -> Iterable[str]:
    for l in range(n_layers):
        for t in LAYER_HEX:
            yield f"blk.{l}.{t}.weight"
