"""Seeded synthetic GSD-LQ models (random-init, Mistral-7B-shaped by default).

No checkpoint can be fetched offline, so benchmarks and parity runs use
random-init models of the real architecture:
  * linear weights and lm_head: bf16 ~N(0, 0.02) (native generator, see
    csrc/gsdpack.cpp), packed by this project's encoder;
  * token embedding: fp16 ~N(0, 0.02);
  * RMSNorm weights: 1.0;
  * a placeholder SentencePiece-style vocabulary (specials, 256 byte tokens,
    then synthetic pieces) that satisfies the header schema.

Modes: "turbo" = radius 8, u8 codes, no low-rank (~4.26 bpw);
       "precision" = radius 6 (127 points, 7-bit codes on the device) with a
       rank-k correction (default k = 2).

SynthSource exposes the same accessors as gsd2.Gsd2File (config, tensors,
avg_bpw, dense(), hex_field()) and packs each tensor on demand, so a 7B model
can be loaded straight into the engine without writing a 3-4 GB file.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

from . import gsd2, pack

MISTRAL_7B = dict(n_layers=32, hidden=4096, ffn=14336, n_heads=32, n_kv_heads=8, head_dim=128,
                  vocab=32768, rms_eps=1e-5, rope_theta=1e6)

MODES = {"turbo": dict(radius=8, k_dim=0), "precision": dict(radius=6, k_dim=2)}


@dataclass
class SynthSpec:
    n_layers: int = 32
    hidden: int = 4096
    ffn: int = 14336
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 32768
    rms_eps: float = 1e-5
    rope_theta: float = 1e6
    mode: str = "precision"
    k_dim: Optional[int] = None
    kinks_per_row: int = 0
    lr_iters: int = 2
    seed: int = 0
    sigma: float = 0.02
    codebook_radius: Optional[int] = None   # overrides the mode's radius (1..8)

    @property
    def radius(self) -> int:
        return MODES[self.mode]["radius"] if self.codebook_radius is None else int(self.codebook_radius)

    @property
    def rank(self) -> int:
        return MODES[self.mode]["k_dim"] if self.k_dim is None else int(self.k_dim)


def tensor_shapes(spec: SynthSpec) -> Dict[str, tuple]:
    h, f, kv = spec.hidden, spec.ffn, spec.n_kv_heads * spec.head_dim
    qd = spec.n_heads * spec.head_dim
    per = {"attn_q": (qd, h), "attn_k": (kv, h), "attn_v": (kv, h), "attn_output": (h, qd),
           "ffn_gate": (f, h), "ffn_up": (f, h), "ffn_down": (h, f)}
    out = {}
    for l in range(spec.n_layers):
        for t, shp in per.items():
            out[f"blk.{l}.{t}.weight"] = shp
    out["output.weight"] = (spec.vocab, h)
    return out


def tensor_stream(name: str) -> int:
    """Stable RNG stream id of each synthetic tensor."""
    if name == "token_embd.weight":
        return 1
    if name == "output.weight":
        return 99
    parts = name.split(".")
    l = int(parts[1])
    return 100 + 16 * l + gsd2.LAYER_HEX.index(parts[2])


def placeholder_vocab(n: int):
    toks, scores, types = ["<unk>", "<s>", "</s>"], [0.0, 0.0, 0.0], [2, 3, 3]
    for b in range(256):
        toks.append(f"<0x{b:02X}>")
        scores.append(0.0)
        types.append(6)
    i = 0
    while len(toks) < n:
        toks.append(f"▁w{i}")
        scores.append(-float(i))
        types.append(1)
        i += 1
    return toks[:n], scores[:n], types[:n]


def make_config(spec: SynthSpec) -> dict:
    toks, scores, types = placeholder_vocab(spec.vocab)
    return {"n_layers": spec.n_layers, "hidden_size": spec.hidden, "n_heads": spec.n_heads,
            "n_kv_heads": spec.n_kv_heads, "head_dim": spec.head_dim, "ffn_size": spec.ffn,
            "rms_eps": spec.rms_eps, "rope_theta": spec.rope_theta, "vocab_size": spec.vocab,
            "tokens": toks, "scores": scores, "token_types": types, "bos_id": 1, "eos_id": 2}


def synth_weight(spec: SynthSpec, name: str) -> np.ndarray:
    rows, cols = tensor_shapes(spec)[name]
    return pack.synth_bf16(spec.seed, tensor_stream(name), rows * cols, spec.sigma).reshape(rows, cols)


def pack_synth(spec: SynthSpec, name: str) -> dict:
    W = synth_weight(spec, name)
    return pack.pack_tensor(W, spec.radius, spec.rank, spec.kinks_per_row, spec.lr_iters)


class SynthSource:
    """Lazily packed synthetic model with the Gsd2File accessor surface."""

    def __init__(self, spec: SynthSpec):
        self.spec = spec
        self.config = make_config(spec)
        self._cache_name = None
        self._cache = None
        shapes = tensor_shapes(spec)
        self.tensors = {"token_embd.weight": {"data": {"shape": [spec.vocab, spec.hidden]}}}
        for l in range(spec.n_layers):
            for nm in ("attn_norm", "ffn_norm"):
                self.tensors[f"blk.{l}.{nm}.weight"] = {"data": {"shape": [spec.hidden]}}
        self.tensors["output_norm.weight"] = {"data": {"shape": [spec.hidden]}}
        for name, (r, c) in shapes.items():
            self.tensors[name] = {"radius": spec.radius, "rows": r, "cols": c, "k_dim": spec.rank}
        self.file_size = 0
        self.avg_bpw = None   # known once every tensor is packed

    @property
    def header(self):
        return {"config": self.config, "avg_bpw": self.avg_bpw, "tensors": self.tensors}

    def dense(self, name: str, dtype):
        if name == "token_embd.weight":
            arr = pack.synth_f16(self.spec.seed, 1, self.spec.vocab * self.spec.hidden, self.spec.sigma)
            return arr.view(np.float16).reshape(self.spec.vocab, self.spec.hidden).view(dtype)
        return np.ones(self.spec.hidden, dtype=np.float32).view(dtype)

    def packed(self, name: str) -> dict:
        if self._cache_name != name:
            self._cache = pack_synth(self.spec, name)
            self._cache_name = name
        return self._cache

    def hex_field(self, name: str, field: str) -> np.ndarray:
        return self.packed(name)[field]

    def close(self):
        self._cache = None


def write_gsd2(spec: SynthSpec, path: str, code_bits: int = 8) -> dict:
    """Pack every tensor and write a .gsd2 file; returns {name: nk}.
    code_bits = 7 writes the codes of radius <= 6 tensors as 7-bit streams."""
    shapes = tensor_shapes(spec)
    config = make_config(spec)
    packed = {}
    total_bits = 0
    total_w = 0
    bits_of = lambda f: code_bits if f["radius"] <= 6 else 8
    for name in shapes:
        f = pack_synth(spec, name)
        packed[name] = f
        total_bits += 8 * pack.packed_nbytes(f)
        if bits_of(f) == 7:   # the code stream is 7/8 of the u8 codes
            total_bits -= 8 * (f["codes"].size - (7 * f["codes"].size + 7) // 8)
        total_w += f["rows"] * f["cols"]
    w = gsd2.Gsd2Writer(config, total_bits / total_w)
    emb = pack.synth_f16(spec.seed, 1, spec.vocab * spec.hidden, spec.sigma).view(np.float16)
    w.add_dense("token_embd.weight", emb.reshape(spec.vocab, spec.hidden))
    ones = np.ones(spec.hidden, dtype=np.float32)
    for l in range(spec.n_layers):
        w.add_dense(f"blk.{l}.attn_norm.weight", ones)
        w.add_dense(f"blk.{l}.ffn_norm.weight", ones)
        for t in gsd2.LAYER_HEX:
            name = f"blk.{l}.{t}.weight"
            f = packed[name]
            w.add_hex(name, f["radius"], f["rows"], f["cols"], f["k_dim"], fields=f, code_bits=bits_of(f))
    w.add_dense("output_norm.weight", ones)
    f = packed["output.weight"]
    w.add_hex("output.weight", f["radius"], f["rows"], f["cols"], f["k_dim"], fields=f, code_bits=bits_of(f))
    w.write(path)
    return {n: f["nk"] for n, f in packed.items()}
