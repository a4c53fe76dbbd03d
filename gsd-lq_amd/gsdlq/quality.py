"""Encoder quality report: reconstruction error and bits per weight of the
packed tensors of a synthetic Mistral-7B layer in each mode, and how close
the encoder's rank-k term comes to the best rank-k fit of its residual.

The reference ships no encoder and no quality figures for its packer; its
README claims ~4.26 bpw (Turbo) and ~3.76 bpw (Precision) for Mistral-7B
(README.md:16-21, 32-33).  Per tensor this reports

  rel_err_codes   ||W - W_codes|| / ||W||    (codebook point x fp16 scale + kinks)
  rel_err         ||W - W_hat|| / ||W||      (plus U diag(S) Vt)
  rel_err_svd     the same with the best rank-k term: the top-k singular
                  triplets of the residual E = W - W_codes (exact, float64)
  lowrank_capture (||E||^2 - ||W - W_hat||^2) / sum of the top-k sigma^2:
                  the share of the best possible rank-k energy reduction the
                  encoder's subspace iteration (plus fp16 rounding of U, Vt)
                  achieves
  bpw             bits per weight of all blobs with u8 codes, and with the
                  7-bit code stream (radius <= 6) of the compact variant

    python -m gsdlq.quality [--mode precision|turbo|both] [--tensors q,k,...] [--json out.json]
"""
from __future__ import annotations

import argparse
import json
import sys
import time

import numpy as np

from . import pack, synth


def _svd_topk(E: np.ndarray, k: int) -> np.ndarray:
    """The k largest singular values of E (float64)."""
    from scipy.sparse.linalg import svds
    s = svds(E, k=k, which="LM", return_singular_vectors=False, random_state=0, tol=1e-10)
    return np.sort(s)[::-1]


def tensor_quality(W: np.ndarray, f: dict) -> dict:
    W = np.asarray(W, dtype=np.float64)
    rows, cols, k = f["rows"], f["cols"], f["k_dim"]
    nW = float(np.linalg.norm(W))
    base = pack.dequantize(f, include_lowrank=False)
    E = W - base
    r = {"rows": rows, "cols": cols, "radius": f["radius"], "k_dim": k, "kinks": f["nk"],
         "rel_err_codes": float(np.linalg.norm(E)) / nW}
    if k > 0:
        full = pack.dequantize(f, include_lowrank=True)
        err = float(np.linalg.norm(W - full))
        s = _svd_topk(E, k)
        e2 = float(np.sum(E * E))
        best = max(e2 - float(np.sum(s * s)), 0.0)
        r.update(rel_err=err / nW, rel_err_svd=np.sqrt(best) / nW,
                 lowrank_capture=(e2 - err * err) / float(np.sum(s * s)) if np.sum(s * s) > 0 else 1.0,
                 sigma=[float(v) for v in s])
    else:
        r["rel_err"] = r["rel_err_codes"]
    nb = pack.packed_nbytes(f)
    r["bpw_u8_codes"] = 8.0 * nb / (rows * cols)
    if f["radius"] <= 6:
        n = f["codes"].size
        r["bpw_7bit_codes"] = 8.0 * (nb - n + (7 * n + 7) // 8) / (rows * cols)
    return r


def layer_report(mode: str, tensors=None, layer: int = 0) -> dict:
    spec = synth.SynthSpec(n_layers=max(layer + 1, 1), mode=mode)
    names = tensors or ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
    out, wsum, bits8, bits7, e2, n2 = {}, 0, 0.0, 0.0, 0.0, 0.0
    for t in names:
        name = f"blk.{layer}.{t}.weight"
        t0 = time.time()
        W = synth.synth_weight(spec, name)
        f = synth.pack_synth(spec, name)
        q = tensor_quality(W, f)
        q["seconds"] = round(time.time() - t0, 1)
        out[t] = q
        n = q["rows"] * q["cols"]
        wsum += n
        bits8 += q["bpw_u8_codes"] * n
        bits7 += q.get("bpw_7bit_codes", q["bpw_u8_codes"]) * n
        e2 += (q["rel_err"] ** 2) * float(np.sum(np.asarray(W, np.float64) ** 2))
        n2 += float(np.sum(np.asarray(W, np.float64) ** 2))
        print(f"[quality] {mode} {t}: rel_err {q['rel_err']:.4f} (codes {q['rel_err_codes']:.4f}"
              + (f", best rank-{q['k_dim']} {q['rel_err_svd']:.4f}, capture {q['lowrank_capture']:.3f}"
                 if q["k_dim"] else "") + f"), bpw {q['bpw_u8_codes']:.3f}"
              + (f" / {q['bpw_7bit_codes']:.3f} (7-bit)" if "bpw_7bit_codes" in q else ""), flush=True)
    return {"mode": mode, "radius": spec.radius, "k_dim": spec.rank, "tensors": out,
            "layer_rel_err": float(np.sqrt(e2 / n2)), "layer_bpw_u8_codes": bits8 / wsum,
            "layer_bpw_7bit_codes": bits7 / wsum}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--mode", default="both", choices=["precision", "turbo", "both"])
    ap.add_argument("--tensors", default=None, help="comma-separated subset of attn_q,...,ffn_down")
    ap.add_argument("--json", default=None)
    a = ap.parse_args(argv)
    modes = ["turbo", "precision"] if a.mode == "both" else [a.mode]
    names = a.tensors.split(",") if a.tensors else None
    rep = {m: layer_report(m, names) for m in modes}
    for m, r in rep.items():
        print(f"[quality] {m}: layer rel_err {r['layer_rel_err']:.4f}, bpw {r['layer_bpw_u8_codes']:.3f} (u8 codes)"
              f" / {r['layer_bpw_7bit_codes']:.3f} (7-bit codes where radius <= 6)", flush=True)
    if a.json:
        with open(a.json, "w") as fh:
            json.dump(rep, fh, indent=1)
    return rep


if __name__ == "__main__":
    sys.exit(0 if main() else 1)
