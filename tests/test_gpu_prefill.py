"""Batched projection for prefill (gsdh_model_matmul) on the GPU against the
oracle's fused matvec (gsd_cpu_hex2d_matvec restated) of each token's
bf16-rounded row: 1e-3 relative L2 per token.  Covers the 7B Turbo layer
shapes at M = 16 / 128 / 512, padded token counts, columns that are not a
multiple of 128, and Precision tensors with kinks and rank-2 terms."""
import ctypes
import os
import sys

import numpy as np
import pytest

import oracle as O
from conftest import rel_l2
from gpu_util import D, E, H, banner

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SLOTS = {"attn_q": 0, "attn_k": 1, "attn_v": 2, "attn_output": 3, "ffn_gate": 4, "ffn_up": 5, "ffn_down": 6}


def bf16(x):
    """Round-to-nearest-even to bf16: (bits, float32 values)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r, (r.astype(np.uint32) << 16).view(np.float32)


def run_matmul(model, layer, slot, xb, M, rows):
    lib = model.cl.lib
    dx = D(xb)
    dy = E(M * rows * 4)
    lib.gsdh_model_matmul(model._m, layer, slot, dx.ptr, M, dy.ptr)
    lib.gsdh_stream_sync(lib.gsdh_model_stream(model._m))
    return H(dy, np.float32, M * rows).reshape(M, rows)


def check(model, t, layer, slot, M, seed, tokens=None):
    rows, cols = t["rows"], t["cols"]
    rng = np.random.default_rng(seed)
    xb, xf = bf16(rng.standard_normal((M, cols)).astype(np.float32))
    Y = run_matmul(model, layer, slot, xb, M, rows)
    assert np.isfinite(Y).all()
    worst = 0.0
    for m in (range(M) if tokens is None else tokens):
        y = O.hex2d_matvec(xf[m], t)
        e = rel_l2(Y[m], y)
        worst = max(worst, e)
        assert e < 1e-3, (m, e)
    return worst


@pytest.fixture(scope="module")
def turbo_7b():
    sys.path.insert(0, ROOT)
    import bench
    bank = bench.LayerBank("turbo", 1)
    model = bench.build_model(bank, 1)
    yield bank, model
    model.close()


@pytest.mark.parametrize("name,M", [("attn_q", 16), ("ffn_gate", 128), ("ffn_down", 16), ("attn_k", 512),
                                    ("attn_output", 37)])
def test_matmul_7b_turbo(turbo_7b, name, M):
    bank, model = turbo_7b
    banner(f"prefill matmul 7B turbo {name} M={M}")
    t = bank.packed[(0, name)]
    toks = sorted({0, 1, M // 2, M - 1})
    worst = check(model, t, 0, SLOTS[name], M, seed=7 + M, tokens=toks)
    print(f"[gpu-test] worst rel L2 {worst:.2e}", flush=True)


def _small_model(spec):
    from gsdlq import synth
    import run_gpu_native_chat as chat
    src = synth.SynthSource(spec)
    return src, chat.GPUMistralV2Model(src, max_seq_len=64, verbose=False)


@pytest.mark.parametrize("mode,kpr,shape,M", [
    ("precision", 2, dict(), 33),
    ("turbo", 1, dict(hidden=320, ffn=448, n_heads=5, n_kv_heads=5, head_dim=64), 5),
    ("precision", 0, dict(hidden=384, ffn=704, n_heads=6, n_kv_heads=3, head_dim=64), 200),
    # generic-codebook kernels: radius 5 (7-bit tiles), radius 7 (u8 tiles)
    ("turbo", 1, dict(codebook_radius=5), 20),
    ("precision", 0, dict(codebook_radius=7), 17),
])
def test_matmul_small_vs_oracle(mode, kpr, shape, M):
    from gsdlq import synth
    base = dict(n_layers=1, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
                mode=mode, kinks_per_row=kpr)
    base.update(shape)
    spec = synth.SynthSpec(**base)
    banner(f"prefill matmul small {mode} kinks {kpr} {shape} M={M}")
    src, model = _small_model(spec)
    try:
        for name in ("attn_q", "attn_v", "ffn_gate", "ffn_down"):
            key = f"blk.0.{name}.weight"
            t = dict(src.tensors[key])
            for f in ("codes", "scales", "row_ptr", "kink_cols", "kink_deltas") + (("U", "S", "Vt") if t["k_dim"] else ()):
                t[f] = np.ascontiguousarray(src.hex_field(key, f))
            check(model, t, 0, SLOTS[name], M, seed=M + SLOTS[name])
    finally:
        model.close()


def test_matmul_rejects_bad_arguments():
    from gsdlq import synth, hip
    spec = synth.SynthSpec(n_layers=1, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
                           mode="turbo")
    banner("prefill matmul argument checks")
    _, model = _small_model(spec)
    try:
        buf = E(1024)
        with pytest.raises(hip.HipError):
            model.cl.lib.gsdh_model_matmul(model._m, 0, 9, buf.ptr, 4, buf.ptr)
        with pytest.raises(hip.HipError):
            model.cl.lib.gsdh_model_matmul(model._m, 0, 0, buf.ptr, 0, buf.ptr)
        with pytest.raises(hip.HipError):
            model.cl.lib.gsdh_model_matmul(model._m, 5, 0, buf.ptr, 4, buf.ptr)
    finally:
        model.close()
