"""Batched prefill on the GPU against the oracle.

1. The batched projection (gsdh_model_matmul) against the oracle's fused
   matvec (gsd_cpu_hex2d_matvec restated) of each token's bf16-rounded row:
   1e-3 relative L2 per token.  Covers the 7B Turbo layer shapes at
   M = 16 / 128 / 512, padded token counts, columns that are not a multiple
   of 128, and Precision tensors with kinks and rank-2 terms.
2. The batched prefill forward (gsdh_model_prefill): the last prompt
   position's logits within 1e-3 of the oracle's token-by-token forward, the
   K/V cache rows it writes, decoding on from it, a reused prefix, and
   generate_greedy's tokens with either prefill mode."""
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


# ---------------------------------------------------------------------------
# Batched prefill as a model forward (gsdh_model_prefill): the prompt's
# tokens through every layer at once against the oracle's token-by-token
# forward (gsd_lq_cpu_runtime.py:302-420, the reference's prefill loop
# run_gpu_native_chat.py:1128-1130).
# ---------------------------------------------------------------------------
def _spec(**kw):
    from gsdlq import synth
    base = dict(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
                mode="precision", kinks_per_row=2)
    base.update(kw)
    return synth.SynthSpec(**base)


def _pair(spec, max_seq=512, il=1):
    from gsdlq import synth
    import run_gpu_native_chat as chat
    src = synth.SynthSource(spec)
    gpu = chat.GPUMistralV2Model(src, rope_interleaved=il, max_seq_len=max_seq, verbose=False)
    ref = O.OracleModel(src, kind="port", max_seq_len=max_seq, rope_interleaved=il)
    return gpu, ref


def _kv_close(gpu, ref, layers, positions):
    from gsdlq import hip
    kvd = gpu.n_kv_heads * gpu.head_dim
    for l in layers:
        for p in positions:
            kr, vr = np.empty(kvd, np.uint16), np.empty(kvd, np.uint16)
            gpu.cl.lib.gsdh_model_read_kv(gpu._m, l, p, hip.ptr(kr), hip.ptr(vr))
            assert rel_l2(O.f16_to_f32(kr), O.f16_to_f32(ref.k_cache[l, p].reshape(-1))) < 1e-3, (l, p)
            assert rel_l2(O.f16_to_f32(vr), O.f16_to_f32(ref.v_cache[l, p].reshape(-1))) < 1e-3, (l, p)


PREFILL_CASES = [
    ("precision", 2, 1, 40, dict()),
    ("turbo", 0, 1, 300, dict()),                        # three chunks (128, 128, 44)
    ("precision", 1, 0, 33, dict(n_heads=8, n_kv_heads=8)),          # half-split RoPE, group size 1
    ("turbo", 1, 1, 130, dict(n_layers=1, hidden=512, ffn=1344, n_heads=8, n_kv_heads=2, head_dim=128,
                              vocab=1000)),              # ragged ffn, group size 4, hd 128
    ("precision", 0, 1, 17, dict(k_dim=3)),              # rank 3
    ("precision", 2, 1, 20, dict(codebook_radius=7)),    # u8 tiles, generic codebook
]


@pytest.mark.parametrize("mode,kpr,il,n,shape", PREFILL_CASES)
def test_prefill_vs_oracle(mode, kpr, il, n, shape):
    banner(f"batched prefill {mode} kinks {kpr} interleaved {il} n {n} {shape}")
    gpu, ref = _pair(_spec(mode=mode, kinks_per_row=kpr, **shape), il=il)
    toks = np.random.default_rng(n).integers(0, gpu.vocab_size, n).tolist()
    got = gpu.prefill(toks, 0)
    want = None
    for pos, t in enumerate(toks):
        want = ref.forward_token(t, pos, return_logits=pos == n - 1)
    e = rel_l2(got, want)
    print(f"[prefill-parity] {mode} n {n}: last-position logits rel L2 {e:.2e}", flush=True)
    assert e < 1e-3
    _kv_close(gpu, ref, range(gpu.n_layers), sorted({0, n // 2, n - 1}))
    # decoding continues from the prefilled cache
    for pos in range(n, n + 3):
        nxt = int(np.argmax(want))
        a, want = gpu.forward_token(nxt, pos), ref.forward_token(nxt, pos)
        assert rel_l2(a, want) < 1e-3, pos
    gpu.close()


def test_prefill_prefix_reuse():
    """A second prefill at start_pos = the cached prefix length attends to the
    prefix (run_gpu_native_chat.py:1112-1115 reuses it across turns)."""
    banner("batched prefill with a cached prefix")
    gpu, ref = _pair(_spec(mode="precision", kinks_per_row=1))
    toks = np.random.default_rng(77).integers(0, gpu.vocab_size, 60).tolist()
    gpu.prefill(toks[:25], 0, return_logits=False)
    got = gpu.prefill(toks[25:], 25)
    want = None
    for pos, t in enumerate(toks):
        want = ref.forward_token(t, pos, return_logits=pos == len(toks) - 1)
    assert rel_l2(got, want) < 1e-3
    # rewinding: a shorter prompt over the same cache
    got = gpu.prefill(toks[10:20], 10)
    for pos in range(10, 20):
        want = ref.forward_token(toks[pos], pos, return_logits=pos == 19)
    assert rel_l2(got, want) < 1e-3
    gpu.close()


@pytest.mark.parametrize("batched", [True, False])
def test_generate_greedy_prefill_modes(batched):
    """generate_greedy with the batched prefill (default) and with one
    decode step per prompt token gives the oracle's tokens."""
    banner(f"generate_greedy, batched prefill {batched}")
    gpu, ref = _pair(_spec(mode="turbo", kinks_per_row=1))
    gpu.set_prefill(batched)
    prompt = np.random.default_rng(9).integers(0, gpu.vocab_size, 150).tolist()
    toks, margins = gpu.generate_greedy(prompt, 16)
    want, wm = ref.generate_greedy(prompt, 16)
    assert toks == want
    assert np.allclose(margins, wm, rtol=1e-2, atol=1e-4)
    gpu.close()


def test_prefill_rejects_bad_arguments():
    from gsdlq.hip import HipError
    gpu, _ = _pair(_spec(), max_seq=64)
    with pytest.raises(HipError, match="max_seq_len"):
        gpu.prefill(list(range(10)), 60)
    with pytest.raises(HipError, match="vocab"):
        gpu.prefill([1, 2, 512], 0)
    with pytest.raises(ValueError):
        gpu.prefill([], 0)
    gpu.close()
