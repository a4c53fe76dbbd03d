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
    model = bench.build_model(bank, 1, max_seq=640)
    yield bank, model
    model.close()


def plan(lib, M, rows, cols):
    tg, rbw, ns = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    lib.gsdh_matmul_plan(M, rows, cols, ctypes.byref(tg), ctypes.byref(rbw), ctypes.byref(ns))
    return tg.value, rbw.value, ns.value


def group_tokens(M):
    """One token in every 16-token group (a different lane of each), and the
    last token: every token group of a tile and every A-fragment row."""
    return sorted({16 * g + (g % 16) for g in range((M + 15) // 16) if 16 * g + (g % 16) < M} | {M - 1})


C5_TENSORS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


# Every (tensor, M) pair of the C5 benchmark (the 7 Turbo tensors of a
# Mistral-7B layer at M = 16 / 128 / 512), whose plans on a 256-CU MI355X
# are: one token group with 8, 5 or 16 column splits (M = 16), one group
# unsplit (q / o / down at 128, k / v at 512), four groups (gate / up at
# 128, q / o / down at 512), eight groups with two row blocks per wave
# (gate / up at 512); plus a padded token count.  Every output row of each
# checked token is compared, so every row block of every wave is.
@pytest.mark.parametrize("M", [16, 128, 512])
@pytest.mark.parametrize("name", C5_TENSORS)
def test_matmul_7b_turbo(turbo_7b, name, M):
    bank, model = turbo_7b
    t = bank.packed[(0, name)]
    pl = plan(model.cl.lib, M, t["rows"], t["cols"])
    banner(f"prefill matmul 7B turbo {name} M={M} plan (tg, rbw, nsplit) = {pl}")
    worst = check(model, t, 0, SLOTS[name], M, seed=7 + M + SLOTS[name], tokens=group_tokens(M))
    print(f"[gpu-test] worst rel L2 {worst:.2e}", flush=True)


def test_matmul_7b_turbo_padded(turbo_7b):
    bank, model = turbo_7b
    banner("prefill matmul 7B turbo attn_output M=37")
    check(model, bank.packed[(0, "attn_output")], 0, SLOTS["attn_output"], 37, seed=44, tokens=group_tokens(37))


def test_matmul_7b_turbo_plans(turbo_7b):
    """The C5 pairs above reach every tile shape of the batched kernel."""
    bank, model = turbo_7b
    seen = {plan(model.cl.lib, M, *layer_shape(n)) for n in C5_TENSORS for M in (16, 128, 512)}
    assert {(8, 2, 1), (4, 1, 1), (1, 1, 1)} <= seen, seen
    assert any(s > 1 for _, _, s in seen), seen


@pytest.mark.parametrize("names,M", [(("attn_q", "attn_k", "attn_v"), 128), (("ffn_gate", "ffn_up"), 512),
                                     (("attn_q", "attn_k", "attn_v"), 16)])
def test_matmul_shared_input_equals_separate_calls(turbo_7b, names, M):
    """gsdh_model_matmul_shared (one operand prep for tensors that read the
    same X) gives the separate calls' outputs bit for bit, and the oracle's."""
    bank, model = turbo_7b
    lib = model.cl.lib
    banner(f"shared-input matmul {names} M={M}")
    rng = np.random.default_rng(60 + M)
    cols = bank.packed[(0, names[0])]["cols"]
    xb, xf = bf16(rng.standard_normal((M, cols)).astype(np.float32))
    dx = D(xb)
    rows = [bank.packed[(0, n)]["rows"] for n in names]
    ys = [E(M * r * 4) for r in rows]
    sl = (ctypes.c_int * len(names))(*[SLOTS[n] for n in names])
    yp = (ctypes.c_void_p * len(names))(*[y.ptr.value for y in ys])
    lib.gsdh_model_matmul_shared(model._m, 0, sl, len(names), dx.ptr, M, yp)
    lib.gsdh_stream_sync(lib.gsdh_model_stream(model._m))
    got = [H(y, np.float32, M * r).reshape(M, r) for y, r in zip(ys, rows)]
    for n, r, g in zip(names, rows, got):
        want = run_matmul(model, 0, SLOTS[n], xb, M, r)
        assert np.array_equal(g, want), n
        for m in (0, M - 1):
            assert rel_l2(g[m], O.hex2d_matvec(xf[m], bank.packed[(0, n)])) < 1e-3, (n, m)


def test_matmul_shared_rejects_mixed_inputs(turbo_7b):
    from gsdlq.hip import HipError
    bank, model = turbo_7b
    buf = E(1 << 20)
    sl = (ctypes.c_int * 2)(SLOTS["attn_q"], SLOTS["ffn_down"])
    yp = (ctypes.c_void_p * 2)(buf.ptr.value, buf.ptr.value)
    with pytest.raises(HipError, match="share an input"):
        model.cl.lib.gsdh_model_matmul_shared(model._m, 0, sl, 2, buf.ptr, 4, yp)


def layer_shape(name):
    H, F, KV = 4096, 14336, 1024
    return {"attn_q": (H, H), "attn_k": (KV, H), "attn_v": (KV, H), "attn_output": (H, H),
            "ffn_gate": (F, H), "ffn_up": (F, H), "ffn_down": (H, F)}[name]


def test_prefill_7b_turbo_chunks(turbo_7b):
    """The batched prefill forward of the 7B Turbo layer (32 / 8 heads of
    128, ffn 14336, vocab 32768): 514 tokens (a 512-token chunk: eight-group
    tiles with two row blocks per wave; then a 2-token chunk on column-split
    tiles), then 64 more after that prefix (two-group tiles), against the
    oracle's token-by-token forward."""
    import bench
    bank, model = turbo_7b
    banner("batched prefill 7B turbo: 514 tokens, then 64 more")
    lib = model.cl.lib
    for M in (512, 2, 64):
        print(f"[gpu-test] chunk {M}: gate/up plan {plan(lib, M, 14336, 4096)}, q plan {plan(lib, M, 4096, 4096)}, "
              f"down plan {plan(lib, M, 4096, 14336)}", flush=True)
    ref = O.OracleModel(bench.BankSource(bank, 1), kind="port", max_seq_len=640, rope_interleaved=1)
    toks = np.random.default_rng(130).integers(0, model.vocab_size, 578).tolist()
    got = model.prefill(toks[:514], 0)
    want = None
    for pos in range(514):
        want = ref.forward_token(toks[pos], pos, return_logits=pos == 513)
    e = rel_l2(got, want)
    print(f"[prefill-parity] 7B turbo 514 tokens: last-position logits rel L2 {e:.2e}", flush=True)
    assert e < 1e-3
    _kv_close(model, ref, [0], [0, 256, 511, 512, 513])
    got = model.prefill(toks[514:], 514)
    for pos in range(514, 578):
        want = ref.forward_token(toks[pos], pos, return_logits=pos == 577)
    e = rel_l2(got, want)
    print(f"[prefill-parity] 7B turbo +64 tokens: last-position logits rel L2 {e:.2e}", flush=True)
    assert e < 1e-3
    _kv_close(model, ref, [0], [514, 545, 577])


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
    ("turbo", 0, 1, 1100, dict()),                       # three chunks (512, 512, 76)
    ("precision", 1, 0, 33, dict(n_heads=8, n_kv_heads=8)),          # half-split RoPE, group size 1
    ("turbo", 1, 1, 130, dict(n_layers=1, hidden=512, ffn=1344, n_heads=8, n_kv_heads=2, head_dim=128,
                              vocab=1000)),              # ragged ffn, group size 4, hd 128
    ("precision", 0, 1, 17, dict(k_dim=3)),              # rank 3
    ("precision", 2, 1, 20, dict(codebook_radius=7)),    # u8 tiles, generic codebook
]


@pytest.mark.parametrize("mode,kpr,il,n,shape", PREFILL_CASES)
def test_prefill_vs_oracle(mode, kpr, il, n, shape):
    banner(f"batched prefill {mode} kinks {kpr} interleaved {il} n {n} {shape}")
    gpu, ref = _pair(_spec(mode=mode, kinks_per_row=kpr, **shape), max_seq=max(512, n + 8), il=il)
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
