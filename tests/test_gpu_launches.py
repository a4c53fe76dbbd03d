"""Full-shape parity of every fused matvec launch the decode runs (and the
benchmark times), one launch at a time, against the oracle on the same inputs.

The model is one layer of the Mistral-7B shape (hidden 4096, ffn 14336,
32 query / 8 KV heads of 128, vocab 32768), packed like the benchmark's layers
in Turbo mode (radius 8, u8 codes) and Precision mode (radius 6, 7-bit device
codes, rank 2).  Each launch reads the activation vectors a test writes and
its result is read back (gsdh_model_vector / gsdh_model_read_kv):

  qkv      q' = RoPE(Wq xn), K' = fp16(RoPE(Wk xn)), V = fp16(Wv xn),
           xn = rmsnorm(x) * attn_norm        (gsd_lq_cpu_runtime.py:316-340)
  o        x + Wo attn                         (gsd_lq_cpu_runtime.py:376-378)
  gate/up  silu(Wg xn) * (Wu xn), xn = rmsnorm(x) * ffn_norm   (:384-396)
  down     x + Wd h                            (:398-404)
  head     Wlm (rmsnorm(x) * out_norm)         (:414-419)

Bar: 1e-3 relative L2 (the tolerance of the matvec's fp32 accumulation in
another order).  The measured error of every launch is printed; the matrix-core
kernel represents x as fp16 high + low parts (about 2^-22 relative), so it is
also held to 1e-4, a regression guard two orders under the bar."""
import ctypes

import numpy as np
import pytest

import oracle as O
from conftest import rel_l2
from gpu_util import banner

pytestmark = pytest.mark.gpu

TOL = 1e-3
GUARD = 1e-4


@pytest.fixture(scope="module", params=["turbo", "precision"])
def layer7b(request):
    from gsdlq import synth
    import run_gpu_native_chat as chat
    mode = request.param
    banner(f"packing one 7B-shaped layer + 32768-row head ({mode})")
    src = synth.SynthSource(synth.SynthSpec(n_layers=1, mode=mode))
    gpu = chat.GPUMistralV2Model(src, max_seq_len=64, verbose=False)
    ref = O.OracleModel(src, kind="port", max_seq_len=64)
    yield mode, gpu, ref
    gpu.close()


def _put(gpu, name, a):
    from gsdlq import hip
    a = np.ascontiguousarray(a, np.float32)
    gpu.cl.lib.gsdh_model_vector(gpu._m, hip.VECTORS[name], 1, hip.ptr(a), a.nbytes)


def _get(gpu, name, n):
    from gsdlq import hip
    a = np.empty(n, np.float32)
    gpu.cl.lib.gsdh_model_vector(gpu._m, hip.VECTORS[name], 0, hip.ptr(a), a.nbytes)
    return a


def _check(label, got, want, tol=TOL):
    e = rel_l2(got, want)
    print(f"[launch-parity] {label}: rel L2 {e:.3e}", flush=True)
    assert e < tol, (label, e)
    assert e < GUARD, (label, e)
    return e


def _rmsnorm(ref, x, w):
    out = np.empty_like(x)
    ref.lib.gsd_cpu_rmsnorm(O.P(x), O.P(w), O.P(out), x.size, float(ref.rms_eps))
    return out


def test_qkv_launch_full_shape(layer7b):
    mode, gpu, ref = layer7b
    rng = np.random.default_rng(101)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    pos = 37
    _put(gpu, "x", x)
    gpu.cl.lib.gsdh_model_set_step(gpu._m, 0, pos)
    gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 1)
    q = _get(gpu, "q", gpu.n_heads * gpu.head_dim)
    kvd = gpu.n_kv_heads * gpu.head_dim
    kr, vr = np.empty(kvd, np.uint16), np.empty(kvd, np.uint16)
    from gsdlq import hip
    gpu.cl.lib.gsdh_model_read_kv(gpu._m, 0, pos, hip.ptr(kr), hip.ptr(vr))

    ly = ref.layers[0]
    xb = _rmsnorm(ref, x, ly["attn_norm"])
    ref.matvec(xb, ly["q"], ref.q)
    ref.matvec(xb, ly["k"], ref.k)
    ref.matvec(xb, ly["v"], ref.v)
    ref.lib.gsd_cpu_rope_and_store_kv(O.P(ref.q), O.P(ref.k), O.P(ref.v), O.P(ref.k_cache), O.P(ref.v_cache),
                                      0, pos, ref.n_heads, ref.n_kv_heads, ref.head_dim, ref.max_seq_len,
                                      float(ref.rope_theta), 1)
    _check(f"{mode} q (4096x4096, RoPE pos {pos})", q, ref.q)
    _check(f"{mode} K cache row (1024x4096, RoPE, fp16)", O.f16_to_f32(kr),
           O.f16_to_f32(ref.k_cache[0, pos].reshape(-1)))
    _check(f"{mode} V cache row (1024x4096, fp16)", O.f16_to_f32(vr), O.f16_to_f32(ref.v_cache[0, pos].reshape(-1)))


def test_o_launch_full_shape(layer7b):
    mode, gpu, ref = layer7b
    rng = np.random.default_rng(102)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    att = rng.standard_normal(gpu.n_heads * gpu.head_dim).astype(np.float32)
    _put(gpu, "x", x)
    _put(gpu, "attn", att)
    gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 2)
    got = _get(gpu, "x", gpu.hidden)
    y = np.empty(gpu.hidden, np.float32)
    ref.matvec(att, ref.layers[0]["o"], y)
    _check(f"{mode} o (4096x4096) without residual", got - x, y)
    _check(f"{mode} o + residual", got, x + y)


def test_gate_up_launch_full_shape(layer7b):
    """The launch the benchmark's roofline figure times: 2 x 14336 x 4096."""
    mode, gpu, ref = layer7b
    rng = np.random.default_rng(103)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    _put(gpu, "x", x)
    gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 4)
    got = _get(gpu, "h", gpu.ffn_size)
    ly = ref.layers[0]
    xb = _rmsnorm(ref, x, ly["ffn_norm"])
    g = np.empty(gpu.ffn_size, np.float32)
    u = np.empty(gpu.ffn_size, np.float32)
    ref.matvec(xb, ly["gate"], g)
    ref.matvec(xb, ly["up"], u)
    ref.lib.gsd_cpu_swiglu(O.P(g), O.P(u), O.P(g), gpu.ffn_size)
    _check(f"{mode} gate/up (2x14336x4096) + SwiGLU", got, g)


@pytest.mark.parametrize("mode", ["turbo", "precision"])
@pytest.mark.parametrize("halves", ["1", "0"])
def test_gate_up_half_units_ragged(mode, halves, monkeypatch):
    """gate/up 2 x 5056 x 2048: 316 units on a 256-CU device's 256 blocks;
    in Turbo mode the last 60 as half units on 120 blocks (rows 8h .. 8h + 7
    of gate and up per block, each wave one of its two chunks), in Precision
    mode (rank-2 term: no half units) 3 or 4 units per block; and the same
    launch with the half units off (GSD_GATEUP_HALVES=0)."""
    from gsdlq import synth
    import run_gpu_native_chat as chat
    monkeypatch.setenv("GSD_GATEUP_HALVES", halves)
    banner(f"gate/up 2x5056x2048 {mode}, half units {halves}")
    spec = synth.SynthSpec(n_layers=1, hidden=2048, ffn=5056, n_heads=16, n_kv_heads=4, head_dim=128, vocab=512,
                           mode=mode, kinks_per_row=2)
    src = synth.SynthSource(spec)
    gpu = chat.GPUMistralV2Model(src, max_seq_len=16, verbose=False)
    ref = O.OracleModel(src, kind="port", max_seq_len=16)
    try:
        x = np.random.default_rng(107).standard_normal(gpu.hidden).astype(np.float32)
        _put(gpu, "x", x)
        gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 4)
        got = _get(gpu, "h", gpu.ffn_size)
        ly = ref.layers[0]
        xb = _rmsnorm(ref, x, ly["ffn_norm"])
        g = np.empty(gpu.ffn_size, np.float32)
        u = np.empty(gpu.ffn_size, np.float32)
        ref.matvec(xb, ly["gate"], g)
        ref.matvec(xb, ly["up"], u)
        ref.lib.gsd_cpu_swiglu(O.P(g), O.P(u), O.P(g), gpu.ffn_size)
        _check(f"{mode} gate/up 2x5056x2048 halves {halves}", got, g)
        assert rel_l2(got[4096:], g[4096:]) < GUARD   # the rows of the last round
    finally:
        gpu.close()


def test_down_launch_full_shape(layer7b):
    mode, gpu, ref = layer7b
    rng = np.random.default_rng(104)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    h = rng.standard_normal(gpu.ffn_size).astype(np.float32)
    _put(gpu, "x", x)
    _put(gpu, "h", h)
    gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 8)
    got = _get(gpu, "x", gpu.hidden)
    y = np.empty(gpu.hidden, np.float32)
    ref.matvec(h, ref.layers[0]["down"], y)
    _check(f"{mode} down (4096x14336) without residual", got - x, y)
    _check(f"{mode} down + residual", got, x + y)


def _ffn_ref(ref, x, layer=0):
    """x + W_down (silu(W_gate x') * (W_up x')), x' = rmsnorm(x) * ffn_norm,
    through the oracle's engine functions (gsd_lq_cpu_runtime.py:380-404);
    returns (h, y, x + y)."""
    ly = ref.layers[layer]
    xb = _rmsnorm(ref, x, ly["ffn_norm"])
    n = ref.ffn_size
    g = np.empty(n, np.float32)
    u = np.empty(n, np.float32)
    ref.matvec(xb, ly["gate"], g)
    ref.matvec(xb, ly["up"], u)
    ref.lib.gsd_cpu_swiglu(O.P(g), O.P(u), O.P(g), n)
    y = np.empty(x.size, np.float32)
    ref.matvec(g, ly["down"], y)
    return g, y, x + y


def test_ffn_launch_full_shape(layer7b):
    """The fused FFN launch (gate/up + SwiGLU + split down + residual in one
    launch, the decode's and the benchmark's): h, the down product and the
    new x against the oracle at the 7B shape."""
    mode, gpu, ref = layer7b
    assert gpu.cl.lib.gsdh_model_fused_ffn(gpu._m, 0) == 2
    rng = np.random.default_rng(108)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    _put(gpu, "x", x)
    gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 12)
    got = _get(gpu, "x", gpu.hidden)
    h = _get(gpu, "h", gpu.ffn_size)
    hr, y, want = _ffn_ref(ref, x)
    _check(f"{mode} FFN launch: h (2x14336x4096 + SwiGLU)", h, hr)
    _check(f"{mode} FFN launch: down (4096x14336) without residual", got - x, y)
    _check(f"{mode} FFN launch: x + down", got, want)


def test_o_ffn_launch_full_shape(layer7b):
    """o, gate/up and down in one launch (the decode's): x + W_o attn formed
    16 rows per block and handed over as tagged words, then the FFN on it;
    against the oracle's o matvec + residual, then its FFN, at the 7B
    shape."""
    mode, gpu, ref = layer7b
    rng = np.random.default_rng(111)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    att = rng.standard_normal(gpu.n_heads * gpu.head_dim).astype(np.float32)
    _put(gpu, "x", x)
    _put(gpu, "attn", att)
    gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 14)
    got = _get(gpu, "x", gpu.hidden)
    yo = np.empty(gpu.hidden, np.float32)
    ref.matvec(att, ref.layers[0]["o"], yo)
    x1 = x + yo
    hr, y, want = _ffn_ref(ref, x1)
    _check(f"{mode} o + FFN launch: h", _get(gpu, "h", gpu.ffn_size), hr)
    _check(f"{mode} o + FFN launch: x + o + down", got, want)
    _check(f"{mode} o + FFN launch: down (4096x14336) without residual", got - x1, y)


def test_ffn_launch_repeat_bit_identical(layer7b):
    """The fused FFN's cross-block sums run in a fixed block order: runs on
    the same x (and attn) give the same bits (each launch with a new tag),
    with and without the o projection in the launch."""
    mode, gpu, _ = layer7b
    rng = np.random.default_rng(109)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    att = rng.standard_normal(gpu.n_heads * gpu.head_dim).astype(np.float32)
    for mask in (12, 14):
        outs = []
        for _ in range(3):
            _put(gpu, "x", x)
            _put(gpu, "attn", att)
            gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, mask)
            outs.append(_get(gpu, "x", gpu.hidden))
        assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2]), mask


@pytest.mark.parametrize("mode", ["turbo", "precision"])
def test_ffn_launch_ragged_kinks(mode):
    """The fused FFN at hidden 2048 / ffn 5056 (79 row blocks of 64, 128
    reducing slices, one chunk of x per wave) with kink terms in gate, up and
    down (down's read h of other blocks through the tagged h words), alone
    (mask 12) and with the o projection in the launch (mask 14: o's kinks
    too, gate / up's kinks reading x + W_o attn from the tagged x words)."""
    from gsdlq import synth
    import run_gpu_native_chat as chat
    banner(f"fused FFN 2048 / 5056 {mode}, kinks")
    spec = synth.SynthSpec(n_layers=1, hidden=2048, ffn=5056, n_heads=16, n_kv_heads=4, head_dim=128, vocab=512,
                           mode=mode, kinks_per_row=2)
    src = synth.SynthSource(spec)
    gpu = chat.GPUMistralV2Model(src, max_seq_len=16, verbose=False)
    ref = O.OracleModel(src, kind="port", max_seq_len=16)
    try:
        assert gpu.cl.lib.gsdh_model_fused_ffn(gpu._m, 0) == 2
        rng = np.random.default_rng(110)
        for mask in (12, 14):
            x = rng.standard_normal(gpu.hidden).astype(np.float32)
            att = rng.standard_normal(gpu.n_heads * gpu.head_dim).astype(np.float32)
            _put(gpu, "x", x)
            _put(gpu, "attn", att)
            gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, mask)
            got = _get(gpu, "x", gpu.hidden)
            if mask & 2:
                yo = np.empty(gpu.hidden, np.float32)
                ref.matvec(att, ref.layers[0]["o"], yo)
                x = x + yo
            hr, y, want = _ffn_ref(ref, x)
            _check(f"{mode} FFN 2048/5056 mask {mask}: h", _get(gpu, "h", gpu.ffn_size), hr)
            _check(f"{mode} FFN 2048/5056 mask {mask}: x + down", got, want)
    finally:
        gpu.close()


def test_head_launch_full_shape(layer7b):
    mode, gpu, ref = layer7b
    rng = np.random.default_rng(105)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    _put(gpu, "x", x)
    gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 16)
    got = _get(gpu, "logits", gpu.vocab_size)
    xb = _rmsnorm(ref, x, ref.final_norm)
    want = np.empty(gpu.vocab_size, np.float32)
    ref.matvec(xb, ref.lm_head, want)
    _check(f"{mode} lm_head (32768x4096)", got, want)


def test_launches_repeat_bit_identical(layer7b):
    """A launch run twice on the same inputs gives the same bits (fixed
    reduction order; no state carried between launches)."""
    mode, gpu, _ = layer7b
    rng = np.random.default_rng(106)
    x = rng.standard_normal(gpu.hidden).astype(np.float32)
    outs = []
    for _ in range(2):
        _put(gpu, "x", x)
        gpu.cl.lib.gsdh_model_run_linear(gpu._m, 0, 4)
        outs.append(_get(gpu, "h", gpu.ffn_size))
    assert np.array_equal(outs[0], outs[1])
