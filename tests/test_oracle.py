"""Pins the CPU oracle (oracle/gsdref.c) before anything is compared with it:
against the reference engine built from source (when present), against the
golden vectors that engine wrote (always), and against closed forms and
float64 brute force chosen so that a dropped term, swapped operand or wrong
index fails."""
import ctypes

import numpy as np
import pytest

import oracle as O
from gsdlq import synth
from conftest import rel_l2

P = O.P
needs_ref = pytest.mark.skipif(not O.have_reference(), reason="reference engine source absent (oracle/_ref)")


# ---------------------------------------------------------------- fp16 ------
def test_f16_to_f32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = O.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _f32_edge_cases():
    # every half boundary and midpoint, +-1 ulp, subnormal range, overflow
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32).view(np.uint32).astype(np.int64)
    mids = (f[:-1] + f[1:]) // 2
    cand = np.concatenate([f, f + 1, f - 1, mids, mids + 1, mids - 1, [0x477FEFFF, 0x477FF000, 0x477FF001,
                                                                       0x33000000, 0x33000001, 0x32FFFFFF]])
    cand = cand[(cand >= 0) & (cand < 0x7F800000)].astype(np.uint32)
    return np.concatenate([cand, cand | 0x80000000]).view(np.float32)


def test_f32_to_f16_rne_vs_numpy():
    rng = np.random.default_rng(0)
    rnd = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for f in (_f32_edge_cases(), rnd):
        ours = O.f32_to_f16(f)
        with np.errstate(over="ignore", invalid="ignore"):
            ref = f.astype(np.float16).view(np.uint16)
        nan = np.isnan(f)
        assert np.array_equal(ours[~nan], ref[~nan])
        assert np.all((ours[nan] & 0x7C00) == 0x7C00) and np.all((ours[nan] & 0x3FF) != 0)


@needs_ref
def test_f16_conversions_vs_reference_engine():
    """Both conversions through the reference's own code paths: the V-cache
    store (fp32->fp16) and a one-column low-rank projection (fp16->fp32)."""
    ref = O.load("reference")
    rng = np.random.default_rng(1)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32),
                           _f32_edge_cases().view(np.uint32)])
    n = (bits.size // 128) * 128
    v = bits[:n].view(np.float32).copy()
    q = np.zeros(128, np.float32)
    k = np.zeros(n, np.float32)
    kc = np.zeros(n, np.uint16)
    vc = np.zeros(n, np.uint16)
    ref.gsd_cpu_rope_and_store_kv(P(q), P(k), P(v), P(kc), P(vc), 0, 0, 1, n // 128, 128, 1, 1e4, 1)
    assert np.array_equal(vc, O.f32_to_f16(v))
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = np.ones(1, np.float32)
    S = np.ones(65536, np.float32)
    out = np.zeros(65536, np.float32)
    ref.gsd_cpu_lowrank_proj(P(x), P(h), P(S), P(out), 65536, 1)
    ours = np.float32(0.0) + O.f16_to_f32(h)      # the harness adds to a 0.0f accumulator
    fin = ~np.isnan(ours)
    assert np.array_equal(out[fin].view(np.uint32), ours[fin].view(np.uint32))
    assert np.all(np.isnan(out[~fin]))


# ------------------------------------------------------------- codebook -----
@pytest.mark.parametrize("R,n", [(6, 127), (8, 217)])
def test_codebook_closed_form(R, n):
    xy, npts = O.codebook(R)
    assert npts == n == 3 * R * R + 3 * R + 1
    lib = O.load("port")
    cxy = np.zeros((256, 2), np.float32)
    r01 = np.zeros((256, 2), np.int8)
    assert lib.gsdref_codebook(R, P(cxy), P(r01)) == n
    assert np.array_equal(cxy[:n].view(np.uint32), xy.view(np.uint32))
    r0, r1 = r01[:n, 0].astype(int), r01[:n, 1].astype(int)
    assert np.all(np.abs(r0 + r1) <= R) and np.all(np.abs(r0) <= R) and np.all(np.abs(r1) <= R)
    # enumeration order: r0 outer, r1 inner, both ascending
    assert np.all(np.diff(r0 * 100 + r1) > 0)
    # exact f32 bits of the closed form evaluated in float64
    s32 = np.sqrt(3.0) / 2.0
    assert np.array_equal(xy[:, 0], (r0 + 0.5 * r1).astype(np.float32))
    assert np.array_equal(xy[:, 1].view(np.uint32), (r1 * s32).astype(np.float32).view(np.uint32))
    # the hexagon is point-symmetric: index i <-> n-1-i negates the point
    assert np.array_equal(r01[:n][::-1].astype(int), -r01[:n].astype(int))


def test_codebook_matches_product_tables():
    from gsdlq import codebook
    for R in (6, 8):
        xy, _ = O.codebook(R)
        assert np.array_equal(codebook.xy_table(R).view(np.uint32), xy.view(np.uint32))
        f = codebook.integer_fields(R)
        lib = O.load("port")
        r01 = np.zeros((256, 2), np.int8)
        n = lib.gsdref_codebook(R, None, P(r01))
        assert np.array_equal(f, r01[:n])


# ------------------------------------------------- goldens (reference) -----
def _hexf(g, tag):
    rows, cols, R, k = (int(v) for v in g[f"mv_{tag}_shape"])
    f = {key: g[f"mv_{tag}_{key}"] for key in ("codes", "scales", "row_ptr", "kink_cols", "kink_deltas",
                                               "U", "S", "Vt")}
    f.update(rows=rows, cols=cols, radius=R, k_dim=k)
    return f


@pytest.mark.parametrize("tag", ["turbo", "prec"])
def test_matvec_golden_bitexact(golden, tag):
    f = _hexf(golden, tag)
    y = O.hex2d_matvec(golden[f"mv_{tag}_x"], f)
    assert np.array_equal(y.view(np.uint32), golden[f"mv_{tag}_y"].view(np.uint32))


def test_small_ops_golden_bitexact(golden):
    lib = O.load("port")
    g = golden
    tk = np.zeros(16, np.float32)
    lib.gsd_cpu_lowrank_proj(P(g["lr_x"]), P(g["lr_Vt"]), P(g["lr_S"]), P(tk), 4, 256)
    assert np.array_equal(tk[:4], g["lr_out"])
    out = np.zeros(4096, np.float32)
    lib.gsd_cpu_rmsnorm(P(g["rms_x"]), P(g["rms_w"]), P(out), 4096, 1e-5)
    assert np.array_equal(out, g["rms_out"])
    out = np.zeros(1000, np.float32)
    lib.gsd_cpu_swiglu(P(g["sw_gate"]), P(g["sw_up"]), P(out), 1000)
    assert np.array_equal(out, g["sw_out"])
    lib.gsd_cpu_vec_add(P(out), P(g["sw_gate"]), P(g["sw_up"]), 1000)
    assert np.array_equal(out, g["add_out"])


@pytest.mark.parametrize("pos", [0, 7, 2047])
@pytest.mark.parametrize("il", [1, 0])
def test_rope_golden_bitexact(golden, pos, il):
    lib = O.load("port")
    t = f"rope_p{pos}_i{il}"
    q = golden[t + "_q"].copy()
    kc = np.zeros((1, 2048, 8, 128), np.uint16)
    vc = np.zeros((1, 2048, 8, 128), np.uint16)
    lib.gsd_cpu_rope_and_store_kv(P(q), P(golden[t + "_k"]), P(golden[t + "_v"]), P(kc), P(vc), 0, pos, 32, 8,
                                  128, 2048, 1e6, il)
    assert np.array_equal(q.view(np.uint32), golden[t + "_qout"].view(np.uint32))
    assert np.array_equal(kc[0, pos], golden[t + "_kc"])
    assert np.array_equal(vc[0, pos], golden[t + "_vc"])


@pytest.mark.parametrize("ctx", [1, 33, 512])
def test_attention_golden_bitexact(golden, ctx):
    from make_golden import attn_cache
    lib = O.load("port")
    kc, vc = attn_cache(ctx, "k", 512, 8, 128), attn_cache(ctx, "v", 512, 8, 128)
    out = np.zeros(32 * 128, np.float32)
    lib.gsd_cpu_gqa_attention(P(golden[f"attn{ctx}_q"]), P(kc), P(vc), P(out), 0, ctx - 1, 32, 8, 128, 512,
                              1.0 / float(np.sqrt(128)))
    assert np.array_equal(out.view(np.uint32), golden[f"attn{ctx}_out"].view(np.uint32))


def test_tiny_model_golden_bitexact(golden):
    from gsdlq import synth
    spec = synth.SynthSpec(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
                           mode="precision", kinks_per_row=2)
    m = O.OracleModel(synth.SynthSource(spec), kind="port")
    prompt = golden["tiny_prompt"].tolist()
    for pos, t in enumerate(prompt):
        lg = m.forward_token(t, pos)
        assert np.array_equal(lg.view(np.uint32), golden["tiny_logits"][pos].view(np.uint32))
    toks = []
    pos = len(prompt)
    for _ in range(8):
        nxt = m.greedy(lg)
        toks.append(nxt)
        lg = m.forward_token(nxt, pos)
        pos += 1
    assert toks == golden["tiny_tokens"].tolist()


# ------------------------------------------- port == reference, random ------
@needs_ref
@pytest.mark.parametrize("mode", ["turbo", "precision"])
def test_port_equals_reference_model(mode):
    from gsdlq import synth
    spec = synth.SynthSpec(n_layers=2, hidden=256, ffn=512, n_heads=8, n_kv_heads=2, head_dim=32, vocab=300,
                           mode=mode, kinks_per_row=3)
    src = synth.SynthSource(spec)
    a, b = O.OracleModel(src, "port"), O.OracleModel(src, "reference")
    for pos, t in enumerate([1, 2, 299, 5, 77, 8]):
        la, lb = a.forward_token(t, pos), b.forward_token(t, pos)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    assert np.array_equal(a.k_cache, b.k_cache) and np.array_equal(a.v_cache, b.v_cache)


@needs_ref
def test_port_equals_reference_attention_random():
    rng = np.random.default_rng(5)
    ref, port = O.load("reference"), O.load("port")
    for nh, nkv, hd, ctx in ((32, 8, 128, 300), (8, 8, 64, 17), (6, 2, 16, 2048)):
        q = rng.standard_normal(nh * hd).astype(np.float32)
        kc = rng.standard_normal((ctx, nkv, hd)).astype(np.float16).view(np.uint16)
        vc = rng.standard_normal((ctx, nkv, hd)).astype(np.float16).view(np.uint16)
        o1, o2 = np.zeros(nh * hd, np.float32), np.zeros(nh * hd, np.float32)
        for lib, o in ((ref, o1), (port, o2)):
            lib.gsd_cpu_gqa_attention(P(q), P(kc), P(vc), P(o), 0, ctx - 1, nh, nkv, hd, ctx, 0.125)
        assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))


# --------------------------------------------------- closed forms -----------
def _pack(rows, cols, R, k=0, kpr=0, seed=3):
    from gsdlq import pack
    W = pack.synth_bf16(seed, rows * 7 + cols, rows * cols).reshape(rows, cols)
    return pack.pack_tensor(W, R, k, kpr)


def _dense(f):
    """float64 W from the format via the oracle's brute-force decoder."""
    lib = O.load("port")
    xy, _ = O.codebook(f["radius"])
    W = np.zeros((f["rows"], f["cols"]), np.float64)
    kc = f["kink_cols"] if f["kink_cols"].size else np.zeros(1, np.uint16)
    kd = f["kink_deltas"] if f["kink_deltas"].size else np.zeros(1, np.float32)
    lib.gsdref_dequant(P(f["codes"]), P(f["scales"]), P(xy), P(f["row_ptr"]), P(kc), P(kd), P(W), f["rows"], f["cols"])
    return W


def test_dequant_brute_force_independent():
    """gsdref_dequant against a numpy decode written from the format spec."""
    f = _pack(16, 192, 8, 0, 3)
    xy, _ = O.codebook(8)
    i = np.arange(16 * 192)
    pts = xy[f["codes"][i >> 1].astype(int), i & 1].astype(np.float64)
    sc = f["scales"][i >> 6].view(np.float16).astype(np.float64)
    W = (pts * sc).reshape(16, 192)
    for r in range(16):
        for j in range(f["row_ptr"][r], f["row_ptr"][r + 1]):
            W[r, f["kink_cols"][j]] += f["kink_deltas"][j]
    assert np.array_equal(W, _dense(f))


@pytest.mark.parametrize("R,k,kpr", [(8, 0, 0), (8, 0, 4), (6, 2, 0), (6, 4, 2)])
def test_matvec_vs_float64_dense(R, k, kpr):
    f = _pack(96, 320, R, k, kpr)
    x = np.random.default_rng(9).standard_normal(320).astype(np.float32)
    W = _dense(f)
    if k:
        U = f["U"].view(np.float16).astype(np.float64).reshape(96, k)
        Vt = f["Vt"].view(np.float16).astype(np.float64).reshape(k, 320)
        W = W + U @ (f["S"].astype(np.float64)[:, None] * Vt)
    y = O.hex2d_matvec(x, f)
    assert rel_l2(y, W @ x.astype(np.float64)) < 1e-6


def test_matvec_special_cases():
    from gsdlq import codebook
    f = _pack(32, 128, 6, 2, 2)
    x = np.random.default_rng(2).standard_normal(128).astype(np.float32)
    # all codes at the origin -> y = kinks + low-rank only
    g = dict(f)
    g["codes"] = np.full_like(f["codes"], codebook.index_of(6)[6, 6])
    U = f["U"].view(np.float16).astype(np.float64).reshape(32, 2)
    Vt = f["Vt"].view(np.float16).astype(np.float64).reshape(2, 128)
    kinks = np.zeros(32)
    for r in range(32):
        for j in range(f["row_ptr"][r], f["row_ptr"][r + 1]):
            kinks[r] += f["kink_deltas"][j] * x[f["kink_cols"][j]]
    want = kinks + U @ (f["S"].astype(np.float64) * (Vt @ x))
    assert rel_l2(O.hex2d_matvec(x, g), want) < 1e-6
    # one-hot x extracts a column of the dense matrix
    h = _pack(16, 128, 8)
    Wd = _dense(h)
    for c in (0, 1, 63, 64, 127):
        e = np.zeros(128, np.float32)
        e[c] = 1.0
        assert np.array_equal(O.hex2d_matvec(e, h).astype(np.float64), Wd[:, c].astype(np.float32).astype(np.float64))


def test_lowrank_rmsnorm_swiglu_closed_forms():
    lib = O.load("port")
    rng = np.random.default_rng(4)
    x = rng.standard_normal(512).astype(np.float32)
    Vt = (rng.standard_normal((3, 512)) * 0.1).astype(np.float16)
    S = np.array([0.5, 2.0, 1.25], np.float32)
    tk = np.zeros(16, np.float32)
    lib.gsd_cpu_lowrank_proj(P(x), P(Vt.view(np.uint16)), P(S), P(tk), 3, 512)
    assert rel_l2(tk[:3], S * (Vt.astype(np.float64) @ x)) < 1e-6
    w = rng.uniform(0.5, 2, 512).astype(np.float32)
    out = np.zeros(512, np.float32)
    lib.gsd_cpu_rmsnorm(P(x), P(w), P(out), 512, 1e-5)
    xd = x.astype(np.float64)
    assert rel_l2(out, xd / np.sqrt(np.mean(xd * xd) + 1e-5) * w) < 1e-6
    u = rng.standard_normal(512).astype(np.float32)
    lib.gsd_cpu_swiglu(P(x), P(u), P(out), 512)
    assert rel_l2(out, xd / (1 + np.exp(-xd)) * u) < 1e-6


def test_rope_closed_form():
    lib = O.load("port")
    rng = np.random.default_rng(6)
    nh, nkv, hd, ms = 4, 2, 64, 16
    for il in (1, 0):
        for pos in (0, 5, 15):
            q = rng.standard_normal(nh * hd).astype(np.float32)
            k = rng.standard_normal(nkv * hd).astype(np.float32)
            v = rng.standard_normal(nkv * hd).astype(np.float32)
            kc = np.zeros((1, ms, nkv, hd), np.uint16)
            vc = np.zeros((1, ms, nkv, hd), np.uint16)
            q0 = q.copy()
            lib.gsd_cpu_rope_and_store_kv(P(q), P(k), P(v), P(kc), P(vc), 0, pos, nh, nkv, hd, ms, 1e4, il)
            assert np.array_equal(vc[0, pos].reshape(-1), O.f32_to_f16(v))
            i = np.arange(hd // 2)
            ang = pos * (1e4 ** (-(2.0 * i) / hd))
            a = q0.reshape(nh, hd).astype(np.float64)
            i0, i1 = (2 * i, 2 * i + 1) if il else (i, i + hd // 2)
            want = a.copy()
            want[:, i0] = a[:, i0] * np.cos(ang) - a[:, i1] * np.sin(ang)
            want[:, i1] = a[:, i0] * np.sin(ang) + a[:, i1] * np.cos(ang)
            assert rel_l2(q, want.reshape(-1)) < 1e-5
            if pos == 0:
                assert np.array_equal(q, q0)
                assert np.array_equal(kc[0, 0].reshape(-1), O.f32_to_f16(k))


def test_attention_closed_forms():
    lib = O.load("port")
    rng = np.random.default_rng(7)
    nh, nkv, hd, ms = 8, 2, 64, 64
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal((ms, nkv, hd)).astype(np.float16)
    vc = rng.standard_normal((ms, nkv, hd)).astype(np.float16)
    out = np.zeros(nh * hd, np.float32)
    # pos 0: out = V_0 exactly
    lib.gsd_cpu_gqa_attention(P(q), P(kc.view(np.uint16)), P(vc.view(np.uint16)), P(out), 0, 0, nh, nkv, hd, ms, 0.125)
    for h in range(nh):
        assert np.array_equal(out[h * hd:(h + 1) * hd], vc[0, h // 4].astype(np.float32))
    # brute-force float64 softmax at pos 40
    lib.gsd_cpu_gqa_attention(P(q), P(kc.view(np.uint16)), P(vc.view(np.uint16)), P(out), 0, 40, nh, nkv, hd, ms, 0.125)
    K, V = kc[:41].astype(np.float64), vc[:41].astype(np.float64)
    want = np.zeros((nh, hd))
    for h in range(nh):
        s = K[:, h // 4] @ q[h * hd:(h + 1) * hd].astype(np.float64) * 0.125
        p = np.exp(s - s.max())
        want[h] = (p / p.sum()) @ V[:, h // 4]
    assert rel_l2(out, want.reshape(-1)) < 1e-6
    # identical keys -> mean of V
    kc2 = np.repeat(kc[:1], ms, axis=0)
    lib.gsd_cpu_gqa_attention(P(q), P(kc2.view(np.uint16)), P(vc.view(np.uint16)), P(out), 0, 9, nh, nkv, hd, ms, 0.125)
    for h in range(nh):
        assert rel_l2(out[h * hd:(h + 1) * hd], V[:10, h // 4].mean(0)) < 1e-6


# ---------------------------------------------------------------------------
# The oracle's composition (OracleModel.forward_token) against an independent
# float64 NumPy forward written from the reference's per-token order
# (gsd_lq_cpu_runtime.py:302-420) with its own dense dequantisation of every
# packed tensor (codebook closed form, fp16 block scales, CSR kinks,
# U diag(S) Vt), so a misreading shared by the oracle's driver and the
# engine's (a head mapping, a residual, the RoPE pairing) cannot hide.
# ---------------------------------------------------------------------------
def _dense_f64(src, name):
    m = src.tensors[name]
    R, rows, cols, k = m["radius"], m["rows"], m["cols"], m["k_dim"]
    s3 = np.sqrt(3.0) / 2.0
    T = np.array([(a + 0.5 * b, b * s3) for a in range(-R, R + 1) for b in range(-R, R + 1) if abs(a + b) <= R])
    codes = np.asarray(src.hex_field(name, "codes")).reshape(rows, cols // 2)
    W = T[codes].reshape(rows, cols)
    sc = np.asarray(src.hex_field(name, "scales")).view(np.float16).astype(np.float64).reshape(rows, cols // 64)
    W = W * np.repeat(sc, 64, axis=1)
    rp = np.asarray(src.hex_field(name, "row_ptr"))
    kc = np.asarray(src.hex_field(name, "kink_cols"))
    kd = np.asarray(src.hex_field(name, "kink_deltas")).astype(np.float64)
    for r in range(rows):
        for i in range(rp[r], rp[r + 1]):
            W[r, kc[i]] += kd[i]
    if k > 0:
        U = np.asarray(src.hex_field(name, "U")).view(np.float16).astype(np.float64).reshape(rows, k)
        S = np.asarray(src.hex_field(name, "S")).astype(np.float64)
        Vt = np.asarray(src.hex_field(name, "Vt")).view(np.float16).astype(np.float64).reshape(k, cols)
        W = W + U @ (S[:, None] * Vt)
    return W


class _F64Model:
    def __init__(self, src, interleaved):
        c = src.config
        self.L, self.H, self.nh, self.nkv = c["n_layers"], c["hidden_size"], c["n_heads"], c["n_kv_heads"]
        self.hd, self.eps, self.theta = c["head_dim"], c["rms_eps"], c["rope_theta"]
        self.il = interleaved
        self.emb = np.asarray(src.dense("token_embd.weight", np.float16)).astype(np.float64)
        self.W = {n: _dense_f64(src, n) for n in src.tensors if "k_dim" in src.tensors[n]}
        self.norm = {n: np.asarray(src.dense(n, np.float32)).astype(np.float64)
                     for n in src.tensors if n.endswith("norm.weight")}
        self.kc = {}
        self.vc = {}

    def rms(self, x, w):
        return x / np.sqrt(np.mean(x * x) + self.eps) * w

    def rope(self, v, pos):
        hd, half = self.hd, self.hd // 2
        ang = pos / self.theta ** (np.arange(half) * 2.0 / hd)
        c, s = np.cos(ang), np.sin(ang)
        v = v.reshape(-1, hd).copy()
        i0 = np.arange(half) * 2 if self.il else np.arange(half)
        i1 = i0 + 1 if self.il else i0 + half
        a, b = v[:, i0].copy(), v[:, i1].copy()
        v[:, i0], v[:, i1] = a * c - b * s, a * s + b * c
        return v

    def forward(self, tok, pos):
        x = self.emb[tok].copy()
        g = self.nh // self.nkv
        for l in range(self.L):
            p = f"blk.{l}."
            xb = self.rms(x, self.norm[p + "attn_norm.weight"])
            q = self.rope(self.W[p + "attn_q.weight"] @ xb, pos)
            k = self.rope(self.W[p + "attn_k.weight"] @ xb, pos)
            v = (self.W[p + "attn_v.weight"] @ xb).reshape(self.nkv, self.hd)
            f16 = lambda a: a.astype(np.float16).astype(np.float64)
            self.kc[(l, pos)], self.vc[(l, pos)] = f16(k), f16(v)
            K = np.stack([self.kc[(l, t)] for t in range(pos + 1)])      # [t, nkv, hd]
            V = np.stack([self.vc[(l, t)] for t in range(pos + 1)])
            att = np.empty((self.nh, self.hd))
            for h in range(self.nh):
                sc = K[:, h // g] @ q[h] / np.sqrt(self.hd)
                e = np.exp(sc - sc.max())
                att[h] = (e / e.sum()) @ V[:, h // g]
            x = x + self.W[p + "attn_output.weight"] @ att.reshape(-1)
            xb = self.rms(x, self.norm[p + "ffn_norm.weight"])
            gt, up = self.W[p + "ffn_gate.weight"] @ xb, self.W[p + "ffn_up.weight"] @ xb
            x = x + self.W[p + "ffn_down.weight"] @ (gt / (1.0 + np.exp(-gt)) * up)
        return self.W["output.weight"] @ self.rms(x, self.norm["output_norm.weight"])


@pytest.mark.parametrize("mode,il,kpr", [("precision", 1, 2), ("turbo", 0, 1)])
def test_oracle_forward_vs_float64_numpy(mode, il, kpr):
    spec = synth.SynthSpec(n_layers=2, hidden=128, ffn=256, n_heads=4, n_kv_heads=2, head_dim=32, vocab=300,
                           mode=mode, kinks_per_row=kpr)
    src = synth.SynthSource(spec)
    ref = O.OracleModel(src, kind="port", max_seq_len=32, rope_interleaved=il)
    f64 = _F64Model(src, il)
    toks = np.random.default_rng(5).integers(0, spec.vocab, 9).tolist()
    for pos, t in enumerate(toks):
        want = f64.forward(t, pos)
        got = ref.forward_token(t, pos)
        assert rel_l2(got, want) < 1e-4, (mode, pos)
