"""Operator parity on the GPU: each C-ABI twin against the oracle on the same
seeded inputs.  Bar: bit-exact for integer decode and for RoPE/KV append
(whose arithmetic is fixed by the reference), 1e-3 relative L2 for matvec and
attention (fp32 accumulation in a different order)."""
import ctypes

import numpy as np
import pytest

import oracle as O
from conftest import rel_l2
from gpu_util import D, E, H, banner, p

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def lib():
    from gsdlq import hip
    name, total, ncu = hip.device_info()     # raises when no GPU is visible
    assert ncu > 0, name
    return hip.lib()


def _pack(rows, cols, R, k=0, kpr=0, seed=1):
    from gsdlq import pack
    W = pack.synth_bf16(seed, rows * 13 + cols, rows * cols).reshape(rows, cols)
    return pack.pack_tensor(W, R, k, kpr)


def _gpu_matvec(lib, f, x, tmp_k=None):
    rows, cols, k = f["rows"], f["cols"], f["k_dim"]
    xy, n_pts = O.codebook(f["radius"])
    y = E(rows * 4)
    tk = None
    if k:
        tk = D(np.asarray(tmp_k, np.float32))
    bufs = {key: D(f[key]) for key in ("codes", "scales", "row_ptr", "kink_cols", "kink_deltas", "U")}
    dx, dxy = D(x), D(xy)    # hold every buffer until the result is read back
    lib.gsdh_hex2d_matvec(None, p(dx), p(bufs["codes"]), p(bufs["scales"]), p(dxy), p(bufs["U"]) if k else None,
                          p(tk), p(bufs["row_ptr"]), p(bufs["kink_cols"]), p(bufs["kink_deltas"]), p(y), rows, cols,
                          k, n_pts)
    return H(y, np.float32, rows)


MV_CASES = [(64, 128, 8, 0, 2), (37, 192, 8, 0, 1), (1, 64, 6, 0, 0), (4096, 4096, 8, 0, 0),
            (1024, 4096, 6, 2, 3), (4096, 14336, 8, 0, 0), (300, 1024, 6, 16, 4), (14336, 4096, 6, 2, 0)]


@pytest.mark.parametrize("rows,cols,R,k,kpr", MV_CASES)
def test_hex2d_matvec_vs_oracle(lib, rows, cols, R, k, kpr):
    banner(f"matvec {rows}x{cols} R{R} k{k} kinks/row {kpr}")
    f = _pack(rows, cols, R, k, kpr)
    x = np.random.default_rng(rows + cols).standard_normal(cols).astype(np.float32)
    tk = None
    if k:
        tk = np.zeros(16, np.float32)
        O.load("port").gsd_cpu_lowrank_proj(O.P(x), O.P(f["Vt"]), O.P(f["S"]), O.P(tk), k, cols)
        tk = tk[:k]
    want = O.hex2d_matvec(x, f, tmp_k=tk)
    got = _gpu_matvec(lib, f, x, tk)
    assert rel_l2(got, want) < TOL
    assert rel_l2(got, want) < 1e-5   # fp32 accumulation order only


@pytest.mark.parametrize("tag", ["turbo", "prec"])
def test_hex2d_matvec_golden(lib, golden, tag):
    rows, cols, R, k = (int(v) for v in golden[f"mv_{tag}_shape"])
    f = {key: golden[f"mv_{tag}_{key}"] for key in ("codes", "scales", "row_ptr", "kink_cols", "kink_deltas",
                                                    "U", "S", "Vt")}
    f.update(rows=rows, cols=cols, radius=R, k_dim=k)
    x = golden[f"mv_{tag}_x"]
    tk = None
    if k:
        tk = np.zeros(16, np.float32)
        O.load("port").gsd_cpu_lowrank_proj(O.P(x), O.P(f["Vt"]), O.P(f["S"]), O.P(tk), k, cols)
        tk = tk[:k]
    assert rel_l2(_gpu_matvec(lib, f, x, tk), golden[f"mv_{tag}_y"]) < TOL


def test_hex2d_matvec_rejects_bad_shapes(lib):
    from gsdlq.hip import HipError
    y = E(64)
    with pytest.raises(HipError, match="multiple of 64"):
        lib.gsdh_hex2d_matvec(None, p(y), p(y), p(y), p(y), None, None, p(y), p(y), p(y), p(y), 4, 96, 0, 217)
    with pytest.raises(HipError, match="n_pts"):
        lib.gsdh_hex2d_matvec(None, p(y), p(y), p(y), p(y), None, None, p(y), p(y), p(y), p(y), 4, 64, 0, 300)


@pytest.mark.parametrize("R", [6, 8])
def test_unpack_codes_bitexact(lib, R):
    from gsdlq import codebook
    n_pts = codebook.n_points(R)
    codes = np.concatenate([np.arange(n_pts, dtype=np.uint8),
                            np.random.default_rng(R).integers(0, n_pts, 100000).astype(np.uint8)])
    idx, r01, dc = E(codes.size * 4), E(codes.size * 2), D(codes)
    lib.gsdh_unpack_codes(None, p(dc), codes.size, R, p(idx), p(r01))
    assert np.array_equal(H(idx, np.int32, codes.size), codes.astype(np.int32))
    want = codebook.integer_fields(R)[codes]
    assert np.array_equal(H(r01, np.int8, codes.size * 2).reshape(-1, 2), want)


def test_lowrank_rmsnorm_swiglu_add(lib, golden):
    g = golden
    d = {k: D(g[k]) for k in ("lr_x", "lr_Vt", "lr_S", "rms_x", "rms_w", "sw_gate", "sw_up")}
    tk = E(64)
    lib.gsdh_lowrank_proj(None, p(d["lr_x"]), p(d["lr_Vt"]), p(d["lr_S"]), p(tk), 4, 256)
    assert rel_l2(H(tk, np.float32, 4), g["lr_out"]) < 1e-6
    out = E(4096 * 4)
    lib.gsdh_rmsnorm(None, p(d["rms_x"]), p(d["rms_w"]), p(out), 4096, 1e-5)
    assert rel_l2(H(out, np.float32, 4096), g["rms_out"]) < 1e-6
    out = E(4000)
    lib.gsdh_swiglu(None, p(d["sw_gate"]), p(d["sw_up"]), p(out), 1000)
    assert rel_l2(H(out, np.float32, 1000), g["sw_out"]) < 1e-6
    lib.gsdh_vec_add(None, p(out), p(d["sw_gate"]), p(d["sw_up"]), 1000)
    assert np.array_equal(H(out, np.float32, 1000), g["add_out"])


@pytest.mark.parametrize("pos", [0, 7, 2047])
@pytest.mark.parametrize("il", [1, 0])
def test_rope_kv_bitexact(lib, golden, pos, il):
    t = f"rope_p{pos}_i{il}"
    q, dk, dv = D(golden[t + "_q"]), D(golden[t + "_k"]), D(golden[t + "_v"])
    kc, vc = E(2048 * 8 * 128 * 2), E(2048 * 8 * 128 * 2)
    lib.gsdh_rope_and_store_kv(None, p(q), p(dk), p(dv), p(kc), p(vc), 0, pos,
                               32, 8, 128, 2048, 1e6, il)
    assert np.array_equal(H(q, np.uint32, 32 * 128), golden[t + "_qout"].view(np.uint32))
    assert np.array_equal(H(kc, np.uint16, 2048 * 8 * 128).reshape(2048, 8, 128)[pos], golden[t + "_kc"])
    assert np.array_equal(H(vc, np.uint16, 2048 * 8 * 128).reshape(2048, 8, 128)[pos], golden[t + "_vc"])


@pytest.mark.parametrize("ctx", [1, 33, 512])
def test_attention_golden(lib, golden, ctx):
    from make_golden import attn_cache
    kc, vc = attn_cache(ctx, "k", 512, 8, 128), attn_cache(ctx, "v", 512, 8, 128)
    out, dq, dk, dv = E(32 * 128 * 4), D(golden[f"attn{ctx}_q"]), D(kc), D(vc)
    lib.gsdh_gqa_attention(None, p(dq), p(dk), p(dv), p(out), 0, ctx - 1, 32, 8,
                           128, 512, 1.0 / float(np.sqrt(128)))
    assert rel_l2(H(out, np.float32, 32 * 128), golden[f"attn{ctx}_out"]) < TOL


@pytest.mark.parametrize("ctx,nh,nkv,hd,layers", [(2048, 32, 8, 128, 2), (8192, 32, 8, 128, 1), (100, 8, 8, 64, 1),
                                                  (777, 16, 2, 256, 1), (4000, 32, 8, 128, 1)])
def test_attention_vs_oracle(lib, ctx, nh, nkv, hd, layers):
    banner(f"attention ctx {ctx} heads {nh}/{nkv} hd {hd}")
    from gsdlq import pack
    ms = ctx + 5
    kc = pack.synth_f16(21, ctx, layers * ms * nkv * hd, 1.0)
    vc = pack.synth_f16(22, ctx, layers * ms * nkv * hd, 1.0)
    q = np.random.default_rng(ctx).standard_normal(nh * hd).astype(np.float32)
    want = np.zeros(nh * hd, np.float32)
    layer = layers - 1
    O.load("port").gsd_cpu_gqa_attention(O.P(q), O.P(kc), O.P(vc), O.P(want), layer, ctx - 1, nh, nkv, hd, ms,
                                         1.0 / float(np.sqrt(hd)))
    out = E(nh * hd * 4)
    dk, dv, dq = D(kc), D(vc), D(q)
    for _ in range(2):   # twice: the split counters must be reset by the kernel itself
        lib.gsdh_gqa_attention(None, p(dq), p(dk), p(dv), p(out), layer, ctx - 1, nh, nkv, hd, ms,
                               1.0 / float(np.sqrt(hd)))
        assert rel_l2(H(out, np.float32, nh * hd), want) < TOL


# head_dim 256 with 4 query heads per KV head (16 waves), 2 query heads per KV
# head at hd 128 and 64
@pytest.mark.parametrize("ctx,nh,nkv,hd", [(777, 8, 2, 256), (1500, 16, 8, 128), (3000, 8, 4, 64), (300, 8, 2, 256)])
def test_attention_group_sizes_vs_oracle(lib, ctx, nh, nkv, hd):
    banner(f"attention ctx {ctx} heads {nh}/{nkv} hd {hd}")
    _attention_case(lib, ctx, nh, nkv, hd, seed=ctx + hd)


# the split merge: 16 KV heads x 17 splits (272 blocks, more than the CUs of
# an MI355X: the last split's block merges alone), 1 slice of 64 outputs per
# KV head (one merger), 4 slices over 24 splits (4 mergers, waves whose third
# split is past the last), and 8 slices over 32 splits (8 mergers); with at
# most 8 splits and fewer mergers than slices, every wave of a merger takes a
# slice of its own: 8 slices over 4, 7 and 3 splits (2, 2 and 3 slices in the
# first merger); each twice, the second call reusing the split words of the
# first
@pytest.mark.parametrize("ctx,nh,nkv,hd", [(4100, 32, 16, 64), (1000, 8, 8, 64), (3000, 16, 8, 128),
                                           (8000, 32, 8, 128), (200, 32, 8, 128), (400, 32, 8, 128),
                                           (150, 16, 4, 128)])
def test_attention_merge_paths_vs_oracle(lib, ctx, nh, nkv, hd):
    banner(f"attention merge ctx {ctx} heads {nh}/{nkv} hd {hd}")
    for rep in range(2):
        _attention_case(lib, ctx, nh, nkv, hd, seed=ctx + nkv + rep)


def _attention_case(lib, ctx, nh, nkv, hd, seed, ms=None):
    from gsdlq import pack
    ms = ms or ctx + 3
    kc = pack.synth_f16(seed, ctx, ms * nkv * hd, 1.0)
    vc = pack.synth_f16(seed + 1, ctx, ms * nkv * hd, 1.0)
    q = np.random.default_rng(seed).standard_normal(nh * hd).astype(np.float32)
    want = np.zeros(nh * hd, np.float32)
    O.load("port").gsd_cpu_gqa_attention(O.P(q), O.P(kc), O.P(vc), O.P(want), 0, ctx - 1, nh, nkv, hd, ms,
                                         1.0 / float(np.sqrt(hd)))
    out, dk, dv, dq = E(nh * hd * 4), D(kc), D(vc), D(q)
    lib.gsdh_gqa_attention(None, p(dq), p(dk), p(dv), p(out), 0, ctx - 1, nh, nkv, hd, ms, 1.0 / float(np.sqrt(hd)))
    got = H(out, np.float32, nh * hd)
    assert rel_l2(got, want) < TOL, (ctx, nh, nkv, hd)


@pytest.mark.parametrize("ctx,nkv,hd", [(1, 8, 128), (100, 8, 128), (255, 8, 128), (256, 8, 128), (700, 8, 128),
                                         (60, 8, 64)])
def test_attention_ignores_cache_rows_past_context(lib, ctx, nkv, hd):
    """Rows past the context hold NaN (the cache's unwritten slots may hold
    anything): the kernel loads whole chunks and masks, so no NaN may reach
    the output, which must equal the oracle's on the valid rows."""
    banner(f"attention ctx {ctx} with NaN rows past the context")
    from gsdlq import pack
    nh, ms = 4 * nkv, ctx + 300
    kc = pack.synth_f16(71, ctx, ms * nkv * hd, 1.0).reshape(ms, nkv * hd)
    vc = pack.synth_f16(72, ctx, ms * nkv * hd, 1.0).reshape(ms, nkv * hd)
    q = np.random.default_rng(ctx).standard_normal(nh * hd).astype(np.float32)
    want = np.zeros(nh * hd, np.float32)
    O.load("port").gsd_cpu_gqa_attention(O.P(q), O.P(kc), O.P(vc), O.P(want), 0, ctx - 1, nh, nkv, hd, ms,
                                         1.0 / float(np.sqrt(hd)))
    kc, vc = kc.copy(), vc.copy()
    kc[ctx:] = 0x7E00   # fp16 NaN
    vc[ctx:] = 0x7E00
    out, dk, dv, dq = E(nh * hd * 4), D(kc), D(vc), D(q)
    lib.gsdh_gqa_attention(None, p(dq), p(dk), p(dv), p(out), 0, ctx - 1, nh, nkv, hd, ms, 1.0 / float(np.sqrt(hd)))
    got = H(out, np.float32, nh * hd)
    assert np.isfinite(got).all()
    assert rel_l2(got, want) < TOL


@pytest.mark.parametrize("ctx,nh,nkv,hd,il", [(1, 32, 8, 128, 1), (100, 32, 8, 128, 0), (256, 32, 8, 128, 1),
                                               (700, 32, 8, 128, 1), (5000, 32, 8, 128, 0), (300, 8, 8, 64, 1),
                                               (90, 8, 4, 64, 0), (777, 16, 2, 256, 1)])
def test_rope_store_attention_equals_two_calls(lib, ctx, nh, nkv, hd, il):
    """gsdh_rope_store_gqa_attention (one launch where the shape allows)
    against gsdh_rope_and_store_kv + gsdh_gqa_attention on copies of the same
    inputs: rotated q, the cache rows at pos and the output, bit for bit
    (head dim 256 runs the two launches)."""
    banner(f"rope + attention fused: ctx {ctx} heads {nh}/{nkv} hd {hd} interleaved {il}")
    from gsdlq import pack
    ms, pos = ctx + 4, ctx - 1
    kc = pack.synth_f16(81, ctx, ms * nkv * hd, 1.0)
    vc = pack.synth_f16(82, ctx, ms * nkv * hd, 1.0)
    rng = np.random.default_rng(ctx + il)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    sc = 1.0 / float(np.sqrt(hd))
    outs = []
    for fused in (False, True):
        dq, dk, dv, dkc, dvc, out = D(q), D(k), D(v), D(kc), D(vc), E(nh * hd * 4)
        if fused:
            assert lib.gsdh_rope_store_gqa_attention(None, p(dq), p(dk), p(dv), p(dkc), p(dvc), p(out), 0, pos, nh,
                                                     nkv, hd, ms, 1e6, il, sc) == 0
        else:
            assert lib.gsdh_rope_and_store_kv(None, p(dq), p(dk), p(dv), p(dkc), p(dvc), 0, pos, nh, nkv, hd, ms,
                                              1e6, il) == 0
            assert lib.gsdh_gqa_attention(None, p(dq), p(dkc), p(dvc), p(out), 0, pos, nh, nkv, hd, ms, sc) == 0
        outs.append((H(dq, np.uint32, nh * hd), H(dkc, np.uint16, ms * nkv * hd), H(dvc, np.uint16, ms * nkv * hd),
                     H(out, np.float32, nh * hd)))
    (q0, k0, v0, o0), (q1, k1, v1, o1) = outs
    assert np.array_equal(q0, q1), "rotated q"
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1), "cache"
    assert np.isfinite(o1).all()
    assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32)), rel_l2(o1, o0)


@pytest.mark.parametrize("p0,M,nh,nkv,hd,layers,ms", [
    (0, 512, 32, 8, 128, 1, 600),     # the 7B shape, a prompt's first 512 tokens
    (512, 512, 32, 8, 128, 2, 1100),  # its next 512 (layer 1 of 2)
    (37, 40, 8, 4, 64, 1, 96),        # 2 query heads per KV head, ragged groups
    (70, 9, 8, 1, 256, 1, 90),        # 8 per KV head, head dim 256
    (5, 70, 4, 4, 128, 1, 80),        # 1 per KV head
    (0, 1, 32, 8, 128, 1, 8),         # one token at position 0
    (100, 28, 16, 4, 128, 1, 128),    # the batch ends at the last cache row
])
def test_prefill_attention_vs_oracle(lib, p0, M, nh, nkv, hd, layers, ms):
    """gsdh_prefill_attention: token t at position p0 + t over positions
    0 .. p0 + t, against the oracle's one-token attention at that position,
    for every token; cache rows past the batch hold NaN, which must not
    reach the output.  Then the last token against gsdh_gqa_attention."""
    banner(f"prefill attention p0 {p0} M {M} heads {nh}/{nkv} hd {hd}")
    from gsdlq import pack
    layer = layers - 1
    n = layers * ms * nkv * hd
    kc = pack.synth_f16(81, p0 + M, n, 1.0).reshape(layers, ms, nkv * hd)
    vc = pack.synth_f16(82, p0 + M, n, 1.0).reshape(layers, ms, nkv * hd)
    kc[layer, p0 + M:] = 0x7E00   # fp16 NaN past the context
    vc[layer, p0 + M:] = 0x7E00
    q = np.random.default_rng(p0 + M).standard_normal((M, nh * hd)).astype(np.float32)
    sc = 1.0 / float(np.sqrt(hd))
    want = np.zeros((M, nh * hd), np.float32)
    ref = O.load("port")
    for t in range(M):
        ref.gsd_cpu_gqa_attention(O.P(q[t]), O.P(kc), O.P(vc), O.P(want[t]), layer, p0 + t, nh, nkv, hd, ms, sc)
    dq, dk, dv, out = D(q), D(kc), D(vc), E(M * nh * hd * 4)
    lib.gsdh_prefill_attention(None, p(dq), p(dk), p(dv), p(out), layer, p0, M, nh, nkv, hd, ms, sc)
    got = H(out, np.float32, M * nh * hd).reshape(M, nh * hd)
    assert np.isfinite(got).all()
    worst = max(rel_l2(got[t], want[t]) for t in range(M))
    assert worst < 1e-4, worst   # fp16 high + low operands: ~1e-6 measured
    one = E(nh * hd * 4)
    lib.gsdh_gqa_attention(None, p(D(q[M - 1])), p(dk), p(dv), p(one), layer, p0 + M - 1, nh, nkv, hd, ms, sc)
    assert rel_l2(got[M - 1], H(one, np.float32, nh * hd)) < 1e-4


def test_prefill_attention_rejects_bad_shapes(lib):
    from gsdlq.hip import HipError
    y = E(64)
    with pytest.raises(HipError, match="max_seq_len"):
        lib.gsdh_prefill_attention(None, p(y), p(y), p(y), p(y), 0, 100, 29, 32, 8, 128, 128, 0.088)
    with pytest.raises(HipError, match="head_dim"):
        lib.gsdh_prefill_attention(None, p(y), p(y), p(y), p(y), 0, 0, 4, 32, 8, 96, 128, 0.1)
    with pytest.raises(HipError, match="query heads"):
        lib.gsdh_prefill_attention(None, p(y), p(y), p(y), p(y), 0, 0, 4, 48, 3, 128, 128, 0.088)


def test_attention_shape_changes_between_calls(lib):
    """One call per shape, in an order whose split-word regions overlap: 8 KV
    heads, then 2 KV heads of 256 dims, then 8 KV heads again (a word left by
    an earlier call of another shape must never be taken for this call's)."""
    banner("attention: 8 KV heads -> 2 KV heads (hd 256) -> 8 KV heads")
    _attention_case(lib, 2048, 32, 8, 128, seed=61)
    _attention_case(lib, 1200, 8, 2, 256, seed=62)
    _attention_case(lib, 2048, 32, 8, 128, seed=63)
    _attention_case(lib, 5000, 32, 8, 128, seed=64)
    _attention_case(lib, 700, 16, 2, 64, seed=65)
    _attention_case(lib, 2048, 32, 8, 128, seed=66)


@pytest.mark.parametrize("pos", [2048, 4095, 8191])
@pytest.mark.parametrize("il", [1, 0])
def test_rope_kv_bitexact_long_positions(lib, pos, il):
    """RoPE + K/V append past the reference's 2048-position cache, up to the
    last slot of an 8192-position cache, bit-exact against the oracle (the
    same C library cos/sin)."""
    ms, nh, nkv, hd = 8192, 32, 8, 128
    rng = np.random.default_rng(pos + il)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    qr, kcr, vcr = q.copy(), np.zeros((ms, nkv, hd), np.uint16), np.zeros((ms, nkv, hd), np.uint16)
    O.load("port").gsd_cpu_rope_and_store_kv(O.P(qr), O.P(k), O.P(v), O.P(kcr), O.P(vcr), 0, pos, nh, nkv, hd, ms,
                                             1e6, il)
    dq, dk, dv = D(q), D(k), D(v)
    kc, vc = E(ms * nkv * hd * 2), E(ms * nkv * hd * 2)
    lib.gsdh_rope_and_store_kv(None, p(dq), p(dk), p(dv), p(kc), p(vc), 0, pos, nh, nkv, hd, ms, 1e6, il)
    assert np.array_equal(H(dq, np.uint32, nh * hd), qr.view(np.uint32))
    assert np.array_equal(H(kc, np.uint16, ms * nkv * hd).reshape(ms, nkv, hd)[pos], kcr[pos])
    assert np.array_equal(H(vc, np.uint16, ms * nkv * hd).reshape(ms, nkv, hd)[pos], vcr[pos])


def _argmax_cases():
    rng = np.random.default_rng(7)
    n = 32768
    base = rng.standard_normal(n).astype(np.float32) * 5
    cases = {}
    a = base.copy(); a[[3, 900, 20000]] = np.nan; cases["nan"] = a
    a = base.copy(); a[:] = np.nan; cases["all_nan"] = a
    a = base.copy(); a[12345] = np.inf; cases["posinf"] = a
    a = base.copy(); a[12345] = np.inf; a[77] = 150.0; cases["posinf_below_finite"] = a
    a = base.copy(); a[500] = np.inf; a[40] = 100.0; cases["posinf_ties_100"] = a
    a = base.copy(); a[9] = np.inf; a[10] = np.inf; cases["two_posinf"] = a
    a = base.copy(); a[:] = -np.inf; a[31000] = -3.0; cases["neginf"] = a
    a = base.copy(); a[:] = -np.inf; cases["all_neginf"] = a
    a = np.zeros(n, np.float32); cases["all_equal"] = a
    a = base.copy(); m = a.max() + 1; a[[25000, 7000, 7001, 31999]] = m; cases["ties_first_index"] = a
    a = base.copy(); a[0] = a.max() + 2; a[n - 1] = a[0]; cases["ties_ends"] = a
    a = base.copy(); a[5] = np.nan; a[6] = -1e4; a[:] = -1e5; a[5] = np.nan; cases["nan_is_minus_1e4"] = a
    cases["n1"] = np.array([-2.5], np.float32)
    a = rng.standard_normal(1000).astype(np.float32); a[999] = 40; cases["n1000"] = a
    a = rng.standard_normal(100003).astype(np.float32); a[70001] = 9; a[100002] = 9; cases["n100003_two_rounds"] = a
    return cases


@pytest.mark.parametrize("split", [False, True], ids=["one_block", "split"])
@pytest.mark.parametrize("name", sorted(_argmax_cases()))
def test_greedy_argmax_special_values(lib, name, split):
    """The device greedy step against gsd_lq_cpu_runtime.py:422-425:
    nan_to_num(nan=-1e4, posinf=100, neginf=-1e4), then the first index of
    the maximum; the margin is top1 - top2 of the cleaned values.  split: the
    32-block form of the model's decode graph, called twice on one workspace
    (the second call's hand-off words carry the next tag); a case's ties and
    special values then fall in different blocks (1024 entries each at 32768)."""
    lg = _argmax_cases()[name]
    want = O.OracleModel.greedy(lg)
    clean = np.nan_to_num(lg, nan=-1e4, posinf=100.0, neginf=-1e4)
    srt = np.sort(clean)
    want_margin = np.float32(srt[-1] - (srt[-2] if clean.size > 1 else -np.inf))
    d = D(lg)
    if not split:
        tok, mg = E(4), E(4)
        lib.gsdh_greedy_argmax(None, p(d), lg.size, p(tok), p(mg))
        assert int(H(tok, np.int32, 1)[0]) == want, name
        assert H(mg, np.float32, 1)[0] == want_margin, name
        return
    words, ctr = D(np.zeros(96, np.uint64)), D(np.zeros(32, np.uint32))
    for call in range(2):
        tok, mg = D(np.full(1, -7, np.int32)), E(4)
        assert lib.gsdh_greedy_argmax_split(None, p(d), lg.size, p(tok), p(mg), p(words), p(ctr)) == 0
        assert int(H(tok, np.int32, 1)[0]) == want, (name, call)
        assert H(mg, np.float32, 1)[0] == want_margin, (name, call)
    assert np.all(H(ctr, np.uint32) == 2), name
