"""End-to-end parity of the drop-in model on the GPU against the oracle:
per-token logits within 1e-3 relative L2 and identical greedy tokens, on
small synthetic models (every step checked) and on the 32-layer
Mistral-7B-shaped Precision model (128 greedy steps, golden sequence written
by the reference engine)."""
import json
import sys
import os

import numpy as np
import pytest

import oracle as O
from conftest import GOLDEN, rel_l2
from gpu_util import banner

pytestmark = pytest.mark.gpu


def _spec(**kw):
    from gsdlq import synth
    base = dict(n_layers=2, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=512,
                mode="precision", kinks_per_row=2)
    base.update(kw)
    return synth.SynthSpec(**base)


def _models(spec, max_seq=256, interleaved=1):
    from gsdlq import synth
    import run_gpu_native_chat as chat
    src = synth.SynthSource(spec)
    gpu = chat.GPUMistralV2Model(src, rope_interleaved=interleaved, max_seq_len=max_seq, verbose=False)
    ref = O.OracleModel(src, kind="port", max_seq_len=max_seq, rope_interleaved=interleaved)
    return gpu, ref


def test_tiny_model_golden(golden):
    banner("tiny model vs reference-engine golden")
    gpu, _ = _models(_spec())
    prompt = golden["tiny_prompt"].tolist()
    for pos, t in enumerate(prompt):
        lg = gpu.forward_token(t, pos)
        assert rel_l2(lg, golden["tiny_logits"][pos]) < 1e-3
    toks = []
    pos = len(prompt)
    for _ in range(8):
        nxt = gpu.sample_token(lg, temperature=0.0)
        toks.append(nxt)
        lg = gpu.forward_token(nxt, pos)
        pos += 1
    assert toks == golden["tiny_tokens"].tolist()
    gpu.close()


@pytest.mark.parametrize("mode,kpr,il,shape", [
    ("turbo", 0, 1, dict()),
    ("precision", 3, 1, dict()),
    ("precision", 0, 0, dict(n_heads=8, n_kv_heads=8, head_dim=32 * 2)),
    ("turbo", 1, 1, dict(n_layers=3, hidden=512, ffn=1344, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000)),
])
def test_model_stepwise_vs_oracle(mode, kpr, il, shape):
    banner(f"stepwise model {mode} kinks {kpr} interleaved {il} {shape}")
    gpu, ref = _models(_spec(mode=mode, kinks_per_row=kpr, **shape), interleaved=il)
    rng = np.random.default_rng(3)
    toks = rng.integers(0, gpu.vocab_size, 40).tolist()
    for pos, t in enumerate(toks):
        want_logits = pos % 5 == 4 or pos == len(toks) - 1
        a = gpu.forward_token(t, pos, return_logits=want_logits)
        b = ref.forward_token(t, pos, return_logits=want_logits)
        if want_logits:
            assert rel_l2(a, b) < 1e-3, pos
        else:
            assert a is None
    # rewind: re-running from an earlier position overwrites the cache
    a = gpu.forward_token(toks[10], 10)
    b = ref.forward_token(toks[10], 10)
    assert rel_l2(a, b) < 1e-3
    gpu.close()


CODE_SHAPES = [
    ("precision", dict()),
    ("turbo", dict()),
    # ragged: down has 1344 columns (a half-filled last chunk), lm_head 1000 rows
    ("precision", dict(n_layers=1, hidden=512, ffn=1344, n_heads=8, n_kv_heads=2, head_dim=64, vocab=1000)),
    ("turbo", dict(n_layers=1, codebook_radius=5)),
    ("turbo", dict(n_layers=1, codebook_radius=7)),
]


@pytest.mark.parametrize("mode,shape", CODE_SHAPES)
def test_device_codes_bit_exact(mode, shape):
    """The codes the matvec kernels decode from the device tiles (7 bits per
    code up to radius 6, one byte for radius 7-8) equal the file's u8 codes,
    tensor by tensor."""
    from gsdlq import synth, hip as _hip
    import run_gpu_native_chat as chat
    spec = _spec(mode=mode, kinks_per_row=1, **shape)
    banner(f"device codes bit-exact {mode} {shape}")
    src = synth.SynthSource(spec)
    gpu = chat.GPUMistralV2Model(src, max_seq_len=64, verbose=False)
    names = [(f"blk.{l}.{t}.weight", l, _hip.SLOTS[t]) for l in range(spec.n_layers)
             for t in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")]
    names.append(("output.weight", 0, _hip.SLOTS["output"]))
    for name, layer, slot in names:
        want = np.ascontiguousarray(src.hex_field(name, "codes"), dtype=np.uint8)
        got = np.full(want.shape, 0xFF, dtype=np.uint8)
        gpu.cl.lib.gsdh_model_read_codes(gpu._m, layer, slot, _hip.ptr(got))
        assert np.array_equal(got, want), name
    gpu.close()


@pytest.mark.parametrize("radius", [5, 7])
def test_model_generic_codebook_vs_oracle(radius):
    """Codebooks other than radius 6 / 8 run the generic-codebook matvec
    (7-bit tiles at radius 5, u8 tiles at radius 7), ."""
    banner(f"stepwise model radius {radius}")
    gpu, ref = _models(_spec(mode="precision", kinks_per_row=2, codebook_radius=radius))
    rng = np.random.default_rng(30 + radius)
    toks = rng.integers(0, gpu.vocab_size, 10).tolist()
    for pos, t in enumerate(toks):
        a = gpu.forward_token(t, pos)
        b = ref.forward_token(t, pos)
        assert rel_l2(a, b) < 1e-3, pos
    gpu.close()


@pytest.mark.parametrize("k_dim", [1, 3])
def test_model_rank_sizes_vs_oracle(k_dim):
    """Rank 1 runs the matvec's in-block projection with one row per tensor;
    rank 3 the launches whose projections leading blocks publish ."""
    banner(f"stepwise model precision rank {k_dim}")
    gpu, ref = _models(_spec(mode="precision", kinks_per_row=1, k_dim=k_dim))
    rng = np.random.default_rng(11 + k_dim)
    toks = rng.integers(0, gpu.vocab_size, 12).tolist()
    for pos, t in enumerate(toks):
        a = gpu.forward_token(t, pos)
        b = ref.forward_token(t, pos)
        assert rel_l2(a, b) < 1e-3, pos
    gpu.close()


@pytest.mark.parametrize("mode", ["turbo", "precision"])
@pytest.mark.parametrize("shape", [
    # gate/up: 272 units of 16 rows on 256 blocks (16 blocks with two units)
    dict(hidden=2048, ffn=4352, n_heads=16, n_kv_heads=4, head_dim=128),
    # q/k/v: 384 units, gate/up 288 units (7B hidden size, one layer)
    dict(hidden=4096, ffn=4608, n_heads=32, n_kv_heads=8, head_dim=128),
])
def test_model_uneven_units_vs_oracle(mode, shape):
    """Launches with more row-block units than blocks, not a multiple of them
    (blocks with one unit more than others), ."""
    banner(f"stepwise model {mode} {shape} uneven units")
    gpu, ref = _models(_spec(mode=mode, kinks_per_row=2, n_layers=1, vocab=1000, **shape), max_seq=64)
    rng = np.random.default_rng(41)
    toks = rng.integers(0, gpu.vocab_size, 8).tolist()
    for pos, t in enumerate(toks):
        a = gpu.forward_token(t, pos)
        b = ref.forward_token(t, pos)
        assert rel_l2(a, b) < 1e-3, pos
    # the same token twice: same bits
    assert np.array_equal(gpu.forward_token(toks[3], 3), gpu.forward_token(toks[3], 3))
    gpu.close()


def test_generate_greedy_matches_oracle():
    banner("generate_greedy vs oracle")
    gpu, ref = _models(_spec(mode="turbo", kinks_per_row=1))
    prompt = [1, 5, 9, 200, 33, 2]
    toks, margins = gpu.generate_greedy(prompt, 24)
    want, wm = ref.generate_greedy(prompt, 24)
    assert toks == want
    assert np.allclose(margins, wm, rtol=1e-2, atol=1e-4)
    # forward_token after generate keeps working and agrees
    a = gpu.forward_token(toks[0], len(prompt))
    b = ref.forward_token(toks[0], len(prompt))
    assert rel_l2(a, b) < 1e-3
    gpu.close()


def test_decode_across_short_context_switch():
    """Below 256 positions attention is one split (one block per KV head and
    no merge), later ones are split and merged: decoding through the switch
    matches the oracle token for token, and forward_token agrees on both
    sides of it."""
    banner("greedy decode across position 256")
    gpu, ref = _models(_spec(mode="precision", kinks_per_row=1), max_seq=512)
    rng = np.random.default_rng(20)     # smallest oracle margin 6e-3 over the 48 steps
    prompt = rng.integers(0, gpu.vocab_size, 230).tolist()
    toks, margins = gpu.generate_greedy(prompt, 48)
    want, wm = ref.generate_greedy(prompt, 48)
    assert toks == want
    assert np.allclose(margins, wm, rtol=1e-2, atol=1e-4)
    # rewrite positions 255 and 256, then the last generated token's position
    # (the oracle's loop has already run it, the engine's need not) and 278
    for pos in (255, 256, len(prompt) + 47, len(prompt) + 48):
        a = gpu.forward_token(toks[0], pos)
        b = ref.forward_token(toks[0], pos)
        assert rel_l2(a, b) < 1e-3, pos
    gpu.close()


@pytest.mark.parametrize("mode,shape", [
    ("precision", dict(kinks_per_row=2)),                                            # head dim 64, 2 heads per KV head
    ("turbo", dict(n_layers=1, hidden=1024, ffn=1024, n_heads=8, n_kv_heads=2, head_dim=128)),   # 128, 4
])
def test_fused_attention_matches_two_launches(mode, shape, monkeypatch):
    """Positions below 256 run the attention inside the q/k/v launch (its
    last blocks wait for the q/k/v words of the same launch); with
    GSD_FUSED_ATTN=0 the model issues the q/k/v launch and the attention
    launch instead.  Both match the oracle at every position up to 300 (the
    fused path through 255, the split path after), and each other closely."""
    banner(f"fused q/k/v + attention vs two launches {mode} {shape}")
    from gsdlq import synth
    import run_gpu_native_chat as chat
    src = synth.SynthSource(_spec(mode=mode, **shape))
    models = []
    for fa in ("1", "0"):
        monkeypatch.setenv("GSD_FUSED_ATTN", fa)
        models.append(chat.GPUMistralV2Model(src, max_seq_len=512, verbose=False))
    fused, plain = models
    ref = O.OracleModel(src, kind="port", max_seq_len=512)
    toks = np.random.default_rng(7).integers(0, fused.vocab_size, 300).tolist()
    for pos, t in enumerate(toks):
        want = pos % 7 == 0 or pos in (63, 64, 127, 128, 255, 256, 299)
        a = fused.forward_token(t, pos, return_logits=want)
        b = plain.forward_token(t, pos, return_logits=want)
        r = ref.forward_token(t, pos, return_logits=want)
        if want:
            assert rel_l2(a, r) < 1e-3, pos
            assert rel_l2(b, r) < 1e-3, pos
            assert rel_l2(a, b) < 1e-4, pos
    for m in models:
        m.close()


@pytest.mark.parametrize("mode,shape", [
    ("precision", dict(kinks_per_row=2)),                                     # 2 chunks of x, 8 FFN blocks
    ("turbo", dict(n_layers=3, hidden=512, ffn=1344, n_heads=8, n_kv_heads=2, head_dim=128, vocab=1000,
                   kinks_per_row=1)),                                         # 21 FFN blocks, 32 slices
    ("precision", dict(codebook_radius=5, kinks_per_row=1)),                  # 91-point codebook, 7-bit tiles
])
def test_fused_ffn_matches_two_launches(mode, shape, monkeypatch):
    """Every decode token runs o, gate/up and down as one launch where it
    covers the model (2), or gate/up + down as one (1); with GSD_FUSED_FFN=0
    the model issues the o, gate/up and down launches.  All match the oracle
    at every checked position, and each other closely; greedy tokens are
    equal."""
    banner(f"fused FFN vs separate launches {mode} {shape}")
    from gsdlq import synth
    import run_gpu_native_chat as chat
    src = synth.SynthSource(_spec(mode=mode, **shape))
    models = []
    for ff, of in (("1", "1"), ("1", "0"), ("0", "1")):
        monkeypatch.setenv("GSD_FUSED_FFN", ff)
        monkeypatch.setenv("GSD_FUSED_OFFN", of)
        models.append(chat.GPUMistralV2Model(src, max_seq_len=128, verbose=False))
    kinds = [m.cl.lib.gsdh_model_fused_ffn(m._m, 0) for m in models]
    square = src.config["n_heads"] * src.config["head_dim"] == src.config["hidden_size"]
    assert kinds == [2 if square else 1, 1, 0], kinds
    ref = O.OracleModel(src, kind="port", max_seq_len=128)
    toks = np.random.default_rng(8).integers(0, models[0].vocab_size, 40).tolist()
    for pos, t in enumerate(toks):
        want = pos % 5 == 0 or pos == len(toks) - 1
        outs = [m.forward_token(t, pos, return_logits=want) for m in models]
        r = ref.forward_token(t, pos, return_logits=want)
        if want:
            for o in outs:
                assert rel_l2(o, r) < 1e-3, pos
                assert rel_l2(o, outs[-1]) < 1e-4, pos
    tr, _ = ref.generate_greedy(toks[:5], 12)
    for m in models:
        assert m.generate_greedy(toks[:5], 12)[0] == tr
    for m in models:
        m.close()


def test_model_rejects_invalid_codes():
    from gsdlq import synth
    import run_gpu_native_chat as chat

    class Bad(synth.SynthSource):
        def hex_field(self, name, field):
            a = super().hex_field(name, field)
            if field == "codes" and name == "blk.1.ffn_up.weight":
                a = a.copy()
                a[5] = 200   # >= 127 points of radius 6
            return a

    with pytest.raises(ValueError, match="n_pts"):
        chat.GPUMistralV2Model(Bad(_spec()), max_seq_len=32, verbose=False)


def test_forward_token_bounds():
    from gsdlq.hip import HipError
    gpu, _ = _models(_spec(), max_seq=16)
    with pytest.raises(HipError, match="pos"):
        gpu.forward_token(1, 16)
    with pytest.raises(HipError, match="vocab"):
        gpu.forward_token(512, 0)
    gpu.close()


GREEDY_7B = os.path.join(GOLDEN, "greedy_7b_precision.json")


@pytest.mark.slow
@pytest.mark.skipif(not os.path.exists(GREEDY_7B), reason="7B golden sequence not generated")
def test_greedy_7b_precision_128_steps():
    """Mistral-7B-shaped, 32 layers, Precision (radius 6, rank 2): 64-token
    seeded prompt (batched prefill) then 128 greedy steps must equal the
    reference engine's."""
    from gsdlq import synth
    import run_gpu_native_chat as chat
    g = json.load(open(GREEDY_7B))
    spec = synth.SynthSpec(mode="precision")
    for k, v in g["spec"].items():
        if k != "rank":
            assert getattr(spec, k) == v, k
    banner("packing the synthetic 7B model (one tensor at a time) ...")
    gpu = chat.GPUMistralV2Model(synth.SynthSource(spec), max_seq_len=256, verbose=True)
    banner("greedy decode 64 + 128")
    toks, margins = gpu.generate_greedy(g["prompt"], len(g["tokens"]))
    first_diff = next((i for i, (a, b) in enumerate(zip(toks, g["tokens"])) if a != b), None)
    if first_diff is not None:
        print(f"first mismatch at step {first_diff}: gpu {toks[first_diff]} ref {g['tokens'][first_diff]} "
              f"ref margin {g['margins'][first_diff]:.3e} gpu margin {margins[first_diff]:.3e}", flush=True)
    assert toks == g["tokens"]
    # top-5 logits of the first step against the reference's values: from
    # the batched prefill of the whole prompt and from one decode step
    top = g["top5"][0]
    for lg in (gpu.prefill(g["prompt"], 0), gpu.forward_token(g["prompt"][-1], len(g["prompt"]) - 1)):
        for i, v in top:
            assert abs(lg[i] - v) <= 1e-3 * max(1.0, abs(v))
    gpu.close()


def test_7b_shape_decode_past_256():
    """The split decode attention inside the model's token graph at the 7B
    head shape (32 / 8 heads of 128; positions from 256 on leave the fused
    short-context launch): a 2-layer Mistral-7B-shaped Precision model takes
    a 270-token prompt through the batched prefill, then decodes positions
    270-273, each against the oracle's forward (logits within 1e-3)."""
    from gsdlq import synth
    import run_gpu_native_chat as chat
    banner("7B-shaped 2-layer model: prefill 270, decode 270-273 (split attention)")
    src = synth.SynthSource(synth.SynthSpec(n_layers=2, mode="precision"))
    gpu = chat.GPUMistralV2Model(src, max_seq_len=512, verbose=False)
    ref = O.OracleModel(src, kind="port", max_seq_len=512)
    toks = np.random.default_rng(270).integers(0, gpu.vocab_size, 274).tolist()
    got = gpu.prefill(toks[:270], 0)
    want = None
    for pos in range(270):
        want = ref.forward_token(toks[pos], pos, return_logits=pos == 269)
    e = rel_l2(got, want)
    print(f"[model-parity] 7B-shaped prefill 270: rel L2 {e:.2e}", flush=True)
    assert e < 1e-3
    for pos in range(270, 274):
        a, b = gpu.forward_token(toks[pos], pos), ref.forward_token(toks[pos], pos)
        e = rel_l2(a, b)
        print(f"[model-parity] 7B-shaped decode position {pos}: rel L2 {e:.2e}", flush=True)
        assert e < 1e-3, pos
    gpu.close()


_LONG = {}


def _long_oracle():
    """Oracle greedy run through positions 0 .. 4113 of an 8192-position model
    (computed once)."""
    if not _LONG:
        from gsdlq import synth
        spec = _spec(mode="precision", kinks_per_row=1, n_layers=1)
        ref = O.OracleModel(synth.SynthSource(spec), kind="port", max_seq_len=8192)
        rng = np.random.default_rng(LONG_SEED)
        prompt = rng.integers(0, spec.vocab, 4090).tolist()
        toks, margins = ref.generate_greedy(prompt, 24)
        rewrites = {}
        for pos in (2047, 2048, 4095, 4096, 4113):
            rewrites[pos] = ref.forward_token(toks[0], pos)
        _LONG.update(spec=spec, prompt=prompt, toks=toks, margins=margins, rewrites=rewrites)
    return _LONG


LONG_SEED = 5


def test_decode_past_2048_to_4096():
    """A model with an 8192-position cache decodes through positions 2048
    (the reference's fixed cache size) and 4096: 4090 prompt tokens, then 24
    greedy steps equal to the oracle's (heap score buffer), and forward_token
    on both sides of each boundary within 1e-3."""
    from gsdlq import synth
    import run_gpu_native_chat as chat
    L = _long_oracle()
    banner("decode to position 4113 of an 8192-position cache")
    gpu = chat.GPUMistralV2Model(synth.SynthSource(L["spec"]), max_seq_len=8192, verbose=False)
    toks, margins = gpu.generate_greedy(L["prompt"], 24)
    assert toks == L["toks"]
    assert np.allclose(margins, L["margins"], rtol=1e-2, atol=1e-4)
    for pos, want in L["rewrites"].items():
        assert rel_l2(gpu.forward_token(L["toks"][0], pos), want) < 1e-3, pos
    gpu.close()


def test_gsd2_file_through_drop_in(tmp_path, monkeypatch, capsys):
    """The drop-in's file path: a written .gsd2 (Precision, kinks) loaded by
    GPUMistralV2Model(path) against the oracle reading the same file with its
    own reader (FileSource), the smoke command main([path, '--smoke']) and two
    chat turns of main([path]) over stdin (the second reusing the first's KV
    prefix, run_gpu_native_chat.py:1112-1131)."""
    import io
    from gsdlq import synth
    import run_gpu_native_chat as chat
    spec = _spec(mode="precision", kinks_per_row=2, n_layers=2)
    path = str(tmp_path / "tiny.gsd2")
    synth.write_gsd2(spec, path)
    banner(f"drop-in from {os.path.basename(path)}")
    gpu = chat.GPUMistralV2Model(path, rope_interleaved=1, verbose=False)
    ref = O.OracleModel(O.FileSource(path), kind="port", max_seq_len=gpu.max_seq_len)
    assert gpu.n_layers == 2 and gpu.vocab_size == spec.vocab
    toks = np.random.default_rng(12).integers(0, gpu.vocab_size, 12).tolist()
    for pos, t in enumerate(toks):
        assert rel_l2(gpu.forward_token(t, pos), ref.forward_token(t, pos)) < 1e-3, pos
    # the smoke verify's greedy text equals the oracle's greedy continuation
    ids = gpu.tokenizer.encode("The capital of France is", add_bos=True)
    want_ids, _ = ref.generate_greedy(ids, 8)
    eos = gpu.tokenizer.eos_id
    want_ids = want_ids[:want_ids.index(eos)] if eos in want_ids else want_ids
    got = chat.run_smoke_verify(gpu)
    assert got == gpu.tokenizer.decode(want_ids)
    gpu.close()
    capsys.readouterr()
    chat.main([path, "--smoke"])
    assert "[SMOKE TEST]" in capsys.readouterr().out
    # two chat turns, then quit; turns are logged
    log = tmp_path / "chat_log.md"
    monkeypatch.setattr(chat, "LOG_FILE", str(log))
    monkeypatch.setattr(sys, "stdin", io.StringIO("Hello there\nAnd again\nquit\n"))
    chat.main([path])
    out = capsys.readouterr().out
    assert out.count("[GPU Stats: Prefill") == 2
    text = log.read_text(encoding="utf-8")
    assert "### Turn 1" in text and "### Turn 2" in text


def test_gsd2_7bit_file_same_results(tmp_path):
    """The compact Precision file (7-bit code streams) loads into the same
    device tiles as the u8 file: identical logits, bit for bit."""
    from gsdlq import synth
    import run_gpu_native_chat as chat
    spec = _spec(mode="precision", kinks_per_row=1, n_layers=2)
    p8, p7 = str(tmp_path / "m8.gsd2"), str(tmp_path / "m7.gsd2")
    synth.write_gsd2(spec, p8)
    synth.write_gsd2(spec, p7, code_bits=7)
    banner("7-bit .gsd2 vs u8 .gsd2")
    a = chat.GPUMistralV2Model(p8, verbose=False)
    b = chat.GPUMistralV2Model(p7, verbose=False)
    assert b.avg_bpw < a.avg_bpw - 0.4
    for pos, t in enumerate([1, 50, 7, 299, 3]):
        assert np.array_equal(a.forward_token(t, pos), b.forward_token(t, pos)), pos
    a.close()
    b.close()
