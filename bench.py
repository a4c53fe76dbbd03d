"""Benchmark of the GSD-LQ batch-1 decode path on one MI355X.

Workload (the metric's configuration): the full Mistral-7B linear set of one
layer -- q 4096x4096, k/v 1024x4096, o 4096x4096, gate/up 14336x4096,
down 4096x14336 -- packed in Turbo mode (radius 8, ~4.26 bpw), batch 1, fp32
activations.  A step is one pass of the layer's fused unpack-matvec launches
(qkv with fused RMSNorm; one launch for o + residual, RMSNorm, gate/up,
SwiGLU, down split over the FFN rows and residual).  Steps rotate over
`--layers` distinct packed layers
(> 256 MB) so the Infinity Cache cannot serve the weights, and are timed with
HIP events around a captured HIP graph on the engine's stream.

value = algorithmic bytes per step / time per step (GB/s), bytes of the
streams a matvec must read or write once: codes in the device format (one
byte each for radius 8, seven bits for radius <= 6) + fp16 scales + row_ptr +
6 B per kink + low-rank factors + x (4 B/col) + y (4 B/row).

Also reported: the same for Precision mode (radius 6: 7-bit codes, rank 2),
the dominant kernel's roofline (the fused o + FFN launch: 4096x4096 +
2 x 14336x4096 + 4096x14336 of weights, attn and x in, x out), decode attention with RoPE + K/V append at contexts 512 / 2048 /
8192 (GB/s of K/V cache read), end-to-end greedy decode tok/s of a 32-layer
7B-shaped model, and the reference CPU engine timed on this host's cores on a
bounded sample.

    python bench.py [--gpus 1] [--steps 100] [--warmup 3]
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gsd-lq_amd"))

HBM_PEAK_GBS = 8000.0
H, F, KV, V = 4096, 14336, 1024, 32768


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def layer_shapes():
    return {"attn_q": (H, H), "attn_k": (KV, H), "attn_v": (KV, H), "attn_output": (H, H),
            "ffn_gate": (F, H), "ffn_up": (F, H), "ffn_down": (H, F)}


def code_bytes(f):
    """Bytes of a tensor's codes in the device format: 7 bits per code for
    codebooks of at most 128 points (radius <= 6), one byte otherwise."""
    n = f["codes"].size
    return (7 * n + 7) // 8 if f["radius"] <= 6 else n


def weight_bytes(f):
    """Bytes of packed tensor f a matvec streams: codes in the device format,
    scales, row_ptr, kinks, low-rank factors."""
    rows, cols, k = f["rows"], f["cols"], f["k_dim"]
    b = code_bytes(f) + f["scales"].nbytes + f["row_ptr"].nbytes + 6 * f["nk"]
    if k:
        b += 2 * rows * k + 2 * k * cols + 4 * k
    return b


def alg_bytes(f):
    """Algorithmic bytes of one fused matvec over packed tensor f (weights +
    x read + y written)."""
    return weight_bytes(f) + 4 * f["cols"] + 4 * f["rows"]


def ffn_bytes(bank, l, with_o=True):
    """Algorithmic bytes of the fused o + FFN launch of layer l: the o, gate,
    up and down weights, attn read, x read once and x written (x + W_o attn
    and h stay inside the launch); with_o=False: the FFN launch alone."""
    b = sum(weight_bytes(bank.packed[(l, t)]) for t in ("ffn_gate", "ffn_up", "ffn_down")) + 8 * H
    return b + (weight_bytes(bank.packed[(l, "attn_output")]) + 4 * H if with_o else 0)


class LayerBank:
    """Distinct packed 7B layers (each tensor packed from its own seed) plus
    an lm_head; a `copies` option repeats the distinct layers to fill a
    32-layer model for the end-to-end decode timing."""

    def __init__(self, mode: str, n_distinct: int):
        from gsdlq import synth
        self.spec = synth.SynthSpec(n_layers=n_distinct, mode=mode)
        self.mode = mode
        self.n = n_distinct
        self.packed = {}
        t0 = time.time()
        for l in range(n_distinct):
            for t in layer_shapes():
                self.packed[(l, t)] = synth.pack_synth(self.spec, f"blk.{l}.{t}.weight")
            log(f"{mode}: packed layer {l + 1}/{n_distinct} ({time.time() - t0:.0f}s)")
        self.packed["lm"] = synth.pack_synth(self.spec, "output.weight")
        self.layer_bytes = [sum(alg_bytes(self.packed[(l, t)]) for t in layer_shapes()) for l in range(n_distinct)]


class BankSource:
    """Gsd2File-like source serving LayerBank tensors, layer l -> bank l % n."""

    def __init__(self, bank: LayerBank, n_layers: int):
        from gsdlq import synth
        spec = synth.SynthSpec(n_layers=n_layers, mode=bank.mode)
        self.src = synth.SynthSource(spec)
        self.config = self.src.config
        self.tensors = self.src.tensors
        self.bank = bank
        self.header = {"avg_bpw": None}

    def dense(self, name, dtype):
        return self.src.dense(name, dtype)

    def hex_field(self, name, field):
        if name == "output.weight":
            return self.bank.packed["lm"][field]
        parts = name.split(".")
        return self.bank.packed[(int(parts[1]) % self.bank.n, parts[2])][field]


def build_model(bank, n_layers, max_seq=256):
    import run_gpu_native_chat as chat
    return chat.GPUMistralV2Model(BankSource(bank, n_layers), max_seq_len=max_seq, verbose=False)


def capture(model, fn):
    lib = model.cl.lib
    lib.gsdh_model_capture_begin(model._m)
    try:
        fn()
    finally:
        ge = ctypes.c_void_p()
        lib.gsdh_model_capture_end(model._m, ctypes.byref(ge))
    return ge


def time_graph(model, ge, n):
    ms = ctypes.c_float()
    model.cl.lib.gsdh_graph_time(model._m, ge, n, ctypes.byref(ms))
    return ms.value


def bench_linear(bank, steps, warmup):
    """GB/s of the layer linear set; returns (gbs, ms_per_step, roofline dict).
    Step i runs the four launches of distinct layer i % layers; the warm-up
    steps and the timed steps are each one captured graph, so exactly
    `steps` steps lie between the two timing events."""
    model = build_model(bank, bank.n)
    lib = model.cl.lib
    model.forward_token(1, 0)   # realistic activations in every buffer
    L = bank.n
    if warmup > 0:
        gw = capture(model, lambda: [lib.gsdh_model_run_linear(model._m, i % L, 15) for i in range(warmup)])
        time_graph(model, gw, 1)
        lib.gsdh_graph_destroy(gw)
    ge = capture(model, lambda: [lib.gsdh_model_run_linear(model._m, i % L, 15) for i in range(steps)])
    ms = time_graph(model, ge, 1)
    ms_step = ms / steps
    gbs = sum(bank.layer_bytes[i % L] for i in range(steps)) / (ms * 1e-3) / 1e9
    # dominant kernel: the fused o + FFN launch (o 4096 x 4096 + residual,
    # RMSNorm, gate/up 2 x 14336 x 4096, SwiGLU, down 4096 x 14336 +
    # residual), timed alone over 128 launches rotating the distinct layers
    ng = 128
    assert lib.gsdh_model_fused_ffn(model._m, 0) == 2, "the fused o + FFN launch does not cover this model"
    gu = capture(model, lambda: [lib.gsdh_model_run_linear(model._m, i % L, 14) for i in range(ng)])
    time_graph(model, gu, 1)
    gms = time_graph(model, gu, 1)
    per_launch_ms = gms / ng
    fb = sum(ffn_bytes(bank, i % L) for i in range(ng)) / ng
    ach = fb / (per_launch_ms * 1e-3) / 1e9
    roof = {"kernel": "ffn_kernel (MFMA fused o + residual, RMSNorm + gate/up + SwiGLU + split-K down + "
                      "residual: 4096x4096 + 2x14336x4096 + 4096x14336)",
            "bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(),
            "launch_us": round(per_launch_ms * 1e3, 2), "alg_bytes_per_launch": int(fb),
            "launches_timed": ng}
    for g in (ge, gu):
        lib.gsdh_graph_destroy(g)
    model.close()
    return gbs, ms_step, roof


class C1Source(BankSource):
    """A Turbo model whose 4096x4096 o projections are all distinct (seeded
    per layer), the other tensors the bank's: C1's matvec rotated over more
    weights than the Infinity Cache holds."""

    def __init__(self, bank, n_layers):
        from gsdlq import synth
        super().__init__(bank, n_layers)
        self.o = [synth.pack_synth(synth.SynthSpec(n_layers=n_layers, mode="turbo"), f"blk.{l}.attn_output.weight")
                  for l in range(n_layers)]

    def hex_field(self, name, field):
        parts = name.split(".")
        if name != "output.weight" and parts[2] == "attn_output":
            return self.o[int(parts[1])][field]
        return super().hex_field(name, field)


def bench_c1(bank, n=48, reps=4):
    """C1: one fused unpack-matvec of a 4096x4096 Turbo tensor (the o
    projection launch: x += W attn), over n distinct tensors (n x 9 MB beyond
    the 256 MB Infinity Cache), graph-captured back to back."""
    import run_gpu_native_chat as chat
    src = C1Source(bank, n)
    model = chat.GPUMistralV2Model(src, max_seq_len=16, verbose=False)
    lib = model.cl.lib
    model.forward_token(1, 0)
    ge = capture(model, lambda: [lib.gsdh_model_run_linear(model._m, l, 2) for l in range(n)])
    time_graph(model, ge, 1)
    ms = time_graph(model, ge, reps)
    lib.gsdh_graph_destroy(ge)
    us = ms * 1e3 / (reps * n)
    b = sum(alg_bytes(f) for f in src.o) / n
    model.close()
    gbs = b / (us * 1e-6) / 1e9
    return {"us_per_matvec": round(us, 3), "alg_bytes": int(b), "GBs": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "distinct_tensors": n,
            "workload": "4096x4096 Turbo (R=8) fused unpack-matvec + residual (o launch), batch 1"}


MFMA_F16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 / bf16 matrix peak


def bench_prefill(bank, ms=(16, 128, 512), reps=3):
    """Batched projection (prefill) over the bank's Turbo layer sets: for each
    M, the 7 tensors of every distinct layer (q/k/v and gate/up each sharing
    one operand prep of their common input: gsdh_model_matmul_shared; o and
    down alone), graph-captured; FLOPs = 2*M*rows*cols, bytes = packed
    weights + bf16 X + fp32 Y.  Roofline: MFMA (fp16 dense peak) for M >=
    128, HBM for M = 16."""
    model = build_model(bank, bank.n)
    lib = model.cl.lib
    shapes = [(t, bank.packed[(0, t)]["rows"], bank.packed[(0, t)]["cols"]) for t in layer_shapes()]
    slot = {"attn_q": 0, "attn_k": 1, "attn_v": 2, "attn_output": 3, "ffn_gate": 4, "ffn_up": 5, "ffn_down": 6}
    mmax, cmax = max(ms), max(c for _, _, c in shapes)
    rmax = max(r for _, r, _ in shapes)
    x = ctypes.c_void_p()
    y = ctypes.c_void_p()
    lib.gsdh_malloc(ctypes.byref(x), mmax * cmax * 2)
    lib.gsdh_malloc(ctypes.byref(y), mmax * rmax * 4)
    rng = np.random.default_rng(5)
    xb = (rng.standard_normal(mmax * cmax).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    lib.gsdh_memcpy_h2d(x, xb.ctypes.data_as(ctypes.c_void_p), xb.nbytes, None)
    lib.gsdh_stream_sync(None)
    out = {}
    flops_layer = sum(2 * r * c for _, r, c in shapes)
    wbytes_layer = bank.layer_bytes[0]
    groups = [("attn_q", "attn_k", "attn_v"), ("attn_output",), ("ffn_gate", "ffn_up"), ("ffn_down",)]
    garg = [((ctypes.c_int * len(g))(*[slot[t] for t in g]), (ctypes.c_void_p * len(g))(*[y] * len(g))) for g in groups]
    for M in ms:
        issue = lambda: [lib.gsdh_model_matmul_shared(model._m, l, sl, len(sl), x, M, ys)
                         for l in range(bank.n) for sl, ys in garg]
        issue()                                   # workspace for this M, outside the capture
        lib.gsdh_stream_sync(lib.gsdh_model_stream(model._m))
        ge = capture(model, issue)
        time_graph(model, ge, 1)
        ms_total = time_graph(model, ge, reps)
        lib.gsdh_graph_destroy(ge)
        us_layer = ms_total * 1e3 / (reps * bank.n)
        tflops = M * flops_layer / (us_layer * 1e-6) / 1e12
        nbytes = wbytes_layer + sum(2 * M * c + 4 * M * r for _, r, c in shapes)
        gbs = nbytes / (us_layer * 1e-6) / 1e9
        bound = "mfma" if M >= 128 else "hbm"
        out[f"M{M}"] = {"us_per_layer": round(us_layer, 2), "tflops": round(tflops, 2), "GBs": round(gbs, 1),
                        "tokens_per_s_per_layer": round(M / (us_layer * 1e-6), 1), "bound": bound,
                        "frac": round(tflops / MFMA_F16_PEAK_TFLOPS if bound == "mfma" else gbs / HBM_PEAK_GBS, 4)}
        log(f"prefill M={M}: {us_layer:.1f} us/layer, {tflops:.1f} TFLOP/s, {gbs:.0f} GB/s")
    lib.gsdh_free(x)
    lib.gsdh_free(y)
    model.close()
    return out


def bench_decode(bank, n_prompt=64, n_new=128, long_prompt=1024):
    """Greedy decode tok/s of a 32-layer 7B-shaped model (layers are copies of
    the bank's distinct layers, each copy its own HBM allocation): one HIP
    graph of per-phase launches per token; weight_GBs = packed weight bytes
    streamed per token x tok/s.  Then the 64-token prompt alone (batched
    prefill and one decode step per token) and a `long_prompt`-token prompt
    through the batched prefill (chunks of 512 tokens)."""
    model = build_model(bank, 32, max_seq=max(n_prompt + n_new, long_prompt) + 8)
    prompt = np.random.default_rng(4).integers(0, V, n_prompt).tolist()
    wbytes = 32 * bank.layer_bytes[0] + alg_bytes(bank.packed["lm"])
    out = {"n_prompt": n_prompt, "n_new": n_new, "weight_bytes_per_token": wbytes}
    model.generate_greedy(prompt[:8], 4)   # warm
    t0 = time.time()
    model.generate_greedy(prompt, n_new)
    total = time.time() - t0
    # decode-only rate: n_new steps after a 1-token prefill
    t0 = time.time()
    model.generate_greedy(prompt[:1], n_new)
    dec = time.time() - t0
    out["decode_tok_s"] = round(n_new / dec, 1)
    out["weight_GBs"] = round(wbytes * n_new / dec / 1e9, 1)
    out["frac_hbm"] = round(wbytes * n_new / dec / 1e9 / HBM_PEAK_GBS, 4)
    out["prompt_plus_decode_s"] = round(total, 3)
    # the 64-token prompt alone: batched prefill vs one decode step per token
    for batched, key in ((True, "prefill_batched"), (False, "prefill_token_by_token")):
        model.set_prefill(batched)
        model.prefill(prompt, 0, return_logits=False) if batched else None
        t0 = time.time()
        reps = 5
        for _ in range(reps):
            if batched:
                model.prefill(prompt, 0)
            else:
                for pos, t in enumerate(prompt):
                    model.forward_token(t, pos, return_logits=pos == n_prompt - 1)
        dt = (time.time() - t0) / reps
        out[key + "_ms"] = round(dt * 1e3, 2)
        out[key + "_tok_s"] = round(n_prompt / dt, 1)
    model.set_prefill(True)
    if long_prompt:
        lp = np.random.default_rng(5).integers(0, V, long_prompt).tolist()
        model.prefill(lp, 0, return_logits=False)
        reps = 3
        t0 = time.time()
        for _ in range(reps):
            model.prefill(lp, 0)
        dt = (time.time() - t0) / reps
        out[f"prefill_{long_prompt}_ms"] = round(dt * 1e3, 2)
        out[f"prefill_{long_prompt}_tok_s"] = round(long_prompt / dt, 1)
    model.close()
    return out


def host_cpu():
    """CPU model and core count of this host (reported with every CPU figure)."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"model": model, "nproc": os.cpu_count() or 1,
            "omp_threads": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))}


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    return O, ("reference" if O.have_reference() else "port")


def cpu_baseline(bank, seconds=12.0):
    """The reference CPU engine (built from its source into oracle/_ref; the
    oracle restatement if absent) on one Turbo layer's 7 matvecs, repeated for
    a bounded time on all host cores."""
    O, kind = _oracle()
    x = np.random.default_rng(1).standard_normal(F).astype(np.float32)
    fs = [bank.packed[(0, t)] for t in layer_shapes()]
    for f in fs:   # warm
        O.hex2d_matvec(x[:f["cols"]], f, kind=kind)
    t0 = time.time()
    n = 0
    while time.time() - t0 < seconds:
        for f in fs:
            O.hex2d_matvec(x[:f["cols"]], f, kind=kind)
        n += 1
    dt = time.time() - t0
    cpu = host_cpu()
    return {"value": round(bank.layer_bytes[0] * n / dt / 1e9, 3), "unit": "GB/s",
            "cores": cpu["omp_threads"], "kind": kind, "cpu": cpu["model"], "nproc": cpu["nproc"],
            "sample": f"{n} passes over one Turbo 7B layer's 7 matvecs ({dt:.1f}s), gsd_cpu_hex2d_matvec "
                      f"built with the reference flags (clang -O3 -fopenmp)"}


def cpu_attention(ctxs=(512, 2048, 8192), seconds=2.0):
    """C3 on the CPU: per layer one gsd_cpu_rope_and_store_kv and one
    gsd_cpu_gqa_attention (32 / 8 heads x 128) at pos = ctx - 1, repeated for
    a bounded time.  The reference engine keeps its scores in a fixed
    2048-entry stack array (gsd_lq_cpu_engine.c:292), so contexts beyond 2048
    run the oracle restatement (heap scores, same loops)."""
    O, kind = _oracle()
    nh, nkv, hd = 32, 8, 128
    rng = np.random.default_rng(3)
    out = {}
    for ctx in ctxs:
        k2 = kind if ctx <= 2048 else "port"
        lib = O.load(k2)
        kc = rng.standard_normal(ctx * nkv * hd, dtype=np.float32).astype(np.float16).view(np.uint16)
        vc = rng.standard_normal(ctx * nkv * hd, dtype=np.float32).astype(np.float16).view(np.uint16)
        q0 = rng.standard_normal(nh * hd, dtype=np.float32)
        k = rng.standard_normal(nkv * hd, dtype=np.float32)
        v = rng.standard_normal(nkv * hd, dtype=np.float32)
        o = np.zeros(nh * hd, np.float32)
        n, t0 = 0, time.time()
        while time.time() - t0 < seconds or n < 3:
            q = q0.copy()
            lib.gsd_cpu_rope_and_store_kv(O.P(q), O.P(k), O.P(v), O.P(kc), O.P(vc), 0, ctx - 1, nh, nkv, hd, ctx,
                                          1e6, 1)
            lib.gsd_cpu_gqa_attention(O.P(q), O.P(kc), O.P(vc), O.P(o), 0, ctx - 1, nh, nkv, hd, ctx,
                                      float(1.0 / np.sqrt(hd)))
            n += 1
        us = (time.time() - t0) * 1e6 / n
        out[f"ctx{ctx}"] = {"us_per_layer": round(us, 1), "kind": k2, "calls": n}
    out["cpu"] = host_cpu()
    return out


def cpu_decode(bank, n_prompt=2, n_new=6):
    """C4 on the CPU: greedy decode of the 32-layer 7B Precision model
    (the bank's distinct layers repeated) by the reference engine through the
    reference's forward order (gsd_lq_cpu_runtime.py:302-420), a bounded
    sample of n_prompt + n_new tokens."""
    O, kind = _oracle()
    src = BankSource(bank, 32)
    ref = O.OracleModel(src, kind=kind, max_seq_len=64)
    prompt = np.random.default_rng(4).integers(0, V, n_prompt).tolist()
    logits = None
    for pos, t in enumerate(prompt):
        logits = ref.forward_token(int(t), pos, return_logits=pos == len(prompt) - 1)
    t0 = time.time()
    pos = len(prompt)
    for _ in range(n_new):
        logits = ref.forward_token(ref.greedy(logits), pos)
        pos += 1
    dt = time.time() - t0
    return {"decode_tok_s": round(n_new / dt, 3), "kind": kind, "cpu": host_cpu(),
            "sample": f"{n_prompt}-token prompt, then {n_new} greedy tokens ({dt:.1f}s)"}


def probe(kind: str, n: int, ctx: int = 8192, m: int = 128):
    """Launch one kernel repeatedly for counter collection under rocprofv3:
    'gateup' = the fused gate/up matvec over 8 rotated Turbo layers,
    'ffn' = the fused o + FFN launch (o + residual, gate/up + SwiGLU + down +
    residual) over 8 rotated Turbo layers,
    'copy' = a 256 MiB device copy (the calibration of FETCH/WRITE_SIZE),
    'attn' = RoPE + K/V append and decode attention at context `ctx`,
    'prefill' = the batched projection of 8 Turbo layer sets for `m` tokens,
    'prompt' = an `m`-token prompt through the batched prefill of the 32-layer
    7B Precision model, `n` times,
    'decode' = `n` greedy tokens of the 32-layer 7B Precision model."""
    from gsdlq import hip
    lib = hip.lib()
    if kind == "attn":
        r = bench_attention(ctxs=(ctx,), reps=n)
        print(f"[probe] attention ctx {ctx}: {r}", flush=True)
        return
    if kind == "prefill":
        r = bench_prefill(LayerBank("turbo", 8), ms=(m,), reps=n)
        print(f"[probe] prefill M {m}: {r}", flush=True)
        return
    if kind == "prompt":
        bank = LayerBank("precision", 3)
        model = build_model(bank, 32, max_seq=m + 8)
        toks = np.random.default_rng(5).integers(0, V, m).tolist()
        model.prefill(toks, 0, return_logits=False)   # warm
        t0 = time.time()
        for _ in range(n):
            model.prefill(toks, 0)
        dt = (time.time() - t0) / n
        model.close()
        print(f"[probe] {m}-token prompt, 32-layer 7B Precision: {dt * 1e3:.2f} ms ({m / dt:.0f} tok/s)", flush=True)
        return
    if kind == "decode":
        bank = LayerBank("precision", 3)
        model = build_model(bank, 32, max_seq=n + 16)
        model.generate_greedy([1], 4)   # warm (graphs captured)
        t0 = time.time()
        model.generate_greedy([1], n)
        dt = time.time() - t0
        model.close()
        print(f"[probe] decode {n} tokens of the 32-layer 7B Precision model: {n / dt:.1f} tok/s", flush=True)
        return
    if kind == "copy":
        nbytes = 256 << 20
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        lib.gsdh_malloc(ctypes.byref(a), nbytes)
        lib.gsdh_malloc(ctypes.byref(b), nbytes)
        for _ in range(n):
            lib.gsdh_stream_copy(None, b, a, nbytes)
        lib.gsdh_stream_sync(None)
        lib.gsdh_free(a)
        lib.gsdh_free(b)
        print(f"[probe] copy {nbytes} bytes x {n}", flush=True)
        return
    bank = LayerBank("turbo", 8)
    model = build_model(bank, bank.n)
    model.forward_token(1, 0)
    mask = 14 if kind == "ffn" else 4
    for i in range(n):
        lib.gsdh_model_run_linear(model._m, i % bank.n, mask)
    lib.gsdh_stream_sync(lib.gsdh_model_stream(model._m))
    if kind == "ffn":
        print(f"[probe] o + FFN launches {n}, algorithmic bytes per launch {ffn_bytes(bank, 0)}", flush=True)
    else:
        gu = sum(alg_bytes(bank.packed[(0, t)]) for t in ("ffn_gate", "ffn_up")) - 4 * H
        print(f"[probe] gate/up launches {n}, algorithmic bytes per launch {gu}", flush=True)
    model.close()


def bench_attention(ctxs=(512, 2048, 8192), reps=20):
    """Decode attention with K/V append (32 query heads, 8 KV heads, head dim
    128, RoPE theta 1e6) at contexts 512 / 2048 / 8192: per layer one launch
    (gsdh_rope_store_gqa_attention) that rotates q and the new K row, appends
    fp16 K/V at pos = ctx - 1 and attends over the cache filled to ctx - 1,
    the two reference calls in one (gsd_lq_cpu_engine.c:185-330 computes the
    same).
    Enough layers are rotated that the caches exceed 512 MB (beyond the
    Infinity Cache), at most 512 (below ctx 256 the caches are smaller); the
    launches of all layers are captured in one graph on the stream of a small
    model context and timed with HIP events there.  (rocprofv3's kernel trace
    of a graph of 1024 of these launches, 672 bytes of kernel arguments each,
    ended in a host segmentation fault before any kernel ran; graphs of up to
    512 trace normally.)
    Algorithmic bytes per layer: K + V read (ctx * 8 * 128 * 2 * 2) + the
    4096-byte append + q and the output (2 * 4 * 4096)."""
    import run_gpu_native_chat as chat
    from gsdlq import hip, synth
    n_heads, n_kv, hd, theta = 32, 8, 128, 1.0e6
    sm_scale = float(1.0 / np.sqrt(hd))
    # a small model context: its stream, graph capture and event timing
    spec = synth.SynthSpec(n_layers=1, hidden=256, ffn=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=256,
                           mode="turbo")
    model = chat.GPUMistralV2Model(synth.SynthSource(spec), max_seq_len=16, verbose=False)
    lib = model.cl.lib
    sp = ctypes.c_void_p(lib.gsdh_model_stream(model._m))
    rng = np.random.default_rng(3)
    res = {}
    for ctx in ctxs:
        kv_layer = ctx * n_kv * hd * 2 * 2
        L = min(512, max(4, -(-(512 << 20) // kv_layer)))
        bufs = {}
        sizes = {"kc": L * kv_layer // 2, "vc": L * kv_layer // 2, "q": L * n_heads * hd * 4,
                 "k": L * n_kv * hd * 4, "v": L * n_kv * hd * 4, "out": L * n_heads * hd * 4}
        for nm, nb in sizes.items():
            bufs[nm] = ctypes.c_void_p()
            lib.gsdh_malloc(ctypes.byref(bufs[nm]), nb)
        # one layer's worth of fp16 N(0,1) values, repeated over the layers
        lay = rng.standard_normal(kv_layer // 4, dtype=np.float32).astype(np.float16)
        for nm in ("kc", "vc"):
            for l in range(L):
                lib.gsdh_memcpy_h2d(ctypes.c_void_p(bufs[nm].value + l * lay.nbytes),
                                    lay.ctypes.data_as(ctypes.c_void_p), lay.nbytes, None)
        host = [rng.standard_normal(sizes[nm] // 4, dtype=np.float32) for nm in ("q", "k", "v")]
        for nm, h in zip(("q", "k", "v"), host):
            lib.gsdh_memcpy_h2d(bufs[nm], h.ctypes.data_as(ctypes.c_void_p), h.nbytes, None)
        lib.gsdh_stream_sync(None)   # (host arrays referenced until here)
        pos = ctx - 1
        at = lambda nm, l, n: ctypes.c_void_p(bufs[nm].value + l * n * 4)

        def run():
            for l in range(L):
                lib.gsdh_rope_store_gqa_attention(sp, at("q", l, n_heads * hd), at("k", l, n_kv * hd),
                                                  at("v", l, n_kv * hd), bufs["kc"], bufs["vc"],
                                                  at("out", l, n_heads * hd), l, pos, n_heads, n_kv, hd, ctx,
                                                  ctypes.c_float(theta), 1, ctypes.c_float(sm_scale))

        run()                                    # warm-up, outside the capture
        lib.gsdh_stream_sync(sp)
        ge = capture(model, run)
        time_graph(model, ge, 2)
        us = time_graph(model, ge, reps) * 1e3 / (reps * L)
        lib.gsdh_graph_destroy(ge)
        for nm in bufs:
            lib.gsdh_free(bufs[nm])
        b = kv_layer + 4096 + 2 * 4 * n_heads * hd
        gbs = b / (us * 1e-6) / 1e9
        res[f"ctx{ctx}"] = {"us_per_layer": round(us, 2), "bytes_per_layer": b, "GBs": round(gbs, 1),
                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "layers_rotated": L}
    model.close()
    res["workload"] = ("32 q heads / 8 KV heads x 128, fp16 KV cache ~N(0,1) filled to ctx-1, RoPE + append at "
                       "ctx-1 and attention in one launch per layer (gsdh_rope_store_gqa_attention); graph of all "
                       "layers, HIP events")
    return res


def traffic_from_profile():
    """HBM bytes per fused FFN launch from the committed counter summary
    (profiles/ffn_kernel_traffic.txt: FETCH_SIZE and WRITE_SIZE per dispatch
    of the kernel and of a 256 MiB copy), or None."""
    path = os.path.join(ROOT, "profiles", "ffn_kernel_traffic.txt")
    if not os.path.exists(path):
        return None
    kv = {}
    for line in open(path):
        if "=" in line and not line.lstrip().startswith("#"):
            k, v = line.split("=", 1)
            kv[k.strip()] = v.strip().split()[0]
    try:
        copy_bytes = float(kv["copy_bytes"])
        f_scale = copy_bytes / float(kv["copy_fetch_kib"])
        w_scale = copy_bytes / float(kv["copy_write_kib"])
        return int(float(kv["ffn_fetch_kib"]) * f_scale + float(kv["ffn_write_kib"]) * w_scale)
    except (KeyError, ValueError, ZeroDivisionError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=8, help="distinct packed layers rotated (Turbo)")
    ap.add_argument("--no-precision", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-attention", action="store_true")
    ap.add_argument("--no-c1", action="store_true")
    ap.add_argument("--probe", choices=["gateup", "ffn", "copy", "attn", "prefill", "prompt", "decode"],
                    help="run one kernel for rocprofv3 counters")
    ap.add_argument("--ctx", type=int, default=8192, help="--probe attn: context length")
    ap.add_argument("--m", type=int, default=128, help="--probe prefill / prompt: tokens")
    a = ap.parse_args()
    if a.probe:
        probe(a.probe, max(a.steps, 1), a.ctx, a.m)
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the decode path has no multi-GPU mode in this build "
              "(sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    from gsdlq import hip
    name, total, ncu = hip.device_info()
    log(f"device {name}, {ncu} CUs, {total / 2**30:.0f} GiB")

    turbo = LayerBank("turbo", a.layers)
    gbs, ms_step, roof = bench_linear(turbo, a.steps, a.warmup)
    log(f"turbo layer set: {gbs:.1f} GB/s, {ms_step * 1e3:.1f} us/step; FFN launch {roof['achieved']} GB/s")
    extra = {}
    if not a.no_prefill:
        extra["prefill_turbo"] = dict(bench_prefill(turbo), workload="Turbo 7B layer set (7 tensors), X bf16 "
                                      "[M][cols] -> Y fp32, fp16 MFMA with fp32 accumulation")
    if not a.no_c1:
        extra["c1_matvec_4096"] = bench_c1(turbo)
        log(f"C1 matvec: {extra['c1_matvec_4096']}")
    if not a.no_attention:
        extra["attention_c3"] = bench_attention()
        log(f"attention: {extra['attention_c3']}")
    if not a.no_precision:
        prec = LayerBank("precision", max(3, a.layers // 2))
        pg, pms, proof = bench_linear(prec, a.steps, a.warmup)
        extra["precision"] = {"value": round(pg, 1), "unit": "GB/s", "us_per_step": round(pms * 1e3, 2),
                              "frac_hbm": round(pg / HBM_PEAK_GBS, 4), "codes": "7-bit device tiles (radius 6)",
                              "ffn_GBs": proof["achieved"], "ffn_us": proof["launch_us"],
                              "bytes_per_step": prec.layer_bytes[0]}
        log(f"precision layer set: {pg:.1f} GB/s")
        if not a.no_decode:
            extra["decode_7b_precision"] = bench_decode(prec)
            log(f"decode: {extra['decode_7b_precision']}")
        if not a.no_cpu_baseline and not a.no_decode:
            extra["cpu_c4_decode"] = cpu_decode(prec)
            log(f"CPU C4: {extra['cpu_c4_decode']}")
    cpu = None if a.no_cpu_baseline else cpu_baseline(turbo)
    if not a.no_cpu_baseline and not a.no_attention:
        extra["cpu_c3_attention"] = cpu_attention()
        log(f"CPU C3: {extra['cpu_c3_attention']}")
    out = {
        "metric": "fused unpack-matvec GB/s (% HBM peak); batch-1 decode tok/s, 7B shape",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded bf16 ~N(0,0.02) weights packed by this build's encoder)",
        "config": {"workload": "Mistral-7B layer linear set q,k,v,o,gate,up,down (4096/1024/14336), Turbo R=8 "
                               "u8 codes, batch 1, fp32 activations",
                   "distinct_layers_rotated": a.layers, "bytes_per_step": turbo.layer_bytes[0],
                   "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "device": name},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    out.update(extra)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
