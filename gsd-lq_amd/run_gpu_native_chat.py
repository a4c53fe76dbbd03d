"""
GSD-LQ decode engine for AMD Instinct MI355X (gfx950) -- drop-in for
gsd_lq_v2/run_gpu_native_chat.py.

Same module surface as the reference module: GPUMistralV2Model,
MistralSentencePieceTokenizer, format_mistral_prompt, run_smoke_verify, main,
MAX_SEQ_LEN, SYSTEM_RULES, LOG_FILE, ensure_model_file, ensure_log_header,
log_turn, _get_turbo_codebook.  Underneath, the OpenCL runtime and kernels
(run_gpu_native_chat.py:101-657) are replaced by libgsdhip.so, hand-written
HIP kernels for CDNA4 called through a C ABI (include/gsdhip.h):

  * the packed weights stay packed in HBM and are expanded inside the fused
    matvec (RMSNorm and the rank-k projection fused into its prologue; kinks,
    the U term, residual adds and SwiGLU into its epilogue);
  * RoPE + fp16 KV append, split-context GQA attention;
  * one token (all layers, lm_head and the greedy argmax) is one HIP graph
    launch instead of 450-675 Python-side kernel launches.

Differences a caller can see:
  * model.device_name exists (the reference reads it in main() but never sets
    it, so its chat silently fell back to the CPU engine);
  * max_seq_len is a constructor argument (default 2048, or GSD_MAX_SEQ_LEN);
  * there is no CPU fallback and no network download: a missing GPU or engine
    library raises RuntimeError, a missing model file FileNotFoundError.
"""
from __future__ import annotations

import ctypes
import datetime
import os
import re
import sys
import time

import numpy as np

V2_DIR = os.path.dirname(os.path.abspath(__file__))
if V2_DIR not in sys.path:
    sys.path.insert(0, V2_DIR)

from gsdlq import codebook as _codebook  # noqa: E402
from gsdlq import gsd2 as _gsd2  # noqa: E402
from gsdlq import hip as _hip  # noqa: E402

MAX_SEQ_LEN = 2048
MODEL_PATH = os.path.join(V2_DIR, "mistral_v2_native_turbo.gsd2")
LOG_FILE = os.path.join(V2_DIR, "GPU_NATIVE_CHAT_LOG.md")


def _get_turbo_codebook(radius: int = 8):
    """(float32 [n_pts, 2], n_pts) of the radius-R A2 hexagon
    (run_gpu_native_chat.py:26-33)."""
    return _codebook.get_turbo_codebook(radius)


def ensure_model_file(model_path: str) -> str:
    """Resolve a packed model path among the reference's candidate names
    (run_gpu_native_chat.py:37-52).  This build never downloads."""
    if os.path.exists(model_path):
        return model_path
    base = os.path.basename(model_path)
    for c in (os.path.join(V2_DIR, base),
              os.path.join(V2_DIR, "mistral_v2_native_turbo.gsd2"),
              os.path.join(V2_DIR, "mistral_v2_native_precision.gsd2"),
              os.path.join(V2_DIR, "mistral_v2_native_hex2d.gsd2")):
        if os.path.exists(c):
            return c
    raise FileNotFoundError(f"packed model {model_path} not found (offline build: no download)")


class HIPRuntime:
    """Stands where the reference's OpenCLRuntime object stood (model.cl):
    device_name, total_vram_mb, allocated_bytes, finish(), release_all()."""

    def __init__(self):
        self.lib = _hip.lib()
        name, total, ncu = _hip.device_info()
        self.device_name = name
        self.total_vram_mb = total / (1024 * 1024)
        self.n_cu = ncu
        self.allocated_bytes = 0
        self._model = None

    def finish(self):
        if self._model:
            self.lib.gsdh_stream_sync(self.lib.gsdh_model_stream(self._model))

    def release_all(self):
        if self._model:
            self.lib.gsdh_model_destroy(self._model)
            self._model = None
        self.allocated_bytes = 0


class MistralSentencePieceTokenizer:
    """SentencePiece-style tokenizer over the vocabulary carried in the .gsd2
    header (behaviour of run_gpu_native_chat.py:660-729): specials split out
    first, spaces become U+2581, a leading U+2581 on the first text piece,
    characters outside the vocabulary fall back to <0xNN> byte tokens, then
    adjacent symbols are merged greedily by the highest merged-token score."""

    def __init__(self, tokens, scores, token_types, bos_id=1, eos_id=2):
        self.tokens = tokens
        self.scores = scores
        self.token_types = token_types
        self.bos_id = bos_id
        self.eos_id = eos_id
        self.vocab = {t: i for i, t in enumerate(tokens)}
        self.specials = sorted((t for t, ty in zip(tokens, token_types) if ty == 3), key=len, reverse=True)
        self.byte_tokens = {}
        for i, (t, ty) in enumerate(zip(tokens, token_types)):
            if ty == 6 and len(t) == 6 and t.startswith("<0x"):
                self.byte_tokens[i] = int(t[3:5], 16)

    def _bpe_piece(self, text: str):
        if not text:
            return []
        syms = []
        for ch in text:
            if ch in self.vocab:
                syms.append(ch)
            else:
                syms.extend(f"<0x{b:02X}>" for b in ch.encode("utf-8"))
        while len(syms) > 1:
            best, where = -1e30, -1
            for i in range(len(syms) - 1):
                tid = self.vocab.get(syms[i] + syms[i + 1])
                if tid is not None and self.scores[tid] > best:
                    best, where = self.scores[tid], i
            if where < 0:
                break
            syms[where:where + 2] = [syms[where] + syms[where + 1]]
        return [self.vocab.get(s, 0) for s in syms]

    def encode(self, text: str, add_bos: bool = True):
        ids = [self.bos_id] if add_bos else []
        # with no special tokens the pattern is "()", which matches the empty
        # string: every character becomes a part of its own, as in the reference
        parts = re.split("(" + "|".join(re.escape(s) for s in self.specials) + ")", text)
        first = True
        for part in parts:
            if not part:
                continue
            if part in self.vocab and self.token_types[self.vocab[part]] == 3:
                ids.append(self.vocab[part])
                first = False
                continue
            norm = part.replace(" ", "▁")
            if first and not norm.startswith("▁"):
                norm = "▁" + norm
            first = False
            ids.extend(self._bpe_piece(norm))
        return ids

    def decode(self, ids) -> str:
        out = bytearray()
        for tid in ids:
            if tid in (self.bos_id, self.eos_id):
                continue
            if tid in self.byte_tokens:
                out.append(self.byte_tokens[tid])
            else:
                out.extend(self.tokens[tid].replace("▁", " ").encode("utf-8"))
        return out.decode("utf-8", errors="replace")


def _open_source(src):
    """A path opens a .gsd2 file; any object with config/tensors/dense()/
    hex_field() (e.g. gsdlq.synth.SynthSource) is used as is."""
    if isinstance(src, (str, os.PathLike)):
        return _gsd2.Gsd2File(os.fspath(src)), True
    return src, False


class GPUMistralV2Model:
    """GPUMistralV2Model(gsd2_path, rope_interleaved=1) with the reference's
    attributes (cfg, n_layers, hidden, ffn_size, n_heads, n_kv_heads,
    head_dim, rope_theta, rms_eps, vocab_size, avg_bpw, tokenizer, embed,
    layers, vram_used_mb, cl) and methods forward_token / sample_token
    (run_gpu_native_chat.py:732-984)."""

    def __init__(self, gsd2_path, rope_interleaved: int = 1, max_seq_len: int | None = None,
                 verbose: bool = True):
        self.rope_interleaved = int(rope_interleaved)
        self.cl = HIPRuntime()
        self.device_name = self.cl.device_name
        self.max_seq_len = int(max_seq_len or os.environ.get("GSD_MAX_SEQ_LEN", MAX_SEQ_LEN))
        if verbose:
            print(f"GPU Device Detected : {self.device_name} ({self.cl.total_vram_mb:.0f} MB VRAM)", flush=True)
        t0 = time.time()
        src, owned = _open_source(gsd2_path)
        try:
            self._load(src)
        finally:
            if owned:
                src.close()
        if verbose:
            print(f"Model Loaded 100% Resident in GPU VRAM in {time.time() - t0:.2f}s!\n"
                  f"  Packed VRAM Footprint ({self.n_layers} Layers + LM Head + KV Cache): "
                  f"{self.vram_used_mb:.1f} MB ({self.vram_used_mb / 1024:.2f} GB / "
                  f"{self.cl.total_vram_mb / 1024:.2f} GB)", flush=True)

    # -- loading ----------------------------------------------------------
    def _load(self, src):
        cfg = src.config
        self.cfg = cfg
        self.n_layers = cfg["n_layers"]
        self.hidden = cfg["hidden_size"]
        self.ffn_size = cfg["ffn_size"]
        self.n_heads = cfg["n_heads"]
        self.n_kv_heads = cfg["n_kv_heads"]
        self.head_dim = cfg["head_dim"]
        self.rope_theta = cfg["rope_theta"]
        self.rms_eps = cfg["rms_eps"]
        self.vocab_size = cfg["vocab_size"]
        self.tokenizer = MistralSentencePieceTokenizer(cfg["tokens"], cfg["scores"], cfg["token_types"],
                                                       cfg["bos_id"], cfg["eos_id"])
        lib = self.cl.lib
        c = _hip.GsdModelConfig(self.n_layers, self.hidden, self.ffn_size, self.n_heads, self.n_kv_heads,
                                self.head_dim, self.vocab_size, self.max_seq_len, self.rope_interleaved,
                                float(self.rms_eps), float(self.rope_theta))
        handle = ctypes.c_void_p()
        lib.gsdh_model_create(ctypes.byref(c), ctypes.byref(handle))
        self._m = handle
        self.cl._model = handle
        tensors = src.tensors
        emb = np.ascontiguousarray(src.dense("token_embd.weight", np.float16))
        if emb.shape != (self.vocab_size, self.hidden):
            raise ValueError(f"token_embd.weight shape {emb.shape}")
        self.embed = emb
        lib.gsdh_model_set_embedding(self._m, _hip.ptr(emb.view(np.uint16)))
        packed_bits, packed_w = 0, 0
        self.layers = []
        for l in range(self.n_layers):
            p = f"blk.{l}."
            entry = {}
            for which, nm in ((0, "attn_norm"), (1, "ffn_norm")):
                w = np.ascontiguousarray(src.dense(p + nm + ".weight", np.float32))
                if w.size != self.hidden:
                    raise ValueError(f"{p}{nm}.weight has {w.size} values, expected {self.hidden}")
                lib.gsdh_model_set_norm(self._m, l, which, _hip.ptr(w))
                entry[nm] = w
            for key, t in (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output"),
                           ("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
                entry[key], bits = self._upload_hex(src, tensors, f"{p}{t}.weight", l, _hip.SLOTS[t])
                packed_bits += bits
                packed_w += entry[key]["rows"] * entry[key]["cols"]
            self.layers.append(entry)
        w = np.ascontiguousarray(src.dense("output_norm.weight", np.float32))
        lib.gsdh_model_set_norm(self._m, -1, 0, _hip.ptr(w))
        self.final_norm = w
        self.lm_head, bits = self._upload_hex(src, tensors, "output.weight", 0, _hip.SLOTS["output"])
        packed_bits += bits
        packed_w += self.lm_head["rows"] * self.lm_head["cols"]
        lib.gsdh_model_finalize(self._m)
        hdr_bpw = getattr(src, "header", {}).get("avg_bpw") if hasattr(src, "header") else None
        self.avg_bpw = float(hdr_bpw) if hdr_bpw is not None else packed_bits / max(packed_w, 1)
        dev = int(lib.gsdh_model_device_bytes(self._m))
        self.cl.allocated_bytes = dev
        self.vram_used_mb = dev / (1024 * 1024)
        self._logits = np.empty(self.vocab_size, dtype=np.float32)

    def _upload_hex(self, src, tensors, name, layer, slot):
        m = tensors[name]
        radius, rows, cols, k = int(m["radius"]), int(m["rows"]), int(m["cols"]), int(m["k_dim"])
        if radius not in (1, 2, 3, 4, 5, 6, 7, 8):
            raise ValueError(f"{name}: radius {radius} unsupported")
        if cols % 64:
            raise ValueError(f"{name}: cols {cols} is not a multiple of 64")
        if not 0 <= k <= 16:
            raise ValueError(f"{name}: k_dim {k} outside 0..16")
        g = {f: np.ascontiguousarray(src.hex_field(name, f)) for f in _gsd2.HEX_FIELDS}
        if k > 0:
            g.update({f: np.ascontiguousarray(src.hex_field(name, f)) for f in _gsd2.LOWRANK_FIELDS})
        need = _gsd2.hex_nbytes(rows, cols, k, g["kink_cols"].size)
        for f, n in need.items():
            if g[f].nbytes != n:
                raise ValueError(f"{name}.{f}: {g[f].nbytes} bytes, expected {n}")
        nk = int(g["kink_cols"].size)
        if g["kink_deltas"].size != nk:
            raise ValueError(f"{name}: {nk} kink columns but {g['kink_deltas'].size} deltas")
        try:
            self.cl.lib.gsdh_model_set_hex(self._m, layer, slot, radius, rows, cols, k,
                                           _hip.ptr(g["codes"]), _hip.ptr(g["scales"]), _hip.ptr(g["row_ptr"]),
                                           _hip.ptr(g["kink_cols"]) if nk else None,
                                           _hip.ptr(g["kink_deltas"]) if nk else None, nk,
                                           _hip.ptr(g.get("U")), _hip.ptr(g.get("S")), _hip.ptr(g.get("Vt")))
        except _hip.HipError as e:
            if "set_hex:" in str(e):
                raise ValueError(str(e)) from None
            raise
        bits = 8 * sum(int(a.nbytes) for a in g.values())
        info = {"rows": rows, "cols": cols, "k_dim": k, "radius": radius,
                "n_pts": _codebook.n_points(radius), "nk": nk}
        return info, bits

    # -- decode -----------------------------------------------------------
    def forward_token(self, token_id: int, pos: int, return_logits: bool = True):
        """One token at position pos through every layer; returns the f32
        logits (vocab,) when return_logits, else None (run_gpu_native_chat.py:892-969)."""
        am = ctypes.c_int(-1)
        if return_logits:
            self.cl.lib.gsdh_forward_token(self._m, int(token_id), int(pos), 1, _hip.ptr(self._logits),
                                           ctypes.byref(am))
            return self._logits.copy()
        self.cl.lib.gsdh_forward_token(self._m, int(token_id), int(pos), 0, None, None)
        return None

    def prefill(self, token_ids, start_pos: int = 0, return_logits: bool = True):
        """The prompt tokens token_ids at positions start_pos.. through every
        layer at once (batched projections on the matrix cores, causal
        attention over the cache; positions below start_pos are reused as
        cached).  Returns the last token's f32 logits (vocab,) when
        return_logits, else None.  The reference runs forward_token per prompt
        token (run_gpu_native_chat.py:1128-1130); the results agree with it."""
        ids = np.ascontiguousarray(np.asarray(token_ids, dtype=np.int32))
        if ids.size == 0:
            raise ValueError("prefill: no tokens")
        am = ctypes.c_int(-1)
        if return_logits:
            self.cl.lib.gsdh_model_prefill(self._m, _hip.ptr(ids), int(ids.size), int(start_pos), 1,
                                           _hip.ptr(self._logits), ctypes.byref(am))
            return self._logits.copy()
        self.cl.lib.gsdh_model_prefill(self._m, _hip.ptr(ids), int(ids.size), int(start_pos), 0, None, None)
        return None

    def set_prefill(self, batched: bool) -> None:
        """generate_greedy's prompt: batched (default) or one decode step per token."""
        self.cl.lib.gsdh_model_set_prefill(self._m, 1 if batched else 0)

    def generate_greedy(self, prompt_ids, n_new: int, start_pos: int = 0):
        """Prefill prompt_ids at start_pos.. then n_new greedy tokens, all on
        the device (one graph launch per token, no logits round trip).
        Returns (tokens, top1-top2 margins)."""
        p = np.ascontiguousarray(np.asarray(prompt_ids, dtype=np.int32))
        toks = np.empty(n_new, dtype=np.int32)
        margins = np.empty(n_new, dtype=np.float32)
        self.cl.lib.gsdh_generate_greedy(self._m, _hip.ptr(p), int(p.size), int(start_pos), int(n_new),
                                         _hip.ptr(toks), _hip.ptr(margins))
        return toks.tolist(), margins.tolist()

    def sample_token(self, logits: np.ndarray, temperature: float = 0.4, top_p: float = 0.9) -> int:
        """Greedy when temperature <= 1e-4, else temperature + nucleus sampling
        (run_gpu_native_chat.py:971-984)."""
        if temperature <= 1e-4:
            return int(np.argmax(logits))
        scaled = logits / temperature
        scaled = scaled - np.max(scaled)
        probs = np.exp(scaled)
        probs /= np.sum(probs)
        order = np.argsort(probs)[::-1]
        cum = np.cumsum(probs[order])
        cut = int(np.searchsorted(cum, top_p)) + 1
        top = order[:cut]
        p = probs[top]
        p /= np.sum(p)
        return int(np.random.choice(top, p=p))

    def close(self):
        self.cl.release_all()

    def __del__(self):
        try:
            self.cl.release_all()
        except Exception:
            pass


SYSTEM_RULES = (
    "You are Mistral-7B-GSD-LQ-v2.0 running natively on an AMD Instinct MI355X GPU "
    "using packed hex2d on-the-fly unpacking. "
    "You have continuous memory of this entire conversation. "
    "If the user asks about facts or hardware details mentioned earlier, quote them accurately. "
    "If they ask about something not mentioned yet, say you do not know rather than guessing."
)


def format_mistral_prompt(history, new_user_msg: str, is_cpu: bool = False) -> str:
    """[INST] chat formatting of run_gpu_native_chat.py:996-1013."""
    parts = []
    if is_cpu:
        parts.extend(f"[INST] {u} [/INST] {a}</s>" for u, a in history)
        parts.append(f"[INST] {new_user_msg} [/INST]")
        return "".join(parts)
    if not history:
        return f"[INST] {SYSTEM_RULES}\n\nUser: {new_user_msg} [/INST]"
    for i, (u, a) in enumerate(history):
        head = f"{SYSTEM_RULES}\n\nUser: {u}" if i == 0 else u
        parts.append(f"[INST] {head} [/INST] {a}</s>")
    parts.append(f"[INST] {new_user_msg} [/INST]")
    return "".join(parts)


def ensure_log_header(vram_mb: float, total_vram_mb: float, avg_bpw: float):
    if os.path.exists(LOG_FILE):
        return
    with open(LOG_FILE, "w", encoding="utf-8") as f:
        f.write("# NATIVE GPU CHAT LOG: GSD-LQ v2.0 (HIP, MI355X)\n\n")
        f.write(f"**Session Initialized**: {datetime.datetime.now().strftime('%Y-%m-%d %H:%M:%S')}\n")
        f.write("**Runtime Engine**: libgsdhip (HIP, gfx950)\n")
        f.write(f"**Average Weight Footprint**: {avg_bpw:.3f} bits/weight (Native Packed Hex2D)\n")
        f.write(f"**Live VRAM Footprint**: {vram_mb:.1f} MB / {total_vram_mb:.0f} MB\n\n---\n\n")


def log_turn(turn_num, prompt, response, prefill_s, p_toks, gen_s, g_toks, vram_mb):
    tps = g_toks / max(gen_s, 0.001)
    with open(LOG_FILE, "a", encoding="utf-8") as f:
        f.write(f"### Turn {turn_num} at {datetime.datetime.now().strftime('%H:%M:%S')}\n\n")
        f.write(f"**User Prompt**:\n> {prompt}\n\n**Response**:\n{response}\n\n")
        f.write(f"*Stats*: Prefill {p_toks} tok in {prefill_s:.2f}s | Generated {g_toks} tok in {gen_s:.2f}s "
                f"(**{tps:.2f} tok/s**) | *GPU VRAM*: {vram_mb:.1f} MB\n\n---\n\n")


def run_smoke_verify(model) -> str:
    """Greedy 8 tokens after "The capital of France is" (run_gpu_native_chat.py:1039-1055)."""
    prompt = "The capital of France is"
    ids = model.tokenizer.encode(prompt, add_bos=True)
    logits = model.prefill(ids, 0)
    out_ids = []
    pos = len(ids)
    for _ in range(8):
        nxt = model.sample_token(logits, temperature=0.0)
        if nxt == model.tokenizer.eos_id:
            break
        out_ids.append(nxt)
        logits = model.forward_token(nxt, pos, return_logits=True)
        pos += 1
    decoded = model.tokenizer.decode(out_ids)
    print(f"[SMOKE TEST] '{prompt}' -> '{decoded}'", flush=True)
    return decoded


def main(argv=None):
    argv = list(sys.argv[1:] if argv is None else argv)
    paths = [a for a in argv if not a.startswith("--")]
    model_path = paths[0] if paths else MODEL_PATH
    if "--smoke" in argv:
        m = GPUMistralV2Model(ensure_model_file(model_path), rope_interleaved=1)
        run_smoke_verify(m)
        m.cl.release_all()
        return
    model = GPUMistralV2Model(ensure_model_file(model_path), rope_interleaved=1)
    ensure_log_header(model.vram_used_mb, model.cl.total_vram_mb, model.avg_bpw)
    print("=" * 84)
    print(f"GSD-LQ v2.0 (HIP GPU: {model.device_name})")
    print(f"Logging all turns to: {LOG_FILE}")
    print("Commands: type 'reset' to clear chat memory, 'quit' or 'exit' to stop.")
    print("=" * 84)
    history, cached, turn = [], [], 1
    max_seq = model.max_seq_len
    while True:
        try:
            print(f"\n[Turn {turn}] You > ", end="", flush=True)
            line = sys.stdin.readline()
            if not line:
                break
            msg = line.strip()
            if msg.lower() in ("quit", "exit", "q"):
                break
            if msg.lower() == "reset":
                history.clear()
                cached.clear()
                print("[Memory cleared]")
                continue
            if not msg:
                continue
            ids = model.tokenizer.encode(format_mistral_prompt(history, msg), add_bos=True)
            prefix = 0
            while prefix < len(cached) and prefix < len(ids) - 1 and cached[prefix] == ids[prefix]:
                prefix += 1
            if len(ids) >= max_seq - 64:
                print(f"[Context window full, resetting conversation history to fit {max_seq} tokens]")
                history.clear()
                cached.clear()
                prefix = 0
                ids = model.tokenizer.encode(format_mistral_prompt(history, msg), add_bos=True)
            t0 = time.time()
            # the new prompt tokens in one batched pass over the reused prefix
            logits = model.prefill(ids[prefix:], prefix)
            pre_s = time.time() - t0
            print("\nMistral-7B (GPU Native) > ", end="", flush=True)
            t1, gen, prev, pos = time.time(), [], "", len(ids)
            for _ in range(min(512, max_seq - pos - 1)):
                nxt = model.sample_token(logits, temperature=0.4, top_p=0.9)
                if nxt == model.tokenizer.eos_id:
                    break
                gen.append(nxt)
                cur = model.tokenizer.decode(gen)
                print(cur[len(prev):], end="", flush=True)
                prev = cur
                logits = model.forward_token(nxt, pos, return_logits=True)
                pos += 1
            gen_s = time.time() - t1
            resp = model.tokenizer.decode(gen).strip()
            print(f"\n\n[GPU Stats: Prefill {len(ids) - prefix} tok ({pre_s:.2f}s) | Gen {len(gen)} tok in "
                  f"{gen_s:.2f}s ({len(gen) / max(gen_s, 1e-3):.2f} tok/s) | VRAM: {model.vram_used_mb:.1f} MB]")
            history.append((msg, resp))
            cached = ids + gen
            log_turn(turn, msg, resp, pre_s, len(ids) - prefix, gen_s, len(gen), model.vram_used_mb)
            turn += 1
        except KeyboardInterrupt:
            print("\nInterrupted. Log saved.")
            break
    model.cl.release_all()


if __name__ == "__main__":
    main()
