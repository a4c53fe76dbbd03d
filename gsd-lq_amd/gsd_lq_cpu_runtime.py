"""
Drop-in for gsd_lq_v2/gsd_lq_cpu_runtime.py on an MI355X build.

Keeps the module's names -- MAX_SEQ_LEN, build_c_library, CPUEngine,
_get_turbo_codebook, CPUMistralV2Model -- so callers written against the
reference runtime keep importing and running.  On this build every one of
them drives the HIP engine (libgsdhip.so): there is no CPU inference path in
the product.  CPUMistralV2Model is the GPU model with the CPU runtime's
sampling defaults (temperature 0.0, nan_to_num before the argmax,
gsd_lq_cpu_runtime.py:422-443).

The reference CPU engine itself (gsd_lq_cpu_engine.c) is restated only as the
test oracle under oracle/, which the product never loads.
"""
from __future__ import annotations

import os
import sys

import numpy as np

V2_DIR = os.path.dirname(os.path.abspath(__file__))
if V2_DIR not in sys.path:
    sys.path.insert(0, V2_DIR)

from gsdlq import build as _build  # noqa: E402
from gsdlq import codebook as _codebook  # noqa: E402
from gsdlq import hip as _hip  # noqa: E402
from run_gpu_native_chat import GPUMistralV2Model, MistralSentencePieceTokenizer  # noqa: E402,F401

MAX_SEQ_LEN = 2048
LIB_NAME = "libgsdhip.so"
LIB_PATH = os.path.join(V2_DIR, LIB_NAME)


def build_c_library() -> str:
    """Builds the engine library when it is missing or older than its sources
    (the reference compiled gsd_lq_cpu_engine.c here, gsd_lq_cpu_runtime.py:25-73).
    Returns its path, or "" when no compiler is available."""
    try:
        if _build.hip_sources_newer_than(LIB_PATH):
            _build.build_hip(LIB_PATH)
        return LIB_PATH
    except Exception as e:  # no hipcc: mirror the reference's "" result
        print(f"[!] Engine build failed: {e}")
        return LIB_PATH if os.path.exists(LIB_PATH) else ""


class CPUEngine:
    """Holds the bound engine library in .lib (gsd_lq_cpu_runtime.py:76-108).
    Its entry points take device pointers and a stream (include/gsdhip.h)."""

    def __init__(self):
        self.lib_path = build_c_library()
        if not self.lib_path:
            raise RuntimeError("libgsdhip.so unavailable; this build has no CPU fallback")
        self.lib = _hip.lib()


def _get_turbo_codebook(radius: int = 6):
    return _codebook.get_turbo_codebook(radius)


class CPUMistralV2Model(GPUMistralV2Model):
    """CPUMistralV2Model(gsd2_path, rope_interleaved=1): same surface as the
    reference CPU model, executed by the HIP engine."""

    def __init__(self, gsd2_path, rope_interleaved: int = 1, max_seq_len: int | None = None,
                 verbose: bool = True):
        self.cpu = CPUEngine()
        super().__init__(gsd2_path, rope_interleaved=rope_interleaved,
                         max_seq_len=max_seq_len or MAX_SEQ_LEN, verbose=verbose)

    def sample_token(self, logits, temperature: float = 0.0, top_p: float = 0.9):
        """gsd_lq_cpu_runtime.py:422-443: nan_to_num, argmax at T <= 0, else
        temperature + nucleus sampling."""
        logits = np.nan_to_num(logits, nan=-1e4, posinf=100.0, neginf=-1e4)
        if temperature <= 0.0:
            return int(np.argmax(logits))
        logits = logits / max(temperature, 1e-4)
        logits = logits - np.max(logits)
        probs = np.exp(logits)
        s = np.sum(probs)
        if s <= 0 or np.isnan(s):
            return int(np.argmax(logits))
        probs /= s
        order = np.argsort(probs)[::-1]
        sp = probs[order]
        cut = int(np.argmax(np.cumsum(sp) > top_p)) + 1
        top, p = order[:cut], sp[:cut]
        ps = np.sum(p)
        if ps <= 0 or np.isnan(ps):
            return int(top[0])
        return int(np.random.choice(top, p=p / ps))
