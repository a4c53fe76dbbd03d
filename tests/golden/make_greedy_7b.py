"""Writes greedy_7b_precision.json: the 128-step greedy decode of the seeded
32-layer Mistral-7B-shaped synthetic model (Precision mode: radius 6, rank-2
correction) after a 64-token prompt of seeded uniform token ids.

The token sequence comes from the reference CPU engine compiled from its own
source (oracle/_ref/libgsd_cpu.so, built by oracle/Makefile), driven in the
order of gsd_lq_v2/gsd_lq_cpu_runtime.py:302-425; when that library is absent
the oracle restatement (bit-identical, see tests/test_oracle.py) is used and
the file records which one ran.  Takes ~15 minutes on 8 cores.

    python tests/golden/make_greedy_7b.py [--steps 128] [--kind reference]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "gsd-lq_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from gsdlq import synth  # noqa: E402
import oracle as O  # noqa: E402

PROMPT_SEED = 4
PROMPT_LEN = 64


def prompt_ids(vocab: int = 32768):
    return [int(t) for t in np.random.default_rng(PROMPT_SEED).integers(0, vocab, PROMPT_LEN)]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--kind", default="reference" if O.have_reference() else "port")
    ap.add_argument("--out", default=os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                  "greedy_7b_precision.json"))
    a = ap.parse_args()
    spec = synth.SynthSpec(mode="precision")
    t0 = time.time()
    src = synth.SynthSource(spec)
    model = O.OracleModel(src, kind=a.kind)
    print(f"model packed and loaded in {time.time() - t0:.0f}s", flush=True)
    prompt = prompt_ids(spec.vocab)
    t0 = time.time()
    logits = None
    for pos, tid in enumerate(prompt):
        logits = model.forward_token(tid, pos, return_logits=(pos == len(prompt) - 1))
        print(f"prefill {pos} {time.time() - t0:.0f}s", flush=True)
    toks, margins, top5 = [], [], []
    pos = len(prompt)
    for step in range(a.steps):
        nxt = model.greedy(logits)
        order = np.argsort(-logits, kind="stable")[:5]
        top5.append([[int(i), float(logits[i])] for i in order])
        srt = np.sort(logits)
        margins.append(float(srt[-1] - srt[-2]))
        toks.append(nxt)
        logits = model.forward_token(nxt, pos, return_logits=True)
        pos += 1
        print(f"step {step} tok {nxt} margin {margins[-1]:.4g} {time.time() - t0:.0f}s", flush=True)
    out = {"spec": {k: getattr(spec, k) for k in ("n_layers", "hidden", "ffn", "n_heads", "n_kv_heads",
                                                  "head_dim", "vocab", "mode", "rank", "kinks_per_row",
                                                  "lr_iters", "seed", "sigma")},
           "engine": a.kind, "prompt": prompt, "tokens": toks, "margins": margins, "top5": top5}
    with open(a.out, "w") as f:
        json.dump(out, f)
    print("wrote", a.out)


if __name__ == "__main__":
    main()
