"""Writes tests/golden/tokenizer_golden.json: input/output vectors of the
reference's tokenizer and prompt formatting, for the CPU test that pins this
build's restatement (gsd-lq_amd/run_gpu_native_chat.py) against them.

The reference ships no tests, fixtures or vocabulary files for these
functions, so this script imports the reference module in the build
container (run_gpu_native_chat.py: MistralSentencePieceTokenizer at
:660-729, format_mistral_prompt at :996-1013, SYSTEM_RULES at :987-993) and
records what it returns.  Only the vectors are committed; nothing here runs
on the GPU box or in the test suite.

Vocabulary: a small SentencePiece-style table built here (specials, the 256
<0xNN> byte tokens, single characters, and multi-character pieces with
seeded scores so merges happen in a non-trivial order), in two variants:
with type-3 special tokens, and with none (every type 1).

    python tests/golden/make_tokenizer_golden.py [/root/reference]
"""
import importlib.util
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"


def load_reference():
    path = os.path.join(REF, "gsd_lq_v2", "run_gpu_native_chat.py")
    spec = importlib.util.spec_from_file_location("ref_chat", path)
    mod = importlib.util.module_from_spec(spec)
    argv = sys.argv
    sys.argv = [path]          # the module reads sys.argv[1] as a model path at import
    try:
        spec.loader.exec_module(mod)
    finally:
        sys.argv = argv
    return mod


def vocabulary(with_specials: bool):
    toks, types = ["<unk>", "<s>", "</s>", "[INST]", "[/INST]"], [2, 3, 3, 3, 3]
    if not with_specials:
        types = [2, 1, 1, 1, 1]
    toks += [f"<0x{b:02X}>" for b in range(256)]
    types += [6] * 256
    chars = list("▁abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789.,!?'-:é")
    toks += chars
    types += [1] * len(chars)
    words = ["▁the", "▁Hello", "▁world", "▁in", "▁hat", "▁cat", "▁caf",
             "▁na", "ing", "tion", "▁Wo", "lo", "▁line", "er", "▁a", "▁is"]
    pieces = []
    for w in words:
        for i in range(len(w)):
            for j in range(i + 2, len(w) + 1):
                p = w[i:j]
                if p not in pieces and p not in toks:
                    pieces.append(p)
    toks += pieces
    types += [1] * len(pieces)
    rng = np.random.default_rng(11)
    scores = [0.0] * 261 + [float(-5.0 - i * 0.01) for i in range(len(chars))]
    scores += [float(v) for v in np.round(rng.uniform(-4.0, 0.0, len(pieces)), 4)]
    return toks, [float(s) for s in scores], types


TEXTS = ["Hello world", "the cat in the hat", "[INST] Hello [/INST] world</s>", "  leading spaces",
         "naïve café — \U0001F600", "line1\nline2", "", "[INST][/INST]", "</s></s>x",
         "tHe WoRlD 123!?", "is a tion-ing", "▁already marked"]
HISTORIES = [([], "hi there"), ([("a", "b")], "c"), ([("first q", "first a"), ("second q", "second a")], "third")]


def main():
    ref = load_reference()
    out = {"vocabularies": {}, "format": [], "system_rules": ref.SYSTEM_RULES}
    for name, sp in (("with_specials", True), ("no_specials", False)):
        toks, scores, types = vocabulary(sp)
        tk = ref.MistralSentencePieceTokenizer(toks, scores, types, 1, 2)
        cases = []
        for t in TEXTS:
            for bos in (True, False):
                ids = tk.encode(t, add_bos=bos)
                cases.append({"text": t, "add_bos": bos, "ids": ids, "decoded": tk.decode(ids)})
        smile = [5 + b for b in "\U0001F600".encode("utf-8")]
        extra = [{"ids": smile + [1, 2], "decoded": tk.decode(smile + [1, 2])},
                 {"ids": [5 + 0xE9], "decoded": tk.decode([5 + 0xE9])}]
        out["vocabularies"][name] = {"tokens": toks, "scores": scores, "token_types": types,
                                      "encode": cases, "decode": extra}
    for hist, msg in HISTORIES:
        for cpu in (False, True):
            out["format"].append({"history": hist, "msg": msg, "is_cpu": cpu,
                                  "prompt": ref.format_mistral_prompt(hist, msg, is_cpu=cpu)})
    with open(os.path.join(HERE, "tokenizer_golden.json"), "w", encoding="utf-8") as f:
        json.dump(out, f, ensure_ascii=True, indent=0)
    print("wrote tokenizer_golden.json")


if __name__ == "__main__":
    main()
