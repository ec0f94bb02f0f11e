"""Writes tests/golden/decode_1b_greedy.json: the oracle's greedy trace on the
synthetic Llama-3.2-1B-shaped model of benchmark config 5.

Model: alpacca_amd.model.synthetic_llama_1b(seed=SEED) (16 layers, hidden
2048, 32/8 heads, head_dim 64, FFN 8192, vocab 128256, Q4_K with Q6_K attn_v,
8 ffn_down and the output head).  Prompt: N_PROMPT token ids drawn with
numpy.random.default_rng(PROMPT_SEED).integers(0, 128256).  The oracle
(oracle/model_ref.py, a restatement of alpacca/model.py) prefills the prompt
in chunks of 256 (Model.prefill, model.py:610-641) and decodes N_GEN tokens
greedily (argmax of the logits, tensor.py:187-194), recording the top-1 /
top-2 logit margin of every step.  CPU only; takes a few minutes.

With --repeat-penalty P (and --repeat-last-n L, default 64) it writes
decode_1b_greedy_penalty.json instead: the decode loop of tests/bench.py:78-90,
a temperature-0 Sampler that accepts the prompt and each chosen token and
divides (or, for values <= 0, multiplies) the logits of the last L accepted
tokens by P before the argmax (sample.py:31-45).

Run: python tests/golden/make_decode_1b.py [--repeat-penalty 1.1]
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

SEED, PROMPT_SEED, N_PROMPT, N_GEN = 0, 2048, 2048, 256
OUT = Path(__file__).resolve().parent / "decode_1b_greedy.json"
OUT_PENALTY = Path(__file__).resolve().parent / "decode_1b_greedy_penalty.json"


def prompt_tokens(n_vocab: int = 128256) -> list[int]:
    rng = np.random.default_rng(PROMPT_SEED)
    return [int(t) for t in rng.integers(0, n_vocab, N_PROMPT)]


def main() -> None:
    import argparse

    from alpacca_amd.model import synthetic_llama_1b
    from oracle.model_ref import RefModel
    ap = argparse.ArgumentParser()
    ap.add_argument("--repeat-penalty", type=float, default=1.0)
    ap.add_argument("--repeat-last-n", type=int, default=64)
    args = ap.parse_args()
    penalized = args.repeat_penalty not in (0.0, 1.0)
    out = OUT_PENALTY if penalized else OUT

    t0 = time.time()
    hp, tensors = synthetic_llama_1b(seed=SEED)
    model = RefModel(hp, tensors, n_ctx=N_PROMPT + N_GEN, fast=True)
    print(f"model built in {time.time() - t0:.1f} s", flush=True)
    prompt = prompt_tokens(hp.n_vocab)

    def progress(i, t):
        if i % 32 == 0:
            print(f"step {i}: token {t} ({time.time() - t0:.0f} s)", flush=True)

    toks, margins = model.greedy(prompt, N_GEN, progress=progress,
                                 repeat_penalty=args.repeat_penalty,
                                 repeat_last_n=args.repeat_last_n)
    rec = {
        "model": "alpacca_amd.model.synthetic_llama_1b", "seed": SEED,
        "prompt_seed": PROMPT_SEED, "n_prompt": N_PROMPT, "n_gen": N_GEN,
        "n_ctx": N_PROMPT + N_GEN, "prefill_chunk": 256,
        "tokens": toks, "margins": [round(m, 6) for m in margins],
        "min_margin": round(min(margins), 6),
    }
    if penalized:
        rec["repeat_penalty"] = args.repeat_penalty
        rec["repeat_last_n"] = args.repeat_last_n
    out.write_text(json.dumps(rec, indent=0))
    print(f"wrote {out} in {time.time() - t0:.0f} s; min margin {min(margins):.3e}")


if __name__ == "__main__":
    main()
