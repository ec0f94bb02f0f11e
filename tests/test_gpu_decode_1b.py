"""Greedy-token parity on the synthetic Llama-3.2-1B-shaped model of
benchmark config 5: the device-resident decode (graph-replayed steps) must
produce exactly the oracle's 256 tokens after a 2048-token prompt.

The expected tokens are the committed trace tests/golden/decode_1b_greedy.json,
written on the CPU by tests/golden/make_decode_1b.py with oracle/model_ref.py
(which prefills the prompt in chunks of 256 as the reference does,
model.py:610-641); the model weights and prompt are regenerated here from the
same seeds.  decode_1b_greedy_penalty.json is the same with the reference
benchmark's selection (tests/bench.py:78-90: repetition penalty 1.1 over the
last 64 accepted tokens).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "decode_1b_greedy.json"
GOLDEN_PENALTY = GOLDEN.with_name("decode_1b_greedy_penalty.json")
TRACES = [GOLDEN, GOLDEN_PENALTY]


@pytest.mark.parametrize("path", TRACES, ids=["argmax", "penalty"])
def test_golden_trace_is_consistent(path):
    """CPU: the committed trace matches the recipe the GPU test regenerates."""
    g = json.loads(path.read_text())
    assert g["n_prompt"] == 2048 and g["n_gen"] == 256 == len(g["tokens"])
    assert len(g["margins"]) == 256 and min(g["margins"]) >= 0
    assert all(0 <= t < 128256 for t in g["tokens"])
    assert len(set(g["tokens"])) > 8  # a non-degenerate random model


@pytest.fixture(scope="module")
def model_1b():
    from alpacca_amd.model import Model, synthetic_llama_1b
    g = json.loads(GOLDEN.read_text())
    print("building the synthetic 1B model", flush=True)
    hp, tensors = synthetic_llama_1b(seed=g["seed"])
    model = Model(hp, tensors, n_ctx=g["n_ctx"])
    del tensors
    return model


@pytest.mark.gpu
@pytest.mark.parametrize("path", TRACES, ids=["argmax", "penalty"])
def test_greedy_tokens_match_oracle_1b(model_1b, path):
    g = json.loads(path.read_text())
    prompt = [int(t) for t in
              np.random.default_rng(g["prompt_seed"]).integers(0, model_1b.hp.n_vocab,
                                                                g["n_prompt"])]
    print(f"generating ({path.name})", flush=True)
    toks = model_1b.generate_greedy(prompt, g["n_gen"], graph=True,
                                    repeat_penalty=g.get("repeat_penalty", 1.0),
                                    repeat_last_n=g.get("repeat_last_n", 64))
    first_diff = next((i for i, (a, b) in enumerate(zip(toks, g["tokens"])) if a != b), None)
    assert first_diff is None, (
        f"first mismatch at step {first_diff}: got {toks[first_diff]}, oracle "
        f"{g['tokens'][first_diff]} (oracle top-1/top-2 margin {g['margins'][first_diff]})")
