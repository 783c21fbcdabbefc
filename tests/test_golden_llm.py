"""The oracle model reproduces golden vectors written by the reference itself.

tests/golden/make_llm_golden.py ran the reference LastKV LLM (llm/src, under the transformers
version recorded in tiny_llm_meta.json) on the reference test's tiny model; here the oracle
(oracle/model.py) loads the same weights and must reproduce its full-prefill logits, the logits
of an incremental segmentation across chunk boundaries, and its greedy ids, within the
reference test's tolerance (rtol 2e-5, atol 2e-6; llm/tests/test_llm_inference.py:103)."""

from __future__ import annotations

import json
import pathlib

import torch
from safetensors.torch import load_file

from oracle import model as M

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _load():
    model = M.ForCausalLM(M.tiny_config()).eval()
    state = load_file(str(GOLDEN / "tiny_llm_weights.safetensors"))
    missing, unexpected = model.load_state_dict(state, strict=True), None
    return model, load_file(str(GOLDEN / "tiny_llm_vectors.safetensors"))


def test_golden_state_dict_is_a_strict_match():
    model = M.ForCausalLM(M.tiny_config())
    state = load_file(str(GOLDEN / "tiny_llm_weights.safetensors"))
    assert sorted(state) == sorted(model.state_dict())
    model.load_state_dict(state, strict=True)


def test_oracle_reproduces_reference_logits_and_greedy_ids():
    model, vec = _load()
    meta = json.loads((GOLDEN / "tiny_llm_meta.json").read_text())
    tokens = vec["tokens"]
    with torch.inference_mode():
        full, _ = model(tokens)
        torch.testing.assert_close(full, vec["full_logits"], rtol=2e-5, atol=2e-6)
        torch.testing.assert_close(M.reference_logits(model, tokens), vec["full_logits"], rtol=2e-5, atol=2e-6)
        cache, start, parts = None, 0, []
        for size in meta["segments"]:
            out, cache = model(tokens[:, start:start + size], cache)
            parts.append(out)
            start += size
        torch.testing.assert_close(torch.cat(parts, 1), vec["incremental_logits"], rtol=2e-5, atol=2e-6)
        prompt = vec["prompt"]
        ids = model.generate_greedy(prompt, 10)
    assert torch.equal(torch.cat((prompt, ids), 1), vec["generated"])
