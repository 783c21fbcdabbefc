"""The decisive test model (tests/decisive_model.py) gives its closed-form greedy ids on the oracle
model in fp32 and in bf16 on the CPU, with wide logit margins; its lookups land in both the older
shared segment and the local ring, so the ids depend on the region semantics."""

from __future__ import annotations

import torch

import decisive_model as DM
from oracle import model as M


def test_closed_form_ids_on_the_oracle_model():
    cfg = M.config_8b(hidden_size=768, intermediate_size=1024, num_attention_heads=4, num_key_value_heads=2,
                      num_hidden_layers=3, vocab_size=1024, chunk_size=32)
    model, tables = DM.build(cfg, 100, seed=3)
    prompt = DM.prompts(tables, 2)
    want = DM.expected_ids(tables, prompt, 20, 32)
    with torch.no_grad():
        got = model.generate_greedy(prompt, 20, prefill_chunk=40)
        logits, _ = model(torch.cat([prompt, got], 1)[:, :-1])
        got16 = model.to(torch.bfloat16).generate_greedy(prompt, 20, prefill_chunk=40)
    assert torch.equal(got, want) and torch.equal(got16, want)
    top = logits[:, 99:].topk(2, -1).values
    assert (top[..., 0] - top[..., 1]).min() > 5.0
    sigma, row = tables["sigma"], prompt[0].tolist()
    where = {t: i for i, t in enumerate(row)}
    older = [where[int(sigma[t])] < max(0, (99 + n) // 32 * 32 - 32) for n, t in enumerate([row[-1]] + want[0, :-1].tolist())]
    assert any(older) and not all(older)
