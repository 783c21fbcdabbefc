"""Module-level drop-in: the reference's own decoder loop driving lastkv_amd's attention module and
cache (GPU).

``oracle/model.py`` restates the reference decoder (llm/src/lastkv/llm/modeling.py): its chunk loop
assigns ``cache.deep = _append(cache.deep, cache.current[-1])``, ``cache.previous =
cache.current`` and ``cache.current = [None] * L`` at every boundary (:203-207).  With
``lastkv_amd.llm.LastKVAttention`` substituted in every layer (the reference's parameter names,
loaded from the oracle's state dict) and ``lastkv_amd.llm.LastKVCache`` as the cache, that loop
must give the logits of ``lastkv_amd``'s own model bit for bit, across chunk boundaries and for
any segmentation of the calls, and leave the cache fields with the reference test's shapes
(llm/tests/test_llm_inference.py:118-121).
"""

from __future__ import annotations

import pytest
import torch

from lastkv_amd.llm import LastKVAttention, LastKVCache
from oracle import model as M

from test_gpu_llm import _tiny

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _reference_loop_with_swapped_modules(oracle, ours, monkeypatch):
    for i, layer in enumerate(oracle.model.layers):
        att = LastKVAttention(ours.config, i).to(DEV, torch.bfloat16).eval()
        att.load_state_dict(layer.self_attn.state_dict(), strict=True)
        layer.self_attn = att
    # the restated decoder checks isinstance(cache, Cache) and builds Cache(L, C) itself
    monkeypatch.setattr(M, "Cache", LastKVCache)
    return oracle


@pytest.mark.parametrize("chunk,pieces", [(4, [5, 1, 1, 7, 2, 1, 3, 3, 1, 1]), (32, [40, 1, 23, 1, 1, 64, 2]),
                                          (16, [1] * 40)])
def test_reference_decoder_loop_with_swapped_attention_and_cache(chunk, pieces, monkeypatch):
    oracle, ours = _tiny(chunk=chunk)
    ref = _reference_loop_with_swapped_modules(oracle, ours, monkeypatch)
    total = sum(pieces)
    ids = torch.randint(3, 97, (2, total), generator=torch.Generator().manual_seed(chunk)).to(DEV)
    rcache = ocache = None
    start = 0
    with torch.inference_mode():
        for n in pieces:
            mine = ours(ids[:, start:start + n], past_key_values=ocache)
            ocache = mine.past_key_values
            got, rcache = ref(ids[:, start:start + n], rcache)
            assert isinstance(rcache, LastKVCache)
            assert torch.equal(got, mine.logits), f"chunk {chunk}: call at position {start} (+{n}) differs"
            start += n
            s = rcache.seen_tokens
            assert s == start == ocache.seen_tokens
            assert rcache.deep is None if s < chunk else rcache.deep[0].shape[2] == s // chunk * chunk
            assert all(kv is None or kv[0].shape[2] == s % chunk for kv in rcache.current)
            assert all(kv is None or kv[0].shape[2] == chunk for kv in rcache.previous)
        # the shared history and the recent chunks the two caches hold are the same
        for a, b in zip(rcache.deep, ocache.deep):
            assert torch.equal(a, b)
        for l in range(ours.config.num_hidden_layers):
            for a, b in zip(rcache.previous[l], ocache.previous[l]):
                assert torch.equal(a, b)
    print(f"chunk {chunk}: {len(pieces)} calls, {total} tokens bit-identical", flush=True)


def test_cache_assignments_with_foreign_tensors(monkeypatch):
    """The boundary assignments with copies instead of the cache's own read-backs (the tensors are
    written into the cache) and the error when a completed chunk is never committed."""

    oracle, ours = _tiny(chunk=8)
    ids = torch.randint(3, 97, (2, 21), generator=torch.Generator().manual_seed(4)).to(DEV)
    with torch.inference_mode():
        want = ours(ids).logits
        # drive the model's layers by hand through a boundary with cloned fields
        cache = LastKVCache(ours.config.num_hidden_layers, 8)
        inner = ours.model
        hidden = inner.embed_tokens(ids)
        outs = []
        for start, n in ((0, 8), (8, 8), (16, 5)):
            chunk = hidden[:, start:start + n]
            pe = inner.rotary(torch.arange(start, start + n, device=DEV)[None], chunk.dtype)
            for layer in inner.layers:
                chunk = layer(chunk, pe, cache)
            outs.append(chunk)
            cache.seen_tokens += n
            if cache.seen_tokens % 8 == 0:
                cur = [tuple(t.clone() for t in kv) for kv in cache.current]
                deep = cache.deep
                cache.deep = cur[-1] if deep is None else tuple(torch.cat((a, b.clone()), 2) for a, b in zip(deep, cur[-1]))
                cache.previous = cur
                cache.current = [None] * len(cur)
        got = ours.lm_head(inner.norm(torch.cat(outs, 1)))
        assert torch.equal(got, want)
        # a boundary passed without a commit is refused at the next attention call
        cache2 = LastKVCache(ours.config.num_hidden_layers, 8)
        chunk = hidden[:, :8]
        pe = inner.rotary(torch.arange(0, 8, device=DEV)[None], chunk.dtype)
        for layer in inner.layers:
            chunk = layer(chunk, pe, cache2)
        cache2.seen_tokens = 8
        pe = inner.rotary(torch.arange(8, 9, device=DEV)[None], chunk.dtype)
        with pytest.raises(RuntimeError, match="committed"):
            inner.layers[0](hidden[:, 8:9], pe, cache2)
