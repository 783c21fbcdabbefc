"""Pins the oracle LastKV model (oracle/model.py) on the CPU, following the reference's own tests
(llm/tests/test_llm_inference.py) plus library and degenerate-case checks."""

from __future__ import annotations

import pytest
import torch
from torch.nn import functional as F

from oracle import model as M

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig  # noqa: E402
from transformers.models.llama import modeling_llama as hf  # noqa: E402


def _hf_config(**kw):
    return LlamaConfig(**kw)


# ------------------------------------------------------------------ Llama pieces vs the library
@pytest.mark.parametrize("scaling", [None, {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                                            "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}])
def test_rope_tables_match_transformers(scaling):
    cfg = M.Config(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
                   num_hidden_layers=2, rope_theta=500000.0, rope_scaling=scaling, max_position_embeddings=8192)
    kw = dict(hidden_size=4096, num_attention_heads=32, num_key_value_heads=8, head_dim=128,
              max_position_embeddings=8192)
    if scaling is None:
        kw["rope_theta"] = 500000.0
    else:
        kw["rope_parameters"] = dict(scaling, rope_theta=500000.0)
    hcfg = _hf_config(**kw)
    if scaling is None:
        hcfg.rope_parameters = {"rope_type": "default", "rope_theta": 500000.0}
    rot = hf.LlamaRotaryEmbedding(hcfg)
    inv, sc = M.rope_inv_freq(cfg)
    assert torch.equal(inv, rot.inv_freq.float()) and sc == rot.attention_scaling
    pos = torch.tensor([[0, 1, 7, 1000, 8191, 131071]])
    x = torch.zeros(1, 6, 8, dtype=torch.bfloat16)
    cos, sin = rot(x, pos)
    mcos, msin = M.rotary_cos_sin(inv, sc, pos, torch.bfloat16)
    assert torch.equal(cos, mcos) and torch.equal(sin, msin)


def test_apply_rope_rmsnorm_and_mlp_match_transformers():
    torch.manual_seed(0)
    q = torch.randn(2, 4, 5, 16).bfloat16()
    k = torch.randn(2, 2, 5, 16).bfloat16()
    cos = torch.randn(2, 5, 16).bfloat16()
    sin = torch.randn(2, 5, 16).bfloat16()
    a = M.apply_rope(q, k, cos, sin)
    b = hf.apply_rotary_pos_emb(q, k, cos, sin)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    x = torch.randn(3, 7, 16).bfloat16()
    ours, theirs = M.RMSNorm(16, 1e-5), hf.LlamaRMSNorm(16, eps=1e-5)
    with torch.no_grad():
        ours.weight.copy_(torch.linspace(0.5, 1.5, 16))
        theirs.weight.copy_(torch.linspace(0.5, 1.5, 16))
    ours, theirs = ours.bfloat16(), theirs.bfloat16()
    assert torch.equal(ours(x), theirs(x))
    cfg = M.Config(hidden_size=16, intermediate_size=24, num_attention_heads=2, num_hidden_layers=1)
    mlp, hmlp = M.MLP(cfg), hf.LlamaMLP(_hf_config(hidden_size=16, intermediate_size=24, num_attention_heads=2))
    hmlp.load_state_dict(mlp.state_dict())
    xf = torch.randn(3, 16)
    assert torch.equal(mlp(xf), hmlp(xf))


# ------------------------------------------------------------------ the reference's own tests
@pytest.mark.parametrize("backend", ["sdpa", "eager"])
def test_full_prefill_matches_chunk_recurrence(backend):
    model = M.tiny_model(backend)
    tokens = torch.randint(3, 71, (2, 15), generator=torch.Generator().manual_seed(1))
    with torch.inference_mode():
        actual, _ = model(tokens)
        expected = M.reference_logits(model, tokens)
    torch.testing.assert_close(actual, expected, rtol=2e-5, atol=2e-6)


@pytest.mark.parametrize("segments", [[1] * 15, [3, 2, 7, 3], [4, 4, 4, 3], [9, 6]])
def test_incremental_decoding_matches_reference_across_boundaries(segments):
    model = M.tiny_model()
    tokens = torch.randint(3, 71, (1, sum(segments)), generator=torch.Generator().manual_seed(2))
    cache, start, logits = None, 0, []
    with torch.inference_mode():
        expected = M.reference_logits(model, tokens)
        for size in segments:
            out, cache = model(tokens[:, start:start + size], cache)
            logits.append(out)
            start += size
            assert cache.get_seq_length() == start
            assert cache.deep is None or cache.deep[0].shape[2] == start // 4 * 4
            assert all(kv is None or kv[0].shape[2] == start % 4 for kv in cache.current)
            assert all(kv is None or kv[0].shape[2] == 4 for kv in cache.previous)
    torch.testing.assert_close(torch.cat(logits, dim=1), expected, rtol=2e-5, atol=2e-6)


def test_generate_matches_full_prefix_replay():
    model = M.tiny_model()
    prompt = torch.tensor([[1, 5, 17]])
    replay = prompt.clone()
    with torch.inference_mode():
        generated = model.generate_greedy(prompt, 10)
        for _ in range(10):
            logits = M.reference_logits(model, replay)
            replay = torch.cat((replay, logits[:, -1].argmax(-1, keepdim=True)), dim=1)
    assert torch.equal(generated, replay[:, 3:])


def test_published_8b_parameter_layout_without_allocating_weights():
    with torch.device("meta"):
        model = M.ForCausalLM(M.config_8b())
    state = model.state_dict()
    assert len(state) == 419
    assert sum(t.numel() for t in state.values()) == 8_030_269_952
    assert state["model.layers.31.self_attn.prev_chunk_alphas"].shape == (8,)
    assert state["model.layers.0.self_attn.deep_v_scale"].shape == (8,)
    assert state["model.layers.0.self_attn.q_norm.weight"].shape == (128,)
    assert state["lm_head.weight"].shape == (128256, 4096)


def test_cache_reorder_and_rejections():
    model = M.tiny_model()
    tokens = torch.randint(3, 71, (2, 7), generator=torch.Generator().manual_seed(3))
    order = torch.tensor([1, 0])
    with torch.inference_mode():
        _, cache = model(tokens[:, :5])
        cache.reorder_cache(order)
        actual, _ = model(tokens[order, 5:], cache)
        expected = M.reference_logits(model, tokens[order])[:, 5:]
    torch.testing.assert_close(actual, expected, rtol=2e-5, atol=2e-6)
    with pytest.raises(ValueError, match="Cache architecture"):
        model(tokens[:1], M.Cache(3, 5))
    with pytest.raises(TypeError):
        model(tokens[:1], object())
    with pytest.raises(ValueError, match="chunk_size"):
        M.Config(chunk_size=0)


# ------------------------------------------------------------------ degenerate case
def test_chunk_longer_than_sequence_is_plain_causal_gqa():
    """With C >= length no chunk completes: each layer is standard Llama attention with
    post-RoPE q/k RMSNorm, i.e. one causal GQA SDPA call per layer."""

    torch.manual_seed(4)
    cfg = M.tiny_config()
    cfg.chunk_size = 64
    model = M.ForCausalLM(cfg).init_weights().eval()
    tokens = torch.randint(3, 71, (2, 13))
    with torch.inference_mode():
        got, cache = model(tokens)
        assert cache.deep is None
        dec = model.model
        h = dec.embed_tokens(tokens)
        cos, sin = M.rotary_cos_sin(dec.inv_freq, 1.0, torch.arange(13)[None], h.dtype)
        for layer in dec.layers:
            att = layer.self_attn
            x = layer.input_layernorm(h)
            q = att.q_proj(x).view(2, 13, 4, 8).transpose(1, 2)
            k = att.k_proj(x).view(2, 13, 2, 8).transpose(1, 2)
            v = att.v_proj(x).view(2, 13, 2, 8).transpose(1, 2)
            q, k = hf.apply_rotary_pos_emb(q, k, cos, sin)
            q, k = att.q_norm(q), att.k_norm(k)
            o = F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
            h = h + att.o_proj(o.transpose(1, 2).reshape(2, 13, -1))
            h = h + layer.mlp(layer.post_attention_layernorm(h))
        want = model.lm_head(dec.norm(h))
    torch.testing.assert_close(got, want, rtol=2e-5, atol=2e-6)


# ------------------------------------------------------------------ BASELINE config 1 (plumbing)
@pytest.mark.parametrize("chunk", [1024, 32])
def test_config1_124m_greedy_64_steps_matches_full_prefix_replay(chunk):
    """124M-shape, fp32, CPU: 12 layers, d_model 768, 12 heads (= kv heads), head_dim 64,
    vocab 50304, FFN 2048 (SwiGLU-equivalent of a 4x MLP), weights N(0, 0.02) seed 0, prompt of
    128 uniform ids (Generator seed 1), 64 greedy steps.  C = 1024 crosses no boundary; C = 32
    exercises the shared and blended regions.  Each generated id must equal the argmax of a
    cache-free replay of the whole sequence."""

    torch.manual_seed(0)
    cfg = M.Config(hidden_size=768, intermediate_size=2048, num_attention_heads=12, num_key_value_heads=12,
                   num_hidden_layers=12, head_dim=64, vocab_size=50304, chunk_size=chunk,
                   max_position_embeddings=1024)
    model = M.ForCausalLM(cfg).init_weights(torch.Generator().manual_seed(0)).eval()
    prompt = torch.randint(0, 50304, (1, 128), generator=torch.Generator().manual_seed(1))
    with torch.inference_mode():
        ids = model.generate_greedy(prompt, 64)
        full = torch.cat((prompt, ids), dim=1)
        replay = M.reference_logits(model, full)[:, 127:-1].argmax(-1)
    assert torch.equal(ids, replay)
