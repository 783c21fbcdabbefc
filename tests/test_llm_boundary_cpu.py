"""The HF-boundary entry points reject what the MI355X build cannot honour, with the reference's
error types, before touching a GPU (llm/src/lastkv/llm/__init__.py:13-26,
llm/examples/generate.py:27-33)."""

from __future__ import annotations

import json

import pytest
import torch

from lastkv_amd.llm import LastKVConfig, load_model
from lastkv_amd.llm.modeling import CustomRecurrentMarinAKV254ReuseKVForCausalLM, GenerationConfig


def _checkpoint_dir(tmp_path):
    cfg = LastKVConfig(hidden_size=256, intermediate_size=384, num_attention_heads=4, num_key_value_heads=2,
                       num_hidden_layers=2, head_dim=128, vocab_size=97, chunk_size=4)
    (tmp_path / "config.json").write_text(json.dumps(cfg.to_dict()))
    return tmp_path


def test_load_model_rejects_unknown_attention_backend(tmp_path):
    with pytest.raises(ValueError, match="attention_backend must be 'sdpa' or 'eager'"):
        load_model(str(_checkpoint_dir(tmp_path)), attention_backend="flash_attention_2")


def test_load_model_needs_a_local_checkpoint(tmp_path):
    with pytest.raises(ValueError, match="local LastKV checkpoint"):
        load_model("ZefanCai/LastKV-LLM-8B-Base", revision="256k-step-001209", device="cuda")
    with pytest.raises(ValueError, match="256k-step-001209"):
        load_model(str(tmp_path / "missing"), revision="256k-step-001209")


@pytest.mark.parametrize("kw,message", [(dict(device="cpu"), "GPU"), (dict(dtype=torch.float32), "bfloat16")])
def test_load_model_rejects_cpu_and_fp32(tmp_path, kw, message):
    args = dict(revision="main", device="cuda", dtype=torch.bfloat16, attention_backend="eager")
    args.update(kw)
    with pytest.raises(ValueError, match=message):
        load_model(str(_checkpoint_dir(tmp_path)), **args)


def test_generation_config_from_model_config():
    cfg = LastKVConfig(hidden_size=256, intermediate_size=384, num_attention_heads=4, num_key_value_heads=2,
                       num_hidden_layers=2, head_dim=128, vocab_size=97, chunk_size=4, eos_token_id=7, pad_token_id=0)
    with torch.device("meta"):
        model = CustomRecurrentMarinAKV254ReuseKVForCausalLM(cfg)
    assert model.generation_config == GenerationConfig(bos_token_id=1, eos_token_id=7, pad_token_id=0)
    ids = torch.zeros((1, 3), dtype=torch.long)
    with pytest.raises(ValueError, match="greedy only"):
        model.generate(ids, max_new_tokens=4, do_sample=True)
    with pytest.raises(ValueError, match="not supported"):
        model.generate(ids, max_new_tokens=4, num_beams=4)
    with pytest.raises(ValueError, match="unpadded"):
        model.generate(ids, max_new_tokens=4, attention_mask=torch.tensor([[0, 1, 1]]))


def test_model_built_on_meta_keeps_real_rope_tables():
    """from_pretrained builds the modules on the meta device; the RoPE inverse frequencies are not
    parameters, so they must still be real (CPU) tensors afterwards."""

    from lastkv_amd.llm.modeling import rope_inv_freq

    cfg = LastKVConfig(hidden_size=256, intermediate_size=384, num_attention_heads=4, num_key_value_heads=2,
                       num_hidden_layers=2, head_dim=128, vocab_size=97, chunk_size=4)
    with torch.device("meta"):
        model = CustomRecurrentMarinAKV254ReuseKVForCausalLM(cfg)
    assert model.model.inv_freq.device.type == "cpu"
    assert torch.equal(model.model.inv_freq, rope_inv_freq(cfg)[0])
