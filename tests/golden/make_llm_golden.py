"""Write golden vectors of the reference LastKV LLM (llm/src) for tests/test_golden_llm.py.

Imports the reference package from /root/reference/llm/src in the container that holds it (the
GPU box does not), builds the reference test's tiny model (llm/tests/test_llm_inference.py:18-36,
seed 19), and stores: its weights, a token batch, the reference's full-prefill logits, the
logits of an incremental segmentation, and 10 greedy ids from a prompt.  Records the
transformers version the reference ran under.  Usage: python tests/golden/make_llm_golden.py
"""

from __future__ import annotations

import json
import pathlib
import sys

import torch
from safetensors.torch import save_file

sys.path.insert(0, "/root/reference/llm/src")

import transformers  # noqa: E402
from lastkv.llm import CustomRecurrentMarinAKV254ReuseKVConfig as Config  # noqa: E402
from lastkv.llm import CustomRecurrentMarinAKV254ReuseKVForCausalLM as Model  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent


def tiny_model(backend="sdpa"):
    torch.manual_seed(19)
    config = Config(
        hidden_size=32, intermediate_size=48, num_attention_heads=4, num_key_value_heads=2, num_hidden_layers=3,
        head_dim=8, vocab_size=71, chunk_size=4, max_position_embeddings=64, bos_token_id=1, eos_token_id=None,
        pad_token_id=0, deep_v_scale_init=[[0.3, 0.7], [0.8, 1.2], [1.1, 0.9]], rope_theta=500000.0,
        attn_implementation=backend,
    )
    model = Model(config).eval()
    with torch.no_grad():
        for i, layer in enumerate(model.model.layers):
            layer.self_attn.prev_chunk_alphas.copy_(torch.tensor([-1.2 + i * 0.2, 0.8 - i * 0.3]))
            layer.self_attn.q_norm.weight.copy_(torch.linspace(0.7, 1.3, config.head_dim))
            layer.self_attn.k_norm.weight.copy_(torch.linspace(1.2, 0.8, config.head_dim))
    return model


def main():
    model = tiny_model()
    tokens = torch.randint(3, 71, (2, 15), generator=torch.Generator().manual_seed(123))
    segments = [3, 2, 7, 3]
    with torch.inference_mode():
        full = model(tokens, use_cache=False).logits
        cache, start, parts = None, 0, []
        for size in segments:
            result = model(tokens[:, start:start + size], past_key_values=cache, use_cache=True)
            parts.append(result.logits)
            cache = result.past_key_values
            start += size
        incremental = torch.cat(parts, dim=1)
        prompt = torch.tensor([[1, 5, 17]])
        generated = model.generate(prompt, max_new_tokens=10, do_sample=False, use_cache=True)
    state = {k: v.contiguous() for k, v in model.state_dict().items()}
    save_file(state, str(OUT / "tiny_llm_weights.safetensors"))
    save_file({"tokens": tokens, "full_logits": full.contiguous(), "incremental_logits": incremental.contiguous(),
               "prompt": prompt, "generated": generated}, str(OUT / "tiny_llm_vectors.safetensors"))
    meta = {"reference": "llm/src/lastkv/llm (Zefan-Cai/LastKV)", "transformers": transformers.__version__,
            "torch": torch.__version__, "segments": segments, "model": "llm/tests/test_llm_inference.py:18-36",
            "tokens_generator_seed": 123}
    (OUT / "tiny_llm_meta.json").write_text(json.dumps(meta, indent=1) + "\n")
    print(json.dumps(meta))


if __name__ == "__main__":
    main()
