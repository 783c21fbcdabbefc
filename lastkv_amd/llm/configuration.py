"""Configuration of the LastKV decoder (mirror of llm/src/lastkv/llm/configuration.py:10-48).

Field names and defaults follow the reference config class, a transformers LlamaConfig
subclass; the LlamaConfig defaults the model reads are restated here so the package does not
depend on a particular transformers release.
"""

from __future__ import annotations

import json
import pathlib
from dataclasses import asdict, dataclass, field, fields


@dataclass
class CustomRecurrentMarinAKV254ReuseKVConfig:
    vocab_size: int = 32000
    hidden_size: int = 4096
    intermediate_size: int = 11008
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int | None = None
    head_dim: int | None = None
    hidden_act: str = "silu"
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    rope_scaling: dict | None = None
    max_position_embeddings: int = 2048
    initializer_range: float = 0.02
    attention_bias: bool = False
    mlp_bias: bool = False
    pad_token_id: int | None = None
    bos_token_id: int | None = 1
    eos_token_id: int | list | None = 2
    tie_word_embeddings: bool = False
    use_cache: bool = True
    # LastKV (configuration.py:13-24)
    chunk_size: int = 1024
    v_gap: int = 95
    use_qk_norm: bool = True
    use_nope: bool = False
    deep_kv_rescale: bool = True
    deep_rescale_mode: str = "v"
    deep_v_scale_init: float | list = 1.0
    deep_scale_frozen: bool = False
    architectures: list = field(default_factory=lambda: ["CustomRecurrentMarinAKV254ReuseKVForCausalLM"])
    model_type: str = "custom_recurrent_marin_akv254_reusekv"

    def __post_init__(self):
        if self.num_key_value_heads is None:
            self.num_key_value_heads = self.num_attention_heads
        if self.head_dim is None:
            self.head_dim = self.hidden_size // self.num_attention_heads
        if self.rope_scaling is not None and "rope_theta" in self.rope_scaling:
            self.rope_theta = self.rope_scaling["rope_theta"]
        if type(self.chunk_size) is not int or self.chunk_size < 1:
            raise ValueError("chunk_size must be a positive integer")
        if self.v_gap is None or self.v_gap < self.num_hidden_layers - 1:
            raise ValueError("This inference implementation requires final-layer KV reuse")
        if self.deep_rescale_mode != "v" or self.deep_scale_frozen:
            raise ValueError("The released checkpoints use learnable deep_rescale_mode='v'")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
        if self.hidden_act not in ("silu", "swish"):
            raise ValueError(f"hidden_act {self.hidden_act!r} is not supported")

    @classmethod
    def from_dict(cls, d: dict) -> "CustomRecurrentMarinAKV254ReuseKVConfig":
        known = {f.name for f in fields(cls)}
        kw = {k: v for k, v in d.items() if k in known}
        # transformers >= 5 stores RoPE settings as rope_parameters
        params = d.get("rope_parameters")
        if isinstance(params, dict):
            kw.setdefault("rope_theta", params.get("rope_theta", kw.get("rope_theta", 10000.0)))
            if params.get("rope_type", "default") != "default":
                kw.setdefault("rope_scaling", params)
        return cls(**kw)

    @classmethod
    def from_pretrained(cls, path) -> "CustomRecurrentMarinAKV254ReuseKVConfig":
        return cls.from_dict(json.loads((pathlib.Path(path) / "config.json").read_text()))

    def to_dict(self) -> dict:
        return asdict(self)


LastKVConfig = CustomRecurrentMarinAKV254ReuseKVConfig
