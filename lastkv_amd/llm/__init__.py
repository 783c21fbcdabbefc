"""LastKV LLM on MI355X: drop-in counterpart of ``lastkv.llm`` (llm/src/lastkv/llm/__init__.py)."""

from .cache import LastKVCache
from .configuration import CustomRecurrentMarinAKV254ReuseKVConfig, LastKVConfig
from .modeling import (
    CustomRecurrentMarinAKV254ReuseKVForCausalLM,
    CustomRecurrentMarinAKV254ReuseKVModel,
    LastKVAttention,
    LastKVDecoderLayer,
    load_model,
)

__all__ = [
    "CustomRecurrentMarinAKV254ReuseKVConfig",
    "CustomRecurrentMarinAKV254ReuseKVForCausalLM",
    "CustomRecurrentMarinAKV254ReuseKVModel",
    "LastKVAttention",
    "LastKVCache",
    "LastKVConfig",
    "LastKVDecoderLayer",
    "load_model",
]
