"""The LastKV decoder restated in torch (test infrastructure only; see oracle/__init__.py).

Restates llm/src/lastkv/llm/modeling.py (the LastKV cache, attention, decoder layer, chunk loop
and greedy decoding) and llm/src/lastkv/llm/configuration.py (defaults and validation), with the
Llama building blocks the reference takes from transformers 4.57.6 (modeling.py:21-26) restated
from their definitions: RMSNorm, SiLU-gated MLP, neox RoPE (``rotate_half``) and the llama3
RoPE frequency rescaling.  ``reference_logits`` is a separate, cache-free transcription of the
chunk recurrence following the reference's own test (llm/tests/test_llm_inference.py:39-93).

Parameter names equal the reference's (419 tensors for the 8B geometry), so a state dict moves
between this oracle, the reference and ``lastkv_amd.llm`` unchanged.

Pinned by (tests/test_oracle_model_cpu.py):
  - RoPE tables, RMSNorm, MLP and apply-rotary against transformers' own Llama routines
    (library; the installed 5.15.0 keeps the same arithmetic as the pinned 4.57.6 for these);
  - cached inference (any segmentation, SDPA and eager) == ``reference_logits`` within the
    reference test's tolerance rtol 2e-5 / atol 2e-6, with its cache-shape invariants;
  - greedy generation == full-prefix replay; the 8B parameter layout (419 / 8,030,269,952);
  - with chunk >= sequence length the model is plain causal GQA attention (SDPA);
  - golden vectors written by importing the reference itself in this container
    (tests/golden/make_llm_golden.py) where that import works.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
from torch import nn
from torch.nn import functional as F

from . import reference_path


@dataclass
class Config:
    """LlamaConfig fields the model reads, with LlamaConfig's defaults, plus the LastKV fields."""

    vocab_size: int = 32000
    hidden_size: int = 4096
    intermediate_size: int = 11008
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int | None = None
    head_dim: int | None = None
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    rope_scaling: dict | None = None
    max_position_embeddings: int = 2048
    initializer_range: float = 0.02
    attention_bias: bool = False
    mlp_bias: bool = False
    pad_token_id: int | None = None
    tie_word_embeddings: bool = False
    # LastKV (configuration.py:13-24)
    chunk_size: int = 1024
    v_gap: int = 95
    use_qk_norm: bool = True
    use_nope: bool = False
    deep_kv_rescale: bool = True
    deep_rescale_mode: str = "v"
    deep_v_scale_init: float | list = 1.0
    deep_scale_frozen: bool = False
    attn_implementation: str = "sdpa"

    def __post_init__(self):
        if self.num_key_value_heads is None:
            self.num_key_value_heads = self.num_attention_heads
        if self.head_dim is None:
            self.head_dim = self.hidden_size // self.num_attention_heads
        # configuration.py:31-38
        if type(self.chunk_size) is not int or self.chunk_size < 1:
            raise ValueError("chunk_size must be a positive integer")
        if self.v_gap is None or self.v_gap < self.num_hidden_layers - 1:
            raise ValueError("This inference implementation requires final-layer KV reuse")
        if self.deep_rescale_mode != "v" or self.deep_scale_frozen:
            raise ValueError("The released checkpoints use learnable deep_rescale_mode='v'")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
        if self.attn_implementation not in ("sdpa", "eager"):
            self.attn_implementation = "sdpa"

    @classmethod
    def from_dict(cls, d: dict) -> "Config":
        known = {f for f in cls.__dataclass_fields__}
        kwargs = {k: v for k, v in d.items() if k in known}
        if "attn_implementation" in d and d["attn_implementation"] not in ("sdpa", "eager"):
            kwargs["attn_implementation"] = "sdpa"
        return cls(**kwargs)


# ----------------------------------------------------------------------------- Llama pieces
def rope_inv_freq(config: Config) -> tuple[torch.Tensor, float]:
    """Inverse frequencies and cos/sin scaling of the default and llama3 RoPE types.

    default: inv_freq_i = theta^(-2i/d).  llama3 (Llama 3.1 rescaling): with wavelength
    w_i = 2 pi / inv_freq_i, low = orig / low_freq_factor, high = orig / high_freq_factor:
    w_i > low -> inv_freq_i / factor; w_i < high -> inv_freq_i; otherwise interpolate with
    smooth = (orig / w_i - low_freq_factor) / (high_freq_factor - low_freq_factor):
    (1 - smooth) * inv_freq_i / factor + smooth * inv_freq_i.  attention scaling is 1.
    """

    dim = config.head_dim
    inv = 1.0 / (config.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.int64).float() / dim))
    scaling = config.rope_scaling or {}
    kind = scaling.get("rope_type", scaling.get("type", "default"))
    if kind == "default":
        return inv, 1.0
    if kind != "llama3":
        raise NotImplementedError(f"rope_type {kind}")
    factor = scaling["factor"]
    low_f, high_f = scaling["low_freq_factor"], scaling["high_freq_factor"]
    orig = scaling["original_max_position_embeddings"]
    low_wavelen, high_wavelen = orig / low_f, orig / high_f
    wavelen = 2 * math.pi / inv
    scaled = torch.where(wavelen > low_wavelen, inv / factor, inv)
    smooth = (orig / wavelen - low_f) / (high_f - low_f)
    smoothed = (1 - smooth) * scaled / factor + smooth * scaled
    medium = ~(wavelen < high_wavelen) & ~(wavelen > low_wavelen)
    return torch.where(medium, smoothed, scaled), 1.0


def rotary_cos_sin(inv_freq: torch.Tensor, scaling: float, positions: torch.Tensor, dtype: torch.dtype):
    """cos/sin [B, L, D] in ``dtype`` (fp32 math, then one cast), as LlamaRotaryEmbedding.forward."""

    inv = inv_freq.to(positions.device)
    freqs = positions[:, :, None].float() * inv[None, None, :].float()
    emb = torch.cat((freqs, freqs), dim=-1)
    return (emb.cos() * scaling).to(dtype), (emb.sin() * scaling).to(dtype)


def rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(q, k, cos, sin):
    """q/k [B, H, L, D], cos/sin [B, L, D] (unsqueezed on the head dim)."""

    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) in fp32, cast back, times the weight (in the weight's dtype)."""

    def __init__(self, size: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(size))
        self.variance_epsilon = eps

    def forward(self, x):
        dtype = x.dtype
        h = x.to(torch.float32)
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * h.to(dtype)


class MLP(nn.Module):
    def __init__(self, config: Config):
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=config.mlp_bias)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=config.mlp_bias)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=config.mlp_bias)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


# ----------------------------------------------------------------------------- LastKV
@dataclass
class Cache:
    """modeling.py:37-67: completed shared history plus per-layer previous/current chunks."""

    num_layers: int
    chunk_size: int
    seen_tokens: int = 0
    deep: tuple | None = None
    previous: list = field(default_factory=list)
    current: list = field(default_factory=list)

    def __post_init__(self):
        self.previous = [None] * self.num_layers
        self.current = [None] * self.num_layers

    def get_seq_length(self, layer_idx=0):
        return self.seen_tokens

    def reorder_cache(self, beam_idx):
        pick = lambda kv: None if kv is None else tuple(t.index_select(0, beam_idx.to(t.device)) for t in kv)
        self.deep = pick(self.deep)
        self.previous = [pick(kv) for kv in self.previous]
        self.current = [pick(kv) for kv in self.current]


def _concat(old, new):
    return new if old is None else tuple(torch.cat((a, b), dim=2) for a, b in zip(old, new))


class Attention(nn.Module):
    """modeling.py:70-148."""

    def __init__(self, config: Config, layer_idx: int):
        super().__init__()
        self.config, self.layer_idx = config, layer_idx
        H, Hkv, D = config.num_attention_heads, config.num_key_value_heads, config.head_dim
        self.q_proj = nn.Linear(config.hidden_size, H * D, bias=config.attention_bias)
        self.k_proj = nn.Linear(config.hidden_size, Hkv * D, bias=config.attention_bias)
        self.v_proj = nn.Linear(config.hidden_size, Hkv * D, bias=config.attention_bias)
        self.o_proj = nn.Linear(H * D, config.hidden_size, bias=config.attention_bias)
        self.prev_chunk_alphas = nn.Parameter(torch.zeros(Hkv))
        if config.deep_kv_rescale:
            init = config.deep_v_scale_init
            value = init[layer_idx] if isinstance(init, (list, tuple)) else init
            values = value if isinstance(value, (list, tuple)) else [value] * Hkv
            if len(values) != Hkv:
                raise ValueError("deep_v_scale_init must match the number of KV heads")
            self.deep_v_scale = nn.Parameter(torch.tensor(values, dtype=torch.float32))
        self.q_norm = RMSNorm(D, config.rms_norm_eps) if config.use_qk_norm else nn.Identity()
        self.k_norm = RMSNorm(D, config.rms_norm_eps) if config.use_qk_norm else nn.Identity()
        self.attn_compute_dtype: torch.dtype | None = None  # fp32 evaluation of the SDPA step

    def forward(self, hidden, position_embeddings, cache: Cache):
        c = self.config
        B, L, _ = hidden.shape
        q = self.q_proj(hidden).view(B, L, c.num_attention_heads, c.head_dim).transpose(1, 2)
        k = self.k_proj(hidden).view(B, L, c.num_key_value_heads, c.head_dim).transpose(1, 2)
        v = self.v_proj(hidden).view(B, L, c.num_key_value_heads, c.head_dim).transpose(1, 2)
        if not c.use_nope:
            q, k = apply_rope(q, k, *position_embeddings)
        q, k = self.q_norm(q), self.k_norm(k)
        current = _concat(cache.current[self.layer_idx], (k, v))
        cache.current[self.layer_idx] = current
        scale = self.deep_v_scale if c.deep_kv_rescale else torch.ones_like(self.prev_chunk_alphas)
        full_k, full_v = reference_path.compose(cache.deep, cache.previous[self.layer_idx], current,
                                                self.prev_chunk_alphas, scale, c.chunk_size)
        if c.attn_implementation == "eager":
            attended = _eager_attention(q, full_k, full_v, c.head_dim)
        else:
            attended = reference_path.sdpa_bottom_right(q, full_k, full_v, compute_dtype=self.attn_compute_dtype)
        return self.o_proj(attended.transpose(1, 2).reshape(B, L, -1))


def _eager_attention(q, full_k, full_v, head_dim):
    """modeling.py:131-141: repeat_interleave GQA, fp32 softmax cast back, bottom-right mask."""

    L, S = q.shape[2], full_k.shape[2]
    group = q.shape[1] // full_k.shape[1]
    k = full_k.repeat_interleave(group, dim=1)
    v = full_v.repeat_interleave(group, dim=1)
    scores = q @ k.transpose(-1, -2) * head_dim ** -0.5
    qpos = torch.arange(L, device=q.device) + S - L
    mask = torch.arange(S, device=q.device)[None, :] <= qpos[:, None]
    scores = scores.masked_fill(~mask, torch.finfo(scores.dtype).min)
    return F.softmax(scores, dim=-1, dtype=torch.float32).to(q.dtype) @ v


class DecoderLayer(nn.Module):
    def __init__(self, config: Config, layer_idx: int):
        super().__init__()
        self.self_attn = Attention(config, layer_idx)
        self.mlp = MLP(config)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(self, hidden, position_embeddings, cache):
        hidden = hidden + self.self_attn(self.input_layernorm(hidden), position_embeddings, cache)
        return hidden + self.mlp(self.post_attention_layernorm(hidden))


class Decoder(nn.Module):
    def __init__(self, config: Config):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, config.pad_token_id)
        self.layers = nn.ModuleList(DecoderLayer(config, i) for i in range(config.num_hidden_layers))
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        # kept out of the module's buffers so that casting the model to bf16 leaves it fp32
        # (on the CPU whatever the default device, so a model built on "meta" keeps real tables)
        with torch.device("cpu"):
            self.inv_freq, self.rope_scaling_factor = rope_inv_freq(config)

    def forward(self, input_ids, cache: Cache | None = None):
        """modeling.py:173-212 (input validation :175-193, chunk loop :196-208)."""

        hidden = self.embed_tokens(input_ids)
        B, L, _ = hidden.shape
        if not L:
            raise ValueError("At least one new token is required")
        if cache is not None and not isinstance(cache, Cache):
            raise TypeError("Use a LastKVCache returned by this model, not a standard Llama cache")
        cache = cache or Cache(len(self.layers), self.config.chunk_size)
        if cache.chunk_size != self.config.chunk_size or cache.num_layers != len(self.layers):
            raise ValueError("Cache architecture does not match this model")
        positions = torch.arange(cache.seen_tokens, cache.seen_tokens + L, device=hidden.device)[None, :]
        C = self.config.chunk_size
        outputs, start = [], 0
        while start < L:
            take = min(L - start, C - cache.seen_tokens % C)
            chunk = hidden[:, start:start + take]
            pe = rotary_cos_sin(self.inv_freq, self.rope_scaling_factor, positions[:, start:start + take], chunk.dtype)
            for layer in self.layers:
                chunk = layer(chunk, pe, cache)
            outputs.append(chunk)
            cache.seen_tokens += take
            if cache.seen_tokens % C == 0:
                cache.deep = _concat(cache.deep, cache.current[-1])
                cache.previous = cache.current
                cache.current = [None] * len(self.layers)
            start += take
        return self.norm(torch.cat(outputs, dim=1)), cache


class ForCausalLM(nn.Module):
    def __init__(self, config: Config):
        super().__init__()
        self.config = config
        self.model = Decoder(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def init_weights(self, generator: torch.Generator | None = None):
        """Reference init (modeling.py:228-236): N(0, initializer_range) Linear/Embedding, zero
        biases and padding row, unit norms; alphas stay 0 and scales at deep_v_scale_init."""

        std = self.config.initializer_range
        with torch.no_grad():
            for module in self.modules():
                if isinstance(module, (nn.Linear, nn.Embedding)):
                    module.weight.normal_(0.0, std, generator=generator)
                    if isinstance(module, nn.Linear) and module.bias is not None:
                        module.bias.zero_()
                    if isinstance(module, nn.Embedding) and module.padding_idx is not None:
                        module.weight[module.padding_idx].zero_()
                elif isinstance(module, RMSNorm):
                    module.weight.fill_(1.0)
        return self

    def set_attn_compute_dtype(self, dtype):
        for layer in self.model.layers:
            layer.self_attn.attn_compute_dtype = dtype

    def forward(self, input_ids, cache: Cache | None = None, logits_to_keep: int = 0):
        hidden, cache = self.model(input_ids, cache)
        return self.lm_head(hidden[:, -logits_to_keep:] if logits_to_keep else hidden), cache

    @torch.no_grad()
    def generate_greedy(self, prompt, steps: int, prefill_chunk: int | None = None):
        """Prefill the prompt (optionally in calls of ``prefill_chunk`` tokens), then ``steps``
        greedy tokens, feeding only new tokens (modeling.py:263-274); returns [B, steps] ids."""

        cache, start, L = None, 0, prompt.shape[1]
        step = prefill_chunk or L
        while start < L:
            logits, cache = self(prompt[:, start:start + step], cache, logits_to_keep=1)
            start += step
        out = []
        for _ in range(steps):
            token = logits[:, -1].argmax(-1, keepdim=True)
            out.append(token)
            logits, cache = self(token, cache, logits_to_keep=1)
        return torch.cat(out, dim=1)


@torch.no_grad()
def reference_logits(model: ForCausalLM, tokens: torch.Tensor) -> torch.Tensor:
    """Cache-free recomputation of the chunk recurrence (test_llm_inference.py:39-93).

    Each chunk is recomputed from the per-chunk history list: older chunks use the final layer's
    K and s-scaled V, the latest completed chunk blends final/own K/V, the current chunk uses its
    own K/V under a causal mask.  Uses no Cache and no compose(), only the model's weights.
    """

    dec, c = model.model, model.config
    B, L = tokens.shape
    histories, outputs = [], []
    for start in range(0, L, c.chunk_size):
        hidden = dec.embed_tokens(tokens[:, start:start + c.chunk_size])
        n = hidden.shape[1]
        pos = torch.arange(start, start + n, device=tokens.device)[None]
        cos, sin = rotary_cos_sin(dec.inv_freq, dec.rope_scaling_factor, pos, hidden.dtype)
        local = []
        for index, layer in enumerate(dec.layers):
            att = layer.self_attn
            x = layer.input_layernorm(hidden)
            q = att.q_proj(x).view(B, n, c.num_attention_heads, c.head_dim).transpose(1, 2)
            k = att.k_proj(x).view(B, n, c.num_key_value_heads, c.head_dim).transpose(1, 2)
            v = att.v_proj(x).view(B, n, c.num_key_value_heads, c.head_dim).transpose(1, 2)
            q, k = apply_rope(q, k, cos, sin)
            q, k = att.q_norm(q), att.k_norm(k)
            local.append((k, v))
            keys, values = [], []
            s = att.deep_v_scale.view(1, -1, 1, 1)
            a = att.prev_chunk_alphas.sigmoid().view(1, -1, 1, 1)
            for past_index, past in enumerate(histories):
                src_k, src_v = past[-1]
                if past_index == len(histories) - 1:
                    own_k, own_v = past[index]
                    src_k = a * src_k + (1 - a) * own_k
                    src_v = a * (src_v * s) + (1 - a) * own_v
                else:
                    src_v = src_v * s
                keys.append(src_k)
                values.append(src_v)
            keys.append(k)
            values.append(v)
            g = c.num_attention_heads // c.num_key_value_heads
            kk = torch.cat(keys, dim=2).repeat_interleave(g, dim=1)
            vv = torch.cat(values, dim=2).repeat_interleave(g, dim=1)
            scores = q @ kk.transpose(-1, -2) / math.sqrt(c.head_dim)
            masked = torch.arange(start + n, device=tokens.device)[None] > pos.T
            scores.masked_fill_(masked, torch.finfo(scores.dtype).min)
            probs = scores.float().softmax(-1).to(q.dtype)
            hidden = hidden + att.o_proj((probs @ vv).transpose(1, 2).reshape(B, n, -1))
            hidden = hidden + layer.mlp(layer.post_attention_layernorm(hidden))
        histories.append(local)
        outputs.append(hidden)
    return model.lm_head(dec.norm(torch.cat(outputs, dim=1)))


def tiny_config(attn_implementation: str = "sdpa") -> Config:
    """The reference test's tiny model (test_llm_inference.py:18-27)."""

    return Config(hidden_size=32, intermediate_size=48, num_attention_heads=4, num_key_value_heads=2,
                  num_hidden_layers=3, head_dim=8, vocab_size=71, chunk_size=4, max_position_embeddings=64,
                  pad_token_id=0, deep_v_scale_init=[[0.3, 0.7], [0.8, 1.2], [1.1, 0.9]], rope_theta=500000.0,
                  attn_implementation=attn_implementation)


def tiny_model(attn_implementation: str = "sdpa", seed: int = 19) -> ForCausalLM:
    """Tiny model with the reference test's non-trivial alphas and norm gains (:28-36)."""

    torch.manual_seed(seed)
    model = ForCausalLM(tiny_config(attn_implementation)).init_weights().eval()
    with torch.no_grad():
        for i, layer in enumerate(model.model.layers):
            layer.self_attn.prev_chunk_alphas.copy_(torch.tensor([-1.2 + i * 0.2, 0.8 - i * 0.3]))
            layer.self_attn.q_norm.weight.copy_(torch.linspace(0.7, 1.3, 8))
            layer.self_attn.k_norm.weight.copy_(torch.linspace(1.2, 0.8, 8))
    return model


def config_8b(**overrides) -> Config:
    """The released 8B geometry (llm/train/configs/8B/lastkv_8B_reusekv.json)."""

    base = dict(hidden_size=4096, intermediate_size=14336, num_attention_heads=32, num_key_value_heads=8,
                num_hidden_layers=32, head_dim=128, vocab_size=128256, rms_norm_eps=1e-5, rope_theta=500000.0,
                max_position_embeddings=8192, chunk_size=1024,
                rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                              "original_max_position_embeddings": 8192})
    base.update(overrides)
    return Config(**base)
