"""LastKV decoder on MI355X: the reference's module interface with the attention path on HIP kernels.

Mirrors llm/src/lastkv/llm/modeling.py.  ``LastKVAttention.forward(hidden_states,
position_embeddings, cache)`` keeps the reference signature and parameter names
(``q_proj/k_proj/v_proj/o_proj/prev_chunk_alphas/deep_v_scale/q_norm/k_norm``, :78-91) so state
dicts move unchanged; its body replaces :103-146 (RoPE, q/k norm, append, region composition,
mask and SDPA) with two C-ABI calls: ``lkv_qkv_epilogue`` and ``lkv_decode_attn`` (one new token)
or ``lkv_prefill_attn`` (several).  The decoder's chunk loop (:196-208) is unchanged except that
the boundary commit blends every layer's finished chunk once (``lkv_blend_chunk``) instead of
re-blending it at every later step.  Projections, norms, MLP, embeddings and lm_head stay torch
ops in the reference's order.  The model runs in bf16 on the GPU; there is no CPU path.
"""

from __future__ import annotations

import json
import math
import pathlib
from dataclasses import dataclass

import torch
from torch import nn
from torch.nn import functional as F

from .. import ops
from .cache import LastKVCache
from .configuration import CustomRecurrentMarinAKV254ReuseKVConfig


class RMSNorm(nn.Module):
    """transformers LlamaRMSNorm: fp32 normalisation, cast back, times the weight."""

    def __init__(self, size: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(size))
        self.variance_epsilon = eps

    def forward(self, x):
        dtype = x.dtype
        h = x.to(torch.float32)
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * h.to(dtype)


class LlamaMLP(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=config.mlp_bias)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=config.mlp_bias)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=config.mlp_bias)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


def rope_inv_freq(config) -> tuple[torch.Tensor, float]:
    """Default and llama3 RoPE inverse frequencies (transformers' rope init functions)."""

    dim = config.head_dim
    inv = 1.0 / (config.rope_theta ** (torch.arange(0, dim, 2, dtype=torch.int64).float() / dim))
    scaling = config.rope_scaling or {}
    kind = scaling.get("rope_type", scaling.get("type", "default"))
    if kind == "default":
        return inv, 1.0
    if kind != "llama3":
        raise NotImplementedError(f"rope_type {kind!r} is not supported")
    factor, lo, hi = scaling["factor"], scaling["low_freq_factor"], scaling["high_freq_factor"]
    orig = scaling["original_max_position_embeddings"]
    wavelen = 2 * math.pi / inv
    scaled = torch.where(wavelen > orig / lo, inv / factor, inv)
    smooth = (orig / wavelen - lo) / (hi - lo)
    smoothed = (1 - smooth) * scaled / factor + smooth * scaled
    medium = ~(wavelen < orig / hi) & ~(wavelen > orig / lo)
    return torch.where(medium, smoothed, scaled), 1.0


class LastKVAttention(nn.Module):
    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_dim = config.head_dim
        self.num_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        H, Hkv, D = self.num_heads, self.num_key_value_heads, self.head_dim
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
        self._vscale_key = None
        self._vscale = None

    def blend_params(self, dtype=torch.bfloat16) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]:
        """(alpha, 1 - alpha, s) exactly as the reference's ops produce them in ``dtype``
        (modeling.py:96, :117), carried as fp32."""

        alpha = self.prev_chunk_alphas.sigmoid().to(dtype)
        om = (1 - alpha).to(dtype)
        s = self.deep_v_scale.to(dtype).float() if self.config.deep_kv_rescale else None
        return alpha.float(), om.float(), s

    def _older_vscale(self) -> torch.Tensor | None:
        if not self.config.deep_kv_rescale:
            return None
        p = self.deep_v_scale
        key = (p.data_ptr(), p._version, p.dtype)
        if key != self._vscale_key:
            self._vscale = p.detach().to(torch.bfloat16).float().contiguous()
            self._vscale_key = key
        return self._vscale

    def forward(self, hidden_states, position_embeddings, cache: LastKVCache):
        c = self.config
        B, L, _ = hidden_states.shape
        H, Hkv, D = self.num_heads, self.num_key_value_heads, self.head_dim
        if D != ops.HEAD_DIM:
            raise ValueError(f"the MI355X kernels support head_dim {ops.HEAD_DIM}, not {D}")
        q = self.q_proj(hidden_states)
        k = self.k_proj(hidden_states)
        v = self.v_proj(hidden_states)
        cos, sin = position_embeddings
        if c.use_nope:
            cos, sin = torch.ones_like(cos), torch.zeros_like(sin)
        p0 = cache.seen_tokens
        # a cache driven by the reference's own decoder loop: allocate on first use, run this
        # layer's boundary blend scheduled by its `cache.previous = ...` (modeling.py:203-207)
        cache.reserve(B, Hkv, hidden_states.device, p0 + L)
        if cache._pending[self.layer_idx] is not None:
            cache.commit_layer(self.layer_idx, self.blend_params())
        cache.check_layer(self.layer_idx, p0, L)
        ring = cache.ring(self.layer_idx)
        last = self.layer_idx == cache.num_layers - 1
        qn = ops.qkv_epilogue(
            q, k, v, cos, sin, num_q_heads=H, num_kv_heads=Hkv,
            q_norm_weight=self.q_norm.weight if c.use_qk_norm else None,
            k_norm_weight=self.k_norm.weight if c.use_qk_norm else None,
            eps=c.rms_norm_eps, positions=p0, ring=ring, deep=cache.store if last else None,
        )
        C = c.chunk_size
        cur = (p0 + L - 1) // C * C
        rec = max(0, cur - C)
        segments = dict(older=cache.store, older_len=rec, vscale=self._older_vscale(), local=ring,
                        local_len=p0 + L - rec, local_start=rec % cache.ring_tokens)
        if L == 1:
            out = ops.decode_attention(qn.view(B, H, D), **segments)
        else:
            # (room for the tile kernel's key splits, which calls of few query tiles take)
            ws = cache.prefill_workspace(ops.prefill_workspace_bytes(B, Hkv, rec, p0 + L - rec, rec % ops.BLOCK_TOKENS,
                                                                     query_rows=B * L, num_q_heads=H))
            out = ops.prefill_attention(qn, causal=True, workspace=ws, **segments)
        return self.o_proj(out.reshape(B, L, H * D))


class LastKVDecoderLayer(nn.Module):
    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.self_attn = LastKVAttention(config, layer_idx)
        self.mlp = LlamaMLP(config)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)

    def forward(self, hidden_states, position_embeddings, cache):
        hidden_states = hidden_states + self.self_attn(self.input_layernorm(hidden_states), position_embeddings, cache)
        return hidden_states + self.mlp(self.post_attention_layernorm(hidden_states))


class CustomRecurrentMarinAKV254ReuseKVModel(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, config.pad_token_id)
        self.layers = nn.ModuleList(LastKVDecoderLayer(config, i) for i in range(config.num_hidden_layers))
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        # fp32 and outside the module's buffers: casting the model to bf16 must not round it
        # (on the CPU whatever the default device: from_pretrained builds the modules on "meta")
        with torch.device("cpu"):
            self.inv_freq, self.rope_attention_scaling = rope_inv_freq(config)
        self._inv_freq_dev: dict[torch.device, torch.Tensor] = {}
        self._blend_key = None
        self._blend = None

    def rotary(self, positions: torch.Tensor, dtype: torch.dtype):
        """cos/sin [B, L, D] as LlamaRotaryEmbedding.forward: fp32 math, one cast."""

        inv = self._inv_freq_dev.get(positions.device)
        if inv is None:
            inv = self._inv_freq_dev.setdefault(positions.device, self.inv_freq.to(positions.device))
        freqs = positions[:, :, None].float() * inv[None, None, :].float()
        emb = torch.cat((freqs, freqs), dim=-1)
        s = self.rope_attention_scaling
        return (emb.cos() * s).to(dtype), (emb.sin() * s).to(dtype)

    def _blend_params(self):
        key = tuple((l.self_attn.prev_chunk_alphas._version, l.self_attn.prev_chunk_alphas.data_ptr()) for l in self.layers)
        if key != self._blend_key:
            parts = [l.self_attn.blend_params() for l in self.layers]
            alpha = torch.cat([p[0] for p in parts]).contiguous()
            om = torch.cat([p[1] for p in parts]).contiguous()
            s = torch.cat([p[2] for p in parts]).contiguous() if self.config.deep_kv_rescale else None
            self._blend = (alpha, om, s)
            self._blend_key = key
        return self._blend

    def _commit_chunk(self, cache: LastKVCache, batch: int):
        """Boundary commit (modeling.py:203-207): the chunk just completed becomes every layer's
        recent region, materialised once as alpha * shared + (1 - alpha) * own, for all layers in
        one launch."""

        cache.commit_all(self._blend_params())

    def forward(self, input_ids=None, inputs_embeds=None, attention_mask=None, position_ids=None,
                past_key_values=None, use_cache=True):
        """modeling.py:173-212."""

        if (input_ids is None) == (inputs_embeds is None):
            raise ValueError("Provide exactly one of input_ids or inputs_embeds")
        if attention_mask is not None and not bool(torch.all(attention_mask != 0)):
            raise ValueError("LastKV supports unpadded sequences; generate each padded prompt separately")
        hidden = self.embed_tokens(input_ids) if inputs_embeds is None else inputs_embeds
        batch, length, _ = hidden.shape
        if not length:
            raise ValueError("At least one new token is required")
        if past_key_values is not None and not isinstance(past_key_values, LastKVCache):
            raise TypeError("Use a LastKVCache returned by this model, not a standard Llama cache")
        cache = past_key_values or LastKVCache(len(self.layers), self.config.chunk_size)
        if cache.chunk_size != self.config.chunk_size or cache.num_layers != len(self.layers):
            raise ValueError("Cache architecture does not match this model")
        if not hidden.is_cuda or hidden.dtype != torch.bfloat16:
            raise ValueError("the MI355X LastKV model runs in bfloat16 on the GPU")
        if position_ids is None:
            position_ids = torch.arange(cache.seen_tokens, cache.seen_tokens + length, device=hidden.device)[None, :]
        elif position_ids.ndim == 1:
            position_ids = position_ids[None, :]
        if position_ids.shape[-1] != length or position_ids.shape[0] not in (1, batch):
            raise ValueError("position_ids must describe the new input tokens")
        cache.reserve(batch, self.config.num_key_value_heads, hidden.device, cache.seen_tokens + length)
        C = self.config.chunk_size
        outputs, start = [], 0
        while start < length:
            take = min(length - start, C - cache.seen_tokens % C)
            chunk = hidden[:, start:start + take]
            positions = self.rotary(position_ids[:, start:start + take], chunk.dtype)
            for layer in self.layers:
                chunk = layer(chunk, positions, cache)
            outputs.append(chunk)
            cache.seen_tokens += take
            if cache.seen_tokens % C == 0:
                self._commit_chunk(cache, batch)
            start += take
        return self.norm(torch.cat(outputs, dim=1) if len(outputs) > 1 else outputs[0]), (cache if use_cache else None)


@dataclass
class CausalLMOutput:
    logits: torch.Tensor
    past_key_values: LastKVCache | None


@dataclass
class GenerationConfig:
    """The fields of transformers' ``GenerationConfig`` that greedy generation reads (its
    defaults; token ids from the model config, as ``GenerationConfig.from_model_config``)."""

    max_length: int = 20
    max_new_tokens: int | None = None
    do_sample: bool = False
    use_cache: bool = True
    bos_token_id: int | None = None
    eos_token_id: int | list | None = None
    pad_token_id: int | None = None


class CustomRecurrentMarinAKV254ReuseKVForCausalLM(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.config = config
        self.generation_config = GenerationConfig(bos_token_id=config.bos_token_id, eos_token_id=config.eos_token_id,
                                                  pad_token_id=config.pad_token_id)
        self.model = CustomRecurrentMarinAKV254ReuseKVModel(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def init_weights(self, generator: torch.Generator | None = None):
        """Reference initialisation (modeling.py:228-236)."""

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

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                inputs_embeds=None, use_cache=True, logits_to_keep=0, labels=None,
                output_attentions=False, output_hidden_states=False, **kwargs):
        """modeling.py:276-293."""

        if labels is not None or output_attentions or output_hidden_states:
            raise ValueError("This release provides inference logits and a KV cache only")
        if kwargs.get("cu_seqlens") is not None:
            raise ValueError("Packed-document inputs are unsupported; process each document separately")
        hidden, cache = self.model(input_ids=input_ids, inputs_embeds=inputs_embeds, attention_mask=attention_mask,
                                   position_ids=position_ids, past_key_values=past_key_values, use_cache=use_cache)
        index = slice(-logits_to_keep, None) if isinstance(logits_to_keep, int) else logits_to_keep
        return CausalLMOutput(logits=self.lm_head(hidden[:, index]), past_key_values=cache)

    @torch.no_grad()
    def generate(self, input_ids=None, max_new_tokens: int | None = None, *, attention_mask=None, do_sample=None,
                 use_cache=None, pad_token_id=None, eos_token_id=None, max_length=None,
                 prefill_chunk: int | None = None, cache=None, **kwargs):
        """Greedy decoding with the semantics of transformers' ``GenerationMixin.generate`` as the
        reference calls it (llm/examples/generate.py:30-33: ``generate(**inputs, max_new_tokens=..,
        do_sample=False, use_cache=True, pad_token_id=..)``, modeling.py:263-274): only new tokens
        are fed (``use_cache=True``) or the whole sequence is recomputed every step
        (``use_cache=False``), ``logits_to_keep=1``, argmax; a sequence that emits an EOS id is
        continued with ``pad_token_id`` and generation stops once every sequence has finished
        or ``max_new_tokens`` (else ``max_length`` in total) is reached.  ``attention_mask`` must
        be all ones (LastKV takes unpadded prompts).  The prompt is prefilled in calls of
        ``prefill_chunk`` tokens (default: one call).  Returns the [B, prompt + new] ids."""

        gc = self.generation_config
        if kwargs:
            raise ValueError(f"The following generation arguments are not supported: {sorted(kwargs)}")
        if input_ids is None:
            raise ValueError("generate needs input_ids")
        if do_sample if do_sample is not None else gc.do_sample:
            raise ValueError("LastKV generation on MI355X is greedy only (do_sample=False)")
        use_cache = gc.use_cache if use_cache is None else bool(use_cache)
        L = input_ids.shape[1]
        if max_new_tokens is None:
            max_new_tokens = gc.max_new_tokens
        if max_new_tokens is None:
            max_new_tokens = (gc.max_length if max_length is None else max_length) - L
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be positive")
        eos = gc.eos_token_id if eos_token_id is None else eos_token_id
        eos = [] if eos is None else ([eos] if isinstance(eos, int) else list(eos))
        pad = gc.pad_token_id if pad_token_id is None else pad_token_id
        if pad is None and eos:
            pad = eos[0]
        eos_ids = torch.tensor(eos, dtype=input_ids.dtype, device=input_ids.device)

        if attention_mask is not None and not bool(torch.all(attention_mask != 0)):
            raise ValueError("LastKV supports unpadded sequences; generate each padded prompt separately")

        def run(ids, cache):
            step = prefill_chunk or ids.shape[1]
            start, out = 0, None
            while start < ids.shape[1]:
                out = self(ids[:, start:start + step], past_key_values=cache, logits_to_keep=1)
                cache = out.past_key_values
                start += step
            return out

        out = run(input_ids, cache if use_cache else None)
        cache = out.past_key_values if use_cache else None
        sequence = input_ids
        unfinished = torch.ones(input_ids.shape[0], dtype=torch.bool, device=input_ids.device)
        for i in range(max_new_tokens):
            token = out.logits[:, -1].argmax(-1).to(input_ids.dtype)
            if eos:
                token = torch.where(unfinished, token, torch.full_like(token, pad))
                unfinished &= ~torch.isin(token, eos_ids)
            sequence = torch.cat((sequence, token[:, None]), dim=1)
            if i + 1 == max_new_tokens or (eos and not bool(unfinished.any())):
                break
            if use_cache:
                out = self(token[:, None], past_key_values=cache, logits_to_keep=1)
                cache = out.past_key_values
            else:
                out = run(sequence, None)
        return sequence

    @classmethod
    def from_pretrained(cls, path, *, dtype=torch.bfloat16, device="cuda"):
        """Strict local load of a config.json + safetensors checkpoint (single file or sharded
        index), modeling.py:242-249: any missing, unexpected or mis-shaped tensor raises."""

        from safetensors import safe_open

        path = pathlib.Path(path)
        config = CustomRecurrentMarinAKV254ReuseKVConfig.from_pretrained(path)
        with torch.device("meta"):
            model = cls(config)
        model = model.to_empty(device=device)
        expected = model.state_dict()
        index = path / "model.safetensors.index.json"
        files = sorted(set(json.loads(index.read_text())["weight_map"].values())) if index.exists() else ["model.safetensors"]
        seen, problems = set(), {}
        for name in files:
            with safe_open(str(path / name), framework="pt", device="cpu") as f:
                for key in f.keys():
                    if key not in expected:
                        problems.setdefault("unexpected_keys", []).append(key)
                        continue
                    t = f.get_tensor(key)
                    if tuple(t.shape) != tuple(expected[key].shape):
                        problems.setdefault("mismatched_keys", []).append(key)
                        continue
                    with torch.no_grad():
                        expected[key].copy_(t.to(expected[key].dtype))
                    seen.add(key)
        missing = sorted(set(expected) - seen)
        if missing:
            problems["missing_keys"] = missing
        if problems:
            raise ValueError(f"Checkpoint is not a strict LastKV model match: {problems}")
        return model.to(dtype).eval()


ATTENTION_BACKENDS = ("sdpa", "eager")


def load_model(model_name_or_path="ZefanCai/LastKV-LLM-8B-Base", *, revision=None, device="cuda",
               dtype=torch.bfloat16, attention_backend="sdpa"):
    """Strictly load a LastKV checkpoint for cached inference (llm/src/lastkv/llm/__init__.py:13-26).

    Same keywords as the reference.  ``model_name_or_path`` must be a local checkpoint directory:
    this build has no hub access, so a hub name raises ``ValueError`` (as does a ``revision`` of
    one); for a local directory ``revision`` is ignored, as transformers ignores it there.
    ``attention_backend`` 'sdpa' and 'eager' both select the HIP attention kernels (the
    reference's two backends compute the same attention); anything else raises ``ValueError``.
    The model runs in bfloat16 on the GPU; other devices or dtypes raise ``ValueError``."""

    if attention_backend not in ATTENTION_BACKENDS:
        raise ValueError("attention_backend must be 'sdpa' or 'eager'")
    path = pathlib.Path(model_name_or_path)
    if not (path / "config.json").is_file():
        rev = f" at revision {revision!r}" if revision not in (None, "main") else ""
        raise ValueError(f"{str(model_name_or_path)!r}{rev} is not a local LastKV checkpoint directory (config.json "
                         "missing); this build loads local checkpoints only, download the revision first")
    if torch.device(device).type != "cuda":
        raise ValueError("the MI355X LastKV model runs on the GPU (device='cuda')")
    if dtype != torch.bfloat16:
        raise ValueError("the MI355X LastKV model runs in bfloat16")
    model = CustomRecurrentMarinAKV254ReuseKVForCausalLM.from_pretrained(path, dtype=dtype, device=device)
    model.config._attn_implementation = attention_backend
    model.config.use_cache = True
    model.generation_config.use_cache = True
    return model.eval()
