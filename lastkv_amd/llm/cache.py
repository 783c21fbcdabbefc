"""LastKVCache: the shared last-layer history and per-layer rings, preallocated in HBM.

Counterpart of llm/src/lastkv/llm/modeling.py:37-67.  The reference keeps ``deep`` (final-layer
K/V of completed chunks), ``previous[l]`` and ``current[l]`` as tensors grown with torch.cat on
every append.  Here they live in tiled buffers (see include/lastkv_amd.h) written in place:

  deep store  [B, Hkv, capacity / 32, 4096] x (K, V)   final layer's K/V at every position
                                                        (written by its QKV epilogue)
  rings       [L, B, Hkv, R / 32, 4096] x (K, V)         per layer, token p at ring slot p mod R,
                                                        R = ring_tokens_for_chunk(C) >= 2C

At a chunk boundary the model blends each layer's just-completed chunk with the shared chunk in
place (lkv_blend_chunk), so the ring's previous chunk holds exactly the recent-region K/V the
layer attends to.  The observable fields ``seen_tokens``, ``deep``, ``previous``, ``current``,
``get_seq_length()`` and ``reorder_cache()`` keep the reference's shapes; ``deep`` / ``previous``
/ ``current`` return [B, Hkv, T, D] copies read back from the tiled buffers (inspection only).
``previous[l]`` is the blended recent chunk, which is what the reference's serving path also
keeps (it blends in place, vllm/.../rmarin_flashinfer/batching.py:1099-1155); the HF
reference instead keeps the layer's raw chunk and re-blends it at every step.
"""

from __future__ import annotations

import torch

from .. import ops


class LastKVCache:
    def __init__(self, num_layers: int, chunk_size: int, *, capacity_tokens: int | None = None):
        if num_layers < 1 or chunk_size < 1:
            raise ValueError("num_layers and chunk_size must be positive")
        self.num_layers = num_layers
        self.chunk_size = chunk_size
        self.seen_tokens = 0
        self.ring_tokens = ops.ring_tokens_for_chunk(chunk_size)
        self._initial_capacity = capacity_tokens
        self._store: ops.TiledKV | None = None
        self._ring_k: torch.Tensor | None = None
        self._ring_v: torch.Tensor | None = None
        self._workspace: torch.Tensor | None = None

    # ------------------------------------------------------------------ storage
    @property
    def allocated(self) -> bool:
        return self._store is not None

    @property
    def batch(self) -> int:
        return 0 if self._store is None else self._store.slots

    @property
    def capacity_tokens(self) -> int:
        return 0 if self._store is None else self._store.capacity_tokens

    def reserve(self, batch: int, kv_heads: int, device: torch.device, tokens: int) -> None:
        """Allocate on first use and grow the shared store to hold ``tokens`` positions."""

        if self._store is None:
            cap = max(tokens, self._initial_capacity or 0, self.chunk_size)
            cap = -(-cap // ops.BLOCK_TOKENS) * ops.BLOCK_TOKENS
            self._store = ops.TiledKV.zeros(batch, kv_heads, cap, device)
            shape = (self.num_layers, batch, kv_heads, self.ring_tokens // ops.BLOCK_TOKENS, ops.BLOCK_ELEMS)
            self._ring_k = torch.zeros(shape, dtype=torch.bfloat16, device=device)
            self._ring_v = torch.zeros(shape, dtype=torch.bfloat16, device=device)
            return
        if batch != self._store.slots or kv_heads != self._store.heads:
            raise ValueError("Cache batch / head geometry does not match this input")
        if self._store.device != torch.device(device) and str(device) != str(self._store.device):
            raise ValueError("Cache lives on another device")
        if tokens > self._store.capacity_tokens:
            cap = max(tokens, 2 * self._store.capacity_tokens)
            cap = -(-cap // ops.BLOCK_TOKENS) * ops.BLOCK_TOKENS
            old = self._store
            new = ops.TiledKV.zeros(old.slots, old.heads, cap, old.device)
            new.k[:, :, : old.blocks].copy_(old.k)
            new.v[:, :, : old.blocks].copy_(old.v)
            self._store = new

    @property
    def store(self) -> ops.TiledKV:
        """Shared last-layer K/V (older region source)."""

        if self._store is None:
            raise RuntimeError("cache is not allocated yet")
        return self._store

    def ring(self, layer: int) -> ops.TiledKV:
        return ops.TiledKV(self._ring_k[layer], self._ring_v[layer])

    def prefill_workspace(self, nbytes: int) -> torch.Tensor:
        """Scratch for the prefill kernel's fp16 V copy, shared by all layers and grown on demand
        (each layer's call has finished with it before the next layer's call runs on the stream)."""

        if self._store is None:
            raise RuntimeError("cache is not allocated yet")
        if self._workspace is None or self._workspace.numel() < nbytes:
            self._workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=self._store.device)
        return self._workspace

    @property
    def ring_k(self) -> torch.Tensor:
        return self._ring_k

    @property
    def ring_v(self) -> torch.Tensor:
        return self._ring_v

    # ------------------------------------------------------------------ reference interface
    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.seen_tokens

    def _ring_range(self, layer: int, start: int, length: int):
        ring = self.ring(layer)
        R = self.ring_tokens
        first = min(length, R - start % R)
        k, v = ops.unpack_kv(ring, start % R, first)
        if first < length:
            k2, v2 = ops.unpack_kv(ring, 0, length - first)
            k, v = torch.cat((k, k2), 2), torch.cat((v, v2), 2)
        return k, v

    @property
    def deep(self):
        done = self.seen_tokens // self.chunk_size * self.chunk_size
        if self._store is None or done == 0:
            return None
        return ops.unpack_kv(self._store, 0, done)

    @property
    def previous(self):
        C = self.chunk_size
        if self._store is None or self.seen_tokens < C:
            return [None] * self.num_layers
        start = (self.seen_tokens // C - 1) * C
        return [self._ring_range(layer, start, C) for layer in range(self.num_layers)]

    @property
    def current(self):
        C = self.chunk_size
        n = self.seen_tokens % C
        if self._store is None or n == 0:
            return [None] * self.num_layers
        start = self.seen_tokens - n
        return [self._ring_range(layer, start, n) for layer in range(self.num_layers)]

    def reorder_cache(self, beam_idx: torch.Tensor) -> None:
        """Select sequences (beam search), modeling.py:59-67."""

        if self._store is None:
            return
        idx = beam_idx.to(self._store.device)
        self._store = ops.TiledKV(self._store.k.index_select(0, idx).contiguous(), self._store.v.index_select(0, idx).contiguous())
        self._ring_k = self._ring_k.index_select(1, idx).contiguous()
        self._ring_v = self._ring_v.index_select(1, idx).contiguous()
