"""LastKVCache: the shared last-layer history and per-layer rings, preallocated in HBM.

Counterpart of llm/src/lastkv/llm/modeling.py:37-67.  The reference keeps ``deep`` (final-layer
K/V of completed chunks), ``previous[l]`` and ``current[l]`` as tensors grown with torch.cat on
every append.  Here they live in tiled buffers (see include/lastkv_amd.h) written in place:

  deep store  [B, Hkv, capacity / 32, 4096] x (K, V)   final layer's K/V at every position
                                                        (written by its QKV epilogue)
  rings       [L, B, Hkv, R / 32, 4096] x (K, V)         per layer, token p at ring slot p mod R,
                                                        R = ring_tokens_for_chunk(C) >= 2C

At a chunk boundary each layer's just-completed chunk is blended in place with the shared chunk
(lkv_blend_chunk), so the ring's previous chunk holds exactly the recent-region K/V the layer
attends to.

The reference's fields keep their shapes and can be read and assigned as the reference's decoder
does at a boundary (modeling.py:203-207: ``cache.deep = _append(cache.deep, cache.current[-1])``,
``cache.previous = cache.current``, ``cache.current = [None] * L``):
  - ``deep``: (K, V) [B, Hkv, D, 128] of the D committed tokens (a copy read back); assigning
    (K, V) writes tokens [0, D) of the shared store and commits D;
  - ``current``: per layer (K, V) of the tokens since the last commit (lazy: a layer's tensors are
    read back when indexed); assigning ``[None] * L`` starts a new chunk;
  - ``previous``: per layer (K, V) of the chunk before the committed end; assigning it (e.g. the
    ``current`` view of the chunk just completed, or tensors of C tokens) schedules that layer's
    blend, which runs at the layer's next attention call (or ``commit()``); read back, a layer's
    chunk is the blended one once that has run (the reference's serving path also blends in place,
    vllm/.../rmarin_flashinfer/batching.py:1099-1155; its HF path keeps the raw chunk and
    re-blends it at every step).
``LastKVAttention.forward`` allocates (``reserve``) on first use and checks that every completed
chunk has been committed.  The model's own chunk loop commits all layers at once (``commit_all``).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from .. import ops


class _RingRange(Sequence):
    """Layer l's (K, V) ``[B, Hkv, n, 128]`` at ring positions ``[start, start + n)`` of a cache,
    read back when indexed (``None`` when n is 0 or nothing is allocated)."""

    def __init__(self, cache: "LastKVCache", start: int, n: int):
        self.cache, self.start, self.n = cache, start, n

    def __len__(self) -> int:
        return self.cache.num_layers

    def __getitem__(self, index):
        if isinstance(index, slice):
            return [self[i] for i in range(*index.indices(len(self)))]
        layer = range(len(self))[index]
        if self.n == 0 or not self.cache.allocated:
            return None
        k, v = self.cache._ring_range(layer, self.start, self.n)
        k._lkv_ring = v._lkv_ring = (id(self.cache), layer, self.start, self.n)
        return k, v

    def __setitem__(self, index, value):
        raise TypeError("assign the whole per-layer list (cache.current = [...]), not one layer of it")


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
        self._deep_len = 0  # committed tokens (the reference's deep length)
        self._cur_start = 0  # current holds positions [_cur_start, seen_tokens)
        self._prev_start: int | None = None  # previous holds [_prev_start, _prev_start + C)
        # per layer: None, or a scheduled blend of the chunk before the committed end, carrying the
        # (K, V) to write there first (None: the ring already holds that layer's raw chunk)
        self._pending: list = [None] * num_layers
        self._blended = [0] * num_layers  # committed end through which each layer's chunk is blended

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

    # ------------------------------------------------------------------ chunk commits
    def commit_all(self, blend: tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]) -> None:
        """The boundary commit at ``seen_tokens`` (a multiple of C) for every layer in one launch:
        the chunk just completed becomes each layer's recent region, blended in place as
        alpha * shared + (1 - alpha) * own; ``blend`` = (alpha, 1 - alpha, s) fp32 ``[L * Hkv]``."""

        C = self.chunk_size
        if self.seen_tokens % C or self.seen_tokens == 0:
            raise ValueError(f"a commit needs a chunk boundary, not position {self.seen_tokens}")
        alpha, om, s = blend
        ops.blend_chunk(self._ring_k, self._ring_v, self.store, batch=self.batch, chunk_start=self.seen_tokens - C,
                        chunk_len=C, alpha=alpha, one_minus_alpha=om, vscale=s)
        self._deep_len = self._cur_start = self.seen_tokens
        self._prev_start = self.seen_tokens - C
        self._pending = [None] * self.num_layers
        self._blended = [self.seen_tokens] * self.num_layers

    def commit_layer(self, layer: int, blend: tuple[torch.Tensor, torch.Tensor, torch.Tensor | None]) -> None:
        """Run ``layer``'s scheduled blend, if any (``blend`` = that layer's (alpha, 1 - alpha, s)
        fp32 ``[Hkv]``): write the assigned previous chunk into the ring unless it already holds
        it, then blend it with the shared store's last committed chunk."""

        job = self._pending[layer]
        if job is None:
            return
        C, D = self.chunk_size, self._deep_len
        if D < C:
            raise ValueError("cache.previous was set but cache.deep holds no completed chunk to blend it with")
        if self._prev_start is not None and self._prev_start != D - C:
            raise ValueError(f"cache.previous holds positions [{self._prev_start}, {self._prev_start + C}) but the "
                             f"shared history ends at {D}: it must be the chunk [{D - C}, {D})")
        if job is not True:  # tensors to place first
            k, v = job
            self._write_ring(layer, D - C, k, v)
        alpha, om, s = blend
        ring = self._ring_k[layer:layer + 1], self._ring_v[layer:layer + 1]
        ops.blend_chunk(*ring, self.store, batch=self.batch, chunk_start=D - C, chunk_len=C, alpha=alpha,
                        one_minus_alpha=om, vscale=s)
        self._pending[layer] = None
        self._blended[layer] = D
        self._prev_start = D - C

    def check_layer(self, layer: int, position: int, tokens: int) -> None:
        """Raise unless the state matches an attention call of ``tokens`` new tokens at
        ``position``: every completed chunk committed, and the layer's recent chunk blended."""

        C = self.chunk_size
        cur = (position + tokens - 1) // C * C
        if self._deep_len != cur:
            raise RuntimeError(f"LastKVCache: tokens [{position}, {position + tokens}) need the shared history "
                               f"committed through {cur}, but cache.deep holds {self._deep_len} tokens (commit each "
                               "completed chunk: cache.deep / cache.previous / cache.current, modeling.py:203-207)")
        if cur >= C and self._blended[layer] != cur:
            raise RuntimeError(f"LastKVCache: layer {layer}'s recent chunk [{cur - C}, {cur}) is not blended "
                               "(assign cache.previous at the boundary)")

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

    def _write_ring(self, layer: int, start: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Ring positions [start, start + n) of ``layer`` := (k, v) ``[B, Hkv, n, 128]``."""

        n = k.shape[2]
        if tuple(k.shape) != tuple(v.shape) or k.shape[0] != self.batch or k.shape[1] != self.store.heads:
            raise ValueError(f"K/V for the ring must be [{self.batch}, {self.store.heads}, n, 128]")
        if n > self.ring_tokens:
            raise ValueError("more tokens than the ring holds")
        ring, R = self.ring(layer), self.ring_tokens
        first = min(n, R - start % R)
        k, v = k.to(self.store.device, torch.bfloat16), v.to(self.store.device, torch.bfloat16)
        ops.pack_kv(k[:, :, :first], v[:, :, :first], ring, token0=start % R)
        if first < n:
            ops.pack_kv(k[:, :, first:], v[:, :, first:], ring, token0=0)

    def _holds(self, kv, layer: int, start: int, n: int) -> bool:
        """Whether (k, v) are this cache's own read-back of ``layer``'s ring positions [start, start + n)."""

        tag = (id(self), layer, start, n)
        return kv is not None and all(getattr(t, "_lkv_ring", None) == tag for t in kv)

    @property
    def deep(self):
        if self._store is None or self._deep_len == 0:
            return None
        return ops.unpack_kv(self._store, 0, self._deep_len)

    @deep.setter
    def deep(self, value) -> None:
        if value is None:
            self._deep_len = 0
            return
        k, v = value
        n = k.shape[2]
        if n % self.chunk_size or n > self.seen_tokens:
            raise ValueError(f"cache.deep must hold whole chunks of the {self.seen_tokens} seen tokens, got {n}")
        if self._store is None:
            self.reserve(k.shape[0], k.shape[1], k.device, n)
        self.reserve(self.batch, self.store.heads, self.store.device, n)
        ops.pack_kv(k.to(self.store.device, torch.bfloat16), v.to(self.store.device, torch.bfloat16), self.store)
        self._deep_len = n

    @property
    def previous(self):
        if self._prev_start is None:
            return [None] * self.num_layers
        return _RingRange(self, self._prev_start, self.chunk_size)

    @previous.setter
    def previous(self, value) -> None:
        C = self.chunk_size
        items = list(value) if not isinstance(value, _RingRange) else None
        if items is not None and len(items) != self.num_layers:
            raise ValueError(f"cache.previous needs one entry per layer ({self.num_layers})")
        if isinstance(value, _RingRange) and value.cache is self:
            if value.n != C:
                raise ValueError(f"cache.previous must be a whole chunk of {C} tokens, got {value.n}")
            self._prev_start = value.start
            self._pending = [True] * self.num_layers
            return
        if all(kv is None for kv in items):
            self._prev_start = None
            self._pending = [None] * self.num_layers
            return
        starts = set()
        for layer, kv in enumerate(items):
            if kv is None or kv[0].shape[2] != C:
                raise ValueError(f"cache.previous[{layer}] must be (K, V) of one chunk of {C} tokens")
            tag = getattr(kv[0], "_lkv_ring", None)
            if tag is not None and self._holds(kv, layer, tag[2], C):
                starts.add(tag[2])
                self._pending[layer] = True
            else:
                self._pending[layer] = (kv[0], kv[1])
        self._prev_start = starts.pop() if len(starts) == 1 else None

    @property
    def current(self):
        return _RingRange(self, self._cur_start, max(0, self.seen_tokens - self._cur_start))

    @current.setter
    def current(self, value) -> None:
        items = list(value)
        if len(items) != self.num_layers:
            raise ValueError(f"cache.current needs one entry per layer ({self.num_layers})")
        if all(kv is None for kv in items):
            self._cur_start = self.seen_tokens
            return
        n = {kv[0].shape[2] for kv in items if kv is not None}
        if len(n) != 1 or any(kv is None for kv in items):
            raise ValueError("cache.current must give every layer (K, V) of the same length")
        n = n.pop()
        start = self.seen_tokens - n
        if start < 0:
            raise ValueError("cache.current holds more tokens than have been seen")
        for layer, kv in enumerate(items):
            if not self._holds(kv, layer, start, n):
                self._write_ring(layer, start, kv[0], kv[1])
        self._cur_start = start

    def reorder_cache(self, beam_idx: torch.Tensor) -> None:
        """Select sequences (beam search), modeling.py:59-67."""

        if self._store is None:
            return
        idx = beam_idx.to(self._store.device)
        self._store = ops.TiledKV(self._store.k.index_select(0, idx).contiguous(), self._store.v.index_select(0, idx).contiguous())
        self._ring_k = self._ring_k.index_select(1, idx).contiguous()
        self._ring_v = self._ring_v.index_select(1, idx).contiguous()
        self._pending = [job if job is None or job is True else tuple(t.index_select(0, beam_idx.to(t.device)) for t in job)
                         for job in self._pending]
