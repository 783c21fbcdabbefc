"""Wan video-model history on MI355X: the shared last-layer cache and per-block attention of
videogen/src/lastkv/videogen (cache.py, model.py:153-272) on one paged K/V pool.

The reference composes each layer's history per block with torch.cat
(``_compose_history_kv``, model.py:200-272): [per-layer prefix of ``keep`` tokens | shared
final-layer K/V | previous block blended alpha * shared + (1 - alpha) * own], appends the
current block and runs bidirectional SDPA.  Here nothing is concatenated.  The pool holds

  shared pages   final-layer K/V of every committed position (append_shared's store, cache.py:33-50);
  prefix pages   per layer, the first ``keep`` positions of the layer's own K/V (the retained prefix,
                 cache.py:15-31), padded to a whole page with copies of the shared values;
  ring pages     per layer, ``ring_tokens_for_chunk(block)`` tokens: the previous block, blended
                 once at commit (in bf16, first ``keep`` positions kept local, model.py:174-198),
                 and the current block's K/V.

A block's attention is one ``lkv_prefill_attn`` call with causal = 0: the older segment reads the
layer's table [prefix pages | shared pages] over [0, prev_start), the local segment reads the ring
over [prev_start, current_start + block).  ``commit`` is ``_update_caches_akv`` (model.py:716-730):
shared append of the final layer, prefix appends, ring append and one ``lkv_blend_chunk`` for all
layers.  There is no V scale on this path.  ``keep=None`` keeps the whole first block local, which
is the reference's behaviour for ``force_first_local_kv_tokens=None`` (model.py:158-160, :187-188).
"""

from __future__ import annotations

import numpy as np
import torch

from . import ops

BLOCK = ops.BLOCK_TOKENS


class WanKVCache:
    """History of one rollout (``batch`` sequences) for ``num_layers`` layers of ``num_heads``
    heads of 128 dims, committed in blocks of ``block_tokens`` up to ``total_tokens`` positions."""

    def __init__(self, *, num_layers: int, num_heads: int, block_tokens: int, total_tokens: int,
                 keep_tokens: int | None = None, batch: int = 1, device: torch.device | str = "cuda"):
        if min(num_layers, num_heads, block_tokens, batch) < 1 or total_tokens < 0:
            raise ValueError("cache sizes must be positive")
        if keep_tokens is not None and keep_tokens < 1:
            raise ValueError("keep_tokens must be a positive integer")
        self.num_layers, self.num_heads, self.block, self.total, self.batch = (
            num_layers, num_heads, block_tokens, total_tokens, batch)
        self.keep = block_tokens if keep_tokens is None else int(keep_tokens)
        dev = torch.device(device)
        if dev.type == "cuda" and dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.ring_tokens = ops.ring_tokens_for_chunk(block_tokens)
        rb = self.ring_tokens // BLOCK
        wsh = max(1, -(-total_tokens // BLOCK))
        wpre = -(-min(self.keep, total_tokens) // BLOCK)
        self.prefix_tokens = wpre * BLOCK
        L, B = num_layers, batch
        n_shared, n_prefix, n_ring = B * wsh, L * B * wpre, L * B * rb
        self.pool = ops.PagedKV.zeros(n_shared + n_prefix + n_ring, num_heads, self.device)
        ids = np.arange(n_shared + n_prefix + n_ring, dtype=np.int32)
        shared = ids[:n_shared].reshape(B, wsh)
        prefix = ids[n_shared:n_shared + n_prefix].reshape(L, B, wpre)
        ring = ids[n_shared + n_prefix:].reshape(L, B, rb)
        older = np.concatenate([prefix, np.broadcast_to(shared[None, :, wpre:], (L, B, wsh - wpre))], axis=2)
        dev = self.device
        self.shared_table = torch.from_numpy(np.ascontiguousarray(shared)).to(dev)
        self.prefix_table = torch.from_numpy(np.ascontiguousarray(prefix)).to(dev)
        self.ring_table = torch.from_numpy(np.ascontiguousarray(ring)).to(dev)
        self.older_table = torch.from_numpy(np.ascontiguousarray(older)).to(dev)
        self.cache_len = 0
        self.alpha = self.one_minus_alpha = None
        self._ws = torch.empty(16, dtype=torch.uint8, device=dev)

    def set_alphas(self, prev_block_alphas: torch.Tensor) -> None:
        """alpha = bf16(sigmoid(prev_block_alphas[l, h])) and bf16(1 - alpha), as the reference's
        bf16 blend computes them (model.py:589-591, :185-190); ``prev_block_alphas`` is [L, H]."""

        if tuple(prev_block_alphas.shape) != (self.num_layers, self.num_heads):
            raise ValueError(f"prev_block_alphas must be [{self.num_layers}, {self.num_heads}]")
        a = prev_block_alphas.detach().float().sigmoid().to(torch.bfloat16)
        self.alpha = a.float().reshape(-1).contiguous().to(self.device)
        self.one_minus_alpha = (1 - a).float().reshape(-1).contiguous().to(self.device)

    def _check(self, name: str, t: torch.Tensor) -> None:
        if t.dtype != torch.bfloat16 or t.device != self.device or t.dim() != 4:
            raise ValueError(f"{name} must be a bf16 [B, S, H, 128] tensor on {self.device}")
        if t.shape[0] != self.batch or t.shape[1] != self.block or t.shape[2] != self.num_heads or t.shape[3] != 128:
            raise ValueError(f"{name} must be [{self.batch}, {self.block}, {self.num_heads}, 128]")

    def attention(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, current_start: int,
                  out: torch.Tensor | None = None) -> torch.Tensor:
        """Block attention of layer ``layer`` at ``current_start`` (model.py:362-383 with
        ``_compose_history_kv``): writes the block's K/V into the layer's ring and attends ``q``
        (bidirectionally) over [history | block].  q/k/v: roped bf16 ``[B, block, H, 128]``."""

        for name, t in (("q", q), ("k", k), ("v", v)):
            self._check(name, t)
        if current_start != self.cache_len:
            raise ValueError(f"block attention at {current_start} but the cache holds {self.cache_len} positions")
        S, R = self.block, self.ring_tokens
        ops.append_paged(k, v, self.pool, self.ring_table[layer], token0=current_start, wrap_tokens=R)
        prev_len = min(S, current_start)
        prev_start = current_start - prev_len
        local_len = prev_len + S
        seg = dict(local=self.pool, local_table=self.ring_table[layer], local_len=local_len,
                   local_start=prev_start % R)
        if prev_start > 0:
            width = -(-prev_start // BLOCK)
            seg.update(older=self.pool, older_table=self.older_table[layer][:, :width], older_len=prev_start)
        need = ops.prefill_workspace_bytes(self.batch, self.num_heads, prev_start, local_len, prev_start % BLOCK)
        if self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=self.device)
        qc = q if q.is_contiguous() else q.contiguous()
        return ops.prefill_attention(qc, causal=False, out=out, workspace=self._ws, **seg)

    def commit(self, current_start: int, layer_kvs) -> None:
        """``_update_caches_akv`` (model.py:716-730) for the clean block at ``current_start``:
        ``layer_kvs[l]`` = layer l's roped K and V ``[B, block, H, 128]``; the last entry is the
        final layer, whose K/V every layer shares beyond its retained prefix."""

        if len(layer_kvs) != self.num_layers:
            raise ValueError("one (k, v) pair per layer is required")
        if current_start != self.cache_len or current_start + self.block > self.total:
            raise ValueError(f"commit at {current_start}: the cache holds {self.cache_len} of {self.total} positions")
        if self.alpha is None:
            raise RuntimeError("set_alphas() first")
        for l, (k, v) in enumerate(layer_kvs):
            self._check(f"layer {l} k", k)
            self._check(f"layer {l} v", v)
        s, S, keep = current_start, self.block, self.keep
        fk, fv = layer_kvs[-1]
        ops.append_paged(fk, fv, self.pool, self.shared_table, token0=s)
        own_end = min(keep, s + S)
        tail_lo, tail_hi = max(s, keep), min(s + S, self.prefix_tokens)
        for l, (k, v) in enumerate(layer_kvs):
            ops.append_paged(k, v, self.pool, self.ring_table[l], token0=s, wrap_tokens=self.ring_tokens)
            if s < own_end:  # retained prefix: the layer's own K/V
                ops.append_paged(k[:, : own_end - s], v[:, : own_end - s], self.pool, self.prefix_table[l], token0=s)
            if tail_lo < tail_hi:  # the prefix pages' tail repeats the shared values
                ops.append_paged(fk[:, tail_lo - s: tail_hi - s], fv[:, tail_lo - s: tail_hi - s], self.pool,
                                 self.prefix_table[l], token0=tail_lo)
        lo = max(s, keep)
        if lo < s + S:  # the block becomes every layer's blended previous block
            ops.blend_chunk(self.pool.k, self.pool.v, self.pool, batch=self.batch, chunk_start=lo, chunk_len=s + S - lo,
                            alpha=self.alpha, one_minus_alpha=self.one_minus_alpha, vscale=None,
                            ring_table=self.ring_table, ring_tokens=self.ring_tokens, deep_table=self.shared_table)
        self.cache_len = s + S

    # ------------------------------------------------------------------ inspection
    def _gather(self, table: torch.Tensor, start: int, length: int, wrap: int = 0):
        """K/V of positions [start, start + length) through ``table`` [B, W], as [B, T, H, 128]."""

        pos = torch.arange(start, start + length, device=self.device)
        c = pos % wrap if wrap else pos
        pages = table[:, (c // BLOCK)].long()  # [B, T]
        w = c % BLOCK
        d = torch.arange(128, device=self.device)
        koff = ((((w[:, None] >> 2) & 1) * 4 + (d[None, :] >> 5)) * 16 + (((w[:, None] >> 3) << 2) | (w[:, None] & 3))) * 32 \
            + (d[None, :] & 31)
        voff = d[None, :] * 32 + w[:, None]
        kp = self.pool.kp[pages]  # [B, T, H, 4096]
        vp = self.pool.vp[pages]
        idx_k = koff[None, :, None, :].expand(kp.shape[0], -1, kp.shape[2], -1)
        idx_v = voff[None, :, None, :].expand(vp.shape[0], -1, vp.shape[2], -1)
        return kp.gather(3, idx_k), vp.gather(3, idx_v)

    def history(self, layer: int, length: int | None = None):
        """The history layer ``layer`` attends to for the block at ``length`` (default: the
        committed length), as the reference's ``_compose_history_kv`` returns it."""

        length = self.cache_len if length is None else length
        if length > self.cache_len or length <= 0:
            return None
        prev_start = length - min(self.block, length)
        k0, v0 = self._gather(self.older_table[layer], 0, prev_start)
        k1, v1 = self._gather(self.ring_table[layer], prev_start, length - prev_start, self.ring_tokens)
        return torch.cat([k0, k1], 1), torch.cat([v0, v1], 1)
