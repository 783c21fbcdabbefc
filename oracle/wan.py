"""Wan (video) shared-history cache and history composition in numpy (test infrastructure only;
see oracle/__init__.py).

Restates, with [B, T, H, D] arrays of bf16-representable float32 values:
  - the shared cache of videogen/src/lastkv/videogen/cache.py: one final-layer store for all
    layers (append_shared :33-50) plus a per-layer retained prefix of ``keep`` tokens, read back
    by history_kv (:53-65) as [prefix (own) | shared];
  - the per-layer ("native") cache of model.py:597-618 / append_to_cache :67-84, whose store
    receives each layer's own append (the reference's test_videogen_inference.py:63-78 checks that
    the two modes give the same rollout);
  - the appended values (_update_caches_akv, model.py:716-730 with
    _select_first_local_kv_segment :153-171): the layer's own K/V for positions < keep, the
    final layer's beyond;
  - the previous-block blend (_blend_first_local_kv_segment :174-198) in the bf16 op order
    alpha * source + (1 - alpha) * local, each op rounded, with the first ``keep`` positions kept
    local, and the history composition (_compose_history_kv :200-272):
    [history [0, prev_start) | blended previous block [prev_start, history_len)];
  - the block attention: bidirectional softmax attention over [history | current block]
    (attention.py:9-32, SDPA with is_causal=False).

Pinned by tests/test_oracle_wan_cpu.py: shared == native rollouts bit for bit; the reference
test's retained-prefix known answer (test_videogen_inference.py:84-98); a per-position brute
force of the composed history; the alpha -> 1 / alpha -> 0 / keep >= history limits.
"""

from __future__ import annotations

import numpy as np

from . import attention as A
from . import bf16


def select_first_local(own, source, segment_start: int, keep: int | None):
    """model.py:153-171: own values for positions < keep, source values beyond."""

    n = source.shape[1]
    keep = n if keep is None else keep
    keep_n = min(max(keep - segment_start, 0), n, own.shape[1])
    if keep_n <= 0:
        return source
    out = source.copy()
    out[:, :keep_n] = own[:, :keep_n]
    return out


def blend_first_local(own, source, segment_start: int, keep: int | None, alpha):
    """model.py:174-198.  ``alpha`` [H] (values already in the model dtype)."""

    n = min(source.shape[1], own.shape[1])
    keep = n if keep is None else keep
    own, source = own[:, :n], source[:, :n]
    a = np.asarray(alpha, np.float32).reshape(1, 1, -1, 1)
    blended = bf16.add(bf16.mul(a, source), bf16.mul(bf16.rsub(a, 1.0), own))
    keep_n = min(max(keep - segment_start, 0), n)
    if keep_n <= 0:
        return blended
    if keep_n >= n:
        return own.copy()
    out = blended.copy()
    out[:, :keep_n] = own[:, :keep_n]
    return out


def alpha_bf16(logits) -> np.ndarray:
    """sigmoid(prev_block_alphas[l]) cast to bf16 (model.py:589-591)."""

    return bf16.round_bf16(A.sigmoid(np.asarray(logits, np.float64)).astype(np.float32))


class WanCache:
    """The reference's cache state for one rollout, in either storage mode.

    shared=True: one store (all layers append into it; last writer wins) + per-layer prefix of
    min(total, keep) tokens (cache.py:6-50).  shared=False: one store per layer (model.py:597-618).
    Both keep the layer's own K/V of the last committed block (``curr``, model.py:621-635).
    """

    def __init__(self, layers: int, batch: int, heads: int, total: int, block: int, keep: int | None,
                 shared: bool, dim: int = 128):
        self.layers, self.block, self.keep, self.shared, self.total = layers, block, keep, shared, total
        shape = (batch, total, heads, dim)
        if shared:
            if keep is None:
                raise ValueError("the shared cache needs keep (cache.py:15 takes min(total, keep))")
            store = np.zeros(shape, np.float32)
            self.k = [store] * layers
            self.v = [np.zeros(shape, np.float32)] * layers
            pre = (batch, min(total, keep), heads, dim)
            self.prefix_k = [np.zeros(pre, np.float32) for _ in range(layers)]
            self.prefix_v = [np.zeros(pre, np.float32) for _ in range(layers)]
        else:
            self.k = [np.zeros(shape, np.float32) for _ in range(layers)]
            self.v = [np.zeros(shape, np.float32) for _ in range(layers)]
        self.cache_len = 0
        self.curr = [None] * layers  # (k, v, start)

    def commit(self, layer_kvs, start: int) -> None:
        """_update_caches_akv (model.py:716-730): every layer appends its selected K/V, then keeps
        its own block as ``curr``."""

        if start != self.cache_len:
            raise ValueError("noncontiguous append")
        src_k, src_v = layer_kvs[-1]
        end = start + src_k.shape[1]
        if end > self.total:
            raise ValueError("cache capacity exceeded")
        for l, (k, v) in enumerate(layer_kvs):
            nk = select_first_local(k, src_k, start, self.keep)
            nv = select_first_local(v, src_v, start, self.keep)
            self.k[l][:, start:end] = nk  # shared mode: the same array for every layer
            self.v[l][:, start:end] = nv
            if self.shared:
                pe = min(end, self.prefix_k[l].shape[1])
                if start < pe:
                    self.prefix_k[l][:, start:pe] = nk[:, : pe - start]
                    self.prefix_v[l][:, start:pe] = nv[:, : pe - start]
        self.cache_len = end
        for l, (k, v) in enumerate(layer_kvs):
            self.curr[l] = (k.copy(), v.copy(), start)

    def deep(self, layer: int, length: int):
        """history_kv (cache.py:53-65) or the per-layer store."""

        if length > self.cache_len:
            raise ValueError("history beyond the committed cache")
        if not self.shared:
            return self.k[layer][:, :length], self.v[layer][:, :length]
        r = min(length, self.prefix_k[layer].shape[1])
        k = np.concatenate([self.prefix_k[layer][:, :r], self.k[layer][:, r:length]], 1)
        v = np.concatenate([self.prefix_v[layer][:, :r], self.v[layer][:, r:length]], 1)
        return k, v

    def history(self, layer: int, history_len: int, prev_block_len: int, alpha):
        """_compose_history_kv (model.py:200-272); None when there is no history."""

        history_len = min(history_len, self.cache_len)
        if history_len <= 0:
            return None
        dk, dv = self.deep(layer, history_len)
        prev_len = min(prev_block_len, history_len)
        prev_start = history_len - prev_len
        ck, cv, cs = self.curr[layer]
        if cs > prev_start or cs + ck.shape[1] < history_len:
            raise RuntimeError("curr does not cover the previous block")
        own_k = ck[:, prev_start - cs: history_len - cs]
        own_v = cv[:, prev_start - cs: history_len - cs]
        bk = blend_first_local(own_k, dk[:, prev_start:history_len], prev_start, self.keep, alpha)
        bv = blend_first_local(own_v, dv[:, prev_start:history_len], prev_start, self.keep, alpha)
        return np.concatenate([dk[:, :prev_start], bk], 1), np.concatenate([dv[:, :prev_start], bv], 1)


def block_attention(q, k_cur, v_cur, history):
    """Bidirectional attention of the current block over [history | current] (attention.py:9-32,
    model.py:372-383).  q, k_cur, v_cur [B, S, H, D]; returns fp64 [B, S, H, D]."""

    if history is not None:
        k = np.concatenate([history[0], k_cur], 1)
        v = np.concatenate([history[1], v_cur], 1)
    else:
        k, v = k_cur, v_cur
    out, _ = A.attention(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3))
    return out.transpose(0, 2, 1, 3)
