"""The tiled K/V cache layout as closed-form index maps (test infrastructure only).

The layout is this build's own (the reference keeps [B, H, T, D] tensors,
llm/src/lastkv/llm/modeling.py:31-67), so nothing in the reference pins it.  Pinned by:
tests/test_oracle_cpu.py checks that each block map is a bijection of 0..4095 and that the
MFMA-operand loads the decode kernel issues read contiguous 1 KiB runs; the GPU tests check
that lkv_cache_pack / lkv_cache_unpack reproduce these maps bit for bit and invert each other.
"""

from __future__ import annotations

import numpy as np

HEAD_DIM = 128
BLOCK = 32
BLOCK_ELEMS = BLOCK * HEAD_DIM


def k_offset(w, d):
    """Offset of K element (token w of the block, dim d) inside its 4096-element block."""

    w = np.asarray(w)
    d = np.asarray(d)
    u = (w >> 2) & 1
    r = ((w >> 3) << 2) | (w & 3)
    return ((u * 4 + (d >> 5)) * 16 + r) * 32 + (d & 31)


def v_offset(w, d):
    """Offset of V element (token w, dim d): the block stores V transposed."""

    return np.asarray(d) * 32 + np.asarray(w)


def pack(x: np.ndarray, kind: int, capacity: int) -> np.ndarray:
    """[B, H, T, 128] -> [B, H, capacity / 32, 4096] (tokens beyond T are zero)."""

    B, H, T, D = x.shape
    assert D == HEAD_DIM and capacity % BLOCK == 0 and T <= capacity
    out = np.zeros((B, H, capacity // BLOCK, BLOCK_ELEMS), dtype=x.dtype)
    t = np.arange(T)[:, None]
    d = np.arange(D)[None, :]
    off = (k_offset if kind == 0 else v_offset)(t % BLOCK, d)
    blk = np.broadcast_to(t // BLOCK, off.shape)
    out[:, :, blk, off] = x
    return out


def unpack(cache: np.ndarray, kind: int, token0: int, tokens: int) -> np.ndarray:
    t = np.arange(token0, token0 + tokens)[:, None]
    d = np.arange(HEAD_DIM)[None, :]
    off = (k_offset if kind == 0 else v_offset)(t % BLOCK, d)
    blk = np.broadcast_to(t // BLOCK, off.shape)
    return cache[:, :, blk, off]
