"""Torch-facing wrappers of the C-ABI kernels.

Each wrapper validates shapes, dtypes and devices, then passes raw device pointers and the
current HIP stream of the tensors' device to ``liblastkv_amd.so``.  Nothing here computes on
the CPU; a missing library raises ``LastKVNativeError``.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib

HEAD_DIM = 128
BLOCK_TOKENS = 32
BLOCK_ELEMS = BLOCK_TOKENS * HEAD_DIM
KIND_K, KIND_V = 0, 1


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require(cond: bool, message: str) -> None:
    if not cond:
        raise ValueError(message)


def _require_bf16_cuda(name: str, t: torch.Tensor) -> None:
    _require(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _require(t.is_cuda, f"{name} must be on a GPU (the kernels have no CPU path)")
    _require(t.dtype == torch.bfloat16, f"{name} must be bfloat16, got {t.dtype}")


@dataclass
class TiledKV:
    """K and V caches in the tiled block layout: ``[slots, heads, blocks, 4096]`` bf16 each.

    Slot ``s`` / head ``h`` owns ``blocks`` consecutive 32-token blocks; a slot is one
    sequence's shared history (older region) or one layer's ring (recent + current chunk).
    """

    k: torch.Tensor
    v: torch.Tensor

    def __post_init__(self) -> None:
        for name, t in (("k", self.k), ("v", self.v)):
            _require_bf16_cuda(f"TiledKV.{name}", t)
            _require(t.dim() == 4 and t.shape[-1] == BLOCK_ELEMS, f"TiledKV.{name} must be [slots, heads, blocks, 4096]")
            _require(t.is_contiguous(), f"TiledKV.{name} must be contiguous")
        _require(self.k.shape == self.v.shape, "TiledKV k and v shapes differ")

    @classmethod
    def zeros(cls, slots: int, heads: int, capacity_tokens: int, device: torch.device | str) -> "TiledKV":
        _require(capacity_tokens % BLOCK_TOKENS == 0, "capacity must be a multiple of 32 tokens")
        shape = (slots, heads, capacity_tokens // BLOCK_TOKENS, BLOCK_ELEMS)
        return cls(torch.zeros(shape, dtype=torch.bfloat16, device=device), torch.zeros(shape, dtype=torch.bfloat16, device=device))

    @property
    def slots(self) -> int:
        return int(self.k.shape[0])

    @property
    def heads(self) -> int:
        return int(self.k.shape[1])

    @property
    def blocks(self) -> int:
        return int(self.k.shape[2])

    @property
    def capacity_tokens(self) -> int:
        return self.blocks * BLOCK_TOKENS

    @property
    def seq_stride(self) -> int:
        return self.heads * self.blocks * BLOCK_ELEMS

    @property
    def head_stride(self) -> int:
        return self.blocks * BLOCK_ELEMS

    @property
    def device(self) -> torch.device:
        return self.k.device


@dataclass
class PagedKV:
    """K and V page pools in the tiled block layout, head-major: ``[heads, pages, 4096]`` bf16 each.

    A page holds 32 tokens of every kv head; which pages form a sequence's segment is given per
    call by an int32 block table ``[B, W]`` (block j of sequence b is page ``table[b, j]``).  The
    pages of one head are contiguous, so a sequence whose pages were handed out in order streams
    each head's keys from one contiguous run, as a contiguous cache does (with page-major storage,
    [pages, heads, 4096], consecutive blocks of one head sit heads * 8 KiB apart, and the decode
    kernel measured ~10 % slower on MI355X).  ``kp`` / ``vp`` are ``[pages, heads, 4096]`` views
    for indexing by page id."""

    k: torch.Tensor
    v: torch.Tensor

    def __post_init__(self) -> None:
        for name, t in (("k", self.k), ("v", self.v)):
            _require_bf16_cuda(f"PagedKV.{name}", t)
            _require(t.dim() == 3 and t.shape[-1] == BLOCK_ELEMS, f"PagedKV.{name} must be [heads, pages, 4096]")
            _require(t.is_contiguous(), f"PagedKV.{name} must be contiguous")
        _require(self.k.shape == self.v.shape, "PagedKV k and v shapes differ")

    @classmethod
    def zeros(cls, pages: int, heads: int, device: torch.device | str) -> "PagedKV":
        shape = (heads, pages, BLOCK_ELEMS)
        return cls(torch.zeros(shape, dtype=torch.bfloat16, device=device), torch.zeros(shape, dtype=torch.bfloat16, device=device))

    @property
    def pages(self) -> int:
        return int(self.k.shape[1])

    @property
    def heads(self) -> int:
        return int(self.k.shape[0])

    @property
    def page_stride(self) -> int:
        return BLOCK_ELEMS

    @property
    def head_stride(self) -> int:
        return self.pages * BLOCK_ELEMS

    @property
    def kp(self) -> torch.Tensor:
        return self.k.transpose(0, 1)

    @property
    def vp(self) -> torch.Tensor:
        return self.v.transpose(0, 1)

    @property
    def device(self) -> torch.device:
        return self.k.device


def cache_pack(src: torch.Tensor, cache: torch.Tensor, kind: int, token0: int = 0, *, capacity_tokens: int | None = None) -> None:
    """Write ``src`` ``[B, H, T, 128]`` into cache tokens ``[token0, token0 + T)`` of slots ``0..B-1``."""

    _require_bf16_cuda("src", src)
    _require(src.dim() == 4 and src.shape[-1] == HEAD_DIM and src.stride(-1) == 1, "src must be [B, H, T, 128] with unit dim stride")
    _require(cache.dim() == 4 and cache.shape[-1] == BLOCK_ELEMS, "cache must be [slots, heads, blocks, 4096]")
    _require_bf16_cuda("cache", cache)
    B, H, T, _ = src.shape
    _require(B <= cache.shape[0] and H == cache.shape[1], "src batch/heads do not fit the cache")
    cap = cache.shape[2] * BLOCK_TOKENS if capacity_tokens is None else capacity_tokens
    lib = _lib.load()
    _lib.check(
        lib.lkv_cache_pack(
            src.data_ptr(), src.stride(0), src.stride(1), src.stride(2), B, H, T, kind,
            cache.data_ptr(), cache.stride(0), cache.stride(1), token0, cap, _stream(src.device),
        ),
        "lkv_cache_pack",
    )


def cache_unpack(cache: torch.Tensor, kind: int, token0: int, tokens: int, batch: int | None = None) -> torch.Tensor:
    """Read cache tokens ``[token0, token0 + tokens)`` back as ``[B, H, tokens, 128]``."""

    _require_bf16_cuda("cache", cache)
    _require(cache.dim() == 4 and cache.shape[-1] == BLOCK_ELEMS, "cache must be [slots, heads, blocks, 4096]")
    B = cache.shape[0] if batch is None else batch
    H = cache.shape[1]
    out = torch.empty((B, H, tokens, HEAD_DIM), dtype=torch.bfloat16, device=cache.device)
    lib = _lib.load()
    _lib.check(
        lib.lkv_cache_unpack(
            cache.data_ptr(), cache.stride(0), cache.stride(1), token0, cache.shape[2] * BLOCK_TOKENS,
            B, H, tokens, kind, out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), _stream(cache.device),
        ),
        "lkv_cache_unpack",
    )
    return out


def pack_kv(k: torch.Tensor, v: torch.Tensor, cache: TiledKV, token0: int = 0) -> None:
    cache_pack(k, cache.k, KIND_K, token0)
    cache_pack(v, cache.v, KIND_V, token0)


def unpack_kv(cache: TiledKV, token0: int, tokens: int, batch: int | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    return cache_unpack(cache.k, KIND_K, token0, tokens, batch), cache_unpack(cache.v, KIND_V, token0, tokens, batch)


_CU_COUNT: dict[int, int] = {}


def _cu_count(device: torch.device) -> int:
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _CU_COUNT:
        _CU_COUNT[index] = int(torch.cuda.get_device_properties(index).multi_processor_count)
    return _CU_COUNT[index]


def default_decode_splits(batch: int, kv_heads: int, max_tokens: int, cu_count: int) -> int:
    """Key splits per (sequence, kv head): as many as fit one round of workgroups (one 4-wave
    workgroup runs per CU).  A second round costs more than the CUs one round leaves idle: at 8K
    keys and 8 kv heads, B = 20 takes 99 us with one split (160 workgroups) against 124 us with two,
    B = 12 71 us with two (192) against 93 us with three."""

    pairs = max(1, batch * kv_heads)
    blocks = max(1, math.ceil(max_tokens / BLOCK_TOKENS))
    splits = max(1, cu_count // pairs)
    return int(max(1, min(splits, math.ceil(blocks / 4), 1024)))


def _len_arg(value: int | torch.Tensor | None, batch: int, name: str, device: torch.device) -> tuple[int | None, int]:
    if value is None:
        return None, 0
    if isinstance(value, torch.Tensor):
        _require(value.dtype == torch.int32 and value.device == device and value.numel() == batch and value.is_contiguous(),
                 f"{name} must be a contiguous int32 tensor of {batch} entries on {device}")
        return value.data_ptr(), 0
    return None, int(value)


def _table_arg(table: torch.Tensor, B: int, name: str, device: torch.device) -> None:
    _require(table is not None, f"a paged {name} segment needs a block table")
    _require(table.dtype == torch.int32 and table.device == device and table.dim() == 2 and table.shape[0] == B
             and table.stride(1) == 1, f"{name}_table must be an int32 [B, W] tensor with contiguous rows on {device}")


def _fill_segments(a, B: int, device: torch.device, older, older_len, older_slot, vscale, local, local_len,
                   local_start, local_slot, older_table=None, local_table=None, local_ring_blocks=None) -> int:
    """Fill the older/local segment fields shared by DecodeArgs and PrefillArgs; returns Hkv.

    ``older`` / ``local`` are a TiledKV (contiguous per slot) or a PagedKV with a block table
    (``older_table`` [B, W]: older block j of sequence b is page ``older_table[b, j]``;
    ``local_table`` [B, >= ring blocks]: ring block rb is page ``local_table[b, rb]``)."""

    _require(older is not None or local is not None, "at least one key segment is required")
    Hkv = (older if older is not None else local).heads
    if older is not None and local is not None:
        _require(older.heads == local.heads, "older and local caches have different kv head counts")
    if vscale is not None:
        _require(vscale.dtype == torch.float32 and vscale.numel() == Hkv and vscale.is_contiguous() and vscale.device == device,
                 "vscale must be a contiguous fp32 [Hkv] tensor on the query's device")
    a.older_vscale_mode = 1 if vscale is not None else 0
    a.vscale = _ptr(vscale)
    for name, t in (("older_slot", older_slot), ("local_slot", local_slot)):
        if t is not None:
            _require(t.dtype == torch.int32 and t.device == device and t.numel() == B and t.is_contiguous(),
                     f"{name} must be a contiguous int32 tensor of {B} entries on {device}")
    if older is not None:
        _require(older.device == device, "older cache on another device")
        a.older_k, a.older_v = older.k.data_ptr(), older.v.data_ptr()
        a.older_head_stride = older.head_stride
        a.older_len, a.older_len_const = _len_arg(older_len, B, "older_len", device)
        if isinstance(older, PagedKV):
            _table_arg(older_table, B, "older", device)
            _require(older_slot is None, "older_slot does not apply to a paged segment")
            a.older_block_table, a.older_table_stride = older_table.data_ptr(), older_table.stride(0)
            a.older_page_stride, a.older_num_pages = older.page_stride, older.pages
            a.older_capacity_tokens = older_table.shape[1] * BLOCK_TOKENS
        else:
            _require(older_table is None, "older_table needs a PagedKV older segment")
            a.older_seq_stride = older.seq_stride
            a.older_capacity_tokens = older.capacity_tokens
            a.older_slot = _ptr(older_slot)
            a.older_num_slots = older.slots
            if older_slot is None:
                _require(older.slots >= B, "older cache has fewer slots than sequences")
        if not isinstance(older_len, torch.Tensor):
            _require(0 <= older_len <= a.older_capacity_tokens, "older_len exceeds the cache capacity")
    if local is not None:
        _require(local.device == device, "local cache on another device")
        a.local_k, a.local_v = local.k.data_ptr(), local.v.data_ptr()
        a.local_head_stride = local.head_stride
        if isinstance(local, PagedKV):
            _table_arg(local_table, B, "local", device)
            _require(local_slot is None, "local_slot does not apply to a paged segment")
            a.local_ring_blocks = int(local_ring_blocks if local_ring_blocks is not None else local_table.shape[1])
            _require(0 < a.local_ring_blocks <= local_table.shape[1], "local_ring_blocks exceeds the table width")
            a.local_block_table, a.local_table_stride = local_table.data_ptr(), local_table.stride(0)
            a.local_page_stride, a.local_num_pages = local.page_stride, local.pages
        else:
            _require(local_table is None, "local_table needs a PagedKV local segment")
            a.local_seq_stride = local.seq_stride
            a.local_ring_blocks = local.blocks
            a.local_slot = _ptr(local_slot)
            a.local_num_slots = local.slots
            if local_slot is None:
                _require(local.slots >= B, "local cache has fewer slots than sequences")
        ring_tokens = a.local_ring_blocks * BLOCK_TOKENS
        a.local_len, a.local_len_const = _len_arg(local_len, B, "local_len", device)
        a.local_start, a.local_start_const = _len_arg(local_start, B, "local_start", device)
        if not isinstance(local_len, torch.Tensor):
            _require(0 <= local_len <= ring_tokens, "local_len exceeds the ring capacity")
        if not isinstance(local_start, torch.Tensor):
            _require(0 <= local_start < ring_tokens, "local_start outside the ring")
    return Hkv


def _out_scale_arg(a, out_scale: torch.Tensor | None, Hkv: int, device: torch.device) -> None:
    if out_scale is not None:
        _require(out_scale.dtype == torch.float32 and out_scale.numel() == Hkv and out_scale.is_contiguous()
                 and out_scale.device == device, "out_scale must be a contiguous fp32 [Hkv] tensor on the query's device")
    a.out_scale = _ptr(out_scale)


def decode_attention(
    q: torch.Tensor,
    *,
    older: TiledKV | PagedKV | None = None,
    older_len: int | torch.Tensor = 0,
    older_slot: torch.Tensor | None = None,
    vscale: torch.Tensor | None = None,
    local: TiledKV | PagedKV | None = None,
    local_len: int | torch.Tensor = 0,
    local_start: int | torch.Tensor = 0,
    local_slot: torch.Tensor | None = None,
    older_table: torch.Tensor | None = None,
    local_table: torch.Tensor | None = None,
    local_ring_blocks: int | None = None,
    sm_scale: float | None = None,
    num_splits: int | None = None,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    kv_cache_hint: int = 0,
    no_alloc: bool = False,
    out_scale: torch.Tensor | None = None,
) -> torch.Tensor:
    """One-token-per-sequence attention over ``[older shared segment | local ring segment]``.

    ``q`` is ``[B, Hq, 128]`` bf16 (or ``[B, Hq, 1, 128]``).  ``vscale`` ``[Hkv]`` fp32 switches
    the older segment's V to ``bf16(V * vscale[h])``.  ``out_scale`` ``[Hkv]`` fp32 (bf16 values)
    makes the output ``bf16(bf16(o) * out_scale[h])``, the vLLM path's rescale of an attention over
    rings of V / s.  Returns ``out`` ``[B, Hq, 128]`` bf16.
    ``kv_cache_hint`` selects the cache policy of the K/V loads (0 = by the call's K/V size,
    1 = default, 2 = non-temporal); the results do not depend on it.  ``no_alloc`` calls
    ``lkv_decode_attn_noalloc``: the split states go to the library's static per-GPU scratch
    (LKV_NOALLOC_SCRATCH_BYTES) instead of a workspace (pass ``out`` too for a call that allocates
    nothing); calls overlapping on one GPU then race.
    """

    _require_bf16_cuda("q", q)
    if q.dim() == 4:
        _require(q.shape[2] == 1, "decode_attention takes one query token per sequence")
        q = q[:, :, 0]
    _require(q.dim() == 3 and q.shape[-1] == HEAD_DIM, "q must be [B, Hq, 128]")
    _require(q.stride(-1) == 1 and q.stride(1) == HEAD_DIM, "q heads must be contiguous rows of 128")
    B, Hq, _ = q.shape
    device = q.device
    a = _lib.DecodeArgs()
    a.struct_size = ctypes.sizeof(_lib.DecodeArgs)
    Hkv = _fill_segments(a, B, device, older, older_len, older_slot, vscale, local, local_len, local_start, local_slot,
                         older_table, local_table, local_ring_blocks)
    _require(Hq % Hkv == 0 and Hq // Hkv <= 64, "Hq must be a multiple of Hkv with group <= 64")
    if out is None:
        out = torch.empty((B, Hq, HEAD_DIM), dtype=torch.bfloat16, device=device)
    _require_bf16_cuda("out", out)
    if out.dim() == 4:
        out = out[:, :, 0]
    _require(out.shape[0] == B and out.shape[1] == Hq and out.shape[-1] == HEAD_DIM, "out shape mismatch")
    _require(out.stride(-1) == 1 and out.stride(1) == HEAD_DIM, "out heads must be contiguous rows of 128")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() == B * Hq and lse.device == device,
                 "lse must be a contiguous fp32 [B, Hq] tensor")
    max_tokens = 0
    if older is not None:
        max_tokens += a.older_capacity_tokens if isinstance(older_len, torch.Tensor) else int(older_len)
    if local is not None:
        max_tokens += a.local_ring_blocks * BLOCK_TOKENS if isinstance(local_len, torch.Tensor) else int(local_len)
    if num_splits is None:
        num_splits = default_decode_splits(B, Hkv, max_tokens, _cu_count(device))
    lib = _lib.load()
    need = lib.lkv_decode_workspace_bytes(B, Hq, num_splits)
    if no_alloc:
        _require(workspace is None, "no_alloc calls use the library's static scratch, not a workspace")
    elif need > 0:
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=device)
        _require(workspace.device == device and workspace.numel() * workspace.element_size() >= need, "workspace too small")
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim = B, Hq, Hkv, HEAD_DIM
    a.num_splits = num_splits
    a.kv_cache_hint = int(kv_cache_hint)
    _out_scale_arg(a, out_scale, Hkv, device)
    a.sm_scale = HEAD_DIM ** -0.5 if sm_scale is None else float(sm_scale)
    a.q, a.q_stride_b = q.data_ptr(), q.stride(0)
    a.out, a.out_stride_b = out.data_ptr(), out.stride(0)
    a.lse = _ptr(lse)
    a.workspace = _ptr(workspace)
    a.workspace_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if no_alloc:
        _lib.check(lib.lkv_decode_attn_noalloc(ctypes.byref(a), _stream(device)), "lkv_decode_attn_noalloc")
    else:
        _lib.check(lib.lkv_decode_attn(ctypes.byref(a), _stream(device)), "lkv_decode_attn")
    return out


def prefill_attention(
    q: torch.Tensor,
    *,
    older: TiledKV | PagedKV | None = None,
    older_len: int | torch.Tensor = 0,
    older_slot: torch.Tensor | None = None,
    vscale: torch.Tensor | None = None,
    local: TiledKV | PagedKV | None = None,
    local_len: int | torch.Tensor = 0,
    local_start: int | torch.Tensor = 0,
    local_slot: torch.Tensor | None = None,
    older_table: torch.Tensor | None = None,
    local_table: torch.Tensor | None = None,
    local_ring_blocks: int | None = None,
    causal: bool = True,
    sm_scale: float | None = None,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    tile_waves: int = 0,
    out_scale: torch.Tensor | None = None,
    cu_seqlens_q: torch.Tensor | None = None,
    max_seqlen_q: int | None = None,
    num_splits: int = 0,
    cu_seqlens_q_host=None,
) -> torch.Tensor:
    """Attention of ``q`` ``[B, L, Hq, 128]`` (L query tokens per sequence, the last L tokens of
    the local segment) over ``[older | local]``; the local segment is bottom-right causal
    (``causal``) or fully visible.  Returns ``out`` ``[B, L, Hq, 128]`` bf16.

    Ragged rows (FlashAttention's varlen form): with ``cu_seqlens_q`` (int32 ``[B + 1]`` on the
    device, ``cu[0] = 0``, non-decreasing) ``q`` is ``[T, Hq, 128]``, sequence b's queries being rows
    ``cu[b] .. cu[b + 1] - 1`` (each sequence's L_b queries are the last L_b tokens of its local
    segment); ``max_seqlen_q`` (a host int) bounds every L_b, and ``out`` / ``lse`` are ``[T, Hq, 128]``
    / ``[T, Hq]``.  One call runs every sequence: those of at most 64 query rows per kv head on the
    decode kernel, the others on the tile kernel.  ``num_splits`` fixes the decode kernel's key
    splits for those sequences (0: chosen from the grid).  ``cu_seqlens_q_host`` (optional: the same
    offsets on the host, a sequence of ints or an int32 array) lets the call launch only the decode
    column classes that hold a sequence and skip merges of one split; it must equal ``cu_seqlens_q``.

    ``workspace`` (uint8, 16-byte aligned, at least ``prefill_workspace_bytes`` of the same
    arguments) receives the fp16 V of every key block; without it one is allocated per call.
    ``tile_waves`` (0, 4 or 8) fixes the workgroup size of the tile kernel; 0 lets the library
    choose from the grid size and the device's CU count.  4 or 8 put a uniform call on the tile
    kernel at any size; in a ragged call they apply to its sequences above 64 query rows per kv
    head, and its shorter ones stay on the decode kernel unless all of its sequences are short.
    ``out_scale`` as in ``decode_attention``."""

    _require_bf16_cuda("q", q)
    ragged = cu_seqlens_q is not None
    if ragged:
        _require(q.dim() == 3 and q.shape[-1] == HEAD_DIM, "a ragged q must be [T, Hq, 128]")
        _require(cu_seqlens_q.dtype == torch.int32 and cu_seqlens_q.dim() == 1 and cu_seqlens_q.numel() >= 2
                 and cu_seqlens_q.is_contiguous() and cu_seqlens_q.device == q.device,
                 "cu_seqlens_q must be a contiguous int32 [B + 1] tensor on the query's device")
        _require(max_seqlen_q is not None and int(max_seqlen_q) >= 1, "a ragged call needs max_seqlen_q >= 1")
        q = q.unsqueeze(0)  # [1, T, Hq, 128]: the row stride is the token stride
        B, L, Hq = cu_seqlens_q.numel() - 1, q.shape[1], q.shape[2]
    else:
        _require(max_seqlen_q is None, "max_seqlen_q applies to ragged calls (cu_seqlens_q)")
        _require(q.dim() == 4 and q.shape[-1] == HEAD_DIM, "q must be [B, L, Hq, 128]")
        B, L, Hq, _ = q.shape
    _require(q.stride(-1) == 1 and q.stride(2) == HEAD_DIM, "q heads must be contiguous rows of 128")
    device = q.device
    a = _lib.PrefillArgs()
    a.struct_size = ctypes.sizeof(_lib.PrefillArgs)
    Hkv = _fill_segments(a, B, device, older, older_len, older_slot, vscale, local, local_len, local_start, local_slot,
                         older_table, local_table, local_ring_blocks)
    _require(Hq % Hkv == 0, "Hq must be a multiple of Hkv")
    QB = 1 if ragged else B  # leading dim of q / out
    if out is None:
        out = torch.empty((QB, L, Hq, HEAD_DIM), dtype=torch.bfloat16, device=device)
    elif ragged:
        _require(out.dim() == 3, "a ragged out must be [T, Hq, 128]")
        out = out.unsqueeze(0)
    _require_bf16_cuda("out", out)
    _require(tuple(out.shape) == (QB, L, Hq, HEAD_DIM), "out must be [B, L, Hq, 128] ([T, Hq, 128] ragged)")
    _require(out.stride(-1) == 1 and out.stride(2) == HEAD_DIM, "out heads must be contiguous rows of 128")
    if lse is not None:
        _require(lse.dtype == torch.float32 and lse.is_contiguous() and lse.numel() == QB * L * Hq and lse.device == device,
                 "lse must be a contiguous fp32 [B, L, Hq] tensor ([T, Hq] ragged)")
    a.batch, a.tokens, a.num_q_heads, a.num_kv_heads, a.head_dim = B, L, Hq, Hkv, HEAD_DIM
    host_cu = None
    if ragged:
        a.cu_seqlens_q, a.max_seqlen_q = cu_seqlens_q.data_ptr(), int(max_seqlen_q)
        if cu_seqlens_q_host is not None:
            host_cu = np.ascontiguousarray(np.asarray(cu_seqlens_q_host, dtype=np.int32))
            _require(host_cu.ndim == 1 and host_cu.size == B + 1 and host_cu[0] == 0 and bool(np.all(np.diff(host_cu) >= 0)),
                     "cu_seqlens_q_host must hold the B + 1 non-decreasing offsets of cu_seqlens_q, from 0")
            a.cu_seqlens_q_host = host_cu.ctypes.data
    else:
        _require(cu_seqlens_q_host is None, "cu_seqlens_q_host applies to ragged calls (cu_seqlens_q)")
    _require(0 <= int(num_splits) <= 1024, "num_splits must be in [0, 1024]")
    a.num_splits = int(num_splits)
    a.sm_scale = HEAD_DIM ** -0.5 if sm_scale is None else float(sm_scale)
    a.causal = 1 if causal else 0
    a.tile_waves = int(tile_waves)
    _out_scale_arg(a, out_scale, Hkv, device)
    a.q, a.q_stride_b, a.q_stride_t = q.data_ptr(), q.stride(0), q.stride(1)
    a.out, a.out_stride_b, a.out_stride_t = out.data_ptr(), out.stride(0), out.stride(1)
    a.lse = _ptr(lse)
    lib = _lib.load()
    if workspace is None:  # room for the tile kernel's key splits too
        workspace = torch.empty(max(int(lib.lkv_prefill_workspace_bytes(ctypes.byref(a))), 16), dtype=torch.uint8,
                                device=device)
    _require(workspace.device == device and workspace.is_contiguous(), "workspace must be a contiguous tensor on the query's device")
    a.workspace = workspace.data_ptr()
    a.workspace_bytes = workspace.numel() * workspace.element_size()
    need = int(lib.lkv_prefill_workspace_min_bytes(ctypes.byref(a)))
    _require(a.workspace_bytes >= need, f"prefill workspace too small: {a.workspace_bytes} < {need} bytes")
    _lib.check(lib.lkv_prefill_attn(ctypes.byref(a), _stream(device)), "lkv_prefill_attn")
    return out[0] if ragged else out


def decode_workspace_bytes(batch: int, num_q_heads: int, num_splits: int) -> int:
    """Bytes of the split-K workspace ``decode_attention`` needs (0 for one split)."""

    return int(_lib.load().lkv_decode_workspace_bytes(batch, num_q_heads, num_splits))


def prefill_workspace_bytes(batch: int, kv_heads: int, older_tokens: int, local_tokens: int, local_lead: int = 31,
                            query_rows: int = 0, num_q_heads: int = 0, cu_count: int | None = None) -> int:
    """Upper bound of the prefill workspace for segments of at most ``older_tokens`` and
    ``local_tokens`` keys (``local_lead``: the ring start's offset inside its 32-token block).  With
    ``query_rows`` (the call's output rows: B * L, or T ragged) and ``num_q_heads`` it also holds the
    tile kernel's key-split states: a call splits its tiles' keys (at most 4 ways) only when its tile
    grid leaves CUs idle (fewer 4-wave workgroups of 128 rows than two per CU), so only when
    query_rows * num_q_heads < 256 * CUs, and then needs rows * Hq * splits * 129 fp32 values."""

    blocks = -(-older_tokens // 32) + (-(-(local_lead + local_tokens) // 32) if local_tokens > 0 else 0)
    # fp16 V of every block, then one flag byte per block (rows padded to 16 bytes), then one 16-byte word
    v16 = batch * kv_heads * (blocks * 8192 + -(-blocks // 16) * 16) + 16
    cus = cu_count if cu_count is not None else (_cu_count(torch.device("cuda")) if query_rows > 0 else 0)
    if query_rows > 0 and num_q_heads > 0 and query_rows * num_q_heads < 256 * cus:
        v16 += query_rows * num_q_heads * 4 * (HEAD_DIM + 1) * 4
    return v16


def prefill_split_state_bytes(rows: int, num_q_heads: int, num_splits: int) -> int:
    """Workspace a uniform prefill call with a fixed ``num_splits`` > 1 needs for the decode kernel's
    split states of ``rows`` query tokens (batch x tokens)."""

    return 0 if num_splits <= 1 else rows * num_q_heads * num_splits * (HEAD_DIM + 2) * 4


# the largest split count of a ragged call's decode-kernel classes (kRaggedSplitCap in the library)
RAGGED_SPLIT_CAP = 32


def ragged_split_state_bytes(batch: int, num_q_heads: int, num_kv_heads: int, max_seqlen: int, num_splits: int,
                             cu_count: int) -> int:
    """Upper bound of the split states a ragged prefill call keeps for its sequences of at most 64
    query rows per kv head (what ``lkv_prefill_workspace_bytes`` adds for them): per column class
    (16, 32, 64 columns) the worst case over the number n of its sequences of n * lmax * Hq * S(n)
    states, S(n) = ``num_splits`` or min(RAGGED_SPLIT_CAP, floor(CUs / Hkv), max(1, floor(CUs / (n Hkv))))."""

    group = num_q_heads // num_kv_heads
    cap = min(RAGGED_SPLIT_CAP, max(1, cu_count // num_kv_heads))
    worst = 0
    for col_hi in (16, 32, 64):
        lmax = min(col_hi // group, max_seqlen)
        if lmax < 1:
            continue
        for n in range(1, batch + 1):
            S = num_splits if num_splits > 0 else min(cap, max(1, cu_count // (n * num_kv_heads)))
            if S > 1:
                worst = max(worst, n * lmax * num_q_heads * S)
    return worst * (HEAD_DIM + 2) * 4


def merge_states(
    prefix_out: torch.Tensor,
    prefix_lse: torch.Tensor,
    suffix_out: torch.Tensor,
    suffix_lse: torch.Tensor,
    *,
    prefix_scale: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    out_lse: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Exact merge of two attention states over disjoint key sets (``lkv_merge_states``).

    Outputs are bf16 ``[T, H, D]``; LSEs are fp32 natural-log tensors indexed ``[t, h]`` through
    their strides (pass ``lse.t()`` for an ``[H, T]`` tensor).  ``prefix_scale`` (fp32 ``[H]``)
    multiplies the prefix output in bf16 before the merge.  Returns ``(out, out_lse)``."""

    for name, t in (("prefix_out", prefix_out), ("suffix_out", suffix_out)):
        _require_bf16_cuda(name, t)
        _require(t.dim() == 3 and t.stride(-1) == 1, f"{name} must be [T, H, D] with contiguous rows")
    _require(prefix_out.shape == suffix_out.shape, "prefix and suffix outputs differ in shape")
    T, H, D = prefix_out.shape
    device = prefix_out.device
    for name, t in (("prefix_lse", prefix_lse), ("suffix_lse", suffix_lse), ("out_lse", out_lse)):
        if t is not None:
            _require(t.dtype == torch.float32 and t.device == device and tuple(t.shape) == (T, H),
                     f"{name} must be an fp32 [T, H] view on {device}")
    if prefix_scale is not None:
        _require(prefix_scale.dtype == torch.float32 and prefix_scale.numel() == H and prefix_scale.is_contiguous()
                 and prefix_scale.device == device, "prefix_scale must be a contiguous fp32 [H] tensor")
    if out is None:
        out = torch.empty_like(suffix_out)
    _require_bf16_cuda("out", out)
    _require(tuple(out.shape) == (T, H, D) and out.stride(-1) == 1, "out must be [T, H, D] with contiguous rows")
    a = _lib.MergeArgs()
    a.struct_size = ctypes.sizeof(_lib.MergeArgs)
    a.tokens, a.num_heads, a.head_dim = T, H, D
    a.prefix_out, a.prefix_out_stride_t, a.prefix_out_stride_h = prefix_out.data_ptr(), prefix_out.stride(0), prefix_out.stride(1)
    a.prefix_lse, a.prefix_lse_stride_t, a.prefix_lse_stride_h = prefix_lse.data_ptr(), prefix_lse.stride(0), prefix_lse.stride(1)
    a.suffix_out, a.suffix_out_stride_t, a.suffix_out_stride_h = suffix_out.data_ptr(), suffix_out.stride(0), suffix_out.stride(1)
    a.suffix_lse, a.suffix_lse_stride_t, a.suffix_lse_stride_h = suffix_lse.data_ptr(), suffix_lse.stride(0), suffix_lse.stride(1)
    a.prefix_scale = _ptr(prefix_scale)
    a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    if out_lse is not None:
        a.out_lse, a.out_lse_stride_t, a.out_lse_stride_h = out_lse.data_ptr(), out_lse.stride(0), out_lse.stride(1)
    _lib.check(_lib.load().lkv_merge_states(ctypes.byref(a), _stream(device)), "lkv_merge_states")
    return out, out_lse


def merge_attn_states(output, prefix_output, prefix_lse, suffix_output, suffix_lse, output_lse=None) -> None:
    """vLLM's ``merge_attn_states`` argument order (fastpath.py:709-719): LSEs are ``[H, T]``."""

    merge_states(prefix_output, prefix_lse.t(), suffix_output, suffix_lse.t(), out=output,
                 out_lse=None if output_lse is None else output_lse.t())


def merge_state(v_a, s_a, v_b, s_b):
    """FlashInfer's ``cascade.merge_state`` argument order (flashinfer_executor.py:185-231): LSEs
    ``[T, H]`` (natural log here); returns ``(v, s)``."""

    s = torch.empty_like(s_a)
    v, _ = merge_states(v_a, s_a, v_b, s_b, out_lse=s)
    return v, s


def _rows(name: str, t: torch.Tensor, heads: int) -> tuple[int, int, int]:
    """(ptr, stride_b, stride_t) of a [B, L, heads * 128] (or [B, L, heads, 128]) bf16 tensor."""

    _require_bf16_cuda(name, t)
    if t.dim() == 4:
        _require(t.shape[2] == heads and t.shape[3] == HEAD_DIM and t.stride(3) == 1 and t.stride(2) == HEAD_DIM,
                 f"{name} must be [B, L, {heads}, 128] with contiguous heads")
    else:
        _require(t.dim() == 3 and t.shape[2] == heads * HEAD_DIM and t.stride(2) == 1, f"{name} must be [B, L, {heads}*128]")
    _require(t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0 and t.data_ptr() % 16 == 0, f"{name} rows must be 16-byte aligned")
    return t.data_ptr(), t.stride(0), t.stride(1)


# rounding contracts of lkv_qkv_epilogue (lkv_qkv_args.rounding)
ROUNDINGS = {"torch": 0, "vllm": 1}


def qkv_epilogue(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    num_q_heads: int,
    num_kv_heads: int,
    q_norm_weight: torch.Tensor | None,
    k_norm_weight: torch.Tensor | None,
    eps: float,
    positions: int | torch.Tensor,
    ring: TiledKV | PagedKV,
    ring_slot: torch.Tensor | None = None,
    deep: TiledKV | PagedKV | None = None,
    deep_slot: torch.Tensor | None = None,
    q_out: torch.Tensor | None = None,
    ring_table: torch.Tensor | None = None,
    ring_tokens: int | None = None,
    deep_table: torch.Tensor | None = None,
    rounding: str = "torch",
    ring_v_mul: torch.Tensor | None = None,
    cu_seqlens: torch.Tensor | None = None,
    max_seqlen: int | None = None,
) -> torch.Tensor:
    """RoPE + q/k RMSNorm of the projections and the append of K/V to the layer ring (and, for
    the final layer, the shared cache) at positions ``positions + i``; returns the normalised
    queries ``[B, L, Hq, 128]``.  A PagedKV ring / deep store takes an int32 page table ``[B, W]``
    (``ring_tokens``: the ring length, default ``32 * W``).

    Ragged rows: with ``cu_seqlens`` (int32 ``[B + 1]`` on the device) ``q`` / ``k`` / ``v`` are
    ``[T, heads * 128]`` (or ``[T, heads, 128]``) and ``cos`` / ``sin`` ``[T, 128]`` (or ``[1, T,
    128]``), sequence b's tokens being rows ``cu[b] .. cu[b + 1] - 1`` at positions ``positions[b] +
    i``; ``max_seqlen`` bounds each sequence's count; returns ``[T, Hq, 128]``.

    ``rounding``: ``"torch"``, the HF model's bf16 op order, or ``"vllm"``, the reference's fused
    QKV kernel (single-FMA rotary, fixed RMSNorm summation order).  ``ring_v_mul`` ``[Hkv]`` fp32
    writes the ring's V as ``bf16(v * ring_v_mul[g])`` (the vLLM path's V / s rings); the shared
    cache keeps the raw V."""

    ragged = cu_seqlens is not None
    if ragged:
        _require(cu_seqlens.dtype == torch.int32 and cu_seqlens.dim() == 1 and cu_seqlens.numel() >= 2
                 and cu_seqlens.is_contiguous() and cu_seqlens.device == q.device,
                 "cu_seqlens must be a contiguous int32 [B + 1] tensor on the query's device")
        _require(max_seqlen is not None and int(max_seqlen) >= 1, "a ragged call needs max_seqlen >= 1")
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)  # [1, T, ...]
        if cos.dim() == 2:
            cos, sin = cos.unsqueeze(0), sin.unsqueeze(0)
        _require(cos.dim() == 3 and cos.shape[0] == 1, "ragged cos / sin must be [T, 128] or [1, T, 128]")
        if q_out is not None:
            _require(q_out.dim() == 3, "a ragged q_out must be [T, Hq, 128]")
            q_out = q_out.unsqueeze(0)
    else:
        _require(max_seqlen is None, "max_seqlen applies to ragged calls (cu_seqlens)")
    B, L = int(q.shape[0]), int(q.shape[1])
    qp, qsb, qst = _rows("q", q, num_q_heads)
    kp, ksb, kst = _rows("k", k, num_kv_heads)
    vp, vsb, vst = _rows("v", v, num_kv_heads)
    _require(tuple(k.shape[:2]) == (B, L) and tuple(v.shape[:2]) == (B, L), "q/k/v token shapes differ")
    for name, t in (("cos", cos), ("sin", sin)):
        _require_bf16_cuda(name, t)
        _require(t.dim() == 3 and t.shape[1] == L and t.shape[2] == HEAD_DIM and t.shape[0] in (1, B) and t.stride(2) == 1,
                 f"{name} must be [1 or B, L, 128]")
    _require(cos.stride() == sin.stride(), "cos and sin strides differ")
    device = q.device
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w is not None:
            _require_bf16_cuda(name, w)
            _require(w.numel() == HEAD_DIM and w.is_contiguous(), f"{name} must be a contiguous bf16 [128] tensor")
    _require(ring.heads == num_kv_heads, "ring kv heads mismatch")
    if q_out is None:
        q_out = torch.empty((B, L, num_q_heads, HEAD_DIM), dtype=torch.bfloat16, device=device)
    _require(q_out.is_contiguous() and tuple(q_out.shape) == (B, L, num_q_heads, HEAD_DIM), "q_out must be contiguous [B, L, Hq, 128]")
    _require(rounding in ROUNDINGS, f"rounding must be one of {sorted(ROUNDINGS)}, got {rounding!r}")
    if ring_v_mul is not None:
        _require(ring_v_mul.dtype == torch.float32 and ring_v_mul.numel() == num_kv_heads and ring_v_mul.is_contiguous()
                 and ring_v_mul.device == device, "ring_v_mul must be a contiguous fp32 [Hkv] tensor on the query's device")
    a = _lib.QkvArgs()
    a.struct_size = ctypes.sizeof(_lib.QkvArgs)
    NB = cu_seqlens.numel() - 1 if ragged else B  # sequences
    a.batch, a.tokens, a.num_q_heads, a.num_kv_heads, a.head_dim = NB, L, num_q_heads, num_kv_heads, HEAD_DIM
    if ragged:
        a.cu_seqlens, a.max_seqlen = cu_seqlens.data_ptr(), int(max_seqlen)
    a.rounding = ROUNDINGS[rounding]
    a.ring_v_mul = _ptr(ring_v_mul)
    a.eps = float(eps)
    a.positions, a.position_const = _len_arg(positions, NB, "positions", device)
    a.q, a.q_stride_b, a.q_stride_t = qp, qsb, qst
    a.k, a.k_stride_b, a.k_stride_t = kp, ksb, kst
    a.v, a.v_stride_b, a.v_stride_t = vp, vsb, vst
    a.cos, a.sin = cos.data_ptr(), sin.data_ptr()
    a.cs_stride_b = cos.stride(0) if cos.shape[0] == B and B > 1 else 0
    a.cs_stride_t = cos.stride(1)
    a.q_norm_w, a.k_norm_w = _ptr(q_norm_weight), _ptr(k_norm_weight)
    a.q_out, a.q_out_stride_b, a.q_out_stride_t = q_out.data_ptr(), q_out.stride(0), q_out.stride(1)
    a.ring_k, a.ring_v = ring.k.data_ptr(), ring.v.data_ptr()
    a.ring_head_stride = ring.head_stride
    if isinstance(ring, PagedKV):
        _table_arg(ring_table, NB, "ring", device)
        a.ring_block_table, a.ring_table_stride = ring_table.data_ptr(), ring_table.stride(0)
        a.ring_page_stride, a.ring_num_pages = ring.page_stride, ring.pages
        a.ring_tokens = int(ring_tokens if ring_tokens is not None else ring_table.shape[1] * BLOCK_TOKENS)
        _require(0 < a.ring_tokens <= ring_table.shape[1] * BLOCK_TOKENS and a.ring_tokens % BLOCK_TOKENS == 0,
                 "ring_tokens must be a multiple of 32 within the ring table")
    else:
        a.ring_seq_stride = ring.seq_stride
        a.ring_tokens, a.ring_num_slots, a.ring_slot = ring.capacity_tokens, ring.slots, _ptr(ring_slot)
    if deep is not None:
        _require(deep.heads == num_kv_heads, "deep kv heads mismatch")
        a.deep_k, a.deep_v = deep.k.data_ptr(), deep.v.data_ptr()
        a.deep_head_stride = deep.head_stride
        if isinstance(deep, PagedKV):
            _table_arg(deep_table, NB, "deep", device)
            a.deep_block_table, a.deep_table_stride = deep_table.data_ptr(), deep_table.stride(0)
            a.deep_page_stride, a.deep_num_pages = deep.page_stride, deep.pages
            a.deep_capacity_tokens = deep_table.shape[1] * BLOCK_TOKENS
        else:
            a.deep_seq_stride = deep.seq_stride
            a.deep_capacity_tokens, a.deep_num_slots, a.deep_slot = deep.capacity_tokens, deep.slots, _ptr(deep_slot)
        if not isinstance(positions, torch.Tensor):
            _require(positions + (int(max_seqlen) if ragged else L) <= a.deep_capacity_tokens,
                     "positions exceed the shared cache capacity")
    lib = _lib.load()
    _lib.check(lib.lkv_qkv_epilogue(ctypes.byref(a), _stream(device)), "lkv_qkv_epilogue")
    return q_out[0] if ragged else q_out


def blend_chunk(
    ring_k: torch.Tensor,
    ring_v: torch.Tensor,
    deep: TiledKV | PagedKV,
    *,
    batch: int,
    chunk_start: int,
    chunk_len: int,
    alpha: torch.Tensor,
    one_minus_alpha: torch.Tensor,
    vscale: torch.Tensor | None,
    ring_table: torch.Tensor | None = None,
    ring_tokens: int | None = None,
    deep_table: torch.Tensor | None = None,
) -> None:
    """Boundary commit: for every layer's ring blend tokens ``[chunk_start, chunk_start +
    chunk_len)`` with the shared cache in place.  ``alpha``, ``one_minus_alpha``, ``vscale``: fp32
    ``[layers * H]`` bf16 values.

    Contiguous rings: ``ring_k``/``ring_v`` ``[layers, slots, H, blocks, 4096]``.  Paged rings: a
    PagedKV pool's ``k``/``v`` (``[H, pages, 4096]``) and ``ring_table`` int32 ``[layers, batch, W]``
    (ring block rb of layer l, sequence b is page ``ring_table[l, b, rb]``; ``ring_tokens`` defaults
    to ``32 * W``).
    A PagedKV ``deep`` takes ``deep_table`` ``[batch, W']``."""

    for name, t in (("ring_k", ring_k), ("ring_v", ring_v)):
        _require_bf16_cuda(name, t)
    _require(ring_k.shape == ring_v.shape and ring_k.is_contiguous() and ring_v.is_contiguous(), "ring k/v must be contiguous and alike")
    device = deep.device
    a = _lib.BlendArgs()
    a.struct_size = ctypes.sizeof(_lib.BlendArgs)
    if ring_table is None:
        _require(ring_k.dim() == 5 and ring_k.shape[-1] == BLOCK_ELEMS, "ring_k must be [layers, slots, H, blocks, 4096]")
        layers, slots, H, blocks, _ = ring_k.shape
        _require(batch <= slots, "ring has fewer slots than sequences")
        a.ring_layer_stride, a.ring_seq_stride, a.ring_head_stride = ring_k.stride(0), ring_k.stride(1), ring_k.stride(2)
        a.ring_tokens = blocks * BLOCK_TOKENS
    else:
        _require(ring_k.dim() == 3 and ring_k.shape[-1] == BLOCK_ELEMS, "a paged ring pool must be [H, pages, 4096]")
        _require(ring_table.dtype == torch.int32 and ring_table.dim() == 3 and ring_table.shape[1] == batch
                 and ring_table.stride(2) == 1 and ring_table.device == device, "ring_table must be int32 [layers, batch, W]")
        layers, H, pages = int(ring_table.shape[0]), int(ring_k.shape[0]), int(ring_k.shape[1])
        a.ring_head_stride = pages * BLOCK_ELEMS
        a.ring_block_table = ring_table.data_ptr()
        a.ring_table_layer_stride, a.ring_table_stride = ring_table.stride(0), ring_table.stride(1)
        a.ring_page_stride, a.ring_num_pages = BLOCK_ELEMS, pages
        a.ring_tokens = int(ring_tokens if ring_tokens is not None else ring_table.shape[2] * BLOCK_TOKENS)
    _require(H == deep.heads, "ring/deep head counts differ")
    for name, t in (("alpha", alpha), ("one_minus_alpha", one_minus_alpha), ("vscale", vscale)):
        if t is not None:
            _require(t.dtype == torch.float32 and t.is_contiguous() and t.numel() == layers * H and t.device == device,
                     f"{name} must be a contiguous fp32 [layers * H] tensor")
    a.layers, a.batch, a.kv_heads, a.chunk_start, a.chunk_len = layers, batch, H, chunk_start, chunk_len
    a.ring_k, a.ring_v = ring_k.data_ptr(), ring_v.data_ptr()
    a.deep_k, a.deep_v = deep.k.data_ptr(), deep.v.data_ptr()
    a.deep_head_stride = deep.head_stride
    if isinstance(deep, PagedKV):
        _table_arg(deep_table, batch, "deep", device)
        a.deep_block_table, a.deep_table_stride = deep_table.data_ptr(), deep_table.stride(0)
        a.deep_page_stride, a.deep_num_pages = deep.page_stride, deep.pages
        a.deep_capacity_tokens = deep_table.shape[1] * BLOCK_TOKENS
    else:
        _require(batch <= deep.slots, "shared cache has fewer slots than sequences")
        a.deep_seq_stride, a.deep_capacity_tokens = deep.seq_stride, deep.capacity_tokens
    a.alpha, a.one_minus_alpha, a.vscale = alpha.data_ptr(), one_minus_alpha.data_ptr(), _ptr(vscale)
    _lib.check(_lib.load().lkv_blend_chunk(ctypes.byref(a), _stream(device)), "lkv_blend_chunk")


def append_paged(k: torch.Tensor, v: torch.Tensor, pool: PagedKV, table: torch.Tensor, *, token0: int,
                 wrap_tokens: int = 0) -> None:
    """Write ``k``/``v`` ``[B, T, H, 128]`` (any batch/token/head strides, unit dim stride) to
    absolute positions ``[token0, token0 + T)`` of each sequence's pages: position p lands at
    cache position ``p mod wrap_tokens`` (a ring) or ``p``, in page ``table[b, c // 32]``."""

    for name, t in (("k", k), ("v", v)):
        _require_bf16_cuda(name, t)
        _require(t.dim() == 4 and t.shape[-1] == HEAD_DIM and t.stride(-1) == 1, f"{name} must be [B, T, H, 128]")
    _require(k.shape == v.shape, "k and v shapes differ")
    B, T, H, _ = k.shape
    _require(H == pool.heads, "k/v heads differ from the pool's")
    _table_arg(table, B, "append", pool.device)
    a = _lib.AppendArgs()
    a.struct_size = ctypes.sizeof(_lib.AppendArgs)
    a.batch, a.tokens, a.heads, a.head_dim, a.token0, a.wrap_tokens = B, T, H, HEAD_DIM, int(token0), int(wrap_tokens)
    a.k, a.k_stride_b, a.k_stride_t, a.k_stride_h = k.data_ptr(), k.stride(0), k.stride(1), k.stride(2)
    a.v, a.v_stride_b, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1), v.stride(2)
    a.pool_k, a.pool_v = pool.k.data_ptr(), pool.v.data_ptr()
    a.page_stride, a.head_stride, a.num_pages = pool.page_stride, pool.head_stride, pool.pages
    a.block_table, a.table_stride, a.table_width = table.data_ptr(), table.stride(0), int(table.shape[1])
    _lib.check(_lib.load().lkv_append_paged(ctypes.byref(a), _stream(pool.device)), "lkv_append_paged")


def ring_tokens_for_chunk(chunk: int) -> int:
    """Ring capacity of one layer: the two live chunks, rounded up to whole 32-token blocks, plus
    one spare block when chunks straddle block boundaries (so no two blocks of one chunk share a
    ring block)."""

    _require(chunk >= 1, "chunk must be positive")
    ring = -(-2 * chunk // BLOCK_TOKENS) * BLOCK_TOKENS
    if chunk % BLOCK_TOKENS and BLOCK_TOKENS % chunk:
        ring += BLOCK_TOKENS
    return ring


def _rows2d(name: str, t: torch.Tensor) -> tuple[int, int, int]:
    """(rows, width, row stride) of a bf16 CUDA tensor viewed as [rows, width] with contiguous rows."""

    _require_bf16_cuda(name, t)
    _require(t.dim() >= 1 and t.stride(-1) == 1, f"{name} rows must be contiguous")
    width = t.shape[-1]
    if t.dim() == 1:
        return 1, width, width
    try:
        flat = t.view(-1, width)
    except RuntimeError:
        flat = None
    _require(flat is not None, f"{name} must be viewable as [rows, {width}] with one row stride")
    return flat.shape[0], width, flat.stride(0)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, *, residual: torch.Tensor | None = None,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """LlamaRMSNorm of the rows of ``x`` (bf16 ``[..., hidden]``); with ``residual`` first
    ``residual += x`` in bf16 (in place) and the sum is normalised.  Returns ``out``."""

    rows, hidden, xs = _rows2d("x", x)
    _require_bf16_cuda("weight", weight)
    _require(weight.is_contiguous() and weight.numel() == hidden, "weight must be a contiguous bf16 [hidden] tensor")
    rs = 0
    if residual is not None:
        r_rows, r_hidden, rs = _rows2d("residual", residual)
        _require((r_rows, r_hidden) == (rows, hidden), "residual shape must match x")
    if out is None:
        out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    o_rows, o_hidden, os_ = _rows2d("out", out)
    _require((o_rows, o_hidden) == (rows, hidden), "out shape must match x")
    a = _lib.NormArgs()
    a.struct_size = ctypes.sizeof(_lib.NormArgs)
    a.rows, a.hidden, a.eps = rows, hidden, float(eps)
    a.x, a.x_stride = x.data_ptr(), xs
    a.residual, a.residual_stride = _ptr(residual), rs
    a.weight = weight.data_ptr()
    a.out, a.out_stride = out.data_ptr(), os_
    _lib.check(_lib.load().lkv_rmsnorm(ctypes.byref(a), _stream(x.device)), "lkv_rmsnorm")
    return out


def silu_mul(gate: torch.Tensor, up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``F.silu(gate) * up`` for bf16 ``[..., width]`` tensors, as torch rounds it."""

    rows, width, gs = _rows2d("gate", gate)
    u_rows, u_width, us = _rows2d("up", up)
    _require((u_rows, u_width) == (rows, width), "up shape must match gate")
    if out is None:
        out = torch.empty(gate.shape, dtype=torch.bfloat16, device=gate.device)
    o_rows, o_width, os_ = _rows2d("out", out)
    _require((o_rows, o_width) == (rows, width), "out shape must match gate")
    _lib.check(_lib.load().lkv_silu_mul(gate.data_ptr(), gs, up.data_ptr(), us, out.data_ptr(), os_, rows, width,
                                        _stream(gate.device)), "lkv_silu_mul")
    return out


PROBE_THREADS = 256


def probe_read(src: torch.Tensor, workgroups: int = 256, sink: torch.Tensor | None = None) -> torch.Tensor:
    """One ``lkv_probe_read`` launch over the bytes of contiguous device tensor ``src`` (16-byte
    non-temporal loads, the decode kernel's access pattern); returns the sink it wrote."""

    _require(src.is_cuda and src.is_contiguous(), "src must be a contiguous device tensor")
    nbytes = src.numel() * src.element_size()
    if sink is None:
        sink = torch.empty(workgroups * PROBE_THREADS, dtype=torch.int32, device=src.device)
    _require(sink.numel() >= workgroups * PROBE_THREADS and sink.dtype == torch.int32, "sink too small")
    lib = _lib.load()
    _lib.check(lib.lkv_probe_read(src.data_ptr(), nbytes, sink.data_ptr(), workgroups, _stream(src.device)),
               "lkv_probe_read")
    return sink


def probe_mfma(device: torch.device | str, workgroups: int, iters: int, seed: int = 1,
               sink: torch.Tensor | None = None) -> tuple[torch.Tensor, int]:
    """One ``lkv_probe_mfma`` launch (``workgroups`` x 4 waves of independent bf16 MFMA chains on
    changing operands); returns (sink, FLOPs performed)."""

    device = torch.device(device)
    if sink is None:
        sink = torch.empty(workgroups * PROBE_THREADS, dtype=torch.int32, device=device)
    _require(sink.numel() >= workgroups * PROBE_THREADS and sink.dtype == torch.int32, "sink too small")
    lib = _lib.load()
    _lib.check(lib.lkv_probe_mfma(sink.data_ptr(), workgroups, iters, seed & 0xFFFFFFFF, _stream(device)),
               "lkv_probe_mfma")
    return sink, workgroups * 4 * iters * 8 * 16 * 16 * 32 * 2
