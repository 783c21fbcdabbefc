"""Serving fast path over one paged K/V pool: the MI355X counterpart of the reference's vLLM
decode fast path (``vllm/src/lastkv/vllm/backends/rmarin_flashinfer/fastpath.py``), its fused
slab pool (``batching.py:1971-2122``) and the model runner that calls it per layer
(``vllm_model.py``, ``vllm_backend.py:637-664``).

``LastKVPagePool`` holds every sequence's K/V in 32-token pages of one head-major ``[Hkv, pages, 4096]`` pool
(K and V): per slot, the shared last-layer pages of its positions (handed out as the sequence
grows, like vLLM blocks) and, per layer, a fixed ring of ``ring_tokens_for_chunk(C)`` tokens (the
recent + current chunk, the reference's per-layer ring pages).  ``LastKVFastPath.prepare`` is the
host prologue of one step (``fastpath.py:455-575``, row plan ``:427-453``): boundary commits of
sequences that completed a chunk, and the per-row positions, key lengths, ring starts and page
table rows staged in device memory.  ``run_layer`` is the per-layer op sequence
(``fastpath.py:619-651``): the fused QKV epilogue (RoPE + q/k RMSNorm + ring append, plus the
shared append on the final layer) and one attention pass over [shared older pages | ring pages]
written into ``output``.  For a decode step every per-layer call reads only device-resident
metadata and preallocated buffers.

Two rounding contracts (``contract=``):
  - ``"hf"`` (default): the numbers of ``lastkv_amd.llm`` -- RoPE and RMSNorm in the torch op order,
    the older segment's V used as bf16(V * s_l) inside the attention kernel, the recent chunk
    blended once per boundary in bf16;
  - ``"vllm"``: the reference's merged serving path (``fastpath.py:619-651``, ``fused_qkv.py``) --
    RoPE with one FMA and one rounding per output and RMSNorm in the fused kernel's summation order,
    rings holding bf16(V * fp32(1 / s_l)) next to the raw V of the shared pages, one attention pass
    over both, the bf16 output rescaled by s_l (``_head_scale``), and the boundary blend of the rings
    with the unscaled shared V (``batching.py:1124-1140``).  The attention then reads every V as
    stored, with no per-element scaling of the older segment.
"""

from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np
import torch

from . import ops

BLOCK = ops.BLOCK_TOKENS


def plan_row(position: int, tokens: int, chunk: int, ring_tokens: int) -> tuple[int, int, int]:
    """Key segments of a row whose ``tokens`` new tokens start at ``position`` and stay inside one
    chunk: (older keys = rec, local keys = position + tokens - rec, ring start = rec mod R), with
    cur = floor(last / C) * C and rec = max(0, cur - C) (``access_plan.py:237-253``,
    ``fastpath.py:427-453``)."""

    if position < 0 or tokens < 1 or chunk < 1:
        raise ValueError("position >= 0, tokens >= 1 and chunk >= 1 are required")
    if position % chunk + tokens > chunk:
        raise ValueError(f"tokens [{position}, {position + tokens}) cross a chunk boundary of C={chunk}")
    rec = max(0, (position + tokens - 1) // chunk * chunk - chunk)
    local = position + tokens - rec
    if local > ring_tokens:
        raise ValueError("the ring cannot hold the local window")
    return rec, local, rec % ring_tokens


class PinnedStager:
    """Host-to-device copies of small host arrays through pinned staging slots, so that the host
    prologue never waits for the stream: each copy is queued behind the work already on it (the
    previous step), and a slot is rewritten only after the copy that last read it has completed."""

    def __init__(self, device: torch.device, slots: int = 16, nbytes: int = 1 << 16):
        self.device = device
        self.nbytes = nbytes
        self._bufs = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(slots)]
        self._done: list[torch.cuda.Event | None] = [None] * slots
        self._next = 0
        self._big: torch.Tensor | None = None
        self._big_done: torch.cuda.Event | None = None

    def copy(self, dst: torch.Tensor, src: np.ndarray) -> None:
        """``dst`` (a device tensor or view with the shape and dtype of ``src``) := ``src``."""

        src = np.ascontiguousarray(src)
        if src.nbytes > self.nbytes:  # large: one grow-on-demand buffer of its own
            if self._big is None or self._big.numel() < src.nbytes:
                if self._big_done is not None:
                    self._big_done.synchronize()
                self._big = torch.empty(src.nbytes, dtype=torch.uint8, pin_memory=True)
                self._big_done = None
            buf, i = self._big, -1
        else:
            i = self._next
            self._next = (i + 1) % len(self._bufs)
            buf = self._bufs[i]
        done = self._big_done if i < 0 else self._done[i]
        if done is not None:
            done.synchronize()
        staged = buf[: src.nbytes].view(dst.dtype).view(dst.shape)
        staged.copy_(torch.from_numpy(src))
        dst.copy_(staged, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        if i < 0:
            self._big_done = ev
        else:
            self._done[i] = ev


class PageAllocator:
    """Host bookkeeping of sequence slots and shared-cache pages: per slot a table row of page ids
    (unused entries name ``scratch``), pages handed out in order as a sequence grows and returned
    when its slot closes."""

    def __init__(self, *, max_slots: int, pages: int, width: int, scratch: int):
        self.width, self.scratch = width, scratch
        self.table = np.full((max_slots, width), scratch, dtype=np.int32)
        self.used = np.zeros(max_slots, dtype=np.int64)
        self._free_pages = list(range(pages - 1, -1, -1))
        self._free_slots = list(range(max_slots - 1, -1, -1))

    @property
    def free_pages(self) -> int:
        return len(self._free_pages)

    def open_slot(self) -> int:
        if not self._free_slots:
            raise RuntimeError("no free sequence slot in the pool")
        return self._free_slots.pop()

    def close_slot(self, slot: int) -> None:
        n = int(self.used[slot])
        self._free_pages.extend(int(p) for p in self.table[slot, :n][::-1])
        self.table[slot, :] = self.scratch
        self.used[slot] = 0
        self._free_slots.append(slot)

    def reserve(self, slot: int, tokens: int) -> tuple[int, int]:
        """Pages for positions ``[0, tokens)`` of ``slot``; returns the table columns it filled."""

        need = -(-tokens // BLOCK)
        if need > self.width:
            raise ValueError(f"sequence of {tokens} tokens exceeds the pool's {self.width * BLOCK} tokens per slot")
        have = int(self.used[slot])
        if need <= have:
            return have, have
        if need - have > len(self._free_pages):
            raise RuntimeError("the page pool is out of shared-cache pages")
        for j in range(have, need):
            self.table[slot, j] = self._free_pages.pop()
        self.used[slot] = need
        return have, need


class LastKVPagePool:
    """One head-major ``[Hkv, pages, 4096]`` K/V pool: shared last-layer pages (handed out per slot on demand)
    and per-layer ring pages (fixed per slot), plus one scratch page that padded rows and unused
    table entries name.  Device copies of the page tables sit beside the host bookkeeping."""

    def __init__(self, *, num_layers: int, kv_heads: int, chunk_size: int, max_slots: int, source_pages: int,
                 max_tokens_per_slot: int, device: torch.device | str):
        if min(num_layers, kv_heads, chunk_size, max_slots, source_pages, max_tokens_per_slot) < 1:
            raise ValueError("pool sizes must be positive")
        self.num_layers, self.kv_heads, self.chunk_size, self.max_slots = num_layers, kv_heads, chunk_size, max_slots
        self.device = torch.device(device)
        self.ring_tokens = ops.ring_tokens_for_chunk(chunk_size)
        self.ring_blocks = self.ring_tokens // BLOCK
        self.src_width = -(-max_tokens_per_slot // BLOCK)
        self.source_pages = source_pages
        ring_pages = num_layers * max_slots * self.ring_blocks
        self.scratch_page = source_pages + ring_pages
        self.pool = ops.PagedKV.zeros(self.scratch_page + 1, kv_heads, self.device)
        # ring pages: static table [L, slots, ring_blocks] behind the shared pages
        ring = source_pages + np.arange(ring_pages, dtype=np.int64).reshape(num_layers, max_slots, self.ring_blocks)
        self.ring_table = torch.from_numpy(ring.astype(np.int32)).to(self.device)
        self.pages = PageAllocator(max_slots=max_slots, pages=source_pages, width=self.src_width, scratch=self.scratch_page)
        self.src_table = torch.from_numpy(self.pages.table.copy()).to(self.device)
        self.stager = PinnedStager(self.device)
        self._dirty_lo, self._dirty_hi = max_slots, 0  # table rows changed since the last flush

    @property
    def free_pages(self) -> int:
        return self.pages.free_pages

    def open_slot(self) -> int:
        return self.pages.open_slot()

    def close_slot(self, slot: int) -> None:
        self.pages.close_slot(slot)
        self.src_table[slot].fill_(self.scratch_page)

    def reserve(self, slot: int, tokens: int) -> None:
        """Give ``slot`` shared pages for positions ``[0, tokens)`` (host table; ``flush`` copies
        the changed rows to the device table)."""

        lo, hi = self.pages.reserve(slot, tokens)
        if hi > lo:
            self._dirty_lo = min(self._dirty_lo, slot)
            self._dirty_hi = max(self._dirty_hi, slot + 1)

    def flush(self) -> None:
        """One host-to-device copy of the table rows changed since the last flush."""

        if self._dirty_hi > self._dirty_lo:
            lo, hi = self._dirty_lo, self._dirty_hi
            self.stager.copy(self.src_table[lo:hi], self.pages.table[lo:hi])
            self._dirty_lo, self._dirty_hi = self.max_slots, 0


@dataclass
class _Row:
    slot: int
    position: int  # first position of this step's tokens
    tokens: int
    older: int = 0  # older (shared) keys: rec = max(0, cur - C)
    local: int = 0  # ring keys: positions [rec, position + tokens)


class LastKVFastPath:
    """Per-step prologue and per-layer op sequence of the serving path over a LastKVPagePool.

    ``layer_params[l]`` = (q_norm_weight bf16 [128] or None, k_norm_weight or None, eps, vscale
    fp32 [Hkv] or None); ``blend`` = (alpha, one_minus_alpha, vscale-or-None), fp32 ``[L * Hkv]``
    as ``blend_chunk`` takes them; ``rotary(positions [B, n]) -> (cos, sin)`` bf16 ``[B, n, 128]``.
    ``from_model`` takes all three from a ``lastkv_amd.llm`` model.  ``num_splits`` fixes the
    decode split count (default: chosen per step from the longest row).  ``contract`` selects the
    rounding contract (module docstring): ``"hf"`` or ``"vllm"``."""

    def __init__(self, pool: LastKVPagePool, *, num_q_heads: int, layer_params, blend, rotary, max_batch: int,
                 num_splits: int | None = None, contract: str = "hf"):
        self.pool = pool
        self.num_q_heads = num_q_heads
        self.layer_params = list(layer_params)
        if len(self.layer_params) != pool.num_layers:
            raise ValueError("one parameter tuple per layer is required")
        if num_q_heads % pool.kv_heads:
            raise ValueError("num_q_heads must be a multiple of the pool's kv heads")
        if contract not in ("hf", "vllm"):
            raise ValueError(f"contract must be 'hf' or 'vllm', got {contract!r}")
        self.contract = contract
        # vLLM contract: per layer the ring's V multiplier fp32(1 / s) and the output scale s
        # (fastpath.py:254-267: scales must be finite and non-zero)
        self._ring_v_mul: list[torch.Tensor | None] = [None] * pool.num_layers
        if contract == "vllm":
            for l, (_, _, _, vs) in enumerate(self.layer_params):
                if vs is None:
                    continue
                if not bool(torch.isfinite(vs).all()) or bool((vs == 0).any()):
                    raise ValueError("value scales must be finite and non-zero for the vLLM contract")
                self._ring_v_mul[l] = (1.0 / vs.float()).contiguous()
        self.blend = blend
        self.rotary = rotary
        self.max_batch = max_batch
        self.num_splits = num_splits
        dev = pool.device
        self._seen = np.zeros(pool.max_slots, dtype=np.int64)
        self._committed = np.zeros(pool.max_slots, dtype=np.int64)  # boundary blended through
        self._open = np.zeros(pool.max_slots, dtype=bool)
        i32 = dict(dtype=torch.int32, device=dev)
        self._meta = torch.zeros((4, max_batch), **i32)  # positions, older_len, local_len, local_start
        self._cu = torch.zeros(max_batch + 1, **i32)  # row offsets of a ragged step (cu_seqlens)
        self._cu_host = None  # the same offsets on the host
        self._slots = torch.zeros(max_batch, dtype=torch.long, device=dev)
        self._older_table = torch.full((max_batch, pool.src_width), pool.scratch_page, **i32)
        self._ring_table = torch.full((pool.num_layers, max_batch, pool.ring_blocks), pool.scratch_page, **i32)
        self._cos1 = torch.zeros((max_batch, 1, ops.HEAD_DIM), dtype=torch.bfloat16, device=dev)
        self._sin1 = torch.zeros_like(self._cos1)
        self._q_out = torch.empty((max_batch, num_q_heads, ops.HEAD_DIM), dtype=torch.bfloat16, device=dev)
        self._decode_ws = torch.empty(16, dtype=torch.uint8, device=dev)
        self._prefill_ws = torch.empty(16, dtype=torch.uint8, device=dev)
        # The reference's runtime self-check (RMARIN_MERGED_CHECK, fastpath.py:198-202), also read as
        # LASTKV_MERGED_CHECK: "1" recomputes every eager layer call in two passes from the same pool
        # and reports the distance (_merged_check); "2" also hands the two-pass result to the model.
        mode = os.environ.get("LASTKV_MERGED_CHECK") or os.environ.get("RMARIN_MERGED_CHECK")
        self.check = mode in ("1", "2")
        self.check_replace = mode == "2"
        self._check_calls = 0
        self.rows: list[_Row] = []
        self.batch = 0  # rows of this step, padding included
        self.tokens = 0  # query tokens of this step, padding included
        self.splits = 1
        self.uniform = True  # every row of this step has the same token count
        self.max_rows = 1  # query tokens of this step's longest row
        self._row_rope: list[tuple[torch.Tensor, torch.Tensor]] = []

    @classmethod
    def from_model(cls, model, pool: LastKVPagePool, *, max_batch: int, num_splits: int | None = None,
                   contract: str = "hf") -> "LastKVFastPath":
        """Parameters of a ``lastkv_amd.llm`` decoder: its layers' q/k norms, V scales and blend gates."""

        inner = getattr(model, "model", model)
        cfg = inner.config
        params = []
        for layer in inner.layers:
            att = layer.self_attn
            qn = att.q_norm.weight if cfg.use_qk_norm else None
            kn = att.k_norm.weight if cfg.use_qk_norm else None
            params.append((qn, kn, cfg.rms_norm_eps, att._older_vscale()))

        def rotary(positions):
            cos, sin = inner.rotary(positions, torch.bfloat16)
            if cfg.use_nope:
                return torch.ones_like(cos), torch.zeros_like(sin)
            return cos, sin

        return cls(pool, num_q_heads=cfg.num_attention_heads, layer_params=params, blend=inner._blend_params(),
                   rotary=rotary, max_batch=max_batch, num_splits=num_splits, contract=contract)

    # -------------------------------------------------------------- sequences
    def add_sequence(self) -> int:
        slot = self.pool.open_slot()
        self._seen[slot] = self._committed[slot] = 0
        self._open[slot] = True
        return slot

    def free_sequence(self, slot: int) -> None:
        if not self._open[slot]:
            raise ValueError(f"slot {slot} is not in use")
        self._open[slot] = False
        self.pool.close_slot(slot)

    def seen(self, slot: int) -> int:
        return int(self._seen[slot])

    # -------------------------------------------------------------- host prologue
    def prepare(self, rows: list[tuple[int, int]], pad_to: int | None = None, num_splits: int | None = None) -> None:
        """Stage one step: ``rows`` = (slot, new tokens) per sequence, in the order their tokens
        appear in the step's q/k/v rows; each row continues its sequence at ``seen(slot)``.

        Commits the previous chunk of every row that starts on a chunk boundary (blend of every
        layer's ring with the shared pages, ``batching.py:1099-1155``; as in the reference it runs
        at the first step after the boundary), hands out shared pages, and copies positions,
        lengths, ring starts and table rows to device memory.  A row must not cross a chunk
        boundary (split prompts at multiples of C).  ``pad_to`` pads a decode step with empty rows
        that read and write only the scratch page.  ``num_splits`` fixes a decode step's key
        splits (default: the path's ``num_splits``, else chosen from the longest row)."""

        P = self.pool
        C = P.chunk_size
        if not rows:
            raise ValueError("a step needs at least one row")
        if len({r[0] for r in rows}) != len(rows):
            raise ValueError("a slot appears twice in one step")
        parsed = []
        for slot, n in rows:
            if not (0 <= slot < P.max_slots) or not self._open[slot]:
                raise ValueError(f"slot {slot} is not in use")
            p = int(self._seen[slot])
            rec, local, _ = plan_row(p, n, C, P.ring_tokens)
            parsed.append(_Row(slot, p, n, rec, local))
        uniform = all(r.tokens == parsed[0].tokens for r in parsed)
        B = len(parsed)
        Bp = B if pad_to is None else max(B, int(pad_to))
        if pad_to is not None and not (uniform and parsed[0].tokens == 1):
            raise ValueError("pad_to applies to decode steps (one token per row)")
        if Bp > self.max_batch:
            raise ValueError(f"{Bp} rows exceed max_batch {self.max_batch}")
        for r in parsed:
            P.reserve(r.slot, r.position + r.tokens)
        P.flush()
        for r in parsed:
            if r.position > 0 and r.position % C == 0 and self._committed[r.slot] < r.position:
                self._commit(r.slot, r.position)
        meta = np.zeros((4, Bp), dtype=np.int32)  # padded rows: position 0, no keys
        for b, r in enumerate(parsed):
            meta[:, b] = (r.position, r.older, r.local, r.older % P.ring_tokens)
        P.stager.copy(self._meta[:, :Bp], meta)
        slots = self._slots[:B]
        P.stager.copy(slots, np.array([r.slot for r in parsed], dtype=np.int64))
        self._older_table[:B].copy_(P.src_table.index_select(0, slots))
        self._ring_table[:, :B].copy_(P.ring_table.index_select(1, slots))
        if Bp > B:
            self._older_table[B:Bp].fill_(P.scratch_page)
            self._ring_table[:, B:Bp].fill_(P.scratch_page)
        Hq = self.num_q_heads
        self.tokens = sum(r.tokens for r in parsed) + (Bp - B)
        if uniform and parsed[0].tokens == 1:
            cos, sin = self.rotary(self._meta[0, :Bp].long()[:, None])
            self._cos1[:Bp].copy_(cos)
            self._sin1[:Bp].copy_(sin)
            keys = max(r.older + r.local for r in parsed)
            self.splits = num_splits or self.num_splits or ops.default_decode_splits(Bp, P.kv_heads, keys,
                                                                                      ops._cu_count(P.device))
            need = ops.decode_workspace_bytes(Bp, Hq, self.splits)
            if self._decode_ws.numel() < need:
                self._decode_ws = torch.empty(need, dtype=torch.uint8, device=P.device)
        else:
            if uniform:
                n = parsed[0].tokens
                pos = self._meta[0, :B].long()[:, None] + torch.arange(n, device=P.device)[None, :]
            else:
                # ragged step: the rows' tokens back to back (cu_seqlens), RoPE rows for each
                cu = np.zeros(B + 1, dtype=np.int32)
                cu[1:] = np.cumsum([r.tokens for r in parsed])
                P.stager.copy(self._cu[:B + 1], cu)
                self._cu_host = cu  # (the attention call plans its launches from the host copy)
                pos = torch.from_numpy(np.concatenate([np.arange(r.position, r.position + r.tokens)
                                                       for r in parsed])).to(P.device, non_blocking=True)[None, :]
            self._row_rope = [self.rotary(pos)]
            # device-resident lengths: the kernel sizes its fp16 V copy by the older table's width
            # and the whole ring (a ragged call's short rows share it for their split state)
            width = max(1, -(-max(r.older for r in parsed) // BLOCK))
            # (with room for the tile kernel's key splits, which steps of few prefill rows take)
            need = ops.prefill_workspace_bytes(B, P.kv_heads, width * BLOCK, P.ring_tokens, query_rows=self.tokens,
                                               num_q_heads=Hq, cu_count=ops._cu_count(P.device))
            if uniform:
                need = max(need, ops.prefill_split_state_bytes(self.tokens, Hq, self.num_splits or 0))
            else:
                need = max(need, ops.ragged_split_state_bytes(B, Hq, P.kv_heads, max(r.tokens for r in parsed),
                                                              self.num_splits or 0, ops._cu_count(P.device)))
            if self._prefill_ws.numel() < need:
                self._prefill_ws = torch.empty(need, dtype=torch.uint8, device=P.device)
        if self._q_out.shape[0] < self.tokens:
            self._q_out = torch.empty((self.tokens, Hq, ops.HEAD_DIM), dtype=torch.bfloat16, device=P.device)
        for r in parsed:
            self._seen[r.slot] = r.position + r.tokens
        self.rows, self.batch, self.uniform = parsed, Bp, uniform
        self.max_rows = max(r.tokens for r in parsed)

    def _commit(self, slot: int, boundary: int) -> None:
        """Blend chunk [boundary - C, boundary) of every layer's ring of ``slot`` with its shared pages."""

        P = self.pool
        alpha, om, s = self.blend
        if self.contract == "vllm":  # rings hold V / s: blend with the unscaled shared V
            s = None
        ops.blend_chunk(P.pool.k, P.pool.v, P.pool, batch=1, chunk_start=boundary - P.chunk_size, chunk_len=P.chunk_size,
                        alpha=alpha, one_minus_alpha=om, vscale=s, ring_table=P.ring_table[:, slot:slot + 1],
                        ring_tokens=P.ring_tokens, deep_table=P.src_table[slot:slot + 1])
        self._committed[slot] = boundary

    # -------------------------------------------------------------- per-layer op sequence
    def run_layer(self, layer_index: int, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                  output: torch.Tensor) -> torch.Tensor:
        """``query`` ``[T, Hq * 128]`` (or ``[T, Hq, 128]``), ``key``/``value`` ``[T, Hkv * 128]``
        (row views of a fused projection are fine): this step's projections, rows in ``prepare``
        order.  Writes the attention output ``[T, Hq, 128]`` (contiguous) and returns it."""

        P = self.pool
        B, T = self.batch, self.tokens
        Hq, Hkv = self.num_q_heads, P.kv_heads
        if min(query.shape[0], key.shape[0], value.shape[0], output.shape[0]) < T:
            raise ValueError(f"this step has {T} query tokens")
        qn_w, kn_w, eps, vs = self.layer_params[layer_index]
        # vLLM contract: rings of V / s (the epilogue scales the ring's V), attention over V as stored,
        # output rescaled by s; HF contract: the older segment's V scaled inside the attention
        vllm = self.contract == "vllm"
        epi = dict(rounding="vllm", ring_v_mul=self._ring_v_mul[layer_index]) if vllm else {}
        out_scale = vs if vllm else None
        if vllm:
            vs = None
        top = layer_index == P.num_layers - 1
        ring_tab = self._ring_table[layer_index]
        pos, older_len, local_len, local_start = self._meta
        n = self.rows[0].tokens
        if self.uniform:  # every row has n tokens (padding only for n == 1)
            cos, sin = (self._cos1[:B], self._sin1[:B]) if n == 1 else self._row_rope[0]
            q_out = ops.qkv_epilogue(
                query[:T].reshape(B, n, Hq * 128), key[:T].reshape(B, n, Hkv * 128), value[:T].reshape(B, n, Hkv * 128),
                cos, sin, num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=qn_w, k_norm_weight=kn_w, eps=eps,
                positions=pos[:B], ring=P.pool, ring_table=ring_tab[:B], ring_tokens=P.ring_tokens,
                deep=P.pool if top else None, deep_table=self._older_table[:B] if top else None,
                q_out=self._q_out[:T].view(B, n, Hq, 128), **epi)
            seg = dict(older=P.pool, older_table=self._older_table[:B], older_len=older_len[:B], vscale=vs, local=P.pool,
                       local_table=ring_tab[:B], local_ring_blocks=P.ring_blocks, local_len=local_len[:B],
                       local_start=local_start[:B], out_scale=out_scale)
            if n == 1:
                ops.decode_attention(q_out.view(B, Hq, 128), out=output[:T].view(B, Hq, 128), num_splits=self.splits,
                                     workspace=self._decode_ws, **seg)
            else:
                width = max(1, -(-max(r.older for r in self.rows) // BLOCK))
                seg["older_table"] = self._older_table[:B, :width]
                ops.prefill_attention(q_out, causal=True, out=output[:T].view(B, n, Hq, 128),
                                      workspace=self._prefill_ws, num_splits=self.num_splits or 0, **seg)
            if self.check:
                self._merged_check(layer_index, q_out.view(B, n, Hq, 128), output[:T].view(B, n, Hq, 128), seg)
            return output
        # ragged step (prefill pieces and decode tokens of different lengths): one epilogue and one
        # attention call over the rows back to back (cu_seqlens), as the reference's single varlen
        # FA3 call per layer (fastpath.py:643-648)
        cu = self._cu[:B + 1]
        cos, sin = self._row_rope[0]
        q_out = ops.qkv_epilogue(
            query[:T].reshape(T, Hq * 128), key[:T].reshape(T, Hkv * 128), value[:T].reshape(T, Hkv * 128),
            cos, sin, num_q_heads=Hq, num_kv_heads=Hkv, q_norm_weight=qn_w, k_norm_weight=kn_w, eps=eps,
            positions=pos[:B], ring=P.pool, ring_table=ring_tab[:B], ring_tokens=P.ring_tokens,
            deep=P.pool if top else None, deep_table=self._older_table[:B] if top else None,
            q_out=self._q_out[:T], cu_seqlens=cu, max_seqlen=self.max_rows, **epi)
        width = max(1, -(-max(r.older for r in self.rows) // BLOCK))
        seg = dict(older=P.pool, older_table=self._older_table[:B, :width], older_len=older_len[:B], vscale=vs,
                   local=P.pool, local_table=ring_tab[:B], local_ring_blocks=P.ring_blocks, local_len=local_len[:B],
                   local_start=local_start[:B], out_scale=out_scale)
        ops.prefill_attention(q_out, causal=True, out=output[:T].view(T, Hq, 128), workspace=self._prefill_ws,
                              cu_seqlens_q=cu, max_seqlen_q=self.max_rows, num_splits=self.num_splits or 0,
                              cu_seqlens_q_host=self._cu_host, **seg)
        if self.check:
            self._merged_check(layer_index, q_out, output[:T].view(T, Hq, 128), seg, ragged=(cu, self.max_rows))
        return output

    def _merged_check(self, layer_index: int, q: torch.Tensor, out: torch.Tensor, seg: dict, ragged=None) -> None:
        """The reference's merged-path self-check (``_merged_check``, fastpath.py:737-773): the layer
        call again in two passes from the same pool, the older segment alone (every key visible) and
        the ring segment alone (bottom-right causal), each with its LSE, merged exactly
        (``merge_states``; a sequence without older keys has LSE -inf there); prints the relative L2
        distance of the one-pass output to it for the first 192 calls and for any call above 0.02,
        and with ``check_replace`` writes the two-pass result into ``out``.  Eager calls only: a call
        made under HIP graph capture is not checked."""

        if torch.cuda.is_current_stream_capturing():
            return
        H = out.shape[-2]
        rg = {} if ragged is None else dict(cu_seqlens_q=ragged[0], max_seqlen_q=ragged[1])
        older = {k: seg[k] for k in ("older", "older_table", "older_len", "vscale")}
        local = {k: seg[k] for k in ("local", "local_table", "local_ring_blocks", "local_len", "local_start")}
        so, lo = torch.empty_like(out), torch.empty_like(out)
        sl = torch.empty(out.shape[:-1], dtype=torch.float32, device=out.device)
        ll = torch.empty_like(sl)
        ops.prefill_attention(q, causal=False, out=so, lse=sl, out_scale=seg["out_scale"], **older, **rg)
        ops.prefill_attention(q, causal=True, out=lo, lse=ll, out_scale=seg["out_scale"], **local, **rg)
        ref, _ = ops.merge_states(so.reshape(-1, H, ops.HEAD_DIM), sl.reshape(-1, H), lo.reshape(-1, H, ops.HEAD_DIM),
                                  ll.reshape(-1, H))
        real = sum(r.tokens for r in self.rows)  # (a padded decode step's empty rows follow)
        got, want = out.reshape(-1, H, ops.HEAD_DIM)[:real].float(), ref[:real].float()
        rel = float((want - got).norm() / want.norm().clamp(min=1e-6))
        self._check_calls += 1
        if self._check_calls <= 32 * 6 or rel > 0.02:
            print({"lastkv_merged_check": {"layer": layer_index, "batch": len(self.rows), "tokens": real,
                                           "older": [r.older for r in self.rows][:4],
                                           "local": [r.local for r in self.rows][:4], "rel": round(rel, 5),
                                           "out_absmax": round(float(got.abs().max()), 2),
                                           "ref_absmax": round(float(want.abs().max()), 2)}}, flush=True)
        if self.check_replace:
            out.reshape(-1, H, ops.HEAD_DIM)[:real].copy_(ref[:real])


def fuse_linears(mods) -> tuple[torch.Tensor, torch.Tensor | None]:
    """One ``[sum(out), in]`` weight (and bias) for ``nn.Linear`` modules that read the same input,
    as vLLM's ``QKVParallelLinear`` / ``MergedColumnParallelLinear`` hold them: the modules' own
    parameters are re-pointed to row ranges of the fused tensors (values unchanged, no second
    copy), so one GEMM produces every module's output as a column range.  Modules already fused
    this way (an earlier runner over the same model) keep their buffers."""

    mods = list(mods)
    have = getattr(mods[0], "_lkv_fused", None)
    if have is not None and len(have[0]) == len(mods) and all(a is b for a, b in zip(have[0], mods)) and all(
            m.weight.data_ptr() == have[1][r0:].data_ptr() for m, r0 in zip(mods, have[3])):
        return have[1], have[2]
    weight = torch.cat([m.weight.detach() for m in mods])
    with_bias = [m.bias is not None for m in mods]
    if any(with_bias) and not all(with_bias):
        raise ValueError("fused projections must all have a bias or none")
    bias = torch.cat([m.bias.detach() for m in mods]) if all(with_bias) else None
    r0, starts = 0, []
    for m in mods:
        rows = m.weight.shape[0]
        starts.append(r0)
        m.weight.data = weight[r0:r0 + rows]
        if bias is not None:
            m.bias.data = bias[r0:r0 + rows]
        r0 += rows
    mods[0]._lkv_fused = (mods, weight, bias, starts)
    return weight, bias


class LastKVServingModel:
    """Continuous-batching runner of a ``lastkv_amd.llm`` causal LM over a LastKVFastPath: one
    ``step`` runs the decoder over ragged rows (prefill pieces and decode tokens of different
    sequences in one batch), the role of the reference's vLLM model class + backend forward
    (``vllm_model.py``, ``vllm_backend.py:637-664``).  Norms and the MLP's down projection are the
    model's own modules; q / k / v and gate / up run as one GEMM each over weights fused in place
    (``fuse_linears``, the layout of vLLM's ``qkv_proj`` / ``gate_up_proj``): at decode (M = 32 rows)
    hipBLASLt takes ~19 us per projection GEMM whatever its width, so three q / k / v GEMMs cost
    59 us per layer against 19 us for the fused one."""

    def __init__(self, model, *, max_batch: int, max_tokens_per_slot: int, source_pages: int | None = None,
                 num_splits: int | None = None, device=None, contract: str = "hf"):
        self.model = model
        inner = model.model
        cfg = inner.config
        if cfg.head_dim != ops.HEAD_DIM:
            raise ValueError(f"the MI355X kernels support head_dim {ops.HEAD_DIM}")
        device = device or next(model.parameters()).device
        per_slot = -(-max_tokens_per_slot // BLOCK)
        self.pool = LastKVPagePool(num_layers=cfg.num_hidden_layers, kv_heads=cfg.num_key_value_heads,
                                   chunk_size=cfg.chunk_size, max_slots=max_batch,
                                   source_pages=source_pages or max_batch * per_slot,
                                   max_tokens_per_slot=max_tokens_per_slot, device=device)
        self.fast = LastKVFastPath.from_model(model, self.pool, max_batch=max_batch, num_splits=num_splits,
                                              contract=contract)
        self.config = cfg
        self._qkv = [fuse_linears((l.self_attn.q_proj, l.self_attn.k_proj, l.self_attn.v_proj)) for l in inner.layers]
        self._gate_up = [fuse_linears((l.mlp.gate_proj, l.mlp.up_proj)) for l in inner.layers]

    def add_sequence(self) -> int:
        return self.fast.add_sequence()

    def free_sequence(self, slot: int) -> None:
        self.fast.free_sequence(slot)

    @torch.no_grad()
    def step(self, rows: list[tuple[int, torch.Tensor]], pad_to: int | None = None) -> torch.Tensor:
        """``rows`` = (slot, new token ids [n]); returns the logits of each row's last token ``[B, vocab]``."""

        self.fast.prepare([(slot, int(ids.numel())) for slot, ids in rows], pad_to=pad_to)
        T = self.fast.tokens
        ids = torch.cat([ids.reshape(-1).to(self.pool.device) for _, ids in rows])
        if T > ids.numel():
            ids = torch.cat([ids, ids.new_zeros(T - ids.numel())])
        normed = self._layers(ids)
        last = torch.tensor(np.cumsum([int(ids.numel()) for _, ids in rows]) - 1, device=normed.device)
        return self.model.lm_head(normed.index_select(0, last))

    def _layers(self, ids: torch.Tensor) -> torch.Tensor:
        """Device part of a prepared step: embeddings and every decoder layer over the step's
        ``[T]`` token ids; returns the final norm's output ``[T, hidden]``.  The residual adds and
        RMSNorms run fused (``lkv_rmsnorm``, LlamaRMSNorm arithmetic) and the MLP's SiLU product as
        ``lkv_silu_mul``, the roles of vLLM's fused_add_rms_norm and silu_and_mul."""

        inner = self.model.model
        layers = inner.layers
        eps = self.config.rms_norm_eps
        T = ids.numel()
        hidden = inner.embed_tokens(ids)  # the residual stream, updated in place
        Hq = self.config.num_attention_heads
        out = torch.empty((T, Hq, ops.HEAD_DIM), dtype=hidden.dtype, device=hidden.device)
        widths = [Hq * ops.HEAD_DIM, self.config.num_key_value_heads * ops.HEAD_DIM]
        widths.append(widths[1])
        inter = self.config.intermediate_size
        h = ops.rmsnorm(hidden, layers[0].input_layernorm.weight, eps)
        for i, layer in enumerate(layers):
            att, mlp = layer.self_attn, layer.mlp
            q, k, v = torch.nn.functional.linear(h, *self._qkv[i]).split(widths, dim=-1)
            self.fast.run_layer(i, q, k, v, out)
            h = ops.rmsnorm(att.o_proj(out.view(T, Hq * ops.HEAD_DIM)), layer.post_attention_layernorm.weight, eps,
                            residual=hidden)
            gate_up = torch.nn.functional.linear(h, *self._gate_up[i])
            m = mlp.down_proj(ops.silu_mul(gate_up[:, :inter], gate_up[:, inter:]))
            nxt = layers[i + 1].input_layernorm.weight if i + 1 < len(layers) else inner.norm.weight
            h = ops.rmsnorm(m, nxt, eps, residual=hidden)
        return h

    def decode_graph(self, slots: list[int], num_splits: int | None = None) -> "DecodeGraph":
        """A HIP-graph replay of greedy decode steps for ``slots`` (one token each per step)."""

        return DecodeGraph(self, slots, num_splits)

    @torch.no_grad()
    def generate(self, prompts: list[torch.Tensor], max_new_tokens: int, *, prefill_chunk: int | None = None
                 ) -> list[torch.Tensor]:
        """Greedy continuous batching: every step carries each unfinished sequence's next prompt
        piece (cut at chunk boundaries and at ``prefill_chunk``) or its last generated token.
        Returns each prompt followed by its ``max_new_tokens`` generated ids."""

        C = self.config.chunk_size
        slots = [self.add_sequence() for _ in prompts]
        fed = [0] * len(prompts)  # prompt tokens fed so far
        gen: list[list[int]] = [[] for _ in prompts]
        try:
            while any(len(g) < max_new_tokens for g in gen):
                rows, owners = [], []
                for i, (slot, prompt) in enumerate(zip(slots, prompts)):
                    if len(gen[i]) >= max_new_tokens:
                        continue
                    flat = prompt.reshape(-1)
                    if fed[i] < flat.numel():
                        p = self.fast.seen(slot)
                        take = min(flat.numel() - fed[i], C - p % C, prefill_chunk or flat.numel())
                        rows.append((slot, flat[fed[i]:fed[i] + take]))
                        fed[i] += take
                    else:
                        rows.append((slot, torch.tensor([gen[i][-1]], dtype=flat.dtype)))
                    owners.append(i)
                tokens = self.step(rows).argmax(-1).tolist()
                for i, tok in zip(owners, tokens):
                    if fed[i] >= prompts[i].numel():
                        gen[i].append(int(tok))
        finally:
            for slot in slots:
                self.free_sequence(slot)
        return [torch.cat([p.reshape(-1).cpu(), torch.tensor(g, dtype=p.dtype)]) for p, g in zip(prompts, gen)]


class DecodeGraph:
    """Greedy decode steps of a fixed set of sequences, one token each, replayed from one HIP graph.

    The host prologue of a step (``LastKVFastPath.prepare``: boundary commits, page hand-out, and
    positions, key lengths, ring starts, page-table rows and RoPE rows written into persistent
    device buffers) runs eagerly before every replay.  The captured part is the device work of the
    step: embeddings, every layer's projections, fused QKV epilogue, paged decode attention, o_proj
    and MLP, the final norm, lm_head and the argmax, all reading only those buffers.  This is the
    reference's graph-captured decode fast path (``fastpath.py:1-9``, ``:619-651``).  The split
    count is fixed for the graph's lifetime (default: the one for the longest context a slot can
    reach), so that every captured kernel argument stays valid."""

    def __init__(self, runner: "LastKVServingModel", slots: list[int], num_splits: int | None = None):
        if not slots:
            raise ValueError("a decode graph needs at least one slot")
        self.runner = runner
        self.slots = list(slots)
        fast, pool = runner.fast, runner.pool
        B = len(self.slots)
        if B > fast.max_batch:
            raise ValueError(f"{B} slots exceed max_batch {fast.max_batch}")
        max_keys = pool.src_width * BLOCK + pool.ring_tokens
        self.num_splits = num_splits or fast.num_splits or ops.default_decode_splits(
            B, pool.kv_heads, max_keys, ops._cu_count(pool.device))
        self.ids = torch.zeros(B, dtype=torch.long, device=pool.device)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.logits: torch.Tensor | None = None
        self.tokens: torch.Tensor | None = None
        self._key = None

    def _device_step(self):
        logits = self.runner.model.lm_head(self.runner._layers(self.ids))
        return logits, logits.argmax(-1)

    def _buffers(self):
        f = self.runner.fast
        return (f.splits, f.batch, f.tokens, f._decode_ws.data_ptr(), f._q_out.data_ptr(), f._meta.data_ptr(),
                f._older_table.data_ptr(), f._ring_table.data_ptr(), f._cos1.data_ptr(), f._sin1.data_ptr())

    @torch.no_grad()
    def step(self, tokens: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Feed ``tokens`` (``[B]`` ids on the device, one per slot in order) and return
        (logits ``[B, vocab]``, greedy next ids ``[B]``), views of the graph's outputs that the next
        step overwrites."""

        fast = self.runner.fast
        fast.prepare([(slot, 1) for slot in self.slots], num_splits=self.num_splits)
        self.ids.copy_(tokens.reshape(-1))
        key = self._buffers()
        if self.graph is None:
            # warm-up run (library handles, allocator); it writes this step's K/V, which the
            # replay below writes again with the same values
            self._device_step()
            torch.cuda.current_stream().synchronize()
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.logits, self.tokens = self._device_step()
            self._key = key
        elif key != self._key:
            raise RuntimeError("the decode graph's buffers changed since capture (split count or workspace)")
        self.graph.replay()
        return self.logits, self.tokens
