"""The C-ABI library loads, exports every declared entry point and rejects bad arguments (no GPU)."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

from lastkv_amd import _lib

HEADERS = sorted((pathlib.Path(__file__).resolve().parents[1] / "include").glob("*.h"))


def declared_functions() -> list[str]:
    names = []
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^[A-Za-z_][\w \*]*?\b(lkv_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert "lkv_decode_attn" in names and "lkv_cache_pack" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    # and the Python binding types each of them
    assert set(names) <= set(_lib.SIGNATURES), set(names) - set(_lib.SIGNATURES)


def test_abi_version_and_struct_size_guard():
    lib = _lib.load()
    assert lib.lkv_abi_version() == _lib.ABI_VERSION
    a = _lib.DecodeArgs()
    a.struct_size = ctypes.sizeof(a) - 8
    assert lib.lkv_decode_attn(ctypes.byref(a), None) == 1
    assert b"size mismatch" in lib.lkv_last_error()


@pytest.mark.parametrize(
    "field,value,message",
    [
        ("head_dim", 64, b"head_dim"),
        ("num_kv_heads", 3, b"multiple"),
        ("num_splits", 0, b"num_splits"),
        ("older_vscale_mode", 1, b"vscale"),
        ("kv_cache_hint", 3, b"kv_cache_hint"),
    ],
)
def test_decode_rejects_bad_arguments_before_any_launch(field, value, message):
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.struct_size = ctypes.sizeof(a)
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.num_splits = 1, 8, 2, 128, 1
    a.q = a.out = 16
    setattr(a, field, value)
    assert lib.lkv_decode_attn(ctypes.byref(a), None) == 1
    assert message in lib.lkv_last_error()


def test_decode_workspace_size():
    lib = _lib.load()
    assert lib.lkv_decode_workspace_bytes(32, 32, 1) == 0
    assert lib.lkv_decode_workspace_bytes(32, 32, 4) == 32 * 32 * 4 * 130 * 4


def test_pack_rejects_capacity_overflow():
    lib = _lib.load()
    st = lib.lkv_cache_pack(16, 0, 0, 128, 1, 1, 40, 0, 16, 0, 0, 0, 32, None)
    assert st == 1 and b"capacity" in lib.lkv_last_error()


@pytest.mark.parametrize("field,value,message", [("tile_waves", 5, b"tile_waves"), ("causal", 2, b"causal"),
                                                 ("head_dim", 96, b"head_dim")])
@pytest.mark.parametrize("batch", [0, 1])
def test_prefill_rejects_bad_arguments_before_any_launch(field, value, message, batch):
    """Checked before the empty-call early return, so a bad value never passes silently."""

    lib = _lib.load()
    a = _lib.PrefillArgs()
    a.struct_size = ctypes.sizeof(a)
    a.batch, a.tokens, a.num_q_heads, a.num_kv_heads, a.head_dim, a.causal = batch, 4, 8, 2, 128, 1
    a.q = a.out = 16
    setattr(a, field, value)
    assert lib.lkv_prefill_attn(ctypes.byref(a), None) == 1
    assert message in lib.lkv_last_error()


@pytest.mark.parametrize("local_len,ok_expected", [(3, False), (1, False), (4, True), (0, True)])
def test_prefill_causal_needs_the_queries_own_keys(local_len, ok_expected):
    """A causal call whose host-constant local length is shorter than its query count (but not
    empty) is rejected: the bottom-right rule would have to hide older keys from early rows."""

    lib = _lib.load()
    a = _lib.PrefillArgs()
    a.struct_size = ctypes.sizeof(a)
    a.batch, a.tokens, a.num_q_heads, a.num_kv_heads, a.head_dim, a.causal = 0, 4, 8, 2, 128, 1
    a.q = a.out = 16
    a.local_k = a.local_v = 16
    a.local_ring_blocks, a.local_num_slots, a.local_len_const = 1, 1, local_len
    status = lib.lkv_prefill_attn(ctypes.byref(a), None)
    if ok_expected:
        assert status == 0  # batch 0: validated, nothing launched
    else:
        assert status == 1 and b"local_len >= tokens" in lib.lkv_last_error()


@pytest.mark.parametrize("batch,splits,workspace,message", [(64, 16, 0, b"static scratch"), (1, 2, 64, b"workspace must be NULL")])
def test_noalloc_decode_rejections_before_any_launch(batch, splits, workspace, message):
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.struct_size = ctypes.sizeof(a)
    a.batch, a.num_q_heads, a.num_kv_heads, a.head_dim, a.num_splits = batch, 64, 8, 128, splits
    a.q = a.out = 16
    a.workspace, a.workspace_bytes = (16, workspace) if workspace else (None, 0)
    assert lib.lkv_decode_attn_noalloc(ctypes.byref(a), None) == 1
    assert message in lib.lkv_last_error()


@pytest.mark.parametrize("field,value,message", [("num_splits", 2000, b"num_splits"), ("max_seqlen_q", 0, b"max_seqlen_q")])
def test_prefill_ragged_and_split_arguments_rejected(field, value, message):
    """A ragged call (cu_seqlens_q set) needs max_seqlen_q >= 1; num_splits stays within [0, 1024]."""

    lib = _lib.load()
    a = _lib.PrefillArgs()
    a.struct_size = ctypes.sizeof(a)
    a.batch, a.tokens, a.num_q_heads, a.num_kv_heads, a.head_dim, a.causal = 2, 6, 8, 2, 128, 1
    a.q = a.out = a.cu_seqlens_q = 16
    a.max_seqlen_q = 4
    setattr(a, field, value)
    assert lib.lkv_prefill_attn(ctypes.byref(a), None) == 1
    assert message in lib.lkv_last_error()


def _qkv_args():
    a = _lib.QkvArgs()
    a.struct_size = ctypes.sizeof(a)
    a.batch, a.tokens, a.num_q_heads, a.num_kv_heads, a.head_dim = 1, 4, 8, 2, 128
    a.q = a.k = a.v = a.cos = a.sin = a.q_out = a.ring_k = a.ring_v = 16
    a.ring_tokens, a.ring_num_slots = 64, 1
    return a


@pytest.mark.parametrize("field,value,message", [("head_dim", 64, b"head_dim"), ("rounding", 2, b"rounding"),
                                                 ("ring_tokens", 40, b"multiple of 32"), ("q", None, b"null tensor"),
                                                 ("ring_num_slots", 0, b"ring_num_slots"),
                                                 ("position_const", -1, b"negative position")])
def test_epilogue_rejects_bad_arguments_before_any_launch(field, value, message):
    lib = _lib.load()
    a = _qkv_args()
    setattr(a, field, value)
    assert lib.lkv_qkv_epilogue(ctypes.byref(a), None) == 1
    assert message in lib.lkv_last_error()


@pytest.mark.parametrize("field,value,message", [("chunk_len", 96, b"chunk longer than the ring"),
                                                 ("deep_capacity_tokens", 32, b"deep capacity"),
                                                 ("alpha", None, b"null pointer"), ("kv_heads", 0, b"bad sizes")])
def test_blend_rejects_bad_arguments_before_any_launch(field, value, message):
    lib = _lib.load()
    a = _lib.BlendArgs()
    a.struct_size = ctypes.sizeof(a)
    a.layers, a.batch, a.kv_heads, a.chunk_start, a.chunk_len = 1, 1, 2, 32, 32
    a.ring_tokens, a.deep_capacity_tokens = 64, 128
    a.ring_k = a.ring_v = a.deep_k = a.deep_v = a.alpha = a.one_minus_alpha = 16
    setattr(a, field, value)
    assert lib.lkv_blend_chunk(ctypes.byref(a), None) == 1
    assert message in lib.lkv_last_error()
