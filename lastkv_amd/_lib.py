"""ctypes binding of ``liblastkv_amd.so`` (the C ABI in ``include/lastkv_amd.h``).

The library is loaded lazily from this package directory.  There is no fallback: if it is
missing, every op raises ``LastKVNativeError`` naming the build command.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / "liblastkv_amd.so"
ABI_VERSION = 11


class LastKVNativeError(RuntimeError):
    """A C-ABI call failed, or the native library is unavailable."""


c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_ptr = ctypes.c_void_p


class DecodeArgs(ctypes.Structure):
    """Mirror of ``lkv_decode_args``."""

    _fields_ = [
        ("struct_size", c_i32),
        ("batch", c_i32),
        ("num_q_heads", c_i32),
        ("num_kv_heads", c_i32),
        ("head_dim", c_i32),
        ("num_splits", c_i32),
        ("sm_scale", c_f32),
        ("older_vscale_mode", c_i32),
        ("q", c_ptr),
        ("q_stride_b", c_i64),
        ("out", c_ptr),
        ("out_stride_b", c_i64),
        ("lse", c_ptr),
        ("older_k", c_ptr),
        ("older_v", c_ptr),
        ("older_seq_stride", c_i64),
        ("older_head_stride", c_i64),
        ("older_len", c_ptr),
        ("older_len_const", c_i32),
        ("older_capacity_tokens", c_i32),
        ("older_slot", c_ptr),
        ("older_num_slots", c_i32),
        ("vscale", c_ptr),
        ("local_k", c_ptr),
        ("local_v", c_ptr),
        ("local_seq_stride", c_i64),
        ("local_head_stride", c_i64),
        ("local_ring_blocks", c_i32),
        ("local_len_const", c_i32),
        ("local_len", c_ptr),
        ("local_start", c_ptr),
        ("local_start_const", c_i32),
        ("local_slot", c_ptr),
        ("local_num_slots", c_i32),
        ("workspace", c_ptr),
        ("workspace_bytes", c_i64),
        ("older_block_table", c_ptr),
        ("older_table_stride", c_i64),
        ("older_page_stride", c_i64),
        ("older_num_pages", c_i32),
        ("local_block_table", c_ptr),
        ("local_table_stride", c_i64),
        ("local_page_stride", c_i64),
        ("local_num_pages", c_i32),
        ("kv_cache_hint", c_i32),
        ("out_scale", c_ptr),
    ]


class PrefillArgs(ctypes.Structure):
    """Mirror of ``lkv_prefill_args``."""

    _fields_ = [
        ("struct_size", c_i32),
        ("batch", c_i32),
        ("tokens", c_i32),
        ("num_q_heads", c_i32),
        ("num_kv_heads", c_i32),
        ("head_dim", c_i32),
        ("sm_scale", c_f32),
        ("causal", c_i32),
        ("older_vscale_mode", c_i32),
        ("q", c_ptr),
        ("q_stride_b", c_i64),
        ("q_stride_t", c_i64),
        ("out", c_ptr),
        ("out_stride_b", c_i64),
        ("out_stride_t", c_i64),
        ("lse", c_ptr),
        ("older_k", c_ptr),
        ("older_v", c_ptr),
        ("older_seq_stride", c_i64),
        ("older_head_stride", c_i64),
        ("older_len", c_ptr),
        ("older_len_const", c_i32),
        ("older_capacity_tokens", c_i32),
        ("older_slot", c_ptr),
        ("older_num_slots", c_i32),
        ("vscale", c_ptr),
        ("local_k", c_ptr),
        ("local_v", c_ptr),
        ("local_seq_stride", c_i64),
        ("local_head_stride", c_i64),
        ("local_ring_blocks", c_i32),
        ("local_len_const", c_i32),
        ("local_len", c_ptr),
        ("local_start", c_ptr),
        ("local_start_const", c_i32),
        ("local_slot", c_ptr),
        ("local_num_slots", c_i32),
        ("workspace", c_ptr),
        ("workspace_bytes", c_i64),
        ("older_block_table", c_ptr),
        ("older_table_stride", c_i64),
        ("older_page_stride", c_i64),
        ("older_num_pages", c_i32),
        ("local_block_table", c_ptr),
        ("local_table_stride", c_i64),
        ("local_page_stride", c_i64),
        ("local_num_pages", c_i32),
        ("tile_waves", c_i32),
        ("out_scale", c_ptr),
        ("cu_seqlens_q", c_ptr),
        ("max_seqlen_q", c_i32),
        ("num_splits", c_i32),
        ("cu_seqlens_q_host", c_ptr),
    ]


class AppendArgs(ctypes.Structure):
    """Mirror of ``lkv_append_args``."""

    _fields_ = [
        ("struct_size", c_i32),
        ("batch", c_i32),
        ("tokens", c_i32),
        ("heads", c_i32),
        ("head_dim", c_i32),
        ("token0", c_i32),
        ("wrap_tokens", c_i32),
        ("k", c_ptr),
        ("k_stride_b", c_i64),
        ("k_stride_t", c_i64),
        ("k_stride_h", c_i64),
        ("v", c_ptr),
        ("v_stride_b", c_i64),
        ("v_stride_t", c_i64),
        ("v_stride_h", c_i64),
        ("pool_k", c_ptr),
        ("pool_v", c_ptr),
        ("page_stride", c_i64),
        ("head_stride", c_i64),
        ("num_pages", c_i32),
        ("block_table", c_ptr),
        ("table_stride", c_i64),
        ("table_width", c_i32),
    ]


class MergeArgs(ctypes.Structure):
    """Mirror of ``lkv_merge_args``."""

    _fields_ = [
        ("struct_size", c_i32),
        ("tokens", c_i32),
        ("num_heads", c_i32),
        ("head_dim", c_i32),
        ("prefix_out", c_ptr),
        ("prefix_out_stride_t", c_i64),
        ("prefix_out_stride_h", c_i64),
        ("prefix_lse", c_ptr),
        ("prefix_lse_stride_t", c_i64),
        ("prefix_lse_stride_h", c_i64),
        ("suffix_out", c_ptr),
        ("suffix_out_stride_t", c_i64),
        ("suffix_out_stride_h", c_i64),
        ("suffix_lse", c_ptr),
        ("suffix_lse_stride_t", c_i64),
        ("suffix_lse_stride_h", c_i64),
        ("prefix_scale", c_ptr),
        ("out", c_ptr),
        ("out_stride_t", c_i64),
        ("out_stride_h", c_i64),
        ("out_lse", c_ptr),
        ("out_lse_stride_t", c_i64),
        ("out_lse_stride_h", c_i64),
    ]


class QkvArgs(ctypes.Structure):
    """Mirror of ``lkv_qkv_args``."""

    _fields_ = [
        ("struct_size", c_i32),
        ("batch", c_i32),
        ("tokens", c_i32),
        ("num_q_heads", c_i32),
        ("num_kv_heads", c_i32),
        ("head_dim", c_i32),
        ("eps", c_f32),
        ("position_const", c_i32),
        ("positions", c_ptr),
        ("q", c_ptr),
        ("q_stride_b", c_i64),
        ("q_stride_t", c_i64),
        ("k", c_ptr),
        ("k_stride_b", c_i64),
        ("k_stride_t", c_i64),
        ("v", c_ptr),
        ("v_stride_b", c_i64),
        ("v_stride_t", c_i64),
        ("cos", c_ptr),
        ("sin", c_ptr),
        ("cs_stride_b", c_i64),
        ("cs_stride_t", c_i64),
        ("q_norm_w", c_ptr),
        ("k_norm_w", c_ptr),
        ("q_out", c_ptr),
        ("q_out_stride_b", c_i64),
        ("q_out_stride_t", c_i64),
        ("ring_k", c_ptr),
        ("ring_v", c_ptr),
        ("ring_seq_stride", c_i64),
        ("ring_head_stride", c_i64),
        ("ring_tokens", c_i32),
        ("ring_num_slots", c_i32),
        ("ring_slot", c_ptr),
        ("deep_k", c_ptr),
        ("deep_v", c_ptr),
        ("deep_seq_stride", c_i64),
        ("deep_head_stride", c_i64),
        ("deep_capacity_tokens", c_i32),
        ("deep_num_slots", c_i32),
        ("deep_slot", c_ptr),
        ("ring_block_table", c_ptr),
        ("ring_table_stride", c_i64),
        ("ring_page_stride", c_i64),
        ("ring_num_pages", c_i32),
        ("deep_block_table", c_ptr),
        ("deep_table_stride", c_i64),
        ("deep_page_stride", c_i64),
        ("deep_num_pages", c_i32),
        ("rounding", c_i32),
        ("ring_v_mul", c_ptr),
        ("cu_seqlens", c_ptr),
        ("max_seqlen", c_i32),
    ]


class BlendArgs(ctypes.Structure):
    """Mirror of ``lkv_blend_args``."""

    _fields_ = [
        ("struct_size", c_i32),
        ("layers", c_i32),
        ("batch", c_i32),
        ("kv_heads", c_i32),
        ("chunk_start", c_i32),
        ("chunk_len", c_i32),
        ("ring_k", c_ptr),
        ("ring_v", c_ptr),
        ("ring_layer_stride", c_i64),
        ("ring_seq_stride", c_i64),
        ("ring_head_stride", c_i64),
        ("ring_tokens", c_i32),
        ("deep_k", c_ptr),
        ("deep_v", c_ptr),
        ("deep_seq_stride", c_i64),
        ("deep_head_stride", c_i64),
        ("deep_capacity_tokens", c_i32),
        ("alpha", c_ptr),
        ("one_minus_alpha", c_ptr),
        ("vscale", c_ptr),
        ("ring_block_table", c_ptr),
        ("ring_table_layer_stride", c_i64),
        ("ring_table_stride", c_i64),
        ("ring_page_stride", c_i64),
        ("ring_num_pages", c_i32),
        ("deep_block_table", c_ptr),
        ("deep_table_stride", c_i64),
        ("deep_page_stride", c_i64),
        ("deep_num_pages", c_i32),
    ]


# name -> (restype, argtypes)
class NormArgs(ctypes.Structure):
    """Mirror of ``lkv_rmsnorm_args``."""

    _fields_ = [
        ("struct_size", c_i32),
        ("rows", c_i32),
        ("hidden", c_i32),
        ("eps", c_f32),
        ("x", c_ptr),
        ("x_stride", c_i64),
        ("residual", c_ptr),
        ("residual_stride", c_i64),
        ("weight", c_ptr),
        ("out", c_ptr),
        ("out_stride", c_i64),
    ]


SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "lkv_abi_version": (c_i32, []),
    "lkv_last_error": (ctypes.c_char_p, []),
    "lkv_cache_pack": (
        c_i32,
        [c_ptr, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_ptr, c_i64, c_i64, c_i32, c_i32, c_ptr],
    ),
    "lkv_cache_unpack": (
        c_i32,
        [c_ptr, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_ptr, c_i64, c_i64, c_i64, c_ptr],
    ),
    "lkv_decode_workspace_bytes": (c_i64, [c_i32, c_i32, c_i32]),
    "lkv_decode_attn": (c_i32, [ctypes.POINTER(DecodeArgs), c_ptr]),
    "lkv_decode_attn_noalloc": (c_i32, [ctypes.POINTER(DecodeArgs), c_ptr]),
    "lkv_prefill_workspace_bytes": (c_i64, [ctypes.POINTER(PrefillArgs)]),
    "lkv_prefill_workspace_min_bytes": (c_i64, [ctypes.POINTER(PrefillArgs)]),
    "lkv_prefill_attn": (c_i32, [ctypes.POINTER(PrefillArgs), c_ptr]),
    "lkv_merge_states": (c_i32, [ctypes.POINTER(MergeArgs), c_ptr]),
    "lkv_append_paged": (c_i32, [ctypes.POINTER(AppendArgs), c_ptr]),
    "lkv_qkv_epilogue": (c_i32, [ctypes.POINTER(QkvArgs), c_ptr]),
    "lkv_blend_chunk": (c_i32, [ctypes.POINTER(BlendArgs), c_ptr]),
    "lkv_rmsnorm": (c_i32, [ctypes.POINTER(NormArgs), c_ptr]),
    "lkv_silu_mul": (c_i32, [c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_i32, c_i32, c_ptr]),
    "lkv_probe_read": (c_i32, [c_ptr, c_i64, c_ptr, c_i32, c_ptr]),
    "lkv_probe_mfma": (c_i32, [c_ptr, c_i32, c_i32, ctypes.c_uint32, c_ptr]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load and type the native library (once per process)."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise LastKVNativeError(
                f"{LIB_PATH.name} is not built; run `python -m lastkv_amd.build` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.lkv_abi_version()
        if version != ABI_VERSION:
            raise LastKVNativeError(f"{LIB_PATH.name} ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Raise ``LastKVNativeError`` carrying the library's message for a failed call."""

    if status != 0:
        message = load().lkv_last_error().decode(errors="replace")
        raise LastKVNativeError(f"{what} failed (status {status}): {message}")
