"""ctypes binding of libvapi_kv.so, the gfx950 C-ABI library (include/vapi_kv.h).

There is no fallback: if the library is missing, loading raises, and every
operation in this package fails loudly.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libvapi_kv.so"

F32, F16, BF16 = 0, 1, 2
LAYOUT_HND, LAYOUT_NHD = 0, 1
SLOT_SKIP = 0xFFFFFFFF

OK, EINVAL, EUNSUP, EHIP, ESPACE = 0, -1, -2, -3, -4
ATTN_DETERMINISTIC, ATTN_NO_DECODE_ROWS = 0x1, 0x2
ATTN_SCRATCH_BYTES = 16 << 20  # VAPI_ATTN_SCRATCH_BYTES
APPEND_COLD_SOURCE = 0x1  # VAPI_APPEND_COLD_SOURCE

# Every symbol include/vapi_kv.h declares.
EXPORTS = (
    "vapi_kv_last_error", "vapi_kv_version", "vapi_kv_block_bytes",
    "vapi_kv_layer_bytes", "vapi_kv_append", "vapi_kv_append_ex", "vapi_kv_gather",
    "vapi_paged_attention_workspace_size", "vapi_paged_attention",
    "vapi_paged_attention_append", "vapi_kv_append_layers",
    "vapi_kv_copy_blocks", "vapi_kv_export_blocks", "vapi_kv_import_blocks",
    "vapi_kv_swap_out", "vapi_kv_swap_in", "vapi_forward_batch_validate",
    "vapi_pack_block_tables", "vapi_cache_new", "vapi_cache_free",
    "vapi_cache_pool", "vapi_cache_num_slots", "vapi_cache_write_kv",
    "vapi_cache_block_bytes", "vapi_cache_export_block",
    "vapi_cache_import_block", "vapi_cache_copy_blocks",
    "vapi_spill_open", "vapi_spill_close", "vapi_spill_contains", "vapi_spill_put",
    "vapi_spill_get", "vapi_spill_get_stats", "vapi_spill_evicted", "vapi_spill_promote",
    "vapi_spill_evicted_async", "vapi_spill_drain",
    "vapi_paged_attention_ex", "vapi_paged_attention_append_ex",
    "vapi_paged_attention_noalloc",
    "vapi_paged_attention_prepared", "vapi_paged_attention_prepared_workspace_size",
)


class VapiKvError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class Pool(ctypes.Structure):
    """vapi_kv_pool."""
    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("layer_stride_bytes", ctypes.c_uint64),
        ("num_layers", ctypes.c_uint32),
        ("num_blocks", ctypes.c_uint32),
        ("block_size", ctypes.c_uint32),
        ("num_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("dtype", ctypes.c_uint32),
        ("layout", ctypes.c_uint32),
        ("next", ctypes.c_void_p),
        ("block_stride_bytes", ctypes.c_uint64),
    ]


_lib = None
_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t
_u32p = ctypes.POINTER(ctypes.c_uint32)
_poolp = ctypes.POINTER(Pool)


class SpillStats(ctypes.Structure):
    """vapi_spill_stats (SpillStats, spill.rs:27-40)."""
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "ram_blocks", "ram_bytes", "disk_blocks", "disk_bytes", "hits", "misses", "writes",
        "drops", "errors")]


def lib():
    """Load libvapi_kv.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m vapi_amd.build` "
            "(there is no CPU fallback)")
    L = ctypes.CDLL(str(LIB_PATH))
    L.vapi_kv_last_error.restype = ctypes.c_char_p
    L.vapi_kv_version.restype = ctypes.c_char_p
    L.vapi_kv_block_bytes.argtypes = [_poolp]
    L.vapi_kv_block_bytes.restype = _sz
    L.vapi_kv_layer_bytes.argtypes = [_poolp]
    L.vapi_kv_layer_bytes.restype = _sz
    L.vapi_kv_append.argtypes = [_poolp, _u32, _vp, _vp, _vp, _u32, _vp]
    L.vapi_kv_append_ex.argtypes = [_poolp, _u32, _vp, _vp, _vp, _u32, _u32, _vp]
    L.vapi_kv_gather.argtypes = [_poolp, _u32, _vp, _u32, _u32, _vp, _vp, _vp]
    L.vapi_paged_attention_workspace_size.argtypes = [_poolp, _u32, _u32, _u32, _u32]
    L.vapi_paged_attention_workspace_size.restype = _sz
    L.vapi_paged_attention.argtypes = [
        _poolp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
        ctypes.c_float, _i32, _i32, _vp, _sz, _vp]
    L.vapi_paged_attention_append.argtypes = [
        _poolp, _u32, _vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
        _u32, ctypes.c_float, _i32, _i32, _vp, _sz, _vp]
    L.vapi_paged_attention_ex.argtypes = [
        _poolp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
        ctypes.c_float, _i32, _i32, _u32, _vp, _sz, _vp]
    L.vapi_paged_attention_append_ex.argtypes = [
        _poolp, _u32, _vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
        _u32, ctypes.c_float, _i32, _i32, _u32, _vp, _sz, _vp]
    L.vapi_paged_attention_prepared_workspace_size.argtypes = [_poolp, _u32, _u32, _u32, _u32,
                                                               _u32]
    L.vapi_paged_attention_prepared_workspace_size.restype = _sz
    L.vapi_paged_attention_prepared.argtypes = [
        _poolp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
        ctypes.c_float, _i32, _i32, _u32, _vp, _u32, _vp, _sz, _vp]
    L.vapi_paged_attention_noalloc.argtypes = [
        _poolp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32,
        ctypes.c_float, _i32, _i32, _u32, _vp]
    L.vapi_kv_append_layers.argtypes = [_poolp, _u32, _u32, _vp, _vp, ctypes.c_uint64, _vp,
                                         _u32, _vp]
    L.vapi_kv_copy_blocks.argtypes = [_poolp, _vp, _u32, _vp]
    L.vapi_kv_export_blocks.argtypes = [_poolp, _vp, _u32, _vp, _vp]
    L.vapi_kv_import_blocks.argtypes = [_poolp, _vp, _u32, _vp, _vp]
    L.vapi_kv_swap_out.argtypes = [_poolp, _vp, _u32, _vp, _vp, _sz, _vp]
    L.vapi_kv_swap_in.argtypes = [_poolp, _vp, _u32, _vp, _vp, _sz, _vp]
    L.vapi_forward_batch_validate.argtypes = [
        _u32, _u32p, _u32p, _u32p, _u32p, _u32, _u32p, _u32p, _u32p, _u32, _u32, _u32]
    L.vapi_pack_block_tables.argtypes = [_u32, _u32p, _u32p, _u32p, _sz]
    L.vapi_pack_block_tables.restype = ctypes.c_int64
    L.vapi_cache_new.argtypes = [_u32] * 7 + [ctypes.POINTER(_vp)]
    L.vapi_cache_free.argtypes = [_vp]
    L.vapi_cache_free.restype = None
    L.vapi_cache_pool.argtypes = [_vp, _poolp]
    L.vapi_cache_num_slots.argtypes = [_vp]
    L.vapi_cache_num_slots.restype = ctypes.c_uint64
    L.vapi_cache_write_kv.argtypes = [_vp, _u32, _vp, _vp, _u32, _u32, _u32p, _u32, _vp]
    L.vapi_cache_block_bytes.argtypes = [_vp]
    L.vapi_cache_block_bytes.restype = _sz
    L.vapi_cache_export_block.argtypes = [_vp, _u32, _vp, _sz]
    L.vapi_cache_import_block.argtypes = [_vp, _u32, _vp, _sz]
    L.vapi_cache_copy_blocks.argtypes = [_vp, _u32p, _u32]
    L.vapi_spill_open.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_uint64,
                                  ctypes.POINTER(_vp)]
    L.vapi_spill_close.argtypes = [_vp]
    L.vapi_spill_close.restype = None
    L.vapi_spill_contains.argtypes = [_vp, _vp]
    L.vapi_spill_put.argtypes = [_vp, _vp, _vp, _sz]
    L.vapi_spill_get.argtypes = [_vp, _vp, _vp, _sz]
    L.vapi_spill_get.restype = ctypes.c_int64
    L.vapi_spill_get_stats.argtypes = [_vp, ctypes.POINTER(SpillStats)]
    L.vapi_spill_get_stats.restype = None
    L.vapi_spill_evicted.argtypes = [_vp, _poolp, _u32p, _vp, _u32, _vp, _sz, _vp]
    L.vapi_spill_evicted.restype = ctypes.c_int64
    L.vapi_spill_promote.argtypes = [_vp, _poolp, _vp, _u32p, _u32, _vp, _sz, _vp]
    L.vapi_spill_promote.restype = ctypes.c_int64
    L.vapi_spill_evicted_async.argtypes = [_vp, _poolp, _u32p, _vp, _u32, _vp, _sz, _vp, _sz,
                                           _vp, _vp]
    L.vapi_spill_evicted_async.restype = ctypes.c_int64
    L.vapi_spill_drain.argtypes = [_vp, ctypes.c_int]
    L.vapi_spill_drain.restype = ctypes.c_int64
    _lib = L
    return L


def check(rc: int) -> int:
    """Raise VapiKvError with the library's message on a negative status."""
    if rc < 0:
        raise VapiKvError(rc, lib().vapi_kv_last_error().decode())
    return rc
