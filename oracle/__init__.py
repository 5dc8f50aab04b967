"""CPU oracle for the paged KV hot path — TEST INFRASTRUCTURE ONLY.

numpy wrappers over oracle/liboracle.so (a C restatement of vapi's candle CPU
path, see oracle.c for the per-function reference citations). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker or the timed CPU baseline; the product path
(vapi_amd/) never calls it.

Pools here are the reference layout: per layer [num_blocks, block_size,
num_kv_heads, head_dim] (cache.rs:7-11).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None

SKIP = 0xFFFFFFFF

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)


def lib():
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle.so"
        if not path.exists():
            from . import build as _b  # noqa: PLC0415
            _b.build()
        L = ctypes.CDLL(str(path))
        L.oracle_write_rows.argtypes = [_u8p, ctypes.c_uint64, ctypes.c_uint64, _u8p,
                                        _u32p, ctypes.c_uint32, ctypes.c_int, _u32p, ctypes.c_int]
        L.oracle_write_rows.restype = ctypes.c_int
        L.oracle_gather_kv.argtypes = [_u8p, ctypes.c_uint64, ctypes.c_uint32, _u32p,
                                       ctypes.c_uint32, ctypes.c_uint32, _u8p]
        L.oracle_gather_kv.restype = ctypes.c_int
        L.oracle_pack_block_tables.argtypes = [ctypes.c_uint32, _u32p, _u32p, _u32p]
        L.oracle_pack_block_tables.restype = ctypes.c_uint32
        L.oracle_paged_attention.argtypes = [
            _f32p, _f32p, _f32p, _u32p, _u32p, ctypes.c_uint32, _u32p, _u32p,
            ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
            ctypes.c_float, ctypes.c_int32, ctypes.c_int32, _f32p, ctypes.c_int]
        L.oracle_paged_attention.restype = None
        L.oracle_dense_attention_f64.argtypes = [
            _f64p, _f64p, _f64p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
            ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double, ctypes.c_int32,
            ctypes.c_int32, _f64p]
        L.oracle_dense_attention_f64.restype = None
        _u64p = ctypes.POINTER(ctypes.c_uint64)
        L.oracle_block_bytes.argtypes = [_u64p, ctypes.c_uint32]
        L.oracle_block_bytes.restype = ctypes.c_uint64
        pp = ctypes.POINTER(_u8p)
        L.oracle_export_block.argtypes = [pp, _u64p, ctypes.c_uint32, ctypes.c_uint32, _u8p]
        L.oracle_export_block.restype = None
        L.oracle_import_block.argtypes = [pp, _u64p, ctypes.c_uint32, ctypes.c_uint32, _u8p,
                                          ctypes.c_uint64]
        L.oracle_import_block.restype = ctypes.c_int
        L.oracle_copy_blocks.argtypes = [pp, _u64p, ctypes.c_uint32, _u32p, ctypes.c_uint32,
                                         ctypes.c_int]
        L.oracle_copy_blocks.restype = None
        _LIB = L
    return _LIB


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(t)


def write_rows(pool: np.ndarray, src: np.ndarray, slots, force_scatter=False, threads=1):
    """write_rows (cache.rs:217-273) in place on `pool` [nb, bs, kvh, d] (or
    any array whose leading dims flatten to slots). Returns the run count;
    raises ValueError on the reference's error cases. threads > 1 (CPU
    baseline timing) is only for slot lists without repeats."""
    slots = np.ascontiguousarray(slots, dtype=np.uint32)
    n = src.shape[0]
    if n != slots.shape[0]:
        raise ValueError(f"{n} tokens but {slots.shape[0]} cache slots")
    if src.dtype != pool.dtype:
        raise ValueError(f"cache is {pool.dtype} but the rows are {src.dtype}")
    row_bytes = src[0].nbytes if n else 0
    num_slots = pool.nbytes // row_bytes if row_bytes else 0
    src = np.ascontiguousarray(src)
    runs = ctypes.c_uint32(0)
    rc = lib().oracle_write_rows(
        _p(pool.view(np.uint8).reshape(-1), _u8p), num_slots, row_bytes,
        _p(src.view(np.uint8).reshape(-1), _u8p), _p(slots, _u32p), n,
        int(force_scatter), ctypes.byref(runs), int(threads))
    if rc != 0:
        raise ValueError("slot is past the end of the cache")
    return runs.value


def gather_kv(pool: np.ndarray, table, len_k: int) -> np.ndarray:
    """gather_kv (cache.rs:283-290): pool [nb, bs, kvh, d] -> [len_k, kvh, d]."""
    nb, bs, kvh, d = pool.shape
    table = np.ascontiguousarray(table, dtype=np.uint32)
    out = np.zeros((len_k, kvh, d), dtype=pool.dtype)
    rc = lib().oracle_gather_kv(
        _p(pool.view(np.uint8).reshape(-1), _u8p), pool[0].nbytes, bs,
        _p(table, _u32p), table.shape[0], len_k, _p(out.view(np.uint8).reshape(-1), _u8p))
    if rc != 0:
        raise ValueError("len_k exceeds the block table")
    return out


def ragged(tables):
    offs = np.zeros(len(tables) + 1, dtype=np.uint32)
    for i, t in enumerate(tables):
        offs[i + 1] = offs[i] + len(t)
    data = (np.concatenate([np.asarray(t, dtype=np.uint32) for t in tables])
            if tables and offs[-1] > 0 else np.zeros(1, dtype=np.uint32))
    return offs, np.ascontiguousarray(data, dtype=np.uint32)


def pack_block_tables(tables) -> np.ndarray:
    """pack_block_tables (attention.rs:42-62)."""
    offs, data = ragged(tables)
    width = max([len(t) for t in tables] + [1])
    out = np.zeros((len(tables), width), dtype=np.uint32)
    w = lib().oracle_pack_block_tables(len(tables), _p(offs, _u32p), _p(data, _u32p),
                                       _p(out, _u32p))
    assert w == width
    return out


def paged_attention(q, k_cache, v_cache, cu_q, cu_k, tables, scale,
                    sliding_window=None, window_right=0, threads=1):
    """paged_attention_cpu (attention.rs:90-163) in f32.

    q [total_q, heads, d]; k_cache/v_cache [nb, bs, kvh, d]; any float dtype
    is upcast to f32 exactly first. Returns f32 [total_q, heads, d]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(k_cache, dtype=np.float32)
    vc = np.ascontiguousarray(v_cache, dtype=np.float32)
    _, bs, kvh, d = kc.shape
    heads = q.shape[1]
    cu_q = np.ascontiguousarray(cu_q, dtype=np.uint32)
    cu_k = np.ascontiguousarray(cu_k, dtype=np.uint32)
    offs, data = ragged(tables)
    out = np.zeros_like(q)
    win = -1 if sliding_window is None else int(sliding_window)
    lib().oracle_paged_attention(
        _p(q, _f32p), _p(kc, _f32p), _p(vc, _f32p), _p(cu_q, _u32p), _p(cu_k, _u32p),
        len(tables), _p(offs, _u32p), _p(data, _u32p), bs, heads, kvh, d, scale,
        win, int(window_right), _p(out, _f32p), int(threads))
    return out


def dense_attention_f64(q, k, v, scale, sliding_window=None, window_right=0):
    """Dense attention over one sequence in f64 (attention.rs:297-321
    dense_causal, with GQA and window). q [len_q, heads, d]; k, v
    [len_k, kvh, d] in logical order."""
    q = np.ascontiguousarray(q, dtype=np.float64)
    k = np.ascontiguousarray(k, dtype=np.float64)
    v = np.ascontiguousarray(v, dtype=np.float64)
    len_q, heads, d = q.shape
    len_k, kvh, _ = k.shape
    out = np.zeros_like(q)
    win = -1 if sliding_window is None else int(sliding_window)
    lib().oracle_dense_attention_f64(_p(q, _f64p), _p(k, _f64p), _p(v, _f64p), len_q,
                                     len_k, heads, kvh, d, scale, win,
                                     int(window_right), _p(out, _f64p))
    return out


def block_bytes(layers, block_size, kvh, d, elt):
    """block_bytes (backend.rs:695-708) of a uniform cache."""
    per = np.full(2 * layers, block_size * kvh * d * elt, dtype=np.uint64)
    return lib().oracle_block_bytes(_p(per, _u64p), per.size)


def _buffers(k_layers, v_layers):
    """The reference's buffer order k[0..L] ++ v[0..L] as (pointers, per-block
    bytes, count); a V layer that is None or empty (a rows layer) is
    skipped, as the reference skips buffers of rank < 2."""
    bufs = list(k_layers) + list(v_layers)
    real = [b is not None and b.ndim >= 2 and b.size > 0 for b in bufs]
    ptrs = (_u8p * len(bufs))(*[_p(b.view(np.uint8).reshape(-1), _u8p) if r else None
                                for b, r in zip(bufs, real)])
    per = np.array([b[0].nbytes if r else 0 for b, r in zip(bufs, real)], dtype=np.uint64)
    return ptrs, per, len(bufs)


def cache_block_bytes(k_layers, v_layers) -> int:
    """block_bytes (backend.rs:695-708) of per-layer pools of any shapes."""
    _, per, n = _buffers(k_layers, v_layers)
    return lib().oracle_block_bytes(_p(per, _u64p), n)


def export_block(k_layers, v_layers, block_id) -> bytes:
    """export_block (backend.rs:718-734). k_layers/v_layers: per-layer pools
    (None or an empty array for a rows layer's V)."""
    ptrs, per, n = _buffers(k_layers, v_layers)
    out = np.zeros(max(int(per.sum()), 1), dtype=np.uint8)
    lib().oracle_export_block(ptrs, _p(per, _u64p), n, block_id, _p(out, _u8p))
    return out[:int(per.sum())].tobytes()


def import_block(k_layers, v_layers, block_id, data: bytes) -> None:
    """import_block (backend.rs:738-773), in place."""
    ptrs, per, n = _buffers(k_layers, v_layers)
    buf = np.frombuffer(data, dtype=np.uint8).copy()
    rc = lib().oracle_import_block(ptrs, _p(per, _u64p), n, block_id, _p(buf, _u8p), buf.size)
    if rc != 0:
        raise ValueError(f"spilled block is {buf.size} bytes, this cache wants "
                         f"{int(per.sum())}")


def copy_blocks(k_layers, v_layers, pairs, threads=1) -> None:
    """copy_blocks (backend.rs:781-797), in place. threads > 1 (CPU baseline
    timing) is only for pairs whose destinations are distinct and no pair's
    source."""
    pairs = np.ascontiguousarray(np.asarray(pairs, dtype=np.uint32).reshape(-1, 2))
    ptrs, per, n = _buffers(k_layers, v_layers)
    lib().oracle_copy_blocks(ptrs, _p(per, _u64p), n, _p(pairs, _u32p), pairs.shape[0],
                             int(threads))
