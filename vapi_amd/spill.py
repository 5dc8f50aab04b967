"""Spill tier on libvapi_kv.so: SpillStore (crates/vapi-cache/src/spill.rs)
and the engine's batched spill_evicted / promote_from_spill
(crates/vapi-worker/src/engine.rs:369-456) over a PagedKvCache.

The store is native (spill.cpp); this module is its Python handle. Hashes
are 32-byte keys (the prefix cache's block hashes); blobs are in the export
byte order, so "<hex>.kv" files are interchangeable with the reference's.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import check, lib
from .cache import PagedKvCache, stream_handle

PIN_HEAD = 4096  # the pinned buffer's first 4 KiB stage block ids


def _hash_bytes(h: bytes) -> ctypes.Array:
    if len(h) != 32:
        raise ValueError(f"a block hash is 32 bytes, not {len(h)}")
    return (ctypes.c_uint8 * 32).from_buffer_copy(h)


class SpillStore:
    """Host-memory tier with an optional disk tier behind it, both LRU
    (SpillStore::open, spill.rs:59-94)."""

    def __init__(self, directory: str | None, ram_max: int, disk_max: int):
        h = ctypes.c_void_p()
        check(lib().vapi_spill_open(None if directory is None else str(directory).encode(),
                                    ram_max, disk_max, ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            lib().vapi_spill_close(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def contains(self, h: bytes) -> bool:
        return bool(lib().vapi_spill_contains(self._h, _hash_bytes(h)))

    def put(self, h: bytes, data: bytes) -> None:
        buf = (ctypes.c_uint8 * max(len(data), 1)).from_buffer_copy(data or b"\0")
        check(lib().vapi_spill_put(self._h, _hash_bytes(h), buf, len(data)))

    def get(self, h: bytes, max_len: int = 1 << 26) -> bytes | None:
        """The blob, or None if the store does not hold it (a miss)."""
        out = (ctypes.c_uint8 * max_len)()
        n = lib().vapi_spill_get(self._h, _hash_bytes(h), out, max_len)
        if n == -1:
            return None
        check(n)
        return bytes(out[:n])

    def stats(self) -> dict:
        st = _lib.SpillStats()
        lib().vapi_spill_get_stats(self._h, ctypes.byref(st))
        return {n: getattr(st, n) for n, _ in st._fields_}

    @property
    def handle(self):
        return self._h


def pinned_buffer(cache: PagedKvCache, blocks: int) -> torch.Tensor:
    """Pinned host memory for `blocks` blobs per round, plus the id stage."""
    return torch.empty(PIN_HEAD + blocks * cache.block_bytes(), dtype=torch.uint8,
                       pin_memory=True)


def spill_evicted(store: SpillStore, cache: PagedKvCache, evicted, pinned: torch.Tensor,
                  stream=None) -> int:
    """Export the evicted (hash, block id) pairs the store does not hold yet
    and put their blobs in it (engine.rs:369-393), in batches. Returns the
    number exported; the blocks may be reused once it returns."""
    evicted = list(evicted)
    ids = np.array([i for _, i in evicted], dtype=np.uint32)
    hashes = b"".join(h for h, _ in evicted)
    if any(len(h) != 32 for h, _ in evicted):
        raise ValueError("block hashes are 32 bytes")
    hb = (ctypes.c_uint8 * max(len(hashes), 1)).from_buffer_copy(hashes or b"\0")
    return check(lib().vapi_spill_evicted(
        store.handle, cache.pool, ids.ctypes.data_as(_lib._u32p), hb, len(ids),
        pinned.data_ptr(), pinned.numel(), stream_handle(stream)))


def spill_evicted_async(store: SpillStore, cache: PagedKvCache, evicted, staging: torch.Tensor,
                        pinned: torch.Tensor, stream=None, side=None) -> int:
    """spill_evicted overlapped with the forward: the blocks are packed into
    device `staging` on `stream` and copied to `pinned` on `side`; they
    enter the store at a drain (drain(), or any later store call once their
    copy has completed). Returns how many. Up to 16 exports are in flight,
    each owning its buffers until drained: rotate a ring of them (a call
    reusing an in-flight export's buffers waits for it)."""
    evicted = list(evicted)
    if any(len(h) != 32 for h, _ in evicted):
        raise ValueError("block hashes are 32 bytes")
    if not staging.is_cuda:
        raise ValueError("staging is device memory")
    ids = np.array([i for _, i in evicted], dtype=np.uint32)
    hashes = b"".join(h for h, _ in evicted)
    hb = (ctypes.c_uint8 * max(len(hashes), 1)).from_buffer_copy(hashes or b"\0")
    return check(lib().vapi_spill_evicted_async(
        store.handle, cache.pool, ids.ctypes.data_as(_lib._u32p), hb, len(ids),
        staging.data_ptr(), staging.numel() * staging.element_size(), pinned.data_ptr(),
        pinned.numel(), stream_handle(stream), stream_handle(side)))


def drain(store: SpillStore, wait: bool = True) -> int:
    """Put the in-flight asynchronous export into the store; returns how
    many blobs (0 if none, or if not `wait` and its copy is still running)."""
    return check(lib().vapi_spill_drain(store.handle, int(wait)))


def promote(store: SpillStore, cache: PagedKvCache, hashes, ids, pinned: torch.Tensor,
            stream=None) -> int:
    """Import the held prefix of a block chain into `ids` (the device half
    of promote_from_spill, engine.rs:400-456). Returns how many."""
    hashes = list(hashes)
    ids = np.asarray(ids, dtype=np.uint32)
    if len(ids) != len(hashes) or any(len(h) != 32 for h in hashes):
        raise ValueError("one 32-byte hash per block id")
    hb = b"".join(hashes)
    buf = (ctypes.c_uint8 * max(len(hb), 1)).from_buffer_copy(hb or b"\0")
    return check(lib().vapi_spill_promote(
        store.handle, cache.pool, buf, ids.ctypes.data_as(_lib._u32p), len(ids),
        pinned.data_ptr(), pinned.numel(), stream_handle(stream)))
