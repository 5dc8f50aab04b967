"""Block methods of the execution backend, host side.

Mirrors ExecutionBackend::{block_bytes, export_block, import_block,
copy_blocks} (crates/vapi-engine/src/backend.rs:339-367) as CandleBackend
implements them (crates/vapi-backend-candle/src/backend.rs:695-797), plus
the batched forms the spill tier and fork path want: export/import of many
blocks in one launch and swap through pinned host memory.
"""
from __future__ import annotations

import numpy as np
import torch

from ._lib import check, lib
from .cache import PagedKvCache, stream_handle


def _dev_u32(values, device) -> torch.Tensor:
    a = np.ascontiguousarray(np.asarray(values, dtype=np.int64).astype(np.uint32))
    return torch.from_numpy(a.view(np.int32)).to(device)


class KvBlockBackend:
    """The block-moving half of a backend over one PagedKvCache."""

    def __init__(self, cache: PagedKvCache):
        self.cache = cache

    def num_blocks(self) -> int:
        return self.cache.num_blocks

    def block_bytes(self) -> int:
        """Bytes of one block across every layer, K and V (backend.rs:695-708)."""
        return lib().vapi_kv_block_bytes(self.cache.pool)

    def _check_ids(self, ids):
        for i in ids:
            if not 0 <= int(i) < self.cache.num_blocks:
                raise ValueError(f"block {int(i)} of {self.cache.num_blocks}")

    def export_blocks(self, ids, out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
        """Blobs of `ids` back to back, in the reference's byte order
        (backend.rs:718-734), into `out` (device or pinned host uint8)."""
        self._check_ids(ids)
        bb = self.block_bytes()
        if out is None:
            out = torch.empty(len(ids) * bb, dtype=torch.uint8, device=self.cache.device)
        if out.numel() < len(ids) * bb:
            raise ValueError(f"export buffer is {out.numel()} bytes, need {len(ids) * bb}")
        if len(ids):
            d_ids = _dev_u32(ids, self.cache.device)
            check(lib().vapi_kv_export_blocks(self.cache.pool, d_ids.data_ptr(), len(ids),
                                              out.data_ptr(), stream_handle(stream)))
        return out

    def import_blocks(self, ids, blobs: torch.Tensor, stream=None) -> None:
        """Inverse of export_blocks (backend.rs:738-773)."""
        self._check_ids(ids)
        bb = self.block_bytes()
        if blobs.numel() != len(ids) * bb:
            raise ValueError(f"spilled blocks are {blobs.numel()} bytes, this cache "
                             f"wants {len(ids) * bb}")
        if len(ids):
            d_ids = _dev_u32(ids, self.cache.device)
            check(lib().vapi_kv_import_blocks(self.cache.pool, d_ids.data_ptr(), len(ids),
                                              blobs.data_ptr(), stream_handle(stream)))

    def export_block(self, block_id: int) -> bytes:
        """ExecutionBackend::export_block: one block's bytes on the host."""
        blob = self.export_blocks([block_id])
        return blob.cpu().numpy().tobytes()

    def import_block(self, block_id: int, data: bytes) -> None:
        """ExecutionBackend::import_block: length must equal block_bytes."""
        bb = self.block_bytes()
        if len(data) != bb:
            raise ValueError(f"spilled block is {len(data)} bytes, this cache wants {bb}")
        blob = torch.frombuffer(bytearray(data), dtype=torch.uint8).to(self.cache.device)
        self.import_blocks([block_id], blob)
        torch.cuda.current_stream().synchronize()

    def copy_blocks(self, pairs, stream=None) -> None:
        """Copy-on-write (backend.rs:781-797): every pair, every layer, K and V,
        in one launch. A destination must not be another pair's source."""
        pairs = [(int(s), int(d)) for s, d in pairs]
        if not pairs:
            return
        self._check_ids([x for p in pairs for x in p])
        srcs = {s for s, _ in pairs}
        dsts = [d for _, d in pairs]
        if len(set(dsts)) != len(dsts) or srcs.intersection(dsts):
            raise ValueError("copy_blocks: destinations must be distinct and not sources")
        d_pairs = _dev_u32([x for p in pairs for x in p], self.cache.device)
        check(lib().vapi_kv_copy_blocks(self.cache.pool, d_pairs.data_ptr(), len(pairs),
                                        stream_handle(stream)))

    def swap_out(self, ids_dev: torch.Tensor, host: torch.Tensor, staging: torch.Tensor,
                 stream=None) -> None:
        """Pack blocks through device staging and DMA them to pinned `host`."""
        check(lib().vapi_kv_swap_out(self.cache.pool, ids_dev.data_ptr(), ids_dev.numel(),
                                     host.data_ptr(), staging.data_ptr(), staging.numel(),
                                     stream_handle(stream)))

    def swap_in(self, ids_dev: torch.Tensor, host: torch.Tensor, staging: torch.Tensor,
                stream=None) -> None:
        """DMA pinned `host` blobs to staging and unpack them into `ids_dev`."""
        check(lib().vapi_kv_swap_in(self.cache.pool, ids_dev.data_ptr(), ids_dev.numel(),
                                    host.data_ptr(), staging.data_ptr(), staging.numel(),
                                    stream_handle(stream)))


def fork_copy_pairs(parent_blocks, computed: int, block_size: int, extra: int,
                    allocate) -> tuple[list[list[int]], list[tuple[int, int]]]:
    """The copy pairs Scheduler::fork emits (crates/vapi-engine/src/scheduler.rs:217-281).

    Blocks the prompt fills completely are shared; the open block after them
    gets a private copy per child, and a (parent_open, private) copy pair is
    emitted only when the open block holds content (computed % block_size
    != 0). `allocate()` returns a fresh block id. Returns (child tables, pairs).
    """
    full = computed // block_size
    has_content = computed % block_size != 0
    children, pairs = [], []
    for _ in range(extra):
        child = list(parent_blocks[:min(full, len(parent_blocks))])
        if len(parent_blocks) > full:
            private = allocate()
            if has_content:
                pairs.append((parent_blocks[full], private))
            child.append(private)
        children.append(child)
    return children, pairs
