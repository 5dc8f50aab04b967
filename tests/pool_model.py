"""Test infrastructure: the host-side block bookkeeping that decides which
block ids the paged-KV data path shares, copies, evicts and restores.

None of this is product code. The reference's BlockPool
(crates/vapi-cache/src/pool.rs:60-410) and the engine's spill steps
(crates/vapi-worker/src/engine.rs:364-456) are control plane that this
build leaves to the caller; the tests use this restatement to drive the
device calls (copy_blocks, export/import, the spill tier) in the order the
reference's engine would issue them. MockKvBackend restates the reference's
MockBackend movable-block simulation (crates/vapi-engine/src/backend.rs:
452-539): a block's bytes are a stamp of the step that last wrote it.

Block hashes here are SHA-256 chains over token blocks: the reference's
hash_block_chain (crates/vapi-cache/src/hash.rs) is not restated, since the
data path treats a hash as an opaque 32-byte key.
"""
from __future__ import annotations

import hashlib

NONE = None


class Exhausted(Exception):
    pass


def hash_chain(tokens, block_size: int, salt: bytes = b"ns") -> list[bytes]:
    """One 32-byte key per full block, each depending on every block before
    it (a prefix's identity, as a chained hash gives)."""
    out, prev = [], salt
    for i in range(len(tokens) // block_size):
        blk = tokens[i * block_size:(i + 1) * block_size]
        prev = hashlib.sha256(prev + b"".join(int(t).to_bytes(4, "little") for t in blk)).digest()
        out.append(prev)
    return out


class BlockPool:
    """pool.rs:60-410: refcounts, a hash index over filled blocks and an LRU
    free list (uncached blocks at the front, evicted first; cached blocks at
    the back), with eviction tracking for the spill tier."""

    def __init__(self, num_blocks: int, block_size: int, watermark: int = 0):
        self.block_size = block_size
        self.watermark = min(watermark, num_blocks)
        self.refcount = [0] * num_blocks
        self.hash_of = [None] * num_blocks
        self.by_hash: dict[bytes, int] = {}
        # The free list in LRU order (head first); a dict keeps insertion
        # order and O(1) removal.
        self.free_list: dict[int, None] = {i: None for i in range(num_blocks)}
        self.evictions = 0
        self.evicted_content: list[tuple[bytes, int]] = []
        self.track = False

    def num_free(self) -> int:
        return len(self.free_list)

    def can_allocate(self, want: int) -> bool:
        return self.num_free() >= want + self.watermark

    def allocate(self) -> int:
        """pool.rs:170-188: the LRU head; a cached block loses its hash."""
        if not self.free_list:
            raise Exhausted()
        bid = next(iter(self.free_list))
        del self.free_list[bid]
        h = self.hash_of[bid]
        if h is not None:
            self.hash_of[bid] = None
            del self.by_hash[h]
            self.evictions += 1
            if self.track:
                self.evicted_content.append((h, bid))
        self.refcount[bid] = 1
        return bid

    def allocate_guarded(self) -> int:
        if not self.can_allocate(1):
            raise Exhausted("watermark")
        return self.allocate()

    def track_evictions(self, on: bool) -> None:
        self.track = on
        if not on:
            self.evicted_content.clear()

    def take_evicted(self) -> list[tuple[bytes, int]]:
        out, self.evicted_content = self.evicted_content, []
        return out

    def contains(self, h: bytes) -> bool:
        return h in self.by_hash

    def incref(self, bid: int) -> None:
        assert self.refcount[bid] > 0
        self.refcount[bid] += 1

    def free(self, bid: int) -> None:
        """pool.rs:232-248: cached blocks to the back, empty ones to the front."""
        assert self.refcount[bid] > 0, f"double free of {bid}"
        self.refcount[bid] -= 1
        if self.refcount[bid] == 0:
            if self.hash_of[bid] is not None:
                self.free_list[bid] = None
            else:
                self.free_list = {bid: None, **self.free_list}

    def free_all(self, blocks) -> None:
        for b in blocks:
            self.free(b)

    def publish(self, bid: int, h: bytes) -> int:
        """pool.rs:262-284: the first publisher of a hash wins."""
        existing = self.by_hash.get(h)
        if existing is not None and existing != bid:
            self._reference(existing)
            return existing
        stale = self.hash_of[bid]
        self.hash_of[bid] = h
        if stale is not None and stale != h:
            del self.by_hash[stale]
        self.by_hash[h] = bid
        return bid

    def _reference(self, bid: int) -> None:
        if self.refcount[bid] == 0:
            del self.free_list[bid]
        self.refcount[bid] += 1

    def lookup(self, h: bytes):
        bid = self.by_hash.get(h)
        if bid is None:
            return None
        self._reference(bid)
        return bid

    def match_prefix(self, hashes) -> list[int]:
        """pool.rs:303-318: stops at the first miss."""
        blocks = []
        for h in hashes:
            b = self.lookup(h)
            if b is None:
                break
            blocks.append(b)
        return blocks

    def check_invariants(self) -> None:
        """pool.rs:377-413."""
        for i, rc in enumerate(self.refcount):
            assert (rc == 0) == (i in self.free_list), f"block {i}: refcount {rc}"
        for h, b in self.by_hash.items():
            assert self.hash_of[b] == h
        assert sum(h is not None for h in self.hash_of) == len(self.by_hash)


class MockKvBackend:
    """MockBackend's movable blocks (backend.rs:452-539): each block holds
    what the forward last stamped into it, stamp(block)[i] = (block + i +
    step) & 0xFF; export returns it (zeros if never written); import checks
    the length."""

    def __init__(self, num_blocks: int, block_bytes: int):
        self.num_blocks = num_blocks
        self._bb = block_bytes
        self.store: dict[int, bytes] = {}
        self.step = 0

    def block_bytes(self) -> int:
        return self._bb

    def stamp(self, block: int) -> bytes:
        return bytes((block + i + self.step) & 0xFF for i in range(self._bb))

    def forward(self, slot_mapping, block_size: int) -> None:
        for slot in slot_mapping:
            b = slot // block_size
            self.store[b] = self.stamp(b)
        self.step += 1

    def export_block(self, bid: int) -> bytes:
        if self._bb == 0:
            raise RuntimeError("blocks are not movable")
        return self.store.get(bid, bytes(self._bb))

    def import_block(self, bid: int, data: bytes) -> None:
        if self._bb == 0:
            raise RuntimeError("blocks are not movable")
        if len(data) != self._bb:
            raise ValueError(f"block is {self._bb} bytes, got {len(data)}")
        self.store[bid] = bytes(data)


class SpillEngine:
    """The engine's two spill steps over a pool, a backend with export/import
    and a spill store (engine.rs:364-456), restated for the tests:
    run_prompt allocates (and spills what the allocation evicts before the
    forward writes it), prefills the missing blocks, publishes them and
    frees the sequence; promote_from_spill restores the held prefix first."""

    def __init__(self, pool: BlockPool, backend, store, forward):
        self.pool, self.backend, self.store, self.forward = pool, backend, store, forward
        pool.track_evictions(True)

    def spill_evicted(self) -> int:
        n = 0
        for h, bid in self.pool.take_evicted():
            if self.store.contains(h):
                continue
            self.store.put(h, self.backend.export_block(bid))
            n += 1
        return n

    def promote_from_spill(self, hashes) -> int:
        restored = 0
        for h in hashes:
            if self.pool.contains(h):
                continue
            data = self.store.get(h)
            if data is None or self.pool.num_free() <= 1:
                break
            bid = self.pool.allocate()
            self.spill_evicted()
            self.backend.import_block(bid, data)
            canon = self.pool.publish(bid, h)
            if canon != bid:
                self.pool.free(bid)
            self.pool.free(canon)
            restored += 1
        return restored

    def run_prompt(self, tokens) -> tuple[int, list[int]]:
        """Returns (cached prefix tokens, the sequence's block table)."""
        bs = self.pool.block_size
        hashes = hash_chain(tokens, bs)
        self.promote_from_spill(hashes)
        table = self.pool.match_prefix(hashes)
        # A fully cached prompt recomputes its last block (the forward must
        # produce logits from somewhere).
        if len(table) * bs >= len(tokens):
            self.pool.free(table.pop())
        cached = len(table) * bs
        while len(table) * bs < len(tokens):
            table.append(self.pool.allocate())
        self.spill_evicted()  # before the forward overwrites evicted blocks
        self.forward(table, cached, len(tokens))
        for i, h in enumerate(hashes):
            if i >= cached // bs:
                canon = self.pool.publish(table[i], h)
                if canon != table[i]:
                    self.pool.free(table[i])
                    table[i] = canon
        self.pool.free_all(table)
        return cached, table
