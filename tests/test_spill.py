"""The native spill store (spill.cpp) against SpillStore's own tests
(crates/vapi-cache/src/spill.rs:218-296) and the behaviour its code fixes:
LRU order, the host-memory and disk caps, drops, misses, re-indexing a
directory, forgetting unreadable disk entries. Host-only: no GPU work."""
import hashlib

import pytest

from vapi_amd import _lib
from vapi_amd.spill import SpillStore


def hashes(n):
    # Any distinct 32-byte keys (the reference draws them from
    # hash_block_chain, spill.rs:219-223).
    return [hashlib.sha256(b"block %d" % i).digest() for i in range(n)]


def test_host_memory_only_keeps_the_most_recently_used():
    """spill.rs:225-241."""
    h = hashes(4)
    s = SpillStore(None, 20, 0)
    s.put(h[0], bytes(10))
    s.put(h[1], bytes([1]) * 10)
    assert s.get(h[0])[0] == 0
    s.put(h[2], bytes([2]) * 10)  # h[0] is now the most recent: h[1] goes
    assert s.get(h[0]) is not None
    assert s.get(h[1]) is None
    assert s.get(h[2]) is not None
    st = s.stats()
    assert st["ram_blocks"] == 2
    assert st["drops"] == 1, "no disk tier, so the evicted block is dropped"


def test_blocks_pushed_out_of_memory_are_readable_from_disk_and_survive_reopening(tmp_path):
    """spill.rs:243-265."""
    d = tmp_path / "spill"
    h = hashes(4)
    s = SpillStore(d, 10, 1 << 20)
    s.put(h[0], bytes([7]) * 10)
    s.put(h[1], bytes([8]) * 10)
    assert s.stats()["ram_blocks"] == 1  # h[0] was pushed to disk
    assert s.stats()["disk_blocks"] == 1
    assert s.get(h[0]) == bytes([7]) * 10
    assert (d / (h[0].hex() + ".kv")).read_bytes() == bytes([7]) * 10
    s.close()
    s = SpillStore(d, 10, 1 << 20)  # a fresh store indexes what is on disk
    assert s.contains(h[0])
    assert s.get(h[0]) == bytes([7]) * 10
    assert s.get(h[3]) is None
    assert s.stats()["misses"] == 1


def test_the_disk_cap_is_enforced(tmp_path):
    """spill.rs:267-283."""
    h = hashes(4)
    s = SpillStore(tmp_path, 0, 25)
    for i in range(3):
        s.put(h[i], bytes([i]) * 10)
    st = s.stats()
    assert st["disk_bytes"] <= 25, st
    assert st["disk_blocks"] == 2
    assert s.get(h[0]) is None, "the oldest was deleted"
    assert s.get(h[2]) is not None
    assert not (tmp_path / (h[0].hex() + ".kv")).exists()


def test_put_ignores_held_hashes_and_drops_what_fits_nowhere(tmp_path):
    """spill.rs:130-146: a held hash is not written again; a blob larger
    than both caps is dropped, not an error."""
    h = hashes(3)
    s = SpillStore(tmp_path, 16, 32)
    s.put(h[0], b"a" * 8)
    s.put(h[0], b"b" * 8)
    assert s.get(h[0]) == b"a" * 8
    assert s.stats()["writes"] == 1
    s.put(h[1], b"c" * 33)
    assert not s.contains(h[1])
    st = s.stats()
    assert (st["drops"], st["writes"]) == (1, 1)
    # Larger than host memory but within the disk cap: host memory evicts
    # from its oldest entry until under the cap, which takes h[0] and then
    # h[2] itself to disk (spill.rs:179-201).
    s.put(h[2], b"d" * 20)
    st = s.stats()
    assert (st["ram_blocks"], st["disk_blocks"], st["disk_bytes"]) == (0, 2, 28)
    assert s.get(h[2]) == b"d" * 20
    assert s.get(h[0]) == b"a" * 8


def test_a_disk_hit_is_not_promoted_and_lru_order_follows_gets(tmp_path):
    """spill.rs:148-171: a disk hit stays on disk; disk eviction takes the
    least recently used, where a get counts as a use."""
    h = hashes(4)
    s = SpillStore(tmp_path, 0, 30)
    for i in range(3):
        s.put(h[i], bytes([i]) * 10)
    assert s.get(h[0]) is not None  # h[1] is now the oldest
    st = s.stats()
    assert (st["ram_blocks"], st["disk_blocks"]) == (0, 3)
    s.put(h[3], bytes([3]) * 10)
    assert not s.contains(h[1])
    assert all(s.contains(x) for x in (h[0], h[2], h[3]))


def test_an_entry_deleted_under_the_store_is_forgotten_as_an_error(tmp_path):
    """spill.rs:160-166."""
    h = hashes(1)
    s = SpillStore(tmp_path, 0, 100)
    s.put(h[0], b"x" * 10)
    (tmp_path / (h[0].hex() + ".kv")).unlink()
    assert s.get(h[0]) is None
    st = s.stats()
    assert (st["errors"], st["misses"], st["disk_blocks"], st["disk_bytes"]) == (1, 1, 0, 0)
    assert not s.contains(h[0])


def test_reopening_ignores_stray_files_and_applies_the_cap(tmp_path):
    """spill.rs:75-92: only "<64 hex>.kv" files are indexed, then the cap."""
    h = hashes(3)
    for i, x in enumerate(h):
        (tmp_path / (x.hex() + ".kv")).write_bytes(bytes([i]) * 10)
    (tmp_path / "notes.txt").write_bytes(b"hello")
    (tmp_path / ("ab" * 31 + ".kv")).write_bytes(b"short name")
    s = SpillStore(tmp_path, 0, 20)
    st = s.stats()
    assert (st["disk_blocks"], st["disk_bytes"]) == (2, 20)
    assert (tmp_path / "notes.txt").exists()


def test_a_too_small_buffer_is_an_error_and_counts_nothing():
    h = hashes(1)
    s = SpillStore(None, 100, 0)
    s.put(h[0], b"y" * 50)
    with pytest.raises(_lib.VapiKvError):
        s.get(h[0], max_len=10)
    st = s.stats()
    assert (st["hits"], st["misses"]) == (0, 0)
    assert s.get(h[0]) == b"y" * 50


def test_drain_without_an_export_in_flight_does_nothing_and_null_args_are_errors():
    """vapi_spill_drain / vapi_spill_evicted_async host checks (no GPU call:
    nothing is in flight, and a null store or pool fails before any)."""
    L = _lib.lib()
    s = SpillStore(None, 100, 0)
    assert L.vapi_spill_drain(s.handle, 1) == 0
    assert L.vapi_spill_drain(s.handle, 0) == 0
    assert L.vapi_spill_drain(None, 1) == _lib.EINVAL
    assert L.vapi_spill_evicted_async(None, None, None, None, 0, None, 0, None, 0, None,
                                      None) == _lib.EINVAL
    s.put(hashes(1)[0], b"z" * 5)
    assert s.get(hashes(1)[0]) == b"z" * 5
