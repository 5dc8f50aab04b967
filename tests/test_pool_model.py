"""CPU tests of the test-side block bookkeeping (tests/pool_model.py) on the
reference's own pool tests (crates/vapi-cache/tests/pool.rs:20-260 and
src/pool.rs:427-459), and of the spill flow it drives with the MockBackend
stand-in and the native spill store (spill.cpp), as the reference's engine
tests do (crates/vapi-worker/src/engine.rs:1198-1294)."""
import random

import pytest

from pool_model import BlockPool, Exhausted, MockKvBackend, SpillEngine, hash_chain
from vapi_amd.spill import SpillStore

BS = 4


def test_allocation_refcounts_and_exhaustion():
    p = BlockPool(4, BS)
    a, b = p.allocate(), p.allocate()
    assert (a, b) == (0, 1) and p.num_free() == 2  # ascending from a fresh pool
    p.incref(a)
    p.free(a)
    assert p.num_free() == 2
    p.free(a), p.free(b)
    assert p.num_free() == 4
    q = BlockPool(2, BS)
    q.allocate(), q.allocate()
    with pytest.raises(Exhausted):
        q.allocate()
    p.check_invariants()


def test_the_watermark_stops_admission_before_the_pool_empties():
    p = BlockPool(4, BS, 2)
    assert p.can_allocate(2) and not p.can_allocate(3)
    p.allocate_guarded(), p.allocate_guarded()
    with pytest.raises(Exhausted):
        p.allocate_guarded()
    p.allocate()


def test_prefix_hits_sharing_and_the_first_miss():
    p = BlockPool(16, BS)
    h = hash_chain(list(range(8)), BS)
    assert p.match_prefix(h) == []
    blocks = [p.publish(p.allocate(), x) for x in h]
    p.free_all(blocks)
    assert p.match_prefix(h) == blocks
    p.free_all(blocks)
    system = list(range(100, 108))
    ha, hb = hash_chain(system + [1, 2, 3, 4], BS), hash_chain(system + [9, 9, 9, 9], BS)
    a = [p.publish(p.allocate(), x) for x in ha]
    p.free_all(a)
    assert p.match_prefix(hb) == a[:2]
    q = BlockPool(16, BS)
    h3 = hash_chain(list(range(12)), BS)
    for x in (h3[0], h3[2]):
        q.publish(q.allocate(), x)
    assert len(q.match_prefix(h3)) == 1
    p.check_invariants(), q.check_invariants()


def test_eviction_order_and_pressure():
    h = hash_chain([1, 2, 3, 4], BS)
    p = BlockPool(2, BS)
    held = p.publish(p.allocate(), h[0])
    p.allocate()
    with pytest.raises(Exhausted):
        p.allocate()
    assert p.lookup(h[0]) == held
    p = BlockPool(2, BS)
    b = p.publish(p.allocate(), h[0])
    p.free(b)
    assert p.lookup(h[0]) is not None
    p.free(b)
    p.allocate(), p.allocate()
    assert p.lookup(h[0]) is None and p.evictions == 1
    p = BlockPool(2, BS)
    cached = p.publish(p.allocate(), h[0])
    empty = p.allocate()
    p.free(cached), p.free(empty)
    assert p.allocate() == empty
    assert p.lookup(h[0]) is not None
    p.check_invariants()


def test_concurrent_publishers_converge():
    h = hash_chain([1, 2, 3, 4], BS)
    p = BlockPool(8, BS)
    first, second = p.allocate(), p.allocate()
    assert p.publish(first, h[0]) == first
    assert p.publish(second, h[0]) == first
    p.free(second)
    assert len(p.by_hash) == 1
    p.check_invariants()


def test_evicted_content_is_reported_once_and_only_when_asked():
    h = hash_chain(list(range(6)), 2)
    p = BlockPool(2, 2)
    a = p.publish(p.allocate(), h[0])
    p.free(a)
    b = p.allocate()
    assert p.take_evicted() == []
    p.free(b)
    p.track_evictions(True)
    c = p.publish(p.allocate(), h[1])
    p.free(c)
    taken = [p.allocate(), p.allocate()]
    ev = p.take_evicted()
    assert (h[1], c) in ev and c in taken
    assert all(not p.contains(x) for x, _ in ev)
    assert p.take_evicted() == []


def test_invariants_hold_under_a_random_trace():
    rng = random.Random(5)
    p = BlockPool(12, BS, 1)
    hs = hash_chain(list(range(80)), BS)
    held = []
    for _ in range(3000):
        op = rng.randrange(4)
        try:
            if op == 0:
                held.append(p.allocate())
            elif op == 1 and held:
                p.free(held.pop(rng.randrange(len(held))))
            elif op == 2 and held:
                i = rng.randrange(len(held))
                c = p.publish(held[i], rng.choice(hs))
                if c != held[i]:
                    p.free(held[i])
                    held[i] = c
            else:
                b = p.lookup(rng.choice(hs))
                if b is not None:
                    held.append(b)
        except Exhausted:
            pass
        p.check_invariants()


def test_evicted_blocks_spill_and_come_back_with_their_bytes():
    """engine.rs:1247-1294 with MockBackend's stamps: a prompt's blocks are
    pushed out by two others, exported to the spill store before they are
    overwritten, and restored bytes-for-bytes when the prompt returns."""
    bs, nb, bb = 16, 4, 64
    mock = MockKvBackend(nb, bb)
    store = SpillStore(None, 1 << 20, 0)

    def forward(table, cached, n):
        mock.forward([table[p // bs] * bs + p % bs for p in range(cached, n)], bs)

    eng = SpillEngine(BlockPool(nb, bs), mock, store, forward)
    a = list(range(1, 2 * bs + 1))
    assert eng.run_prompt(a)[0] == 0
    a_bytes = [mock.export_block(b) for b in eng.pool.match_prefix(hash_chain(a, bs))]
    eng.pool.free_all([eng.pool.by_hash[h] for h in hash_chain(a, bs)])
    assert store.stats()["writes"] == 0
    eng.run_prompt([1000 + i for i in range(2 * bs)])
    eng.run_prompt([2000 + i for i in range(2 * bs)])
    assert store.stats()["writes"] >= 2
    cached, table = eng.run_prompt(a)
    assert store.stats()["hits"] >= 2
    assert cached == bs  # the last block is recomputed
    assert mock.export_block(table[0]) == a_bytes[0]
    with pytest.raises(ValueError):
        mock.import_block(0, bytes(bb - 1))
    store.close()
