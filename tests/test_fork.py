"""The copy pairs Scheduler::fork hands to copy_blocks (a13), on the host.

Mirrors the reference's fork tests (crates/vapi-engine/tests/scheduler.rs:
524-637) at the level this path sees: which blocks the children share,
which they get privately, and which (src, dst) pairs the backend must copy.
"""
import itertools

from vapi_amd.backend import fork_copy_pairs

BS = 4


def allocator(start=100):
    it = itertools.count(start)
    return lambda: next(it)


def test_a_partial_prompt_block_is_copied_once_per_child():
    """scheduler.rs:524-594: 10 tokens over 4-token blocks, n = 3 (2 forks):
    two full blocks shared, the partial third copied per fork."""
    parent = [5, 9, 2]
    children, pairs = fork_copy_pairs(parent, computed=10, block_size=BS, extra=2,
                                      allocate=allocator())
    assert len(children) == 2 and len(pairs) == 2
    assert all(src == parent[2] for src, _ in pairs), "the partial block is the one copied"
    for child, (src, dst) in zip(children, pairs):
        assert child[:2] == parent[:2], "full blocks are shared"
        assert child[2] != parent[2] and child[2] == dst, "the partial one is private"
    assert len({dst for _, dst in pairs}) == 2, "one private block per fork"


def test_a_block_aligned_prompt_copies_nothing_but_still_takes_a_private_open_block():
    """scheduler.rs:596-637: 8 tokens = two full blocks; the open third block
    holds nothing to copy, yet each child gets its own."""
    parent = [3, 4, 11]
    children, pairs = fork_copy_pairs(parent, computed=8, block_size=BS, extra=1,
                                      allocate=allocator())
    assert pairs == [], "nothing partial to copy"
    assert children[0][:2] == parent[:2]
    assert children[0][2] != parent[2], "the open block is private"


def test_a_parent_without_an_open_block_shares_everything():
    """scheduler.rs:246-259: no block past the full ones, nothing to allocate."""
    parent = [7, 8]
    calls = []
    children, pairs = fork_copy_pairs(parent, computed=8, block_size=BS, extra=3,
                                      allocate=lambda: calls.append(1) or 99)
    assert pairs == [] and calls == []
    assert children == [parent, parent, parent]


def test_pairs_never_overlap_so_one_copy_launch_covers_a_fork():
    """copy_blocks takes all pairs in one launch; that needs no destination to
    be a source (backend.rs:781-797 copies them one by one)."""
    for computed in range(1, 40):
        nblk = -(-computed // BS) + (computed % BS == 0)
        parent = list(range(nblk))
        _, pairs = fork_copy_pairs(parent, computed=computed, block_size=BS, extra=4,
                                   allocate=allocator(1000))
        srcs = {s for s, _ in pairs}
        dsts = [d for _, d in pairs]
        assert not srcs & set(dsts) and len(dsts) == len(set(dsts))
        assert len(pairs) == (4 if computed % BS else 0)
