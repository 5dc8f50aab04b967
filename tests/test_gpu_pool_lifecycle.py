"""The paged-KV data path driven by the block pool's decisions, on the GPU:
prefix sharing by reference, a fork whose children get copy-on-write copies
of the open block (copy_blocks), eviction under pressure with the evicted
blocks exported to the spill store before they are overwritten, and
promotion of a returning prompt's prefix (import). The bookkeeping is the
test-side restatement in tests/pool_model.py (crates/vapi-cache/src/
pool.rs, crates/vapi-worker/src/engine.rs:364-456); every byte the device
moves is checked bit-exact: against the K/V rows the forward appended, and
a restored prefix's attention output equals the original's exactly.
"""
import numpy as np
import pytest
import torch

from pool_model import BlockPool, SpillEngine, hash_chain
from vapi_amd.attention import ForwardBatch, paged_attention
from vapi_amd.backend import KvBlockBackend, fork_copy_pairs
from vapi_amd.cache import PagedKvCache, gather_kv, write_kv_to_cache
from vapi_amd.spill import SpillStore

pytestmark = pytest.mark.gpu
DEV = "cuda"
BS, L, KVH, D = 16, 2, 2, 128


def rows_for(tokens, layer, which):
    """Deterministic K or V rows of a token sequence (a stand-in for the
    projection of each token at its position)."""
    t = torch.tensor(tokens, dtype=torch.float32, device=DEV)
    pos = torch.arange(len(tokens), dtype=torch.float32, device=DEV)
    i = torch.arange(KVH * D, dtype=torch.float32, device=DEV)
    x = torch.sin(t[:, None] * 0.37 + pos[:, None] * 0.011 + i[None] * 0.05 + layer + 7 * which)
    return x.reshape(len(tokens), KVH, D).to(torch.bfloat16)


class Device:
    """export/import through the GPU cache (ExecutionBackend's block methods)."""

    def __init__(self, cache):
        self.be = KvBlockBackend(cache)

    def export_block(self, bid):
        return self.be.export_block(bid)

    def import_block(self, bid, data):
        self.be.import_block(bid, data)


def kv(cache, l, table, n):
    return (gather_kv(cache, l, table, n, "k"), gather_kv(cache, l, table, n, "v"))


def test_share_fork_evict_spill_and_promote_move_the_right_bytes():
    nb = 6
    cache = PagedKvCache(L, nb, BS, KVH, D, torch.bfloat16, "HND")
    store = SpillStore(None, 1 << 26, 0)
    written = {}

    def forward(table, cached, n, tokens):
        slots = [table[p // BS] * BS + p % BS for p in range(cached, n)]
        for l in range(L):
            k = rows_for(tokens, l, 0)[cached:n]
            v = rows_for(tokens, l, 1)[cached:n]
            write_kv_to_cache(cache, l, k, v, np.array(slots, dtype=np.uint32))

    current = {}
    eng = SpillEngine(BlockPool(nb, BS), Device(cache), store,
                      lambda t, c, n: forward(t, c, n, current["tokens"]))

    def run(tokens):
        current["tokens"] = tokens
        return eng.run_prompt(tokens)

    a = [3 + i for i in range(2 * BS + 5)]  # two full blocks and an open one
    cached, table_a = run(a)
    assert cached == 0
    for l in range(L):
        got = kv(cache, l, table_a, len(a))
        assert torch.equal(got[0], rows_for(a, l, 0)) and torch.equal(got[1], rows_for(a, l, 1))
    # Attention of A's last token over its own context, for comparison after
    # a round trip through the spill tier.
    q = torch.randn(1, 4, D, device=DEV).to(torch.bfloat16)
    batch = ForwardBatch(cu_seqlens_q=[0, 1], cu_seqlens_k=[0, 2 * BS],
                         block_tables=[table_a[:2]], max_seqlen_q=1, max_seqlen_k=2 * BS)
    before = paged_attention(q, cache, 0, batch, D ** -0.5)
    a_blobs = [Device(cache).export_block(b) for b in table_a[:2]]

    # A second user shares A's two full blocks by reference and forks into
    # two children: the open block is copied per child (copy-on-write).
    b = a[:2 * BS] + [900 + i for i in range(7)]
    shared = eng.pool.match_prefix(hash_chain(b, BS))
    assert shared == table_a[:2]
    own = eng.pool.allocate()
    current["tokens"] = b
    forward(shared + [own], 2 * BS, len(b), b)
    children, pairs = fork_copy_pairs(shared + [own], len(b), BS, 2, eng.pool.allocate)
    assert len(pairs) == 2 and all(p[0] == own for p in pairs)
    KvBlockBackend(cache).copy_blocks(pairs)
    torch.cuda.synchronize()
    for child in children:
        assert child[:2] == shared
        for l in range(L):
            got = kv(cache, l, child, len(b))
            assert torch.equal(got[0], rows_for(b, l, 0))
            assert torch.equal(got[1], rows_for(b, l, 1))
    for child in children:
        eng.pool.free(child[-1])
    eng.pool.free_all(shared + [own])

    # Pressure: two other prompts take every block; A's cached blocks are
    # evicted and exported before the new prompts overwrite them.
    for tag in (1, 2):
        run([10000 * tag + i for i in range(3 * BS)])
    assert store.stats()["writes"] >= 2
    assert not eng.pool.contains(hash_chain(a, BS)[0])
    assert store.get(hash_chain(a, BS)[0]) == a_blobs[0]
    assert store.get(hash_chain(a, BS)[1]) == a_blobs[1]

    # A returns: its two full blocks come back from the spill tier (other
    # block ids), the open block is recomputed.
    cached, table_a2 = run(a)
    assert cached == 2 * BS
    assert store.stats()["hits"] >= 2
    for l in range(L):
        got = kv(cache, l, table_a2, len(a))
        assert torch.equal(got[0], rows_for(a, l, 0)) and torch.equal(got[1], rows_for(a, l, 1))
    batch2 = ForwardBatch(cu_seqlens_q=[0, 1], cu_seqlens_k=[0, 2 * BS],
                          block_tables=[table_a2[:2]], max_seqlen_q=1, max_seqlen_k=2 * BS)
    after = paged_attention(q, cache, 0, batch2, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(before, after)
    store.close()
