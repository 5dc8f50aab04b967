"""GPU parity of the data-movement kernels against the oracle: append,
gather, copy-on-write, export/import and swap — all bit-exact.

Mirrors the reference's cache.rs tests (:308-445) on the device, then runs
the BASELINE configurations' shapes.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from vapi_amd import _lib
from vapi_amd.backend import KvBlockBackend
from vapi_amd.cache import PagedKvCache as _PagedKvCache, gather_kv, write_kv_to_cache
from vapi_amd import workload

pytestmark = pytest.mark.gpu

DEV = "cuda"
BS = 4
# "-bm": a block-major pool (every layer's K and V block of a block side by
# side), the same kernels over a block stride.
LAYOUTS = ["HND", "NHD", "HND-bm", "NHD-bm"]


def PagedKvCache(*args, **kw):
    """The cache, with a "-bm" layout suffix meaning block_major=True."""
    args = list(args)
    if len(args) >= 7 and args[6].endswith("-bm"):
        args[6] = args[6][:-3]
        kw["block_major"] = True
    return _PagedKvCache(*args, **kw)


def rows(n, base, heads=2, width=3, dtype=torch.float32):
    return (base + torch.arange(n * heads * width, dtype=torch.float32)).reshape(
        n, heads, width).to(dtype).to(DEV)


def ref_pool(cache, layer, which="k"):
    """Layer buffer in the reference layout [nb, bs, kvh, d] on the host."""
    return cache.reference_view(layer, which).contiguous().cpu()


def as_np(t: torch.Tensor) -> np.ndarray:
    """Host copy with 16-bit floats kept as raw bits."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("layout", LAYOUTS)
def test_a_write_spanning_non_adjacent_blocks_lands_in_exactly_those_slots(layout):
    c = PagedKvCache(2, 8, BS, 2, 3, torch.float32, layout)
    slots = [24, 25, 26, 27, 4, 5, 6, 7, 12]
    k, v = rows(9, 100.0), rows(9, 1000.0)
    write_kv_to_cache(c, 1, k, v, slots)
    assert torch.equal(gather_kv(c, 1, [6, 1, 3], 9, "k"), k)
    assert torch.equal(gather_kv(c, 1, [6, 1, 3], 9, "v"), v)
    assert float(c.k[0].abs().sum()) == 0.0
    flat = ref_pool(c, 1).reshape(32, 2, 3)
    for slot in range(32):
        assert bool((flat[slot] != 0).any()) == (slot in slots), slot


@pytest.mark.parametrize("layout", LAYOUTS)
def test_slot_5_is_block_1_offset_1(layout):
    c = PagedKvCache(2, 2, BS, 2, 3, torch.float32, layout)
    write_kv_to_cache(c, 0, rows(1, 7.0), rows(1, 9.0), [5])
    assert ref_pool(c, 0)[1][1].tolist() == [[7, 8, 9], [10, 11, 12]]


@pytest.mark.parametrize("layout", LAYOUTS)
def test_a_decode_batch_and_an_overwrite(layout):
    c = PagedKvCache(2, 4, BS, 2, 3, torch.float32, layout)
    slots = [3, 9, 0, 14, 6, 11]
    k = rows(6, 1.0)
    write_kv_to_cache(c, 0, k, k, slots)
    flat = ref_pool(c, 0).reshape(16, 2, 3)
    for i, s in enumerate(slots):
        assert torch.equal(flat[s], k[i].cpu())
    write_kv_to_cache(c, 0, rows(1, 50.0), rows(1, 50.0), [2])
    assert ref_pool(c, 0).reshape(16, 2, 3)[2][0][0] == 50.0


def test_mismatched_shapes_and_out_of_range_slots_are_errors():
    c = PagedKvCache(2, 2, BS, 2, 3, torch.float32)
    with pytest.raises(ValueError):
        write_kv_to_cache(c, 0, rows(2, 0.0), rows(2, 0.0), [0])
    with pytest.raises(ValueError):
        write_kv_to_cache(c, 0, rows(1, 0.0), rows(1, 0.0), [8])
    with pytest.raises(ValueError):
        write_kv_to_cache(c, 0, rows(1, 0.0, dtype=torch.float16),
                          rows(1, 0.0, dtype=torch.float16), [0])


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype,kvh,d", [(torch.bfloat16, 8, 128), (torch.float16, 2, 64),
                                         (torch.float32, 3, 5), (torch.bfloat16, 1, 3)])
def test_append_matches_the_oracle_bit_exactly(layout, dtype, kvh, d):
    rng = np.random.default_rng(11)
    bs, nb, n = 16, 64, 300
    c = PagedKvCache(1, nb, bs, kvh, d, dtype, layout)
    init = torch.randn(c._slab.shape, device=DEV).to(dtype)
    c._slab.copy_(init)
    slots = rng.permutation(nb * bs)[:n].astype(np.uint32)
    slots[rng.choice(n, 15, replace=False)] = _lib.SLOT_SKIP
    k = torch.randn(n, kvh, d, device=DEV).to(dtype)
    v = torch.randn(n, kvh, d, device=DEV).to(dtype)
    want_k, want_v = as_np(ref_pool(c, 0, "k")), as_np(ref_pool(c, 0, "v"))
    oracle.write_rows(want_k, as_np(k), slots)
    oracle.write_rows(want_v, as_np(v), slots)
    write_kv_to_cache(c, 0, k, v, slots)
    np.testing.assert_array_equal(as_np(ref_pool(c, 0, "k")), want_k)
    np.testing.assert_array_equal(as_np(ref_pool(c, 0, "v")), want_v)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype,kvh,d", [(torch.bfloat16, 8, 128), (torch.float16, 2, 64),
                                         (torch.float32, 3, 5)])
def test_a_cold_source_append_writes_the_same_bytes(layout, dtype, kvh, d):
    """VAPI_APPEND_COLD_SOURCE (streaming loads of the source rows) against
    the oracle's scatter, padded and past-the-pool slots included."""
    from vapi_amd.cache import write_rows_indexed
    rng = np.random.default_rng(13)
    bs, nb, n = 16, 64, 333
    c = PagedKvCache(1, nb, bs, kvh, d, dtype, layout)
    c._slab.copy_(torch.randn(c._slab.shape, device=DEV).to(dtype))
    slots = rng.permutation(nb * bs)[:n].astype(np.uint32)
    slots[rng.choice(n, 17, replace=False)] = _lib.SLOT_SKIP
    slots[5] = nb * bs + 1
    k = torch.randn(n, kvh, d, device=DEV).to(dtype)
    v = torch.randn(n, kvh, d, device=DEV).to(dtype)
    dropped = slots.copy()
    dropped[5] = _lib.SLOT_SKIP
    want_k, want_v = as_np(ref_pool(c, 0, "k")), as_np(ref_pool(c, 0, "v"))
    oracle.write_rows(want_k, as_np(k), dropped)
    oracle.write_rows(want_v, as_np(v), dropped)
    write_rows_indexed(c, 0, k, v, torch.from_numpy(slots.view(np.int32)).to(DEV),
                       cold_source=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(as_np(ref_pool(c, 0, "k")), want_k)
    np.testing.assert_array_equal(as_np(ref_pool(c, 0, "v")), want_v)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype,kvh,d", [(torch.bfloat16, 8, 128), (torch.float32, 3, 5)])
def test_a_multi_layer_append_is_one_append_per_layer(layout, dtype, kvh, d):
    """vapi_kv_append_layers over layers 1..3 of a 4-layer pool, the rows of
    each layer a slice of a wider tensor (layer stride != rows): every layer
    equals the oracle's scatter of its rows; layer 0 is untouched."""
    from vapi_amd.cache import write_kv_to_cache_layers
    rng = np.random.default_rng(12)
    bs, nb, n, L = 16, 64, 200, 4
    c = PagedKvCache(L, nb, bs, kvh, d, dtype, layout)
    c._slab.copy_(torch.randn(c._slab.shape, device=DEV).to(dtype))
    slots = rng.permutation(nb * bs)[:n].astype(np.uint32)
    slots[rng.choice(n, 9, replace=False)] = _lib.SLOT_SKIP
    slots[0] = nb * bs + 3  # past the end: dropped on the device
    wide_k = torch.randn(L - 1, n + 7, kvh, d, device=DEV).to(dtype)
    wide_v = torch.randn(L - 1, n + 7, kvh, d, device=DEV).to(dtype)
    k, v = wide_k[:, 3:3 + n], wide_v[:, 3:3 + n]
    want = {(l, w): as_np(ref_pool(c, l, w)) for l in range(L) for w in "kv"}
    dropped = slots.copy()
    dropped[0] = _lib.SLOT_SKIP  # the oracle rejects what the device drops
    for l in range(1, L):
        oracle.write_rows(want[(l, "k")], as_np(k[l - 1]), dropped)
        oracle.write_rows(want[(l, "v")], as_np(v[l - 1]), dropped)
    idx = torch.from_numpy(slots.view(np.int32)).to(DEV)
    write_kv_to_cache_layers(c, 1, k, v, idx)
    torch.cuda.synchronize()
    for (l, w), arr in want.items():
        np.testing.assert_array_equal(as_np(ref_pool(c, l, w)), arr, err_msg=f"layer {l} {w}")


@pytest.mark.parametrize("layout", LAYOUTS)
def test_config1_append_full_size_is_bit_exact(layout):
    """BASELINE config 1 at full size: 4,096 tokens (5% padded) into a
    65,536-block bf16 pool pre-filled with noise; the whole pool (4 GiB) must
    equal the oracle's scatter applied to the same starting bytes."""
    w = workload.config1_append()
    c = PagedKvCache(1, w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim,
                     torch.bfloat16, layout)
    workload.fill_normal(c._slab, 1)
    g = torch.Generator(device=DEV).manual_seed(101)
    k = torch.randn(w.n_tokens, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(w.n_tokens, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    want = {"k": as_np(ref_pool(c, 0, "k")), "v": as_np(ref_pool(c, 0, "v"))}
    write_kv_to_cache(c, 0, k, v, w.slots)
    torch.cuda.synchronize()
    for which, src in (("k", k), ("v", v)):
        runs = oracle.write_rows(want[which], as_np(src), w.slots)
        assert runs > 4  # the reference would take its scatter branch
        np.testing.assert_array_equal(as_np(ref_pool(c, 0, which)), want[which])
        del want[which]


@pytest.mark.parametrize("layout", LAYOUTS)
def test_gather_matches_the_oracle(layout):
    rng = np.random.default_rng(2)
    c = PagedKvCache(2, 40, 16, 4, 64, torch.bfloat16, layout)
    workload.fill_normal(c._slab, 2)
    table = rng.permutation(40)[:9].astype(np.uint32)
    for len_k in (1, 17, 130, 144):
        got = gather_kv(c, 1, table, len_k, "v")
        want = oracle.gather_kv(as_np(ref_pool(c, 1, "v")), table, len_k)
        np.testing.assert_array_equal(as_np(got), want)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_copy_blocks_matches_the_oracle(layout):
    rng = np.random.default_rng(3)
    L, nb = 5, 96
    c = PagedKvCache(L, nb, 16, 4, 128, torch.bfloat16, layout)
    workload.fill_normal(c._slab, 3)
    perm = rng.permutation(nb)
    pairs = np.stack([perm[:20], perm[20:40]], 1)
    ks = [as_np(ref_pool(c, l, "k")) for l in range(L)]
    vs = [as_np(ref_pool(c, l, "v")) for l in range(L)]
    oracle.copy_blocks(ks, vs, pairs)
    KvBlockBackend(c).copy_blocks(pairs.tolist())
    for l in range(L):
        np.testing.assert_array_equal(as_np(ref_pool(c, l, "k")), ks[l])
        np.testing.assert_array_equal(as_np(ref_pool(c, l, "v")), vs[l])


def test_copy_blocks_rejects_overlapping_pairs():
    c = PagedKvCache(1, 8, 16, 1, 64, torch.bfloat16)
    with pytest.raises(ValueError):
        KvBlockBackend(c).copy_blocks([(1, 2), (2, 3)])
    with pytest.raises(ValueError):
        KvBlockBackend(c).copy_blocks([(1, 8)])


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("dtype,kvh,d", [(torch.bfloat16, 4, 128), (torch.float32, 2, 3)])
def test_export_matches_the_reference_byte_order_and_import_inverts_it(layout, dtype, kvh, d):
    L, nb = 3, 12
    c = PagedKvCache(L, nb, 16, kvh, d, dtype, layout)
    workload.fill_normal(c._slab, 4)
    be = KvBlockBackend(c)
    ks = [as_np(ref_pool(c, l, "k")) for l in range(L)]
    vs = [as_np(ref_pool(c, l, "v")) for l in range(L)]
    assert be.block_bytes() == oracle.block_bytes(L, 16, kvh, d, c._slab.element_size())
    for bid in (0, 5, 11):
        assert be.export_block(bid) == oracle.export_block(ks, vs, bid)
    blob = be.export_blocks([3, 7])
    c2 = PagedKvCache(L, nb, 16, kvh, d, dtype, layout)
    be2 = KvBlockBackend(c2)
    be2.import_blocks([9, 1], blob)
    assert be2.export_block(9) == be.export_block(3)
    assert be2.export_block(1) == be.export_block(7)
    be2.import_block(4, be.export_block(11))
    assert be2.export_block(4) == be.export_block(11)
    with pytest.raises(ValueError):
        be2.import_block(0, be.export_block(0)[:-2])


@pytest.mark.parametrize("layout", LAYOUTS)
def test_swap_round_trip_through_pinned_host_is_bit_exact(layout):
    L, nb, n = 4, 64, 20
    c = PagedKvCache(L, nb, 16, 4, 128, torch.bfloat16, layout)
    workload.fill_normal(c._slab, 5)
    be = KvBlockBackend(c)
    bb = be.block_bytes()
    rng = np.random.default_rng(6)
    perm = rng.permutation(nb)
    out_ids, in_ids = perm[:n], perm[n:2 * n]
    host = torch.empty(n * bb, dtype=torch.uint8, pin_memory=True)
    staging = torch.empty(3 * bb + 5, dtype=torch.uint8, device=DEV)  # forces chunking
    side = torch.cuda.Stream()
    ids_out = torch.from_numpy(out_ids.astype(np.int32)).to(DEV)
    ids_in = torch.from_numpy(in_ids.astype(np.int32)).to(DEV)
    want = be.export_blocks(out_ids.tolist()).cpu()
    torch.cuda.synchronize()
    be.swap_out(ids_out, host, staging, stream=side)
    side.synchronize()
    assert torch.equal(host, want)
    be.swap_in(ids_in, host, staging, stream=side)
    side.synchronize()
    for a, b in zip(out_ids, in_ids):
        assert be.export_block(int(b)) == be.export_block(int(a))


def test_the_native_cache_object_mirrors_the_backend_block_methods():
    L = _lib.lib()
    h = ctypes.c_void_p()
    _lib.check(L.vapi_cache_new(2, 8, 4, 2, 3, _lib.F32, _lib.LAYOUT_HND, ctypes.byref(h)))
    try:
        assert L.vapi_cache_num_slots(h) == 32
        assert L.vapi_cache_block_bytes(h) == 2 * 2 * 4 * 2 * 3 * 4
        k = rows(9, 100.0)
        v = rows(9, 1000.0)
        slots = (ctypes.c_uint32 * 9)(24, 25, 26, 27, 4, 5, 6, 7, 12)
        _lib.check(L.vapi_cache_write_kv(h, 1, k.data_ptr(), v.data_ptr(), 9, _lib.F32,
                                         slots, 9, None))
        torch.cuda.synchronize()
        bad = (ctypes.c_uint32 * 1)(32)
        assert L.vapi_cache_write_kv(h, 1, k.data_ptr(), v.data_ptr(), 1, _lib.F32, bad, 1,
                                     None) == _lib.EINVAL
        assert b"past the end" in L.vapi_kv_last_error()
        assert L.vapi_cache_write_kv(h, 1, k.data_ptr(), v.data_ptr(), 2, _lib.F32, bad, 1,
                                     None) == _lib.EINVAL
        bb = L.vapi_cache_block_bytes(h)
        buf = (ctypes.c_uint8 * bb)()
        _lib.check(L.vapi_cache_export_block(h, 6, buf, bb))
        blob = np.frombuffer(bytes(buf), np.float32)
        seg = 4 * 2 * 3
        # Layer 1 K of block 6 holds tokens 0..3 (slots 24..27): k rows 0..3.
        np.testing.assert_array_equal(blob[seg:2 * seg], k[:4].cpu().numpy().reshape(-1))
        np.testing.assert_array_equal(blob[3 * seg:4 * seg], v[:4].cpu().numpy().reshape(-1))
        _lib.check(L.vapi_cache_import_block(h, 2, buf, bb))
        assert L.vapi_cache_import_block(h, 2, buf, bb - 4) == _lib.EINVAL
        pairs = (ctypes.c_uint32 * 2)(2, 5)
        _lib.check(L.vapi_cache_copy_blocks(h, pairs, 1))
        buf2 = (ctypes.c_uint8 * bb)()
        _lib.check(L.vapi_cache_export_block(h, 5, buf2, bb))
        assert bytes(buf2) == bytes(buf)
    finally:
        L.vapi_cache_free(h)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_a_fork_executed_through_copy_blocks_gives_every_child_the_parent_kv(layout):
    """a12 + a13 end to end: the parent's prompt K/V is appended, fork's copy
    pairs run through copy_blocks (every layer, K and V, one launch), and each
    child's table gathers exactly the parent's rows, bit for bit; a write to
    one child's private block leaves the parent and the sibling untouched."""
    from vapi_amd.backend import fork_copy_pairs
    L, nb, bs, kvh, d = 3, 64, 16, 4, 64
    cache = PagedKvCache(L, nb, bs, kvh, d, torch.bfloat16, layout)
    be = KvBlockBackend(cache)
    computed = 43  # two full blocks and 11 rows of a third
    parent = [17, 5, 40]
    slots = [parent[p // bs] * bs + p % bs for p in range(computed)]
    for layer in range(L):
        k = torch.randn(computed, kvh, d, device=DEV).to(torch.bfloat16)
        v = torch.randn(computed, kvh, d, device=DEV).to(torch.bfloat16)
        write_kv_to_cache(cache, layer, k, v, slots)
    free = iter([50, 51, 52])
    children, pairs = fork_copy_pairs(parent, computed, bs, extra=3, allocate=lambda: next(free))
    be.copy_blocks(pairs)
    for layer in range(L):
        for which in ("k", "v"):
            want = as_np(gather_kv(cache, layer, parent, computed, which))
            for child in children:
                assert np.array_equal(as_np(gather_kv(cache, layer, child, computed, which)), want)
    # The children diverge: child 0 rewrites position 40 (its private copy of
    # the partial block); the parent and the sibling keep theirs.
    before = [as_np(gather_kv(cache, 0, t, computed, "k")) for t in (parent, children[1])]
    row = torch.full((1, kvh, d), 3.0, device=DEV).to(torch.bfloat16)
    write_kv_to_cache(cache, 0, row, row, [children[0][2] * bs + 40 % bs])
    after = [as_np(gather_kv(cache, 0, t, computed, "k")) for t in (parent, children[1])]
    assert all(np.array_equal(a, b) for a, b in zip(before, after))
    mine = gather_kv(cache, 0, children[0], computed, "k")
    assert torch.equal(mine[40], row[0]) and not torch.equal(mine[40], gather_kv(cache, 0, parent, computed, "k")[40])


@pytest.mark.parametrize("layout", LAYOUTS)
def test_spilled_blocks_come_back_bit_exact_through_host_memory_and_disk(layout, tmp_path):
    """spill_evicted then promote_from_spill (engine.rs:369-456), batched:
    20 evicted blocks go through a pinned buffer of 3 blocks into a store
    whose host memory holds 8 (the rest on disk); every stored blob is the
    reference's export byte order, and the blobs promoted into other blocks
    equal the originals. A chain is restored up to its first missing hash."""
    import hashlib
    from vapi_amd.spill import SpillStore, pinned_buffer, promote, spill_evicted
    L, nb, n = 3, 64, 20
    c = PagedKvCache(L, nb, 16, 4, 128, torch.bfloat16, layout)
    workload.fill_normal(c._slab, 8)
    be = KvBlockBackend(c)
    bb = be.block_bytes()
    rng = np.random.default_rng(9)
    perm = rng.permutation(nb)
    out_ids, in_ids = perm[:n].tolist(), perm[n:2 * n].tolist()
    hs = [hashlib.sha256(b"chain %d" % i).digest() for i in range(n)]
    ks = [as_np(ref_pool(c, l, "k")) for l in range(L)]
    vs = [as_np(ref_pool(c, l, "v")) for l in range(L)]
    store = SpillStore(tmp_path, 8 * bb, 1 << 30)
    pinned = pinned_buffer(c, 3)
    assert spill_evicted(store, c, zip(hs, out_ids), pinned) == n
    st = store.stats()
    assert (st["ram_blocks"], st["disk_blocks"], st["writes"]) == (8, n - 8, n)
    assert spill_evicted(store, c, zip(hs, out_ids), pinned) == 0  # all held already
    for h, b in zip(hs, out_ids):
        assert store.get(h, bb) == oracle.export_block(ks, vs, b)
    assert promote(store, c, hs, in_ids, pinned) == n
    for a, b in zip(out_ids, in_ids):
        assert be.export_block(b) == be.export_block(a)
    missing = hashlib.sha256(b"never spilled").digest()
    chain = hs[:5] + [missing] + hs[5:7]
    before = store.stats()
    assert promote(store, c, chain, perm[40:48].tolist(), pinned) == 5
    after = store.stats()
    assert (after["hits"] - before["hits"], after["misses"] - before["misses"]) == (5, 1)


@pytest.mark.gpu
def test_async_spill_keeps_the_bytes_the_blocks_held_when_it_was_called(tmp_path):
    """vapi_spill_evicted_async: the blocks are overwritten on the same
    stream right after the call (as the next forward would), the copy to
    host runs on a side stream, and after the drain the store holds each
    block's bytes from before the overwrite, in the export byte order.
    Blocks the store already holds are skipped; put/get drain first."""
    import hashlib
    from vapi_amd.spill import SpillStore, drain, pinned_buffer, spill_evicted_async
    L, nb, n = 2, 48, 12
    c = PagedKvCache(L, nb, 16, 4, 128, torch.bfloat16, "HND")
    workload.fill_normal(c._slab, 3)
    be = KvBlockBackend(c)
    bb = be.block_bytes()
    ids = list(range(5, 5 + n))
    want = [oracle.export_block([as_np(ref_pool(c, l, "k")) for l in range(L)],
                                [as_np(ref_pool(c, l, "v")) for l in range(L)], b) for b in ids]
    hs = [hashlib.sha256(b"async %d" % i).digest() for i in range(n)]
    store = SpillStore(None, 1 << 30, 0)
    store.put(hs[0], want[0])
    staging = torch.empty(n * bb, dtype=torch.uint8, device="cuda")
    pinned = pinned_buffer(c, n)
    side = torch.cuda.Stream()
    assert spill_evicted_async(store, c, zip(hs, ids), staging, pinned, side=side) == n - 1
    c._slab.zero_()  # the next forward reuses the blocks, on the same stream
    assert drain(store) == n - 1
    assert drain(store) == 0
    torch.cuda.synchronize()
    for h, w in zip(hs, want):
        assert store.get(h, bb) == w
    # A second export drains by itself at the next store call.
    h2 = hashlib.sha256(b"async second").digest()
    assert spill_evicted_async(store, c, [(h2, 7)], staging, pinned, side=side) == 1
    assert store.get(h2, bb) == bytes(bb)
    with pytest.raises(Exception, match="staging"):
        spill_evicted_async(store, c, [(hashlib.sha256(b"x%d" % i).digest(), i) for i in range(3)],
                            staging[:bb], pinned, side=side)


@pytest.mark.gpu
def test_async_spills_in_flight_on_a_ring_of_buffers_all_arrive_intact():
    """Five asynchronous exports over a ring of three staging/pinned pairs,
    each followed by an overwrite of its blocks on the model's stream: the
    fourth and fifth reuse buffers still in flight (the call waits for those
    first). Hashes already in flight are skipped. After the drain every blob
    is its block's bytes from before the overwrite."""
    import hashlib
    from vapi_amd.spill import SpillStore, drain, pinned_buffer, spill_evicted_async
    L, nb, per = 2, 64, 4
    c = PagedKvCache(L, nb, 16, 4, 128, torch.bfloat16, "HND")
    workload.fill_normal(c._slab, 5)
    be = KvBlockBackend(c)
    bb = be.block_bytes()
    ring = [(torch.empty(per * bb, dtype=torch.uint8, device="cuda"), pinned_buffer(c, per))
            for _ in range(3)]
    side = torch.cuda.Stream()
    store = SpillStore(None, 1 << 30, 0)
    want = {}
    for call in range(5):
        ids = list(range(per * call, per * call + per))
        hs = [hashlib.sha256(b"ring %d" % b).digest() for b in ids]
        for h, b in zip(hs, ids):
            want[h] = be.export_block(b)
        staging, pinned = ring[call % 3]
        assert spill_evicted_async(store, c, zip(hs, ids), staging, pinned, side=side) == per
        if call == 0:  # the same hashes again while in flight: nothing to do
            assert spill_evicted_async(store, c, zip(hs, ids), ring[1][0], ring[1][1],
                                       side=side) == 0
        for b in ids:  # the next forward reuses the blocks
            for t in c.k + c.v:
                t[b].fill_(float(call + 1))
    drain(store)
    torch.cuda.synchronize()
    assert store.stats()["ram_blocks"] == 5 * per
    for h, w in want.items():
        assert store.get(h, bb) == w


# ---- rows layers and caches whose layers differ -------------------------------------------

def _np_layers(c):
    """Per-layer pools as the reference's [nb, bs, kvh, d] numpy arrays (None
    for a rows layer's V)."""
    ks = [as_np(c.reference_view(l, "k").contiguous()) for l in range(c.num_layers)]
    vs = [as_np(c.reference_view(l, "v").contiguous()) if c.v[l].dim() == 4 else None
          for l in range(c.num_layers)]
    return ks, vs


@pytest.mark.gpu
def test_a_rows_layer_stores_one_row_per_token_and_no_v():
    """cache.rs:414-436 on the device: rows 0..9 written at slots 9, 10 of a
    Rows(5) layer come back from block 2 after an untouched slot 8; the K/V
    layer beside it stays zero; V rows or a V gather on it are errors."""
    from vapi_amd.cache import HybridKvCache, write_k_to_cache
    c = HybridKvCache([("kv", 2, 3), ("rows", 5)], 4, 4, torch.float32, "NHD")
    assert tuple(c.k[1].shape) == (4, 4, 1, 5) and c.v[1].numel() == 0
    rows_ = torch.arange(10, dtype=torch.float32, device=DEV).reshape(2, 1, 5)
    write_k_to_cache(c, 1, rows_, [9, 10])
    got = gather_kv(c, 1, [2], 3).reshape(3, 5).cpu().tolist()
    assert got == [[0.0] * 5, [0.0, 1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0, 9.0]]
    assert float(c.k[0].abs().sum()) == 0.0
    with pytest.raises(ValueError):
        write_kv_to_cache(c, 1, rows_, rows_, [0, 1])
    with pytest.raises(ValueError):
        gather_kv(c, 1, [2], 3, which="v")


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["HND", "NHD"])
def test_a_mixed_cache_moves_blocks_like_the_reference(layout):
    """A cache of layers Kv(4, 128), Rows(40), Kv(4, 128), Rows(24), Kv(2, 64)
    (a hybrid model's attention and short-convolution layers), bf16: its
    block bytes, export, import, copy_blocks and swap through pinned memory
    against the oracle's per-buffer restatement of backend.rs:695-797,
    bit-exact; single-buffer writes (write_k_to_cache on a K/V layer,
    write_v_rows_indexed) touch only their buffer."""
    from vapi_amd.cache import HybridKvCache, write_k_to_cache, write_v_rows_indexed
    specs = [("kv", 4, 128), ("rows", 40), ("kv", 4, 128), ("rows", 24), ("kv", 2, 64)]
    nb = 40
    c = HybridKvCache(specs, nb, 16, torch.bfloat16, layout)
    g = torch.Generator(device=DEV).manual_seed(7)
    for t in c.k + c.v:
        if t.numel():
            t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(t.dtype))
    be = KvBlockBackend(c)
    ks, vs = _np_layers(c)
    assert be.block_bytes() == oracle.cache_block_bytes(ks, vs)
    ids = [3, 17, 0, 39, 22]
    blob = be.export_blocks(ids)
    bb = be.block_bytes()
    for j, b in enumerate(ids):
        assert blob[j * bb:(j + 1) * bb].cpu().numpy().tobytes() == oracle.export_block(ks, vs, b)
    # Import into other blocks: they equal the sources, nothing else moves.
    before = [t.clone() for t in c.k + c.v]
    dst = [5, 6, 30, 31, 8]
    be.import_blocks(dst, blob)
    torch.cuda.synchronize()
    for t, t0 in zip(c.k + c.v, before):
        if t.numel():
            assert torch.equal(t[dst], t0[ids])
            keep = [i for i in range(nb) if i not in dst]
            assert torch.equal(t[keep], t0[keep])
    # copy_blocks against the oracle.
    ks, vs = _np_layers(c)
    pairs = [(1, 10), (2, 11), (39, 12)]
    be.copy_blocks(pairs)
    oracle.copy_blocks(ks, vs, pairs)
    got_k, got_v = _np_layers(c)
    for a, b in zip(ks + vs, got_k + got_v):
        if a is not None:
            np.testing.assert_array_equal(a.view(np.uint16), b.view(np.uint16))
    # Swap out through pinned memory and back into other blocks.
    ids_dev = torch.tensor([4, 9], dtype=torch.int32, device=DEV)
    host = torch.empty(2 * bb, dtype=torch.uint8, pin_memory=True)
    staging = torch.empty(bb, dtype=torch.uint8, device=DEV)
    be.swap_out(ids_dev, host, staging)
    back = torch.tensor([13, 14], dtype=torch.int32, device=DEV)
    be.swap_in(back, host, staging)
    torch.cuda.synchronize()
    assert be.export_block(13) == be.export_block(4) and be.export_block(14) == be.export_block(9)
    # Single-buffer writes.
    k0 = c.k[0].clone()
    v0 = c.v[0].clone()
    rows_k = torch.randn(3, 4, 128, generator=g, device=DEV).to(torch.bfloat16)
    write_k_to_cache(c, 0, rows_k, [16 * 20, 16 * 20 + 1, 16 * 21])
    assert torch.equal(c.v[0], v0)
    idx = torch.tensor([16 * 25 + 3], dtype=torch.int32, device=DEV)
    write_v_rows_indexed(c, 0, rows_k[:1], idx)
    ref_k = c.reference_view(0, "k")
    ref_v = c.reference_view(0, "v")
    assert torch.equal(ref_k[20, 0], rows_k[0]) and torch.equal(ref_k[21, 0], rows_k[2])
    assert torch.equal(ref_v[25, 3], rows_k[0])
    changed = (c.k[0] != k0).flatten(1).any(1).nonzero().flatten().tolist()
    assert changed == [20, 21]


@pytest.mark.gpu
def test_a_mixed_cache_spills_and_promotes_bit_exact():
    """The spill tier over a chained cache: blobs are the whole chain's
    blocks in the reference byte order and come back intact."""
    import hashlib
    from vapi_amd.cache import HybridKvCache
    from vapi_amd.spill import SpillStore, pinned_buffer, promote, spill_evicted
    c = HybridKvCache([("rows", 48), ("kv", 2, 128), ("rows", 48)], 32, 16, torch.bfloat16)
    for t in c.k + c.v:
        if t.numel():
            workload.fill_normal(t, 11)
    be = KvBlockBackend(c)
    ks, vs = _np_layers(c)
    hs = [hashlib.sha256(b"mixed %d" % i).digest() for i in range(6)]
    store = SpillStore(None, 1 << 30, 0)
    pinned = pinned_buffer(c, 4)
    assert spill_evicted(store, c, zip(hs, range(6)), pinned) == 6
    for i, h in enumerate(hs):
        assert store.get(h, be.block_bytes()) == oracle.export_block(ks, vs, i)
    assert promote(store, c, hs, list(range(20, 26)), pinned) == 6
    for i in range(6):
        assert be.export_block(20 + i) == be.export_block(i)


@pytest.mark.gpu
def test_block_ids_past_the_pool_move_nothing():
    """Device-side ids the host never checked: an id past the pool is
    skipped by copy and import, leaves its blob untouched on export, and a
    table entry past the pool gathers zeros; host-side ids (the spill
    calls) past the pool are errors."""
    from vapi_amd._lib import VapiKvError, check, lib
    from vapi_amd.backend import _dev_u32
    from vapi_amd.spill import SpillStore, pinned_buffer, spill_evicted
    c = PagedKvCache(2, 8, 16, 2, 64, torch.bfloat16, "HND")
    workload.fill_normal(c._slab, 4)
    be = KvBlockBackend(c)
    bb = be.block_bytes()
    before = c._slab.clone()
    pairs = _dev_u32([1, 2, 100, 3, 4, 100], DEV)
    check(lib().vapi_kv_copy_blocks(c.pool, pairs.data_ptr(), 3, None))
    torch.cuda.synchronize()
    assert torch.equal(c.k[0][2], before[0, 0].view(c.k[0].shape)[1])
    assert torch.equal(c.k[0][3], before[0, 0].view(c.k[0].shape)[3])  # skipped pair
    blob = torch.full((2 * bb,), 7, dtype=torch.uint8, device=DEV)
    ids = _dev_u32([5, 1 << 20], DEV)
    check(lib().vapi_kv_export_blocks(c.pool, ids.data_ptr(), 2, blob.data_ptr(), None))
    torch.cuda.synchronize()
    assert blob[:bb].cpu().numpy().tobytes() == be.export_block(5)
    assert bool((blob[bb:] == 7).all())
    snap = c._slab.clone()
    check(lib().vapi_kv_import_blocks(c.pool, ids.data_ptr(), 2, blob.data_ptr(), None))
    torch.cuda.synchronize()
    assert torch.equal(c._slab, snap)
    table = _dev_u32([0, 99], DEV)
    out = torch.full((32, 2, 64), 3.0, dtype=torch.bfloat16, device=DEV)
    check(lib().vapi_kv_gather(c.pool, 0, table.data_ptr(), 2, 32, out.data_ptr(), None, None))
    torch.cuda.synchronize()
    assert torch.equal(out[:16], ref_pool(c, 0, "k")[0].to(DEV))
    assert bool((out[16:] == 0).all())
    store = SpillStore(None, 1 << 30, 0)
    with pytest.raises(VapiKvError, match="block 8 of 8"):
        spill_evicted(store, c, [(bytes(32), 8)], pinned_buffer(c, 1))


@pytest.mark.gpu
def test_attention_over_a_layer_of_a_mixed_cache_matches_the_oracle():
    """The K/V layers of a mixed cache attend like a uniform cache's (their
    per-layer view is an ordinary pool); a rows layer is refused."""
    from vapi_amd.attention import ForwardBatch, paged_attention
    from vapi_amd.cache import HybridKvCache
    c = HybridKvCache([("rows", 40), ("kv", 2, 64), ("rows", 40), ("kv", 2, 64)], 16, 16,
                      torch.float32, "NHD")
    g = torch.Generator(device=DEV).manual_seed(5)
    for t in c.k + c.v:
        if t.numel():
            t.copy_(torch.randn(t.shape, generator=g, device=DEV))
    batch = ForwardBatch(cu_seqlens_q=[0, 1, 6], cu_seqlens_k=[0, 40, 70],
                         block_tables=[[3, 1, 7], [9, 2]], max_seqlen_q=5, max_seqlen_k=40)
    q = torch.randn(6, 4, 64, generator=g, device=DEV)
    for layer in (1, 3):
        got = paged_attention(q, c, layer, batch, 0.125)
        want = oracle.paged_attention(q.cpu().numpy(), as_np(c.reference_view(layer, "k")),
                                      as_np(c.reference_view(layer, "v")), batch.cu_seqlens_q,
                                      batch.cu_seqlens_k, batch.block_tables, 0.125, None, 0)
        assert float(np.abs(got.cpu().numpy() - want).max()) <= 1e-5
    with pytest.raises(Exception):
        paged_attention(q, c, 0, batch, 0.125)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["HND", "NHD"])
def test_a_bf16_mixed_cache_runs_the_mfma_kernels_per_layer(layout):
    """bf16 K/V layers of different geometry (head_dim 64 and 128, 2 and 4
    kv heads) beside rows layers: each layer's attention (decode and
    prefill rows, so both MFMA kernels) and the fused append + attention
    through one PreparedAttention whose workspace is sized up front for the
    largest layer (no layer reallocates it), against the oracle (bf16
    max-abs <= 2e-2 * max|reference|) and the two-call sequence."""
    from test_gpu_append_attention import dev_slots
    from vapi_amd.attention import (ForwardBatch, PreparedAttention,
                                    paged_attention_append_prepared, paged_attention_prepared)
    from vapi_amd.cache import HybridKvCache, write_rows_indexed
    spec = [("rows", 48), ("kv", 2, 64), ("kv", 4, 128), ("rows", 48), ("kv", 4, 64)]
    c = HybridKvCache(spec, 64, 16, torch.bfloat16, layout)
    g = torch.Generator(device=DEV).manual_seed(11)
    for t in c.k + c.v:
        if t.numel():
            t.copy_(torch.randn(t.shape, generator=g, device=DEV).to(torch.bfloat16))
    tables = [[3, 1, 7, 20, 21, 22], [9, 2, 40], [50, 51, 52, 53, 54, 55, 56, 57]]
    lens_k, lens_q = [90, 40, 128], [1, 7, 1]
    batch = ForwardBatch(cu_seqlens_q=np.concatenate([[0], np.cumsum(lens_q)]).tolist(),
                         cu_seqlens_k=np.concatenate([[0], np.cumsum(lens_k)]).tolist(),
                         block_tables=tables, max_seqlen_q=7, max_seqlen_k=128)
    heads = 8
    prep = PreparedAttention.from_batch(batch, DEV, cache=c, num_heads=heads)
    ws = prep.workspace
    assert ws is not None
    for layer in (1, 2, 4):
        d = spec[layer][2]
        q = torch.randn(sum(lens_q), heads, d, generator=g, device=DEV).to(torch.bfloat16)
        got = paged_attention_prepared(q, c, layer, prep, d ** -0.5)
        assert prep.workspace is ws, "a layer reallocated the step's workspace"
        want = oracle.paged_attention(q.float().cpu().numpy(),
                                      c.reference_view(layer, "k").float().cpu().numpy(),
                                      c.reference_view(layer, "v").float().cpu().numpy(),
                                      batch.cu_seqlens_q, batch.cu_seqlens_k, tables, d ** -0.5)
        want = torch.from_numpy(want).to(torch.bfloat16).float()
        assert float((got.float().cpu() - want).abs().max()) <= 2e-2 * float(want.abs().max())
    # Fused append + attention on a decode batch, per layer, against the two calls.
    dec = ForwardBatch(cu_seqlens_q=[0, 1, 2], cu_seqlens_k=[0, 90, 218],
                       block_tables=[tables[0], tables[1] + tables[2][:6]], max_seqlen_q=1,
                       max_seqlen_k=128)
    slots = [tables[0][89 // 16] * 16 + 89 % 16, dec.block_tables[1][127 // 16] * 16 + 127 % 16]
    s = dev_slots(slots)
    for layer in (1, 2):
        kvh, d = spec[layer][1], spec[layer][2]
        q = torch.randn(2, heads, d, generator=g, device=DEV).to(torch.bfloat16)
        k_new = torch.randn(2, kvh, d, generator=g, device=DEV).to(torch.bfloat16)
        v_new = torch.randn_like(k_new)
        before_k = c.k[layer].clone(), c.v[layer].clone()
        p1 = PreparedAttention.from_batch(dec, DEV, cache=c, num_heads=heads)
        fused = paged_attention_append_prepared(q, k_new, v_new, s, c, layer, p1, d ** -0.5)
        after = c.k[layer].clone(), c.v[layer].clone()
        c.k[layer].copy_(before_k[0]), c.v[layer].copy_(before_k[1])
        write_rows_indexed(c, layer, k_new, v_new, s)
        assert torch.equal(c.k[layer], after[0]) and torch.equal(c.v[layer], after[1])
        p2 = PreparedAttention.from_batch(dec, DEV, cache=c, num_heads=heads)
        two = paged_attention_prepared(q, c, layer, p2, d ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(fused, two)
