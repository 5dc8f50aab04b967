"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Each oracle function is checked against something other than itself:
  write_rows      the reference's known-answer tests (cache.rs:308-445),
                  run-path == scatter-path, overwrite semantics, errors.
  gather_kv       cache.rs:308-337 (gather returns exactly what was written),
                  brute-force slot arithmetic.
  pack_block_tables  attention.rs:414-423.
  paged_attention closed forms (attention.rs:323-353 window means; Q = 0
                  gives the mean of the visible V), the mixed-batch test of
                  attention.rs:355-405 against a dense oracle, an f64 brute
                  force and a vectorised numpy formulation with GQA and
                  windows; len_q == len_k is plain causal; decode sees all.
  export/import/copy  byte order by layer stamps (backend.rs:718-773),
                  import∘export = identity (vapi-worker engine.rs:1282-1293),
                  length check, copy semantics (backend.rs:781-797).
  block_bytes     lib.rs:143-157 (1 GiB holds 1024 blocks of 1 MiB).
"""
import numpy as np
import pytest

import oracle

BS = 4


def rows(n, base, heads=2, width=3):
    """cache.rs:302-306: every element distinct."""
    return (base + np.arange(n * heads * width, dtype=np.float32)).reshape(n, heads, width)


def cache(num_blocks, layers=2, heads=2, width=3, dtype=np.float32):
    k = [np.zeros((num_blocks, BS, heads, width), dtype) for _ in range(layers)]
    v = [np.zeros((num_blocks, BS, heads, width), dtype) for _ in range(layers)]
    return k, v


def write_kv(kc, vc, layer, k, v, slots, force_scatter=False):
    if k.shape != v.shape:
        raise ValueError("k and v differ in shape")
    oracle.write_rows(kc[layer], k, slots, force_scatter)
    return oracle.write_rows(vc[layer], v, slots, force_scatter)


# ---- cache.rs known answers -------------------------------------------------

def test_a_write_spanning_non_adjacent_blocks_lands_in_exactly_those_slots():
    kc, vc = cache(8)
    slots = [24, 25, 26, 27, 4, 5, 6, 7, 12]
    k, v = rows(9, 100.0), rows(9, 1000.0)
    runs = write_kv(kc, vc, 1, k, v, slots)
    assert runs == 3
    np.testing.assert_array_equal(oracle.gather_kv(kc[1], [6, 1, 3], 9), k)
    np.testing.assert_array_equal(oracle.gather_kv(vc[1], [6, 1, 3], 9), v)
    assert kc[0].sum() == 0.0
    flat = kc[1].reshape(32, 2, 3)
    for slot in range(32):
        assert bool(np.any(flat[slot] != 0)) == (slot in slots), slot


def test_the_flat_view_shares_storage_with_the_paged_tensor():
    kc, vc = cache(2)
    write_kv(kc, vc, 0, rows(1, 7.0), rows(1, 9.0), [5])
    np.testing.assert_array_equal(kc[0][1][1], [[7, 8, 9], [10, 11, 12]])


def test_a_decode_batch_is_many_single_slot_runs():
    kc, vc = cache(4)
    slots = [3, 9, 0, 14, 6, 11]
    k = rows(6, 1.0)
    assert write_kv(kc, vc, 0, k, k, slots) == 6
    flat = kc[0].reshape(16, 2, 3)
    for i, s in enumerate(slots):
        np.testing.assert_array_equal(flat[s], k[i])


def test_the_scatter_path_and_the_run_path_agree():
    slots = [30, 31, 5, 6, 7, 12, 20, 2]
    k = rows(8, 3.0)
    a, _ = cache(8)
    b, _ = cache(8)
    assert oracle.write_rows(a[0], k, slots) == 5
    for i, s in enumerate(slots):
        oracle.write_rows(b[0], k[i:i + 1], [s])
    np.testing.assert_array_equal(a[0], b[0])
    assert np.count_nonzero(a[0]) > 0
    c, _ = cache(8)
    oracle.write_rows(c[0], k, slots, force_scatter=True)
    np.testing.assert_array_equal(a[0], c[0])


def test_a_second_write_overwrites_rather_than_accumulates():
    kc, vc = cache(2)
    write_kv(kc, vc, 0, rows(1, 1.0), rows(1, 1.0), [2])
    write_kv(kc, vc, 0, rows(1, 50.0), rows(1, 50.0), [2])
    assert kc[0].reshape(8, 2, 3)[2][0][0] == 50.0


def test_mismatched_shapes_and_out_of_range_slots_are_errors():
    kc, vc = cache(2)
    with pytest.raises(ValueError):
        write_kv(kc, vc, 0, rows(2, 0.0), rows(2, 0.0), [0])
    with pytest.raises(ValueError):
        write_kv(kc, vc, 0, rows(1, 0.0), rows(1, 0.0), [8])
    with pytest.raises(ValueError):
        write_kv(kc, vc, 0, rows(1, 0.0).astype(np.float16), rows(1, 0.0).astype(np.float16), [0])


def test_padded_slots_write_nothing():
    kc, vc = cache(4)
    k = rows(5, 1.0)
    slots = [3, oracle.SKIP, 9, oracle.SKIP, 0]
    write_kv(kc, vc, 0, k, k, slots)
    flat = kc[0].reshape(16, 2, 3)
    for i, s in enumerate(slots):
        if s != oracle.SKIP:
            np.testing.assert_array_equal(flat[s], k[i])
    assert np.count_nonzero(flat) == 3 * 6


def test_gather_kv_is_block_table_arithmetic():
    rng = np.random.default_rng(1)
    pool = rng.standard_normal((6, BS, 2, 3)).astype(np.float32)
    table = [4, 0, 5]
    got = oracle.gather_kv(pool, table, 10)
    for t in range(10):
        np.testing.assert_array_equal(got[t], pool[table[t // BS], t % BS])
    with pytest.raises(ValueError):
        oracle.gather_kv(pool, table, 13)


def test_ragged_block_tables_are_padded_to_a_rectangle():
    t = oracle.pack_block_tables([[0, 1, 2], [7]])
    np.testing.assert_array_equal(t, [[0, 1, 2], [7, 7, 7]])
    np.testing.assert_array_equal(oracle.pack_block_tables([[], [3]]), [[0], [3]])


# ---- attention ------------------------------------------------------------------

def dense_np(q, k, v, scale, window=None, window_right=0):
    """Vectorised dense attention for one sequence (a different formulation
    from the oracle's loops): q [Lq,H,D], k/v [Lk,KVH,D] logical order."""
    lq, h, _ = q.shape
    lk, kvh, _ = k.shape
    g = h // kvh
    kk = np.repeat(k.astype(np.float64), g, axis=1)
    vv = np.repeat(v.astype(np.float64), g, axis=1)
    s = np.einsum("qhd,khd->hqk", q.astype(np.float64), kk) * scale
    p = (lk - lq + np.arange(lq))[:, None]
    key = np.arange(lk)[None, :]
    hidden = np.zeros((lq, lk), bool)
    if window_right is not None and window_right >= 0:
        hidden |= key > p + window_right
    if window is not None:
        hidden |= (key < p) & (p - key >= window)
    s = np.where(hidden[None], -np.inf, s)
    s = np.exp(s - s.max(-1, keepdims=True))
    s /= s.sum(-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", s, vv)


def test_a_sliding_window_hides_keys_older_than_the_window():
    # attention.rs:323-353: window 3, Q = 0, K = (i, 0), V = (1, i).
    kc = np.zeros((2, 4, 1, 2), np.float32)
    vc = np.zeros((2, 4, 1, 2), np.float32)
    k = np.array([[i, 0.0] for i in range(6)], np.float32).reshape(6, 1, 2)
    v = np.array([[1.0, i] for i in range(6)], np.float32).reshape(6, 1, 2)
    oracle.write_rows(kc, k, list(range(6)))
    oracle.write_rows(vc, v, list(range(6)))
    q = np.zeros((6, 1, 2), np.float32)
    out = oracle.paged_attention(q, kc, vc, [0, 6], [0, 6], [[0, 1]], 1.0, sliding_window=3)
    np.testing.assert_array_equal(out[:, 0, 1], [0.0, 0.5, 1.0, 2.0, 3.0, 4.0])


def test_the_cpu_reference_matches_dense_attention_for_a_mixed_batch():
    # attention.rs:355-405.
    kc = np.zeros((8, 4, 1, 4), np.float32)
    vc = np.zeros((8, 4, 1, 4), np.float32)

    def rnd(n, seed):
        return np.array([[np.sin(np.float32((i * 7 + d * 3) * np.float32(0.37)) + np.float32(seed))
                          for d in range(4)] for i in range(n)], np.float32)

    ka, va, kb, vb = rnd(8, 0.1), rnd(8, 0.2), rnd(6, 0.3), rnd(6, 0.4)
    ta, tb = [5, 2], [7, 0]

    def slots(t, n):
        return [t[p // 4] * 4 + p % 4 for p in range(n)]

    oracle.write_rows(kc, ka.reshape(8, 1, 4), slots(ta, 8))
    oracle.write_rows(vc, va.reshape(8, 1, 4), slots(ta, 8))
    oracle.write_rows(kc, kb.reshape(6, 1, 4), slots(tb, 6))
    oracle.write_rows(vc, vb.reshape(6, 1, 4), slots(tb, 6))
    qa, qb = rnd(3, 0.5), rnd(1, 0.6)
    q = np.concatenate([qa, qb]).reshape(4, 1, 4)
    out = oracle.paged_attention(q, kc, vc, [0, 3, 4], [0, 8, 14], [ta, tb], 0.5)
    assert out.shape == (4, 1, 4)
    want_a = oracle.dense_attention_f64(qa.reshape(3, 1, 4), ka.reshape(8, 1, 4),
                                        va.reshape(8, 1, 4), 0.5)
    want_b = oracle.dense_attention_f64(qb.reshape(1, 1, 4), kb.reshape(6, 1, 4),
                                        vb.reshape(6, 1, 4), 0.5)
    want = np.concatenate([want_a, want_b])
    assert np.abs(out - want).max() < 1e-5
    np.testing.assert_allclose(want_a, dense_np(qa.reshape(3, 1, 4), ka.reshape(8, 1, 4),
                                                va.reshape(8, 1, 4), 0.5), atol=1e-12)


def _random_paged(rng, lens_q, lens_k, heads, kvh, d, bs, nb):
    kc = rng.standard_normal((nb, bs, kvh, d)).astype(np.float32)
    vc = rng.standard_normal((nb, bs, kvh, d)).astype(np.float32)
    perm = rng.permutation(nb)
    tables, at = [], 0
    for lk in lens_k:
        n = -(-lk // bs)
        tables.append(perm[at:at + n].astype(np.uint32))
        at += n
    q = rng.standard_normal((sum(lens_q), heads, d)).astype(np.float32)
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.uint32)
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.uint32)
    return q, kc, vc, cu_q, cu_k, tables


@pytest.mark.parametrize("heads,kvh,window,wr", [(4, 2, None, 0), (6, 2, 5, 0),
                                                 (8, 2, None, -1), (3, 3, 7, 0),
                                                 (16, 8, None, 0)])
def test_oracle_matches_f64_and_numpy_dense(heads, kvh, window, wr):
    rng = np.random.default_rng(heads * 100 + kvh)
    d, bs = 16, 4
    lens_q, lens_k = [5, 1, 9, 0], [13, 7, 9, 3]
    q, kc, vc, cu_q, cu_k, tables = _random_paged(rng, lens_q, lens_k, heads, kvh, d, bs, 32)
    scale = d ** -0.5
    out = oracle.paged_attention(q, kc, vc, cu_q, cu_k, tables, scale, window, wr)
    for i in range(len(lens_q)):
        if lens_q[i] == 0:
            continue
        qi = q[cu_q[i]:cu_q[i + 1]]
        ki = oracle.gather_kv(kc, tables[i], lens_k[i])
        vi = oracle.gather_kv(vc, tables[i], lens_k[i])
        f64 = oracle.dense_attention_f64(qi, ki, vi, scale, window, wr)
        npd = dense_np(qi, ki, vi, scale, window, wr)
        np.testing.assert_allclose(f64, npd, atol=1e-12)
        assert np.abs(out[cu_q[i]:cu_q[i + 1]] - f64).max() < 1e-5


def test_zero_queries_give_the_mean_of_the_visible_values():
    # Closed form: uniform weights over keys max(0, p-w+1)..p.
    rng = np.random.default_rng(7)
    heads, kvh, d, bs = 4, 2, 8, 4
    lens_q, lens_k = [6], [11]
    _, kc, vc, cu_q, cu_k, tables = _random_paged(rng, lens_q, lens_k, heads, kvh, d, bs, 8)
    q = np.zeros((6, heads, d), np.float32)
    for window in (None, 3):
        out = oracle.paged_attention(q, kc, vc, cu_q, cu_k, tables, 0.3, window)
        vi = oracle.gather_kv(vc, tables[0], 11)
        for j in range(6):
            p = 11 - 6 + j
            lo = 0 if window is None else max(0, p - window + 1)
            for h in range(heads):
                want = vi[lo:p + 1, h // 2].astype(np.float64).mean(0)
                assert np.abs(out[j, h] - want).max() < 1e-6


def test_equal_lengths_is_plain_causal_and_decode_sees_every_key():
    rng = np.random.default_rng(3)
    heads, kvh, d, bs = 2, 1, 8, 4
    q, kc, vc, cu_q, cu_k, tables = _random_paged(rng, [7, 1], [7, 9], heads, kvh, d, bs, 8)
    out = oracle.paged_attention(q, kc, vc, cu_q, cu_k, tables, 0.5)
    full = oracle.paged_attention(q, kc, vc, cu_q, cu_k, tables, 0.5, None, -1)
    # Row j of the first sequence attends to keys 0..j: equals attention over
    # the prefix alone, computed as a decode of a shorter sequence.
    for j in range(7):
        sub = oracle.paged_attention(q[j:j + 1], kc, vc, [0, 1], [0, j + 1], [tables[0]], 0.5)
        np.testing.assert_allclose(out[j], sub[0], atol=1e-6)
    # The decode row is the same causal or not.
    np.testing.assert_array_equal(out[7], full[7])
    assert np.abs(out[:7] - full[:7]).max() > 1e-3


# ---- block methods ------------------------------------------------------------------

def test_export_order_is_k_layers_then_v_layers_and_import_inverts_it():
    layers, nb, heads, width = 3, 5, 2, 4
    kc = [np.full((nb, BS, heads, width), 10 + l, np.float32) for l in range(layers)]
    vc = [np.full((nb, BS, heads, width), 20 + l, np.float32) for l in range(layers)]
    blob = np.frombuffer(oracle.export_block(kc, vc, 2), np.float32)
    seg = BS * heads * width
    assert blob.size == 2 * layers * seg
    assert oracle.block_bytes(layers, BS, heads, width, 4) == blob.nbytes
    for s in range(2 * layers):
        want = 10 + s if s < layers else 20 + s - layers
        assert (blob[s * seg:(s + 1) * seg] == want).all()
    # Round trip into a different block of a fresh cache.
    rng = np.random.default_rng(0)
    for p in kc + vc:
        p[...] = rng.standard_normal(p.shape)
    data = oracle.export_block(kc, vc, 1)
    k2 = [np.zeros_like(p) for p in kc]
    v2 = [np.zeros_like(p) for p in vc]
    oracle.import_block(k2, v2, 4, data)
    for a, b in zip(kc + vc, k2 + v2):
        np.testing.assert_array_equal(a[1], b[4])
        assert np.count_nonzero(b[:4]) == 0
    assert oracle.export_block(k2, v2, 4) == data
    with pytest.raises(ValueError):
        oracle.import_block(k2, v2, 0, data[:-4])


def test_copy_blocks_copies_every_layer_and_nothing_else():
    rng = np.random.default_rng(5)
    kc = [rng.standard_normal((6, BS, 2, 3)).astype(np.float32) for _ in range(2)]
    vc = [rng.standard_normal((6, BS, 2, 3)).astype(np.float32) for _ in range(2)]
    before = [p.copy() for p in kc + vc]
    oracle.copy_blocks(kc, vc, [(1, 4), (0, 5)])
    for a, b in zip(before, kc + vc):
        np.testing.assert_array_equal(b[4], a[1])
        np.testing.assert_array_equal(b[5], a[0])
        np.testing.assert_array_equal(b[:4], a[:4])


def test_block_sizing_matches_hand_arithmetic():
    # lib.rs:143-157: 16 layers, 8 kv heads, head_dim 64, bf16, BS 32 ->
    # 1 MiB per block, 1024 blocks per GiB; f32 halves the count.
    per_block = oracle.block_bytes(16, 32, 8, 64, 2)
    assert (1 << 30) // per_block == 1024
    assert (1 << 30) // oracle.block_bytes(16, 32, 8, 64, 4) == 512


# ---- rows layers and caches whose layers differ --------------------------------------

def test_a_rows_layer_stores_one_row_per_token_and_no_v():
    """cache.rs:414-436: a Kv(2, 3) layer and a Rows(5) layer; the rows layer
    is [4, BS, 1, 5], K only; rows 0..9 at slots 9, 10 come back from block 2
    (slots 8..11) after an untouched slot 8."""
    k0 = np.zeros((4, BS, 2, 3), np.float32)
    k1 = np.zeros((4, BS, 1, 5), np.float32)
    assert k1.shape == (4, BS, 1, 5)
    assert (2 * 2 * 3) + 5 == 17  # elems_per_token of the two layouts
    rows_ = np.arange(10, dtype=np.float32).reshape(2, 1, 5)
    oracle.write_rows(k1, rows_, [9, 10])
    got = oracle.gather_kv(k1, [2], 3).reshape(3, 5)
    np.testing.assert_array_equal(got[0], np.zeros(5))
    np.testing.assert_array_equal(got[1], [0, 1, 2, 3, 4])
    np.testing.assert_array_equal(got[2], [5, 6, 7, 8, 9])
    assert k0.sum() == 0


def test_a_mixed_cache_exports_k_of_every_layer_then_the_v_that_exist():
    """backend.rs:695-773 over layers Kv(2, 3), Rows(5), Kv(1, 4): buffers of
    rank < 2 (the rows layer's V) are skipped. Each buffer is stamped with
    its own constant, so the blob order and segment sizes are read off
    directly; block_bytes is the hand sum; import inverts export; a length
    mismatch is an error; copy_blocks moves every real buffer."""
    nb = 6
    shapes = [(nb, BS, 2, 3), (nb, BS, 1, 5), (nb, BS, 1, 4)]
    kc = [np.full(s, 10 + i, np.float32) for i, s in enumerate(shapes)]
    vc = [np.full(shapes[0], 20, np.float32), np.zeros((0,), np.float32),
          np.full(shapes[2], 22, np.float32)]
    segs = [(BS * 2 * 3, 10), (BS * 5, 11), (BS * 4, 12), (BS * 2 * 3, 20), (BS * 4, 22)]
    want_bytes = 4 * sum(n for n, _ in segs)
    assert oracle.cache_block_bytes(kc, vc) == want_bytes == 4 * (24 + 20 + 16 + 24 + 16)
    blob = np.frombuffer(oracle.export_block(kc, vc, 3), np.float32)
    assert blob.nbytes == want_bytes
    at = 0
    for n, stamp in segs:
        assert (blob[at:at + n] == stamp).all(), stamp
        at += n
    rng = np.random.default_rng(2)
    for p in kc + vc:
        p[...] = rng.standard_normal(p.shape)
    data = oracle.export_block(kc, vc, 1)
    k2 = [np.zeros_like(p) for p in kc]
    v2 = [np.zeros_like(p) for p in vc]
    oracle.import_block(k2, v2, 5, data)
    for a, b in zip(kc + vc, k2 + v2):
        if a.size:
            np.testing.assert_array_equal(a[1], b[5])
            assert np.count_nonzero(b[:5]) == 0
    with pytest.raises(ValueError):
        oracle.import_block(k2, v2, 0, data + b"\0" * 4)
    before = [p.copy() for p in kc + vc]
    oracle.copy_blocks(kc, vc, [(2, 0)])
    for a, b in zip(before, kc + vc):
        if a.size:
            np.testing.assert_array_equal(b[0], a[2])
            np.testing.assert_array_equal(b[1:], a[1:])


def test_threaded_scatter_and_copy_equal_the_serial_ones():
    """The CPU baseline's multi-threaded write_rows (scatter branch) and
    copy_blocks give the serial results for slot lists without repeats and
    pairs whose destinations are distinct and never a source."""
    rng = np.random.default_rng(11)
    row = 64
    slots = rng.permutation(4096)[:1500].astype(np.uint32)
    slots[::37] = 0xFFFFFFFF
    src = rng.integers(0, 255, size=(len(slots), row), dtype=np.uint8)
    a = np.zeros((4096, row), dtype=np.uint8)
    b = np.zeros_like(a)
    oracle.write_rows(a, src, slots)
    oracle.write_rows(b, src, slots, threads=4)
    assert np.array_equal(a, b)
    perm = rng.permutation(300).astype(np.uint32)
    pairs = np.stack([perm[:100], perm[100:200]], 1)
    ks = [rng.integers(0, 255, size=(300, 96), dtype=np.uint8) for _ in range(3)]
    vs = [x.copy() for x in ks]
    ks2, vs2 = [x.copy() for x in ks], [x.copy() for x in vs]
    oracle.copy_blocks(ks, vs, pairs)
    oracle.copy_blocks(ks2, vs2, pairs, threads=4)
    assert all(np.array_equal(x, y) for x, y in zip(ks + vs, ks2 + vs2))
    assert np.array_equal(ks[1][perm[100:200]], ks[1][perm[:100]])


@pytest.mark.parametrize("window", [None, 5])
def test_the_numpy_candle_path_matches_the_c_oracle(window):
    """oracle/candle_np.py (the candle CPU path with BLAS matmuls, the timed
    CPU baseline) against the C oracle on bf16-valued pools: decode rows,
    prefill chunks and an empty row, GQA 4:1, f32 rounding apart."""
    from oracle import candle_np
    rng = np.random.default_rng(11 + (window or 0))
    nb, bs, kvh, d, heads = 40, 16, 2, 32, 8
    bits = lambda *s: (rng.standard_normal(s).astype(np.float32).view(np.uint32) >> 16
                       ).astype(np.uint16)
    kb, vb = bits(nb, bs, kvh, d), bits(nb, bs, kvh, d)
    lens_q, lens_k = [1, 7, 0, 1, 20], [33, 60, 5, 1, 20]
    perm = rng.permutation(nb)
    tables, at = [], 0
    for lk in lens_k:
        n = -(-lk // bs)
        tables.append(perm[at:at + n].tolist())
        at += n
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.uint32)
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.uint32)
    qb = bits(int(cu_q[-1]), heads, d)
    got = candle_np.paged_attention(qb, kb, vb, cu_q, cu_k, tables, 0.3, window)
    f = candle_np.bf16_bits_to_f32
    want = oracle.paged_attention(f(qb), f(kb), f(vb), cu_q, cu_k, tables, 0.3, window)
    assert got.shape == want.shape
    assert np.abs(got - want).max() <= 1e-5
