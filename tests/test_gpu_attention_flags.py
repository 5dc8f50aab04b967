"""GPU checks of vapi_paged_attention_ex's flags and of the fused append's
bounded table read.

  * VAPI_ATTN_NO_DECODE_ROWS: a prefill-only batch runs the prefill kernel
    alone; deterministic (no key split) its output equals the call with a
    decode launch bit for bit (the decode kernel never writes a prefill
    row); split, and without a workspace, it matches the oracle.
    Forced onto a batch that does have
    decode rows, the prefill kernel takes them too: checked against the
    oracle (bf16 max-abs <= 2e-2 * max|reference|, as every attention test).
  * VAPI_ATTN_DETERMINISTIC: repeated calls on identical inputs are
    bit-identical, also after other batches moved the workspace's shares.
  * The fused append's per-row check reads the block table with the same
    column clamp as every other table read: a row whose len_k runs past its
    table row finishes, and pool and output equal the two-call sequence.
"""
import numpy as np
import pytest
import torch

from test_gpu_append_attention import clone, dev_slots
from test_gpu_attention import max_abs, oracle_out, random_case
from vapi_amd import _lib
from vapi_amd.attention import (ATTN_DETERMINISTIC, ATTN_NO_DECODE_ROWS, ForwardBatch,
                                PreparedAttention, paged_attention_append_prepared,
                                paged_attention_prepared)
from vapi_amd.cache import stream_handle, write_rows_indexed

pytestmark = pytest.mark.gpu
DEV = "cuda"


def call_ex(q, cache, prep, scale, flags, window_left=-1, ws=None):
    """vapi_paged_attention_ex straight through the C ABI with `flags`."""
    out = torch.full_like(q, float("nan"))
    b = prep.seqlens_q.shape[0] - 1
    max_q, max_k = max(prep.max_seqlen_q, 1), max(prep.max_seqlen_k, 1)
    need = _lib.lib().vapi_paged_attention_workspace_size(cache.pool, b, q.shape[1], max_q,
                                                          max_k)
    if ws is None and not (flags & ATTN_NO_DECODE_ROWS):
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=DEV)
    _lib.check(_lib.lib().vapi_paged_attention_ex(
        cache.pool, 0, q.data_ptr(), out.data_ptr(), prep.seqlens_q.data_ptr(),
        prep.seqlens_k.data_ptr(), prep.block_table.data_ptr(), b, prep.block_table.shape[1],
        max_q, max_k, q.shape[1], float(scale), window_left, 0, flags,
        ws.data_ptr() if ws is not None else None, need if ws is not None else 0,
        stream_handle()))
    return out


@pytest.mark.parametrize("heads,kvh,d,window", [(32, 8, 128, None), (16, 2, 64, 40),
                                                (8, 8, 128, None)])
def test_a_prefill_only_batch_runs_one_kernel_with_the_same_output(heads, kvh, d, window):
    rng = np.random.default_rng(heads * 131 + d)
    c, q, batch = random_case(rng, torch.bfloat16, heads, kvh, d, 16, [37, 64, 5, 2],
                              [300, 700, 40, 2], "HND")
    prep = PreparedAttention.from_batch(batch, DEV)
    assert prep.flags == ATTN_NO_DECODE_ROWS
    scale = d ** -0.5
    wl = -1 if window is None else window - 1
    b = prep.seqlens_q.shape[0] - 1
    need = _lib.lib().vapi_paged_attention_workspace_size(
        c.pool, b, q.shape[1], max(prep.max_seqlen_q, 1), max(prep.max_seqlen_k, 1))
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=DEV)
    one = call_ex(q, c, prep, scale, ATTN_NO_DECODE_ROWS, wl, ws=ws)
    two = call_ex(q, c, prep, scale, 0, wl)
    bare = call_ex(q, c, prep, scale, ATTN_NO_DECODE_ROWS, wl)  # no workspace at all
    # Unsplit (deterministic) the two launch shapes give every row the same
    # key order, so the same bits; split, each is within the tolerance.
    one_d = call_ex(q, c, prep, scale, ATTN_NO_DECODE_ROWS | ATTN_DETERMINISTIC, wl, ws=ws)
    two_d = call_ex(q, c, prep, scale, ATTN_DETERMINISTIC, wl)
    torch.cuda.synchronize()
    assert torch.equal(one_d, two_d)
    want = oracle_out(q, c, 0, batch, scale, window)
    for got in (one, two, bare, one_d):
        assert max_abs(got, want) <= 2e-2 * float(want.abs().max())


@pytest.mark.parametrize("dtype,heads,kvh,d", [(torch.bfloat16, 32, 8, 128),
                                                (torch.bfloat16, 16, 2, 64),
                                                (torch.float32, 32, 8, 128),
                                                (torch.float32, 16, 2, 64)])
def test_a_wrong_no_decode_hint_still_gives_every_row(dtype, heads, kvh, d):
    """Decode rows under VAPI_ATTN_NO_DECODE_ROWS go to the prefill kernel
    (f32 pools: paged_prefill_f32, within 1e-5)."""
    rng = np.random.default_rng(heads + d)
    c, q, batch = random_case(rng, dtype, heads, kvh, d, 16, [1, 19, 1, 3, 1],
                              [900, 300, 1, 40, 2049], "NHD")
    prep = PreparedAttention.from_batch(batch, DEV)
    assert prep.flags == 0
    got = call_ex(q, c, prep, d ** -0.5, ATTN_NO_DECODE_ROWS)
    want = oracle_out(q, c, 0, batch, d ** -0.5)
    if dtype == torch.float32:
        assert max_abs(got, want) <= 1e-5
    else:
        assert max_abs(got, want) <= 2e-2 * float(want.abs().max())


def test_deterministic_decode_is_bit_identical_across_calls():
    rng = np.random.default_rng(64)
    lens_k = np.clip(np.exp(rng.normal(np.log(1500), 0.75, 64)), 64, 6000).astype(int).tolist()
    c, q, batch = random_case(rng, torch.bfloat16, 32, 8, 128, 16, [1] * 64, lens_k, "HND")
    _, q2, other = random_case(np.random.default_rng(3), torch.bfloat16, 32, 8, 128, 16,
                               [1] * 7, [5000, 20, 3000, 1, 800, 4000, 64], "HND",
                               nb=c.num_blocks)
    prep = PreparedAttention.from_batch(batch, DEV, deterministic=True)
    assert prep.flags == ATTN_DETERMINISTIC
    adaptive = PreparedAttention.from_batch(other, DEV)
    scale = 128 ** -0.5
    first = paged_attention_prepared(q, c, 0, prep, scale).clone()
    outs = []
    for _ in range(3):
        # Other work on the same workspace moves the adaptive shares.
        adaptive.workspace = prep.workspace
        for _ in range(3):
            paged_attention_prepared(q2, c, 0, adaptive, scale)
        outs.append(paged_attention_prepared(q, c, 0, prep, scale).clone())
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o, first)
    want = oracle_out(q, c, 0, batch, scale)
    assert max_abs(first, want) <= 2e-2 * float(want.abs().max())


def test_fused_append_with_len_k_past_the_table_stays_in_bounds():
    """ForwardBatch::validate refuses such a batch on the host; on the device
    the fused path's table read is clamped like the others, so the call
    finishes and matches the two-call sequence on the same inputs."""
    rng = np.random.default_rng(77)
    c, q, batch = random_case(rng, torch.bfloat16, 32, 8, 128, 16, [1, 1, 1],
                              [300, 33, 700], "HND")
    # Row 1 claims 1,000 keys over a 3-block table row; the packed table is
    # 44 columns wide (700 keys), so its new key's column (62) is past the row.
    over = ForwardBatch(cu_seqlens_q=batch.cu_seqlens_q, cu_seqlens_k=[0, 300, 1300, 2000],
                        block_tables=batch.block_tables, max_seqlen_q=1, max_seqlen_k=1000)
    k_new = torch.randn(3, 8, 128, device=DEV).to(torch.bfloat16)
    v_new = torch.randn_like(k_new)
    # Row 1's new row goes to a block no table names: the fused path's
    # contract is that no row reads a slot the call writes other than its own
    # new key, and row 1's over-long keys re-read its padded last entry.
    spare = sorted(set(range(c.num_blocks)) - {b for t in batch.block_tables for b in t})[0]
    slots = [batch.block_tables[0][299 // 16] * 16 + 299 % 16,
             spare * 16 + 5,
             batch.block_tables[2][699 // 16] * 16 + 699 % 16]
    s = dev_slots(slots)
    scale = 128 ** -0.5
    c2 = clone(c)
    write_rows_indexed(c2, 0, k_new, v_new, s)
    out2 = paged_attention_prepared(q, c2, 0, PreparedAttention.from_batch(over, DEV), scale)
    c1 = clone(c)
    out1 = paged_attention_append_prepared(q, k_new, v_new, s, c1, 0,
                                           PreparedAttention.from_batch(over, DEV), scale)
    torch.cuda.synchronize()
    assert torch.equal(c1._slab, c2._slab)
    assert bool(torch.isfinite(out1.float()).all())
    assert torch.equal(out1, out2)


def call_prepared(q, cache, prep, scale, flags, seqs, window_left=-1):
    """vapi_paged_attention_prepared straight through the C ABI with the
    prefill sequence list `seqs` (host ints), its workspace sized by
    vapi_paged_attention_prepared_workspace_size."""
    out = torch.full_like(q, float("nan"))
    b = prep.seqlens_q.shape[0] - 1
    max_q, max_k = max(prep.max_seqlen_q, 1), max(prep.max_seqlen_k, 1)
    L = _lib.lib()
    need = L.vapi_paged_attention_prepared_workspace_size(cache.pool, b, len(seqs), q.shape[1],
                                                          max_q, max_k)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=DEV)
    dseqs = torch.tensor(list(seqs) or [0], dtype=torch.int32, device=DEV)
    _lib.check(L.vapi_paged_attention_prepared(
        cache.pool, 0, q.data_ptr(), out.data_ptr(), prep.seqlens_q.data_ptr(),
        prep.seqlens_k.data_ptr(), prep.block_table.data_ptr(), b, prep.block_table.shape[1],
        max_q, max_k, q.shape[1], float(scale), window_left, 0, flags, dseqs.data_ptr(),
        len(seqs), ws.data_ptr(), need, stream_handle()))
    return out


@pytest.mark.parametrize("d,window", [(128, None), (128, 300), (64, None)])
def test_a_chunked_prefill_step_with_its_prefill_list_matches_the_oracle(d, window):
    """A serving step of many decode rows and two prefill chunks: the prefill
    grid covers the two chunks only (and splits their keys over the GPU);
    the output matches the oracle, as does the same call without the list."""
    rng = np.random.default_rng(d + (window or 0))
    n_dec = 40
    lens_q = [1] * 20 + [256] + [1] * 20 + [100]
    lens_k = [int(x) for x in rng.integers(50, 3000, 20)] + [1024] + \
             [int(x) for x in rng.integers(50, 3000, 20)] + [100]
    c, q, batch = random_case(rng, torch.bfloat16, 32, 8, d, 16, lens_q, lens_k, "HND")
    prep = PreparedAttention.from_batch(batch, DEV)
    assert prep.n_prefill == 2 and prep.flags == 0
    assert prep.prefill_seqs.cpu().tolist() == [20, 41]
    scale = d ** -0.5
    wl = -1 if window is None else window - 1
    want = oracle_out(q, c, 0, batch, scale, window)  # the oracle takes the window w itself
    tol = 2e-2 * float(want.abs().max())
    listed = call_prepared(q, c, prep, scale, 0, [20, 41], wl)
    assert max_abs(listed, want) <= tol
    assert max_abs(call_ex(q, c, prep, scale, 0, wl), want) <= tol
    # The Python wrapper takes the same path.
    out = paged_attention_prepared(q, c, 0, prep, scale, None if window is None else wl)
    assert max_abs(out, want) <= tol
    assert n_dec + 2 == len(lens_q)


def test_a_prefill_only_call_ignores_the_prefill_list():
    """With VAPI_ATTN_NO_DECODE_ROWS the call covers every sequence whatever
    the list names (here: none of them)."""
    rng = np.random.default_rng(77)
    c, q, batch = random_case(rng, torch.bfloat16, 32, 8, 128, 16, [40, 9], [500, 60], "HND")
    prep = PreparedAttention.from_batch(batch, DEV)
    scale = 128 ** -0.5
    want = oracle_out(q, c, 0, batch, scale)
    out = call_prepared(q, c, prep, scale, ATTN_NO_DECODE_ROWS, [])
    assert max_abs(out, want) <= 2e-2 * float(want.abs().max())


def test_config2_mixed_step_matches_the_oracle():
    """Config 2's pool and sequences as a chunked-prefill step: its first 63
    sequences decoding, the 64th a 512-token chunk at positions 1536..2047
    over its own blocks, through PreparedAttention (the prepared call with
    the prefill list, the chunk's keys split over the GPU); every decode row
    and 16-row samples of the chunk against the oracle."""
    from vapi_amd import workload
    from vapi_amd.cache import PagedKvCache
    import oracle
    from test_gpu_attention import host_f32
    w = workload.config2_decode()
    c = PagedKvCache(1, w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim, torch.bfloat16,
                     "HND")
    workload.fill_normal(c._slab, workload.seed_for(2))
    nd = 63
    lens_q = [1] * nd + [512]
    lens_k = [int(x) for x in w.lens[:nd]] + [2048]
    tables = [t.tolist() for t in w.tables[:nd]] + [w.tables[nd].tolist()[:128]]
    if len(tables[nd]) < 128:
        used = set(x for t in tables for x in t)
        tables[nd] = [x for x in range(w.num_blocks) if x not in used][:128]
    batch = ForwardBatch(cu_seqlens_q=np.concatenate([[0], np.cumsum(lens_q)]).tolist(),
                         cu_seqlens_k=np.concatenate([[0], np.cumsum(lens_k)]).tolist(),
                         block_tables=tables, max_seqlen_q=512, max_seqlen_k=max(lens_k))
    g = torch.Generator(device=DEV).manual_seed(63)
    q = torch.randn(sum(lens_q), w.num_heads, w.head_dim, generator=g, device=DEV).to(
        torch.bfloat16)
    prep = PreparedAttention.from_batch(batch, DEV)
    assert prep.n_prefill == 1 and prep.prefill_seqs.cpu().tolist() == [nd]
    scale = w.head_dim ** -0.5
    got = paged_attention_prepared(q, c, 0, prep, scale)
    torch.cuda.synchronize()
    kc = host_f32(c.reference_view(0, "k").contiguous())
    vc = host_f32(c.reference_view(0, "v").contiguous())
    dec = oracle.paged_attention(host_f32(q[:nd]), kc, vc, list(range(nd + 1)),
                                 batch.cu_seqlens_k[:nd + 1], tables[:nd], scale, threads=8)
    dec = torch.from_numpy(dec).to(torch.bfloat16).float()
    assert max_abs(got[:nd], dec) <= 2e-2 * float(dec.abs().max())
    for j0 in (0, 200, 496):
        rows = q[nd + j0: nd + j0 + 16]
        want = oracle.paged_attention(host_f32(rows), kc, vc, [0, 16], [0, 2048 - 512 + j0 + 16],
                                      [tables[nd]], scale, threads=8)
        want = torch.from_numpy(want).to(torch.bfloat16).float()
        assert max_abs(got[nd + j0: nd + j0 + 16], want) <= 2e-2 * float(want.abs().max()), j0


def test_prefill_key_split_adds_no_error_beyond_the_unsplit_call():
    """The key split keeps each split's partial (m, l, o / l) in f32, so the
    split call's error against the oracle stays within 1.5x the unsplit
    (deterministic, no split) call's on the same inputs."""
    rng = np.random.default_rng(77)
    c, q, batch = random_case(rng, torch.bfloat16, 32, 8, 128, 16, [512], [4096], "HND")
    prep = PreparedAttention.from_batch(batch, DEV)
    scale = 128 ** -0.5
    b = 1
    need = _lib.lib().vapi_paged_attention_workspace_size(c.pool, b, 32, 512, 4096)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=DEV)
    split = call_ex(q, c, prep, scale, ATTN_NO_DECODE_ROWS, ws=ws)
    unsplit = call_ex(q, c, prep, scale, ATTN_NO_DECODE_ROWS | ATTN_DETERMINISTIC, ws=ws)
    torch.cuda.synchronize()
    # oracle at f32, not rounded to bf16, so the two calls' own errors show
    kc = c.reference_view(0, "k").contiguous().float().cpu().numpy()
    vc = c.reference_view(0, "v").contiguous().float().cpu().numpy()
    import oracle
    ref = torch.from_numpy(oracle.paged_attention(q.float().cpu().numpy(), kc, vc,
                                                  batch.cu_seqlens_q, batch.cu_seqlens_k,
                                                  batch.block_tables, scale, threads=8))
    e_split, e_unsplit = max_abs(split, ref), max_abs(unsplit, ref)
    print(f"prefill 1 x 512 over 4096 keys, max-abs vs f32 oracle: split {e_split:.3e}, "
          f"unsplit {e_unsplit:.3e}")
    assert not torch.equal(split, unsplit)  # the split did run
    assert e_split <= 1.5 * e_unsplit, (e_split, e_unsplit)


def test_valu_context_past_max_seqlen_k_stays_inside_its_workspace():
    """An f32 pool with head_dim 82 (not a multiple of 4: the VALU kernel) whose device len_k exceeds the
    max_seqlen_k the call was sized for: the key chunks stop at the launch's
    last chunk (ceil(max_k / c) * c keys, 1,024 here for every chunk size c
    the kernel picks), so neither kernel touches memory past the workspace,
    and the row is the attention over those keys."""
    rng = np.random.default_rng(5)
    lens_k = [3000, 700]
    c, q, batch = random_case(rng, torch.float32, 8, 2, 82, 16, [1, 1], lens_k, "HND")
    prep = PreparedAttention.from_batch(batch, DEV)
    lib = _lib.lib()
    max_k = 1000  # smaller than sequence 0's 3,000 keys
    need = lib.vapi_paged_attention_workspace_size(c.pool, 2, 8, 1, max_k)
    guard = 1 << 16
    ws = torch.full((need + guard,), 0xAB, dtype=torch.uint8, device=DEV)
    ws[:need].zero_()
    out = torch.full_like(q, float("nan"))
    _lib.check(lib.vapi_paged_attention_ex(
        c.pool, 0, q.data_ptr(), out.data_ptr(), prep.seqlens_q.data_ptr(),
        prep.seqlens_k.data_ptr(), prep.block_table.data_ptr(), 2, prep.block_table.shape[1],
        1, max_k, 8, 82 ** -0.5, -1, 0, 0, ws.data_ptr(), need, stream_handle()))
    torch.cuda.synchronize()
    assert bool((ws[need:] == 0xAB).all()), "the call wrote past its workspace"
    trunc = ForwardBatch(cu_seqlens_q=[0, 1, 2], cu_seqlens_k=[0, 1024, 1024 + 700],
                         block_tables=[batch.block_tables[0][:64], batch.block_tables[1]],
                         max_seqlen_q=1, max_seqlen_k=1024)
    want = oracle_out(q, c, 0, trunc, 82 ** -0.5)
    assert max_abs(out[:1], want[:1]) <= 1e-5
    # sequence 1 fits its 1,000-key bound: ordinary attention
    full = oracle_out(q, c, 0, batch, 82 ** -0.5)
    assert max_abs(out[1:], full[1:]) <= 1e-5
