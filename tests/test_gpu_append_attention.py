"""GPU parity of vapi_paged_attention_append: one layer's cache write and
attention in one call, against the two calls it fuses (vapi_kv_append, then
vapi_paged_attention; the pair of models/qwen.rs:371-391).

Both runs start from copies of one pool and from fresh (zeroed) workspaces,
so the decode splits its work at the same points: the pools after the call
must be equal bit for bit (data movement) and so must the outputs (the same
kernels read the same key bytes, from the new rows instead of the pool).
The fused output is also checked against the oracle over the written pool:
bf16/f16 max-abs <= 2e-2 * max|reference|, as for vapi_paged_attention.
"""
import zlib

import numpy as np
import pytest
import torch

from test_gpu_attention import max_abs, oracle_out, random_case
from vapi_amd import _lib, workload
from vapi_amd.attention import (ForwardBatch, PreparedAttention,
                                paged_attention_append_prepared, paged_attention_prepared)
from vapi_amd.cache import PagedKvCache, write_rows_indexed

pytestmark = pytest.mark.gpu
DEV = "cuda"
SKIP = _lib.SLOT_SKIP


def clone(c: PagedKvCache) -> PagedKvCache:
    d = PagedKvCache(c.num_layers, c.num_blocks, c.block_size, c.num_kv_heads, c.head_dim,
                     c.dtype, c.layout, block_major=c.block_major)
    d._slab.copy_(c._slab)
    return d


def step_slots(batch: ForwardBatch, bs: int):
    """The scheduler's slot of every new token (scheduler.rs:525-565): token
    j of a row sits at position len_k - len_q + j of the row's blocks."""
    out = []
    for i, table in enumerate(batch.block_tables):
        lq = batch.cu_seqlens_q[i + 1] - batch.cu_seqlens_q[i]
        lk = batch.cu_seqlens_k[i + 1] - batch.cu_seqlens_k[i]
        for p in range(lk - lq, lk):
            out.append(table[p // bs] * bs + p % bs)
    return out


def dev_slots(values):
    return torch.from_numpy(np.asarray(values, dtype=np.uint32).view(np.int32)).to(DEV)


def both_ways(c, q, batch, k_new, v_new, slots, scale, window=None):
    """(pool, out) of the two-call sequence and of the fused call; a sliding
    window w hides keys w or more behind the query (window_left = w - 1)."""
    s = dev_slots(slots)
    window = None if window is None else window - 1
    c2 = clone(c)
    write_rows_indexed(c2, 0, k_new, v_new, s)
    out2 = paged_attention_prepared(q, c2, 0, PreparedAttention.from_batch(batch, DEV), scale,
                                    window)
    c1 = clone(c)
    out1 = paged_attention_append_prepared(q, k_new, v_new, s, c1, 0,
                                           PreparedAttention.from_batch(batch, DEV), scale,
                                           window)
    torch.cuda.synchronize()
    return c2, out2, c1, out1


def check_step(c, q, batch, k_new, v_new, slots, window=None, same_splits=True):
    scale = c.head_dim ** -0.5
    c2, out2, c1, out1 = both_ways(c, q, batch, k_new, v_new, slots, scale, window)
    assert torch.equal(c1._slab, c2._slab), "pools differ"
    if same_splits:
        assert torch.equal(out1, out2), max_abs(out1, out2)
    want = oracle_out(q, c1, 0, batch, scale, window)
    assert max_abs(out1, want) <= 2e-2 * float(want.abs().max())
    assert max_abs(out2, want) <= 2e-2 * float(want.abs().max())


def new_rows(n, kvh, d, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = torch.randn(n, kvh, d, generator=g, device=DEV).to(dtype)
    v = torch.randn(n, kvh, d, generator=g, device=DEV).to(dtype)
    return k, v


STEPS = [
    # dtype, heads, kvh, d, bs, lens_q, lens_k, window, layout
    (torch.bfloat16, 32, 8, 128, 16, [1, 1, 1, 1, 1], [1, 17, 600, 1500, 33], None, "HND"),
    (torch.float16, 16, 8, 128, 32, [1, 1, 1], [1100, 40, 513], 100, "HND"),
    (torch.bfloat16, 8, 8, 64, 16, [1, 1], [900, 100], None, "NHD"),
    (torch.bfloat16, 64, 4, 64, 32, [1, 1, 1], [70, 64, 2], 9, "NHD"),
    (torch.bfloat16, 16, 4, 256, 16, [1, 1, 1], [900, 31, 2], None, "HND"),
    (torch.float16, 8, 2, 256, 32, [1, 1], [64, 1300], 50, "NHD"),
    (torch.bfloat16, 32, 8, 128, 16, [1, 1, 1], [900, 31, 2], None, "HND-bm"),
    # Prefill rows in the batch: the two calls run inside.
    (torch.bfloat16, 32, 8, 128, 16, [1, 37, 1], [700, 37, 33], None, "HND"),
    (torch.float32, 16, 8, 128, 16, [1, 1], [64, 512], None, "HND"),
]


@pytest.mark.parametrize("case", STEPS, ids=lambda c: f"{str(c[0])[6:]}-h{c[1]}-kv{c[2]}-d{c[3]}-bs{c[4]}-q{max(c[5])}-w{c[7]}-{c[8]}")
def test_fused_step_equals_append_then_attention(case):
    dtype, heads, kvh, d, bs, lens_q, lens_k, window, layout = case
    rng = np.random.default_rng(zlib.crc32(str(case).encode()))
    c, q, batch = random_case(rng, dtype, heads, kvh, d, bs, lens_q, lens_k, layout)
    k_new, v_new = new_rows(sum(lens_q), kvh, d, dtype, int(rng.integers(1 << 30)))
    check_step(c, q, batch, k_new, v_new, step_slots(batch, bs), window)


def test_rows_whose_slot_is_not_their_last_position_read_the_pool():
    """A skipped token (VAPI_KV_SLOT_SKIP), a token sent to an unused block
    and padded tokens past the batch's rows: those rows read the pool's own
    bytes at len_k - 1, as the two calls would, and the writes land as
    vapi_kv_append's."""
    rng = np.random.default_rng(77)
    lens_k = [300, 45, 1, 128, 700]
    c, q, batch = random_case(rng, torch.bfloat16, 32, 8, 128, 16, [1] * 5, lens_k, "HND",
                              nb=sum(-(-l // 16) for l in lens_k) + 8)
    used = {b for t in batch.block_tables for b in t}
    free = [b for b in range(c.num_blocks) if b not in used]
    slots = step_slots(batch, 16)
    slots[1] = SKIP
    slots[3] = free[0] * 16 + 5
    slots += [SKIP, free[1] * 16]  # two padded tokens
    k_new, v_new = new_rows(len(slots), 8, 128, torch.bfloat16, 78)
    check_step(c, q, batch, k_new, v_new, slots)


def test_config2_fused_decode_step():
    """BASELINE config 2's decode batch (64 rows, log-normal contexts) with
    its new tokens appended in the same call."""
    w = workload.config2_decode()
    c = PagedKvCache(1, w.num_blocks, w.block_size, 8, 128, torch.bfloat16)
    workload.fill_normal(c._slab, workload.seed_for(2))
    batch = ForwardBatch(cu_seqlens_q=list(range(len(w.lens) + 1)),
                         cu_seqlens_k=np.concatenate([[0], np.cumsum(w.lens)]).tolist(),
                         block_tables=[list(map(int, t)) for t in w.tables], max_seqlen_q=1,
                         max_seqlen_k=int(max(w.lens)))
    q = torch.randn(len(w.lens), 32, 128, device=DEV).to(torch.bfloat16)
    k_new, v_new = new_rows(len(w.lens), 8, 128, torch.bfloat16, 2)
    check_step(c, q, batch, k_new, v_new, step_slots(batch, 16))


def test_fused_step_over_more_rows_than_one_launch_plans_for():
    """5,000 decode rows: the host splits the decode into launches of at most
    4,096 rows; the new rows are written once, by the first launch pair. The
    second launch splits its work by shares the first one measured (wave
    timings), so the two runs' outputs agree to the tolerance, not bit for
    bit."""
    rng = np.random.default_rng(5001)
    lens_k = rng.integers(1, 80, size=5000).tolist()
    c, q, batch = random_case(rng, torch.bfloat16, 8, 2, 128, 16, [1] * 5000, lens_k, "HND")
    k_new, v_new = new_rows(5000, 2, 128, torch.bfloat16, 5002)
    check_step(c, q, batch, k_new, v_new, step_slots(batch, 16), same_splits=False)
