"""A whole decode step captured in one HIP graph (append + paged attention per
layer), the way the reference's CUDA backend replays steps
(crates/vapi-backend-candle/src/backend.rs:893-1216): every entry point on the
step takes device pointers and sizes only, allocates nothing and uploads
nothing, so capture works. The graph is replayed several times with eager
work and synchronizations in between, and every replay is checked against
the eager step and the oracle.
"""
import numpy as np
import pytest
import torch

import oracle
from vapi_amd.attention import (ForwardBatch, PreparedAttention, paged_attention_append_prepared,
                                paged_attention_prepared)
from vapi_amd.cache import PagedKvCache, scatter_index, write_rows_indexed, write_kv_to_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("fused", [False, True], ids=["append-then-attention", "fused"])
def test_a_captured_decode_step_replays_like_the_eager_step(fused):
    """Per layer either the two calls or vapi_paged_attention_append."""
    rng = np.random.default_rng(33)
    L, nb, bs, hq, kvh, d = 2, 2048, 16, 32, 8, 128
    cache = PagedKvCache(L, nb, bs, kvh, d, torch.bfloat16)
    lens = rng.integers(40, 1500, size=24)
    perm = rng.permutation(nb)
    tables, at = [], 0
    for n in lens:
        tables.append(perm[at:at + -(-int(n) // bs)].tolist())
        at += len(tables[-1])
    # Context before the step: positions 0 .. len-2 of every sequence.
    ctx_slots = [t[p // bs] * bs + p % bs for t, n in zip(tables, lens) for p in range(n - 1)]
    for layer in range(L):
        k = torch.randn(len(ctx_slots), kvh, d, device=DEV).to(torch.bfloat16)
        write_kv_to_cache(cache, layer, k, k.flip(0), ctx_slots)
    # The step: one new token per sequence at position len-1.
    new_slots = [t[(n - 1) // bs] * bs + (n - 1) % bs for t, n in zip(tables, lens)]
    idx = scatter_index(new_slots, DEV)
    k_new = [torch.randn(len(lens), kvh, d, device=DEV).to(torch.bfloat16) for _ in range(L)]
    v_new = [torch.randn(len(lens), kvh, d, device=DEV).to(torch.bfloat16) for _ in range(L)]
    q = [torch.randn(len(lens), hq, d, device=DEV).to(torch.bfloat16) for _ in range(L)]
    batch = ForwardBatch(cu_seqlens_q=list(range(len(lens) + 1)),
                         cu_seqlens_k=np.concatenate([[0], np.cumsum(lens)]).tolist(),
                         block_tables=tables, max_seqlen_q=1, max_seqlen_k=int(lens.max()))
    prep = PreparedAttention.from_batch(batch, DEV)
    out = [torch.empty_like(x) for x in q]
    scale = d ** -0.5

    def step():
        for layer in range(L):
            if fused:
                paged_attention_append_prepared(q[layer], k_new[layer], v_new[layer], idx, cache,
                                                layer, prep, scale, out=out[layer])
            else:
                write_rows_indexed(cache, layer, k_new[layer], v_new[layer], idx)
                paged_attention_prepared(q[layer], cache, layer, prep, scale, out=out[layer])

    step()  # eager; also allocates the workspace outside the capture
    torch.cuda.synchronize()
    eager = [o.clone() for o in out]
    pool = cache._slab.clone()
    want = []
    for layer in range(L):
        kc = cache.reference_view(layer, "k").contiguous().float().cpu().numpy()
        vc = cache.reference_view(layer, "v").contiguous().float().cpu().numpy()
        w = oracle.paged_attention(q[layer].float().cpu().numpy(), kc, vc, batch.cu_seqlens_q,
                                   batch.cu_seqlens_k, tables, scale, threads=8)
        want.append(torch.from_numpy(w).to(torch.bfloat16).float())
        assert float((eager[layer].float().cpu() - want[layer]).abs().max()) <= \
            2e-2 * float(want[layer].abs().max())

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)

    for rep in range(4):
        for o in out:
            o.fill_(float("nan"))
        # Eager work between replays: another attention call on its own
        # workspace and unrelated torch kernels, then a full synchronization.
        other = PreparedAttention.from_batch(batch, DEV)
        paged_attention_prepared(q[0], cache, 0, other, scale)
        _ = (torch.randn(1 << 20, device=DEV) * 2).sum()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cache._slab, pool), f"replay {rep}: the pool changed"
        for layer in range(L):
            got = out[layer].float().cpu()
            assert not torch.isnan(got).any(), f"replay {rep} layer {layer}: rows not written"
            assert float((got - want[layer]).abs().max()) <= 2e-2 * float(want[layer].abs().max())
            # Same step, same inputs: only the split of the decode work (the
            # per-XCD shares move between calls) can change the f32 merge
            # order, so the replay stays within bf16 rounding of the eager step.
            assert float((got - eager[layer].float().cpu()).abs().max()) <= \
                2e-2 * float(want[layer].abs().max())


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 128),
                                     (torch.bfloat16, 256)], ids=["bf16-d128", "f32-d128", "bf16-d256"])
def test_a_captured_chunked_prefill_step_replays_like_the_eager_step(dtype, d):
    """A step of 20 decode rows and one 96-token prefill chunk per layer
    (append, then the prepared attention with the step's prefill list, the
    chunk's keys split over the GPU through the workspace), captured and
    replayed with eager work in between: every replay equals the oracle
    within the dtype's tolerance (f32: 1e-5) and leaves the pool as the
    eager step left it. The f32 pool runs the f32 decode stream and
    paged_prefill_f32; head_dim 256 the decode and prefill as two launches."""
    def close(got, want):
        if dtype == torch.float32:
            return float((got - want).abs().max()) <= 1e-5
        return float((got - want).abs().max()) <= 2e-2 * float(want.abs().max())

    rng = np.random.default_rng(34)
    L, nb, bs, hq, kvh = 2, 2048, 16, 32, 8
    cache = PagedKvCache(L, nb, bs, kvh, d, dtype)
    lens = np.concatenate([rng.integers(40, 1500, size=20), [900]])
    lens_q = [1] * 20 + [96]
    perm = rng.permutation(nb)
    tables, at = [], 0
    for n in lens:
        tables.append(perm[at:at + -(-int(n) // bs)].tolist())
        at += len(tables[-1])
    # Context before the step: every position before the step's new tokens.
    ctx = [t[p // bs] * bs + p % bs for t, n, lq in zip(tables, lens, lens_q)
           for p in range(n - lq)]
    for layer in range(L):
        k = torch.randn(len(ctx), kvh, d, device=DEV).to(dtype)
        write_kv_to_cache(cache, layer, k, k.flip(0), ctx)
    new_slots = [t[p // bs] * bs + p % bs for t, n, lq in zip(tables, lens, lens_q)
                 for p in range(n - lq, n)]
    idx = scatter_index(new_slots, DEV)
    nt = len(new_slots)
    k_new = [torch.randn(nt, kvh, d, device=DEV).to(dtype) for _ in range(L)]
    v_new = [torch.randn(nt, kvh, d, device=DEV).to(dtype) for _ in range(L)]
    q = [torch.randn(nt, hq, d, device=DEV).to(dtype) for _ in range(L)]
    batch = ForwardBatch(cu_seqlens_q=np.concatenate([[0], np.cumsum(lens_q)]).tolist(),
                         cu_seqlens_k=np.concatenate([[0], np.cumsum(lens)]).tolist(),
                         block_tables=tables, max_seqlen_q=96, max_seqlen_k=int(lens.max()))
    prep = PreparedAttention.from_batch(batch, DEV, cache=cache, num_heads=hq)
    assert prep.n_prefill == 1
    out = [torch.empty_like(x) for x in q]
    scale = d ** -0.5

    def step():
        for layer in range(L):
            write_rows_indexed(cache, layer, k_new[layer], v_new[layer], idx)
            paged_attention_prepared(q[layer], cache, layer, prep, scale, out=out[layer])

    step()
    torch.cuda.synchronize()
    pool = cache._slab.clone()
    want = []
    for layer in range(L):
        kc = cache.reference_view(layer, "k").contiguous().float().cpu().numpy()
        vc = cache.reference_view(layer, "v").contiguous().float().cpu().numpy()
        w = oracle.paged_attention(q[layer].float().cpu().numpy(), kc, vc, batch.cu_seqlens_q,
                                   batch.cu_seqlens_k, tables, scale, threads=8)
        want.append(torch.from_numpy(w).to(dtype).float())
        assert close(out[layer].float().cpu(), want[layer])

    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            step()
    torch.cuda.current_stream().wait_stream(side)
    for rep in range(4):
        for o in out:
            o.fill_(float("nan"))
        _ = (torch.randn(1 << 20, device=DEV) * 2).sum()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cache._slab, pool), f"replay {rep}: the pool changed"
        for layer in range(L):
            got = out[layer].float().cpu()
            assert not torch.isnan(got).any(), f"replay {rep} layer {layer}: rows not written"
            assert close(got, want[layer]), f"replay {rep} layer {layer}"
