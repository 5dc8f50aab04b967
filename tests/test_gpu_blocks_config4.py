"""GPU parity of BASELINE config 4 at its own workload (Qwen2.5-7B KV shape:
28 layers, 4 kv heads, head_dim 128, block_size 16, bf16, 40,000-block pool,
36.7 GB), bit-exact against the oracle:

  (a) copy-on-write: vapi_kv_copy_blocks with the config's 2,048 seeded
      (src, dst) pairs in one call (2,048 x 28 x 2 runs of 16 KiB: 117 M
      16-byte items in one 32-bit-indexed launch). Every touched block is
      checked against oracle.copy_blocks run on host copies of just the
      pairs' blocks (renumbered densely), and a sample of untouched blocks
      must be unchanged.
  (b) spill swap: the 4,096 swap_ids out to pinned host memory through a
      256-block device staging buffer (16 staging rounds of 235 MB), on a
      side stream, while one config-2 decode runs on the main stream; every
      blob against oracle.export_block (the reference's byte order,
      backend.rs:718-734), the decode against the oracle; then the blobs
      back into the swap_in_ids, every block bit-exact.

Reference: crates/vapi-backend-candle/src/backend.rs:695-797.
"""
import numpy as np
import pytest
import torch

import oracle
from test_gpu_attention import max_abs
from vapi_amd import workload
from vapi_amd.attention import ForwardBatch, PreparedAttention, paged_attention_prepared
from vapi_amd.backend import KvBlockBackend
from vapi_amd.cache import PagedKvCache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def say(msg):
    print(f"[config4] {msg}", flush=True)


@pytest.fixture(scope="module", params=[False, True], ids=["layer-major", "block-major"])
def cfg4(request):
    w = workload.config4_block_ops()
    say(f"pool: {w.num_layers} layers x {w.num_blocks} blocks, bf16, "
        f"block_major={request.param}")
    c = PagedKvCache(w.num_layers, w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim,
                     torch.bfloat16, "HND", block_major=request.param)
    workload.fill_normal(c._slab, workload.seed_for(4))
    torch.cuda.synchronize()
    yield w, c
    del c
    torch.cuda.empty_cache()


def host_blocks(c: PagedKvCache, ids):
    """Per-layer host copies [n, bs, kvh, d] (raw 16-bit) of blocks `ids`, in
    the reference layout, K layers and V layers."""
    idx = torch.from_numpy(np.asarray(ids, dtype=np.int64)).to(DEV)
    ks, vs = [], []
    for l in range(c.num_layers):
        for which, out in (("k", ks), ("v", vs)):
            t = c.reference_view(l, which)[idx].contiguous().view(torch.int16).cpu()
            out.append(t.numpy().view(np.uint16))
    return ks, vs


def test_config4_copy_on_write_full_size_matches_the_oracle(cfg4):
    w, c = cfg4
    pairs = w.pairs.astype(np.int64)
    n = pairs.shape[0]
    assert n == 2048 and len(np.unique(pairs)) == 2 * n
    blocks = np.unique(pairs.reshape(-1))
    dense = {int(b): i for i, b in enumerate(blocks)}
    dpairs = np.array([[dense[int(s)], dense[int(d)]] for s, d in pairs], dtype=np.uint32)
    say(f"copy: host copy of {len(blocks)} blocks before")
    ks, vs = host_blocks(c, blocks)
    rng = np.random.default_rng(4)
    others = rng.choice(np.setdiff1d(np.arange(w.num_blocks), blocks), 256, replace=False)
    ko, vo = host_blocks(c, others)
    oracle.copy_blocks(ks, vs, dpairs)
    say("copy: one vapi_kv_copy_blocks call, 2,048 pairs x 28 layers x K/V")
    KvBlockBackend(c).copy_blocks(pairs.tolist())
    torch.cuda.synchronize()
    gk, gv = host_blocks(c, blocks)
    for l in range(c.num_layers):
        np.testing.assert_array_equal(gk[l], ks[l], err_msg=f"K layer {l}")
        np.testing.assert_array_equal(gv[l], vs[l], err_msg=f"V layer {l}")
    gko, gvo = host_blocks(c, others)
    for l in range(c.num_layers):
        np.testing.assert_array_equal(gko[l], ko[l])
        np.testing.assert_array_equal(gvo[l], vo[l])


def decode_setup():
    d = workload.config2_decode()
    cache = PagedKvCache(1, d.num_blocks, d.block_size, d.num_kv_heads, d.head_dim,
                         torch.bfloat16, "HND")
    workload.fill_normal(cache._slab, workload.seed_for(2))
    g = torch.Generator(device=DEV).manual_seed(44)
    q = torch.randn(d.batch, d.num_heads, d.head_dim, generator=g, device=DEV).to(torch.bfloat16)
    batch = ForwardBatch(cu_seqlens_q=d.cu_q().tolist(), cu_seqlens_k=d.cu_k().tolist(),
                         block_tables=[t.tolist() for t in d.tables], max_seqlen_q=1,
                         max_seqlen_k=int(d.lens.max()))
    return d, cache, q, batch


def test_config4_swap_full_size_round_trips_bit_exact_beside_a_decode(cfg4):
    w, c = cfg4
    be = KvBlockBackend(c)
    bb = be.block_bytes()
    n = len(w.swap_ids)
    assert n == 4096 and bb == 917504
    d, dcache, q, batch = decode_setup()
    prep = PreparedAttention.from_batch(batch, DEV)
    scale = d.head_dim ** -0.5
    host = torch.empty(n * bb, dtype=torch.uint8, pin_memory=True)
    staging = torch.empty(256 * bb, dtype=torch.uint8, device=DEV)
    ids_out = torch.from_numpy(w.swap_ids.astype(np.int32)).to(DEV)
    ids_in = torch.from_numpy(w.swap_in_ids.astype(np.int32)).to(DEV)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    say("swap out: 4,096 blocks through 256-block staging on a side stream, decode beside it")
    side.wait_stream(torch.cuda.current_stream())
    be.swap_out(ids_out, host, staging, stream=side)
    out = paged_attention_prepared(q, dcache, 0, prep, scale)
    torch.cuda.synchronize()
    say("swap out: checking every blob against oracle.export_block")
    ks, vs = host_blocks(c, w.swap_ids)
    blobs = host.numpy()
    for i in range(n):
        want = np.frombuffer(oracle.export_block(ks, vs, i), dtype=np.uint8)
        got = blobs[i * bb:(i + 1) * bb]
        if not np.array_equal(got, want):
            raise AssertionError(f"blob {i} (block {int(w.swap_ids[i])}) differs")
    say("decode during the swap: checking against the oracle")
    kc = dcache.reference_view(0, "k").contiguous().float().cpu().numpy()
    vc = dcache.reference_view(0, "v").contiguous().float().cpu().numpy()
    want = oracle.paged_attention(q.float().cpu().numpy(), kc, vc, batch.cu_seqlens_q,
                                  batch.cu_seqlens_k, batch.block_tables, scale, threads=8)
    want = torch.from_numpy(want).to(torch.bfloat16).float()
    assert max_abs(out, want) <= 2e-2 * float(want.abs().max())
    del kc, vc, dcache
    say("swap in: 4,096 blobs into other blocks")
    be.swap_in(ids_in, host, staging, stream=side)
    side.synchronize()
    gk, gv = host_blocks(c, w.swap_in_ids)
    for l in range(c.num_layers):
        np.testing.assert_array_equal(gk[l], ks[l], err_msg=f"K layer {l}")
        np.testing.assert_array_equal(gv[l], vs[l], err_msg=f"V layer {l}")
