"""GPU parity of vapi_paged_attention against the oracle.

Tolerances (written here, per dtype):
  f32:  max-abs <= 1e-5 against the f32 oracle (the reference's own CPU bar,
        attention.rs:400-404).
  bf16: max-abs <= 2e-2 * max|reference| (relative) and the reference's own
        CUDA-vs-CPU bound max-abs < 1e-2 on its test shapes (attention.rs:661-664).
  f16:  max-abs < 1e-3 on the reference's test shape (attention.rs:666-669).
The oracle output is cast to the input dtype before comparing, as
paged_attention_cpu does (attention.rs:162).
"""
import zlib

import numpy as np
import pytest
import torch

import oracle
from vapi_amd import _lib, workload
from vapi_amd.attention import (ForwardBatch, PreparedAttention, paged_attention,
                                paged_attention_prepared, paged_attention_windowed)
from vapi_amd.cache import PagedKvCache, stream_handle, write_kv_to_cache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def host_f32(t):
    return t.detach().float().cpu().numpy()


def oracle_out(q, cache, layer, batch: ForwardBatch, scale, window=None, wr=0):
    kc = host_f32(cache.reference_view(layer, "k").contiguous())
    vc = host_f32(cache.reference_view(layer, "v").contiguous())
    out = oracle.paged_attention(host_f32(q), kc, vc, batch.cu_seqlens_q, batch.cu_seqlens_k,
                                 batch.block_tables, scale, window, wr, threads=8)
    return torch.from_numpy(out).to(q.dtype).float()


def max_abs(a, b):
    return float((a.float().cpu() - b.float().cpu()).abs().max())


# ---- the reference's CUDA tests (attention.rs:441-714), same shapes ----------

HEADS, KV_HEADS, HEAD_DIM, BLOCK = 4, 2, 64, 32


def ref_rows(n, seed, heads, d, dtype, mul):
    i = torch.arange(n * heads * d, dtype=torch.float32)
    data = (torch.sin(i * mul + seed) if mul == 0.173 else torch.cos(i * mul + seed)) * 0.5
    return data.reshape(n, heads, d).to(dtype).to(DEV)


def slots(table, positions, bs=BLOCK):
    return [table[p // bs] * bs + p % bs for p in positions]


def mixed(dtype, layout="HND"):
    """attention.rs:476-514: A = 70 cached + 20-token chunk, B = decode over 40."""
    c = PagedKvCache(1, 8, BLOCK, KV_HEADS, HEAD_DIM, dtype, layout)
    ta, tb = [5, 1, 6], [7, 2]
    len_a, chunk_a, len_b = 90, 20, 40
    write_kv_to_cache(c, 0, ref_rows(len_a, 0.1, KV_HEADS, HEAD_DIM, dtype, 0.173),
                      ref_rows(len_a, 0.2, KV_HEADS, HEAD_DIM, dtype, 0.173), slots(ta, range(len_a)))
    write_kv_to_cache(c, 0, ref_rows(len_b, 0.3, KV_HEADS, HEAD_DIM, dtype, 0.173),
                      ref_rows(len_b, 0.4, KV_HEADS, HEAD_DIM, dtype, 0.173), slots(tb, range(len_b)))
    q = ref_rows(chunk_a + 1, 0.5, HEADS, HEAD_DIM, dtype, 0.131)
    batch = ForwardBatch(cu_seqlens_q=[0, chunk_a, chunk_a + 1],
                         cu_seqlens_k=[0, len_a, len_a + len_b], block_tables=[ta, tb],
                         max_seqlen_q=chunk_a, max_seqlen_k=len_a)
    return c, q, batch


@pytest.mark.parametrize("layout", ["HND", "NHD"])
@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 1e-2), (torch.float16, 1e-3)])
def test_the_kernel_matches_the_cpu_reference(dtype, tol, layout):
    c, q, batch = mixed(dtype, layout)
    scale = 1.0 / HEAD_DIM ** 0.5
    want = oracle_out(q, c, 0, batch, scale)
    got = paged_attention(q, c, 0, batch, scale)
    assert got.shape == want.shape
    d = max_abs(got, want)
    assert d < tol, f"{dtype}: max abs diff {d}"


def test_laguna_shapes_match_the_cpu_reference():
    """attention.rs:558-625: head_dim 16, GQA 3:1 and 4:1, window 6."""
    for heads, window in [(6, None), (8, 6), (6, 6)]:
        kvh, hd = 2, 16
        c = PagedKvCache(1, 8, BLOCK, kvh, hd, torch.bfloat16)

        def mk(n, h, seed):
            i = torch.arange(n * h * hd, dtype=torch.float32)
            return (torch.sin(i * 0.173 + seed) * 0.5).reshape(n, h, hd).to(torch.bfloat16).to(DEV)

        ta, tb = [4], [6, 1]
        la, lb = 18, 40
        write_kv_to_cache(c, 0, mk(la, kvh, 0.1), mk(la, kvh, 0.2), slots(ta, range(la)))
        write_kv_to_cache(c, 0, mk(lb, kvh, 0.3), mk(lb, kvh, 0.4), slots(tb, range(lb)))
        q = mk(la + 1, heads, 0.5)
        batch = ForwardBatch(cu_seqlens_q=[0, la, la + 1], cu_seqlens_k=[0, la, la + lb],
                             block_tables=[ta, tb], max_seqlen_q=la, max_seqlen_k=lb)
        scale = 1.0 / hd ** 0.5
        want = oracle_out(q, c, 0, batch, scale, window)
        got = paged_attention(q, c, 0, batch, scale, window)
        d = max_abs(got, want)
        assert d < 1e-2, f"heads {heads} window {window}: max abs diff {d}"


def test_a_sliding_window_matches_the_cpu_reference_and_differs_from_full():
    c, q, batch = mixed(torch.bfloat16)
    scale = 1.0 / HEAD_DIM ** 0.5
    want = oracle_out(q, c, 0, batch, scale, 16)
    got = paged_attention(q, c, 0, batch, scale, 16)
    assert max_abs(got, want) < 1e-2
    full = oracle_out(q, c, 0, batch, scale)
    assert max_abs(full, want) > 1e-2, "the window must hide something"


def test_a_bidirectional_window_is_not_causal():
    c, q, batch = mixed(torch.bfloat16)
    scale = 1.0 / HEAD_DIM ** 0.5
    causal = paged_attention_windowed(q, c, 0, batch, scale, None, 0)
    bidir = paged_attention_windowed(q, c, 0, batch, scale, None, None)
    want = oracle_out(q, c, 0, batch, scale)
    assert max_abs(causal, want) < 1e-2
    assert max_abs(bidir[:20], want[:20]) > 1e-2
    assert max_abs(bidir, oracle_out(q, c, 0, batch, scale, None, -1)) < 1e-2


def test_the_sliding_window_closed_form_on_the_device():
    """attention.rs:323-353 with Q = 0: output[1] is the mean visible key index."""
    c = PagedKvCache(1, 2, 4, 1, 2, torch.float32)
    k = torch.tensor([[i, 0.0] for i in range(6)]).reshape(6, 1, 2).to(DEV)
    v = torch.tensor([[1.0, i] for i in range(6)]).reshape(6, 1, 2).to(DEV)
    write_kv_to_cache(c, 0, k, v, list(range(6)))
    q = torch.zeros(6, 1, 2, device=DEV)
    batch = ForwardBatch(cu_seqlens_q=[0, 6], cu_seqlens_k=[0, 6], block_tables=[[0, 1]],
                         max_seqlen_q=6, max_seqlen_k=6)
    out = paged_attention(q, c, 0, batch, 1.0, 3)
    assert out[:, 0, 1].cpu().tolist() == [0.0, 0.5, 1.0, 2.0, 3.0, 4.0]


# ---- random mixed batches over every kernel path --------------------------------

def random_case(rng, dtype, heads, kvh, d, bs, lens_q, lens_k, layout, nb=None):
    """A random batch over a fresh pool; layout "HND-bm"/"NHD-bm" is a
    two-layer block-major pool (layer 0 attended; blocks 4 blocks apart)."""
    nb = nb or sum(-(-l // bs) for l in lens_k) + 3
    if layout.endswith("-bm"):
        c = PagedKvCache(2, nb, bs, kvh, d, dtype, layout[:-3], block_major=True)
    else:
        c = PagedKvCache(1, nb, bs, kvh, d, dtype, layout)
    workload.fill_normal(c._slab, int(rng.integers(1 << 30)))
    perm = rng.permutation(nb)
    tables, at = [], 0
    for lk in lens_k:
        n = -(-lk // bs)
        tables.append(perm[at:at + n].tolist())
        at += n
    g = torch.Generator(device=DEV).manual_seed(int(rng.integers(1 << 30)))
    q = torch.randn(sum(lens_q), heads, d, generator=g, device=DEV).to(dtype)
    batch = ForwardBatch(cu_seqlens_q=np.concatenate([[0], np.cumsum(lens_q)]).tolist(),
                         cu_seqlens_k=np.concatenate([[0], np.cumsum(lens_k)]).tolist(),
                         block_tables=tables, max_seqlen_q=max(lens_q),
                         max_seqlen_k=max(lens_k))
    return c, q, batch


CASES = [
    # dtype, heads, kvh, d, bs, lens_q, lens_k, window, layout
    (torch.bfloat16, 32, 8, 128, 16, [1, 1, 1, 1], [1, 17, 600, 1500], None, "HND"),
    (torch.bfloat16, 32, 8, 128, 16, [1, 37, 1, 64], [700, 37, 33, 300], None, "NHD"),
    (torch.float16, 16, 8, 128, 32, [1, 5, 1], [1100, 40, 513], None, "HND"),
    (torch.bfloat16, 28, 4, 128, 16, [1, 19], [2000, 300], 100, "HND"),
    (torch.bfloat16, 8, 8, 64, 16, [1, 100], [900, 100], None, "HND"),
    (torch.bfloat16, 64, 4, 64, 32, [2, 1], [70, 64], 9, "NHD"),
    (torch.float32, 16, 8, 128, 16, [1, 1, 9], [64, 512, 200], None, "HND"),
    (torch.float32, 6, 2, 80, 8, [3, 1], [10, 50], 4, "NHD"),
    # Sequences with no new query rows (attention.rs:104-106 skips them).
    (torch.bfloat16, 32, 8, 128, 16, [0, 1, 3, 0, 1], [5, 100, 40, 7, 1], None, "HND"),
    # Larger blocks on the MFMA paths (a 16-key tile is part of one block).
    (torch.bfloat16, 32, 8, 128, 64, [1, 20, 1], [1000, 200, 65], None, "HND"),
    (torch.float16, 16, 4, 64, 128, [1, 33, 1], [700, 300, 129], 50, "NHD"),
    (torch.bfloat16, 8, 8, 128, 256, [1, 1, 17], [2000, 257, 600], None, "HND"),
    # More than 16 query heads per kv head: the decode splits each group
    # into ceil(G / 16) virtual kv heads of at most 16 (G = 32, 24, 48, 64,
    # 128, 80, 96; uneven: 17 as 9 + 8, Falcon-7B's 71 as 4 x 15 + 11, 33);
    # the prefill rows take them as they are.
    (torch.bfloat16, 32, 1, 128, 16, [1, 9, 1], [300, 40, 77], None, "HND"),
    (torch.float16, 48, 2, 64, 16, [1, 1, 20, 1], [700, 2000, 200, 33], 100, "NHD"),
    (torch.bfloat16, 48, 1, 128, 32, [1, 1, 1], [4000, 1, 650], None, "HND"),
    (torch.bfloat16, 64, 1, 128, 16, [1, 5, 1], [1500, 900, 64], 300, "HND"),
    (torch.bfloat16, 17, 1, 128, 16, [1, 4, 1], [500, 60, 1000], None, "HND"),
    (torch.bfloat16, 128, 1, 128, 16, [1, 3, 1], [1200, 300, 80], None, "HND"),
    (torch.float16, 160, 2, 64, 32, [1, 1, 1], [900, 2000, 40], 200, "NHD"),
    (torch.float32, 96, 1, 128, 16, [1, 12], [700, 150], None, "HND"),
    (torch.bfloat16, 80, 1, 80, 16, [1, 1], [1000, 3000], None, "HND-bm"),
    (torch.bfloat16, 71, 1, 64, 32, [1, 1, 7, 1], [2500, 40, 300, 900], None, "HND"),
    (torch.float16, 66, 2, 128, 16, [1, 1], [700, 1800], 250, "NHD"),
    (torch.float32, 71, 1, 64, 16, [1, 1], [600, 1300], None, "HND"),
    (torch.bfloat16, 200, 1, 96, 16, [1, 3, 1], [900, 50, 2100], None, "HND-bm"),
    # head_dim 256 on the MFMA kernels (one 16-row tile per prefill wave):
    # decode-only batches (G = 4, 1, 8, and 32 as two virtual kv heads) and
    # batches with prefill rows (decode and prefill launched separately).
    (torch.float16, 8, 4, 256, 16, [1, 6], [500, 70], 30, "NHD"),
    (torch.bfloat16, 32, 8, 256, 16, [1, 1, 1, 1, 1], [1, 17, 600, 1500, 4000], None, "HND"),
    (torch.float16, 8, 8, 256, 32, [1, 1, 1], [65, 2100, 31], 40, "NHD"),
    (torch.bfloat16, 16, 2, 256, 64, [1, 0, 1], [3000, 9, 129], None, "NHD"),
    (torch.bfloat16, 64, 2, 256, 16, [1, 1], [900, 2500], 300, "HND"),
    (torch.bfloat16, 32, 8, 256, 16, [64, 1, 200, 17], [1000, 300, 200, 900], None, "HND"),
    (torch.float16, 64, 2, 256, 32, [33, 1, 5], [700, 1200, 5], 100, "NHD"),
    # Block-major pools (blocks strided by every layer's K and V block):
    # MFMA decode + prefill, the mixed launch, f32 and head_dim 256.
    (torch.bfloat16, 32, 8, 128, 16, [1, 37, 1, 64], [700, 37, 33, 300], None, "HND-bm"),
    (torch.float16, 16, 4, 64, 32, [1, 1, 20, 1], [900, 65, 300, 2], 50, "NHD-bm"),
    (torch.float32, 16, 8, 128, 16, [1, 9, 1], [64, 512, 200], None, "HND-bm"),
    (torch.bfloat16, 16, 4, 256, 16, [1, 30, 1], [1000, 300, 17], None, "HND-bm"),
    (torch.float32, 12, 4, 80, 16, [1, 20], [1500, 700], None, "NHD-bm"),
    # Other head dims (multiples of 8 up to 256) in decode-only batches: the
    # decode stream at the next of 64, 128, 256, zeros past head_dim.
    (torch.bfloat16, 32, 8, 80, 16, [1, 1, 1, 1, 1], [1, 17, 600, 1500, 4000], None, "HND"),
    (torch.float16, 16, 4, 96, 32, [1, 1, 1], [65, 2100, 31], 40, "NHD"),
    (torch.bfloat16, 8, 8, 48, 16, [1, 1], [900, 129], None, "HND"),
    (torch.bfloat16, 6, 2, 16, 16, [1, 1], [50, 700], 6, "HND"),
    (torch.bfloat16, 64, 2, 160, 16, [1, 1], [900, 2500], 300, "HND"),
    (torch.bfloat16, 12, 4, 112, 64, [1, 0, 1], [3000, 9, 129], None, "NHD-bm"),
    (torch.float16, 6, 2, 192, 16, [1, 1, 1], [500, 70, 2000], 30, "HND"),
    (torch.bfloat16, 24, 8, 80, 16, [1] * 3, [1000, 20, 300], None, "HND"),
    (torch.float32, 32, 8, 80, 16, [1, 1, 1, 1], [1, 600, 1500, 4000], None, "HND"),
    (torch.float32, 16, 4, 96, 32, [1, 1, 1], [65, 2100, 31], 40, "NHD"),
    (torch.float32, 8, 8, 40, 16, [1, 1], [900, 1290], None, "HND-bm"),
    # ... and with prefill rows (16-bit pools): the prefill kernel at the
    # next D, Q and K chunks past head_dim zero, output columns past it
    # unstored; below 128 a batch with both kinds of rows takes the
    # one-launch mixed step with the padded kernels, above it two launches.
    (torch.bfloat16, 32, 8, 80, 16, [1, 37, 1, 64], [700, 37, 33, 300], None, "HND"),
    (torch.float16, 16, 4, 96, 32, [20, 1, 5], [900, 65, 300], 50, "NHD"),
    (torch.bfloat16, 8, 8, 48, 16, [1, 100], [900, 100], None, "HND-bm"),
    (torch.bfloat16, 6, 2, 16, 16, [40, 1], [50, 700], 6, "HND"),
    (torch.bfloat16, 16, 2, 160, 16, [64, 1], [1000, 300], None, "HND"),
    (torch.float16, 64, 2, 200, 32, [33, 1, 5], [700, 1200, 5], 100, "NHD"),
    (torch.bfloat16, 12, 4, 248, 16, [130, 0], [400, 9], None, "HND-bm"),
    # f32 pools: paged_prefill_f32 at the next of 64 and 128 (multiples of 4).
    (torch.float32, 16, 4, 96, 16, [20, 1, 5], [900, 65, 300], 50, "NHD"),
    (torch.float32, 8, 8, 40, 16, [33, 1], [700, 1200], None, "HND-bm"),
    (torch.float32, 32, 1, 120, 32, [9, 1], [300, 40], None, "HND"),
    (torch.float32, 6, 2, 4, 16, [12, 1], [40, 300], None, "HND"),
    # Head dims that end inside the last live d tile of a variant (72 and
    # 88: tiles 5 and 6 of D = 128 partly zero; f32 68 and 20).
    (torch.bfloat16, 16, 4, 72, 16, [1, 33, 1], [900, 300, 2000], None, "HND"),
    (torch.float16, 8, 2, 88, 32, [50, 1], [600, 1500], 200, "NHD-bm"),
    (torch.float32, 8, 2, 68, 16, [1, 40, 1], [2000, 500, 3000], None, "HND"),
    (torch.float32, 12, 4, 20, 16, [1, 25], [1800, 400], None, "NHD"),
    # A 16-bit pool the MFMA paths do not take, on the generic kernel:
    # block_size 8.
    (torch.bfloat16, 16, 8, 128, 8, [1, 12], [210, 50], None, "HND"),
    # The VALU kernel's split contexts (more than 512 visible keys: chunks
    # combined by its merge), odd head dims on its scalar dot path.
    (torch.float32, 12, 4, 80, 8, [1, 20, 1], [3000, 1500, 700], None, "HND"),
    (torch.float32, 4, 2, 3, 4, [1, 5], [1100, 600], 100, "NHD"),
    (torch.float32, 8, 8, 128, 16, [1, 37], [2100, 1100], 700, "HND"),
    (torch.float32, 16, 4, 256, 16, [1, 9], [2000, 800], None, "HND"),
    # More head dims the VALU kernel compiles as constants (96, 32; block
    # sizes below 16 keep a 16-bit pool there), and a block size that is
    # not a power of two.
    (torch.bfloat16, 16, 4, 96, 8, [1, 7], [900, 130], None, "HND"),
    (torch.float16, 8, 2, 32, 12, [1, 3, 1], [260, 45, 1300], 40, "NHD"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{str(c[0])[6:]}-h{c[1]}-kv{c[2]}-d{c[3]}-bs{c[4]}-w{c[7]}-{c[8]}")
def test_random_mixed_batches_match_the_oracle(case):
    dtype, heads, kvh, d, bs, lens_q, lens_k, window, layout = case
    rng = np.random.default_rng(zlib.crc32(str(case).encode()))
    c, q, batch = random_case(rng, dtype, heads, kvh, d, bs, lens_q, lens_k, layout)
    scale = d ** -0.5
    want = oracle_out(q, c, 0, batch, scale, window)
    got = paged_attention(q, c, 0, batch, scale, window)
    d_abs = max_abs(got, want)
    if dtype == torch.float32:
        assert d_abs <= 1e-5, d_abs
    else:
        assert d_abs <= 2e-2 * float(want.abs().max()), d_abs


def drawn_case(seed):
    """A batch drawn from a seed: dtype, GQA group (1-32), head_dim, block
    size, layout (block-major for every fourth seed), window, and 1-6 sequences mixing decode rows with prefill
    chunks of up to 150 tokens over up to 2,500 keys."""
    rng = np.random.default_rng(1000 + seed)
    dtype = [torch.bfloat16, torch.float16, torch.float32][int(rng.integers(3))]
    kvh = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([1, 2, 4, 8, 16, 32]))
    if dtype == torch.float32:
        d = int(rng.choice([64, 128, 128, 80]))
    else:
        d = int(rng.choice([64, 128, 128, 256, 80, 96]))
    bs = int(rng.choice([16, 32, 64]))
    layout = "HND" if rng.random() < 0.7 else "NHD"
    window = None if rng.random() < 0.6 else int(rng.integers(1, 600))
    if seed % 4 == 3:
        layout += "-bm"  # a block-major pool
    n = int(rng.integers(1, 7))
    lens_k = [int(x) for x in rng.integers(1, 2500, n)]
    lens_q = [1 if rng.random() < 0.5 else int(rng.integers(0, min(lk, 150) + 1)) for lk in lens_k]
    return dtype, kvh * group, kvh, d, bs, lens_q, lens_k, window, layout, rng


@pytest.mark.parametrize("seed", range(40))
def test_drawn_batches_match_the_oracle(seed):
    dtype, heads, kvh, d, bs, lens_q, lens_k, window, layout, rng = drawn_case(seed)
    print(f"drawn case {seed}: {dtype} h{heads} kv{kvh} d{d} bs{bs} {layout} w{window} "
          f"q{lens_q} k{lens_k}", flush=True)
    c, q, batch = random_case(rng, dtype, heads, kvh, d, bs, lens_q, lens_k, layout)
    if q.shape[0] == 0:
        pytest.skip("no query rows drawn")
    scale = d ** -0.5
    want = oracle_out(q, c, 0, batch, scale, window)
    got = paged_attention(q, c, 0, batch, scale, window)
    d_abs = max_abs(got, want)
    if dtype == torch.float32:
        assert d_abs <= 1e-5, d_abs
    else:
        assert d_abs <= 2e-2 * float(want.abs().max()), d_abs


@pytest.mark.parametrize("scale", [-0.09, 0.0, 0.7])
def test_negative_zero_and_large_scales_match_the_oracle(scale):
    """The MFMA kernels take the max on raw scores and fold |scale| into the
    exponent, negating Q for a negative scale; a zero scale is a plain mean."""
    rng = np.random.default_rng(7)
    c, q, batch = random_case(rng, torch.bfloat16, 16, 4, 128, 16, [1, 40, 1], [300, 90, 33],
                              "HND")
    want = oracle_out(q, c, 0, batch, scale)
    got = paged_attention(q, c, 0, batch, scale)
    assert max_abs(got, want) <= 2e-2 * float(want.abs().max())


def test_config0_decode_f32_matches_within_1e_5():
    """Qwen3-0.6B-shaped f32 decode; prior context and the
    new token appended through slot_mapping, then attend."""
    w = workload.config0_decode_small()
    c = PagedKvCache(1, w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim, torch.float32)
    g = torch.Generator(device=DEV).manual_seed(workload.seed_for(0))
    for t, l in zip(w.tables, w.lens):
        prev = int(l) - 1
        k = torch.randn(prev, 8, 128, generator=g, device=DEV)
        v = torch.randn(prev, 8, 128, generator=g, device=DEV)
        write_kv_to_cache(c, 0, k, v, workload.slots_for(t, np.arange(prev), 16))
    knew = torch.randn(w.batch, 8, 128, generator=g, device=DEV)
    vnew = torch.randn(w.batch, 8, 128, generator=g, device=DEV)
    write_kv_to_cache(c, 0, knew, vnew, w.new_token_slots())
    q = torch.randn(w.batch, 16, 128, generator=g, device=DEV)
    batch = ForwardBatch(cu_seqlens_q=w.cu_q().tolist(), cu_seqlens_k=w.cu_k().tolist(),
                         block_tables=[t.tolist() for t in w.tables], max_seqlen_q=1,
                         max_seqlen_k=int(w.lens.max()))
    scale = 128 ** -0.5
    want = oracle_out(q, c, 0, batch, scale)
    got = paged_attention(q, c, 0, batch, scale)
    assert max_abs(got, want) <= 1e-5


def test_config2_decode_full_size_matches_the_oracle():
    """BASELINE config 2 at full size (64 sequences, log-normal contexts up to
    8k, 32k-block pool); every sequence checked against the oracle."""
    w = workload.config2_decode()
    c = PagedKvCache(1, w.num_blocks, w.block_size, 8, 128, torch.bfloat16)
    workload.fill_normal(c._slab, workload.seed_for(2))
    g = torch.Generator(device=DEV).manual_seed(7)
    q = torch.randn(w.batch, 32, 128, generator=g, device=DEV).to(torch.bfloat16)
    batch = ForwardBatch(cu_seqlens_q=w.cu_q().tolist(), cu_seqlens_k=w.cu_k().tolist(),
                         block_tables=[t.tolist() for t in w.tables], max_seqlen_q=1,
                         max_seqlen_k=int(w.lens.max()))
    scale = 128 ** -0.5
    want = oracle_out(q, c, 0, batch, scale)
    bound = 2e-2 * float(want.abs().max())
    # Back-to-back launches on one workspace: the work-stealing decode splits
    # the batch differently each time and leaves its counters and marks reset
    # for the next launch, so every repetition must match.
    prep = PreparedAttention.from_batch(batch, DEV)
    outs = [paged_attention_prepared(q, c, 0, prep, scale) for _ in range(4)]
    for got in outs:
        assert max_abs(got, want) <= bound


F32_DECODE_CASES = [
    # heads, kvh, d, bs, lens_k, window, layout: every row a decode row, so
    # the f32 pool runs the decode stream on f32 MFMAs
    (16, 8, 128, 16, [1, 17, 600, 1500, 4000], None, "HND"),
    (32, 8, 128, 16, [5, 33, 800, 2047, 64], 100, "NHD"),
    (8, 2, 64, 32, [1, 31, 640, 3000], None, "HND"),
    (64, 4, 128, 16, [48, 700, 1201], None, "HND"),
    (8, 8, 128, 64, [65, 1000, 129, 2], 40, "NHD"),
    (12, 4, 64, 16, [300] * 39 + [600], None, "HND"),
    # G = 32 and 64 (two and four virtual kv heads of 16 query heads)
    (32, 1, 128, 16, [1, 700, 2500], None, "HND"),
    (64, 1, 64, 16, [90, 3000], 50, "NHD"),
]


@pytest.mark.parametrize("case", F32_DECODE_CASES, ids=lambda c: f"h{c[0]}-kv{c[1]}-d{c[2]}-bs{c[3]}-w{c[5]}-{c[6]}")
def test_f32_decode_on_mfma_matches_within_1e_5(case):
    """f32 pools, pure decode batches (v_mfma_f32_16x16x4_f32 stream):
    max-abs <= 1e-5 against the f32 oracle (the reference's CPU bar), for
    GQA 1..16, head_dim 64 and 128, blocks of 16..64, windows, both layouts,
    and the negated scale on the first case."""
    heads, kvh, d, bs, lens_k, window, layout = case
    rng = np.random.default_rng(zlib.crc32(str(case).encode()))
    c, q, batch = random_case(rng, torch.float32, heads, kvh, d, bs, [1] * len(lens_k), lens_k,
                              layout)
    scales = [d ** -0.5] + ([-(d ** -0.5)] if case is F32_DECODE_CASES[0] else [])
    for scale in scales:
        want = oracle_out(q, c, 0, batch, scale, window)
        got = paged_attention(q, c, 0, batch, scale, window)
        assert max_abs(got, want) <= 1e-5, (scale, max_abs(got, want))


def test_config2_shape_f32_decode_full_size_matches_within_1e_5():
    """Config 2's batch (64 sequences, contexts up to 8k, 32k blocks) over an
    f32 pool: every row within 1e-5 of the f32 oracle, on repeated calls."""
    w = workload.config2_decode()
    c = PagedKvCache(1, w.num_blocks, w.block_size, 8, 128, torch.float32)
    workload.fill_normal(c._slab, workload.seed_for(2))
    g = torch.Generator(device=DEV).manual_seed(9)
    q = torch.randn(w.batch, 32, 128, generator=g, device=DEV)
    batch = ForwardBatch(cu_seqlens_q=w.cu_q().tolist(), cu_seqlens_k=w.cu_k().tolist(),
                         block_tables=[t.tolist() for t in w.tables], max_seqlen_q=1,
                         max_seqlen_k=int(w.lens.max()))
    scale = 128 ** -0.5
    want = oracle_out(q, c, 0, batch, scale)
    prep = PreparedAttention.from_batch(batch, DEV)
    for _ in range(3):
        got = paged_attention_prepared(q, c, 0, prep, scale)
        assert max_abs(got, want) <= 1e-5


F32_PREFILL_CASES = [
    # heads, kvh, d, bs, lens_q, lens_k, window, layout: f32 pools with
    # prefill rows (decode rows on the f32 decode stream, prefill rows on
    # paged_prefill_f32)
    (32, 8, 128, 16, [64, 1, 200, 17], [1000, 300, 200, 900], None, "HND"),
    (16, 8, 128, 32, [1, 37, 1, 3], [700, 37, 33, 2100], 100, "NHD"),
    (8, 2, 64, 16, [100, 1], [900, 100], None, "HND"),
    (64, 4, 64, 64, [2, 1, 45], [70, 64, 3000], 9, "NHD"),
    (12, 4, 128, 16, [0, 5, 1, 0, 130], [5, 100, 40, 7, 1200], None, "HND"),
    (32, 1, 128, 16, [1, 9, 1], [300, 40, 77], None, "HND"),
]


@pytest.mark.parametrize("case", F32_PREFILL_CASES, ids=lambda c: f"h{c[0]}-kv{c[1]}-d{c[2]}-bs{c[3]}-q{max(c[4])}-w{c[6]}-{c[7]}")
def test_f32_prefill_on_mfma_matches_within_1e_5(case):
    """f32 pools with prefill rows (GQA 1-32, head_dim 64 and 128, blocks of
    16-64, windows, both layouts, sequences without rows): max-abs <= 1e-5
    against the f32 oracle."""
    heads, kvh, d, bs, lens_q, lens_k, window, layout = case
    rng = np.random.default_rng(zlib.crc32(str(case).encode()))
    c, q, batch = random_case(rng, torch.float32, heads, kvh, d, bs, lens_q, lens_k, layout)
    scale = d ** -0.5
    want = oracle_out(q, c, 0, batch, scale, window)
    got = paged_attention(q, c, 0, batch, scale, window)
    assert max_abs(got, want) <= 1e-5, max_abs(got, want)


def test_config3_f32_prefill_rows_match_within_1e_5():
    """Config 3's batch over an f32 pool (paged_prefill_f32): rows at the
    start, middle and end of four sequences within 1e-5 of the f32 oracle."""
    w = workload.config3_prefill()
    c = PagedKvCache(1, w.num_blocks, w.block_size, 8, 128, torch.float32)
    workload.fill_normal(c._slab, workload.seed_for(3))
    g = torch.Generator(device=DEV).manual_seed(8)
    q = torch.randn(w.batch * w.len_q, 32, 128, generator=g, device=DEV)
    batch = ForwardBatch(cu_seqlens_q=w.cu_q().tolist(), cu_seqlens_k=w.cu_k().tolist(),
                         block_tables=[t.tolist() for t in w.tables], max_seqlen_q=w.len_q,
                         max_seqlen_k=w.len_k)
    scale = 128 ** -0.5
    got = paged_attention(q, c, 0, batch, scale)
    kc = host_f32(c.reference_view(0, "k").contiguous())
    vc = host_f32(c.reference_view(0, "v").contiguous())
    for s in (0, 9, 18, 31):
        for j0 in (0, 250, w.len_q - 16):
            rows_q = q[s * w.len_q + j0: s * w.len_q + j0 + 16]
            lk = w.len_k - w.len_q + j0 + 16
            want = oracle.paged_attention(host_f32(rows_q), kc, vc, [0, 16], [0, lk],
                                          [w.tables[s].tolist()], scale, threads=8)
            gr = got[s * w.len_q + j0: s * w.len_q + j0 + 16]
            assert max_abs(gr, torch.from_numpy(want)) <= 1e-5, (s, j0)


def test_config3_prefill_rows_match_the_oracle():
    """BASELINE config 3 (32 x 512-token chunks over 4,096 keys, shared
    prefixes): the whole batch runs in one call; rows at the start, middle and
    end of four sequences are checked against the oracle run on those rows."""
    w = workload.config3_prefill()
    c = PagedKvCache(1, w.num_blocks, w.block_size, 8, 128, torch.bfloat16)
    workload.fill_normal(c._slab, workload.seed_for(3))
    g = torch.Generator(device=DEV).manual_seed(8)
    q = torch.randn(w.batch * w.len_q, 32, 128, generator=g, device=DEV).to(torch.bfloat16)
    batch = ForwardBatch(cu_seqlens_q=w.cu_q().tolist(), cu_seqlens_k=w.cu_k().tolist(),
                         block_tables=[t.tolist() for t in w.tables], max_seqlen_q=w.len_q,
                         max_seqlen_k=w.len_k)
    scale = 128 ** -0.5
    got = paged_attention(q, c, 0, batch, scale)
    kc = host_f32(c.reference_view(0, "k").contiguous())
    vc = host_f32(c.reference_view(0, "v").contiguous())
    for s in (0, 9, 18, 31):
        for j0 in (0, 250, w.len_q - 16):
            rows_q = q[s * w.len_q + j0: s * w.len_q + j0 + 16]
            lk = w.len_k - w.len_q + j0 + 16
            want = oracle.paged_attention(host_f32(rows_q), kc, vc, [0, 16], [0, lk],
                                          [w.tables[s].tolist()], scale, threads=8)
            want = torch.from_numpy(want).to(torch.bfloat16).float()
            gr = got[s * w.len_q + j0: s * w.len_q + j0 + 16]
            assert max_abs(gr, want) <= 2e-2 * float(want.abs().max()), (s, j0)


def test_prepared_inputs_are_reusable_across_layers():
    rng = np.random.default_rng(9)
    L = 3
    c = PagedKvCache(L, 64, 16, 8, 128, torch.bfloat16)
    workload.fill_normal(c._slab, 9)
    lens_k = [300, 1, 520]
    perm = rng.permutation(64)
    tables, at = [], 0
    for lk in lens_k:
        n = -(-lk // 16)
        tables.append(perm[at:at + n].tolist())
        at += n
    q = torch.randn(3, 32, 128, device=DEV).to(torch.bfloat16)
    batch = ForwardBatch(cu_seqlens_q=[0, 1, 2, 3], cu_seqlens_k=np.concatenate([[0], np.cumsum(lens_k)]).tolist(),
                         block_tables=tables, max_seqlen_q=1, max_seqlen_k=520)
    prep = PreparedAttention.from_batch(batch, DEV)
    for layer in range(L):
        got = paged_attention_prepared(q, c, layer, prep, 128 ** -0.5)
        want = oracle_out(q, c, layer, batch, 128 ** -0.5)
        assert max_abs(got, want) <= 2e-2 * float(want.abs().max())


def test_a_workspace_reused_across_batches_and_launches_stays_correct():
    """One workspace carries the decode's balance state and partial slots from
    launch to launch: a big batch, then smaller batches with fewer steps than
    waves (empty slices whose partial slots still hold the big batch's data),
    then the big batch again, each against the oracle."""
    rng = np.random.default_rng(21)
    c = PagedKvCache(1, 4096, 16, 8, 128, torch.bfloat16)
    workload.fill_normal(c._slab, 21)
    perm = rng.permutation(4096)

    def make(lens):
        tables, at = [], 0
        for lk in lens:
            n = -(-lk // 16)
            tables.append(perm[at:at + n].tolist())
            at += n
        return ForwardBatch(cu_seqlens_q=list(range(len(lens) + 1)),
                            cu_seqlens_k=np.concatenate([[0], np.cumsum(lens)]).tolist(),
                            block_tables=tables, max_seqlen_q=1, max_seqlen_k=max(lens))

    big = make(rng.integers(1500, 4000, size=16).tolist())
    small = [make([300, 1, 520]), make([33, 2000]), make([1])]
    ws = None
    for batch in [big, *small, big, small[1]]:
        prep = PreparedAttention.from_batch(batch, DEV)
        if ws is not None and ws.numel() >= paged_ws_bytes(c, batch):
            prep.workspace = ws
        q = torch.randn(batch.batch_size(), 32, 128, device=DEV).to(torch.bfloat16)
        for _ in range(2):
            got = paged_attention_prepared(q, c, 0, prep, 128 ** -0.5)
            want = oracle_out(q, c, 0, batch, 128 ** -0.5)
            assert max_abs(got, want) <= 2e-2 * float(want.abs().max()), batch.cu_seqlens_k
        ws = prep.workspace


def paged_ws_bytes(cache, batch):
    from vapi_amd.attention import workspace_bytes
    return workspace_bytes(cache, batch.batch_size(), 32, 1, batch.max_seqlen_k)


def test_more_decode_rows_than_one_launch_plans_for():
    """5,000 decode rows: the host splits the batch into launches of at most
    4,096 sequences that share one workspace; every row against the oracle."""
    rng = np.random.default_rng(5000)
    lens_k = rng.integers(1, 80, size=5000).tolist()
    nb = sum(-(-lk // 16) for lk in lens_k)
    c, q, batch = random_case(rng, torch.bfloat16, 8, 2, 128, 16, [1] * 5000, lens_k, "HND")
    assert c.num_blocks >= nb
    want = oracle_out(q, c, 0, batch, 128 ** -0.5)
    got = paged_attention(q, c, 0, batch, 128 ** -0.5)
    assert max_abs(got, want) <= 2e-2 * float(want.abs().max())


@pytest.mark.parametrize("lens_q,lens_k", [([1], [131072]), ([1, 1], [65536, 3]),
                                           ([16], [32768])])
def test_one_very_long_context_matches_the_oracle(lens_q, lens_k):
    """A single context of 64k-128k keys: each (sequence, kv head) segment of
    the decode is split over a hundred or more wave slices, so the merge
    walks long chains of partials; and a prefill chunk over a long context."""
    rng = np.random.default_rng(sum(lens_k))
    c, q, batch = random_case(rng, torch.bfloat16, 32, 8, 128, 16, lens_q, lens_k, "HND")
    want = oracle_out(q, c, 0, batch, 128 ** -0.5)
    got = paged_attention(q, c, 0, batch, 128 ** -0.5)
    assert max_abs(got, want) <= 2e-2 * float(want.abs().max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_table_entries_past_the_pool_read_the_last_block_instead_of_faulting(dtype):
    """A block table is device data the call cannot check on the host:
    entries past the pool are clamped to the last block (ForwardBatch::
    validate, backend.rs:96-204, is where a bad table is refused), so the
    result equals the same batch with those entries replaced by it. Decode
    and prefill rows, MFMA (bf16) and VALU (f32) paths."""
    c, q, batch = mixed(dtype)
    nb = c.num_blocks
    bad = ForwardBatch(cu_seqlens_q=batch.cu_seqlens_q, cu_seqlens_k=batch.cu_seqlens_k,
                       block_tables=[[5, nb + 3, 6], [7, 1 << 30]],
                       max_seqlen_q=batch.max_seqlen_q, max_seqlen_k=batch.max_seqlen_k)
    clamped = ForwardBatch(cu_seqlens_q=batch.cu_seqlens_q, cu_seqlens_k=batch.cu_seqlens_k,
                           block_tables=[[5, nb - 1, 6], [7, nb - 1]],
                           max_seqlen_q=batch.max_seqlen_q, max_seqlen_k=batch.max_seqlen_k)
    scale = HEAD_DIM ** -0.5
    got = paged_attention(q, c, 0, bad, scale)
    want = paged_attention(q, c, 0, clamped, scale)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_keys_past_the_table_row_read_its_last_entry_instead_of_faulting(dtype):
    """cu_seqlens_k is device data too: a sequence longer than its table row
    (len_k > max_blocks * block_size) reads the row's last entry for the keys
    past it rather than another row or memory past the table. The call must
    finish; the rows within the table are unaffected."""
    c, q, batch = mixed(dtype)
    # B's table has 2 blocks (64 keys) in a [2, 3] table; claim 100 keys.
    over = ForwardBatch(cu_seqlens_q=batch.cu_seqlens_q, cu_seqlens_k=[0, 90, 190],
                        block_tables=batch.block_tables, max_seqlen_q=batch.max_seqlen_q,
                        max_seqlen_k=100)
    prep = PreparedAttention.from_batch(over, DEV)  # no host check of table coverage
    scale = HEAD_DIM ** -0.5
    got = paged_attention_prepared(q, c, 0, prep, scale)
    want = paged_attention(q, c, 0, batch, scale)
    torch.cuda.synchronize()
    assert torch.equal(got[:20], want[:20])
    assert bool(torch.isfinite(got.float()).all())


# ---- small prefill batches: the keys split over more workgroups -------------

SPLIT_CASES = [
    # dtype, heads, kvh, d, bs, lens_q, lens_k, window, layout
    (torch.bfloat16, 32, 8, 128, 16, [64], [4096], None, "HND"),
    (torch.bfloat16, 32, 8, 128, 16, [40, 1, 100], [3000, 2500, 2100], None, "NHD"),
    (torch.float16, 16, 4, 64, 32, [96, 1], [5000, 700], 1500, "HND"),
    (torch.bfloat16, 28, 4, 128, 16, [300], [2600], 700, "HND"),
    # 5 query tiles x 4 kv heads: 13 splits, merged in a batch of eight and
    # a partial batch of five.
    (torch.bfloat16, 16, 4, 128, 16, [320], [4000], None, "HND"),
    (torch.bfloat16, 16, 4, 256, 16, [100, 1], [3000, 2000], None, "HND"),
    (torch.float16, 8, 8, 256, 32, [48], [2500], 900, "NHD"),
    # Padded head dims: the split's partials hold D columns, the merge
    # stores head_dim of them.
    (torch.bfloat16, 16, 4, 80, 16, [100, 1], [3000, 2000], None, "HND"),
    (torch.float16, 8, 8, 192, 32, [48], [2500], 900, "NHD"),
    # f32 pools: paged_prefill_f32's split (waves, not workgroups) and its merge.
    (torch.float32, 32, 8, 128, 16, [128], [8192], None, "HND"),
    (torch.float32, 16, 4, 64, 32, [100, 1], [3000, 2000], 500, "NHD"),
    (torch.float32, 32, 8, 128, 16, [512], [4096], None, "HND-bm"),
    (torch.float32, 16, 4, 80, 16, [100, 1], [3000, 2000], None, "HND"),
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: f"{str(c[0])[6:]}-d{c[3]}-q{c[5]}-w{c[7]}")
def test_small_prefill_batches_split_their_keys_and_match_the_oracle(case):
    """A prefill batch too small to fill the GPU with query tiles splits each
    tile's keys over up to 64 workgroups and merges their partials; with the
    workspace vapi_paged_attention_workspace_size asks for it matches the
    oracle, and so does the same call without a workspace (no split)."""
    dtype, heads, kvh, d, bs, lens_q, lens_k, window, layout = case
    rng = np.random.default_rng(zlib.crc32(str(case).encode()))
    c, q, batch = random_case(rng, dtype, heads, kvh, d, bs, lens_q, lens_k, layout)
    lib = _lib.lib()
    full = lib.vapi_paged_attention_workspace_size(c.pool, len(lens_q), heads, max(lens_q),
                                                   max(lens_k))
    decode_only = lib.vapi_paged_attention_workspace_size(c.pool, len(lens_q), heads, 1,
                                                          max(lens_k))
    assert full > decode_only  # the split asks for room
    wl = -1 if window is None else window - 1
    want = oracle_out(q, c, 0, batch, d ** -0.5, window)
    tol = (1e-5 if dtype == torch.float32 else
           (2e-2 if dtype == torch.bfloat16 else 1e-2) * float(want.abs().max()))
    prep = PreparedAttention.from_batch(batch, DEV, cache=c, num_heads=heads)
    got = torch.full_like(q, float("nan"))
    _lib.check(lib.vapi_paged_attention(
        c.pool, 0, q.data_ptr(), got.data_ptr(), prep.seqlens_q.data_ptr(),
        prep.seqlens_k.data_ptr(), prep.block_table.data_ptr(), len(lens_q),
        prep.block_table.shape[1], max(lens_q), max(lens_k), heads, d ** -0.5, wl, 0,
        prep.workspace.data_ptr(), prep.workspace.numel(), stream_handle()))
    assert max_abs(got, want) <= tol
    if 1 not in lens_q:  # prefill only: no workspace at all, no split
        plain = torch.full_like(q, float("nan"))
        _lib.check(lib.vapi_paged_attention_ex(
            c.pool, 0, q.data_ptr(), plain.data_ptr(), prep.seqlens_q.data_ptr(),
            prep.seqlens_k.data_ptr(), prep.block_table.data_ptr(), len(lens_q),
            prep.block_table.shape[1], max(lens_q), max(lens_k), heads, d ** -0.5, wl, 0,
            _lib.ATTN_NO_DECODE_ROWS, None, 0, stream_handle()))
        assert max_abs(plain, want) <= tol
        assert max_abs(plain, got) <= tol
