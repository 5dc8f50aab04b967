"""vapi_paged_attention_noalloc against vapi_paged_attention_ex through the
C ABI: the allocation-free entry point keeps its decode workspace in the
library's device array instead of a caller's buffer.

Bar: with VAPI_ATTN_DETERMINISTIC on both sides (equal XCD shares, so the
same split points and merge order) the outputs are equal bit for bit; with
adaptive shares both are within the attention tolerance of the oracle
(bf16: max-abs <= 2e-2 * max|reference|; f32 pools: 1e-5). Two calls in a row, the second on a
smaller batch, so the second runs over the first's leftover scratch.
"""
import numpy as np
import pytest
import torch

from test_gpu_attention import max_abs, oracle_out, random_case
from vapi_amd import _lib
from vapi_amd.attention import ATTN_DETERMINISTIC, PreparedAttention
from vapi_amd.cache import stream_handle

pytestmark = pytest.mark.gpu
DEV = "cuda"


def args(q, c, prep, out):
    b = prep.seqlens_q.shape[0] - 1
    return (c.pool, 0, q.data_ptr(), out.data_ptr(), prep.seqlens_q.data_ptr(),
            prep.seqlens_k.data_ptr(), prep.block_table.data_ptr(), b,
            prep.block_table.shape[1], max(prep.max_seqlen_q, 1), max(prep.max_seqlen_k, 1),
            q.shape[1], float(q.shape[2] ** -0.5), -1, 0)


def with_workspace(q, c, prep, flags):
    out = torch.full_like(q, float("nan"))
    a = args(q, c, prep, out)
    need = _lib.lib().vapi_paged_attention_workspace_size(c.pool, a[7], a[11], a[9], a[10])
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=DEV)
    _lib.check(_lib.lib().vapi_paged_attention_ex(*a, flags, ws.data_ptr(), need,
                                                  stream_handle()))
    return out


def no_alloc(q, c, prep, flags):
    out = torch.full_like(q, float("nan"))
    _lib.check(_lib.lib().vapi_paged_attention_noalloc(*args(q, c, prep, out), flags,
                                                       stream_handle()))
    return out


BIG = ([1] * 48 + [40, 1, 7, 1], None)
SMALL = ([1, 1, 12, 1], [3000, 17, 300, 1])


def case(seed, lens_q, lens_k, dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    if lens_k is None:
        lens_k = rng.integers(100, 4000, size=len(lens_q)).tolist()
    return random_case(rng, dtype, 32, 8, 128, 16, lens_q, lens_k, "HND")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("flags", [ATTN_DETERMINISTIC, 0])
def test_no_alloc_matches_the_workspace_entry_point_twice_in_a_row(flags, dtype):
    for seed, (lq, lk) in ((1, BIG), (2, SMALL)):
        c, q, batch = case(seed, lq, lk, dtype)
        prep = PreparedAttention.from_batch(batch, DEV)
        got = no_alloc(q, c, prep, flags)
        want = with_workspace(q, c, prep, flags)
        torch.cuda.synchronize()
        if flags & ATTN_DETERMINISTIC:
            assert torch.equal(got, want), (seed, max_abs(got, want))
        ref = oracle_out(q, c, 0, batch, q.shape[2] ** -0.5)
        tol = 1e-5 if dtype == torch.float32 else 2e-2 * float(ref.abs().max())
        assert max_abs(got, ref) <= tol and max_abs(want, ref) <= tol, seed


def test_no_alloc_refuses_a_batch_past_its_scratch_and_writes_nothing():
    c, q, batch = case(3, [1] * 4096, [16] * 4096)
    prep = PreparedAttention.from_batch(batch, DEV)
    need = _lib.lib().vapi_paged_attention_workspace_size(c.pool, 4096, 32, 1, 16)
    assert need > _lib.ATTN_SCRATCH_BYTES
    out = torch.full_like(q, float("nan"))
    rc = _lib.lib().vapi_paged_attention_noalloc(*args(q, c, prep, out), 0, stream_handle())
    assert rc == _lib.ESPACE
    assert b"scratch" in _lib.lib().vapi_kv_last_error()
    torch.cuda.synchronize()
    assert bool(torch.isnan(out.float()).all())


def first_call_under_capture():
    """Run in a fresh process: the first noalloc call on the device is made
    while a HIP graph is being captured. The share-clearing kernel must not
    be recorded (it would reset the shares on every replay); each replay,
    with eager work between them, must match the workspace entry point
    within the bf16 tolerance."""
    c, q, batch = case(4, *BIG)
    prep = PreparedAttention.from_batch(batch, DEV)
    out = torch.full_like(q, float("nan"))
    a = args(q, c, prep, out)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            _lib.check(_lib.lib().vapi_paged_attention_noalloc(*a, 0, stream_handle()))
    torch.cuda.current_stream().wait_stream(side)
    want = with_workspace(q, c, prep, ATTN_DETERMINISTIC)
    ref = oracle_out(q, c, 0, batch, q.shape[2] ** -0.5)
    tol = 2e-2 * float(ref.abs().max())
    for i in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert max_abs(out, ref) <= tol, ("replay", i, max_abs(out, ref))
        assert max_abs(out, want) <= tol, ("replay", i)
        with_workspace(q, c, prep, 0)  # eager work between replays
    # An eager call after the capture clears the shares once and runs.
    eager = no_alloc(q, c, prep, ATTN_DETERMINISTIC)
    torch.cuda.synchronize()
    assert torch.equal(eager, want)
    print("first-call-under-capture ok", flush=True)


def test_no_alloc_first_call_under_graph_capture():
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    code = ("import sys; sys.path[:0] = [%r, %r]; import test_zz_no_alloc as t; "
            "t.first_call_under_capture()" % (here, os.path.dirname(here)))
    r = subprocess.run([sys.executable, "-c", code], cwd=here, capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "first-call-under-capture ok" in r.stdout
