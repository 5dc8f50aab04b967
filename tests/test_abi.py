"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and its host-only entry points (argument checks,
ForwardBatch::validate, pack_block_tables, block sizing) behave like the
reference. No GPU work is launched here."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import oracle
from vapi_amd import _lib, workload
from vapi_amd.attention import ForwardBatch

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / "include" / "vapi_kv.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vapi_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.EXPORTS)
    assert L.vapi_kv_version().startswith(b"vapi_kv")


def pool(**kw):
    p = dict(k=1 << 12, v=1 << 13, layer_stride_bytes=1 << 20, num_layers=1, num_blocks=8, block_size=16,
             num_kv_heads=2, head_dim=64, dtype=_lib.BF16, layout=_lib.LAYOUT_HND)
    p.update(kw)
    return _lib.Pool(**p)


def test_bad_arguments_are_errors_not_crashes():
    L = _lib.lib()
    assert L.vapi_kv_append(pool(dtype=9), 0, 1, 1, 1, 1, None) == _lib.EINVAL
    assert b"dtype" in L.vapi_kv_last_error()
    assert L.vapi_kv_append(pool(layout=5), 0, 1, 1, 1, 1, None) == _lib.EINVAL
    assert L.vapi_kv_append(pool(), 1, 1, 1, 1, 1, None) == _lib.EINVAL
    assert L.vapi_kv_append(pool(), 0, None, 1, 1, 1, None) == _lib.EINVAL
    assert L.vapi_kv_append(pool(), 0, 1, 1, 1, 0, None) == _lib.OK  # nothing to do
    assert L.vapi_kv_append_ex(pool(), 0, 1, 1, 1, 0, _lib.APPEND_COLD_SOURCE, None) == _lib.OK
    assert L.vapi_kv_append_ex(pool(), 0, 1, 1, 1, 1, 0x2, None) == _lib.EINVAL
    assert b"flags" in L.vapi_kv_last_error()
    assert L.vapi_kv_gather(pool(), 0, 1, 2, 33, 1, 1, None) == _lib.EINVAL
    assert b"exceeds" in L.vapi_kv_last_error()
    args = [16, 16, 16, 16, 16, 2, 4, 1, 100, 5, 0.1, -1, 0, None, 0, None]
    assert L.vapi_paged_attention(pool(), 0, *args) == _lib.EINVAL
    assert b"multiple" in L.vapi_kv_last_error()
    # Workspace too small for a split-K decode.
    need = L.vapi_paged_attention_workspace_size(pool(), 2, 8, 1, 5000)
    assert need > 0
    args = [16, 16, 16, 16, 16, 2, 320, 1, 5000, 8, 0.1, -1, 0, None, 0, None]
    assert L.vapi_paged_attention(pool(), 0, *args) == _lib.ESPACE
    assert L.vapi_kv_copy_blocks(pool(num_layers=2, layer_stride_bytes=16), 1, 1, None) == _lib.EINVAL
    assert L.vapi_kv_swap_out(pool(), 1, 1, 1, 1, 10, None) == _lib.ESPACE
    # Multi-layer append: the layer range, the source layer stride.
    assert L.vapi_kv_append_layers(pool(), 0, 2, 1, 1, 1 << 20, 1, 1, None) == _lib.EINVAL
    assert L.vapi_kv_append_layers(pool(), 0, 0, 1, 1, 0, 1, 1, None) == _lib.EINVAL
    two = pool(num_layers=2, layer_stride_bytes=1 << 20)
    assert L.vapi_kv_append_layers(two, 0, 2, 1, 1, 255, 1, 1, None) == _lib.EINVAL
    assert b"stride" in L.vapi_kv_last_error()
    assert L.vapi_kv_append_layers(two, 1, 1, 1, 1, 0, 1, 0, None) == _lib.OK
    # Fused append + attention: the append's and the attention's errors.
    args = [16, 16, 16, 16, 16, 1, 2, 4, 1, 100, 8, 0.1, -1, 0, None, 0, None]
    assert L.vapi_paged_attention_append(pool(dtype=9), 0, 1, 1, 1, *args) == _lib.EINVAL
    assert L.vapi_paged_attention_append(pool(), 0, None, 1, 1, *args) == _lib.EINVAL
    assert b"null source" in L.vapi_kv_last_error()
    args = [16, 16, 16, 16, 16, 1, 2, 320, 1, 5000, 8, 0.1, -1, 0, None, 0, None]
    assert L.vapi_paged_attention_append(pool(), 0, 1, 1, 1, *args) == _lib.ESPACE


def test_misaligned_pools_and_unknown_flags_are_refused():
    """Pools whose bases or layer stride are not 16-byte multiples are
    refused before any launch (the kernels move 16-byte chunks), and so are
    flag bits the attention call does not know."""
    L = _lib.lib()
    assert L.vapi_kv_append(pool(k=(1 << 12) + 8), 0, 1, 1, 1, 1, None) == _lib.EINVAL
    assert b"16-byte aligned" in L.vapi_kv_last_error()
    assert L.vapi_kv_append(pool(v=(1 << 13) + 2), 0, 1, 1, 1, 1, None) == _lib.EINVAL
    two = pool(num_layers=2, layer_stride_bytes=(1 << 20) + 8)
    assert L.vapi_kv_copy_blocks(two, 1, 1, None) == _lib.EINVAL
    assert b"multiple of 16" in L.vapi_kv_last_error()
    assert L.vapi_kv_export_blocks(two, 1, 1, 1, None) == _lib.EINVAL
    args = [16, 16, 16, 16, 16, 2, 4, 1, 100, 8, 0.1, -1, 0]
    assert L.vapi_paged_attention_ex(pool(), 0, *args, 0x80, None, 0, None) == _lib.EINVAL
    assert b"flags" in L.vapi_kv_last_error()
    # q and out rows are moved in 16-byte chunks.
    for bad in ([24] + args[1:], args[:1] + [8] + args[2:]):
        assert L.vapi_paged_attention_ex(pool(), 0, *bad, 0, None, 0, None) == _lib.EINVAL
        assert b"16-byte aligned" in L.vapi_kv_last_error()
    # The flags call keeps vapi_paged_attention's own checks.
    need = L.vapi_paged_attention_workspace_size(pool(), 2, 8, 1, 5000)
    args = [16, 16, 16, 16, 16, 2, 320, 1, 5000, 8, 0.1, -1, 0]
    assert L.vapi_paged_attention_ex(pool(), 0, *args, _lib.ATTN_DETERMINISTIC, None, 0,
                                     None) == _lib.ESPACE
    assert need > 0


def test_block_major_descriptors_are_checked():
    """block_stride_bytes: a multiple of 16, room for every layer's block
    within a block, layers at least one block apart; refused before any
    launch otherwise. A zero-pair copy on a valid one does nothing."""
    L = _lib.lib()
    blk = 16 * 2 * 64 * 2  # block_size x kv_heads x head_dim x bf16
    ok = pool(num_layers=3, layer_stride_bytes=blk, block_stride_bytes=6 * blk)
    assert L.vapi_kv_copy_blocks(ok, 1, 0, None) == _lib.OK
    assert L.vapi_kv_append(ok, 0, 1, 1, 1, 0, None) == _lib.OK
    bad = [dict(block_stride_bytes=6 * blk + 8),           # not a multiple of 16
           dict(block_stride_bytes=2 * blk),               # 3 layers do not fit
           dict(layer_stride_bytes=blk // 2, block_stride_bytes=6 * blk)]  # layers overlap
    for kw in bad:
        args = dict(num_layers=3, layer_stride_bytes=blk)
        args.update(kw)
        assert L.vapi_kv_copy_blocks(pool(**args), 1, 1, None) == _lib.EINVAL, kw
        assert b"stride" in L.vapi_kv_last_error()


def test_the_prepared_call_checks_its_prefill_list_and_sizes_its_split():
    """vapi_paged_attention_prepared refuses a list longer than the batch or
    a null list, before anything is launched; its workspace size covers the
    key split of the listed sequences alone (a step of 63 decode rows and one
    512-token chunk splits that chunk; counted over all 64 sequences it would
    not)."""
    L = _lib.lib()
    args = [16, 16, 16, 16, 16, 2, 4, 512, 2048, 32, 0.1, -1, 0, 0]
    assert L.vapi_paged_attention_prepared(pool(), 0, *args, 1, 3, None, 0,
                                           None) == _lib.EINVAL
    assert b"prefill sequences" in L.vapi_kv_last_error()
    assert L.vapi_paged_attention_prepared(pool(), 0, *args, None, 1, None, 0,
                                           None) == _lib.EINVAL
    plain = L.vapi_paged_attention_workspace_size(pool(), 64, 32, 512, 2048)
    listed = L.vapi_paged_attention_prepared_workspace_size(pool(), 64, 1, 32, 512, 2048)
    decode_only = L.vapi_paged_attention_prepared_workspace_size(pool(), 64, 0, 32, 512, 2048)
    assert listed > plain >= decode_only > 0


def test_prepared_attention_lists_the_prefill_sequences():
    from vapi_amd.attention import PreparedAttention
    b = ForwardBatch(cu_seqlens_q=[0, 1, 6, 7, 7, 10], cu_seqlens_k=[0, 9, 18, 27, 30, 39],
                     block_tables=[[i] for i in range(5)], max_seqlen_q=5, max_seqlen_k=9)
    prep = PreparedAttention.from_batch(b, "cpu")
    assert prep.n_prefill == 2 and prep.prefill_seqs.tolist() == [1, 4]


def test_launches_too_large_for_one_grid_are_refused():
    """A batch whose prefill or VALU grid would pass 2^32 workgroups is
    refused before anything is launched, not truncated."""
    L = _lib.lib()
    # MFMA prefill: 65,535 sequences x 2^24 query rows x 4 heads per group.
    args = [16, 16, 16, 16, 16, 65535, 1, 1 << 24, 1 << 24, 8, 0.1, -1, 0]
    assert L.vapi_paged_attention_ex(pool(), 0, *args, _lib.ATTN_NO_DECODE_ROWS, None, 0,
                                     None) == _lib.EUNSUP
    assert b"too large" in L.vapi_kv_last_error()
    # VALU path (head_dim 82): row tiles x kv heads x sequences x key chunks.
    args = [16, 16, 16, 16, 16, 60000, 1, 1 << 20, 1 << 20, 8, 0.1, -1, 0]
    assert L.vapi_paged_attention_ex(pool(dtype=_lib.F32, head_dim=82), 0, *args, 0, 1,
                                     1 << 62, None) == _lib.EUNSUP
    assert b"too large" in L.vapi_kv_last_error()
    # f32 MFMA prefill: 32-row tiles x kv heads x sequences waves.
    args = [16, 16, 16, 16, 16, 65535, 1, 1 << 24, 1 << 24, 2, 0.1, -1, 0]
    assert L.vapi_paged_attention_ex(pool(dtype=_lib.F32), 0, *args, _lib.ATTN_NO_DECODE_ROWS,
                                     None, 0, None) == _lib.EUNSUP
    assert b"too large" in L.vapi_kv_last_error()


def test_prepared_attention_flags_follow_the_host_lengths():
    from vapi_amd.attention import ATTN_DETERMINISTIC, ATTN_NO_DECODE_ROWS, PreparedAttention
    mk = lambda lq, lk: ForwardBatch(cu_seqlens_q=np.concatenate([[0], np.cumsum(lq)]).tolist(),
                                     cu_seqlens_k=np.concatenate([[0], np.cumsum(lk)]).tolist(),
                                     block_tables=[[i] for i in range(len(lq))],
                                     max_seqlen_q=max(lq), max_seqlen_k=max(lk))
    assert PreparedAttention.from_batch(mk([5, 7], [9, 9]), "cpu").flags == ATTN_NO_DECODE_ROWS
    assert PreparedAttention.from_batch(mk([5, 1], [9, 9]), "cpu").flags == 0
    assert PreparedAttention.from_batch(mk([1, 1], [9, 9]), "cpu",
                                        deterministic=True).flags == ATTN_DETERMINISTIC


def test_block_bytes_is_layers_times_kv_times_block():
    L = _lib.lib()
    p = pool(num_layers=28, num_kv_heads=4, head_dim=128)
    assert L.vapi_kv_block_bytes(p) == 917504  # BASELINE config 4's block
    assert L.vapi_kv_block_bytes(p) == oracle.block_bytes(28, 16, 4, 128, 2)
    # lib.rs:143-157: 1 GiB holds 1024 blocks of 16 layers x 8 x 64 bf16, BS 32.
    assert (1 << 30) // L.vapi_kv_block_bytes(
        pool(num_layers=16, num_kv_heads=8, head_dim=64, block_size=32)) == 1024


def test_pack_block_tables_matches_the_reference():
    L = _lib.lib()
    for tables in ([[0, 1, 2], [7]], [[], [3, 4]], [[5]], []):
        offs, data = oracle.ragged(tables)
        width = max([len(t) for t in tables] + [1])
        out = np.zeros(max(len(tables), 1) * width, np.uint32)
        u32p = ctypes.POINTER(ctypes.c_uint32)
        w = L.vapi_pack_block_tables(len(tables), offs.ctypes.data_as(u32p),
                                     data.ctypes.data_as(u32p), out.ctypes.data_as(u32p),
                                     out.size)
        assert w == width
        if tables:
            np.testing.assert_array_equal(out[:len(tables) * w].reshape(len(tables), w),
                                          oracle.pack_block_tables(tables))
    out = np.zeros(2, np.uint32)
    offs, data = oracle.ragged([[0, 1, 2]])
    u32p = ctypes.POINTER(ctypes.c_uint32)
    assert L.vapi_pack_block_tables(1, offs.ctypes.data_as(u32p), data.ctypes.data_as(u32p),
                                    out.ctypes.data_as(u32p), 2) == _lib.ESPACE


def good_batch():
    # Two sequences over 4-slot blocks: a 3-token prefill on 5 cached keys and a decode.
    return ForwardBatch(tokens=[1, 2, 3, 4], positions=[5, 6, 7, 5],
                        cu_seqlens_q=[0, 3, 4], cu_seqlens_k=[0, 8, 14],
                        slot_mapping=[21, 22, 23, 1], block_tables=[[4, 5], [7, 0]],
                        logits_indices=[2, 3], max_seqlen_q=3, max_seqlen_k=8)


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b.slot_mapping.__setitem__(3, 22), "two tokens both write KV cache slot 22"),
    (lambda b: b.block_tables.__setitem__(0, [4]), "needs 2 blocks to cover 8 keys"),
    (lambda b: b.positions.__setitem__(1, 9), "non-contiguous positions"),
    (lambda b: b.cu_seqlens_k.__setitem__(2, 7), "not monotonic"),
    (lambda b: b.cu_seqlens_k.__setitem__(1, 2), "3 query tokens but only 2 key tokens"),
    (lambda b: b.block_tables.__setitem__(1, [7, 8]), "references block 8 of 8"),
    (lambda b: b.slot_mapping.__setitem__(3, 40), "past the end of the cache"),
    (lambda b: b.logits_indices.append(4), "logits index 4"),
    (lambda b: b.cu_seqlens_q.__setitem__(0, 1), "must start at 0"),
])
def test_validate_rejects_what_the_reference_rejects(mutate, msg):
    b = good_batch()
    b.validate(8, 4)
    mutate(b)
    with pytest.raises((_lib.VapiKvError, ValueError), match=msg):
        b.validate(8, 4)


def test_validate_checks_the_host_side_lengths_too():
    b = good_batch()
    b.positions.pop()
    with pytest.raises(ValueError, match="positions"):
        b.validate(8, 4)
    b = good_batch()
    b.block_tables.pop()
    with pytest.raises(ValueError, match="block tables"):
        b.validate(8, 4)


def test_the_workloads_have_the_baseline_shapes():
    w0 = workload.config0_decode_small()
    assert w0.batch == 8 and 64 <= w0.lens.min() and w0.lens.max() <= 512
    assert len({b for t in w0.tables for b in t}) == sum(len(t) for t in w0.tables)
    w1 = workload.config1_append()
    assert w1.n_tokens == 4096 and w1.n_tokens - w1.n_valid == 205
    valid = w1.slots[w1.slots != workload.SKIP]
    assert len(np.unique(valid)) == len(valid) and valid.max() < 65536 * 16
    w2 = workload.config2_decode()
    assert w2.batch == 64 and w2.lens.min() >= 256 and w2.lens.max() <= 8192
    assert 1e5 < w2.lens.sum() < 3e5
    assert sum(len(t) for t in w2.tables) <= 32768
    w3 = workload.config3_prefill()
    assert w3.batch == 32 and w3.num_blocks == 4608
    assert all(np.array_equal(w3.tables[0][:128], w3.tables[7][:128]) for _ in [0])
    assert not np.array_equal(w3.tables[0][:128], w3.tables[8][:128])
    assert abs(w3.flops() - 1.031e12) / 1.031e12 < 1e-3
    w4 = workload.config4_block_ops()
    assert w4.pairs.shape == (2048, 2) and len(w4.swap_ids) == 4096
    assert not set(w4.pairs[:, 1]) & set(w4.pairs[:, 0])


def test_block_bytes_walks_a_pool_chain_and_k_only_pools_count_k():
    """A cache whose layers differ is a chain of pools: block_bytes sums
    them (backend.rs:695-708), a K-only pool (a rows layer, v NULL) counts
    its K alone. Checked against the oracle's sum over the same buffers."""
    L = _lib.lib()
    a = pool(num_layers=2, num_kv_heads=2, head_dim=64)
    rows = pool(num_layers=1, num_kv_heads=1, head_dim=40)
    rows.v = None
    b = pool(num_layers=3, num_kv_heads=4, head_dim=128)
    a.next = ctypes.addressof(rows)
    rows.next = ctypes.addressof(b)
    k = [np.zeros((1, 16, 2, 64), np.uint16)] * 2 + [np.zeros((1, 16, 1, 40), np.uint16)] + \
        [np.zeros((1, 16, 4, 128), np.uint16)] * 3
    v = [np.zeros((1, 16, 2, 64), np.uint16)] * 2 + [None] + \
        [np.zeros((1, 16, 4, 128), np.uint16)] * 3
    assert L.vapi_kv_block_bytes(ctypes.byref(a)) == oracle.cache_block_bytes(k, v)
    assert L.vapi_kv_block_bytes(ctypes.byref(rows)) == 16 * 40 * 2 + 3 * 2 * 16 * 4 * 128 * 2


def test_a_chain_of_pools_on_different_blocks_is_an_error():
    L = _lib.lib()
    a = pool(num_layers=1)
    b = pool(num_layers=1, num_blocks=7)
    a.next = ctypes.addressof(b)
    pairs = (ctypes.c_uint32 * 2)(0, 1)
    assert L.vapi_kv_copy_blocks(ctypes.byref(a), pairs, 1, None) == _lib.EINVAL
    assert b"chained pool" in L.vapi_kv_last_error()
    # A K-only pool refuses V rows.
    k = pool(num_layers=1)
    k.v = None
    assert L.vapi_kv_append(ctypes.byref(k), 0, 1, 1, 1, 1, None) == _lib.EINVAL
    assert b"K-only" in L.vapi_kv_last_error()


def test_a_c_program_uses_the_library_through_the_header(tmp_path):
    """tests/c_consumer.c: the header compiles as C11 (-Wall -Werror) and a
    C program links libvapi_kv.so and runs the host-side calls, as a Rust
    -sys crate or any other FFI would bind them."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no gcc")
    root = Path(__file__).resolve().parents[1]
    lib_dir = _lib.LIB_PATH.parent
    exe = tmp_path / "c_consumer"
    subprocess.run([gcc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", str(root / "include"),
                    str(root / "tests" / "c_consumer.c"), "-o", str(exe), f"-L{lib_dir}",
                    "-lvapi_kv", f"-Wl,-rpath,{lib_dir}"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all checks passed" in res.stdout


def test_the_build_refuses_a_prefill_kernel_that_spills():
    """The prefill ring's explicit vmcnt waits count only its direct loads;
    the build parses the compiler's resource remarks and refuses scratch."""
    from vapi_amd import build as b
    ok = ("x: remark: Function Name: _ZN2vk19paged_prefill_tiledINS_6bf16_tE [-R]\n"
          "x: remark:     ScratchSize [bytes/lane]: 0 [-R]\n")
    b._check_no_scratch(Path("attn_prefill.hip"), ok)
    with pytest.raises(RuntimeError, match="scratch"):
        b._check_no_scratch(Path("attn_prefill.hip"), ok.replace(": 0 [", ": 16 ["))
    b._check_no_scratch(Path("kv_ops.hip"), ok.replace(": 0 [", ": 16 ["))  # not checked


def test_the_valu_workspace_follows_its_key_chunks():
    """Head dims without an MFMA kernel (82 here: not a multiple of 4) run the
    VALU kernel: keys split into chunks of 512, halved down to 64 while the
    launch has fewer than 512 workgroups; a call whose keys fit one chunk
    needs no workspace."""
    L = _lib.lib()
    f32 = pool(dtype=_lib.F32, num_kv_heads=8, head_dim=82)
    # 64 rows x 8 kv heads = 512 row tiles: 512-key chunks, one chunk.
    assert L.vapi_paged_attention_workspace_size(f32, 64, 32, 1, 512) == 0
    # Two sequences: 16 tiles, so 64-key chunks (8 of them for 512 keys).
    need = L.vapi_paged_attention_workspace_size(f32, 2, 32, 1, 512)
    tiles, chunks = 2 * 8, 8
    assert need == 256 + tiles * chunks * 16 * (82 + 2) * 4
    assert L.vapi_paged_attention_workspace_size(f32, 2, 32, 1, 64) == 0


def test_f32_decode_and_wide_groups_size_the_decode_workspace():
    """An f32 pool's call sizes the decode stream's workspace
    (balance block, ranges, f32 partials), as a bf16 pool's does; so does a
    group of 32 query heads per kv head (two virtual kv heads of 16), whose
    partials are as large as 32 heads' and whose segments twice as many."""
    L = _lib.lib()
    f32 = pool(dtype=_lib.F32, num_kv_heads=8, head_dim=128)
    bf16 = pool(dtype=_lib.BF16, num_kv_heads=8, head_dim=128)
    a = L.vapi_paged_attention_workspace_size(f32, 64, 32, 1, 4096)
    b = L.vapi_paged_attention_workspace_size(bf16, 64, 32, 1, 4096)
    assert a == b and a > 0
    # f32 prefill rows run without a key split: the decode's part only.
    assert L.vapi_paged_attention_workspace_size(f32, 64, 32, 512, 4096) == a
    one = pool(dtype=_lib.BF16, num_kv_heads=1, head_dim=128)
    two = pool(dtype=_lib.BF16, num_kv_heads=2, head_dim=128)
    # G = 32 on one kv head is decoded as two kv heads of 16: the same
    # workspace as 32 heads over two kv heads.
    assert (L.vapi_paged_attention_workspace_size(one, 64, 32, 1, 4096) ==
            L.vapi_paged_attention_workspace_size(two, 64, 32, 1, 4096))
    # G = 128 on one kv head is decoded as eight kv heads of 16: the same
    # workspace as 128 heads over eight kv heads.
    eight = pool(dtype=_lib.BF16, num_kv_heads=8, head_dim=128)
    assert (L.vapi_paged_attention_workspace_size(one, 64, 128, 1, 4096) ==
            L.vapi_paged_attention_workspace_size(eight, 64, 128, 1, 4096))
    # G = 71 (Falcon-7B's 71 query heads over one kv head) is decoded as five
    # kv heads of 15 (the last serving 11): the workspace of 75 heads over
    # five kv heads.
    five = pool(dtype=_lib.BF16, num_kv_heads=5, head_dim=128)
    assert (L.vapi_paged_attention_workspace_size(one, 64, 71, 1, 4096) ==
            L.vapi_paged_attention_workspace_size(five, 64, 75, 1, 4096))
    # G = 257 has no split into at most 16 parts: the VALU kernel, which
    # needs no decode workspace for short contexts.
    assert L.vapi_paged_attention_workspace_size(one, 64, 257, 1, 64) == 0


def test_padded_head_dims_size_the_workspace_of_the_next_kernel_dim():
    """A 16-bit pool at a head_dim that is a multiple of 8 below 256 runs the
    decode stream and the prefill kernel at the next of 64, 128 and 256:
    decode-only and prefill calls ask for that dim's workspace (the
    prefill's key-split partials hold its columns), and a head_dim that is
    not a multiple of 8 stays on the VALU kernel."""
    L = _lib.lib()
    for hd, kd in ((80, 128), (96, 128), (48, 64), (160, 256), (248, 256)):
        padded = pool(dtype=_lib.BF16, num_kv_heads=4, head_dim=hd)
        full = pool(dtype=_lib.BF16, num_kv_heads=4, head_dim=kd)
        for q, k in ((1, 4096), (100, 3000), (512, 4096)):
            assert (L.vapi_paged_attention_workspace_size(padded, 2, 16, q, k) ==
                    L.vapi_paged_attention_workspace_size(full, 2, 16, q, k)), (hd, q, k)
    odd = pool(dtype=_lib.BF16, num_kv_heads=4, head_dim=84)
    assert (L.vapi_paged_attention_workspace_size(odd, 2, 16, 100, 3000) !=
            L.vapi_paged_attention_workspace_size(
                pool(dtype=_lib.BF16, num_kv_heads=4, head_dim=128), 2, 16, 100, 3000))
