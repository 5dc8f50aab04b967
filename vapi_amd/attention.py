"""Paged attention, host side.

Mirrors vapi's crates/vapi-backend-candle/src/attention.rs: pack_block_tables
(:42-62), cu_seqlens (:69-71), PreparedAttention (:237-256) and the CUDA
entry points paged_attention_cuda / _windowed / _prepared (:170-288), and
the step descriptor ForwardBatch (crates/vapi-engine/src/backend.rs:47-204).
The kernels are libvapi_kv.so's vapi_paged_attention.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np
import torch

from ._lib import check, lib
from .cache import PagedKvCache, _per_layer, stream_handle

_u32p = ctypes.POINTER(ctypes.c_uint32)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64).astype(np.uint32))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_u32p)


def _ragged(tables):
    offs = np.zeros(len(tables) + 1, dtype=np.uint32)
    for i, t in enumerate(tables):
        offs[i + 1] = offs[i] + len(t)
    data = _u32(np.concatenate([_u32(t) for t in tables])) if offs[-1] else np.zeros(1, np.uint32)
    return offs, data


@dataclass
class ForwardBatch:
    """One step's descriptor (crates/vapi-engine/src/backend.rs:47-75)."""
    tokens: list = field(default_factory=list)
    positions: list = field(default_factory=list)
    cu_seqlens_q: list = field(default_factory=list)
    cu_seqlens_k: list = field(default_factory=list)
    slot_mapping: list = field(default_factory=list)
    block_tables: list = field(default_factory=list)
    logits_indices: list = field(default_factory=list)
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0

    def batch_size(self) -> int:
        return max(len(self.cu_seqlens_q) - 1, 0)

    def validate(self, num_blocks: int, block_size: int) -> None:
        """ForwardBatch::validate (backend.rs:96-204); raises VapiKvError."""
        n = len(self.tokens)
        if len(self.positions) != n:
            raise ValueError(f"tokens ({n}) and positions ({len(self.positions)}) disagree")
        if len(self.slot_mapping) != n:
            raise ValueError(f"tokens ({n}) and slot_mapping ({len(self.slot_mapping)}) disagree")
        if len(self.cu_seqlens_q) != len(self.cu_seqlens_k):
            raise ValueError("cu_seqlens_q and cu_seqlens_k differ in length")
        b = self.batch_size()
        if len(self.block_tables) != b:
            raise ValueError(f"{len(self.block_tables)} block tables for {b} sequences")
        pos, slots, cq, ck = (_u32(self.positions or [0]), _u32(self.slot_mapping or [0]),
                              _u32(self.cu_seqlens_q or [0]), _u32(self.cu_seqlens_k or [0]))
        offs, data = _ragged(self.block_tables)
        li = _u32(self.logits_indices or [0])
        check(lib().vapi_forward_batch_validate(
            n, _ptr(pos), _ptr(slots), _ptr(cq), _ptr(ck), b, _ptr(offs), _ptr(data),
            _ptr(li), len(self.logits_indices), num_blocks, block_size))


def pack_block_tables(batch: ForwardBatch, device) -> torch.Tensor:
    """[batch, max_blocks] u32 (as int32 bits), rows padded with their own
    last block (attention.rs:42-62)."""
    offs, data = _ragged(batch.block_tables)
    b = len(batch.block_tables)
    width = max([len(t) for t in batch.block_tables] + [1])
    out = np.zeros((max(b, 1), width), dtype=np.uint32)
    w = check(lib().vapi_pack_block_tables(b, _ptr(offs), _ptr(data), _ptr(out), out.size))
    assert w == width
    return torch.from_numpy(out[:b].view(np.int32)).to(device)


def cu_seqlens(values, device) -> torch.Tensor:
    """Cumulative lengths as u32 bits on the device (attention.rs:69-71)."""
    return torch.from_numpy(_u32(values).view(np.int32)).to(device)


ATTN_DETERMINISTIC = 0x1
ATTN_NO_DECODE_ROWS = 0x2


@dataclass
class PreparedAttention:
    """Per-step device inputs, built once per step rather than per layer
    (attention.rs:237-256). Also holds the decode workspace (per-XCD shares
    and split-context partials), reused by every layer of the step, and the
    call flags the host lengths allow: a batch with no decode row (len_q ==
    1) runs the prefill kernel alone (ATTN_NO_DECODE_ROWS); `deterministic`
    freezes the decode's work split so repeated calls are bit-identical.
    `prefill_seqs` lists the sequences with len_q > 1 (device u32), so that
    the prefill grid of a mixed step covers its prefill chunks only
    (vapi_paged_attention_prepared); None covers every sequence."""
    block_table: torch.Tensor
    seqlens_q: torch.Tensor
    seqlens_k: torch.Tensor
    max_seqlen_q: int
    max_seqlen_k: int
    workspace: torch.Tensor | None = None
    flags: int = 0
    prefill_seqs: torch.Tensor | None = None
    n_prefill: int = 0

    @classmethod
    def from_batch(cls, batch: ForwardBatch, device, cache=None, num_heads: int | None = None,
                   deterministic: bool = False) -> "PreparedAttention":
        """With `cache` and `num_heads`, the workspace is sized here for the
        largest attention layer of the cache (a HybridKvCache's layers may
        differ in heads and head_dim), so no layer of the step allocates."""
        cq = np.asarray(batch.cu_seqlens_q, dtype=np.int64)
        lens_q = np.diff(cq) if cq.size > 1 else np.zeros(0, np.int64)
        flags = ATTN_DETERMINISTIC if deterministic else 0
        if lens_q.size and not np.any(lens_q == 1):
            flags |= ATTN_NO_DECODE_ROWS
        pf = np.nonzero(lens_q > 1)[0]
        prep = cls(block_table=pack_block_tables(batch, device),
                   seqlens_q=cu_seqlens(batch.cu_seqlens_q, device),
                   seqlens_k=cu_seqlens(batch.cu_seqlens_k, device),
                   max_seqlen_q=int(batch.max_seqlen_q),
                   max_seqlen_k=int(batch.max_seqlen_k), flags=flags,
                   prefill_seqs=cu_seqlens(pf if pf.size else [0], device),
                   n_prefill=int(pf.size))
        if cache is not None and num_heads is not None:
            prep.reserve(cache, num_heads, device)
        return prep

    def reserve(self, cache, num_heads: int, device) -> None:
        """Allocate (zeroed) the workspace the largest attention layer of
        `cache` needs for this step."""
        from .cache import HybridKvCache
        b = self.seqlens_q.shape[0] - 1
        max_q, max_k = max(self.max_seqlen_q, 1), max(self.max_seqlen_k, 1)
        layers = ([cache.layer_view(l) for l, s in enumerate(cache.layouts) if s[0] == "kv"]
                  if isinstance(cache, HybridKvCache) else [cache])
        need = max(workspace_bytes(c, b, num_heads, max_q, max_k, self.n_prefill_arg())
                   for c in layers)
        if need and (self.workspace is None or self.workspace.numel() < need):
            self.workspace = torch.zeros(need, dtype=torch.uint8, device=device)

    def n_prefill_arg(self) -> int | None:
        """The prefill sequence count the calls pass (None: no list)."""
        return self.n_prefill if self.prefill_seqs is not None else None


def workspace_bytes(cache: PagedKvCache, batch: int, num_heads: int, max_q: int,
                    max_k: int, n_prefill: int | None = None) -> int:
    """vapi_paged_attention_workspace_size, or with `n_prefill` (a call that
    names its prefill sequences) vapi_paged_attention_prepared_workspace_size."""
    if n_prefill is None:
        return lib().vapi_paged_attention_workspace_size(cache.pool, batch, num_heads,
                                                          max_q, max_k)
    return lib().vapi_paged_attention_prepared_workspace_size(cache.pool, batch, n_prefill,
                                                               num_heads, max_q, max_k)


def _workspace(cache, prepared: PreparedAttention, b: int, num_heads: int, max_q: int,
               max_k: int, device):
    need = workspace_bytes(cache, b, num_heads, max_q, max_k, prepared.n_prefill_arg())
    ws = prepared.workspace
    if need and (ws is None or ws.numel() < need):
        # Zero-filled once: a zeroed workspace starts the decode from equal
        # per-XCD shares; later calls carry the shares over. (A step whose
        # layers differ in geometry sizes it up front with reserve(), so that
        # no layer allocates mid-step or inside a captured graph.)
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
        prepared.workspace = ws
    return need, ws


def paged_attention_prepared(q: torch.Tensor, cache: PagedKvCache, layer: int,
                             prepared: PreparedAttention, softmax_scale: float,
                             window_size_left: int | None = None,
                             window_size_right: int | None = 0,
                             out: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """attention.rs:262-288 on libvapi_kv.so. None for a window side means
    unlimited (flash convention); the default right window 0 is causal.
    `cache` may be a HybridKvCache: `layer` then names one of its K/V
    layers."""
    cache, layer = _per_layer(cache, layer)
    if q.dim() != 3 or q.shape[2] != cache.head_dim:
        raise ValueError(f"q must be (tokens, heads, {cache.head_dim}), got {tuple(q.shape)}")
    if q.dtype != cache.dtype:
        raise ValueError(f"q is {q.dtype} but the cache is {cache.dtype}")
    q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    b = prepared.seqlens_q.shape[0] - 1
    num_heads = q.shape[1]
    max_q = max(int(prepared.max_seqlen_q), 1)
    max_k = max(int(prepared.max_seqlen_k), 1)
    need, ws = _workspace(cache, prepared, b, num_heads, max_q, max_k, q.device)
    args = (cache.pool, layer, q.data_ptr(), out.data_ptr(), prepared.seqlens_q.data_ptr(),
            prepared.seqlens_k.data_ptr(), prepared.block_table.data_ptr(), b,
            prepared.block_table.shape[1], max_q, max_k, num_heads, float(softmax_scale),
            -1 if window_size_left is None else int(window_size_left),
            -1 if window_size_right is None else int(window_size_right), prepared.flags)
    tail = (ws.data_ptr() if need else None, need, stream_handle(stream))
    if prepared.prefill_seqs is None:
        check(lib().vapi_paged_attention_ex(*args, *tail))
    else:
        check(lib().vapi_paged_attention_prepared(
            *args, prepared.prefill_seqs.data_ptr(), prepared.n_prefill, *tail))
    return out


def paged_attention_windowed(q, cache, layer, batch: ForwardBatch, softmax_scale,
                             window_size_left=None, window_size_right=0, stream=None):
    """attention.rs:201-232."""
    prepared = PreparedAttention.from_batch(batch, q.device)
    return paged_attention_prepared(q, cache, layer, prepared, softmax_scale,
                                    window_size_left, window_size_right, stream=stream)


def paged_attention(q, cache, layer, batch: ForwardBatch, softmax_scale,
                    sliding_window: int | None = None, stream=None):
    """paged_attention_cuda (attention.rs:170-195): causal, with an optional
    sliding window w mapped to window_size_left = w - 1 (saturating)."""
    wl = None if sliding_window is None else max(int(sliding_window) - 1, 0)
    return paged_attention_windowed(q, cache, layer, batch, softmax_scale, wl, 0,
                                    stream=stream)


def paged_attention_append_prepared(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                    slot_mapping: torch.Tensor, cache: PagedKvCache,
                                    layer: int, prepared: PreparedAttention,
                                    softmax_scale: float,
                                    window_size_left: int | None = None,
                                    window_size_right: int | None = 0,
                                    out: torch.Tensor | None = None,
                                    stream=None) -> torch.Tensor:
    """One layer's cache write and attention in one call (the pair of
    models/qwen.rs:371-391 and models/llama.rs:157-165): the same result as
    write_kv_to_cache(k, v, slot_mapping) then paged_attention_prepared(q),
    in one launch pair fewer for decode batches.

    k, v: [n, num_kv_heads, head_dim] in the cache dtype; slot_mapping: a
    device u32 (int32 view) tensor of n slots.
    """
    cache, layer = _per_layer(cache, layer)
    if q.dim() != 3 or q.shape[2] != cache.head_dim:
        raise ValueError(f"q must be (tokens, heads, {cache.head_dim}), got {tuple(q.shape)}")
    if q.dtype != cache.dtype or k.dtype != cache.dtype or v.dtype != cache.dtype:
        raise ValueError(f"q/k/v must be {cache.dtype}")
    if tuple(k.shape) != tuple(v.shape) or k.dim() != 3 or \
            tuple(k.shape[1:]) != (cache.num_kv_heads, cache.head_dim):
        raise ValueError(f"k/v must be (n, {cache.num_kv_heads}, {cache.head_dim}), "
                         f"got {tuple(k.shape)} and {tuple(v.shape)}")
    if slot_mapping.numel() != k.shape[0] or slot_mapping.element_size() != 4:
        raise ValueError("slot_mapping must hold one 32-bit slot per row")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if out is None:
        out = torch.empty_like(q)
    b = prepared.seqlens_q.shape[0] - 1
    num_heads = q.shape[1]
    max_q = max(int(prepared.max_seqlen_q), 1)
    max_k = max(int(prepared.max_seqlen_k), 1)
    if max_q > 1 and prepared.prefill_seqs is not None and cache.pool.v:
        # (A K-only pool goes to the library call below, which refuses it
        # before writing anything.)
        # A step with prefill rows is not fused (the library runs the append
        # and then the attention); run that pair here so that the attention
        # gets the step's prefill list.
        check(lib().vapi_kv_append(cache.pool, layer, k.data_ptr(), v.data_ptr(),
                                   slot_mapping.data_ptr(), k.shape[0], stream_handle(stream)))
        return paged_attention_prepared(q, cache, layer, prepared, softmax_scale,
                                        window_size_left, window_size_right, out=out,
                                        stream=stream)
    need, ws = _workspace(cache, prepared, b, num_heads, max_q, max_k, q.device)
    check(lib().vapi_paged_attention_append_ex(
        cache.pool, layer, k.data_ptr(), v.data_ptr(), slot_mapping.data_ptr(), k.shape[0],
        q.data_ptr(), out.data_ptr(), prepared.seqlens_q.data_ptr(),
        prepared.seqlens_k.data_ptr(), prepared.block_table.data_ptr(), b,
        prepared.block_table.shape[1], max_q, max_k, num_heads, float(softmax_scale),
        -1 if window_size_left is None else int(window_size_left),
        -1 if window_size_right is None else int(window_size_right), prepared.flags,
        ws.data_ptr() if need else None, need, stream_handle(stream)))
    return out
