"""The paged KV pool and the KV append, host side.

Mirrors vapi's crates/vapi-backend-candle/src/cache.rs:
  PagedKvCache (:12-118), write_kv_to_cache (:136-148) with write_rows's
  checks (:217-240), scatter_index/write_rows_indexed (:165-215) and
  gather_kv (:283-290).
Device memory comes from torch; every byte the pool sees is moved by
libvapi_kv.so kernels.
"""
from __future__ import annotations

from typing import Sequence

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import APPEND_COLD_SOURCE, Pool, check, lib

_DTYPES = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}
_LAYOUTS = {"HND": _lib.LAYOUT_HND, "NHD": _lib.LAYOUT_NHD}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"unsupported KV dtype {dt}") from None


def stream_handle(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


class PagedKvCache:
    """Per-layer K and V block pools in one device slab.

    layout "HND": each layer buffer is [num_blocks, num_kv_heads, block_size,
    head_dim] (a (block, head) tile is contiguous, the MI355X default);
    "NHD": [num_blocks, block_size, num_kv_heads, head_dim], the reference's
    own layout (cache.rs:7-11). Both are addressed by the same flat slot
    block*block_size + offset (cache.rs:113-117).

    block_major: one allocation [num_blocks, 2, num_layers, block] holding,
    per block, every layer's K block then every layer's V block, so that a
    copy-on-write pair is one contiguous run; each layer buffer is then a
    strided view (block stride 2 * num_layers blocks). The default keeps each
    layer's K and V buffers contiguous, as the reference's per-layer tensors.
    """

    def __init__(self, num_layers: int, num_blocks: int, block_size: int,
                 num_kv_heads: int, head_dim: int, dtype: torch.dtype = torch.bfloat16,
                 layout: str = "HND", device: str | torch.device = "cuda",
                 block_major: bool = False):
        if layout not in _LAYOUTS:
            raise ValueError(f"layout must be HND or NHD, not {layout!r}")
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.layout = layout
        self.block_major = block_major
        self.device = torch.device(device)
        block_elems = block_size * num_kv_heads * head_dim
        layer_elems = num_blocks * block_elems
        elt = torch.tensor([], dtype=dtype).element_size()
        shape = ((num_blocks, num_kv_heads, block_size, head_dim) if layout == "HND"
                 else (num_blocks, block_size, num_kv_heads, head_dim))
        if block_major:
            if (block_elems * elt) % 16:
                raise ValueError("a block-major pool needs blocks of a multiple of 16 bytes")
            self._slab = torch.zeros((num_blocks, 2, num_layers, block_elems), dtype=dtype,
                                     device=self.device)
            self.k = [self._slab[:, 0, i].view(shape) for i in range(num_layers)]
            self.v = [self._slab[:, 1, i].view(shape) for i in range(num_layers)]
            base = self._slab.data_ptr()
            self.pool = Pool(
                k=base if num_layers else None,
                v=base + num_layers * block_elems * elt if num_layers else None,
                layer_stride_bytes=block_elems * elt,
                num_layers=num_layers, num_blocks=num_blocks, block_size=block_size,
                num_kv_heads=num_kv_heads, head_dim=head_dim, dtype=dtype_code(dtype),
                layout=_LAYOUTS[layout], block_stride_bytes=2 * num_layers * block_elems * elt)
            return
        # Pad each layer to a multiple of 256 bytes so every layer is aligned.
        pad_elems = (-(layer_elems * elt) % 256) // elt
        self._stride_elems = layer_elems + pad_elems
        self._slab = torch.zeros((2, num_layers, self._stride_elems), dtype=dtype,
                                 device=self.device)
        self.k = [self._slab[0, i, :layer_elems].view(shape) for i in range(num_layers)]
        self.v = [self._slab[1, i, :layer_elems].view(shape) for i in range(num_layers)]
        self.pool = Pool(
            k=self._slab[0, 0].data_ptr() if num_layers else None,
            v=self._slab[1, 0].data_ptr() if num_layers else None,
            layer_stride_bytes=self._stride_elems * elt,
            num_layers=num_layers, num_blocks=num_blocks, block_size=block_size,
            num_kv_heads=num_kv_heads, head_dim=head_dim, dtype=dtype_code(dtype),
            layout=_LAYOUTS[layout])

    def num_slots(self) -> int:
        return self.num_blocks * self.block_size

    def reference_view(self, layer: int, which: str = "k") -> torch.Tensor:
        """Layer buffer as the reference's [nb, bs, kvh, d] (a permuted view
        for HND; call .contiguous() for bytes)."""
        t = (self.k if which == "k" else self.v)[layer]
        return t.permute(0, 2, 1, 3) if self.layout == "HND" else t

    def block_bytes(self) -> int:
        return lib().vapi_kv_block_bytes(self.pool)


class HybridKvCache:
    """A cache whose layers differ: PagedKvCache::with_layouts
    (cache.rs:71-105). `layouts` holds one entry per layer,
    ("kv", num_kv_heads, head_dim) or ("rows", width); a rows layer stores
    one (1, width) K row per token and no V (cache.rs:24-33, 89-96).

    Each layer is its own pool descriptor (a K-only one for rows layers),
    chained in layer order, so the block-level calls (block_bytes,
    export/import, copy_blocks, swap, the spill tier) cover every layer in
    the reference's byte order; per-layer calls take layer_view(l).
    """

    def __init__(self, layouts, num_blocks: int, block_size: int,
                 dtype: torch.dtype = torch.bfloat16, layout: str = "HND",
                 device: str | torch.device = "cuda"):
        if layout not in _LAYOUTS:
            raise ValueError(f"layout must be HND or NHD, not {layout!r}")
        if not layouts:
            raise ValueError("a cache needs at least one layer")
        self.layouts = [tuple(l) for l in layouts]
        self.num_layers = len(self.layouts)
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.dtype = dtype
        self.layout = layout
        self.device = torch.device(device)
        self.k, self.v, self._pools = [], [], []
        for spec in self.layouts:
            if spec[0] == "kv":
                kvh, d = int(spec[1]), int(spec[2])
                has_v = True
            elif spec[0] == "rows":
                kvh, d = 1, int(spec[1])
                has_v = False
            else:
                raise ValueError(f"unknown layer layout {spec!r}")
            shape = ((num_blocks, kvh, block_size, d) if layout == "HND"
                     else (num_blocks, block_size, kvh, d))
            k = torch.zeros(shape, dtype=dtype, device=self.device)
            v = (torch.zeros(shape, dtype=dtype, device=self.device) if has_v
                 else torch.zeros((0,), dtype=dtype, device=self.device))
            self.k.append(k)
            self.v.append(v)
            self._pools.append(Pool(
                k=k.data_ptr(), v=v.data_ptr() if has_v else None, layer_stride_bytes=0,
                num_layers=1, num_blocks=num_blocks, block_size=block_size, num_kv_heads=kvh,
                head_dim=d, dtype=dtype_code(dtype), layout=_LAYOUTS[layout]))
        for a, b in zip(self._pools, self._pools[1:]):
            a.next = ctypes.addressof(b)
        self.pool = self._pools[0]

    def num_slots(self) -> int:
        return self.num_blocks * self.block_size

    def block_bytes(self) -> int:
        return lib().vapi_kv_block_bytes(self.pool)

    def layer_view(self, layer: int) -> "_LayerView":
        """Layer `layer` as a one-layer cache for the per-layer calls."""
        spec = self.layouts[layer]
        kvh, d = (int(spec[1]), int(spec[2])) if spec[0] == "kv" else (1, int(spec[1]))
        return _LayerView(self, layer, kvh, d, spec[0] == "kv")

    def reference_view(self, layer: int, which: str = "k") -> torch.Tensor:
        """Layer buffer as the reference's [nb, bs, kvh, d] (the rows
        layer's V is the reference's empty tensor)."""
        t = (self.k if which == "k" else self.v)[layer]
        if t.dim() < 4:
            return t
        return t.permute(0, 2, 1, 3) if self.layout == "HND" else t


class _LayerView:
    """One layer of a HybridKvCache with the attributes the per-layer calls
    read (its pool descriptor, unchained, as layer 0)."""

    def __init__(self, cache: HybridKvCache, layer: int, kvh: int, d: int, has_v: bool):
        src = cache._pools[layer]
        self.pool = Pool(k=src.k, v=src.v, layer_stride_bytes=0, num_layers=1,
                         num_blocks=src.num_blocks, block_size=src.block_size,
                         num_kv_heads=kvh, head_dim=d, dtype=src.dtype, layout=src.layout)
        self.num_layers = 1
        self.num_blocks = cache.num_blocks
        self.block_size = cache.block_size
        self.num_kv_heads = kvh
        self.head_dim = d
        self.dtype = cache.dtype
        self.device = cache.device
        self.has_v = has_v

    def num_slots(self) -> int:
        return self.num_blocks * self.block_size


def _per_layer(cache, layer: int):
    """(cache, layer) for a per-layer call: a HybridKvCache's layer becomes
    layer 0 of its view."""
    if isinstance(cache, HybridKvCache):
        return cache.layer_view(layer), 0
    return cache, layer


def _k_only(cache, which: str = "k"):
    """A view of `cache`'s pool that moves one buffer only (K, or V as if it
    were K): the single-buffer writes of cache.rs:150-159, 186-204."""
    p = cache.pool
    base = p.k if which == "k" else p.v
    if base is None:
        raise ValueError("this layer stores no V (a rows layer)")
    return Pool(k=base, v=None, layer_stride_bytes=p.layer_stride_bytes,
                num_layers=p.num_layers, num_blocks=p.num_blocks, block_size=p.block_size,
                num_kv_heads=p.num_kv_heads, head_dim=p.head_dim, dtype=p.dtype,
                layout=p.layout, block_stride_bytes=p.block_stride_bytes)


def _slots_host(slot_mapping) -> np.ndarray:
    if isinstance(slot_mapping, torch.Tensor):
        slot_mapping = slot_mapping.cpu().numpy()
    return np.ascontiguousarray(np.asarray(slot_mapping, dtype=np.int64).astype(np.uint32))


def write_kv_to_cache(cache: PagedKvCache, layer: int, k: torch.Tensor, v: torch.Tensor,
                      slot_mapping: Sequence[int] | np.ndarray | torch.Tensor,
                      stream=None) -> None:
    """Write a step's K/V at `slot_mapping` in place (cache.rs:136-148).

    k, v: [n, num_kv_heads, head_dim] device tensors in the cache dtype.
    slot_mapping: host sequence of u32 slots (SLOT_SKIP = padded, skipped).
    Raises ValueError for the reference's error cases (cache.rs:143-145,
    223-240): k/v shape mismatch, token/slot count mismatch, dtype mismatch,
    a slot past the end.
    """
    cache, layer = _per_layer(cache, layer)
    if getattr(cache, "has_v", True) is False:
        raise ValueError("a rows layer stores K only: use write_k_to_cache")
    if tuple(k.shape) != tuple(v.shape):
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ in shape")
    if k.dim() != 3:
        raise ValueError(f"rows must be (n, heads, width), got {tuple(k.shape)}")
    slots = _slots_host(slot_mapping)
    n = k.shape[0]
    if n != slots.shape[0]:
        raise ValueError(f"{n} tokens but {slots.shape[0]} cache slots")
    if k.dtype != cache.dtype or v.dtype != cache.dtype:
        raise ValueError(f"cache is {cache.dtype} but the rows are {k.dtype}")
    if tuple(k.shape[1:]) != (cache.num_kv_heads, cache.head_dim):
        raise ValueError(f"rows {tuple(k.shape)} do not match the cache's "
                         f"({cache.num_kv_heads}, {cache.head_dim})")
    real = slots[slots != _lib.SLOT_SKIP]
    if real.size and int(real.max()) >= cache.num_slots():
        raise ValueError(f"slot {int(real.max())} is past the end of the cache")
    if n == 0:
        return
    dev_slots = torch.from_numpy(slots.view(np.int32)).to(k.device, non_blocking=False)
    write_rows_indexed(cache, layer, k, v, dev_slots, stream=stream)


def write_k_to_cache(cache, layer: int, rows: torch.Tensor,
                     slot_mapping: Sequence[int] | np.ndarray | torch.Tensor,
                     stream=None) -> None:
    """Write a step's rows into the K buffer only (cache.rs:150-159): a rows
    layer's (n, 1, width) rows, or the K of a K/V layer. Same checks as
    write_kv_to_cache."""
    cache, layer = _per_layer(cache, layer)
    if rows.dim() != 3:
        raise ValueError(f"rows must be (n, heads, width), got {tuple(rows.shape)}")
    slots = _slots_host(slot_mapping)
    n = rows.shape[0]
    if n != slots.shape[0]:
        raise ValueError(f"{n} tokens but {slots.shape[0]} cache slots")
    if rows.dtype != cache.dtype:
        raise ValueError(f"cache is {cache.dtype} but the rows are {rows.dtype}")
    if tuple(rows.shape[1:]) != (cache.num_kv_heads, cache.head_dim):
        raise ValueError(f"rows {tuple(rows.shape)} do not match the cache's "
                         f"({cache.num_kv_heads}, {cache.head_dim})")
    real = slots[slots != _lib.SLOT_SKIP]
    if real.size and int(real.max()) >= cache.num_slots():
        raise ValueError(f"slot {int(real.max())} is past the end of the cache")
    if n == 0:
        return
    dev_slots = torch.from_numpy(slots.view(np.int32)).to(rows.device, non_blocking=False)
    rows = rows.contiguous()
    check(lib().vapi_kv_append(_k_only(cache), layer, rows.data_ptr(), None,
                               dev_slots.data_ptr(), n, stream_handle(stream)))


def scatter_index(slot_mapping, device) -> torch.Tensor:
    """The step's slot index on the device, built once and reused by every
    layer (cache.rs:165-174; one u32 per token here, no broadcast needed)."""
    return torch.from_numpy(_slots_host(slot_mapping).view(np.int32)).to(device)


def write_rows_indexed(cache, layer: int, k: torch.Tensor, v: torch.Tensor | None,
                       idx: torch.Tensor, stream=None, cold_source: bool = False) -> None:
    """Append with a prebuilt device slot index (cache.rs:178-215): one
    launch for K and V, or for K alone when v is None (the reference's
    write_rows_indexed, cache.rs:176-185). Out-of-range slots are dropped
    on the device. cold_source: the rows are not in the GPU's caches (read
    with streaming loads, VAPI_APPEND_COLD_SOURCE); same result."""
    cache, layer = _per_layer(cache, layer)
    if idx.dim() != 1 or idx.shape[0] != k.shape[0]:
        raise ValueError(f"scatter index {tuple(idx.shape)} does not match rows "
                         f"{tuple(k.shape)}")
    if idx.dtype not in (torch.int32, torch.uint32):
        raise TypeError("scatter index must be 32-bit")
    k = k.contiguous()
    if v is None:
        check(lib().vapi_kv_append(_k_only(cache), layer, k.data_ptr(), None,
                                   idx.data_ptr(), k.shape[0], stream_handle(stream)))
        return
    v = v.contiguous()
    check(lib().vapi_kv_append_ex(cache.pool, layer, k.data_ptr(), v.data_ptr(),
                                  idx.data_ptr(), k.shape[0],
                                  APPEND_COLD_SOURCE if cold_source else 0,
                                  stream_handle(stream)))


def write_v_rows_indexed(cache, layer: int, v: torch.Tensor, idx: torch.Tensor,
                         stream=None) -> None:
    """write_rows_indexed for the V buffer alone (cache.rs:187-195)."""
    cache, layer = _per_layer(cache, layer)
    if idx.dim() != 1 or idx.shape[0] != v.shape[0]:
        raise ValueError(f"scatter index {tuple(idx.shape)} does not match rows "
                         f"{tuple(v.shape)}")
    if idx.dtype not in (torch.int32, torch.uint32):
        raise TypeError("scatter index must be 32-bit")
    v = v.contiguous()
    check(lib().vapi_kv_append(_k_only(cache, "v"), layer, v.data_ptr(), None,
                               idx.data_ptr(), v.shape[0], stream_handle(stream)))


def write_kv_to_cache_layers(cache: PagedKvCache, layer0: int, k: torch.Tensor,
                             v: torch.Tensor, idx: torch.Tensor, stream=None) -> None:
    """One step's K/V for layers layer0 .. layer0 + L - 1 in one launch: k, v
    are [L, n, num_kv_heads, head_dim] (any common stride between layers,
    rows contiguous within one) and idx a device u32 (int32 view) slot per
    row. Equals L single-layer appends. (A HybridKvCache's layers are
    separate pools: append to them one layer at a time.)"""
    if isinstance(cache, HybridKvCache):
        raise ValueError("a mixed cache's layers are separate pools: append per layer")
    if k.dim() != 4 or tuple(k.shape) != tuple(v.shape):
        raise ValueError(f"k/v must be (layers, n, heads, width), got {tuple(k.shape)} "
                         f"and {tuple(v.shape)}")
    if tuple(k.shape[2:]) != (cache.num_kv_heads, cache.head_dim):
        raise ValueError(f"rows {tuple(k.shape)} do not match the cache's "
                         f"({cache.num_kv_heads}, {cache.head_dim})")
    if k.dtype != cache.dtype or v.dtype != cache.dtype:
        raise ValueError(f"cache is {cache.dtype} but the rows are {k.dtype}")
    if idx.dim() != 1 or idx.shape[0] != k.shape[1] or idx.dtype not in (torch.int32,
                                                                         torch.uint32):
        raise ValueError("idx must hold one 32-bit slot per row")
    if not (k[0].is_contiguous() and v[0].is_contiguous()) or k.stride(0) != v.stride(0):
        raise ValueError("each layer's rows must be contiguous, with one layer stride for K and V")
    check(lib().vapi_kv_append_layers(cache.pool, layer0, k.shape[0], k.data_ptr(), v.data_ptr(),
                                      k.stride(0) * k.element_size(), idx.data_ptr(),
                                      k.shape[1], stream_handle(stream)))


def gather_kv(cache: PagedKvCache, layer: int, block_table, len_k: int,
              which: str = "k", stream=None) -> torch.Tensor:
    """One sequence's K (or V) rows in logical order, [len_k, kvh, d]
    (cache.rs:283-290)."""
    cache, layer = _per_layer(cache, layer)
    if which == "v" and getattr(cache, "has_v", True) is False:
        raise ValueError("a rows layer stores no V")
    table = torch.from_numpy(_slots_host(block_table).view(np.int32)).to(cache.device)
    if len_k > table.shape[0] * cache.block_size:
        raise ValueError(f"len_k {len_k} exceeds {table.shape[0]} blocks")
    out = torch.empty((len_k, cache.num_kv_heads, cache.head_dim), dtype=cache.dtype,
                      device=cache.device)
    if len_k == 0:
        return out
    kp = out.data_ptr() if which == "k" else None
    vp = out.data_ptr() if which == "v" else None
    check(lib().vapi_kv_gather(cache.pool, layer, table.data_ptr(), table.shape[0],
                               len_k, kp, vp, stream_handle(stream)))
    return out
