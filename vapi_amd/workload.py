"""Seeded synthetic workloads for the five paged-KV configurations.

Each builder returns host-side index data (block tables, slot mappings,
cumulative lengths) drawn from numpy's PCG64 seeded with 0x5EED0000 + the
configuration index; K/V/Q values are N(0,1) (see fill_normal).

  config 0: Qwen3-0.6B-shaped decode, f32 (16 q / 8 kv heads, d 128, bs 16,
            pool 512 blocks, 8 sequences, len_k ~ U[64, 512]).
  config 1: KV append of one chunked-prefill step at Llama-3-8B KV shape
            (8 kv heads, d 128, bs 16, pool 65,536 blocks; 4,096 tokens in
            16 runs of 256, half block-aligned, 5% padded slots).
  config 2: decode at Llama-3-8B shape (32 q / 8 kv heads, d 128, bs 16,
            64 sequences, len_k log-normal median 2,048 sigma 0.75 clipped to
            [256, 8192], tables from a permutation of a 32,768-block pool).
  config 3: chunked prefill with shared prefixes (32 sequences, 512-token
            query chunk over 4,096 keys; the first 128 blocks are shared by
            groups of 8 sequences).
  config 4: block management at Qwen2.5-7B KV shape (28 layers, 4 kv heads,
            d 128, bs 16, pool 40,000 blocks): 2,048 copy pairs and 4,096
            swapped blocks.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

SKIP = 0xFFFFFFFF


def seed_for(config_index: int) -> int:
    return 0x5EED0000 + config_index


def rng_for(config_index: int) -> np.random.Generator:
    return np.random.default_rng(seed_for(config_index))


def slots_for(table, positions, block_size: int) -> np.ndarray:
    """slot = table[pos // bs] * bs + pos % bs (scheduler.rs:536-541)."""
    pos = np.asarray(positions, dtype=np.int64)
    tab = np.asarray(table, dtype=np.int64)
    return (tab[pos // block_size] * block_size + pos % block_size).astype(np.uint32)


def fill_normal(t: torch.Tensor, seed: int) -> torch.Tensor:
    """Fill a device tensor with N(0,1) from a seeded torch generator (in f32,
    rounded to the tensor's dtype)."""
    g = torch.Generator(device=t.device)
    g.manual_seed(seed)
    flat = t.view(-1)
    chunk = 1 << 26
    for i in range(0, flat.numel(), chunk):
        n = min(chunk, flat.numel() - i)
        flat[i:i + n] = torch.randn(n, generator=g, device=t.device, dtype=torch.float32).to(t.dtype)
    return t


@dataclass
class DecodeShape:
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    lens: np.ndarray            # len_k per sequence (includes the new token)
    tables: list                # per-sequence block ids (ceil(len/bs) each)

    @property
    def batch(self) -> int:
        return len(self.lens)

    def cu_q(self) -> np.ndarray:
        return np.arange(self.batch + 1, dtype=np.uint32)

    def cu_k(self) -> np.ndarray:
        return np.concatenate([[0], np.cumsum(self.lens)]).astype(np.uint32)

    def new_token_slots(self) -> np.ndarray:
        return np.array([slots_for(t, [l - 1], self.block_size)[0]
                         for t, l in zip(self.tables, self.lens)], dtype=np.uint32)

    def max_blocks(self) -> int:
        return max(len(t) for t in self.tables)

    def packed_tables(self) -> np.ndarray:
        w = self.max_blocks()
        out = np.zeros((self.batch, w), dtype=np.uint32)
        for i, t in enumerate(self.tables):
            out[i, :len(t)] = t
            out[i, len(t):] = t[-1]
        return out


def config0_decode_small() -> DecodeShape:
    r = rng_for(0)
    bs, nb = 16, 512
    lens = r.integers(64, 513, size=8)
    need = [(int(l) + bs - 1) // bs for l in lens]
    perm = r.permutation(nb)
    tables, at = [], 0
    for n in need:
        tables.append(perm[at:at + n].astype(np.uint32))
        at += n
    return DecodeShape(16, 8, 128, bs, nb, lens.astype(np.int64), tables)


def config2_decode() -> DecodeShape:
    r = rng_for(2)
    bs, nb, batch = 16, 32768, 64
    lens = np.clip(np.round(np.exp(r.normal(np.log(2048.0), 0.75, size=batch))), 256, 8192)
    lens = lens.astype(np.int64)
    perm = r.permutation(nb)
    tables, at = [], 0
    for l in lens:
        n = (int(l) + bs - 1) // bs
        tables.append(perm[at:at + n].astype(np.uint32))
        at += n
    assert at <= nb
    return DecodeShape(32, 8, 128, bs, nb, lens, tables)


@dataclass
class AppendShape:
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    slots: np.ndarray  # u32 [n_tokens], SKIP for padded

    @property
    def n_tokens(self) -> int:
        return len(self.slots)

    @property
    def n_valid(self) -> int:
        return int((self.slots != SKIP).sum())


def config1_append(n_seqs: int = 16, run: int = 256, num_blocks: int = 65536,
                   pad_frac: float = 0.05) -> AppendShape:
    r = rng_for(1)
    bs = 16
    need = (run + bs - 1) // bs + 1
    perm = r.permutation(num_blocks)
    slots = []
    for s in range(n_seqs):
        table = perm[s * need:(s + 1) * need]
        start = 0 if s % 2 == 0 else int(r.integers(1, bs))
        slots.append(slots_for(table, np.arange(start, start + run), bs))
    slots = np.concatenate(slots).astype(np.uint32)
    n_pad = int(round(pad_frac * len(slots)))
    pad_at = r.choice(len(slots), size=n_pad, replace=False)
    slots[pad_at] = SKIP
    return AppendShape(8, 128, bs, num_blocks, slots)


@dataclass
class PrefillShape:
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    len_q: int
    len_k: int
    tables: list

    @property
    def batch(self) -> int:
        return len(self.tables)

    def cu_q(self) -> np.ndarray:
        return (np.arange(self.batch + 1) * self.len_q).astype(np.uint32)

    def cu_k(self) -> np.ndarray:
        return (np.arange(self.batch + 1) * self.len_k).astype(np.uint32)

    def packed_tables(self) -> np.ndarray:
        return np.stack(self.tables).astype(np.uint32)

    def flops(self) -> float:
        """Causal-exact QK^T + PV flops: 4*d*hq per visible (query, key)."""
        off = self.len_k - self.len_q
        visible = sum(off + j + 1 for j in range(self.len_q))
        return 4.0 * self.head_dim * self.num_heads * visible * self.batch


def config3_prefill(batch: int = 32, len_q: int = 512, len_k: int = 4096,
                    group: int = 8, shared_blocks: int = 128) -> PrefillShape:
    r = rng_for(3)
    bs = 16
    n_groups = (batch + group - 1) // group
    per_seq = len_k // bs
    private = per_seq - shared_blocks
    nb = n_groups * shared_blocks + batch * private
    ids = r.permutation(nb).astype(np.uint32)
    prefixes = [ids[g * shared_blocks:(g + 1) * shared_blocks] for g in range(n_groups)]
    base = n_groups * shared_blocks
    tables = []
    for s in range(batch):
        own = ids[base + s * private: base + (s + 1) * private]
        tables.append(np.concatenate([prefixes[s // group], own]))
    return PrefillShape(32, 8, 128, bs, nb, len_q, len_k, tables)


@dataclass
class BlockOpsShape:
    num_layers: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    pairs: np.ndarray      # [n_pairs, 2] (src, dst)
    swap_ids: np.ndarray   # blocks swapped out
    swap_in_ids: np.ndarray  # different blocks they come back into


def config4_block_ops(num_blocks: int = 40000, n_pairs: int = 2048,
                      n_swap: int = 4096, num_layers: int = 28) -> BlockOpsShape:
    r = rng_for(4)
    perm = r.permutation(num_blocks).astype(np.uint32)
    src = perm[:n_pairs]
    dst = perm[n_pairs:2 * n_pairs]
    swap = perm[2 * n_pairs:2 * n_pairs + n_swap]
    back = perm[2 * n_pairs + n_swap:2 * n_pairs + 2 * n_swap]
    return BlockOpsShape(num_layers, 4, 128, 16, num_blocks, np.stack([src, dst], 1),
                         swap, back)
