"""numpy restatement of vapi's candle CPU attention path — TEST
INFRASTRUCTURE ONLY (a timed CPU baseline and a second checker; the product
path never imports it).

paged_attention_cpu (crates/vapi-backend-candle/src/attention.rs:90-163),
step for step as candle runs it: per sequence, gather_kv (cache.rs:280-290:
index_select of the table's blocks, reshape, narrow to len_k) of K and V,
the cast of Q, K, V to f32, repeat_kv (candle-transformers 0.11.0
utils::repeat_kv: each kv head materialised n_rep times), Q K^T times the
scale as a batched matmul (candle's gemm; numpy's BLAS here), the u8 mask
built on the host (k > p, or p - k >= w under a sliding window w) applied as
-inf, softmax over the last dim, P V as a batched matmul, and the transpose
and concatenation of the outputs. The pools hold bf16 bits (uint16, [nb, bs,
kvh, d]), cast to f32 inside the call as candle's to_dtype does.

Checked against the C oracle (oracle.c, attention.rs:90-163 restated) in
tests/test_oracle.py to f32 rounding (max-abs 1e-5).
"""
from __future__ import annotations

import numpy as np


def bf16_bits_to_f32(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) to f32, exactly."""
    return (x.astype(np.uint32) << 16).view(np.float32)


def gather_kv(pool: np.ndarray, table, len_k: int) -> np.ndarray:
    """cache.rs:280-290: the table's blocks in order, flattened to tokens,
    narrowed to len_k: [len_k, kvh, d]."""
    nb, bs, kvh, d = pool.shape
    n = -(-len_k // bs)
    return pool[np.asarray(table[:n], dtype=np.int64)].reshape(n * bs, kvh, d)[:len_k]


def paged_attention(q_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, cu_q, cu_k,
                    tables, scale: float, sliding_window: int | None = None) -> np.ndarray:
    """q_bits [total_q, heads, d], pools [nb, bs, kvh, d], all bf16 bits
    (uint16); returns f32 [total_q, heads, d] (before the cast back to the
    input dtype, attention.rs:162)."""
    heads, d = q_bits.shape[1], q_bits.shape[2]
    kvh = k_bits.shape[2]
    n_rep = heads // kvh
    outs = []
    for i in range(len(cu_q) - 1):
        q0, len_q = int(cu_q[i]), int(cu_q[i + 1]) - int(cu_q[i])
        len_k = int(cu_k[i + 1]) - int(cu_k[i])
        if len_q == 0:
            continue
        qi = np.ascontiguousarray(bf16_bits_to_f32(q_bits[q0:q0 + len_q]).transpose(1, 0, 2))
        ki = bf16_bits_to_f32(gather_kv(k_bits, tables[i], len_k)).transpose(1, 0, 2)
        vi = bf16_bits_to_f32(gather_kv(v_bits, tables[i], len_k)).transpose(1, 0, 2)
        ki = np.ascontiguousarray(np.repeat(ki, n_rep, axis=0))  # repeat_kv
        vi = np.ascontiguousarray(np.repeat(vi, n_rep, axis=0))
        att = np.matmul(qi, np.ascontiguousarray(ki.transpose(0, 2, 1))) * np.float32(scale)
        offset = len_k - len_q
        p = offset + np.arange(len_q)[:, None]
        k = np.arange(len_k)[None, :]
        mask = k > p
        if sliding_window is not None:
            mask |= (k < p) & (p - k >= sliding_window)
        att = np.where(mask.astype(np.uint8)[None].astype(bool), np.float32(-np.inf), att)
        att = att - att.max(axis=-1, keepdims=True)
        np.exp(att, out=att)
        att /= att.sum(axis=-1, keepdims=True)
        outs.append(np.ascontiguousarray(np.matmul(att, vi).transpose(1, 0, 2)))
    if not outs:
        return np.zeros((0, heads, d), np.float32)
    return np.concatenate(outs, 0)
