"""Decode-attention oracle in fp64 (test infrastructure).

Restates what the reference computes for one decode step (T = 1):

* GQA: query head h reads KV head ``h // (H_q / H_kv)``; the reference builds
  this with ``repeat_interleave`` before caching (attn.py:66-83, 308-312).
* mask: for T = 1 with past_len = L the mask ``key_pos <= past_len + 0`` is
  all True over the L + 1 cached keys (attn.py:86-95, 332-339), i.e. the new
  token attends to every cached token including itself.
* ``F.scaled_dot_product_attention(q, K, V, attn_mask, dropout_p=0)``
  (attn.py:420-423) = softmax(q K^T / sqrt(D)) V.

The split-K merge follows the associativity of the (max, sum, output) triple
of online softmax: for partials (m_i, l_i, o_i) with o_i = sum exp(s - m_i) v,
m = max m_i, l = sum exp(m_i - m) l_i, o = sum exp(m_i - m) o_i, out = o / l.

Pinned by tests/test_oracle_attention.py: one key gives out = v; equal keys or
q = 0 give mean(V); a dominant key gives that key's v; torch's SDPA in fp64
on random inputs; split == no split.
"""
from __future__ import annotations

import numpy as np


def gqa_head_map(num_q_heads: int, num_kv_heads: int) -> np.ndarray:
    """q head -> kv head (attn.py:71-83); raises like gqa_impl on bad ratios."""
    if num_kv_heads == num_q_heads:
        return np.arange(num_q_heads)
    if num_kv_heads == 1:
        return np.zeros(num_q_heads, dtype=np.int64)
    if num_q_heads % num_kv_heads == 0:
        return np.arange(num_q_heads) // (num_q_heads // num_kv_heads)
    raise ValueError("num_attention_heads must be divisible by num_key_value_heads")


def attend_one(q: np.ndarray, k: np.ndarray, v: np.ndarray, sm_scale: float) -> np.ndarray:
    """q [D], k/v [L, D] -> [D] in fp64."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    s = (k @ q) * sm_scale
    s = s - s.max()
    p = np.exp(s)
    return (p @ v) / p.sum()


def decode_attention(q: np.ndarray, keys: list, values: list, num_kv_heads: int, sm_scale: float | None = None) -> np.ndarray:
    """q [B, H_q, D]; keys[b] / values[b] [L_b, H_kv, D] -> out [B, H_q, D] (fp64)."""
    B, Hq, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(D)
    hmap = gqa_head_map(Hq, num_kv_heads)
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        kb = np.asarray(keys[b], np.float64)
        vb = np.asarray(values[b], np.float64)
        if kb.shape[0] == 0:
            continue
        for h in range(Hq):
            out[b, h] = attend_one(q[b, h], kb[:, hmap[h]], vb[:, hmap[h]], sm_scale)
    return out


def prefill_attention(q: np.ndarray, keys: list, values: list, positions, new_lens, num_kv_heads: int,
                      sm_scale: float | None = None) -> np.ndarray:
    """Causal attention of a prompt chunk over each sequence's cache (attn.py:321-341).

    q [B, H_q, T, D]: query t of sequence b sits at position positions[b] + t
    and exists for t < new_lens[b]; keys[b] / values[b] [>= positions[b] +
    new_lens[b], H_kv, D] hold the cache after the chunk was appended. Query
    (b, t) attends keys 0 .. positions[b] + t (the reference's mask
    key_pos <= past_len + query_pos; is_causal when past_len = 0).
    Returns [B, T, H_q, D] in fp64, zero for t >= new_lens[b]."""
    B, Hq, T, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(D)
    hmap = gqa_head_map(Hq, num_kv_heads)
    out = np.zeros((B, T, Hq, D), dtype=np.float64)
    for b in range(B):
        kb = np.asarray(keys[b], np.float64)
        vb = np.asarray(values[b], np.float64)
        for t in range(int(new_lens[b])):
            p = int(positions[b]) + t
            for h in range(Hq):
                out[b, t, h] = attend_one(q[b, h, t], kb[:p + 1, hmap[h]], vb[:p + 1, hmap[h]], sm_scale)
    return out


def partial_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, sm_scale: float):
    """(m, l, o) of one split in fp64, natural-log domain."""
    s = (np.asarray(k, np.float64) @ np.asarray(q, np.float64)) * sm_scale
    m = s.max()
    p = np.exp(s - m)
    return m, p.sum(), p @ np.asarray(v, np.float64)


def merge_partials(parts) -> np.ndarray:
    ms = np.array([p[0] for p in parts])
    m = ms.max()
    w = np.exp(ms - m)
    l = sum(wi * p[1] for wi, p in zip(w, parts))
    o = sum(wi * p[2] for wi, p in zip(w, parts))
    return o / l


def split_attention(q, k, v, sm_scale: float, split: int) -> np.ndarray:
    parts = [partial_attention(q, k[s:s + split], v[s:s + split], sm_scale) for s in range(0, len(k), split)]
    return merge_partials(parts)
