"""KV-cache indexing oracle (test infrastructure).

Restates the reference's cache (tinytron/inference/cache.py:11-51) and the
layouts this build adds:

* contiguous (the reference's ``LayerPagedKVCache``): storage
  ``[B, H, ceil(S/P), P, D]`` with flat view ``[B, H, ceil(S/P)*P, D]``
  (cache.py:27-32); token t of sequence b, head h sits at page t // P,
  slot t % P (cache.py:41-42). The reference keeps one batch-wide
  ``current_length`` (cache.py:26); this build keeps one length per sequence
  and the uniform case is the reference's.
* paged pool (new): storage ``[N_pages, H, P, D]``, page table int32
  ``[B, max_pages]``; token t of sequence b lives in physical page
  ``page_table[b, t // P]`` at slot ``t % P``.

Both reduce to one element offset formula
``base(b, t // P) + h * head_stride + (t % P) * D + d`` with
``base = b * seq_stride + (t // P) * page_stride`` (contiguous) or
``page_table[b, t // P] * page_stride`` (paged). fp8 scales use the same
formula with D collapsed (one fp32 per token and head).

Pinned by tests/test_oracle_kvcache.py: closed-form slot math brute-forced on
tiny shapes, the identity page table reproducing the contiguous layout, the
reference's H_q-expanded cache equal to this build's H_kv cache under the
``h -> h // rep`` map (repeat_interleave, attn.py:77-81), append returning the
previous length and overflow raising (cache.py:35-45).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .numerics import quantize_e4m3_rows


@dataclass
class CacheLayout:
    """Element strides of a cache (slot stride is D, d stride is 1)."""

    num_heads: int
    head_dim: int
    page_size: int
    seq_stride: int          # contiguous only
    page_stride: int
    head_stride: int
    page_table: np.ndarray | None = None  # [B, max_pages] int32 (paged)
    capacity: int = 0        # tokens per sequence

    def token_offset(self, b: int, h: int, t: int) -> int:
        """Element offset of (b, h, t, d=0)."""
        j, slot = divmod(int(t), self.page_size)
        if self.page_table is None:
            base = b * self.seq_stride + j * self.page_stride
        else:
            base = int(self.page_table[b, j]) * self.page_stride
        return base + h * self.head_stride + slot * self.head_dim

    def token_offsets(self, b: int, length: int) -> np.ndarray:
        """token_offset(b, h, t) for every t < length and h, as int64 [length, H]."""
        t = np.arange(int(length), dtype=np.int64)
        j, slot = t // self.page_size, t % self.page_size
        if self.page_table is None:
            base = b * self.seq_stride + j * self.page_stride
        else:
            base = self.page_table[b, j].astype(np.int64) * self.page_stride
        h = np.arange(self.num_heads, dtype=np.int64)
        return (base + slot * self.head_dim)[:, None] + h[None, :] * self.head_stride


def contiguous_layout(batch: int, num_heads: int, head_dim: int, max_seq_len: int, page_size: int) -> CacheLayout:
    """The reference's [B, H, ceil(S/P), P, D] store (cache.py:27-28)."""
    pages = math.ceil(max_seq_len / page_size)
    return CacheLayout(
        num_heads=num_heads,
        head_dim=head_dim,
        page_size=page_size,
        seq_stride=num_heads * pages * page_size * head_dim,
        page_stride=page_size * head_dim,
        head_stride=pages * page_size * head_dim,
        page_table=None,
        capacity=max_seq_len,
    )


def contiguous_numel(batch: int, num_heads: int, head_dim: int, max_seq_len: int, page_size: int) -> int:
    return batch * num_heads * math.ceil(max_seq_len / page_size) * page_size * head_dim


def paged_layout(num_pages: int, num_heads: int, head_dim: int, page_size: int, page_table: np.ndarray) -> CacheLayout:
    """Pool [N_pages, H, P, D] addressed through page_table [B, max_pages]."""
    page_table = np.asarray(page_table, dtype=np.int32)
    return CacheLayout(
        num_heads=num_heads,
        head_dim=head_dim,
        page_size=page_size,
        seq_stride=0,
        page_stride=num_heads * page_size * head_dim,
        head_stride=page_size * head_dim,
        page_table=page_table,
        capacity=page_table.shape[1] * page_size,
    )


def identity_page_table(layout: CacheLayout, batch: int) -> np.ndarray:
    """Page table under which the paged formula equals the contiguous one.

    Keeping the contiguous strides, sequence b's logical page j maps to
    physical page b * (seq_stride // page_stride) + j.
    """
    per_seq = layout.seq_stride // layout.page_stride
    pages = -(-layout.capacity // layout.page_size)
    return (np.arange(batch)[:, None] * per_seq + np.arange(pages)[None, :]).astype(np.int32)


def random_page_table(seq_lens, page_size: int, rng: np.random.Generator, extra_pages: int = 0):
    """Pages assigned in (b, logical page) order from a random permutation.

    Sequence b needs ceil(len_b / P) pages (len_b includes room for the
    appended tokens). Returns (page_table [B, max_pages] int32, num_pages).
    Unused entries hold -1.
    """
    seq_lens = np.asarray(seq_lens, dtype=np.int64)
    need = (seq_lens + page_size - 1) // page_size
    total = int(need.sum()) + extra_pages
    perm = rng.permutation(total).astype(np.int32)
    max_pages = int(need.max()) if len(need) else 0
    table = np.full((len(seq_lens), max(max_pages, 1)), -1, dtype=np.int32)
    k = 0
    for b, n in enumerate(need):
        table[b, :n] = perm[k:k + n]
        k += n
    return table, total


def append(cache: np.ndarray, layout: CacheLayout, x: np.ndarray, positions, new_lens=None) -> None:
    """Write x [B, H, T, D] at slots positions[b] + t (flat cache, in place)."""
    B, H, T, D = x.shape
    for b in range(B):
        n = T if new_lens is None else int(new_lens[b])
        for t in range(n):
            pos = int(positions[b]) + t
            for h in range(H):
                off = layout.token_offset(b, h, pos)
                cache[off:off + D] = x[b, h, t]


def fp8_scale_index(row):
    """Scale slot of a (token, head) row of an fp8 cache, row = element offset
    of d = 0 / head_dim (no counterpart in the reference, whose cache has no
    fp8): rows are grouped by 16, and group g's 16 K scales sit at 32g ..
    32g + 15 of the K-scale array, its 16 V scales at the same slots of the
    V-scale array (one array of 2 x rows floats with the V view 16 slots in)."""
    return row + (row // 16) * 16


def fp8_scale_numel(rows: int) -> int:
    """Floats of the one array that holds K and V scales for `rows` rows."""
    return 2 * (-(-int(rows) // 16) * 16)


def append_fp8(codes: np.ndarray, scales: np.ndarray, layout: CacheLayout, x: np.ndarray, positions, new_lens=None) -> None:
    """Quantize x [B, H, T, D] per (token, head) and write codes and scales
    (scales: the K or the V view, slots by fp8_scale_index)."""
    B, H, T, D = x.shape
    q, s = quantize_e4m3_rows(x)
    for b in range(B):
        n = T if new_lens is None else int(new_lens[b])
        for t in range(n):
            pos = int(positions[b]) + t
            for h in range(H):
                off = layout.token_offset(b, h, pos)
                codes[off:off + D] = q[b, h, t]
                scales[fp8_scale_index(off // D)] = s[b, h, t]


def gather(cache: np.ndarray, layout: CacheLayout, b: int, h: int, length: int) -> np.ndarray:
    """Dense [length, D] view of (b, h) tokens 0..length-1."""
    D = layout.head_dim
    out = np.empty((length, D), dtype=cache.dtype)
    for t in range(length):
        off = layout.token_offset(b, h, t)
        out[t] = cache[off:off + D]
    return out


def gather_scales(scales: np.ndarray, layout: CacheLayout, b: int, h: int, length: int) -> np.ndarray:
    D = layout.head_dim
    return np.array([scales[fp8_scale_index(layout.token_offset(b, h, t) // D)] for t in range(length)],
                    dtype=np.float32)


class LayerPagedKVCacheRef:
    """The reference's LayerPagedKVCache (cache.py:11-51), restated in numpy.

    One batch-wide ``current_length``; ``append`` returns the previous length
    and raises ValueError on overflow with the reference's message.
    """

    def __init__(self, batch_size, num_heads, head_dim, max_seq_len, page_size, dtype=np.float32):
        if page_size <= 0:
            raise ValueError(f"page_size must be positive, got {page_size}")
        self.max_seq_len = max_seq_len
        self.page_size = page_size
        self.current_length = 0
        num_pages = math.ceil(max_seq_len / page_size)
        shape = (batch_size, num_heads, num_pages, page_size, head_dim)
        self.k_pages = np.zeros(shape, dtype=dtype)
        self.v_pages = np.zeros(shape, dtype=dtype)
        self.k_flat = self.k_pages.reshape(batch_size, num_heads, num_pages * page_size, head_dim)
        self.v_flat = self.v_pages.reshape(batch_size, num_heads, num_pages * page_size, head_dim)

    def append(self, k, v) -> int:
        append_len = k.shape[2]
        end = self.current_length + append_len
        if end > self.max_seq_len:
            raise ValueError(
                f"KV cache overflow: requested sequence length {end}, max supported is {self.max_seq_len}"
            )
        self.k_flat[:, :, self.current_length:end, :] = k
        self.v_flat[:, :, self.current_length:end, :] = v
        previous = self.current_length
        self.current_length = end
        return previous

    def get_kv(self):
        return self.k_flat[:, :, :self.current_length, :], self.v_flat[:, :, :self.current_length, :]
