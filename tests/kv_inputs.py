"""Seeded inputs shared by the oracle and the GPU parity tests.

Everything is generated on the CPU with numpy from a seed, so the oracle and
the kernels see identical bytes.
"""
from __future__ import annotations

import math

import numpy as np

from oracle import kvcache as okv
from oracle.numerics import f32_to_bf16_bits, bf16_bits_to_f32, round_bf16


def bf16_randn(rng: np.random.Generator, shape, scale: float = 1.0):
    """(bits uint16, values fp32) of N(0, scale^2) rounded to bf16."""
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    bits = f32_to_bf16_bits(x)
    return bits, bf16_bits_to_f32(bits)


def fp8_capacity(max_seq_len, page_size):
    """Token slots of a contiguous fp8 store: whole pages, a multiple of 16 in
    all (its scales group 16 rows; tinytron_amd.cache rounds the same way)."""
    pages = -(-int(max_seq_len) // page_size)
    while (pages * page_size) % 16:
        pages += 1
    return pages * page_size


def contiguous_geometry(batch, num_heads, head_dim, max_seq_len, page_size, fp8=False):
    if fp8:
        max_seq_len = fp8_capacity(max_seq_len, page_size)
    layout = okv.contiguous_layout(batch, num_heads, head_dim, max_seq_len, page_size)
    numel = okv.contiguous_numel(batch, num_heads, head_dim, max_seq_len, page_size)
    return layout, numel


def paged_geometry(seq_capacity, num_heads, head_dim, page_size, rng, extra_pages=3):
    """Random page permutation sized for per-sequence capacities."""
    table, num_pages = okv.random_page_table(seq_capacity, page_size, rng, extra_pages=extra_pages)
    layout = okv.paged_layout(num_pages, num_heads, head_dim, page_size, table)
    layout.capacity = int(table.shape[1] * page_size)
    numel = num_pages * num_heads * page_size * head_dim
    return layout, numel, table, num_pages


def fill_cache_values(layout, numel, batch, lengths, rng, fp8=False, key_gain=None):
    """Random K/V for tokens [0, lengths[b]) of every sequence, NaN elsewhere.
    key_gain(b, L) -> [L] scales sequence b's keys token by token (then
    rounded to bf16), to shape how scores grow along a sequence.

    Returns dict with fp32 value arrays (bf16-representable, or dequantized fp8),
    and the raw storage (bf16 bits or fp8 codes + scales).
    """
    H, D = layout.num_heads, layout.head_dim
    nan_bits = np.uint16(0x7FC0)
    if fp8:
        from oracle.numerics import quantize_e4m3_rows, dequantize_e4m3_rows

        kc = np.full(numel, 0x7F, dtype=np.uint8)
        vc = np.full(numel, 0x7F, dtype=np.uint8)
        kvs = np.full(okv.fp8_scale_numel(numel // D), np.nan, dtype=np.float32)  # K and V scales, 16-row groups
        ks, vs = kvs, kvs[16:]
    else:
        kc = np.full(numel, nan_bits, dtype=np.uint16)
        vc = np.full(numel, nan_bits, dtype=np.uint16)
    keys, values = [], []
    for b in range(batch):
        L = int(lengths[b])
        _, kb = bf16_randn(rng, (L, H, D))
        _, vb = bf16_randn(rng, (L, H, D))
        if key_gain is not None:
            kb = round_bf16(kb * np.asarray(key_gain(b, L), np.float32)[:, None, None])
        if fp8:
            kq, ksc = quantize_e4m3_rows(kb)
            vq, vsc = quantize_e4m3_rows(vb)
            kb = dequantize_e4m3_rows(kq, ksc)
            vb = dequantize_e4m3_rows(vq, vsc)
        offs = layout.token_offsets(b, L)                                   # [L, H]
        idx = (offs[..., None] + np.arange(D, dtype=np.int64)).reshape(-1)  # [L * H * D]
        if fp8:
            kc[idx] = kq.reshape(-1)
            vc[idx] = vq.reshape(-1)
            ks[okv.fp8_scale_index(offs // D).reshape(-1)] = ksc.reshape(-1)
            vs[okv.fp8_scale_index(offs // D).reshape(-1)] = vsc.reshape(-1)
        else:
            kc[idx] = f32_to_bf16_bits(kb).reshape(-1)
            vc[idx] = f32_to_bf16_bits(vb).reshape(-1)
        keys.append(kb)
        values.append(vb)
    out = {"keys": keys, "values": values, "k_store": kc, "v_store": vc}
    if fp8:
        out["k_scale"] = ks
        out["v_scale"] = vs
    return out


def sm_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
