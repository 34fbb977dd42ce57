"""torch-CPU restatement of the reference decode path (test infrastructure).

This is the reference's own op sequence, restated in code of this repository
(not imported from it), for two uses:

* the CPU baseline that bench.py times on the GPU box's host cores
  ("kind": "port"), and
* end-to-end token parity of the restated engine (tests).

Op sequence of one decode step of one layer (T = 1), as in
tinytron/model/modules/attn.py:378-440 with a paged cache:

    rope_impl(q, k, pos)                       attn.py:397 -> 13-63
    gqa_impl(k, v, H_kv, H_q)                  attn.py:310 -> 66-83
    past_len = cache.append(k, v)              attn.py:325 -> cache.py:34-45
    K, V = cache.get_kv()                      attn.py:326 -> cache.py:47-51
    mask = build_cache_causal_mask(1, L+1, L)  attn.py:333-338 -> 86-95
    y = SDPA(q, K, V, attn_mask=mask)          attn.py:420-423

The cache here is the reference's layout: H_q heads (K/V expanded before the
append, attn.py:308-312), one batch-wide current_length (cache.py:26).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def rope_impl(q, k, position_ids, rope_theta: float = 10000.0):
    """attn.py:13-63."""
    B, H, T, D = q.shape
    assert D % 2 == 0, f"head_dim must be even for RoPE, got {D}"
    inv_freq = 1.0 / (rope_theta ** (torch.arange(0, D, 2, dtype=torch.float32, device=q.device) / D))
    if position_ids.dim() == 1:
        position_ids = position_ids.unsqueeze(0).expand(B, -1)
    elif position_ids.dim() == 2:
        if position_ids.size(0) == 1 and B > 1:
            position_ids = position_ids.expand(B, -1)
        elif position_ids.size(0) != B:
            raise ValueError(f"position_ids batch mismatch: got {position_ids.shape}, expected batch={B}")
    else:
        raise ValueError(f"position_ids must be [T] or [B,T], got shape={position_ids.shape}")
    freqs = torch.einsum("bt,d->btd", position_ids.float(), inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos = emb.cos().unsqueeze(1).to(dtype=q.dtype)
    sin = emb.sin().unsqueeze(1).to(dtype=q.dtype)

    def rotate_half(x):
        half = x.shape[-1] // 2
        return torch.cat((-x[..., half:], x[..., :half]), dim=-1)

    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


def gqa_impl(k, v, num_key_value_heads: int, num_attention_heads: int):
    """attn.py:66-83."""
    if num_key_value_heads == num_attention_heads:
        return k, v
    if num_key_value_heads == 1:
        return k.expand(-1, num_attention_heads, -1, -1), v.expand(-1, num_attention_heads, -1, -1)
    if num_attention_heads % num_key_value_heads == 0:
        rep = num_attention_heads // num_key_value_heads
        return k.repeat_interleave(rep, dim=1), v.repeat_interleave(rep, dim=1)
    raise ValueError("num_attention_heads must be divisible by num_key_value_heads")


def build_cache_causal_mask(query_len: int, key_len: int, past_len: int, device) -> torch.Tensor:
    """attn.py:86-95."""
    query_positions = past_len + torch.arange(query_len, device=device).unsqueeze(-1)
    key_positions = torch.arange(key_len, device=device).unsqueeze(0)
    return key_positions <= query_positions


class LayerPagedKVCache:
    """cache.py:11-51 (dense [B, H, pages, P, D] store, batch-wide length)."""

    def __init__(self, batch_size, num_heads, head_dim, max_seq_len, page_size, device, dtype):
        if page_size <= 0:
            raise ValueError(f"page_size must be positive, got {page_size}")
        self.max_seq_len = max_seq_len
        self.page_size = page_size
        self.current_length = 0
        num_pages = math.ceil(max_seq_len / page_size)
        shape = (batch_size, num_heads, num_pages, page_size, head_dim)
        self._k_pages = torch.empty(shape, device=device, dtype=dtype)
        self._v_pages = torch.empty(shape, device=device, dtype=dtype)
        self._k_flat = self._k_pages.view(batch_size, num_heads, num_pages * page_size, head_dim)
        self._v_flat = self._v_pages.view(batch_size, num_heads, num_pages * page_size, head_dim)

    def append(self, k, v) -> int:
        append_len = k.size(2)
        end = self.current_length + append_len
        if end > self.max_seq_len:
            raise ValueError(
                f"KV cache overflow: requested sequence length {end}, max supported is {self.max_seq_len}"
            )
        self._k_flat[:, :, self.current_length:end, :].copy_(k)
        self._v_flat[:, :, self.current_length:end, :].copy_(v)
        previous = self.current_length
        self.current_length = end
        return previous

    def get_kv(self):
        return self._k_flat[:, :, :self.current_length, :], self._v_flat[:, :, :self.current_length, :]


def decode_attention_step(q, k, v, cache: LayerPagedKVCache, num_kv_heads: int, position: int):
    """One decode step's attention (T = 1) in the reference's op order.

    q [B, H_q, 1, D], k/v [B, H_kv, 1, D] before RoPE; returns y [B, H_q, 1, D].
    """
    pos = torch.arange(position, position + q.size(2), device=q.device).unsqueeze(0)
    q, k = rope_impl(q, k, pos)
    k, v = gqa_impl(k, v, num_kv_heads, q.size(1))
    past_len = cache.append(k, v)
    K, V = cache.get_kv()
    mask = None
    causal = True
    if past_len > 0:
        mask = build_cache_causal_mask(q.size(2), K.size(2), past_len, q.device)
        causal = False
    return F.scaled_dot_product_attention(q, K, V, attn_mask=mask, dropout_p=0.0, is_causal=causal)


def filter_logits(logits, temperature: float = 1.0, top_k=None, top_p=None):
    """sampler.py:6-36 in torch (any device): fp32 cast, temperature, top-k
    (values below the k-th largest -> -inf), top-p over the descending sort
    (the first token always kept). bench.py times this op sequence plus
    softmax + multinomial (sampler.py:39-48) on the GPU as the reference's
    sampler; the numpy oracle.sampler.filter_logits is the checker."""
    if temperature <= 0:
        raise ValueError("temperature must be > 0")
    x = logits.float()
    if temperature != 1.0:
        x = x / temperature
    if top_k is not None and top_k > 0:
        kth = torch.topk(x, k=min(top_k, x.size(-1)), dim=-1).values[:, -1:]
        x = torch.where(x < kth, torch.full_like(x, float("-inf")), x)
    if top_p is not None and 0 < top_p < 1.0:
        vals, order = torch.sort(x, descending=True, dim=-1)
        drop = torch.cumsum(torch.softmax(vals, dim=-1), dim=-1) > top_p
        drop[..., 0] = False
        x = torch.full_like(x, float("-inf")).scatter_(-1, order, vals.masked_fill(drop, float("-inf")))
    return x
