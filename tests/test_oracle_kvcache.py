"""Pins oracle/kvcache.py: slot / page arithmetic and the cache protocol.

Closed forms checked by brute force on tiny shapes against the reference's
own storage (a dense [B, H, ceil(S/P), P, D] tensor viewed flat as
[B, H, ceil(S/P)*P, D], cache.py:27-32); the identity page table reproduces
it; a random page table is injective; the H_q-expanded reference cache
equals the H_kv cache under h -> h // rep (repeat_interleave, attn.py:77-81);
append returns the previous length and overflow raises (cache.py:35-45).
"""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import kvcache as okv
from oracle import ref_path


@pytest.mark.parametrize("P", [1, 3, 16, 128])
def test_contiguous_offset_matches_reference_storage(P):
    B, H, S, D = 2, 3, 37, 4
    layout = okv.contiguous_layout(B, H, D, S, P)
    pages = math.ceil(S / P)
    store = np.arange(B * H * pages * P * D).reshape(B, H, pages, P, D)
    flat = store.reshape(B, H, pages * P, D)  # cache.py:31-32
    for b in range(B):
        for h in range(H):
            for t in range(S):
                off = layout.token_offset(b, h, t)
                assert flat[b, h, t, 0] == store.reshape(-1)[off]
                assert store[b, h, t // P, t % P, 0] == off


def test_identity_page_table_reproduces_contiguous():
    B, H, S, D, P = 3, 2, 50, 8, 16
    cont = okv.contiguous_layout(B, H, D, S, P)
    ident = okv.identity_page_table(cont, B)
    paged = okv.CacheLayout(num_heads=H, head_dim=D, page_size=P, seq_stride=0,
                            page_stride=cont.page_stride, head_stride=cont.head_stride,
                            page_table=ident, capacity=S)
    for b in range(B):
        for h in range(H):
            for t in range(S):
                assert paged.token_offset(b, h, t) == cont.token_offset(b, h, t)


def test_vectorized_offsets_equal_scalar_offsets():
    rng = np.random.default_rng(5)
    lens = np.array([1, 16, 17, 100, 33])
    H, D, P = 3, 8, 16
    table, n_pages = okv.random_page_table(lens, P, rng, extra_pages=2)
    for layout in (okv.paged_layout(n_pages, H, D, P, table), okv.contiguous_layout(len(lens), H, D, 112, P)):
        for b, L in enumerate(lens):
            offs = layout.token_offsets(b, int(L))
            assert offs.shape == (L, H)
            for t in range(L):
                for h in range(H):
                    assert offs[t, h] == layout.token_offset(b, h, t)


def test_random_page_table_is_injective_and_in_pool():
    rng = np.random.default_rng(0)
    lens = np.array([1, 16, 17, 100, 33])
    H, D, P = 2, 8, 16
    table, n_pages = okv.random_page_table(lens, P, rng, extra_pages=4)
    layout = okv.paged_layout(n_pages, H, D, P, table)
    seen = set()
    for b, L in enumerate(lens):
        for h in range(H):
            for t in range(L):
                off = layout.token_offset(b, h, t)
                assert 0 <= off and off + D <= n_pages * H * P * D
                assert off not in seen
                seen.add(off)
                j, slot = divmod(t, P)
                assert off == table[b, j] * H * P * D + h * P * D + slot * D


def test_append_and_gather_roundtrip():
    rng = np.random.default_rng(1)
    B, H, D, P = 3, 2, 8, 16
    lens = np.array([5, 40, 17])
    table, n_pages = okv.random_page_table(lens + 3, P, rng)
    layout = okv.paged_layout(n_pages, H, D, P, table)
    cache = np.full(n_pages * H * P * D, -1.0, np.float32)
    x = rng.standard_normal((B, H, 3, D)).astype(np.float32)
    okv.append(cache, layout, x, lens, new_lens=np.array([3, 1, 2]))
    for b, n in enumerate([3, 1, 2]):
        for h in range(H):
            got = okv.gather(cache, layout, b, h, int(lens[b]) + n)
            assert np.array_equal(got[lens[b]:], x[b, h, :n])
            assert np.all(got[:lens[b]] == -1.0)
    # untouched slots of the padding tokens stay untouched
    off = layout.token_offset(1, 0, int(lens[1]) + 1)
    assert np.all(cache[off:off + D] == -1.0)


def test_reference_cache_protocol():
    c = okv.LayerPagedKVCacheRef(2, 3, 4, max_seq_len=10, page_size=4)
    k = np.ones((2, 3, 6, 4), np.float32)
    assert c.append(k, k) == 0
    assert c.current_length == 6
    assert c.append(k[:, :, :4], k[:, :, :4]) == 6
    kk, vv = c.get_kv()
    assert kk.shape == (2, 3, 10, 4)
    with pytest.raises(ValueError, match="KV cache overflow: requested sequence length 11, max supported is 10"):
        c.append(k[:, :, :1], k[:, :, :1])
    with pytest.raises(ValueError, match="page_size must be positive"):
        okv.LayerPagedKVCacheRef(1, 1, 1, 1, 0)


def test_expanded_reference_cache_equals_kv_head_cache():
    """ref_cache[:, h] == build_cache[:, h // rep] for every cached slot."""
    B, Hq, Hkv, D, S, P = 2, 8, 2, 16, 20, 8
    rep = Hq // Hkv
    g = torch.Generator().manual_seed(0)
    k = torch.randn(B, Hkv, 7, D, generator=g)
    v = torch.randn(B, Hkv, 7, D, generator=g)
    ref = ref_path.LayerPagedKVCache(B, Hq, D, S, P, torch.device("cpu"), torch.float32)
    ke, ve = ref_path.gqa_impl(k, v, Hkv, Hq)
    ref.append(ke, ve)
    ours = okv.LayerPagedKVCacheRef(B, Hkv, D, S, P)
    ours.append(k.numpy(), v.numpy())
    rk, rv = ref.get_kv()
    ok, ov = ours.get_kv()
    for h in range(Hq):
        assert np.array_equal(rk[:, h].numpy(), ok[:, h // rep])
        assert np.array_equal(rv[:, h].numpy(), ov[:, h // rep])


def test_fp8_append_writes_codes_and_scales():
    rng = np.random.default_rng(2)
    B, H, D, P = 2, 2, 16, 16
    layout = okv.contiguous_layout(B, H, D, 32, P)
    n = okv.contiguous_numel(B, H, D, 32, P)
    codes = np.zeros(n, np.uint8)
    scales = np.full(okv.fp8_scale_numel(n // D), -1.0, np.float32)
    x = rng.standard_normal((B, H, 1, D)).astype(np.float32)
    okv.append_fp8(codes, scales, layout, x, [3, 9])
    for b, pos in enumerate([3, 9]):
        for h in range(H):
            off = layout.token_offset(b, h, pos)
            row = off // D
            assert scales[32 * (row // 16) + row % 16] == np.float32(np.abs(x[b, h, 0]).max() / np.float32(448))
            assert np.max(codes[off:off + D] & 0x7F) == 0x7E
    assert np.sum(scales != -1.0) == B * H


def test_fp8_scale_slots_group_k_and_v_by_16_rows():
    """Brute force over 0 .. 99 rows: every row's K slot (k) and V slot
    (16 + k in the one array) are distinct from every other slot, lie inside
    fp8_scale_numel, and rows 16g .. 16g + 15 fill exactly the 128-byte line
    [32g, 32g + 32) of the array: K scales first, then V."""
    rows = np.arange(100)
    k = okv.fp8_scale_index(rows)
    v = k + 16
    slots = np.concatenate([k, v])
    assert len(set(slots.tolist())) == 200 and slots.max() < okv.fp8_scale_numel(100) == 224
    for g in range(100 // 16):
        grp = rows[16 * g:16 * g + 16]
        assert set(okv.fp8_scale_index(grp).tolist()) == set(range(32 * g, 32 * g + 16))
        assert set((okv.fp8_scale_index(grp) + 16).tolist()) == set(range(32 * g + 16, 32 * g + 32))
        assert (32 * g * 4) // 128 == ((32 * g + 31) * 4) // 128  # one 128-byte line
