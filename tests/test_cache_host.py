"""Host-side logic of the layer caches (no kernels): the reference protocol's
get_kv on ragged lengths, gathers within each sequence's capacity, and the
page-table bookkeeping (cache.py:34-51 of the reference; the pool and ragged
lengths are this build's).

The caches are built on the CPU here: their gathers and writes are plain
torch indexing, so the index arithmetic can be checked without a GPU.
"""
import pytest

torch = pytest.importorskip("torch")

from tinytron_amd import cache as tc


def _fill(cache, lens, H, D, seed=0):
    """Write distinct values for tokens 0..lens[b]-1 of every sequence; return them [B][H, L, D]."""
    g = torch.Generator().manual_seed(seed)
    vals = []
    for b, n in enumerate(lens):
        k = torch.randn(H, n, D, generator=g)
        v = torch.randn(H, n, D, generator=g)
        cache._write_tokens(b, 0, k, v)
        vals.append((k, v))
    cache.set_lengths(lens)
    return vals


def _no_negative_offsets(monkeypatch, cache):
    seen = []
    orig = cache._token_index

    def checked(b, length):
        idx = orig(b, length)
        seen.append(int(idx.min()) if idx.numel() else 0)
        assert idx.numel() == 0 or int(idx.min()) >= 0, f"negative cache offset for sequence {b}"
        return idx

    monkeypatch.setattr(cache, "_token_index", checked)
    return seen


@pytest.mark.parametrize("kind", [torch.float32, tc.FP8])
def test_pool_get_kv_ragged_reads_only_each_sequence(monkeypatch, kind):
    B, H, D, P = 3, 2, 8, 16
    lens = [5, 40, 17]
    caps = [16, 48, 32]  # page counts 1, 3, 2: the table rows end in -1 entries
    table, n_pages = tc.random_page_table(caps, P, seed=7)
    assert (table < 0).any()
    cache = tc.PagedLayerKVCache(table, n_pages, H, D, P, "cpu", kind)
    cache._k.fill_(float("nan")) if kind != tc.FP8 else cache._k.fill_(0x7F)  # NaN codes in every unused slot
    cache._v.fill_(float("nan")) if kind != tc.FP8 else cache._v.fill_(0x7F)
    vals = _fill(cache, lens, H, D)
    seen = _no_negative_offsets(monkeypatch, cache)
    K, V = cache.get_kv()
    assert K.shape == (B, H, max(lens), D) and seen
    for b, n in enumerate(lens):
        k, v = vals[b]
        if kind == tc.FP8:  # per-(token, head) absmax/448 scales: within half an e4m3 step of the value
            assert torch.allclose(K[b, :, :n].float(), k, rtol=0.07, atol=1e-6)
            assert torch.allclose(V[b, :, :n].float(), v, rtol=0.07, atol=1e-6)
        else:
            assert torch.equal(K[b, :, :n], k) and torch.equal(V[b, :, :n], v)
        assert torch.isfinite(K[b].float()).all() and torch.isfinite(V[b].float()).all()
        assert not K[b, :, n:].float().any() and not V[b, :, n:].float().any()


def test_pool_gather_beyond_capacity_raises():
    table, n_pages = tc.random_page_table([16, 64], 16, seed=1)
    cache = tc.PagedLayerKVCache(table, n_pages, 1, 4, 16, "cpu", torch.float32)
    assert cache.capacity_of(0) == 16 and cache.capacity_of(1) == 64
    cache.gather(0, 16)
    with pytest.raises(ValueError):
        cache.gather(0, 17)  # would index the row's -1 entries
    with pytest.raises(ValueError):
        cache._token_index(0, 33)


def test_pool_capacity_counts_leading_pages_only():
    table = torch.tensor([[3, -1, 2], [0, 1, 4]], dtype=torch.int32)
    cache = tc.PagedLayerKVCache(table, 5, 1, 4, 16, "cpu", torch.float32)
    assert cache.capacity_of(0) == 16 and cache.capacity_of(1) == 48


def test_contiguous_get_kv_uniform_is_a_view_and_ragged_pads():
    B, H, D, S, P = 2, 2, 4, 40, 16
    cache = tc.LayerPagedKVCache(B, H, D, S, P, "cpu", torch.float32)
    vals = _fill(cache, [9, 9], H, D)
    K, V = cache.get_kv()
    assert K.data_ptr() == cache._k_flat.data_ptr()  # the reference's view (cache.py:47-51)
    assert torch.equal(K[1], vals[1][0]) and torch.equal(V[0], vals[0][1])
    cache._k_pages.fill_(float("nan"))
    cache._v_pages.fill_(float("nan"))
    vals = _fill(cache, [3, 11], H, D, seed=1)
    K, V = cache.get_kv()
    assert K.shape == (B, H, 11, D)
    assert torch.equal(K[0, :, :3], vals[0][0]) and not K[0, :, 3:].any()
    assert torch.equal(V[1], vals[1][1])


def test_append_protocol_returns_previous_length_and_overflows():
    cache = tc.LayerPagedKVCache(1, 1, 4, 8, 4, "cpu", torch.float32)
    assert cache.append(torch.ones(1, 1, 5, 4), torch.ones(1, 1, 5, 4)) == 0
    assert cache.append(torch.ones(1, 1, 3, 4), torch.ones(1, 1, 3, 4)) == 5
    with pytest.raises(ValueError, match="KV cache overflow: requested sequence length 9, max supported is 8"):
        cache.append(torch.ones(1, 1, 1, 4), torch.ones(1, 1, 1, 4))
