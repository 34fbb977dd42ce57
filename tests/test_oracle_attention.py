"""Pins oracle/attention.py (fp64 decode attention) and the reference path.

Special cases with closed forms, torch's SDPA in fp64 (the reference's own
attention call, attn.py:420-423) on random inputs, the GQA head map against
repeat_interleave (attn.py:79-80), split-K associativity, and the torch-CPU
restatement of one reference decode step against the fp64 oracle.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
import torch.nn.functional as F

from oracle import attention as oat
from oracle import ref_path


def test_single_key_returns_value():
    rng = np.random.default_rng(0)
    q = rng.standard_normal(64)
    k = rng.standard_normal((1, 64))
    v = rng.standard_normal((1, 64))
    assert np.allclose(oat.attend_one(q, k, v, 0.125), v[0], rtol=0, atol=1e-15)


def test_equal_keys_or_zero_query_give_mean_value():
    rng = np.random.default_rng(1)
    v = rng.standard_normal((33, 16))
    k = np.repeat(rng.standard_normal((1, 16)), 33, 0)
    q = rng.standard_normal(16)
    assert np.allclose(oat.attend_one(q, k, v, 0.25), v.mean(0), atol=1e-14)
    k2 = rng.standard_normal((33, 16))
    assert np.allclose(oat.attend_one(np.zeros(16), k2, v, 0.25), v.mean(0), atol=1e-14)


def test_dominant_key_selects_its_value():
    rng = np.random.default_rng(2)
    k = rng.standard_normal((10, 8))
    v = rng.standard_normal((10, 8))
    q = k[4] * 100.0
    k[4] *= 1.0
    out = oat.attend_one(q, k, v, 1.0)
    assert np.allclose(out, v[4], atol=1e-6)


def test_head_map_matches_repeat_interleave():
    for hq, hkv in [(8, 2), (32, 8), (6, 6), (4, 1)]:
        idx = torch.arange(hkv).view(1, hkv, 1, 1).float()
        exp, _ = ref_path.gqa_impl(idx, idx, hkv, hq)
        assert np.array_equal(oat.gqa_head_map(hq, hkv), exp.view(-1).long().numpy())
    with pytest.raises(ValueError, match="divisible"):
        oat.gqa_head_map(6, 4)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 4), (16, 1)])
def test_matches_torch_sdpa_fp64(hq, hkv):
    rng = np.random.default_rng(hq + hkv)
    B, D = 3, 32
    lens = [1, 9, 40]
    q = rng.standard_normal((B, hq, D))
    keys = [rng.standard_normal((L, hkv, D)) for L in lens]
    vals = [rng.standard_normal((L, hkv, D)) for L in lens]
    ours = oat.decode_attention(q, keys, vals, hkv)
    for b, L in enumerate(lens):
        K = torch.from_numpy(keys[b]).permute(1, 0, 2)[None]  # [1, hkv, L, D]
        V = torch.from_numpy(vals[b]).permute(1, 0, 2)[None]
        K, V = ref_path.gqa_impl(K, V, hkv, hq)
        mask = ref_path.build_cache_causal_mask(1, L, L - 1, "cpu")
        y = F.scaled_dot_product_attention(torch.from_numpy(q[b])[None, :, None], K, V, attn_mask=mask)
        assert np.allclose(ours[b], y[0, :, 0].numpy(), rtol=1e-12, atol=1e-12)


def test_decode_mask_is_all_true():
    m = ref_path.build_cache_causal_mask(1, 17, 16, "cpu")
    assert m.shape == (1, 17) and bool(m.all())
    pre = ref_path.build_cache_causal_mask(4, 4, 0, "cpu")
    assert torch.equal(pre, torch.ones(4, 4, dtype=torch.bool).tril())


@pytest.mark.parametrize("split", [1, 7, 16, 100])
def test_split_merge_equals_unsplit(split):
    rng = np.random.default_rng(split)
    q = rng.standard_normal(64)
    k = rng.standard_normal((250, 64)) * 2
    v = rng.standard_normal((250, 64))
    a = oat.attend_one(q, k, v, 0.125)
    b = oat.split_attention(q, k, v, 0.125, split)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-13)


def test_reference_decode_step_matches_oracle():
    """rope -> gqa -> append -> get_kv -> mask -> SDPA (torch fp32) == fp64 oracle."""
    rng = np.random.default_rng(3)
    B, Hq, Hkv, D, L, P = 2, 8, 2, 64, 25, 16
    cache = ref_path.LayerPagedKVCache(B, Hq, D, 64, P, torch.device("cpu"), torch.float32)
    past_k = torch.from_numpy(rng.standard_normal((B, Hkv, L, D)).astype(np.float32))
    past_v = torch.from_numpy(rng.standard_normal((B, Hkv, L, D)).astype(np.float32))
    cache.append(*ref_path.gqa_impl(past_k, past_v, Hkv, Hq))
    q = torch.from_numpy(rng.standard_normal((B, Hq, 1, D)).astype(np.float32))
    k = torch.from_numpy(rng.standard_normal((B, Hkv, 1, D)).astype(np.float32))
    v = torch.from_numpy(rng.standard_normal((B, Hkv, 1, D)).astype(np.float32))
    y = ref_path.decode_attention_step(q, k, v, cache, Hkv, position=L)
    qr, kr = ref_path.rope_impl(q, k, torch.tensor([[L]]))
    keys = [np.concatenate([past_k[b].permute(1, 0, 2).numpy(), kr[b].permute(1, 0, 2).numpy()], 0) for b in range(B)]
    vals = [np.concatenate([past_v[b].permute(1, 0, 2).numpy(), v[b].permute(1, 0, 2).numpy()], 0) for b in range(B)]
    ref = oat.decode_attention(qr[:, :, 0].numpy(), keys, vals, Hkv)
    assert np.allclose(y[:, :, 0].numpy(), ref, rtol=1e-5, atol=1e-5)
    assert cache.current_length == L + 1


@pytest.mark.parametrize("past", [0, 5])
def test_prefill_matches_torch_sdpa_fp64(past):
    """prefill_attention == the reference's prefill call (attn.py:321-341):
    SDPA with is_causal=True at past_len 0, the key_pos <= past_len + query_pos
    mask (build_cache_causal_mask) otherwise; GQA by repeat_interleave."""
    rng = np.random.default_rng(11 + past)
    B, Hq, Hkv, D, T = 2, 8, 2, 32, 7
    q = rng.standard_normal((B, Hq, T, D))
    keys = [rng.standard_normal((past + T, Hkv, D)) for _ in range(B)]
    vals = [rng.standard_normal((past + T, Hkv, D)) for _ in range(B)]
    ours = oat.prefill_attention(q, keys, vals, [past] * B, [T] * B, Hkv)
    for b in range(B):
        K = torch.from_numpy(keys[b]).permute(1, 0, 2)[None]
        V = torch.from_numpy(vals[b]).permute(1, 0, 2)[None]
        K, V = ref_path.gqa_impl(K, V, Hkv, Hq)
        qb = torch.from_numpy(q[b])[None]
        if past == 0:
            y = F.scaled_dot_product_attention(qb, K, V, is_causal=True)
        else:
            mask = ref_path.build_cache_causal_mask(T, past + T, past, "cpu")
            y = F.scaled_dot_product_attention(qb, K, V, attn_mask=mask)
        assert np.allclose(ours[b], y[0].permute(1, 0, 2).numpy(), rtol=1e-12, atol=1e-12)


def test_prefill_single_token_equals_decode_and_ragged_rows_are_zero():
    rng = np.random.default_rng(4)
    B, Hq, Hkv, D = 3, 4, 2, 16
    past = [3, 0, 9]
    q = rng.standard_normal((B, Hq, 2, D))
    keys = [rng.standard_normal((p + 2, Hkv, D)) for p in past]
    vals = [rng.standard_normal((p + 2, Hkv, D)) for p in past]
    out = oat.prefill_attention(q, keys, vals, past, [1, 2, 1], Hkv)
    dec = oat.decode_attention(q[:, :, 0], [k[:p + 1] for k, p in zip(keys, past)],
                               [v[:p + 1] for v, p in zip(vals, past)], Hkv)
    assert np.allclose(out[:, 0], dec, rtol=1e-13, atol=1e-13)
    assert np.all(out[0, 1] == 0) and np.all(out[2, 1] == 0) and np.any(out[1, 1] != 0)
