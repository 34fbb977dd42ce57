"""Pins oracle/sampler.py against closed forms (sampler.py:6-48)."""
import numpy as np
import pytest

from oracle import sampler as osm


def test_temperature_must_be_positive():
    with pytest.raises(ValueError, match="temperature must be > 0"):
        osm.filter_logits(np.zeros((1, 4)), temperature=0.0)


def test_top_k_one_is_argmax():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((16, 1000)).astype(np.float32)
    f = osm.filter_logits(x, top_k=1)
    keep = np.isfinite(f)
    assert np.all(keep.sum(-1) == 1)
    assert np.array_equal(np.argmax(keep, -1), osm.greedy(x))


def test_top_k_keeps_k_largest():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 50)).astype(np.float32)
    f = osm.filter_logits(x, top_k=7)
    for r in range(4):
        kept = np.sort(x[r][np.isfinite(f[r])])
        assert np.array_equal(kept, np.sort(x[r])[-7:])


def test_top_p_brute_force():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 20)).astype(np.float32) * 2
    p = 0.6
    f = osm.filter_logits(x, top_p=p)
    for r in range(3):
        order = np.argsort(-x[r], kind="stable")
        probs = np.exp(x[r][order] - x[r].max())
        probs /= probs.sum()
        cum = np.cumsum(probs)
        # sampler.py:29-31: drop every sorted position whose cumulative
        # probability exceeds p, but always keep the first
        kept = set(order[cum <= p].tolist()) | {int(order[0])}
        assert set(np.flatnonzero(np.isfinite(f[r])).tolist()) == kept


def test_temperature_scales_logits():
    x = np.array([[1.0, 2.0, 4.0]], np.float32)
    assert np.allclose(osm.filter_logits(x, temperature=2.0), x / 2)


def test_splitmix64_published_sequence():
    # SplitMix64 seeded with 1234567 (the generator of Steele, Lea & Flood as
    # published with Vigna's xoshiro seeding code): first five outputs.
    state = 1234567
    out = []
    for _ in range(5):
        state = (state + 0x9E3779B97F4A7C15) & ((1 << 64) - 1)
        out.append(osm.splitmix64_mix(state))
    assert out == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]


def test_draw_u64_distinct_and_uniform():
    us = [osm.draw_u64(7, off, row) for off in range(40) for row in range(50)]
    assert len(set(us)) == len(us)
    top = np.array([u >> 61 for u in us])  # top 3 bits, 8 bins of 2000 draws
    counts = np.bincount(top, minlength=8)
    chi2 = float(((counts - 250.0) ** 2 / 250.0).sum())
    assert chi2 < 30.0  # df 7: p ~ 1e-4


def test_log_probs_matches_torch():
    import torch
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 300)).astype(np.float32) * 3
    f = osm.filter_logits(x, temperature=0.8, top_k=40, top_p=0.9)
    ref = torch.log_softmax(torch.from_numpy(f).double(), dim=-1).numpy()
    got = osm.log_probs(f)
    assert np.array_equal(np.isfinite(got), np.isfinite(ref))
    assert np.allclose(got[np.isfinite(got)], ref[np.isfinite(ref)], atol=1e-12)


def test_draw_token_frequencies_follow_softmax():
    # Inverse-CDF draws over many uniforms reproduce softmax(filtered).
    x = np.array([[2.0, 0.5, 1.0, -1.0, 0.0, 1.5, -np.inf, 0.25]], np.float32)
    f = osm.filter_logits(x)
    p = np.exp(osm.log_probs(f)[0])
    n = 20000
    toks = np.array([osm.draw_token(f[0], osm.draw_u64(11, off, 0)) for off in range(n)])
    counts = np.bincount(toks, minlength=8)
    assert counts[6] == 0
    live = p > 0
    chi2 = float(((counts[live] - n * p[live]) ** 2 / (n * p[live])).sum())
    assert chi2 < 35.0  # df 6: p ~ 1e-5


def test_draw_token_planted_off_by_one_fails():
    # The target is compared with '>' on the running sum: a '>=' variant would
    # pick token 0 for a zero uniform even when token 0 has no mass.
    f = np.array([-np.inf, 0.0, 0.0], np.float32)
    assert osm.draw_token(f, 0) == 1
    assert osm.draw_token(f, (1 << 64) - 1) == 2
    assert osm.draw_token(f, 1 << 63) == 2  # target = total / 2 = mass of token 1: not exceeded there


def test_top_p_equal_values_kept_in_index_order():
    # ten equal logits (p = 0.1 each): top_p 0.35 keeps the first three by index
    x = np.full((1, 10), 0.5, np.float32)
    f = osm.filter_logits(x, top_p=0.35)
    assert np.flatnonzero(np.isfinite(f[0])).tolist() == [0, 1, 2]
