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
