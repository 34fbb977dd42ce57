"""Sampler oracle in numpy (test infrastructure).

Restates ``filter_logits`` (tinytron/inference/sampler.py:6-36): fp32 cast,
temperature division, top-k keeps values >= the k-th largest (ties kept),
top-p keeps the smallest descending prefix whose cumulative probability
exceeds p (the first token always kept). ``sample_next_token`` (39-48)
samples from softmax of the filtered logits; with top_k = 1 every token but
the maximum gets probability 0, so greedy decode is the argmax (the only
randomness left is between exactly tied maxima).

Pinned by tests/test_oracle_sampler.py: top_k = 1 equals argmax; top-k keeps
exactly k distinct values; top-p against a brute-force prefix search.
"""
from __future__ import annotations

import numpy as np


def filter_logits(logits: np.ndarray, temperature: float = 1.0, top_k=None, top_p=None) -> np.ndarray:
    if temperature <= 0:
        raise ValueError("temperature must be > 0")
    x = np.asarray(logits, dtype=np.float32)
    if temperature != 1.0:
        x = (x / np.float32(temperature)).astype(np.float32)
    if top_k is not None and top_k > 0:
        k = min(top_k, x.shape[-1])
        kth = -np.sort(-x, axis=-1)[:, k - 1:k]
        x = np.where(x < kth, np.float32(-np.inf), x)
    if top_p is not None and 0 < top_p < 1.0:
        order = np.argsort(-x, axis=-1, kind="stable")
        sx = np.take_along_axis(x, order, axis=-1).astype(np.float64)
        e = np.exp(sx - sx[:, :1])
        probs = e / e.sum(-1, keepdims=True)
        cum = np.cumsum(probs, axis=-1)
        drop = cum > top_p
        drop[:, 0] = False
        sx = np.where(drop, -np.inf, sx)
        out = np.full_like(x, -np.inf)
        np.put_along_axis(out, order, sx.astype(np.float32), axis=-1)
        x = out
    return x


def greedy(logits: np.ndarray) -> np.ndarray:
    """top_k = 1 sampling == argmax (first index among exact ties)."""
    return np.argmax(np.asarray(logits, np.float32), axis=-1)
