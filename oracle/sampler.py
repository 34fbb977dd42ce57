"""Sampler oracle in numpy (test infrastructure).

Restates ``filter_logits`` (tinytron/inference/sampler.py:6-36): fp32 cast,
temperature division, top-k keeps values >= the k-th largest (ties kept),
top-p keeps the smallest descending prefix whose cumulative probability
exceeds p (the first token always kept). ``sample_next_token`` (39-48)
samples from softmax of the filtered logits; with top_k = 1 every token but
the maximum gets probability 0, so greedy decode is the argmax (the only
randomness left is between exactly tied maxima).

Pinned by tests/test_oracle_sampler.py: top_k = 1 equals argmax; top-k keeps
exactly k distinct values; top-p against a brute-force prefix search;
log_probs against torch.log_softmax. The device sampler's own draw
(``draw_u64``, ``draw_token``; a counter-based generator, not the reference's
torch.multinomial stream) is pinned by SplitMix64's published output
sequence and by a frequency test against softmax.
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


def log_probs(filtered: np.ndarray) -> np.ndarray:
    """log_softmax of filtered logits (sampler.py:56), in float64; -inf stays -inf."""
    x = np.asarray(filtered, np.float64)
    m = np.max(x, axis=-1, keepdims=True)
    with np.errstate(divide="ignore"):
        return (x - m) - np.log(np.sum(np.exp(x - m), axis=-1, keepdims=True))


# --- the device sampler's draw (this library's own generator, not the
# reference's torch.multinomial stream; pinned by the SplitMix64 published
# output sequence and by a frequency test against softmax) ---

_M64 = (1 << 64) - 1
_GAMMA = 0x9E3779B97F4A7C15


def splitmix64_mix(z: int) -> int:
    """SplitMix64 output function (Steele, Lea & Flood, OOPSLA 2014)."""
    z &= _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def draw_u64(seed: int, offset: int, row: int) -> int:
    """64-bit uniform of (seed, offset, row): three chained SplitMix64 outputs."""
    h = splitmix64_mix(seed + _GAMMA)
    h = splitmix64_mix(h + (offset + 1) * _GAMMA)
    return splitmix64_mix(h + (row + 1) * _GAMMA)


def fixed_masses(filtered_row: np.ndarray) -> list:
    """exp(y - max) of a filtered row as 2^-40 fixed point (fp32 subtraction,
    exp rounded to fp32, scaled by 2^40 and rounded to an integer); 0 where -inf."""
    y = np.asarray(filtered_row, np.float32)
    m = np.float32(np.max(y))
    d = (y - m).astype(np.float32)
    with np.errstate(under="ignore"):
        e = np.exp(d.astype(np.float64)).astype(np.float32)
    return [int(v) for v in np.rint(e * np.float32(2.0 ** 40)).astype(np.float64)]


def draw_token(filtered_row: np.ndarray, u: int) -> int:
    """Inverse CDF in index order: the first token whose running fixed-point
    mass exceeds floor(u * total / 2^64)."""
    w = fixed_masses(filtered_row)
    target = (u * sum(w)) >> 64
    c = 0
    for i, wi in enumerate(w):
        c += wi
        if c > target:
            return i
    raise AssertionError("target beyond the total mass")


def sample(logits: np.ndarray, temperature: float = 1.0, top_k=None, top_p=None, seed: int = 0,
           offset: int = 0) -> np.ndarray:
    """Tokens [B] as the device sampler draws them: the first maximum for
    top_k == 1, else draw_token over filter_logits with draw_u64(seed, offset, row)."""
    f = filter_logits(logits, temperature, top_k, top_p)
    if top_k == 1:
        return greedy(f)
    return np.array([draw_token(f[r], draw_u64(seed, offset, r)) for r in range(f.shape[0])], np.int64)


def top_p_margin(logits: np.ndarray, temperature: float = 1.0, top_k=None, top_p=None) -> np.ndarray:
    """Per row, min |cumulative probability - top_p| over the sorted kept
    tokens: rows where it is tiny sit on a rounding edge of the top-p cut."""
    f = filter_logits(logits, temperature, top_k, None)
    order = np.argsort(-f, axis=-1, kind="stable")
    sx = np.take_along_axis(f, order, axis=-1).astype(np.float64)
    e = np.exp(sx - sx[:, :1])
    cum = np.cumsum(e / e.sum(-1, keepdims=True), axis=-1)
    return np.min(np.abs(cum - top_p), axis=-1)
