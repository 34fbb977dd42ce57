"""Token sampling on the device (tinytron/inference/sampler.py:6-62).

``filter_logits``, ``sample_next_token`` and ``sample_next_token_with_log_prob`` keep the
reference's signatures and run as one kernel launch per call
(``ops.sample_tokens``): fp32 cast, temperature, top-k (values >= the k-th
largest, ties kept), top-p (the shortest descending prefix whose cumulative
probability exceeds p, the first token always kept; equal values ordered by
index), then the draw. With top_k == 1 every token but the maximum has
probability 0, so the token is the argmax (the first of exactly tied maxima,
where the reference picks one at random). Other settings draw from
softmax(filtered) with a counter-based generator keyed by (seed, offset,
row): the reference's distribution, not torch.multinomial's random stream.
Each call takes its seed from torch's default generator (so
``torch.manual_seed`` makes runs repeatable, as in the reference) unless
``manual_seed`` here fixes one.
"""
from __future__ import annotations

import torch

from . import ops


class _SamplerState:
    """Where the device sampler's (seed, offset) come from."""

    def __init__(self):
        self.seed: int | None = None
        self.offset = 0

    def next(self) -> tuple[int, int]:
        if self.seed is None:
            # one 63-bit draw from torch's default (CPU) generator per call:
            # torch.manual_seed makes the sequence of calls repeatable
            return int(torch.randint(0, 2 ** 63 - 1, (1,)).item()), 0
        off = self.offset
        self.offset += 1
        return self.seed, off


_STATE = _SamplerState()


def manual_seed(seed: int | None) -> None:
    """Fix the sampler's seed, call n using offset n (None: draw from torch's generator)."""
    _STATE.seed = None if seed is None else int(seed)
    _STATE.offset = 0


def _rows(logits: torch.Tensor) -> torch.Tensor:
    if logits.dim() != 2:
        raise ValueError(f"logits must be [B, V], got shape={tuple(logits.shape)}")
    if logits.dtype not in ops.SAMPLE_MAX_VOCAB:
        logits = logits.float()
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    return logits


def filter_logits(logits: torch.Tensor, temperature: float = 1.0, top_k: int | None = None,
                  top_p: float | None = None) -> torch.Tensor:
    """sampler.py:6-36: the temperature / top-k / top-p filtered logits [B, V]
    (fp32, -inf where filtered). The kept set comes from the device sampler,
    whose log-probability rows are -inf exactly where these rules filter; the
    kept values are logits.float() / temperature, the reference's own division."""
    if temperature <= 0:
        raise ValueError("temperature must be > 0")
    rows = _rows(logits)
    _, lp = ops.sample_tokens(rows, temperature, top_k, top_p, 0, 0, return_logprobs=True)
    x = rows.float()
    if temperature != 1.0:
        x = x / temperature
    return torch.where(lp == float("-inf"), torch.full_like(x, float("-inf")), x)


def sample_next_token(logits: torch.Tensor, temperature: float = 1.0, top_k: int | None = None,
                      top_p: float | None = None) -> torch.Tensor:
    """sampler.py:39-48: next token ids [B] (int64) from logits [B, V]."""
    if temperature <= 0:
        raise ValueError("temperature must be > 0")
    seed, off = _STATE.next()
    return ops.sample_tokens(_rows(logits), temperature, top_k, top_p, seed, off)


def sample_next_token_with_log_prob(logits: torch.Tensor, temperature: float = 1.0, top_k: int | None = None,
                                    top_p: float | None = None):
    """sampler.py:51-62: token ids [B] and their log-probabilities under the filtered distribution."""
    if temperature <= 0:
        raise ValueError("temperature must be > 0")
    seed, off = _STATE.next()
    return ops.sample_tokens(_rows(logits), temperature, top_k, top_p, seed, off, return_logprob=True)
