"""Token sampling on the device (tinytron/inference/sampler.py:6-62).

Same filtering as the reference: fp32 cast, temperature, top-k keeps values
>= the k-th largest, top-p drops sorted tokens whose cumulative probability
exceeds p (the first always kept). With top_k == 1 every token but the
maximum gets probability 0, so sampling is the argmax; that case skips the
softmax and multinomial draw (identical result except between exactly tied
maxima, where the reference picks at random and this picks the first).
"""
from __future__ import annotations

import torch


def filter_logits(logits: torch.Tensor, temperature: float = 1.0, top_k: int | None = None,
                  top_p: float | None = None) -> torch.Tensor:
    if temperature <= 0:
        raise ValueError("temperature must be > 0")
    logits = logits.float()
    if temperature != 1.0:
        logits = logits / temperature
    if top_k is not None and top_k > 0:
        k = min(top_k, logits.size(-1))
        v, _ = torch.topk(logits, k=k, dim=-1)
        min_keep = v[:, -1].unsqueeze(-1)
        logits = torch.where(logits < min_keep, torch.full_like(logits, float("-inf")), logits)
    if top_p is not None and 0 < top_p < 1.0:
        sorted_logits, sorted_indices = torch.sort(logits, descending=True, dim=-1)
        cum_probs = torch.cumsum(torch.softmax(sorted_logits, dim=-1), dim=-1)
        sorted_mask = cum_probs > top_p
        sorted_mask[..., 0] = False
        keep = sorted_logits.masked_fill(sorted_mask, float("-inf"))
        logits = torch.full_like(logits, float("-inf")).scatter_(-1, sorted_indices, keep)
    return logits


def sample_next_token(logits: torch.Tensor, temperature: float = 1.0, top_k: int | None = None,
                      top_p: float | None = None) -> torch.Tensor:
    if top_k == 1 and temperature > 0:
        return torch.argmax(logits, dim=-1)
    probs = torch.softmax(filter_logits(logits, temperature, top_k, top_p), dim=-1)
    return torch.multinomial(probs, num_samples=1).squeeze(-1)


def sample_next_token_with_log_prob(logits: torch.Tensor, temperature: float = 1.0, top_k: int | None = None,
                                    top_p: float | None = None):
    log_probs = torch.log_softmax(filter_logits(logits, temperature, top_k, top_p), dim=-1)
    if top_k == 1:
        token = torch.argmax(log_probs, dim=-1)
    else:
        token = torch.multinomial(log_probs.exp(), num_samples=1).squeeze(-1)
    return token, log_probs.gather(-1, token.unsqueeze(-1)).squeeze(-1)
