"""Token sampling for ``generate`` (semantics of ``demo/sampling.py:13-70``).

Greedy argmax when ``temperature`` is None or <= 0; otherwise repetition
penalty, temperature, top-k, top-p (nucleus) and a multinomial draw, in that
order, along the last (vocabulary) dimension.
"""

from __future__ import annotations

import torch
from torch import Tensor


def sample_logits(
    logits: Tensor,
    *,
    temperature: float | None = None,
    top_k: int = 0,
    top_p: float = 1.0,
    repetition_penalty: float = 1.0,
    seen: Tensor | None = None,
) -> Tensor:
    """Pick one token id per row of ``logits`` (``[V]`` -> 0-d, ``[B, V]`` -> ``[B]``)."""
    scores = logits.float().clone()
    if repetition_penalty != 1.0 and seen is not None and seen.numel():
        picked = scores[..., seen]
        scores[..., seen] = torch.where(picked > 0, picked / repetition_penalty, picked * repetition_penalty)

    if temperature is None or temperature <= 0:
        return scores.argmax(dim=-1)
    scores = scores / temperature

    vocab = scores.shape[-1]
    if 0 < top_k < vocab:
        kth = torch.topk(scores, top_k, dim=-1).values[..., -1:]
        scores = scores.masked_fill(scores < kth, float("-inf"))

    if top_p < 1.0:
        probs = torch.softmax(scores, dim=-1)
        p_sorted, order = torch.sort(probs, dim=-1, descending=True)
        before = torch.cumsum(p_sorted, dim=-1) - p_sorted  # mass strictly above each entry
        drop_sorted = before > top_p
        drop = torch.zeros_like(drop_sorted).scatter(-1, order, drop_sorted)
        scores = scores.masked_fill(drop, float("-inf"))

    probs = torch.softmax(scores, dim=-1)
    return torch.multinomial(probs, 1).squeeze(-1)
