"""CPU restatement of rwkv-tl's token sampling -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker of the HIP sampling
kernel (``rwkv7_sample``); the product never calls it.

* ``sample_logits_ref`` follows ``demo/sampling.py:13-70`` step by step
  (torch on the CPU): penalty ``:44-47``, greedy ``:49-50``, temperature
  ``:52``, top-k ``:54-60``, top-p ``:62-68``, multinomial ``:70``. Pinned by
  the reference's known answers (``test/test_sampling.py:11-59``) and by the
  brute-force checks of ``kept_mask_brute``.
* ``filtered_logits_ref`` is the same function stopped before the draw: the
  logits the multinomial draws from (-inf where dropped), whose softmax is the
  kept distribution.
* ``kept_mask_brute`` restates the two filters from their definitions with
  Python loops over a sorted list (top-k: rank < k or tied with the k-th;
  top-p: mass strictly before the token in descending order <= top_p), for
  small inputs.
* ``philox4x32_10`` is the counter-based generator of Salmon, Moraes, Dror and
  Shaw, "Parallel random numbers: as easy as 1, 2, 3" (SC'11), 10 rounds;
  pinned by the Random123 known-answer vectors.
* ``draw_ref`` is the kernel's draw rule (not the reference's: torch.multinomial
  draws from its own generator stream, so the reference fixes only the
  distribution): key = seed, counter = (offset, row, 0); the first 64 output
  bits r give t = r / 2^64, and the token is the first index whose inclusive
  cumulative kept probability exceeds t.
"""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

_M0, _M1 = 0xD2511F53, 0xCD9E8D57
_W0, _W1 = 0x9E3779B9, 0xBB67AE85
_MASK = 0xFFFFFFFF


def philox4x32_10(ctr: tuple[int, int, int, int], key: tuple[int, int]) -> tuple[int, int, int, int]:
    c = [int(x) & _MASK for x in ctr]
    k0, k1 = (int(x) & _MASK for x in key)
    for _ in range(10):
        p0, p1 = _M0 * c[0], _M1 * c[2]
        c = [(p1 >> 32) ^ c[1] ^ k0, p1 & _MASK, (p0 >> 32) ^ c[3] ^ k1, p0 & _MASK]
        k0, k1 = (k0 + _W0) & _MASK, (k1 + _W1) & _MASK
    return tuple(c)


def draw_uniform(seed: int, offset: int, row: int) -> float:
    """t = r / 2^64 for the 64 bits r the kernel draws for (seed, offset, row)."""
    c = philox4x32_10((offset & _MASK, (offset >> 32) & _MASK, row, 0), (seed & _MASK, (seed >> 32) & _MASK))
    return (c[0] | (c[1] << 32)) / 2.0**64


def _penalize(l: Tensor, repetition_penalty: float, seen: Tensor | None) -> Tensor:
    if repetition_penalty != 1.0 and seen is not None:  # sampling.py:44-47
        lv = l[..., seen]
        l[..., seen] = torch.where(lv > 0, lv / repetition_penalty, lv * repetition_penalty)
    return l


def filtered_logits_ref(
    logits: Tensor,
    *,
    temperature: float,
    top_k: int = 0,
    top_p: float = 1.0,
    repetition_penalty: float = 1.0,
    seen: Tensor | None = None,
) -> Tensor:
    """The float32 logits ``sample_logits`` draws from (temperature > 0)."""
    l = _penalize(logits.detach().to("cpu", torch.float32).clone(), repetition_penalty, seen)
    l = l / temperature  # sampling.py:52
    if top_k > 0:  # sampling.py:54-60
        k = min(top_k, l.shape[-1])
        if k < l.shape[-1]:
            cutoff = torch.topk(l, k, dim=-1).values[..., -1:]
            l = torch.where(l >= cutoff, l, torch.full_like(l, float("-inf")))
    if top_p < 1.0:  # sampling.py:62-68
        probs = torch.softmax(l, dim=-1)
        sorted_probs, sorted_idx = torch.sort(probs, descending=True, dim=-1)
        cum = torch.cumsum(sorted_probs, dim=-1)
        drop = cum - sorted_probs > top_p
        kept = torch.gather(l, -1, sorted_idx)
        vals = torch.where(drop, torch.full_like(kept, float("-inf")), kept)
        l = l.scatter(-1, sorted_idx, vals)
    return l


def sample_logits_ref(
    logits: Tensor,
    *,
    temperature: float | None = None,
    top_k: int = 0,
    top_p: float = 1.0,
    repetition_penalty: float = 1.0,
    seen: Tensor | None = None,
) -> Tensor:
    """``demo/sampling.py:13-70`` on the CPU."""
    if temperature is None or temperature <= 0:  # sampling.py:49-50
        l = _penalize(logits.detach().to("cpu", torch.float32).clone(), repetition_penalty, seen)
        return l.argmax(dim=-1)
    l = filtered_logits_ref(
        logits, temperature=temperature, top_k=top_k, top_p=top_p,
        repetition_penalty=repetition_penalty, seen=seen,
    )
    return torch.multinomial(torch.softmax(l, dim=-1), 1).squeeze(-1)


def kept_probs(l: Tensor) -> np.ndarray:
    """Softmax of filtered logits in float64 (zero where dropped)."""
    x = l.to(torch.float64)
    return torch.softmax(x, dim=-1).numpy()


def draw_ref(probs: np.ndarray, seed: int, offset: int, row: int = 0) -> tuple[int, float, np.ndarray]:
    """The kernel's draw from one row of kept probabilities: (token, t, cdf)."""
    t = draw_uniform(seed, offset, row)
    cdf = np.cumsum(probs)
    cdf = cdf / cdf[-1]
    return int(np.searchsorted(cdf, t, side="right")), t, cdf


def kept_mask_brute(x: list[float], top_k: int = 0, top_p: float = 1.0) -> list[bool]:
    """Both filters from their definitions (x: already penalised and divided
    by the temperature). Python loops; small inputs only."""
    n = len(x)
    kept = [True] * n
    if 0 < top_k < n:
        kth = sorted(x, reverse=True)[top_k - 1]
        kept = [v >= kth for v in x]
    if top_p < 1.0:
        m = max(x[i] for i in range(n) if kept[i])
        q = [float(np.exp(np.float64(x[i]) - m)) if kept[i] else 0.0 for i in range(n)]
        z = sum(q)
        order = sorted(range(n), key=lambda i: -q[i])
        before = 0.0
        for i in order:
            if kept[i] and before / z > top_p:
                kept[i] = False
            before += q[i]
    return kept
