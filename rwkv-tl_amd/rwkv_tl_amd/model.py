"""The RWKV7 model interface (drop-in for ``demo._rwkv7_abc.RWKV7Model``).

``decode`` / ``prefill`` are abstract; ``forward`` and ``generate`` are built
on them exactly as in ``demo/_rwkv7_abc.py:41-89``. Models are stateless: the
``State`` is passed in and returned.
"""

from __future__ import annotations

from abc import ABC, abstractmethod

import torch
from torch import Tensor

from .sampling import Sampler
from .state import State
from .weight import RWKV7Weight


class RWKV7Model(ABC):
    """Common inference interface of every RWKV7 implementation."""

    def __init__(self, w: RWKV7Weight, *args, **kwargs) -> None:
        self.w = w
        self.L = w.L
        self.C = w.C
        self.N = 64
        self.H = self.C // self.N

    @abstractmethod
    def decode(self, token: Tensor, S: State) -> tuple[Tensor, State]:
        """Advance one token; returns ``(logits, state)``."""

    @abstractmethod
    def prefill(self, tokens: Tensor, S: State) -> State:
        """Consume a token sequence, updating ``S`` in place; returns ``S``."""

    def new_state(self, batch: int | None = None) -> State:
        """A zero state of this model's shape on its device."""
        return State(self.L, self.C, self.N, device=self.w.device, dtype=self.w.dtype, batch=batch)

    def generate(
        self,
        tokens: list[int] | Tensor,
        S: State,
        max_tokens: int = 32,
        *,
        temperature: float | None = None,
        top_k: int = 0,
        top_p: float = 1.0,
        repetition_penalty: float = 1.0,
    ) -> tuple[list[int], State]:
        """Prompt with ``tokens`` and sample ``max_tokens`` more (``_rwkv7_abc.py:41-72``).

        Each step is decode plus one sampling launch that writes the token into
        a device buffer the next decode reads: no host sync until the final
        ``tolist()``. Repetition penalty applies to the generated tokens only,
        as in the reference (``seen=out``). A model with ``raise_if_aborted``
        (the HIP models, also behind ``HIPGraph``) checks after that sync that
        none of its persistent kernel launches gave up."""
        if isinstance(tokens, Tensor) and tokens.ndim != 1:
            raise ValueError(f"Expected 1D token sequence, got {tokens.shape}")
        if isinstance(tokens, list):
            tokens = torch.as_tensor(tokens, device=self.w.device)
        S = self.prefill(tokens[:-1], S)  # raises on a one-token prompt, as the reference does
        out = torch.empty(max_tokens, dtype=torch.long, device=self.w.device)
        sampler = Sampler(
            self.w.head.shape[0], self.w.device, temperature=temperature, top_k=top_k, top_p=top_p,
            repetition_penalty=repetition_penalty,
        )
        token = tokens[-1]
        for i in range(max_tokens):
            logits, S = self.decode(token, S)
            sampler(logits, out[i : i + 1])
            token = out[i]
        ids = out.tolist()
        check = getattr(self, "raise_if_aborted", None)
        if check is not None:
            check()
        return ids, S

    def forward(self, tokens: Tensor, S: State) -> tuple[Tensor, State]:
        """``prefill(tokens[:-1])`` then ``decode(tokens[-1])`` (``_rwkv7_abc.py:74-89``)."""
        if tokens.ndim == 0 and tokens.numel() == 1:
            return self.decode(tokens, S)
        if tokens.ndim != 1:
            raise ValueError(f"Expected 1D token sequence, got {tokens.shape}")
        if tokens.numel() == 1:
            return self.decode(tokens[0], S)
        S = self.prefill(tokens[:-1], S)
        return self.decode(tokens[-1], S)
