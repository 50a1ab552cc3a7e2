"""Recurrent state of RWKV7 inference (drop-in for ``rwkv_tl.state.State``).

Same constructor and per-layer layout as ``src/rwkv_tl/state.py:9-61``:
``State(n_layer, n_embd, head_dim, *, device, dtype)`` is a tuple
``(tmix, cmix)`` with ``tmix[i] = {"x": [C] dtype, "rnn": [H, N, N] fp32}`` and
``cmix[i] = {"x": [C] dtype}``, updated in place.

Two additions:

* ``batch=B`` gives every tensor a leading batch dimension (``x [B, C]``,
  ``rnn [B, H, N, N]``) for B independent sequences.
* The per-layer tensors are views into three layer-major arenas
  (``tmix_x [L, B, C]``, ``rnn [L, B, H, N, N]``, ``cmix_x [L, B, C]``), so the
  whole state is handed to the HIP library as three pointers and a HIP graph
  captured against one State replays against it with no copies.
"""

from __future__ import annotations

import torch
from torch import Tensor


class State(tuple):
    """``(tmix, cmix)`` per-layer state; see the module docstring."""

    def __new__(
        cls,
        n_layer: int,
        n_embd: int,
        head_dim: int,
        *,
        device: torch.device | str | None = None,
        dtype: torch.dtype = torch.float16,
        batch: int | None = None,
    ) -> "State":
        if n_embd % head_dim:
            raise ValueError(f"n_embd={n_embd} is not a multiple of head_dim={head_dim}")
        if batch is not None and batch < 1:
            raise ValueError(f"batch must be >= 1, got {batch}")
        H = n_embd // head_dim
        B = 1 if batch is None else batch
        tx = torch.zeros(n_layer, B, n_embd, dtype=dtype, device=device)
        rnn = torch.zeros(n_layer, B, H, head_dim, head_dim, dtype=torch.float32, device=device)
        cx = torch.zeros(n_layer, B, n_embd, dtype=dtype, device=device)

        def pick(t: Tensor, i: int) -> Tensor:
            return t[i, 0] if batch is None else t[i]

        tmix = [{"x": pick(tx, i), "rnn": pick(rnn, i)} for i in range(n_layer)]
        cmix = [{"x": pick(cx, i)} for i in range(n_layer)]
        obj = super().__new__(cls, (tmix, cmix))
        obj.arenas = (tx, rnn, cx)
        obj.batch = batch
        obj.n_layer, obj.n_embd, obj.head_dim = n_layer, n_embd, head_dim
        return obj

    @property
    def tmix(self) -> list[dict[str, Tensor]]:
        return self[0]

    @property
    def cmix(self) -> list[dict[str, Tensor]]:
        return self[1]

    @property
    def batch_size(self) -> int:
        return 1 if self.batch is None else self.batch

    def reset(self) -> None:
        """Zero all state tensors in place (``state.py:57-61``)."""
        for s in self.tmix + self.cmix:
            for tensor in s.values():
                tensor.zero_()

    def arena_intact(self) -> bool:
        """True if every per-layer tensor is still the arena view it started as.

        Code that rebinds ``state["x"]`` instead of updating it in place breaks
        this; the HIP model then works on a copy (see ``RWKV7HIP``).
        """
        tx, rnn, cx = self.arenas
        for i, (t, c) in enumerate(zip(self.tmix, self.cmix)):
            if (
                t["x"].data_ptr() != tx[i].data_ptr()
                or t["rnn"].data_ptr() != rnn[i].data_ptr()
                or c["x"].data_ptr() != cx[i].data_ptr()
            ):
                return False
        return True

    def copy_(self, other: "State") -> "State":
        """Copy every tensor of ``other`` into this state in place."""
        for ds, ss in zip(self[0] + self[1], other[0] + other[1]):
            for k in ds:
                ds[k].copy_(ss[k])
        return self
