"""HIP-graph replay of decode and small-T prefill (counterpart of ``demo/cuda_graph.py``).

The reference wrapper (``CUDAGraph``, ``demo/cuda_graph.py:61-235``) captures
against a private shadow State and copies the caller's state in and out around
every replay (6L small copies per token plus a ``token.item()`` host sync,
``:123-128``). Here the graph is captured against the caller's own State:
``State`` tensors are views into three arenas, so the graph is keyed by the
arenas' addresses and replays in place. Per replay the only other work is a
device copy of the token ids into the graph's input buffer and a clone of the
logits. A state whose tensors were rebound (not arena views any more) runs
eagerly, and so does a decode step that the library runs as one persistent
kernel (``RWKV7HIP.decode_launches(B) == 1``), where a replay cannot save
launches and would only add the token copy.

Capture is lazy and per exact shape: decode per (state, batch), prefill per
(state, T) for 2 <= T <= ``prefill_graph_max_t``; larger T runs eagerly.
Capturing does not change the caller's state: it is snapshotted before the
warm-up runs and restored afterwards.
"""

from __future__ import annotations

import warnings
from collections import OrderedDict
from typing import Any

import torch
from torch import Tensor

from .model import RWKV7Model
from .state import State
from .weight import RWKV7Weight

__all__ = ["HIPGraph", "make_graph_cls", "wrap_model"]


class HIPGraph(RWKV7Model):
    """Wrap an ``RWKV7HIP`` instance with HIP-graph decode / prefill.

    Args:
        model: the wrapped model (needs ``decode_into`` / ``prefill_into``).
        prefill_graph_max_t: prefill lengths captured as graphs (2..this).
        warmup: eager runs before each capture.
        max_graphs: captured graphs kept (least recently used are dropped).
    """

    def __init__(
        self,
        model: RWKV7Model,
        *,
        prefill_graph_max_t: int = 64,
        warmup: int = 2,
        max_graphs: int = 16,
    ) -> None:
        super().__init__(model.w)
        self.model = model
        self.prefill_graph_max_t = prefill_graph_max_t
        self._warmup = warmup
        self._max_graphs = max_graphs
        self._graphs: OrderedDict[tuple, tuple[Any, ...]] = OrderedDict()
        self._failed: set[tuple] = set()

    def __getattr__(self, name: str) -> Any:
        model = self.__dict__.get("model")
        if model is not None:
            return getattr(model, name)
        raise AttributeError(f"{type(self).__name__!r} has no attribute {name!r}")

    # ------------------------------------------------------------------ #

    @staticmethod
    def _key(kind: str, S: State, n: int) -> tuple:
        return (kind, n) + tuple(a.data_ptr() for a in S.arenas) + (S.batch_size,)

    def _capture(self, key: tuple, S: State, run) -> torch.cuda.CUDAGraph | None:
        if key in self._failed:
            return None
        snapshot = [a.clone() for a in S.arenas]
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(self._warmup):
                    run()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                run()
            torch.cuda.current_stream().wait_stream(side)
        except Exception as e:  # noqa: BLE001 - capture failure -> eager for this key
            warnings.warn(f"HIP graph capture of {key[0]} failed ({e}); running eagerly", stacklevel=3)
            self._failed.add(key)
            graph = None
        for a, s in zip(S.arenas, snapshot):
            a.copy_(s)
        return graph

    def _remember(self, key: tuple, entry: tuple[Any, ...]) -> None:
        self._graphs[key] = entry
        self._graphs.move_to_end(key)
        while len(self._graphs) > self._max_graphs:
            self._graphs.popitem(last=False)

    # ------------------------------------------------------------------ #
    # RWKV7Model interface
    # ------------------------------------------------------------------ #

    def decode(self, token: Tensor, S: State) -> tuple[Tensor, State]:
        m = self.model
        if not (isinstance(S, State) and S.arena_intact()):
            return m.decode(token, S)
        m._check_state(S)
        B = S.batch_size
        if m.decode_launches(B) == 1:
            # one persistent kernel: a replay would only add the token copy
            return m.decode(token, S)
        key = self._key("decode", S, B)
        entry = self._graphs.get(key)
        if entry is None:
            tok = torch.zeros(B, dtype=torch.int64, device=self.w.device)
            logits = torch.empty(B, m.V, dtype=m.kernel_dtype, device=self.w.device)
            ws = m.workspace(B, 1)  # allocated outside the capture; the entry keeps it alive
            graph = self._capture(key, S, lambda: m.decode_into(tok, S, logits))
            if graph is None:
                return m.decode(token, S)
            entry = (graph, tok, logits, ws)
            self._remember(key, entry)
        else:
            self._graphs.move_to_end(key)
        graph, tok, logits, _ = entry
        tok.copy_(m._tokens(token, (B,)))
        graph.replay()
        out = logits.clone()
        return (out[0] if S.batch is None else out), S

    def prefill(self, tokens: Tensor, S: State) -> State:
        m = self.model
        tokens = torch.as_tensor(tokens)
        T = tokens.shape[-1] if tokens.ndim else 1
        if (
            not (isinstance(S, State) and S.arena_intact())
            or T < 2
            or T > self.prefill_graph_max_t
            or tokens.ndim != (1 if S.batch is None else 2)
        ):
            return m.prefill(tokens, S)
        m._check_state(S)
        B = S.batch_size
        key = self._key("prefill", S, T)
        entry = self._graphs.get(key)
        if entry is None:
            tok = torch.zeros(B, T, dtype=torch.int64, device=self.w.device)
            ws = m.workspace(B, T)  # the entry keeps the captured workspace alive
            graph = self._capture(key, S, lambda: m.prefill_into(tok, S))
            if graph is None:
                return m.prefill(tokens, S)
            entry = (graph, tok, ws)
            self._remember(key, entry)
        else:
            self._graphs.move_to_end(key)
        graph, tok, _ = entry
        tok.copy_(m._tokens(tokens, (B, T)))
        graph.replay()
        return S


def wrap_model(model: RWKV7Model, *, prefill_graph_max_t: int = 64, warmup: int = 2) -> HIPGraph:
    """Wrap an existing model instance (``demo/cuda_graph.py:238-249``)."""
    return HIPGraph(model, prefill_graph_max_t=prefill_graph_max_t, warmup=warmup)


def make_graph_cls(
    base_cls: type[RWKV7Model], *, prefill_graph_max_t: int = 64, warmup: int = 2
) -> type[RWKV7Model]:
    """A class whose ``cls(w, **kw)`` builds ``base_cls(w, **kw)`` and wraps it
    (``demo/cuda_graph.py:252-272``)."""

    def _init(self, w: RWKV7Weight, **kwargs) -> None:
        HIPGraph.__init__(self, base_cls(w, **kwargs), prefill_graph_max_t=prefill_graph_max_t, warmup=warmup)

    return type(f"HIPGraph{base_cls.__name__}", (HIPGraph,), {"__init__": _init})
