"""Token sampling on the GPU (drop-in for ``demo/sampling.py:13-70``).

``sample_logits`` keeps the reference's signature and semantics: repetition
penalty on ``seen``, greedy argmax when ``temperature`` is None or <= 0, else
temperature, top-k, top-p and one draw, along the last dimension. All of it is
one call of ``rwkv7_sample``: one workgroup per row, or for top-k sampling
one workgroup per 2048 logits that keeps its slice's candidates and a second
launch that draws from them (the same token either way). The
draw comes from a counter-based generator (Philox4x32-10) keyed by a seed
taken from torch's CPU generator, so ``torch.manual_seed`` makes it
reproducible without a device sync; it is a different random stream from
``torch.multinomial``'s, with the same distribution.

``Sampler`` is the allocation-light form ``generate`` uses: a persistent
``seen`` bitmap that the kernel itself updates after each draw, and the
output written straight into a caller's buffer, so a generation loop never
waits for the host.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib

MAX_VOCAB = 65536


def draw_seed(generator: torch.Generator | None = None) -> int:
    """A 64-bit Philox key from torch's CPU generator (no device sync)."""
    return int(torch.randint(-(2**63), 2**63 - 1, (), dtype=torch.int64, generator=generator)) & (2**64 - 1)


def _params(temperature, top_k, top_p, repetition_penalty, seed: int, offset: int) -> _lib.Sampling:
    return _lib.Sampling(
        temperature=0.0 if temperature is None else float(temperature),
        top_k=int(top_k),
        top_p=float(top_p),
        repetition_penalty=float(repetition_penalty),
        seed=seed,
        offset=offset,
    )


# logits dtypes the kernel reads directly, and their rwkv7_sample code
_LOGIT_DTYPES = {torch.float16: 0, torch.float32: 1, torch.bfloat16: 2}


def _check_logits(logits: Tensor) -> Tensor:
    if not logits.is_cuda:
        raise ValueError("sample_logits runs the HIP sampling kernel: logits must be on the GPU")
    if logits.ndim not in (1, 2):
        raise ValueError(f"expected [V] or [B, V] logits, got {tuple(logits.shape)}")
    if logits.shape[-1] > MAX_VOCAB or logits.shape[-1] == 0:
        raise ValueError(f"vocabulary of {logits.shape[-1]} is outside 1..{MAX_VOCAB}")
    if logits.dtype not in _LOGIT_DTYPES:
        logits = logits.float()
    return logits if logits.stride(-1) == 1 else logits.contiguous()


def seen_bitmap(seen: Tensor | None, B: int, V: int, device) -> Tensor | None:
    """``seen`` token ids -> int32 [B, ceil(V/32)] bitmap (bit t % 32 of word t // 32)."""
    if seen is None:
        return None
    nw = (V + 31) // 32
    mask = torch.zeros(nw * 32, dtype=torch.bool, device=device)
    mask[torch.as_tensor(seen, device=device).reshape(-1).long()] = True
    shifts = torch.arange(32, device=device, dtype=torch.int64)
    words = (mask.view(nw, 32).long() << shifts).sum(-1).to(torch.int32)
    return words.expand(B, nw).contiguous()


def sample_into(
    logits: Tensor,
    out: Tensor,
    *,
    temperature: float | None,
    top_k: int,
    top_p: float,
    repetition_penalty: float,
    seed: int,
    offset: int,
    seen: Tensor | None = None,
    update_seen: bool = False,
    probs: Tensor | None = None,
    workspace: Tensor | None = None,
) -> None:
    """One ``rwkv7_sample`` call: logits f16/f32/bf16 [B, V] (unit column stride)
    -> out int64 [B]; ``seen`` int32 [B, ceil(V/32)]; ``probs`` f32 [B, V].
    ``workspace`` (``workspace_for(B, V)``) lets top-k sampling spread each
    row over many workgroups; the token drawn is the same without it."""
    lib = _lib.load()
    B, V = logits.shape
    if out.dtype != torch.int64 or out.numel() != B or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 tensor of B elements")
    if seen is not None and (seen.dtype != torch.int32 or seen.shape != (B, (V + 31) // 32) or not seen.is_contiguous()):
        raise ValueError(f"seen must be a contiguous int32 [{B}, {(V + 31) // 32}] bitmap")
    if probs is not None and (probs.dtype != torch.float32 or probs.shape != (B, V) or not probs.is_contiguous()):
        raise ValueError(f"probs must be a contiguous float32 [{B}, {V}] tensor")
    p = _params(temperature, top_k, top_p, repetition_penalty, seed, offset)
    rc = lib.rwkv7_sample(
        logits.data_ptr(), _LOGIT_DTYPES[logits.dtype], logits.stride(0), B, V, ctypes.byref(p),
        _lib.ptr(seen), 0 if seen is None else seen.stride(0), int(update_seen), out.data_ptr(),
        _lib.ptr(probs), 0 if probs is None else probs.stride(0),
        _lib.ptr(workspace), 0 if workspace is None else workspace.numel(), _lib.stream_handle(),
    )
    _lib.check(rc, "rwkv7_sample")


def workspace_for(B: int, V: int, device) -> Tensor:
    """Device workspace of ``rwkv7_sample`` for B rows of V logits."""
    n = int(_lib.load().rwkv7_sample_workspace_bytes(B, V))
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


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
    x = _check_logits(logits)
    x2 = x.reshape(1, -1) if x.ndim == 1 else x
    B, V = x2.shape
    out = torch.empty(B, dtype=torch.int64, device=x.device)
    bits = seen_bitmap(seen, B, V, x.device) if repetition_penalty != 1.0 else None
    sample_into(
        x2, out, temperature=temperature, top_k=top_k, top_p=top_p,
        repetition_penalty=repetition_penalty, seed=draw_seed(), offset=0, seen=bits,
        workspace=workspace_for(B, V, x.device),
    )
    return out[0] if logits.ndim == 1 else out


class Sampler:
    """Sampling state of one generation: the seed, the step counter and the
    device bitmap of generated tokens (the ``seen`` of the reference's
    ``generate``, ``demo/_rwkv7_abc.py:60-69``), updated by the kernel."""

    def __init__(self, V: int, device, *, batch: int = 1, temperature=None, top_k=0, top_p=1.0,
                 repetition_penalty=1.0, seed: int | None = None) -> None:
        self.V = V
        self.cfg = dict(temperature=temperature, top_k=top_k, top_p=top_p, repetition_penalty=repetition_penalty)
        self.seed = draw_seed() if seed is None else seed
        self.step = 0
        self.seen = torch.zeros(batch, (V + 31) // 32, dtype=torch.int32, device=device)
        self.workspace = workspace_for(batch, V, device)

    def __call__(self, logits: Tensor, out: Tensor) -> None:
        x = _check_logits(logits)
        x2 = x.reshape(1, -1) if x.ndim == 1 else x
        sample_into(x2, out, **self.cfg, seed=self.seed, offset=self.step, seen=self.seen, update_seen=True,
                    workspace=self.workspace)
        self.step += 1
