"""Seeded random-init RWKV7 checkpoints in the reference's state-dict format.

The reference ships no init code; it only loads checkpoints
(``src/rwkv_tl/weight.py:155-184``). Key names and shapes follow what that
loader reads:

* ``emb.weight`` / ``head.weight``                      ``[V, C]``
* ``blocks.0.ln0.*``, ``ln_out.*``                     ``[C]``
* ``blocks.i.ln1.*`` / ``blocks.i.ln2.*``              ``[C]``
* ``blocks.i.att.{x_r,x_w,x_k,x_v,x_a,x_g,w0,a0,v0,k_k,k_a}``  ``[1, 1, C]``
* ``blocks.i.att.{w1,a1,v1,g1}`` ``[C, R]`` and ``{w2,a2,v2,g2}`` ``[R, C]``
* ``blocks.i.att.r_k``                                  ``[H, 64]``
* ``blocks.i.att.{receptance,key,value,output}.weight`` ``[C, C]`` (``[out, in]``)
* ``blocks.i.att.ln_x.*``                               ``[C]``
* ``blocks.i.ffn.x_k`` ``[1, 1, C]``, ``ffn.key.weight`` ``[F, C]``,
  ``ffn.value.weight`` ``[C, F]``

Init: every matrix and every per-channel vector is N(0, 0.02); every LayerNorm
and GroupNorm weight is 1 and every bias 0. Tensors are drawn in fp32 from one
CPU ``torch.Generator`` seeded once, in sorted key order, so the same seed
yields bit-identical weights on any host with the same torch build.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import torch

HEAD_DIM = 64


@dataclass(frozen=True)
class ModelShape:
    """Sizes of one RWKV7 model (ranks are the LoRA widths of w/a/v/g)."""

    n_layer: int
    n_embd: int
    n_ffn: int
    vocab: int
    rank_w: int
    rank_a: int
    rank_v: int
    rank_g: int

    @property
    def n_head(self) -> int:
        return self.n_embd // HEAD_DIM


# Named shapes used by tests and the benchmark. The 0.1B ranks are the ones
# BASELINE.json states; 0.4B reuses them; 1.5B uses the usual RWKV-LM sizing.
SHAPES: dict[str, ModelShape] = {
    "tiny": ModelShape(3, 256, 1024, 512, 32, 32, 16, 64),
    "0.1b": ModelShape(12, 768, 3072, 65536, 64, 64, 32, 128),
    "0.4b": ModelShape(24, 1024, 4096, 65536, 64, 64, 32, 128),
    "1.5b": ModelShape(24, 2048, 8192, 65536, 96, 96, 64, 256),
}


def _layout(s: ModelShape) -> dict[str, tuple[tuple[int, ...], str]]:
    """Map key -> (shape, init kind) where kind is 'mat', 'vec', 'one', 'zero'."""
    C, F, V, H = s.n_embd, s.n_ffn, s.vocab, s.n_head
    out: dict[str, tuple[tuple[int, ...], str]] = {
        "emb.weight": ((V, C), "mat"),
        "head.weight": ((V, C), "mat"),
        "blocks.0.ln0.weight": ((C,), "one"),
        "blocks.0.ln0.bias": ((C,), "zero"),
        "ln_out.weight": ((C,), "one"),
        "ln_out.bias": ((C,), "zero"),
    }
    ranks = {"w": s.rank_w, "a": s.rank_a, "v": s.rank_v, "g": s.rank_g}
    for i in range(s.n_layer):
        p = f"blocks.{i}"
        for ln in ("ln1", "ln2", "att.ln_x"):
            out[f"{p}.{ln}.weight"] = ((C,), "one")
            out[f"{p}.{ln}.bias"] = ((C,), "zero")
        for v in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g", "w0", "a0", "v0", "k_k", "k_a"):
            out[f"{p}.att.{v}"] = ((1, 1, C), "vec")
        for g, r in ranks.items():
            out[f"{p}.att.{g}1"] = ((C, r), "mat")
            out[f"{p}.att.{g}2"] = ((r, C), "mat")
        out[f"{p}.att.r_k"] = ((H, HEAD_DIM), "vec")
        for m in ("receptance", "key", "value", "output"):
            out[f"{p}.att.{m}.weight"] = ((C, C), "mat")
        out[f"{p}.ffn.x_k"] = ((1, 1, C), "vec")
        out[f"{p}.ffn.key.weight"] = ((F, C), "mat")
        out[f"{p}.ffn.value.weight"] = ((C, F), "mat")
    return out


def make_random_state_dict(
    shape: ModelShape | str,
    seed: int = 0,
    dtype: torch.dtype = torch.float16,
    std: float = 0.02,
) -> dict[str, torch.Tensor]:
    """Build a random-init checkpoint dict (CPU tensors of ``dtype``)."""
    if isinstance(shape, str):
        shape = SHAPES[shape]
    if shape.n_embd % HEAD_DIM:
        raise ValueError(f"n_embd={shape.n_embd} is not a multiple of {HEAD_DIM}")
    gen = torch.Generator(device="cpu").manual_seed(seed)
    sd: dict[str, torch.Tensor] = {}
    for key, (shp, kind) in sorted(_layout(shape).items()):
        if kind == "one":
            t = torch.ones(shp, dtype=torch.float32)
        elif kind == "zero":
            t = torch.zeros(shp, dtype=torch.float32)
        else:
            t = torch.randn(shp, generator=gen, dtype=torch.float32) * std
        sd[key] = t.to(dtype)
    return sd


def state_dict_digest(sd: dict[str, torch.Tensor]) -> str:
    """sha256 over (key, dtype, shape, raw bytes) in sorted key order."""
    h = hashlib.sha256()
    for key in sorted(sd):
        t = sd[key].detach().contiguous().cpu()
        h.update(key.encode())
        h.update(str(t.dtype).encode())
        h.update(str(tuple(t.shape)).encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.numel() else b"")
    return h.hexdigest()


def save_checkpoint(sd: dict[str, torch.Tensor], path: str) -> None:
    """Write ``sd`` as a plain tensor dict that ``torch.load`` reads back."""
    torch.save(sd, path)
