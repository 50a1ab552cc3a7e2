"""RWKV7 weights (drop-in for ``rwkv_tl.weight``) and their HIP device arena.

``RWKV7Weight(model_path, device=None, dtype=torch.float16)`` keeps the
reference's loader contract and attribute layout (``src/rwkv_tl/weight.py``):
tensors are cast to ``dtype`` at load (``:167-169``), matrices are kept
transposed ``[in, out]`` with ``rkvWt`` stacked ``[3, C, C]`` (``:98-106``), the
LoRA first steps in both orientations (``:77-91``) and the embedding
layer-normalised once at load in ``dtype`` (``:175``). Checkpoints are read
with ``torch.load(weights_only=True)``.

``pack_device_weights`` builds what the HIP library reads: one contiguous arena
per layer with every matrix in ``[out, in]`` (K-contiguous) order, the stacked
``[3C + sumR, C]`` projection matrix for decode, per-head-contiguous LoRA
second steps and the small vectors as fp32 (layout from
``rwkv7_layer_layout_get`` in ``include/rwkv7_hip.h``).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib


class LNWeight:
    """LayerNorm weight/bias; ``weight.py:6-15`` (``F.layer_norm``, eps 1e-5)."""

    w: Tensor
    b: Tensor

    def __init__(self, W, prefix: str):
        self.w = W[f"{prefix}.weight"]
        self.b = W[f"{prefix}.bias"]

    def __call__(self, x: Tensor) -> Tensor:
        return F.layer_norm(x, (x.shape[-1],), self.w, self.b)


class RWKV7ATTWeight:
    """Time-mix weights; attribute layout of ``weight.py:18-106``."""

    def __init__(self, W, prefix: str, ln_pre: LNWeight):
        self.ln_pre = ln_pre
        self.ln_x = LNWeight(W, f"{prefix}.ln_x")
        for n in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
            setattr(self, n, W[f"{prefix}.{n}"].squeeze())
        for g in ("w", "a", "v", "g"):
            setattr(self, f"{g}1", W[f"{prefix}.{g}1"])
            setattr(self, f"{g}1t", W[f"{prefix}.{g}1"].t().contiguous())
            setattr(self, f"{g}2", W[f"{prefix}.{g}2"])
        for n in ("w0", "a0", "v0", "r_k", "k_k", "k_a"):
            setattr(self, n, W[f"{prefix}.{n}"])
        self.rkvWt = torch.stack(
            [W[f"{prefix}.{m}.weight"].T.contiguous() for m in ("receptance", "key", "value")]
        )
        self.oWt = W[f"{prefix}.output.weight"].T.contiguous()


class RWKV7FFNWeight:
    """Channel-mix weights; ``weight.py:109-126``."""

    def __init__(self, W, prefix: str, ln_pre: LNWeight):
        self.ln_pre = ln_pre
        self.x_k = W[f"{prefix}.x_k"].squeeze()
        self.kWt = W[f"{prefix}.key.weight"].T.contiguous()
        self.vWt = W[f"{prefix}.value.weight"].T.contiguous()


class RWKV7Block:
    def __init__(self, W, prefix: str):
        self.att = RWKV7ATTWeight(W, f"{prefix}.att", LNWeight(W, f"{prefix}.ln1"))
        self.ffn = RWKV7FFNWeight(W, f"{prefix}.ffn", LNWeight(W, f"{prefix}.ln2"))


class RWKV7Weight:
    """Loaded RWKV7 weights; constructor contract of ``weight.py:155-184``."""

    dtype: torch.dtype
    device: torch.device
    L: int
    C: int

    def __init__(
        self,
        model_path: str | None,
        device: str | torch.device | None = None,
        dtype: torch.dtype = torch.float16,
        *,
        state_dict: dict[str, Tensor] | None = None,
    ):
        if state_dict is None:
            if model_path is None:
                raise ValueError("either model_path or state_dict is required")
            state_dict = torch.load(model_path, map_location=device, weights_only=True)
        W = {
            k: (v.to(device=device, dtype=dtype) if isinstance(v, Tensor) else v)
            for k, v in state_dict.items()
        }
        self.head = W["head.weight"]
        self.ln_in = LNWeight(W, "blocks.0.ln0")
        self.ln_out = LNWeight(W, "ln_out")
        self.emb = self.ln_in(W["emb.weight"])
        self.dtype = dtype
        self.device = self.emb.device
        self.L = 1 + max(int(k.split(".")[1]) for k in W if k.startswith("blocks."))
        self.C = self.emb.shape[1]
        self.blocks = [RWKV7Block(W, f"blocks.{i}") for i in range(self.L)]

    @classmethod
    def from_state_dict(
        cls,
        state_dict: dict[str, Tensor],
        device: str | torch.device | None = None,
        dtype: torch.dtype = torch.float16,
    ) -> "RWKV7Weight":
        return cls(None, device=device, dtype=dtype, state_dict=state_dict)


@dataclass
class DeviceWeights:
    """Device arenas of one model plus the ctypes descriptor pointing at them."""

    dims: _lib.Dims
    layout: _lib.LayerLayout
    layers: Tensor   # uint8 [L, layout.bytes]
    emb: Tensor      # f16 [V, C]
    head: Tensor     # f16 [V, C]
    ln_out: Tensor   # f32 [2, C]
    desc: _lib.Model
    layers_frag: Tensor | None = None  # uint8 [L, layout.frag_bytes]
    head_frag: Tensor | None = None    # f16, the head in fragment order
    layers_q: Tensor | None = None     # uint8 [L, layout.q_bytes]: int8 matrices + row scales
    head_q: Tensor | None = None       # uint8: int8 head [V, C], then f32 row scales [V]

    @property
    def nbytes(self) -> int:
        ts = (self.layers, self.emb, self.head, self.ln_out, self.layers_frag, self.head_frag, self.layers_q,
              self.head_q)
        return sum(t.numel() * t.element_size() for t in ts if t is not None)


def quantize_rows_i8(W: Tensor) -> tuple[Tensor, Tensor]:
    """Symmetric per-row int8: ``scale = max|W[n]| * (1/127)`` (fp32; 0 for an
    all-zero row), ``q = round_half_even(W / scale)`` in [-127, 127], so
    ``|W - scale * q| <= scale / 2``. A weight-format step done once at load
    (torch on W's device), like the checkpoint dtype conversion.

    Both steps give the same bits on every device. The scale is one IEEE fp32
    multiplication by the fp32 constant 1/127 (torch's division by a scalar
    is not bound to round alike on the CPU and the GPU; ~4 % of the scales
    differ by one ulp between a true division and a reciprocal
    multiplication); the quotient is formed in float64, wide enough (fp16
    ``W`` over fp32 ``scale``) that its rounding never crosses a half-step.
    With an fp32 quotient, or scales one ulp apart, ~1 element in 10^5 rounds
    to the neighbouring integer -- enough to move a layer's output by ~1e-4
    relative."""
    w = W.float()
    scale = w.abs().amax(dim=1) * torch.tensor(1.0 / 127.0, dtype=torch.float32, device=w.device)
    div = torch.where(scale > 0, scale, torch.ones_like(scale)).double()
    q = torch.round(w.double() / div[:, None]).clamp_(-127, 127)
    return q.to(torch.int8).contiguous(), scale.contiguous()


def quantize_rows_any4(W: Tensor, iters: int = 12) -> tuple[Tensor, Tensor]:
    """any4: per row a table of 16 values and one 4-bit code per weight
    (the learned 4-bit format, "any4", that the reference's quantisation plan
    names beside int8). The table is a per-row k-means of the row's values:
    Lloyd iterations (assign every weight to its nearest centroid, move each
    centroid to the mean of its weights; a cluster that empties keeps its
    centroid) from the 16 evenly spaced levels of [min, max], so the result is
    never worse than that uniform 4-bit grid (a Lloyd step cannot increase the
    squared error). The table is rounded to f16 and every weight then takes
    the code of its nearest f16 entry. Returns ``codes`` uint8 [N, K/2] (column 2j in the
    low nibble of byte j, 2j+1 in the high nibble) and ``lut`` f16 [N, 16],
    ascending. A weight-format step done once at load (torch on W's device;
    the cluster sums are not bit-reproducible across devices, which only moves
    centroids by float rounding)."""
    w = W.float()
    N, K = w.shape
    if K % 2 or K < 16:
        raise ValueError("any4 packs two codes per byte and needs K >= 16 (even)")
    lo, hi = w.amin(dim=1, keepdim=True), w.amax(dim=1, keepdim=True)
    cent = (lo + (hi - lo) * (torch.arange(16, device=w.device, dtype=torch.float32) / 15)).contiguous()
    ones = torch.ones_like(w)
    for _ in range(iters):
        mid = ((cent[:, 1:] + cent[:, :-1]) * 0.5).contiguous()
        code = torch.searchsorted(mid, w)
        sums = torch.zeros_like(cent).scatter_add_(1, code, w)
        cnt = torch.zeros_like(cent).scatter_add_(1, code, ones)
        # an empty cluster moves to one of the row's worst-represented weights
        # (the e-th empty one to the e-th largest error), which can only lower
        # the squared error at the next assignment
        empty = cnt == 0
        err = (w - cent.gather(1, code)).abs()
        worst = w.gather(1, err.topk(16, dim=1).indices)
        rank = (empty.long().cumsum(1) - 1).clamp(min=0)
        cent = torch.where(empty, worst.gather(1, rank), sums / cnt.clamp(min=1.0)).sort(dim=1).values
    lut = cent.to(torch.float16).contiguous()
    lf = lut.float()
    code = torch.searchsorted(((lf[:, 1:] + lf[:, :-1]) * 0.5).contiguous(), w).to(torch.uint8)
    codes = (code[:, 0::2] | (code[:, 1::2] << 4)).contiguous()
    return codes, lut


def dequantize_rows_any4(codes: Tensor, lut: Tensor) -> Tensor:
    """The f32 matrix an any4 (codes, lut) pair stands for."""
    lo, hi = (codes & 15).long(), (codes >> 4).long()
    idx = torch.stack([lo, hi], dim=2).reshape(codes.shape[0], -1)
    return lut.float().gather(1, idx)


def int8_matrices(w: "RWKV7Weight") -> list[dict[str, Tensor]]:
    """Per layer, the f16 matrices the int8 decode streams, as [out, in] rows
    in the int8 arena's order: ``rkv`` (receptance, key, value rows, then the
    LoRA first steps v1^T, w1^T, a1^T, g1^T), ``o``, ``fk``, ``fv``."""
    out = []
    for blk in w.blocks:
        att, ffn = blk.att, blk.ffn
        rkv = torch.cat([att.rkvWt[j].T for j in range(3)] + [att.v1t, att.w1t, att.a1t, att.g1t], 0)
        out.append({"rkv": rkv, "o": att.oWt.T, "fk": ffn.kWt.T, "fv": ffn.vWt.T})
    return out


def to_fragments(W: Tensor) -> Tensor:
    """``W [N, K]`` in fragment order (``include/rwkv7_hip.h``): zero-padded to
    16-row x 32-column blocks, block (s, j) at ``(s * K'/32 + j) * 512``
    halves, lane ``l`` of a block holding ``W[16 s + l % 16, 32 j + 8 (l // 16) :+8]``."""
    N, K = W.shape
    Np, Kp = -(-N // 16) * 16, -(-K // 32) * 32
    P = torch.zeros(Np, Kp, dtype=W.dtype, device=W.device)
    P[:N, :K] = W
    # [s, r, j, c, e] -> [s, j, c, r, e]: lane = c * 16 + r
    return P.view(Np // 16, 16, Kp // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)


def model_dims(w: RWKV7Weight) -> _lib.Dims:
    att = w.blocks[0].att
    return _lib.Dims(
        n_layer=w.L,
        n_embd=w.C,
        n_head=w.C // 64,
        n_ffn=w.blocks[0].ffn.kWt.shape[1],
        vocab=w.head.shape[0],
        rank_w=att.w1.shape[1],
        rank_a=att.a1.shape[1],
        rank_v=att.v1.shape[1],
        rank_g=att.g1.shape[1],
    )


def layer_layout(dims: _lib.Dims) -> _lib.LayerLayout:
    lib = _lib.load()
    out = _lib.LayerLayout()
    _lib.check(lib.rwkv7_layer_layout_get(ctypes.byref(dims), ctypes.byref(out)), "rwkv7_layer_layout_get")
    return out


def _f16_view(buf: Tensor, off: int, rows: int, cols: int, dtype: torch.dtype = torch.float16) -> Tensor:
    """A [rows, cols] view of 16-bit values (float16 or bfloat16) at byte ``off``."""
    return buf[off : off + rows * cols * 2].view(dtype).view(rows, cols)


def pack_device_weights(w: RWKV7Weight, fragments: bool = True, int8: bool = False) -> DeviceWeights:
    """Build the HIP arenas from reference-layout weights (float16 or
    bfloat16, on the GPU); every 16-bit section keeps the weights' format, and
    a bfloat16 model gets the ``RWKV7_MODEL_BF16`` flag.

    ``fragments`` also builds the fragment-order copy the prefill / batched
    decode GEMMs stream (one contiguous KiB per wave load); it roughly doubles
    the weight memory. ``int8`` also builds the int8 arenas of the batch-1
    decode (``quantize_rows_i8`` per matrix row) and sets the model flag that
    makes batch-1 decode stream them."""
    if w.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"the HIP kernels take float16 or bfloat16 weights, got {w.dtype}")
    dt = w.dtype
    dims = model_dims(w)
    lay = layer_layout(dims)
    C, F_ = dims.n_embd, dims.n_ffn
    SR = dims.rank_w + dims.rank_a + dims.rank_v + dims.rank_g
    dev = w.device
    layers = torch.zeros(dims.n_layer, lay.bytes, dtype=torch.uint8, device=dev)
    for i, blk in enumerate(w.blocks):
        att, ffn, buf = blk.att, blk.ffn, layers[i]
        rkv = _f16_view(buf, lay.w_rkv, 3 * C, C, dt)
        for j in range(3):
            rkv[j * C : (j + 1) * C].copy_(att.rkvWt[j].T)
        _f16_view(buf, lay.w_lora1, SR, C, dt).copy_(torch.cat([att.v1t, att.w1t, att.a1t, att.g1t], 0))
        _f16_view(buf, lay.w_lora2, C, SR, dt).copy_(torch.cat([att.v2.T, att.w2.T, att.a2.T, att.g2.T], 1))
        _f16_view(buf, lay.w_o, C, C, dt).copy_(att.oWt.T)
        _f16_view(buf, lay.w_fk, F_, C, dt).copy_(ffn.kWt.T)
        _f16_view(buf, lay.w_fv, C, F_, dt).copy_(ffn.vWt.T)
        vec = buf[lay.vec : lay.vec + _lib.NVEC * C * 4].view(torch.float32).view(_lib.NVEC, C)
        src = {
            "ln1_w": att.ln_pre.w, "ln1_b": att.ln_pre.b,
            "x_r": att.x_r, "x_w": att.x_w, "x_k": att.x_k, "x_v": att.x_v,
            "x_a": att.x_a, "x_g": att.x_g, "w0": att.w0, "a0": att.a0, "v0": att.v0,
            "k_k": att.k_k, "k_a": att.k_a, "r_k": att.r_k,
            "lnx_w": att.ln_x.w, "lnx_b": att.ln_x.b,
            "ln2_w": ffn.ln_pre.w, "ln2_b": ffn.ln_pre.b, "ffn_x_k": ffn.x_k,
        }
        for j, name in enumerate(_lib.VEC_NAMES):
            vec[j].copy_(src[name].reshape(-1).float())
    emb = w.emb.contiguous()
    head = w.head.contiguous()
    ln_out = torch.stack([w.ln_out.w.float(), w.ln_out.b.float()]).contiguous()
    layers_frag = head_frag = None
    if fragments:
        layers_frag = torch.zeros(dims.n_layer, lay.frag_bytes, dtype=torch.uint8, device=dev)
        R = (dims.rank_v, dims.rank_w, dims.rank_a, dims.rank_g)
        for i in range(dims.n_layer):
            buf, src = layers_frag[i], layers[i]

            def put(off: int, Wm: Tensor) -> None:
                f = to_fragments(Wm)
                buf[off : off + f.numel() * 2].view(dt).copy_(f)

            put(lay.f_rkv, _f16_view(src, lay.w_rkv, 3 * C, C, dt))
            l1 = _f16_view(src, lay.w_lora1, SR, C, dt)
            l2 = _f16_view(src, lay.w_lora2, C, SR, dt)
            r0 = 0
            for g in range(4):
                put(lay.f_l1[g], l1[r0 : r0 + R[g]])
                put(lay.f_l2[g], l2[:, r0 : r0 + R[g]])
                r0 += R[g]
            put(lay.f_o, _f16_view(src, lay.w_o, C, C, dt))
            put(lay.f_fk, _f16_view(src, lay.w_fk, F_, C, dt))
            put(lay.f_fv, _f16_view(src, lay.w_fv, C, F_, dt))
        head_frag = to_fragments(head).contiguous()
    layers_q = head_q = None
    if int8:
        layers_q = torch.zeros(dims.n_layer, lay.q_bytes, dtype=torch.uint8, device=dev)
        N1 = 3 * C + SR
        for i, mats in enumerate(int8_matrices(w)):
            buf = layers_q[i]
            scales = []
            for name, off in (("rkv", lay.q_rkv), ("o", lay.q_o), ("fk", lay.q_fk), ("fv", lay.q_fv)):
                q, sc = quantize_rows_i8(mats[name])
                buf[off : off + q.numel()].view(torch.int8).view(q.shape).copy_(q)
                scales.append(sc)
            sc = torch.cat(scales)
            assert sc.numel() == N1 + C + F_ + C
            buf[lay.q_scale : lay.q_scale + sc.numel() * 4].view(torch.float32).copy_(sc)
        qh, sh = quantize_rows_i8(head)
        soff = int(_lib.load().rwkv7_head_q_scale_offset(ctypes.byref(dims)))
        head_q = torch.zeros(soff + sh.numel() * 4, dtype=torch.uint8, device=dev)
        head_q[: qh.numel()].view(torch.int8).view(qh.shape).copy_(qh)
        head_q[soff:].view(torch.float32).copy_(sh)
    desc = _lib.Model(
        dims=dims,
        layers=layers.data_ptr(),
        emb=emb.data_ptr(),
        head=head.data_ptr(),
        ln_out=ln_out.data_ptr(),
        layers_frag=layers_frag.data_ptr() if layers_frag is not None else None,
        head_frag=head_frag.data_ptr() if head_frag is not None else None,
        flags=(_lib.MODEL_INT8_DECODE if int8 else 0) | (_lib.MODEL_BF16 if dt == torch.bfloat16 else 0),
        layers_q=layers_q.data_ptr() if layers_q is not None else None,
        head_q=head_q.data_ptr() if head_q is not None else None,
    )
    return DeviceWeights(dims, lay, layers, emb, head, ln_out, desc, layers_frag, head_frag, layers_q, head_q)
