"""Operator-level API on the HIP library (counterpart of ``rwkv_tl.kernels.fp16``).

Same names, argument order and return conventions as the reference
(``src/rwkv_tl/kernels/fp16.py:13-30``); tensors must be on the ROCm device
and are validated on the host before any launch (ValueError on a bad shape or
dtype). There is no CPU branch: the reference's in-function torch fallbacks
(for example ``dplr.py:258-267``) are not reproduced.

* ``fused_dplr(S, R, W, K, V, A, B)`` / ``fused_dplr_T(...)``: the wkv7 DPLR
  step / sequence (``dplr.py:256-285``); ``wkv7`` is the batched form.
* ``fused_lerp6`` / ``fused_lerp6_copy`` / ``fused_lerp1_copy``
  (``lerp.py:140-198``).
* ``layer_norm`` (``weight.py:14-15``), ``gemv`` and ``gemm`` (the projection
  GEMMs of ``gemm.py:215-305``), ``fused_rkv_gemm`` (``gemm.py:215-262``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

N = 64

GEMM_EPI = {"f32": 0, "f16": 1, "relu2": 2, "add": 3}


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev(*ts: Tensor) -> None:
    for t in ts:
        _need(t.device.type == "cuda", f"tensor on {t.device}; the HIP kernels need a ROCm device")
        _need(t.is_contiguous(), "tensors must be contiguous")


def wkv7(S: Tensor, r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor) -> Tensor:
    """Batched DPLR recurrence; updates ``S`` [B,H,64,64] fp32 in place.

    ``r, k, v, a, b``: f16 [B, T, H, 64]; ``w``: f16 or f32 of the same shape.
    Returns ``y`` f16 [B, T, H, 64] with ``y_t = S_t r_t``.
    """
    _dev(S, r, w, k, v, a, b)
    _need(S.dtype == torch.float32 and S.dim() == 4 and S.shape[2:] == (N, N), "S must be f32 [B,H,64,64]")
    Bsz, H = S.shape[:2]
    _need(r.dim() == 4 and r.shape[0] == Bsz and r.shape[2] == H and r.shape[3] == N, "r must be [B,T,H,64]")
    T = r.shape[1]
    for name, t in (("k", k), ("v", v), ("a", a), ("b", b)):
        _need(t.shape == r.shape and t.dtype == torch.float16, f"{name} must be f16 {tuple(r.shape)}")
    _need(r.dtype == torch.float16, "r must be f16")
    _need(w.shape == r.shape and w.dtype in (torch.float16, torch.float32), "w must be f16/f32 like r")
    y = torch.empty_like(r)
    lib = _lib.load()
    rc = lib.rwkv7_wkv7(
        S.data_ptr(), r.data_ptr(), w.data_ptr(), int(w.dtype == torch.float32), k.data_ptr(),
        v.data_ptr(), a.data_ptr(), b.data_ptr(), y.data_ptr(), Bsz, T, H, _lib.stream_handle(),
    )
    _lib.check(rc, "rwkv7_wkv7")
    return y


def fused_dplr_T(S: Tensor, R: Tensor, W: Tensor, K: Tensor, V: Tensor, A: Tensor, B: Tensor):
    """Sequence DPLR: S [H,64,64] fp32 (in place), inputs [T,H,64]; returns (y [T,H,64], S)."""
    _need(S.dim() == 3, "S must be [H,64,64]")
    y = wkv7(
        S.unsqueeze(0), R.unsqueeze(0), W.unsqueeze(0), K.unsqueeze(0), V.unsqueeze(0),
        A.unsqueeze(0), B.unsqueeze(0),
    )
    return y[0], S


def fused_dplr(S: Tensor, R: Tensor, W: Tensor, K: Tensor, V: Tensor, A: Tensor, B: Tensor):
    """One DPLR step: S [H,64,64] fp32 (in place), inputs [H,64]; returns (y [H,64], S)."""
    y, S = fused_dplr_T(S, R.unsqueeze(0), W.unsqueeze(0), K.unsqueeze(0), V.unsqueeze(0),
                        A.unsqueeze(0), B.unsqueeze(0))
    return y[0], S


def _lerp(x: Tensor, prev: Tensor, mus: list[Tensor], x_copy: Tensor | None) -> Tensor:
    _dev(x, prev)
    C = x.shape[-1]
    _need(x.dim() == 1 and prev.shape == x.shape, "x and prev must be [C]")
    _need(x.dtype == torch.float16 and prev.dtype == torch.float16, "x and prev must be f16")
    mu = torch.stack([m.reshape(-1).float() for m in mus]).contiguous()
    _need(mu.shape[1] == C, "mix vectors must be [C]")
    out = torch.empty(len(mus), C, dtype=torch.float16, device=x.device)
    if x_copy is not None:
        _dev(x_copy)
        _need(x_copy.shape == x.shape and x_copy.dtype == torch.float16, "x_copy must be f16 [C]")
    lib = _lib.load()
    rc = lib.rwkv7_lerp(
        x.data_ptr(), prev.data_ptr(), mu.data_ptr(), len(mus), out.data_ptr(),
        None if x_copy is None else x_copy.data_ptr(), C, _lib.stream_handle(),
    )
    _lib.check(rc, "rwkv7_lerp")
    return out


def fused_lerp6(x, prev, x_r, x_w, x_k, x_v, x_a, x_g):
    """Six token-shift lerps ``x + mu * (prev - x)`` (``lerp.py:140-161``)."""
    return tuple(_lerp(x, prev, [x_r, x_w, x_k, x_v, x_a, x_g], None).unbind(0))


def fused_lerp6_copy(x, prev, x_r, x_w, x_k, x_v, x_a, x_g, x_copy):
    """``fused_lerp6`` plus ``x_copy <- x`` after prev is read (``lerp.py:163-188``)."""
    return tuple(_lerp(x, prev, [x_r, x_w, x_k, x_v, x_a, x_g], x_copy).unbind(0))


def fused_lerp1_copy(x, prev, w, x_copy):
    """One lerp plus ``x_copy <- x`` (``lerp.py:190-198``); x_copy may alias prev."""
    return _lerp(x, prev, [w], x_copy)[0]


def layer_norm(x: Tensor, weight: Tensor, bias: Tensor) -> Tensor:
    """LayerNorm over the last dim, eps 1e-5; returns f32 (``weight.py:14-15``)."""
    _dev(x)
    C = x.shape[-1]
    _need(x.dtype in (torch.float16, torch.float32), "x must be f16 or f32")
    rows = x.reshape(-1, C)
    y = torch.empty(rows.shape, dtype=torch.float32, device=x.device)
    w32, b32 = weight.float().contiguous(), bias.float().contiguous()
    lib = _lib.load()
    rc = lib.rwkv7_layernorm(
        rows.data_ptr(), int(x.dtype == torch.float32), w32.data_ptr(), b32.data_ptr(), y.data_ptr(),
        rows.shape[0], C, _lib.stream_handle(),
    )
    _lib.check(rc, "rwkv7_layernorm")
    return y.reshape(x.shape)


def gemv(x: Tensor, W: Tensor) -> Tensor:
    """``y = W x`` for f16 W [N, K] (``[out, in]``) and f32 x [K]; returns f32 [N]."""
    _dev(x, W)
    _need(W.dtype == torch.float16 and W.dim() == 2, "W must be f16 [N, K]")
    _need(x.dtype == torch.float32 and x.shape == (W.shape[1],), "x must be f32 [K]")
    y = torch.empty(W.shape[0], dtype=torch.float32, device=x.device)
    lib = _lib.load()
    rc = lib.rwkv7_gemv_f16(x.data_ptr(), W.data_ptr(), W.shape[1], y.data_ptr(), W.shape[0], W.shape[1],
                            _lib.stream_handle())
    _lib.check(rc, "rwkv7_gemv_f16")
    return y


def gemm(A: Tensor, W: Tensor, epi: str = "f32", out: Tensor | None = None) -> Tensor:
    """``epi(A W^T)`` for f16 A [M, K], W [N, K]; ``epi`` in f32/f16/relu2/add.

    ``add`` accumulates into ``out`` (f32 [M, N]) and returns it.
    """
    _dev(A, W)
    _need(A.dtype == torch.float16 and W.dtype == torch.float16, "A and W must be f16")
    _need(A.dim() == 2 and W.dim() == 2 and A.shape[1] == W.shape[1], "A [M,K] and W [N,K] must share K")
    M, K = A.shape
    Nn = W.shape[0]
    code = GEMM_EPI[epi]
    if epi == "add":
        _need(out is not None and out.dtype == torch.float32 and out.shape == (M, Nn), "add needs f32 out [M, N]")
    else:
        dt = torch.float32 if epi == "f32" else torch.float16
        out = torch.empty(M, Nn, dtype=dt, device=A.device)
    _dev(out)
    lib = _lib.load()
    rc = lib.rwkv7_gemm_f16(A.data_ptr(), K, W.data_ptr(), K, out.data_ptr(), Nn, M, Nn, K, code,
                            _lib.stream_handle())
    _lib.check(rc, "rwkv7_gemm_f16")
    return out


def fused_rkv_gemm(xr: Tensor, xk: Tensor, xv: Tensor, Wb: Tensor) -> Tensor:
    """``rkv[b] = X_b @ Wb[b]`` with Wb [3, C, C] in the reference's ``[in, out]``
    orientation (``gemm.py:215-262``); returns f16 [3, T, C]."""
    outs = [gemm(x.contiguous(), Wb[i].T.contiguous(), "f16") for i, x in enumerate((xr, xk, xv))]
    return torch.stack(outs)
