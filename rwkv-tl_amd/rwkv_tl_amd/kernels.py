"""Operator-level API on the HIP library (counterpart of ``rwkv_tl.kernels.fp16``
and ``rwkv_tl.kernels.bf16``).

Same names, argument order and return conventions as the reference
(``src/rwkv_tl/kernels/fp16.py:13-30``, ``bf16.py:13-30``); tensors must be on
the ROCm device and are validated on the host before any launch (ValueError on
a bad shape or dtype). The 16-bit operands of one call are all float16 or all
bfloat16, and the outputs take the same dtype: this one module serves both of
the reference's namespaces, which bind the same kernels to the two dtypes.
There is no CPU branch: the reference's in-function torch fallbacks (for
example ``dplr.py:258-267``) are not reproduced.

* ``fused_dplr(S, R, W, K, V, A, B)`` / ``fused_dplr_T(...)``: the wkv7 DPLR
  step / sequence (``dplr.py:256-285``); ``wkv7`` is the batched form.
* ``fused_lerp6`` / ``fused_lerp6_copy`` / ``fused_lerp1_copy``
  (``lerp.py:140-198``), ``fused_lerp6_rkv_copy`` (``lerp.py:200-219``).
* ``layer_norm`` (``weight.py:14-15``), ``gemv`` and ``gemm`` (the projection
  GEMMs of ``gemm.py:215-305``), ``fused_rkv_gemm`` (``gemm.py:215-262``).
* Weight-only quantised GEMVs (the reference's plan, ``TODO.md:58-63``):
  ``quantize_i8`` / ``gemv_i8`` (per-row int8) and ``quantize_any4`` /
  ``gemv_any4`` (per-row 16-entry tables, 4-bit codes).
* The time-mix stage operators, 16-bit in and out: ``fused_w_gate``,
  ``fused_v_gate``, ``fused_a_kk_k`` (``gates.py:287-313``), ``fused_gates``
  (``gates.py:315-357``), ``fused_rank_gemv`` (``gates.py:254-285``),
  ``fused_l2norm_neg_kk_a`` (``dplr.py:229-235``), ``fused_gn_rkrk``
  (``dplr.py:237-254``).
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _lib

N = 64

GEMM_EPI = {"f32": 0, "f16": 1, "relu2": 2, "add": 3, "tanh": 4, "sigmoid": 5, "relu2_f32": 6, "tanh_f32": 7,
            "sigmoid_f32": 8}
GEMM_BF16, GEMM_A_F32 = 1, 2  # flag bits of rwkv7_gemm_f16's format word


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev(*ts: Tensor) -> None:
    for t in ts:
        if t.device.type != "cuda":
            raise ValueError(f"tensor on {t.device}; the HIP kernels need a ROCm device")
        _need(t.is_contiguous(), "tensors must be contiguous")


_H16 = (torch.float16, torch.bfloat16)


def _h16(*ts: Tensor) -> int:
    """All float16 or all bfloat16 (on the device); returns the kernels' bf16 flag."""
    _dev(*ts)
    dt = ts[0].dtype
    if dt not in _H16:
        raise ValueError(f"expected float16 or bfloat16, got {dt}")
    for t in ts:
        if t.dtype != dt:
            raise ValueError(f"mixed 16-bit dtypes: {dt} and {t.dtype}")
    return int(dt == torch.bfloat16)


# The operator takes the chunked scan for sequences at least this long when
# the serial scan's 4 workgroups per head and sequence would leave CUs idle
# (measured on MI355X: B=1, H=16, T=128 faster chunked; the survey's C2,
# B=8, H=16, T=128, faster serial).
CHUNK_MIN_T = 32
_CUS: dict[int, int] = {}


def _cus(dev: torch.device) -> int:
    i = dev.index if dev.index is not None else torch.cuda.current_device()
    if i not in _CUS:
        _CUS[i] = torch.cuda.get_device_properties(i).multi_processor_count
    return _CUS[i]


def wkv7(S: Tensor, r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor,
         chunked: bool | None = None) -> Tensor:
    """Batched DPLR recurrence; updates ``S`` [B,H,64,64] fp32 in place.

    ``r, k, v, a, b``: f16 or bf16 [B, T, H, 64]; ``w``: the same 16-bit
    dtype or f32. Returns ``y`` [B, T, H, 64] of r's dtype with ``y_t = S_t r_t``.
    ``chunked``: run the chunked (MFMA) algorithm, ``rwkv7_wkv7_chunked``,
    with a workspace allocated per call, or the serial scan ``rwkv7_wkv7``;
    ``None`` chooses the chunked one for ``T >= CHUNK_MIN_T`` when
    ``4 B H`` is below the device's CU count.
    """
    _dev(S, r, w, k, v, a, b)
    _need(S.dtype == torch.float32 and S.dim() == 4 and S.shape[2:] == (N, N), "S must be f32 [B,H,64,64]")
    Bsz, H = S.shape[:2]
    _need(r.dim() == 4 and r.shape[0] == Bsz and r.shape[2] == H and r.shape[3] == N, "r must be [B,T,H,64]")
    T = r.shape[1]
    bf = _h16(r, k, v, a, b)
    for name, t in (("k", k), ("v", v), ("a", a), ("b", b)):
        if t.shape != r.shape:
            raise ValueError(f"{name} must be {tuple(r.shape)}")
    _need(w.shape == r.shape and w.dtype in (r.dtype, torch.float32), "w must be like r, or f32")
    y = torch.empty_like(r)
    lib = _lib.load()
    args = (S.data_ptr(), r.data_ptr(), w.data_ptr(), int(w.dtype == torch.float32), k.data_ptr(), v.data_ptr(),
            a.data_ptr(), b.data_ptr(), y.data_ptr(), Bsz, T, H, bf)
    if chunked is None:
        chunked = T >= CHUNK_MIN_T and 4 * Bsz * H < _cus(S.device)
    if chunked:
        nb = int(lib.rwkv7_wkv7_chunked_workspace_bytes(Bsz, T, H))
        ws = torch.empty(nb, dtype=torch.uint8, device=S.device)
        _lib.check(lib.rwkv7_wkv7_chunked(*args, ws.data_ptr(), nb, _lib.stream_handle()), "rwkv7_wkv7_chunked")
    else:
        _lib.check(lib.rwkv7_wkv7(*args, _lib.stream_handle()), "rwkv7_wkv7")
    return y


def _wkv7_f32_shapes(S: Tensor, r: Tensor, *rest: Tensor) -> tuple[int, int, int]:
    _need(S.dtype == torch.float32 and S.dim() == 4 and S.shape[2:] == (N, N), "S must be f32 [B,H,64,64]")
    Bsz, H = S.shape[:2]
    _need(r.dim() == 4 and r.shape[0] == Bsz and r.shape[2] == H and r.shape[3] == N, "r must be [B,T,H,64]")
    for t in (r, *rest):
        if not (t.shape == r.shape and t.dtype == torch.float32):
            raise ValueError(f"inputs must be f32 {tuple(r.shape)}")
    return Bsz, r.shape[1], H


def wkv7_f32(S: Tensor, r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor,
             hist: Tensor | None = None) -> Tensor:
    """``wkv7`` with every operand f32 (the training forward); ``S`` [B,H,64,64]
    is updated in place and, if given, ``hist`` f32 [B,H,T,64,64] receives the
    state entering each step (what ``wkv7_backward`` needs). Returns ``y``."""
    _dev(S, r, w, k, v, a, b)
    Bsz, T, H = _wkv7_f32_shapes(S, r, w, k, v, a, b)
    if hist is not None:
        _dev(hist)
        _need(hist.dtype == torch.float32 and hist.shape == (Bsz, H, T, N, N), "hist must be f32 [B,H,T,64,64]")
    y = torch.empty_like(r)
    lib = _lib.load()
    rc = lib.rwkv7_wkv7_f32(S.data_ptr(), r.data_ptr(), w.data_ptr(), k.data_ptr(), v.data_ptr(), a.data_ptr(),
                            b.data_ptr(), y.data_ptr(), _lib.ptr(hist), Bsz, T, H, _lib.stream_handle())
    _lib.check(rc, "rwkv7_wkv7_f32")
    return y


def wkv7_backward(hist: Tensor, S_T: Tensor, r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor,
                  gy: Tensor, gS_T: Tensor | None = None) -> tuple[Tensor, ...]:
    """Gradients of ``wkv7_f32``: ``(gS0, gr, gw, gk, gv, ga, gb)`` from
    ``gy = dL/dy`` and ``gS_T = dL/dS_T`` (None: zero), all f32."""
    _dev(hist, S_T, r, w, k, v, a, b, gy)
    Bsz, T, H = _wkv7_f32_shapes(S_T, r, w, k, v, a, b, gy)
    _need(hist.dtype == torch.float32 and hist.shape == (Bsz, H, T, N, N), "hist must be f32 [B,H,T,64,64]")
    if gS_T is not None:
        _dev(gS_T)
        _need(gS_T.shape == S_T.shape and gS_T.dtype == torch.float32, "gS_T must be like S_T")
    gS0 = torch.empty_like(S_T)
    grads = [torch.empty_like(r) for _ in range(6)]
    lib = _lib.load()
    rc = lib.rwkv7_wkv7_backward(hist.data_ptr(), S_T.data_ptr(), r.data_ptr(), w.data_ptr(), k.data_ptr(),
                                 v.data_ptr(), a.data_ptr(), b.data_ptr(), gy.data_ptr(), _lib.ptr(gS_T),
                                 gS0.data_ptr(), *(g.data_ptr() for g in grads), Bsz, T, H, _lib.stream_handle())
    _lib.check(rc, "rwkv7_wkv7_backward")
    return (gS0, *grads)


def dplr_seq_forward(S: Tensor, R: Tensor, W: Tensor, K: Tensor, V: Tensor, A: Tensor, B: Tensor):
    """Functional DPLR sequence for training: ``S`` [H,64,64] or [B,H,64,64]
    f32 is not modified; inputs [T,H,64] or [B,T,H,64] f32. Returns
    ``(y, S_T)``."""
    batched = S.dim() == 4
    S1 = (S if batched else S.unsqueeze(0)).contiguous().clone()
    ins = [(x if batched else x.unsqueeze(0)).contiguous() for x in (R, W, K, V, A, B)]
    y = wkv7_f32(S1, ins[0], ins[1], ins[2], ins[3], ins[4], ins[5])
    return (y, S1) if batched else (y[0], S1[0])


def dplr_seq_backward(S: Tensor, R: Tensor, W: Tensor, K: Tensor, V: Tensor, A: Tensor, B: Tensor,
                      gy: Tensor, gS: Tensor | None) -> tuple[Tensor, ...]:
    """Gradients of ``dplr_seq_forward`` w.r.t. ``(S, R, W, K, V, A, B)``:
    the forward is run again to record the per-step states (the reference's
    plan, TODO.md:46-54), then the reverse-time scan."""
    batched = S.dim() == 4
    u = (lambda x: x) if batched else (lambda x: x.unsqueeze(0))
    S1 = u(S).contiguous().clone()
    ins = [u(x).contiguous() for x in (R, W, K, V, A, B)]
    Bsz, H = S1.shape[:2]
    T = ins[0].shape[1]
    hist = torch.empty(Bsz, H, T, N, N, dtype=torch.float32, device=S.device)
    wkv7_f32(S1, *ins, hist=hist)
    out = wkv7_backward(hist, S1, *ins, u(gy).contiguous(), None if gS is None else u(gS).contiguous())
    return out if batched else tuple(g[0] for g in out)


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
    bf = _h16(x, prev)
    C = x.shape[-1]
    _need(x.dim() == 1 and prev.shape == x.shape, "x and prev must be [C]")
    mu = torch.stack([m.reshape(-1).float() for m in mus]).contiguous()
    _need(mu.shape[1] == C, "mix vectors must be [C]")
    out = torch.empty(len(mus), C, dtype=x.dtype, device=x.device)
    if x_copy is not None:
        _dev(x_copy)
        _need(x_copy.shape == x.shape and x_copy.dtype == x.dtype, "x_copy must be like x [C]")
    lib = _lib.load()
    rc = lib.rwkv7_lerp(
        x.data_ptr(), prev.data_ptr(), mu.data_ptr(), len(mus), out.data_ptr(),
        None if x_copy is None else x_copy.data_ptr(), C, bf, _lib.stream_handle(),
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
    _need(x.dtype in (torch.float16, torch.bfloat16, torch.float32), "x must be f16, bf16 or f32")
    rows = x.reshape(-1, C)
    y = torch.empty(rows.shape, dtype=torch.float32, device=x.device)
    w32, b32 = weight.float().contiguous(), bias.float().contiguous()
    lib = _lib.load()
    rc = lib.rwkv7_layernorm(
        rows.data_ptr(), int(x.dtype == torch.float32), w32.data_ptr(), b32.data_ptr(), y.data_ptr(),
        rows.shape[0], C, int(x.dtype == torch.bfloat16), _lib.stream_handle(),
    )
    _lib.check(rc, "rwkv7_layernorm")
    return y.reshape(x.shape)


def gemv(x: Tensor, W: Tensor) -> Tensor:
    """``y = W x`` for f16 or bf16 W [N, K] (``[out, in]``) and f32 x [K]; returns f32 [N]."""
    _dev(x)
    bf = _h16(W)
    _need(W.dim() == 2, "W must be [N, K]")
    _need(x.dtype == torch.float32 and x.shape == (W.shape[1],), "x must be f32 [K]")
    y = torch.empty(W.shape[0], dtype=torch.float32, device=x.device)
    lib = _lib.load()
    rc = lib.rwkv7_gemv_f16(x.data_ptr(), W.data_ptr(), W.shape[1], y.data_ptr(), W.shape[0], W.shape[1], bf,
                            _lib.stream_handle())
    _lib.check(rc, "rwkv7_gemv_f16")
    return y


def quantize_i8(W: Tensor) -> tuple[Tensor, Tensor]:
    """Symmetric per-row int8 weights for ``gemv_i8``: ``scale = max|W[n]| / 127``
    (fp32; 0 for an all-zero row), ``q = round_half_even(W / scale)`` in
    [-127, 127], so ``|W - scale * q| <= scale / 2``. A weight-format step
    (torch on W's device), like the checkpoint dtype conversion."""
    _need(W.dim() == 2 and W.is_floating_point(), "W must be a floating [N, K] matrix")
    from .weight import quantize_rows_i8

    return quantize_rows_i8(W)


def gemv_i8(x: Tensor, q: Tensor, scale: Tensor) -> Tensor:
    """``y[n] = scale[n] * sum_k x[k] q[n, k]`` for int8 q [N, K], f32 scale [N]
    and f32 x [K] (K % 16 == 0, K <= 8192); returns f32 [N]."""
    _dev(x, q, scale)
    _need(q.dtype == torch.int8 and q.dim() == 2 and q.is_contiguous(), "q must be contiguous int8 [N, K]")
    N, Kd = q.shape
    _need(scale.dtype == torch.float32 and scale.shape == (N,) and scale.is_contiguous(), "scale must be f32 [N]")
    _need(x.dtype == torch.float32 and x.shape == (Kd,) and x.is_contiguous(), "x must be contiguous f32 [K]")
    y = torch.empty(N, dtype=torch.float32, device=x.device)
    lib = _lib.load()
    rc = lib.rwkv7_gemv_i8(x.data_ptr(), q.data_ptr(), Kd, scale.data_ptr(), y.data_ptr(), N, Kd,
                           _lib.stream_handle())
    _lib.check(rc, "rwkv7_gemv_i8")
    return y


def quantize_any4(W: Tensor) -> tuple[Tensor, Tensor]:
    """any4 weights for ``gemv_any4``: codes uint8 [N, K/2], lut f16 [N, 16]
    (``weight.quantize_rows_any4``)."""
    _need(W.dim() == 2 and W.is_floating_point(), "W must be a floating [N, K] matrix")
    from .weight import quantize_rows_any4

    return quantize_rows_any4(W)


def gemv_any4(x: Tensor, codes: Tensor, lut: Tensor) -> Tensor:
    """y = W x for any4 weights (``rwkv7_gemv_any4``): x f32 [K], codes uint8
    [N, K/2] (two 4-bit codes per byte), lut f16 [N, 16]; y f32 [N]."""
    _dev(x, codes, lut)
    _need(codes.dtype == torch.uint8 and codes.dim() == 2, "codes must be uint8 [N, K/2]")
    N, K = codes.shape[0], 2 * codes.shape[1]
    if not (lut.dtype == torch.float16 and lut.shape == (N, 16)):
        raise ValueError(f"lut must be f16 [{N}, 16]")
    if not (x.dtype == torch.float32 and x.shape == (K,)):
        raise ValueError(f"x must be f32 [{K}]")
    y = torch.empty(N, dtype=torch.float32, device=x.device)
    lib = _lib.load()
    rc = lib.rwkv7_gemv_any4(x.data_ptr(), codes.data_ptr(), codes.stride(0), lut.data_ptr(), y.data_ptr(), N, K,
                             _lib.stream_handle())
    _lib.check(rc, "rwkv7_gemv_any4")
    return y


def gemm(A: Tensor, W: Tensor, epi: str = "f32", out: Tensor | None = None) -> Tensor:
    """``epi(A W^T)`` for A [M, K], W [N, K] f16 or bf16; A of W's dtype, or
    float32 (multiplied as its 16-bit part plus the 16-bit remainder: two MFMAs
    per weight fragment, fp32-grade activations). ``epi`` in f32 / f16 / relu2
    / add / tanh / sigmoid / relu2_f32 / tanh_f32 / sigmoid_f32 (the plain
    names store W's 16-bit dtype, ``*_f32`` and ``f32`` float32).

    ``add`` accumulates into ``out`` (f32 [M, N]) and returns it.
    """
    a32 = A.dtype == torch.float32
    bf = _h16(W) if a32 else _h16(A, W)
    _dev(A)
    _need(A.dim() == 2 and W.dim() == 2 and A.shape[1] == W.shape[1], "A [M,K] and W [N,K] must share K")
    _need(A.is_contiguous() and W.is_contiguous(), "A and W must be contiguous")
    M, K = A.shape
    Nn = W.shape[0]
    code = GEMM_EPI[epi]
    if epi == "add":
        _need(out is not None and out.dtype == torch.float32 and out.shape == (M, Nn), "add needs f32 out [M, N]")
    else:
        dt = torch.float32 if epi == "f32" or epi.endswith("_f32") else W.dtype
        out = torch.empty(M, Nn, dtype=dt, device=A.device)
    _dev(out)
    lib = _lib.load()
    flags = (GEMM_BF16 if bf else 0) | (GEMM_A_F32 if a32 else 0)
    rc = lib.rwkv7_gemm_f16(A.data_ptr(), K, W.data_ptr(), K, out.data_ptr(), Nn, M, Nn, K, code, flags,
                            _lib.stream_handle())
    _lib.check(rc, "rwkv7_gemm_f16")
    return out


def fused_rkv_gemm(xr: Tensor, xk: Tensor, xv: Tensor, Wb: Tensor) -> Tensor:
    """``rkv[b] = X_b @ Wb[b]`` with Wb [3, C, C] in the reference's ``[in, out]``
    orientation (``gemm.py:215-262``); returns f16 [3, T, C]."""
    outs = [gemm(x.contiguous(), Wb[i].T.contiguous(), "f16") for i, x in enumerate((xr, xk, xv))]
    return torch.stack(outs)


def fused_lerp6_rkv_copy(x, prev, x_r, x_w, x_k, x_v, x_a, x_g, x_copy, rWt_stack):
    """``fused_lerp6_copy`` then the r/k/v projections of ``xr, xk, xv`` by
    ``rWt_stack`` [3, C, C] (``[in, out]``); returns ``(r, k, v, xv, xw, xa, xg)``
    (``lerp.py:200-219``)."""
    xr, xw, xk, xv, xa, xg = fused_lerp6_copy(x, prev, x_r, x_w, x_k, x_v, x_a, x_g, x_copy)
    rkv = fused_rkv_gemm(xr.unsqueeze(0), xk.unsqueeze(0), xv.unsqueeze(0), rWt_stack)
    return rkv[0, 0], rkv[1, 0], rkv[2, 0], xv, xw, xa, xg


# ---------------------------------------------------------------------------
# time-mix stage operators (f16 or bf16 tensors, fp32 arithmetic inside)
# ---------------------------------------------------------------------------


def _vecs(C: int, *ts: Tensor) -> int:
    bf = _h16(*ts)
    for t in ts:
        if t.numel() != C:
            raise ValueError(f"expected {C} elements, got shape {tuple(t.shape)}")
    return bf


def fused_w_gate(x: Tensor, w0: Tensor) -> Tensor:
    """``exp(-sigmoid(w0 + x) / sqrt(e))`` over [C] (``gates.py:287-291``)."""
    C = x.numel()
    bf = _vecs(C, x, w0)
    out = torch.empty_like(x)
    _lib.check(_lib.load().rwkv7_w_gate(x.data_ptr(), w0.data_ptr(), out.data_ptr(), C, bf, _lib.stream_handle()),
               "rwkv7_w_gate")
    return out


def fused_v_gate(v: Tensor, v_first: Tensor, v0: Tensor, v12: Tensor) -> Tensor:
    """``v + sigmoid(v0 + v12) * (v_first - v)`` over [C] (``gates.py:293-297``)."""
    C = v.numel()
    bf = _vecs(C, v, v_first, v0, v12)
    out = torch.empty_like(v)
    _lib.check(_lib.load().rwkv7_v_gate(v.data_ptr(), v_first.data_ptr(), v0.data_ptr(), v12.data_ptr(),
                                        out.data_ptr(), C, bf, _lib.stream_handle()), "rwkv7_v_gate")
    return out


def fused_a_kk_k(a0: Tensor, a_x: Tensor, k: Tensor, k_k: Tensor, k_a: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    """``(sigmoid(a0 + a_x), k * k_k, k + k_a * (k * a - k))`` over [C] (``gates.py:299-313``)."""
    C = k.numel()
    bf = _vecs(C, a0, a_x, k, k_k, k_a)
    a, kk, kn = (torch.empty_like(k) for _ in range(3))
    _lib.check(_lib.load().rwkv7_a_kk_k(a0.data_ptr(), a_x.data_ptr(), k.data_ptr(), k_k.data_ptr(), k_a.data_ptr(),
                                        a.data_ptr(), kk.data_ptr(), kn.data_ptr(), C, bf, _lib.stream_handle()),
               "rwkv7_a_kk_k")
    return a, kk, kn


def fused_gates(vr: Tensor, wr: Tensor, ar: Tensor, gr: Tensor, v: Tensor, v_first: Tensor, k: Tensor,
                v2t: Tensor, w2t: Tensor, a2t: Tensor, g2t: Tensor, v0: Tensor, w0: Tensor, a0: Tensor,
                k_k: Tensor, k_a: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """LoRA second steps + gate math; returns ``(v, w, a, kk, k, g)``, each [C] (``gates.py:315-357``).

    ``vr/wr/ar/gr`` are the first-step results [R] before activation,
    ``v2t/w2t/a2t/g2t`` the second-step matrices [C, R]."""
    C = v.numel()
    bf = _vecs(C, v, v_first, k, v0, w0, a0, k_k, k_a)
    _need(_h16(v, vr, wr, ar, gr, v2t, w2t, a2t, g2t) == bf, "one 16-bit dtype for every operand")
    ranks = []
    for r_, m_ in ((vr, v2t), (wr, w2t), (ar, a2t), (gr, g2t)):
        if not (m_.dim() == 2 and m_.shape == (C, r_.numel())):
            raise ValueError(f"rank matrix {tuple(m_.shape)} vs [{C}, {r_.numel()}]")
        ranks.append(r_.numel())
    outs = [torch.empty_like(v) for _ in range(6)]
    io = _lib.GatesIO(*(t.data_ptr() for t in (vr, wr, ar, gr, v2t, w2t, a2t, g2t, v, v_first, k, v0, w0, a0,
                                               k_k, k_a, *outs)))
    _lib.check(_lib.load().rwkv7_gates(ctypes.byref(io), *ranks, C, bf, _lib.stream_handle()), "rwkv7_gates")
    return tuple(outs)


def fused_rank_gemv(xv: Tensor, xw: Tensor, xa: Tensor, xg: Tensor, packed: Tensor,
                    rv: int, rw: int, ra: int, rg: int) -> Tensor:
    """``[v1t; w1t; a1t; g1t] @ [xv; xw; xa; xg]`` by row segment; returns [rv+rw+ra+rg] (``gates.py:254-285``)."""
    C = xv.numel()
    bf = _vecs(C, xv, xw, xa, xg)
    _need(_h16(xv, packed) == bf, "one 16-bit dtype for every operand")
    if not (packed.shape == (rv + rw + ra + rg, C)):
        raise ValueError(f"packed {tuple(packed.shape)} vs [{rv + rw + ra + rg}, {C}]")
    out = torch.empty(rv + rw + ra + rg, dtype=xv.dtype, device=xv.device)
    _lib.check(_lib.load().rwkv7_rank_gemv(xv.data_ptr(), xw.data_ptr(), xa.data_ptr(), xg.data_ptr(),
                                           packed.data_ptr(), out.data_ptr(), rv, rw, ra, rg, C, bf,
                                           _lib.stream_handle()), "rwkv7_rank_gemv")
    return out


def fused_l2norm_neg_kk_a(kk: Tensor, a: Tensor) -> tuple[Tensor, Tensor]:
    """Per head ``kk / max(||kk||, 1e-12)`` and ``-(that) * a``, [H, 64] (``dplr.py:229-235``)."""
    bf = _h16(kk, a)
    _need(kk.dim() == 2 and kk.shape[1] == N and a.shape == kk.shape, "kk and a must be [H, 64]")
    kn, b = torch.empty_like(kk), torch.empty_like(kk)
    _lib.check(_lib.load().rwkv7_l2norm_neg_kk_a(kk.data_ptr(), a.data_ptr(), kn.data_ptr(), b.data_ptr(),
                                                 kk.shape[0], bf, _lib.stream_handle()), "rwkv7_l2norm_neg_kk_a")
    return kn, b


def fused_gn_rkrk(y: Tensor, r: Tensor, k: Tensor, v: Tensor, r_k: Tensor, ln_xW: Tensor, ln_xB: Tensor) -> Tensor:
    """GroupNorm per head (eps 64e-5) + ``(sum r k r_k) * v``; [H, 64] in, [H*64] out (``dplr.py:237-254``)."""
    bf = _h16(y, r, k, v, r_k, ln_xW, ln_xB)
    _need(y.dim() == 2 and y.shape[1] == N, "y must be [H, 64]")
    for t in (r, k, v, r_k):
        _need(t.shape == y.shape, "r, k, v, r_k must match y")
    H = y.shape[0]
    _need(ln_xW.numel() == H * N and ln_xB.numel() == H * N, "ln_x weight and bias must have H*64 elements")
    out = torch.empty(H * N, dtype=y.dtype, device=y.device)
    _lib.check(_lib.load().rwkv7_gn_rkrk(y.data_ptr(), r.data_ptr(), k.data_ptr(), v.data_ptr(), r_k.data_ptr(),
                                         ln_xW.data_ptr(), ln_xB.data_ptr(), out.data_ptr(), H, bf,
                                         _lib.stream_handle()), "rwkv7_gn_rkrk")
    return out
