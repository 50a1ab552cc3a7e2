"""The HIP operators registered with ``torch.library`` as ``torch.ops.rwkv_tl.*``.

Drop-in for ``rwkv_tl.operators`` (``src/rwkv_tl/operators/__init__.py:112-375``):
the same namespace, operator names and schemas, with in-place arguments
declared ``Tensor(a!)``, so code written against ``torch.ops.rwkv_tl`` (as
``demo/_rwkv7_base.py:115-119,149,281`` is) runs on the HIP kernels and can be
traced by ``torch.compile``.

Each operator has two implementations:

* ``CUDA`` (the ROCm device in PyTorch-ROCm): the ``rwkv_tl_amd.kernels``
  function of the same name, i.e. one C-ABI call into ``librwkv7_hip.so``.
* ``Meta``: outputs of the right shape and dtype with no data, which is what
  ``torch.compile`` / FakeTensor tracing runs.

There is no ``CPU`` implementation (the reference has a plain-torch one): a
CPU tensor raises torch's "no kernel for the CPU backend" error instead of
silently taking another code path.

Importing this module registers the operators once per process. It uses the
reference's ``rwkv_tl`` namespace, so it cannot be imported into a process
that has already imported ``rwkv_tl`` itself.
"""

from __future__ import annotations

from collections.abc import Callable

import torch
from torch import Tensor

from . import kernels as K

NAMESPACE = "rwkv_tl"

# name -> (schema, CUDA implementation, Meta implementation)
_T = "Tensor"


def _like(n: int) -> Callable[..., tuple[Tensor, ...]]:
    return lambda x, *_: tuple(torch.empty_like(x) for _ in range(n))


def _dplr(S, R, W, K_, V, A, B) -> Tensor:
    y, _ = K.fused_dplr(S, R, W, K_, V, A, B)
    return y


def _lerp6_rkv(x, prev, x_r, x_w, x_k, x_v, x_a, x_g, x_copy, rWt_stack):
    r, k, v, xv, xw, xa, xg = K.fused_lerp6_rkv_copy(x, prev, x_r, x_w, x_k, x_v, x_a, x_g, x_copy, rWt_stack)
    # r, k and v are views of one stacked result: outputs must not share storage
    return r.clone(), k.clone(), v.clone(), xv, xw, xa, xg


def _lerp6_copy(*args):
    return tuple(t.clone() for t in K.fused_lerp6_copy(*args))


OPS: dict[str, tuple[str, Callable, Callable]] = {
    "fused_lerp6_copy": (
        "(Tensor x, Tensor prev, Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, Tensor x_g,"
        " Tensor(a!) x_copy) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
        _lerp6_copy,
        _like(6),
    ),
    "fused_lerp1_copy": (
        "(Tensor x, Tensor prev, Tensor w, Tensor(a!) x_copy) -> Tensor",
        K.fused_lerp1_copy,
        lambda x, *_: torch.empty_like(x),
    ),
    "fused_w_gate": ("(Tensor x, Tensor w0) -> Tensor", K.fused_w_gate, lambda x, *_: torch.empty_like(x)),
    "fused_v_gate": (
        "(Tensor v, Tensor v_first, Tensor v0, Tensor v12) -> Tensor",
        K.fused_v_gate,
        lambda v, *_: torch.empty_like(v),
    ),
    "fused_a_kk_k": (
        "(Tensor a0, Tensor a_x, Tensor k, Tensor k_k, Tensor k_a) -> (Tensor, Tensor, Tensor)",
        K.fused_a_kk_k,
        _like(3),
    ),
    "fused_gates": (
        "(Tensor vr, Tensor wr, Tensor ar, Tensor gr, Tensor v, Tensor v_first, Tensor k, Tensor v2t,"
        " Tensor w2t, Tensor a2t, Tensor g2t, Tensor v0, Tensor w0, Tensor a0, Tensor k_k, Tensor k_a)"
        " -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
        K.fused_gates,
        lambda vr, wr, ar, gr, v, *_: tuple(torch.empty_like(v) for _ in range(6)),
    ),
    "fused_rank_gemv": (
        "(Tensor xv, Tensor xw, Tensor xa, Tensor xg, Tensor packed, int rv, int rw, int ra, int rg) -> Tensor",
        K.fused_rank_gemv,
        lambda xv, xw, xa, xg, packed, *_: torch.empty(packed.shape[0], dtype=xv.dtype, device=xv.device),
    ),
    "fused_l2norm_neg_kk_a": ("(Tensor kk, Tensor a) -> (Tensor, Tensor)", K.fused_l2norm_neg_kk_a, _like(2)),
    "fused_gn_rkrk": (
        "(Tensor y, Tensor r, Tensor k, Tensor v, Tensor r_k, Tensor ln_xW, Tensor ln_xB) -> Tensor",
        K.fused_gn_rkrk,
        lambda y, *_: torch.empty(y.numel(), dtype=y.dtype, device=y.device),
    ),
    "fused_dplr": (
        "(Tensor(a!) S, Tensor R, Tensor W, Tensor K, Tensor V, Tensor A, Tensor B) -> Tensor",
        _dplr,
        lambda S, R, *_: torch.empty_like(R),
    ),
    "fused_lerp6_rkv_copy": (
        "(Tensor x, Tensor prev, Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, Tensor x_g,"
        " Tensor(a!) x_copy, Tensor rWt_stack) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
        _lerp6_rkv,
        _like(7),
    ),
    "fused_rkv_gemm": (
        "(Tensor xr, Tensor xk, Tensor xv, Tensor Wb) -> Tensor",
        K.fused_rkv_gemm,
        lambda xr, *_: torch.empty(3, xr.shape[0], xr.shape[1], dtype=xr.dtype, device=xr.device),
    ),
}

# The training operator (no counterpart in the reference's registry yet; its
# TODO.md:46-54 plans exactly this: a DPLR custom op with register_autograd).
# Functional, f32: S [H,64,64] or [B,H,64,64] is not modified; returns (y, S_T).
TRAIN_OPS: dict[str, tuple[str, Callable, Callable]] = {
    "fused_dplr_seq": (
        "(Tensor S, Tensor R, Tensor W, Tensor K, Tensor V, Tensor A, Tensor B) -> (Tensor, Tensor)",
        K.dplr_seq_forward,
        lambda S, R, *_: (torch.empty_like(R), torch.empty_like(S)),
    ),
}


def _dplr_seq_setup(ctx, inputs, output) -> None:
    ctx.save_for_backward(*inputs)


def _dplr_seq_backward(ctx, gy, gS):
    S, R, W, K_, V, A, B = ctx.saved_tensors
    if gy is None:
        gy = torch.zeros_like(R)
    return K.dplr_seq_backward(S, R, W, K_, V, A, B, gy.contiguous(), None if gS is None else gS.contiguous())


_registered = False


def register() -> None:
    """Define every operator with its CUDA and Meta implementations (idempotent)."""
    global _registered
    if _registered:
        return
    for name, (schema, cuda, meta) in {**OPS, **TRAIN_OPS}.items():
        qual = f"{NAMESPACE}::{name}"
        torch.library.define(qual, schema)
        torch.library.impl(qual, "CUDA")(cuda)
        torch.library.impl(qual, "Meta")(meta)
    torch.library.register_autograd(
        f"{NAMESPACE}::fused_dplr_seq", _dplr_seq_backward, setup_context=_dplr_seq_setup
    )
    _registered = True


register()
