"""torch.ops.rwkv_tl.* (rwkv_tl_amd.operators): the reference's operator
names and schemas (src/rwkv_tl/operators/__init__.py:112-375), Meta shapes for
tracing, no CPU kernel, and on the GPU the same results as the direct kernel
calls, in-place arguments mutated, and torch.compile tracing through them."""

from __future__ import annotations

import pytest
import torch

import rwkv_tl_amd  # noqa: F401  (registers the operators)
from rwkv_tl_amd import kernels as K
from rwkv_tl_amd.operators import OPS

ops = torch.ops.rwkv_tl

# The reference's schemas (operators/__init__.py:112-375), as torch prints them.
REFERENCE_SCHEMAS = {
    "fused_lerp6_copy": "(Tensor x, Tensor prev, Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, "
    "Tensor x_g, Tensor(a!) x_copy) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    "fused_lerp1_copy": "(Tensor x, Tensor prev, Tensor w, Tensor(a!) x_copy) -> Tensor",
    "fused_w_gate": "(Tensor x, Tensor w0) -> Tensor",
    "fused_v_gate": "(Tensor v, Tensor v_first, Tensor v0, Tensor v12) -> Tensor",
    "fused_a_kk_k": "(Tensor a0, Tensor a_x, Tensor k, Tensor k_k, Tensor k_a) -> (Tensor, Tensor, Tensor)",
    "fused_gates": "(Tensor vr, Tensor wr, Tensor ar, Tensor gr, Tensor v, Tensor v_first, Tensor k, Tensor v2t, "
    "Tensor w2t, Tensor a2t, Tensor g2t, Tensor v0, Tensor w0, Tensor a0, Tensor k_k, Tensor k_a) "
    "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    "fused_rank_gemv": "(Tensor xv, Tensor xw, Tensor xa, Tensor xg, Tensor packed, int rv, int rw, int ra, int rg) "
    "-> Tensor",
    "fused_l2norm_neg_kk_a": "(Tensor kk, Tensor a) -> (Tensor, Tensor)",
    "fused_gn_rkrk": "(Tensor y, Tensor r, Tensor k, Tensor v, Tensor r_k, Tensor ln_xW, Tensor ln_xB) -> Tensor",
    "fused_dplr": "(Tensor(a!) S, Tensor R, Tensor W, Tensor K, Tensor V, Tensor A, Tensor B) -> Tensor",
    "fused_lerp6_rkv_copy": "(Tensor x, Tensor prev, Tensor x_r, Tensor x_w, Tensor x_k, Tensor x_v, Tensor x_a, "
    "Tensor x_g, Tensor(a!) x_copy, Tensor rWt_stack) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    "fused_rkv_gemm": "(Tensor xr, Tensor xk, Tensor xv, Tensor Wb) -> Tensor",
}

C, H, RV, RW, RA, RG = 256, 4, 16, 32, 32, 64


def _args(name: str, dev: str, g: torch.Generator | None = None):
    """Arguments of each op at C=256 (H=4) on `dev` ("meta" or "cuda")."""
    def t(*shape, dt=torch.float16, scale=1.0):
        if dev == "meta":
            return torch.empty(*shape, dtype=dt, device="meta")
        return (torch.randn(*shape, generator=g) * scale).to(dt).to(dev)

    vec = lambda: t(C)  # noqa: E731
    return {
        "fused_lerp6_copy": lambda: (vec(), vec(), *[t(C, scale=0.5) for _ in range(6)], vec()),
        "fused_lerp1_copy": lambda: (vec(), vec(), t(C, scale=0.5), vec()),
        "fused_w_gate": lambda: (vec(), vec()),
        "fused_v_gate": lambda: (vec(), vec(), vec(), vec()),
        "fused_a_kk_k": lambda: tuple(vec() for _ in range(5)),
        "fused_gates": lambda: (t(RV), t(RW), t(RA), t(RG), vec(), vec(), vec(), t(C, RV, scale=0.1),
                                t(C, RW, scale=0.1), t(C, RA, scale=0.1), t(C, RG, scale=0.1),
                                vec(), vec(), vec(), vec(), vec()),
        "fused_rank_gemv": lambda: (vec(), vec(), vec(), vec(), t(RV + RW + RA + RG, C, scale=0.05), RV, RW, RA, RG),
        "fused_l2norm_neg_kk_a": lambda: (t(H, 64), t(H, 64)),
        "fused_gn_rkrk": lambda: (t(H, 64), t(H, 64), t(H, 64), t(H, 64), t(H, 64), vec(), vec()),
        "fused_dplr": lambda: (t(H, 64, 64, dt=torch.float32, scale=0.1), t(H, 64), t(H, 64, scale=0).add(0.9)
                               if dev != "meta" else t(H, 64), t(H, 64), t(H, 64), t(H, 64, scale=0.1),
                               t(H, 64, scale=0.1)),
        "fused_lerp6_rkv_copy": lambda: (vec(), vec(), *[t(C, scale=0.5) for _ in range(6)], vec(),
                                         t(3, C, C, scale=0.05)),
        "fused_rkv_gemm": lambda: (t(8, C), t(8, C), t(8, C), t(3, C, C, scale=0.05)),
    }[name]()


def test_schemas_match_the_reference():
    assert set(OPS) == set(REFERENCE_SCHEMAS)
    for name, want in REFERENCE_SCHEMAS.items():
        assert str(getattr(ops, name).default._schema) == f"rwkv_tl::{name}{want}"


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_meta_shapes(name):
    out = getattr(ops, name)(*_args(name, "meta"))
    outs = out if isinstance(out, tuple) else (out,)
    assert all(o.device.type == "meta" for o in outs)
    if name == "fused_rkv_gemm":
        assert outs[0].shape == (3, 8, C)
    elif name in ("fused_dplr", "fused_l2norm_neg_kk_a"):
        assert all(o.shape == (H, 64) for o in outs)
    elif name == "fused_rank_gemv":
        assert outs[0].shape == (RV + RW + RA + RG,)
    else:
        assert all(o.shape == (C,) for o in outs)


def test_no_cpu_kernel():
    with pytest.raises(NotImplementedError):
        ops.fused_w_gate(torch.zeros(C, dtype=torch.float16), torch.zeros(C, dtype=torch.float16))


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_ops_match_direct_kernel_calls(name):
    g = torch.Generator().manual_seed(sum(map(ord, name)))
    args = _args(name, "cuda", g)
    mutated = {"fused_dplr": 0, "fused_lerp6_copy": 8, "fused_lerp1_copy": 3, "fused_lerp6_rkv_copy": 8}.get(name)
    a1 = tuple(x.clone() if isinstance(x, torch.Tensor) else x for x in args)
    a2 = tuple(x.clone() if isinstance(x, torch.Tensor) else x for x in args)
    got = getattr(ops, name)(*a1)
    want = getattr(K, name)(*a2)
    if name == "fused_dplr":
        want = want[0]
    got = got if isinstance(got, tuple) else (got,)
    want = want if isinstance(want, tuple) else (want,)
    assert len(got) == len(want)
    for x, y in zip(got, want):
        assert torch.equal(x, y)
    if mutated is not None:
        assert torch.equal(a1[mutated], a2[mutated]) and not torch.equal(a1[mutated], args[mutated])


@pytest.mark.gpu
def test_torch_compile_traces_through_ops():
    g = torch.Generator().manual_seed(0)
    x, prev, w0 = (torch.randn(C, generator=g).half().cuda() for _ in range(3))
    mus = [torch.rand(C, generator=g).half().cuda() for _ in range(6)]
    S = torch.randn(H, 64, 64, generator=g).cuda() * 0.1
    kk, a, r = (torch.randn(H, 64, generator=g).half().cuda() for _ in range(3))

    def step(x, prev, x_copy, S):
        xr, xw, xk, xv, xa, xg = ops.fused_lerp6_copy(x, prev, *mus, x_copy)
        w = ops.fused_w_gate(xw, w0)
        kn, b = ops.fused_l2norm_neg_kk_a(kk, a)
        y = ops.fused_dplr(S, r, w.view(H, 64), xk.view(H, 64), xv.view(H, 64), kn, b)
        return y, xr + xg

    cx, cS = torch.empty_like(x), S.clone()
    ex, eS = torch.empty_like(x), S.clone()
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    got = compiled(x, prev, cx, cS)
    want = step(x, prev, ex, eS)
    for u, v in zip(got, want):
        assert torch.equal(u, v)
    assert torch.equal(cx, ex) and torch.equal(cx, x) and torch.equal(cS, eS) and not torch.equal(cS, S)
