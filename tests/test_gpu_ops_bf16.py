"""The operator-level API on bfloat16 operands (the reference's
``rwkv_tl.kernels.bf16`` namespace, ``src/rwkv_tl/kernels/bf16.py:13-30``).

Every operator of ``rwkv_tl_amd.kernels`` takes float16 or bfloat16; these
tests call each with bfloat16 inputs and compare with the same references as
the float16 tests in ``test_gpu_kernels.py`` -- the oracle's operator
restatements, or fp32 torch, computed on the very same bf16 values. Both sides
compute in fp32, so the only difference is the rounding of a bf16 output
(8 significant bits, half an ulp = 2^-9 relative): outputs within rtol 8e-3
and atol 8e-3 (two half-ulps at these magnitudes), f32 outputs (GEMV, GEMM,
LayerNorm) at the fp16 tests' bars, and the wkv7 fp32 state at 1e-5.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import rwkv7_ref as R
from rwkv_tl_amd import kernels as K

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
TOL = dict(rtol=8e-3, atol=8e-3)


def _b(g, *shape, scale=1.0, shift=0.0):
    return (torch.randn(*shape, generator=g) * scale + shift).to(BF)


def _rel(x, y):
    return float((x.double() - y.double()).norm() / y.double().norm().clamp_min(1e-30))


@pytest.mark.parametrize("B,H,T,w_f32", [(2, 4, 40, True), (1, 2, 1, False), (3, 3, 17, False)])
def test_wkv7_bf16_matches_oracle(B, H, T, w_f32, cuda):
    g = torch.Generator().manual_seed(B * 10 + T)
    shp = (B, T, H, 64)
    r, k, v = (torch.randn(shp, generator=g).to(BF) for _ in range(3))
    w = torch.exp(-torch.exp(torch.randn(shp, generator=g) * 0.5 - 0.5))
    kap = F.normalize(k.float(), dim=-1)
    a = (-kap).to(BF)
    b = (kap * torch.sigmoid(torch.randn(shp, generator=g))).to(BF)
    w = w if w_f32 else w.to(BF)
    S0 = torch.randn(B, H, 64, 64, generator=g) * 0.1
    y_ref, S_ref = R.wkv7_scan(S0, r, w, k, v, a, b)
    S = S0.clone().to(cuda)
    y = K.wkv7(S, *(t.to(cuda) for t in (r, w, k, v, a, b)))
    assert y.dtype == BF
    assert _rel(S.cpu(), S_ref) < 1e-5
    torch.testing.assert_close(y.cpu().float(), y_ref.float(), **TOL)


def test_gemv_gemm_layernorm_lerp_bf16(cuda):
    g = torch.Generator().manual_seed(3)
    W = (torch.randn(1024, 1024, generator=g) * 0.02).to(BF)
    x = torch.randn(1024, generator=g)
    torch.testing.assert_close(K.gemv(x.to(cuda), W.to(cuda)).cpu(), W.float() @ x, rtol=1e-4, atol=1e-4)
    for M, N, Kd in ((16, 1024, 1024), (128, 4096, 1024), (2048, 8192, 1024)):
        A = torch.randn(M, Kd, generator=g).to(BF)
        Wm = (torch.randn(N, Kd, generator=g) * 0.05).to(BF)
        ref = A.float() @ Wm.float().T
        out = K.gemm(A.to(cuda), Wm.to(cuda), "f32").cpu()
        torch.testing.assert_close(out, ref, rtol=1e-4, atol=1e-4)
        o16 = K.gemm(A.to(cuda), Wm.to(cuda), "f16")
        assert o16.dtype == BF
        torch.testing.assert_close(o16.cpu().float(), ref.to(BF).float(), **TOL)
    xl = (torch.randn(5, 1024, generator=g) * 3 + 1).to(BF)
    lw, lb = torch.randn(1024, generator=g), torch.randn(1024, generator=g)
    torch.testing.assert_close(K.layer_norm(xl.to(cuda), lw.to(cuda), lb.to(cuda)).cpu(),
                               F.layer_norm(xl.float(), (1024,), lw, lb), rtol=1e-5, atol=1e-5)
    xs, prev = _b(g, 768), _b(g, 768)
    mus = [_b(g, 768) for _ in range(6)]
    for mu, o in zip(mus, K.fused_lerp6(xs.to(cuda), prev.to(cuda), *(m.to(cuda) for m in mus))):
        assert o.dtype == BF
        ref = xs.float() + mu.float() * (prev.float() - xs.float())
        torch.testing.assert_close(o.cpu().float(), ref.to(BF).float(), **TOL)


def test_stage_operators_bf16_match_oracle(cuda):
    g = torch.Generator().manual_seed(11)
    C = 1024
    dev = lambda *ts: [t.to(cuda) for t in ts]  # noqa: E731
    x, w0, v, vf, v0, v12, a0, ax, k, kk, ka = (_b(g, C) for _ in range(11))
    torch.testing.assert_close(K.fused_w_gate(*dev(x, w0)).cpu().float(), R.w_gate(x, w0), **TOL)
    torch.testing.assert_close(K.fused_v_gate(*dev(v, vf, v0, v12)).cpu().float(), R.v_gate(v, vf, v0, v12), **TOL)
    for gg, ww in zip(K.fused_a_kk_k(*dev(a0, ax, k, kk, ka)), R.a_kk_k(a0, ax, k, kk, ka)):
        assert gg.dtype == BF
        torch.testing.assert_close(gg.cpu().float(), ww, **TOL)
    ranks = (32, 64, 64, 128)
    vr, wr, ar, gr = (_b(g, r) for r in ranks)
    mats = [_b(g, C, r, scale=0.1) for r in ranks]
    vecs = [_b(g, C) for _ in range(8)]
    args = (vr, wr, ar, gr, *vecs[:3], *mats, *vecs[3:])
    for name, gg, ww in zip(("v", "w", "a", "kk", "k", "g"), K.fused_gates(*dev(*args)), R.gates(*args)):
        torch.testing.assert_close(gg.cpu().float(), ww, **TOL, msg=name)
    xs4 = [_b(g, C) for _ in range(4)]
    packed = _b(g, sum(ranks), C, scale=0.05)
    torch.testing.assert_close(K.fused_rank_gemv(*dev(*xs4), packed.to(cuda), *ranks).cpu().float(),
                               R.rank_gemv(*xs4, packed, *ranks), **TOL)
    H = 16
    kh, ah = _b(g, H, 64), torch.rand(H, 64, generator=g).to(BF)
    kh[0] = 0
    kn, bb = K.fused_l2norm_neg_kk_a(*dev(kh, ah))
    wkn, wb = R.l2norm_neg_kk_a(kh, ah)
    torch.testing.assert_close(kn.cpu().float(), wkn, **TOL)
    torch.testing.assert_close(bb.cpu().float(), wb, **TOL)
    y, r, kx, vx, rk = (_b(g, H, 64) for _ in range(5))
    lw, lb = _b(g, H * 64, scale=0.2, shift=1.0), _b(g, H * 64, scale=0.2)
    got = K.fused_gn_rkrk(*dev(y, r, kx, vx, rk, lw, lb))
    assert got.dtype == BF
    torch.testing.assert_close(got.cpu().float(), R.gn_rkrk(y, r, kx, vx, rk, lw, lb), rtol=2e-2, atol=2e-2)


def test_mixed_16bit_dtypes_are_rejected(cuda):
    h = torch.zeros(8, dtype=torch.float16, device=cuda)
    bf = torch.zeros(8, dtype=BF, device=cuda)
    with pytest.raises(ValueError, match="mixed 16-bit"):
        K.fused_w_gate(h, bf)
    with pytest.raises(ValueError):
        K.gemm(torch.zeros(4, 16, dtype=torch.float16, device=cuda), torch.zeros(8, 16, dtype=BF, device=cuda))
