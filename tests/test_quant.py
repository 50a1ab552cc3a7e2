"""Int8 weight-only GEMV (``rwkv7_gemv_i8``) and its per-row quantisation.

The reference only plans this path (TODO.md:58-63: int8 weights dequantised
inside the decode GEMV), so there is no reference output to match; the CPU
tests pin the float64 oracle (``oracle.quant_ref``) by brute force, one-hot
rows, linearity and the quantisation round-trip bound, and the GPU tests hold
the kernel to the oracle:

* ``|y - y_ref| <= 2e-6 * sum_k |s q x| + 1e-30`` per row: the kernel
  dequantises exactly (int8 -> fp32 is exact) and sums the products in fp32,
  so its only error is fp32 rounding of the sum; 2e-6 of the term magnitudes
  is ~30 fp32 ulps, well above what a tree sum over K <= 8192 terms shows on
  seeded random data and far below a dropped or doubled term.
* ``quantize_i8`` on the GPU: scales within 1 fp32 ulp of the oracle's, q equal
  to the oracle's except where W / scale lies within 1e-4 of a rounding tie,
  and the round-trip bound ``|W - s q| <= s / 2`` everywhere (plus 8 fp32
  ulps of the quotient W / s, which is rounded before it is rounded to q).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant_ref as Q

GPU_TOL = 2e-6
# W / scale is formed in fp32: near a rounding tie the error can pass s/2 by a
# few ulps of a quotient up to 127; allow 8 of them (a wrong scale or a
# truncating round errs by up to a whole s)
RT_SLACK = 127 * 2.0**-21

# ---------------------------------------------------------------- CPU pins


def test_gemv_i8_ref_matches_brute_force():
    rng = np.random.default_rng(7)
    q = rng.integers(-127, 128, size=(5, 48), dtype=np.int8)
    s = rng.random(5).astype(np.float32)
    x = rng.standard_normal(48).astype(np.float32)
    want = [float(s[n]) * sum(float(x[k]) * int(q[n, k]) for k in range(48)) for n in range(5)]
    np.testing.assert_allclose(Q.gemv_i8_ref(x, q, s), want, rtol=1e-12, atol=1e-12)


def test_gemv_i8_ref_one_hot_rows_and_linearity():
    K = 32
    q = np.zeros((K, K), dtype=np.int8)
    q[np.arange(K), (np.arange(K) * 5) % K] = 1  # row n picks x[5n mod K]
    s = np.linspace(0.5, 2.0, K).astype(np.float32)
    x = np.arange(K, dtype=np.float32) - 10
    np.testing.assert_array_equal(Q.gemv_i8_ref(x, q, s), s.astype(np.float64) * x[(np.arange(K) * 5) % K])
    rng = np.random.default_rng(3)
    q2 = rng.integers(-127, 128, size=(6, K), dtype=np.int8)
    x1, x2 = rng.standard_normal(K), rng.standard_normal(K)
    np.testing.assert_allclose(Q.gemv_i8_ref(2 * x1 - x2, q2, s[:6]),
                               2 * Q.gemv_i8_ref(x1, q2, s[:6]) - Q.gemv_i8_ref(x2, q2, s[:6]), rtol=1e-10, atol=1e-9)


def test_quantize_i8_ref_round_trip_and_exact_cases():
    rng = np.random.default_rng(11)
    W = rng.standard_normal((64, 96)).astype(np.float32) * rng.random((64, 1)).astype(np.float32)
    W[3] = 0.0
    q, s = Q.quantize_i8_ref(W)
    assert q.dtype == np.int8 and s.dtype == np.float32
    assert s[3] == 0 and not q[3].any()
    nz = np.arange(64) != 3
    assert (np.abs(q[nz]).max(axis=1) == 127).all()
    err = np.abs(W - s[:, None].astype(np.float64) * q)
    assert (err <= s[:, None] * (0.5 + RT_SLACK)).all()
    # integer multiples of a power-of-two step come back exactly
    k = rng.integers(-127, 128, size=(8, 40)).astype(np.float32)
    k[:, 0] = 127
    q2, s2 = Q.quantize_i8_ref(k * np.float32(0.25))
    assert np.array_equal(q2, k.astype(np.int8))
    np.testing.assert_array_equal(s2, np.full(8, np.float32(0.25) * np.float32(127) / np.float32(127)))


# ---------------------------------------------------------------- GPU parity

SHAPES = [
    (3, 16),        # one chunk, fewer rows than a wave
    (100, 48),      # ragged rows, partial chunk per lane
    (1024, 1024),   # 0.4B C x C (r/k/v/o)
    (4096, 1024),   # 0.4B FFN key
    (1024, 4096),   # 0.4B FFN value
    (65536, 1024),  # 0.4B head (vocab x C)
    (2048, 8192),   # 1.5B FFN value, the largest K
    (9000, 2064),   # rows not a multiple of 4, K not a power of two
]


@pytest.mark.gpu
@pytest.mark.parametrize("N,Kd", SHAPES)
def test_gemv_i8_matches_oracle(N, Kd, cuda):
    from rwkv_tl_amd import kernels as K

    g = torch.Generator().manual_seed(N * 31 + Kd)
    q = torch.randint(-127, 128, (N, Kd), dtype=torch.int8, generator=g)
    s = torch.rand(N, generator=g) * 1e-2 + 1e-4
    x = torch.randn(Kd, generator=g)
    y = K.gemv_i8(x.to(cuda), q.to(cuda), s.to(cuda)).cpu().double().numpy()
    want = Q.gemv_i8_ref(x.numpy(), q.numpy(), s.numpy())
    bound = GPU_TOL * Q.gemv_i8_abs_ref(x.numpy(), q.numpy(), s.numpy()) + 1e-30
    bad = np.abs(y - want) > bound
    assert not bad.any(), f"{bad.sum()} rows off; worst {np.abs(y - want)[bad].max():.3e}"


@pytest.mark.gpu
def test_gemv_i8_extremes_and_zero_rows(cuda):
    from rwkv_tl_amd import kernels as K

    N, Kd = 64, 1024
    q = torch.full((N, Kd), -127, dtype=torch.int8)
    q[1::2] = 127
    q[5] = 0
    s = torch.full((N,), 0.5)
    s[7] = 0.0
    x = torch.ones(Kd)
    y = K.gemv_i8(x.to(cuda), q.to(cuda), s.to(cuda)).cpu().numpy()
    want = Q.gemv_i8_ref(x.numpy(), q.numpy(), s.numpy())
    np.testing.assert_array_equal(y, want.astype(np.float32))  # small integer sums are exact in fp32


@pytest.mark.gpu
def test_quantize_i8_then_gemv_tracks_f16_gemv(cuda):
    from rwkv_tl_amd import kernels as K

    g = torch.Generator().manual_seed(5)
    W = (torch.randn(4096, 1024, generator=g) * 0.02).half()
    q, s = K.quantize_i8(W.to(cuda))
    qr, sr = Q.quantize_i8_ref(W.float().numpy())
    np.testing.assert_allclose(s.cpu().numpy(), sr, rtol=1.2e-7, atol=0)
    ratio = W.float().numpy() / np.where(sr > 0, sr, 1)[:, None]
    near_tie = np.abs(np.abs(ratio - np.floor(ratio)) - 0.5) < 1e-4
    diff = q.cpu().numpy() != qr
    assert not (diff & ~near_tie).any()
    err = np.abs(W.float().numpy() - s.cpu().numpy()[:, None].astype(np.float64) * q.cpu().numpy())
    assert (err <= s.cpu().numpy()[:, None] * (0.5 + RT_SLACK)).all()
    # the int8 product stays within the quantisation error of the f16 one
    x = torch.randn(1024, generator=g)
    y8 = K.gemv_i8(x.to(cuda), q, s).cpu().double()
    y16 = K.gemv(x.to(cuda), W.to(cuda)).cpu().double()
    qerr = s.cpu().double() / 2 * x.abs().double().sum()  # sum_k |W - s q| |x| <= s/2 sum |x|
    assert ((y8 - y16).abs() <= qerr + 1e-4).all()


@pytest.mark.gpu
def test_gemv_i8_rejects_bad_arguments(cuda):
    from rwkv_tl_amd import kernels as K

    q = torch.zeros(8, 24, dtype=torch.int8, device=cuda)
    with pytest.raises((ValueError, RuntimeError)):
        K.gemv_i8(torch.zeros(24, device=cuda), q, torch.ones(8, device=cuda))  # K % 16
    with pytest.raises(ValueError):
        K.gemv_i8(torch.zeros(16), torch.zeros(8, 16, dtype=torch.int8), torch.ones(8))  # CPU tensors
