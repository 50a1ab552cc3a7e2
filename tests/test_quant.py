"""Weight-only quantised GEMVs: int8 (``rwkv7_gemv_i8``) and any4
(``rwkv7_gemv_any4``), and their per-row quantisers.

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
  ulps of the quotient W / s, which the oracle forms in fp32 before rounding
  it to q).
* any4: the same bar for ``gemv_any4`` against the float64 oracle on the
  same (codes, table) pair -- a table entry is an exact f16, so again the
  only error is the fp32 sum. The quantiser (a per-row k-means) has no
  reference output; it is held to what defines it: every weight takes its
  nearest table entry, a row of at most 16 distinct f16 values comes back
  exactly, the tables are ascending, and every row's reconstruction error is
  at most that of the uniform 16-level grid over [min, max] the iterations
  start from (below symmetric absmax / 7 4-bit quantisation on average).
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


def test_gemv_any4_ref_matches_brute_force():
    rng = np.random.default_rng(17)
    codes = rng.integers(0, 256, size=(5, 24), dtype=np.uint8)  # K = 48
    lut = rng.standard_normal((5, 16)).astype(np.float16)
    x = rng.standard_normal(48).astype(np.float32)
    want = []
    for n in range(5):
        acc = 0.0
        for k in range(48):
            byte = int(codes[n, k // 2])
            code = byte & 15 if k % 2 == 0 else byte >> 4
            acc += float(x[k]) * float(lut[n, code])
        want.append(acc)
    np.testing.assert_allclose(Q.gemv_any4_ref(x, codes, lut), want, rtol=1e-12, atol=1e-12)


def test_gemv_any4_ref_one_hot_constant_and_linear():
    K = 32
    lut = np.zeros((16, 16), dtype=np.float16)
    lut[:, 1] = 1.0
    codes = np.zeros((16, K // 2), dtype=np.uint8)
    for n in range(16):  # row n: code 1 only at column 2n (low nibble) -> picks x[2n]
        codes[n, n] = 1
    x = np.arange(K, dtype=np.float32) - 7
    np.testing.assert_array_equal(Q.gemv_any4_ref(x, codes, lut), x[2 * np.arange(16)].astype(np.float64))
    for n in range(16):  # high nibble -> x[2n + 1]
        codes[n, n] = 0x10
    np.testing.assert_array_equal(Q.gemv_any4_ref(x, codes, lut), x[2 * np.arange(16) + 1].astype(np.float64))
    rng = np.random.default_rng(4)
    c = np.float16(0.375)
    const = np.full((3, 16), c, dtype=np.float16)
    rc = rng.integers(0, 256, size=(3, K // 2), dtype=np.uint8)
    np.testing.assert_allclose(Q.gemv_any4_ref(x, rc, const), np.full(3, float(c) * x.astype(np.float64).sum()))
    lut2 = rng.standard_normal((3, 16)).astype(np.float16)
    x1, x2 = rng.standard_normal(K), rng.standard_normal(K)
    np.testing.assert_allclose(Q.gemv_any4_ref(2 * x1 - x2, rc, lut2),
                               2 * Q.gemv_any4_ref(x1, rc, lut2) - Q.gemv_any4_ref(x2, rc, lut2), rtol=1e-10,
                               atol=1e-9)


def _any4_properties(W: torch.Tensor, codes: torch.Tensor, lut: torch.Tensor) -> None:
    from rwkv_tl_amd.weight import dequantize_rows_any4

    w = W.float().cpu()
    codes, lut = codes.cpu(), lut.cpu()
    N, K = w.shape
    assert codes.dtype == torch.uint8 and codes.shape == (N, K // 2)
    assert lut.dtype == torch.float16 and lut.shape == (N, 16)
    lf = lut.float()
    assert bool((lf[:, 1:] >= lf[:, :-1]).all()), "tables ascending"
    deq = dequantize_rows_any4(codes, lut)
    np.testing.assert_array_equal(deq.numpy(), Q.dequant_any4_ref(codes.numpy(), lut.numpy()).astype(np.float32))
    # nearest entry: no other entry of the row's table is closer (ties allowed)
    best = (w[:, :, None] - lf[:, None, :]).abs().min(dim=2).values
    assert bool(((w - deq).abs() <= best + 1e-7 * w.abs().clamp(min=1e-30)).all()), "a weight not at its nearest entry"
    # never worse than the uniform 16-level grid over [min, max] it starts from
    # (Lloyd steps do not increase the squared error; 2% for the f16 table),
    # and on these Gaussian rows clearly better than symmetric absmax / 7
    lo, hi = w.amin(1, keepdim=True), w.amax(1, keepdim=True)
    step = ((hi - lo) / 15).clamp(min=1e-30)
    grid = lo + torch.round((w - lo) / step).clamp(0, 15) * step
    e4 = ((w - deq) ** 2).mean(1)
    assert bool((e4 <= 1.02 * ((w - grid) ** 2).mean(1) + 1e-12).all()), "worse than the uniform grid"
    s = w.abs().amax(1, keepdim=True) / 7
    sym = torch.round(w / s.clamp(min=1e-30)).clamp(-7, 7) * s
    assert float(e4.mean()) < 0.9 * float(((w - sym) ** 2).mean())


def test_quantize_any4_properties_cpu():
    from rwkv_tl_amd.weight import dequantize_rows_any4, quantize_rows_any4

    g = torch.Generator().manual_seed(21)
    W = (torch.randn(64, 256, generator=g) * 0.02).half()
    W[5] = W[5] * 40  # one wide row
    codes, lut = quantize_rows_any4(W)
    _any4_properties(W, codes, lut)
    # rows with at most 16 distinct f16 values come back exactly
    vals = (torch.randn(3, 16, generator=g) * 0.1).half()
    pick = torch.randint(0, 16, (3, 96), generator=g)
    E = vals.gather(1, pick)
    ce, le = quantize_rows_any4(E)
    assert torch.equal(dequantize_rows_any4(ce, le), E.float())


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


@pytest.mark.gpu
@pytest.mark.parametrize("N,Kd", SHAPES)
def test_gemv_any4_matches_oracle(N, Kd, cuda):
    from rwkv_tl_amd import kernels as K

    g = torch.Generator().manual_seed(N * 37 + Kd)
    codes = torch.randint(0, 256, (N, Kd // 2), dtype=torch.uint8, generator=g)
    lut = (torch.randn(N, 16, generator=g) * 0.05).half()
    x = torch.randn(Kd, generator=g)
    y = K.gemv_any4(x.to(cuda), codes.to(cuda), lut.to(cuda)).cpu().double().numpy()
    want = Q.gemv_any4_ref(x.numpy(), codes.numpy(), lut.numpy())
    bound = GPU_TOL * Q.gemv_any4_abs_ref(x.numpy(), codes.numpy(), lut.numpy()) + 1e-30
    bad = np.abs(y - want) > bound
    assert not bad.any(), f"{bad.sum()} rows off; worst {np.abs(y - want)[bad].max():.3e}"


@pytest.mark.gpu
def test_quantize_any4_on_gpu_then_gemv(cuda):
    """The quantiser on the GPU meets the same properties, and the any4
    product stays within its quantisation error of the f16 product."""
    from rwkv_tl_amd import kernels as K

    g = torch.Generator().manual_seed(9)
    W = (torch.randn(4096, 1024, generator=g) * 0.02).half()
    codes, lut = K.quantize_any4(W.to(cuda))
    _any4_properties(W, codes, lut)
    x = torch.randn(1024, generator=g)
    y4 = K.gemv_any4(x.to(cuda), codes, lut).cpu().double().numpy()
    want = Q.gemv_any4_ref(x.numpy(), codes.cpu().numpy(), lut.cpu().numpy())
    bound = GPU_TOL * Q.gemv_any4_abs_ref(x.numpy(), codes.cpu().numpy(), lut.cpu().numpy()) + 1e-30
    assert (np.abs(y4 - want) <= bound).all()
    y16 = W.double().numpy() @ x.double().numpy()
    # per-row error of a 4-bit product: a few percent of the row's norm times |x|
    rel = np.linalg.norm(y4 - y16) / np.linalg.norm(y16)
    assert rel < 0.15, f"any4 product off the f16 one by {rel:.3f}"


@pytest.mark.gpu
def test_gemv_any4_rejects_bad_arguments(cuda):
    from rwkv_tl_amd import _lib
    from rwkv_tl_amd import kernels as K

    codes = torch.zeros(8, 8, dtype=torch.uint8, device=cuda)  # K = 16
    lut = torch.zeros(8, 16, dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError):
        K.gemv_any4(torch.zeros(15, device=cuda), codes, lut)
    with pytest.raises(ValueError):
        K.gemv_any4(torch.zeros(16, device=cuda), codes, lut.float())
    lib = _lib.load()
    y = torch.empty(8, device=cuda)
    x = torch.zeros(16, device=cuda)
    rc = lib.rwkv7_gemv_any4(x.data_ptr(), codes.data_ptr(), 4, lut.data_ptr(), y.data_ptr(), 8, 16,
                             _lib.stream_handle())
    assert rc == 2  # RWKV7_ESHAPE: row stride shorter than K / 2
