// Decode-time GEMV over int8 weights with one fp32 scale per output row
// (symmetric weight-only quantisation): y[n] = scale[n] * sum_k x[k] q[n, k].
//
// This is the fused-dequant GEMV the reference plans as its quantisation step
// (TODO.md:58-63: int8 weights dequantised inside the hand-written GEMV, the
// recurrent state kept fp32); it has no kernel there yet. Decode streams every
// weight once per token, so one byte per weight instead of two halves the
// bytes of the HBM-bound GEMVs.
//
// Q is [N, K] int8, K-contiguous rows of ldq bytes. A wavefront owns ROWS
// consecutive rows at a time; lane l reads the 16-byte chunks l, l+64, ... of
// each row, so one wave instruction streams 1 KiB of contiguous weights. x is
// held in registers for the whole launch (16 floats per chunk a lane owns).
// Dequantisation is exact: each byte is sign-extended and converted to fp32,
// the products are summed in fp32 and the row scale is applied once.
#include "rwkv7_kernels.h"

namespace rwkv7 {
namespace {

// 16 signed bytes -> 16 exact floats (bit-field sign extension + convert)
RWKV7_DEV void i8x16_to_f(const uint4 v, float f[16]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int b = 0; b < 4; ++b) f[4 * i + b] = (float)((int32_t)(w[i] << (24 - 8 * b)) >> 24);
}

template <int CPL, int ROWS>
__global__ __launch_bounds__(256) void gemv_i8_kernel(const float *__restrict__ x, const int8_t *__restrict__ Q,
                                                      int64_t ldq, const float *__restrict__ scale,
                                                      float *__restrict__ y, int N, int K) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nwave = gridDim.x * 4;
  const int nchunk = K >> 4;
  float xb[CPL][16];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int j = lane + kWave * c;
    if (j < nchunk) {
      const float4 *p = reinterpret_cast<const float4 *>(x) + 4 * j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 u = p[i];
        xb[c][4 * i] = u.x;
        xb[c][4 * i + 1] = u.y;
        xb[c][4 * i + 2] = u.z;
        xb[c][4 * i + 3] = u.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) xb[c][e] = 0.f;
    }
  }
  const int ngroups = (N + ROWS - 1) / ROWS;
  for (int g = wave; g < ngroups; g += nwave) {
    const int n0 = g * ROWS;
    uint4 w[ROWS][CPL];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const int n = min(n0 + r, N - 1);  // rows past N re-read the last row; their sums are dropped
      const uint4 *row = reinterpret_cast<const uint4 *>(Q + (int64_t)n * ldq);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int j = lane + kWave * c;
        w[r][c] = j < nchunk ? ld_stream(row + j) : make_uint4(0, 0, 0, 0);
      }
    }
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float t = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        float wf[16];
        i8x16_to_f(w[r][c], wf);
#pragma unroll
        for (int e = 0; e < 16; ++e) t = fmaf(wf[e], xb[c][e], t);
      }
      acc[r] = wave_sum(t);
    }
    if (lane < ROWS && n0 + lane < N) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < ROWS; ++r) v = lane == r ? acc[r] : v;
      y[n0 + lane] = v * scale[n0 + lane];
    }
  }
}

// At most 16 weight chunks in flight per lane; more rows per wave only when
// there are enough rows to give every CU several workgroups (8 rows per wave
// at K = 1024 measured no faster than 4 on the 65536 x 1024 head).
template <int CPL>
int launch_gemv_i8(const float *x, const int8_t *Q, int64_t ldq, const float *scale, float *y, int N, int K,
                   hipStream_t st) {
  constexpr int kMaxRows = 16 / CPL >= 4 ? 4 : 16 / CPL;
  auto grid_for = [&](int rows) {
    const int64_t waves = ((int64_t)N + rows - 1) / rows;
    return (int)std::min<int64_t>((waves + 3) / 4, 4096);
  };
  if (kMaxRows >= 4 && N / 4 >= 4096)
    gemv_i8_kernel<CPL, (kMaxRows >= 4 ? 4 : 1)><<<grid_for(4), 256, 0, st>>>(x, Q, ldq, scale, y, N, K);
  else if (kMaxRows >= 2 && N / 2 >= 2048)
    gemv_i8_kernel<CPL, (kMaxRows >= 2 ? 2 : 1)><<<grid_for(2), 256, 0, st>>>(x, Q, ldq, scale, y, N, K);
  else
    gemv_i8_kernel<CPL, 1><<<grid_for(1), 256, 0, st>>>(x, Q, ldq, scale, y, N, K);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

}  // namespace
}  // namespace rwkv7

using namespace rwkv7;

extern "C" int rwkv7_gemv_i8(const float *x, const void *Q, int64_t ldq, const float *scale, float *y, int32_t N,
                             int32_t K, void *stream) {
  if (!x || !Q || !scale || !y) return RWKV7_EINVAL;
  if (N < 1 || K < 16 || K % 16 || K > 8192 || ldq < K || ldq % 16) return RWKV7_ESHAPE;
  if (reinterpret_cast<uintptr_t>(Q) % 16 || reinterpret_cast<uintptr_t>(x) % 16) return RWKV7_ESHAPE;
  const int8_t *q = static_cast<const int8_t *>(Q);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nchunk = K / 16;
  if (nchunk <= 64) return launch_gemv_i8<1>(x, q, ldq, scale, y, N, K, st);
  if (nchunk <= 128) return launch_gemv_i8<2>(x, q, ldq, scale, y, N, K, st);
  if (nchunk <= 256) return launch_gemv_i8<4>(x, q, ldq, scale, y, N, K, st);
  return launch_gemv_i8<8>(x, q, ldq, scale, y, N, K, st);
}
