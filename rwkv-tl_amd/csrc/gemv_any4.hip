// Decode-time GEMV over any4 weights: y[n] = sum_k x[k] lut[n][code[n, k]].
//
// any4 (the learned 4-bit format the reference names for its quantisation
// step, TODO.md:58-63: "int8/any4" weights dequantised inside the
// hand-written GEMV): every weight row keeps a table of 16 values (here the
// centroids of a per-row k-means over the row, stored f16) and one 4-bit code
// per weight, so a row of K weights costs K / 2 bytes plus 32 bytes of table
// -- a quarter of the f16 bytes, half of int8's.
//
// codes is [N, K / 2] bytes, K-contiguous rows of ldc bytes; byte j of a row
// holds the codes of columns 2j (low nibble) and 2j + 1 (high nibble). A
// wavefront owns ROWS consecutive rows at a time; lane l reads the 8-byte
// chunks l, l + 64, ... of each row (16 codes each), so one wave instruction
// streams 512 contiguous bytes of a row. x is held in registers for the whole
// launch (16 floats per chunk a lane owns). The tables of the wave's rows are
// widened to fp32 into the wave's own LDS slots; every code is then one LDS
// read (the 16 entries sit in 16 different banks, so a wave's 64 lookups into
// one table never conflict) and one fp32 FMA.
#include "rwkv7_kernels.h"

namespace rwkv7 {
namespace {

constexpr int kA4Rows = 4;  // rows per wave at a time (tables staged per wave)
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int CPL, int ROWS>
__global__ __launch_bounds__(256) void gemv_any4_kernel(const float *__restrict__ x, const uint8_t *__restrict__ codes,
                                                        int64_t ldc, const uint16_t *__restrict__ lut,
                                                        float *__restrict__ y, int N, int K) {
  __shared__ float s_lut[4][kA4Rows * 16];
  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x >> 6;
  const int wave = blockIdx.x * 4 + wv;
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
  float *tab = s_lut[wv];
  const int ngroups = (N + ROWS - 1) / ROWS;
  for (int g = wave; g < ngroups; g += nwave) {
    const int n0 = g * ROWS;
    u32x2 w[ROWS][CPL];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const int n = min(n0 + r, N - 1);  // rows past N re-read the last row; their sums are dropped
      const u32x2 *row = reinterpret_cast<const u32x2 *>(codes + (int64_t)n * ldc);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int j = lane + kWave * c;
        w[r][c] = j < nchunk ? __builtin_nontemporal_load(row + j) : u32x2{0u, 0u};
      }
    }
    // this wave's tables: lane l < 16 ROWS holds entry l % 16 of row l / 16
    // (LDS accesses of one wave are serviced in order, so the previous
    // group's lookups are done before these writes land)
    if (lane < ROWS * 16) tab[lane] = h2f(lut[(int64_t)min(n0 + (lane >> 4), N - 1) * 16 + (lane & 15)]);
    __builtin_amdgcn_wave_barrier();
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const float *t = tab + 16 * r;
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint32_t q[2] = {w[r][c][0], w[r][c][1]};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int e = 8 * h + 2 * b;  // column 16 j + e of the chunk
            a0 = fmaf(t[(q[h] >> (8 * b)) & 15u], xb[c][e], a0);
            a1 = fmaf(t[(q[h] >> (8 * b + 4)) & 15u], xb[c][e + 1], a1);
          }
        }
      }
      acc[r] = wave_sum(a0 + a1);
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < ROWS && n0 + lane < N) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < ROWS; ++r) v = lane == r ? acc[r] : v;
      y[n0 + lane] = v;
    }
  }
}

template <int CPL>
int launch_gemv_any4(const float *x, const uint8_t *codes, int64_t ldc, const uint16_t *lut, float *y, int N, int K,
                     hipStream_t st) {
  auto grid_for = [&](int rows) {
    const int64_t waves = ((int64_t)N + rows - 1) / rows;
    return (int)std::min<int64_t>((waves + 3) / 4, 4096);
  };
  if (N / kA4Rows >= 2048)
    gemv_any4_kernel<CPL, kA4Rows><<<grid_for(kA4Rows), 256, 0, st>>>(x, codes, ldc, lut, y, N, K);
  else
    gemv_any4_kernel<CPL, 1><<<grid_for(1), 256, 0, st>>>(x, codes, ldc, lut, y, N, K);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

}  // namespace
}  // namespace rwkv7

using namespace rwkv7;

extern "C" int rwkv7_gemv_any4(const float *x, const void *codes, int64_t ldc, const void *lut, float *y, int32_t N,
                               int32_t K, void *stream) {
  if (!x || !codes || !lut || !y) return RWKV7_EINVAL;
  if (N < 1 || K < 16 || K % 16 || K > 8192 || ldc < K / 2 || ldc % 8) return RWKV7_ESHAPE;
  if (reinterpret_cast<uintptr_t>(codes) % 8 || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(lut) % 2)
    return RWKV7_ESHAPE;
  const uint8_t *q = static_cast<const uint8_t *>(codes);
  const uint16_t *t = static_cast<const uint16_t *>(lut);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nchunk = K / 16;
  if (nchunk <= 64) return launch_gemv_any4<1>(x, q, ldc, t, y, N, K, st);
  if (nchunk <= 128) return launch_gemv_any4<2>(x, q, ldc, t, y, N, K, st);
  if (nchunk <= 256) return launch_gemv_any4<4>(x, q, ldc, t, y, N, K, st);
  return launch_gemv_any4<8>(x, q, ldc, t, y, N, K, st);
}
