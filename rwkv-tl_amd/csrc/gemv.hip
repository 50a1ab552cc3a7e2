// Decode-time (one token) 16-bit-weight GEMV kernels: y[n] = sum_k x[k] W[n, k].
//
// W is [N, K] f16 (bfloat16 for a bf16 model), K-contiguous rows (the checkpoint's [out, in] layout). A
// wavefront owns ROWS consecutive rows at a time; lane l reads the 16-byte
// chunks l, l+64, ... of each row, so one wave instruction streams 1 KiB of
// contiguous weights. The input vector is built once per wave in registers by
// a prologue: a plain f32 vector, or LayerNorm of the residual stream followed
// by the token-shift lerp (x + mu * (prev - x)). Every wave recomputes the
// LayerNorm statistics from the residual row (a few KiB from L2) instead of
// waiting for a separate normalisation kernel.
//
// Reference counterparts: the r/k/v projections and LoRA first step
// (src/rwkv_tl/kernels/lerp.py:200-219, gates.py:215-285), o-projection
// (demo/_rwkv7_base.py:206), FFN (:290) and head (:86-87).
#include "rwkv7_kernels.h"

namespace rwkv7 {

template <int CPL, int ROWS, int PRO, int EPI, bool BF>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  using T16 = F16T<BF>;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int nwave = gridDim.x * 4;
  const int nchunk = a.K >> 3;

  float xb[CPL][8];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int j = lane + kWave * c;
    if (j < nchunk) {
      if (PRO == PRO_F16) {
        T16::to_f8(reinterpret_cast<const uint4 *>(a.x)[j], xb[c]);
      } else {
        const float4 *p = reinterpret_cast<const float4 *>(a.x) + 2 * j;
        float4 u = p[0], v = p[1];
        xb[c][0] = u.x; xb[c][1] = u.y; xb[c][2] = u.z; xb[c][3] = u.w;
        xb[c][4] = v.x; xb[c][5] = v.y; xb[c][6] = v.z; xb[c][7] = v.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xb[c][e] = 0.f;
    }
  }

  float xp[CPL][8];
  if (PRO == PRO_TMIX || PRO == PRO_CMIX || PRO == PRO_LN) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) s += xb[c][e];
    const float mean = wave_sum(s) / (float)a.K;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      if (lane + kWave * c < nchunk) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = xb[c][e] - mean;
          q += d * d;
        }
      }
    }
    const float rstd = rsqrtf(wave_sum(q) / (float)a.K + kLnEps);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int j = lane + kWave * c;
      if (j < nchunk) {
        const float4 *pw = reinterpret_cast<const float4 *>(a.ln_w) + 2 * j;
        const float4 *pb = reinterpret_cast<const float4 *>(a.ln_b) + 2 * j;
        float w8[8], b8[8];
        float4 t0 = pw[0], t1 = pw[1], u0 = pb[0], u1 = pb[1];
        w8[0] = t0.x; w8[1] = t0.y; w8[2] = t0.z; w8[3] = t0.w;
        w8[4] = t1.x; w8[5] = t1.y; w8[6] = t1.z; w8[7] = t1.w;
        b8[0] = u0.x; b8[1] = u0.y; b8[2] = u0.z; b8[3] = u0.w;
        b8[4] = u1.x; b8[5] = u1.y; b8[6] = u1.z; b8[7] = u1.w;
#pragma unroll
        for (int e = 0; e < 8; ++e) xb[c][e] = (xb[c][e] - mean) * rstd * w8[e] + b8[e];
        if (a.xln_out && blockIdx.x == 0 && threadIdx.x < kWave) {
          float4 *o = reinterpret_cast<float4 *>(a.xln_out) + 2 * j;
          o[0] = make_float4(xb[c][0], xb[c][1], xb[c][2], xb[c][3]);
          o[1] = make_float4(xb[c][4], xb[c][5], xb[c][6], xb[c][7]);
        }
        if (PRO == PRO_TMIX || PRO == PRO_CMIX) T16::to_f8(reinterpret_cast<const uint4 *>(a.prev)[j], xp[c]);
      }
    }
  }

  float xm[CPL][8];
  auto apply_mix = [&](const float *mu) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int j = lane + kWave * c;
      if (j < nchunk) {
        const float4 *pm = reinterpret_cast<const float4 *>(mu) + 2 * j;
        float4 m0 = pm[0], m1 = pm[1];
        const float m8[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) xm[c][e] = xb[c][e] + m8[e] * (xp[c][e] - xb[c][e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xm[c][e] = 0.f;
      }
    }
  };
  if (PRO == PRO_CMIX) {
    apply_mix(a.mu);
  } else if (PRO != PRO_TMIX) {
#pragma unroll
    for (int c = 0; c < CPL; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) xm[c][e] = xb[c][e];
  }

  int cur_seg = -1;
  const int ngroups = a.N / ROWS;
  for (int g = wave; g < ngroups; g += nwave) {
    const int n0 = g * ROWS;
    uint4 w[ROWS][CPL];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      const uint4 *row = reinterpret_cast<const uint4 *>(a.W + (int64_t)(n0 + r) * a.ldw);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int j = lane + kWave * c;
        w[r][c] = j < nchunk ? ld_stream(row + j) : make_uint4(0, 0, 0, 0);
      }
    }
    if (PRO == PRO_TMIX) {
      int s = 0;
#pragma unroll
      for (int i = 0; i < 6; ++i) s += n0 >= a.seg_end[i];
      if (s != cur_seg) {
        cur_seg = s;
        apply_mix(a.mu + (int64_t)a.seg_mu[s] * a.K);
      }
    }
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float t = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        float wf[8];
        T16::to_f8(w[r][c], wf);
#pragma unroll
        for (int e = 0; e < 8; ++e) t = fmaf(wf[e], xm[c][e], t);
      }
      acc[r] = wave_sum(t);
    }
    if (lane < ROWS) {
      float v = acc[0];
#pragma unroll
      for (int r = 1; r < ROWS; ++r) v = lane == r ? acc[r] : v;
      const int n = n0 + lane;
      if (EPI == EPI_F32) {
        reinterpret_cast<float *>(a.y)[n] = v;
      } else if (EPI == EPI_RESID) {
        reinterpret_cast<float *>(a.y)[n] += v;
      } else if (EPI == EPI_RELUSQ) {
        const float t = fmaxf(v, 0.f);
        reinterpret_cast<float *>(a.y)[n] = t * t;
      } else {
        reinterpret_cast<uint16_t *>(a.y)[n] = T16::from_f(v);
      }
    }
  }
}

// Chooses rows-per-wave and grid size: at most 16 weight chunks in flight per
// lane, and more rows per wave only when there are enough rows to keep every
// CU busy. The grid-stride loop covers the rest.
template <int CPL, int PRO, int EPI, bool BF>
static void launch_gemv_rows(const GemvArgs &a, hipStream_t st) {
  constexpr int kMaxRows = CPL >= 16 ? 1 : 16 / CPL >= 4 ? 4 : 16 / CPL;
  if (kMaxRows >= 4 && a.N % 4 == 0 && a.N / 4 >= 4096) {
    int grid = (a.N / 4 + 3) / 4;
    if (grid > 4096) grid = 4096;
    gemv_kernel<CPL, (kMaxRows >= 4 ? 4 : 1), PRO, EPI, BF><<<grid, 256, 0, st>>>(a);
  } else if (kMaxRows >= 2 && a.N % 2 == 0 && a.N / 2 >= 2048) {
    int grid = (a.N / 2 + 3) / 4;
    gemv_kernel<CPL, (kMaxRows >= 2 ? 2 : 1), PRO, EPI, BF><<<grid, 256, 0, st>>>(a);
  } else {
    int grid = (a.N + 3) / 4;
    gemv_kernel<CPL, 1, PRO, EPI, BF><<<grid, 256, 0, st>>>(a);
  }
}

template <int CPL, int PRO, int EPI>
static int launch_gemv_cpl(const GemvArgs &a, hipStream_t st) {
  if (a.bf) launch_gemv_rows<CPL, PRO, EPI, true>(a, st);
  else launch_gemv_rows<CPL, PRO, EPI, false>(a, st);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

template <int PRO, int EPI>
int launch_gemv(const GemvArgs &a, hipStream_t st) {
  const int nchunk = a.K / 8;
  if (a.K % 256 != 0 || a.K <= 0) return RWKV7_ESHAPE;
  if (nchunk <= 64) return launch_gemv_cpl<1, PRO, EPI>(a, st);
  if (nchunk <= 128) return launch_gemv_cpl<2, PRO, EPI>(a, st);
  if (nchunk <= 256) return launch_gemv_cpl<4, PRO, EPI>(a, st);
  if (nchunk <= 512) return launch_gemv_cpl<8, PRO, EPI>(a, st);
  if (nchunk <= 1024) return launch_gemv_cpl<16, PRO, EPI>(a, st);
  return RWKV7_ESHAPE;
}

template int launch_gemv<PRO_F32, EPI_F32>(const GemvArgs &, hipStream_t);
template int launch_gemv<PRO_F32, EPI_RESID>(const GemvArgs &, hipStream_t);
template int launch_gemv<PRO_TMIX, EPI_F32>(const GemvArgs &, hipStream_t);
template int launch_gemv<PRO_CMIX, EPI_RELUSQ>(const GemvArgs &, hipStream_t);
template int launch_gemv<PRO_LN, EPI_F16>(const GemvArgs &, hipStream_t);

}  // namespace rwkv7
