// Operator-level kernels of the time-mix stages, for callers of the
// reference's kernel namespace (rwkv_tl.kernels.fp16): the single gates, the
// packed LoRA first step, the LoRA second step with all gate math, the L2 norm
// of kk and the GroupNorm + r.k.r_k stage. The model paths run these stages
// fused (decode_mk.hip, tmix.hip); here each is one launch with 16-bit inputs
// and outputs (IEEE half, or bfloat16 when bf is set: the reference's fp16 and
// bf16 kernel namespaces) and fp32 arithmetic.
#include "rwkv7_kernels.h"

namespace rwkv7 {

// ---- single gates (src/rwkv_tl/kernels/gates.py:41-123, 287-313) -------------

__global__ __launch_bounds__(256) void w_gate_kernel(const uint16_t *x, const uint16_t *w0, uint16_t *out, int C, int bf) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < C) out[i] = f_to_u16(expf(-sigmoidf_(u16_to_f(w0[i], bf) + u16_to_f(x[i], bf)) * kInvSqrtE), bf);
}

__global__ __launch_bounds__(256) void v_gate_kernel(const uint16_t *v, const uint16_t *vf, const uint16_t *v0,
                                                     const uint16_t *v12, uint16_t *out, int C, int bf) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < C) {
    const float x = u16_to_f(v[i], bf);
    out[i] = f_to_u16(x + sigmoidf_(u16_to_f(v0[i], bf) + u16_to_f(v12[i], bf)) * (u16_to_f(vf[i], bf) - x), bf);
  }
}

__global__ __launch_bounds__(256) void a_kk_k_kernel(const uint16_t *a0, const uint16_t *ax, const uint16_t *k,
                                                     const uint16_t *k_k, const uint16_t *k_a, uint16_t *a_out,
                                                     uint16_t *kk_out, uint16_t *k_out, int C, int bf) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < C) {
    const float kv = u16_to_f(k[i], bf);
    const float a = sigmoidf_(u16_to_f(a0[i], bf) + u16_to_f(ax[i], bf));
    a_out[i] = f_to_u16(a, bf);
    kk_out[i] = f_to_u16(kv * u16_to_f(k_k[i], bf), bf);
    k_out[i] = f_to_u16(kv + u16_to_f(k_a[i], bf) * (kv * a - kv), bf);
  }
}

// ---- LoRA second step + gate math (gates.py:125-213, 315-357) -----------------
// One wave per output channel i: lanes split each rank sum (row i of v2t, w2t,
// a2t, g2t is contiguous), the first-step results are activated per lane
// (tanh for w, sigmoid for g), then lane 0 finishes the channel.

__global__ __launch_bounds__(256) void gates_kernel(rwkv7_gates_io io, int rv, int rw, int ra, int rg, int C, int bf) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (i >= C) return;
  auto part = [&](const uint16_t *vec, const uint16_t *mat, int R, int act) {
    float acc = 0.f;
    for (int j = lane; j < R; j += 64) {
      float x = u16_to_f(vec[j], bf);
      if (act == 1) x = tanhf(x);
      else if (act == 2) x = sigmoidf_(x);
      acc = fmaf(u16_to_f(mat[(int64_t)i * R + j], bf), x, acc);
    }
    return wave_sum(acc);
  };
  const float v12 = part(static_cast<const uint16_t *>(io.vr), static_cast<const uint16_t *>(io.v2t), rv, 0);
  const float w12 = part(static_cast<const uint16_t *>(io.wr), static_cast<const uint16_t *>(io.w2t), rw, 1);
  const float a12 = part(static_cast<const uint16_t *>(io.ar), static_cast<const uint16_t *>(io.a2t), ra, 0);
  const float g12 = part(static_cast<const uint16_t *>(io.gr), static_cast<const uint16_t *>(io.g2t), rg, 2);
  if (lane != 0) return;
  auto in = [&](const void *p) { return u16_to_f(static_cast<const uint16_t *>(p)[i], bf); };
  auto out = [&](void *p, float x) { static_cast<uint16_t *>(p)[i] = f_to_u16(x, bf); };
  const float v = in(io.v), k = in(io.k);
  out(io.v_out, v + sigmoidf_(in(io.v0) + v12) * (in(io.v_first) - v));
  out(io.w_out, expf(-sigmoidf_(in(io.w0) + w12) * kInvSqrtE));
  const float a = sigmoidf_(in(io.a0) + a12);
  out(io.a_out, a);
  out(io.kk_out, k * in(io.k_k));
  out(io.k_out, k + in(io.k_a) * (k * a - k));
  out(io.g_out, g12);
}

// ---- packed LoRA first step (gates.py:215-285) -------------------------------
// out[j] = W[j, :] . x_seg(j) with the input chosen by the row's segment
// (v, w, a, g). One wave per row, 16-byte loads along the row.

__global__ __launch_bounds__(256) void rank_gemv_kernel(const uint16_t *xv, const uint16_t *xw, const uint16_t *xa,
                                                        const uint16_t *xg, const uint16_t *W, uint16_t *out,
                                                        int rv, int rw, int ra, int rg, int C, int bf) {
  const int j = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (j >= rv + rw + ra + rg) return;
  const uint16_t *x = j < rv ? xv : j < rv + rw ? xw : j < rv + rw + ra ? xa : xg;
  const uint16_t *row = W + (int64_t)j * C;
  float acc = 0.f;
  for (int c = 8 * lane; c < C; c += 8 * 64) {
    float wf[8], xf[8];
    u16x8_to_f(*reinterpret_cast<const uint4 *>(row + c), wf, bf);
    u16x8_to_f(*reinterpret_cast<const uint4 *>(x + c), xf, bf);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(wf[e], xf[e], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) out[j] = f_to_u16(acc, bf);
}

// ---- L2 norm of kk and B = -kk_hat * a (dplr.py:45-71, 229-235) ---------------
// One wave per head, lane n = channel n.

__global__ __launch_bounds__(256) void l2norm_kernel(const uint16_t *kk, const uint16_t *a, uint16_t *kn,
                                                     uint16_t *b, int H, int bf) {
  const int h = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (h >= H) return;
  const int64_t o = (int64_t)h * kN + lane;
  const float x = u16_to_f(kk[o], bf);
  const float den = fmaxf(sqrtf(wave_sum(x * x)), 1e-12f);
  const float xn = x / den;
  kn[o] = f_to_u16(xn, bf);
  b[o] = f_to_u16(-(xn * u16_to_f(a[o], bf)), bf);
}

// ---- GroupNorm + r.k.r_k bonus (dplr.py:73-124, 237-254) ----------------------
// One wave per head: mean and biased variance over the head's 64 values, eps
// 64e-5, affine, plus (sum_n r k r_k) * v.

__global__ __launch_bounds__(256) void gn_rkrk_kernel(const uint16_t *y, const uint16_t *r, const uint16_t *k,
                                                      const uint16_t *v, const uint16_t *r_k, const uint16_t *lw,
                                                      const uint16_t *lb, uint16_t *out, int H, int bf) {
  const int h = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (h >= H) return;
  const int64_t o = (int64_t)h * kN + lane;
  const float yv = u16_to_f(y[o], bf);
  const float mean = wave_sum(yv) * (1.f / kN);
  const float d = yv - mean;
  const float var = wave_sum(d * d) * (1.f / kN);
  const float rk = wave_sum(u16_to_f(r[o], bf) * u16_to_f(k[o], bf) * u16_to_f(r_k[o], bf));
  out[o] = f_to_u16(d * rsqrtf(var + kGnEps) * u16_to_f(lw[o], bf) + u16_to_f(lb[o], bf) + rk * u16_to_f(v[o], bf), bf);
}

// ---- launchers ------------------------------------------------------------------

#define RWKV7_OPS_LAUNCH(kernel, n, ...)                                 \
  do {                                                                   \
    kernel<<<((n) + 255) / 256, 256, 0, st>>>(__VA_ARGS__);              \
    RWKV7_CHECK_LAUNCH();                                                \
    return RWKV7_OK;                                                     \
  } while (0)

int launch_w_gate(const uint16_t *x, const uint16_t *w0, uint16_t *out, int C, int bf, hipStream_t st) {
  RWKV7_OPS_LAUNCH(w_gate_kernel, C, x, w0, out, C, bf);
}

int launch_v_gate(const uint16_t *v, const uint16_t *vf, const uint16_t *v0, const uint16_t *v12, uint16_t *out,
                  int C, int bf, hipStream_t st) {
  RWKV7_OPS_LAUNCH(v_gate_kernel, C, v, vf, v0, v12, out, C, bf);
}

int launch_a_kk_k(const uint16_t *a0, const uint16_t *ax, const uint16_t *k, const uint16_t *k_k,
                  const uint16_t *k_a, uint16_t *a_out, uint16_t *kk_out, uint16_t *k_out, int C, int bf,
                  hipStream_t st) {
  RWKV7_OPS_LAUNCH(a_kk_k_kernel, C, a0, ax, k, k_k, k_a, a_out, kk_out, k_out, C, bf);
}

int launch_gates(const rwkv7_gates_io &io, int rv, int rw, int ra, int rg, int C, int bf, hipStream_t st) {
  RWKV7_OPS_LAUNCH(gates_kernel, C * 64, io, rv, rw, ra, rg, C, bf);
}

int launch_rank_gemv(const uint16_t *xv, const uint16_t *xw, const uint16_t *xa, const uint16_t *xg,
                     const uint16_t *W, uint16_t *out, int rv, int rw, int ra, int rg, int C, int bf,
                     hipStream_t st) {
  RWKV7_OPS_LAUNCH(rank_gemv_kernel, (rv + rw + ra + rg) * 64, xv, xw, xa, xg, W, out, rv, rw, ra, rg, C, bf);
}

int launch_l2norm(const uint16_t *kk, const uint16_t *a, uint16_t *kn, uint16_t *b, int H, int bf, hipStream_t st) {
  RWKV7_OPS_LAUNCH(l2norm_kernel, H * 64, kk, a, kn, b, H, bf);
}

int launch_gn_rkrk(const uint16_t *y, const uint16_t *r, const uint16_t *k, const uint16_t *v, const uint16_t *r_k,
                   const uint16_t *lw, const uint16_t *lb, uint16_t *out, int H, int bf, hipStream_t st) {
  RWKV7_OPS_LAUNCH(gn_rkrk_kernel, H * 64, y, r, k, v, r_k, lw, lb, out, H, bf);
}

}  // namespace rwkv7
