// fp16 MFMA GEMM for prefill and batched decode: Y = epi(A W^T).
//
// A is [M, K] f16 (activations, row stride lda), W is [N, K] f16 (weights in
// the checkpoint's [out, in] orientation, row stride ldw): both operands are
// K-contiguous, which is what v_mfma_f32_16x16x32_f16 wants in every lane
// (8 consecutive k of one row). Accumulation is fp32.
//
// Workgroup tile BM x 64, 4 waves; wave w owns output columns [16w, 16w+16)
// and all BM rows (BM/16 accumulators). The A tile (BM x 32 per k-step) is
// staged in LDS and shared by the 4 waves; each wave reads its W fragment
// straight from global memory (each weight byte is used by exactly one wave).
// Both are double-buffered in registers one k-step ahead.
//
// One launch runs a group of up to 8 problems that share M (the r/k/v
// projections and the four LoRA first steps of one layer, for instance).
// Reference counterparts: fused_rkv_gemm, ffn_h, ffn_v, out_mm
// (src/rwkv_tl/kernels/gemm.py:215-305) and the torch LoRA matmuls of prefill
// (demo/_rwkv7_base.py:243-269).
#include "rwkv7_kernels.h"

namespace rwkv7 {

constexpr int kMaxProb = 8;

struct GemmGroup {
  GemmProb p[kMaxProb];
  int tile_begin[kMaxProb + 1];
  int nprob, M, m_tiles;
};

constexpr int kBN = 64, kBK = 32, kLdsPad = 8;

template <int BM>
__global__ __launch_bounds__(256) void gemm_kernel(GemmGroup g) {
  __shared__ uint4 s_a[2][BM][(kBK + kLdsPad) / 8];

  int bx = blockIdx.x, pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProb; ++i) pi += (i < g.nprob && bx >= g.tile_begin[i]);
  const GemmProb &P = g.p[pi];
  const int local = bx - g.tile_begin[pi];
  const int mt = local % g.m_tiles, nt = local / g.m_tiles;
  const int m0 = mt * BM, n0 = nt * kBN;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int M = g.M, N = P.N, K = P.K;

  // A tile loader: BM rows x 4 chunks of 8 halfs.
  constexpr int kAChunks = BM * 4;
  constexpr int kAPer = (kAChunks + 255) / 256;
  uint4 a_reg[kAPer];
  auto load_a = [&](int k0) {
#pragma unroll
    for (int u = 0; u < kAPer; ++u) {
      const int idx = t + 256 * u;
      const int r = idx >> 2, kc = (idx & 3) * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (idx < kAChunks && m0 + r < M && k0 + kc < K)
        v = *reinterpret_cast<const uint4 *>(P.A + (int64_t)(m0 + r) * P.lda + k0 + kc);
      a_reg[u] = v;
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kAPer; ++u) {
      const int idx = t + 256 * u;
      if (idx < kAChunks) s_a[buf][idx >> 2][idx & 3] = a_reg[u];
    }
  };
  // W fragment: lane -> row n0 + 16 wv + (lane & 15), k-chunk (lane >> 4).
  const int wn = n0 + wv * 16 + (lane & 15);
  const uint16_t *wrow = P.W + (int64_t)(wn < N ? wn : 0) * P.ldw + (lane >> 4) * 8;
  auto load_w = [&](int k0) -> uint4 {
    if (wn < N && k0 + (lane >> 4) * 8 < K) return ld_stream(reinterpret_cast<const uint4 *>(wrow + k0));
    return make_uint4(0, 0, 0, 0);
  };

  floatx4 acc[BM / 16];
#pragma unroll
  for (int i = 0; i < BM / 16; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  load_a(0);
  uint4 w_cur = load_w(0);
  store_a(0);
  __syncthreads();
  const int nk = (K + kBK - 1) / kBK;
  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
    uint4 w_next = make_uint4(0, 0, 0, 0);
    if (ks + 1 < nk) {
      load_a((ks + 1) * kBK);
      w_next = load_w((ks + 1) * kBK);
    }
    const half8 bfrag = __builtin_bit_cast(half8, w_cur);
#pragma unroll
    for (int mb = 0; mb < BM / 16; ++mb) {
      const half8 afrag = __builtin_bit_cast(half8, s_a[buf][mb * 16 + (lane & 15)][lane >> 4]);
      acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afrag, bfrag, acc[mb], 0, 0, 0);
    }
    if (ks + 1 < nk) store_a(buf ^ 1);
    w_cur = w_next;
    __syncthreads();
  }

  // Epilogue: lane holds rows 4 * (lane >> 4) + {0..3} of column (lane & 15).
  const int col = n0 + wv * 16 + (lane & 15);
  if (col >= N) return;
#pragma unroll
  for (int mb = 0; mb < BM / 16; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + mb * 16 + (lane >> 4) * 4 + r;
      if (row >= M) continue;
      const float v = acc[mb][r];
      const int64_t o = (int64_t)row * P.ldy + col;
      switch (P.epi) {
        case GEPI_F32: reinterpret_cast<float *>(P.Y)[o] = v; break;
        case GEPI_F16: reinterpret_cast<uint16_t *>(P.Y)[o] = f2h(v); break;
        case GEPI_RELUSQ: {
          const float q = fmaxf(v, 0.f);
          reinterpret_cast<uint16_t *>(P.Y)[o] = f2h(q * q);
          break;
        }
        case GEPI_ADD_F32: reinterpret_cast<float *>(P.Y)[o] += v; break;
        case GEPI_TANH_F16: reinterpret_cast<uint16_t *>(P.Y)[o] = f2h(tanhf(v)); break;
        default: reinterpret_cast<uint16_t *>(P.Y)[o] = f2h(sigmoidf_(v)); break;
      }
    }
  }
}

// Checks shapes and launches one group. Every problem needs K % 8 == 0 and
// 16-byte aligned rows (lda, ldw multiples of 8).
int launch_gemm_group(const GemmProb *probs, int nprob, int M, hipStream_t st) {
  if (nprob < 1 || nprob > kMaxProb || M <= 0) return RWKV7_ESHAPE;
  GemmGroup g;
  const int BM = M <= 16 ? 16 : M <= 32 ? 32 : M <= 64 ? 64 : 128;
  g.M = M;
  g.m_tiles = (M + BM - 1) / BM;
  g.nprob = nprob;
  int tiles = 0;
  for (int i = 0; i < kMaxProb; ++i) {
    g.tile_begin[i] = tiles;
    if (i < nprob) {
      const GemmProb &p = probs[i];
      if (p.K <= 0 || p.N <= 0 || p.K % 8 || p.lda % 8 || p.ldw % 8) return RWKV7_ESHAPE;
      if (!p.A || !p.W || !p.Y) return RWKV7_EINVAL;
      g.p[i] = p;
      tiles += g.m_tiles * ((p.N + kBN - 1) / kBN);
    } else {
      g.p[i] = probs[0];
    }
  }
  g.tile_begin[kMaxProb] = tiles;
  switch (BM) {
    case 16: gemm_kernel<16><<<tiles, 256, 0, st>>>(g); break;
    case 32: gemm_kernel<32><<<tiles, 256, 0, st>>>(g); break;
    case 64: gemm_kernel<64><<<tiles, 256, 0, st>>>(g); break;
    default: gemm_kernel<128><<<tiles, 256, 0, st>>>(g); break;
  }
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

}  // namespace rwkv7
