// Large-M plain GEMMs through hipBLASLt.
//
// The long-prefill GEMMs (M = B*T in the thousands: the 1.5B-shaped 4 x 1024
// prefill) are MFMA-bound, and there the vendor library's kernels run at
// ~0.4-0.5 of the dense f16 peak where this library's own large-M kernel
// (gemm.hip, gemm_big_tile) reaches ~0.2-0.3: with 16-bit operands and a plain
// epilogue -- store f32, store 16-bit, or add into an f32 output -- such a
// problem is a plain library GEMM, so it goes to hipBLASLt. The FFN key's
// relu^2 into half goes there too, as a half product followed by an in-place
// pass that stores relu(y)^2 (relusq_half_kernel): the product is rounded to
// half before it is squared -- the arithmetic of the reference's own fp16 path
// (relu(x @ W^T) ** 2 on a half product), within 4 units of half roundoff
// (2^-9 relative) of the singly rounded value. In bfloat16 the same double
// rounding costs up to 2^-6 relative (1.4 % measured at 2048 x 8192 x 1024),
// so bf16 relu^2 keeps the large-M kernel's single rounding. Everything else
// (f32 activations, tanh / sigmoid epilogues, the small-M shapes of decode and
// short prefills) stays on the hand-written kernels, and so does any problem
// hipBLASLt returns no algorithm for.
//
// Mapping: hipBLASLt is column-major, so Y[M, N] = A[M, K] W[N, K]^T (row
// major) is computed as D = op(W') op(A') with W' = W seen as a K x N
// column-major matrix (ld = ldw, transposed), A' = A as K x M (ld = lda, not
// transposed) and D = Y as N x M (ld = ldy). The add epilogue is beta = 1 with
// C = D = Y. Algorithms are chosen with no workspace, so calls on different
// streams share nothing but the handle; the chosen algorithm is cached per
// device and shape.
#include <hipblaslt/hipblaslt.h>

#include <deque>
#include <mutex>

#include "rwkv7_kernels.h"

namespace rwkv7 {
namespace {

struct LtKey {
  int M, N, K, epi, bf;
  int64_t lda, ldw, ldy;
  int batch;              // problems of one strided-batched call
  int64_t sa, sw, sy;     // their strides, in elements of A, W and Y
  bool operator==(const LtKey &o) const {
    return M == o.M && N == o.N && K == o.K && epi == o.epi && bf == o.bf && lda == o.lda && ldw == o.ldw &&
           ldy == o.ldy && batch == o.batch && sa == o.sa && sw == o.sw && sy == o.sy;
  }
};

struct LtPlan {
  LtKey key;
  bool ok = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, ly = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

struct LtDevice {
  std::mutex mu;
  bool tried = false;
  hipblasLtHandle_t h = nullptr;
  std::deque<LtPlan> plans;  // elements stay put as plans are added
};

constexpr int kLtDevices = 64;
LtDevice g_lt[kLtDevices];

// The plan of a shape on the current device, built on first use (nullptr if
// hipBLASLt is unavailable or has no algorithm for it). Nothing is created
// while the stream is being captured into a graph (the handle may allocate):
// such a call runs the library's own kernel, and the plan is built by the
// next call outside a capture.
const LtPlan *lt_plan(const LtKey &k, hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kLtDevices) return nullptr;
  LtDevice &d = g_lt[dev];
  std::lock_guard<std::mutex> lock(d.mu);
  for (const LtPlan &p : d.plans)
    if (p.key == k) return p.ok ? &p : nullptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  if (!d.tried) {
    d.tried = true;
    if (hipblasLtCreate(&d.h) != HIPBLAS_STATUS_SUCCESS) d.h = nullptr;
  }
  if (!d.h) return nullptr;
  LtPlan p;
  p.key = k;
  const hipDataType t16 = k.bf ? HIP_R_16BF : HIP_R_16F;
  const hipDataType ty = k.epi == GEPI_F16 ? t16 : HIP_R_32F;
  bool ok = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)) ==
                 HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.lw, t16, k.K, k.N, k.ldw) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.la, t16, k.K, k.M, k.lda) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&p.ly, ty, k.N, k.M, k.ldy) == HIPBLAS_STATUS_SUCCESS;
  if (ok && k.batch > 1) {
    const int32_t bc = k.batch;
    const hipblasLtMatrixLayout_t lays[3] = {p.lw, p.la, p.ly};
    const int64_t strides[3] = {k.sw, k.sa, k.sy};
    for (int i = 0; i < 3 && ok; ++i)
      ok = hipblasLtMatrixLayoutSetAttribute(lays[i], HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc)) ==
               HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutSetAttribute(lays[i], HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &strides[i],
                                             sizeof(strides[i])) == HIPBLAS_STATUS_SUCCESS;
  }
  if (ok) {
    hipblasLtMatmulPreference_t pref = nullptr;
    uint64_t ws = 0;
    ok = hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)) ==
             HIPBLAS_STATUS_SUCCESS;
    hipblasLtMatmulHeuristicResult_t res[1];
    int n = 0;
    ok = ok && hipblasLtMatmulAlgoGetHeuristic(d.h, p.desc, p.lw, p.la, p.ly, p.ly, pref, 1, res, &n) ==
                   HIPBLAS_STATUS_SUCCESS &&
         n > 0 && res[0].state == HIPBLAS_STATUS_SUCCESS && res[0].workspaceSize == 0;
    if (ok) p.algo = res[0].algo;
    if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  }
  p.ok = ok;
  d.plans.push_back(p);
  return p.ok ? &d.plans.back() : nullptr;
}

// y <- relu(y)^2 in place on M rows of N half values (row stride ldy): one
// workgroup per row at a time, eight values per 16-byte access when VEC (N and
// ldy multiples of 8, Y 16-byte aligned), each thread's accesses of a row
// issued together (up to 4 at a time). The square of a half value is exact in
// f32, so each value is rounded once, to half, after the square.
template <bool VEC>
__global__ __launch_bounds__(256) void relusq_half_kernel(uint16_t *Y, int64_t ldy, int N, int M) {
  auto sq = [](uint16_t u) -> uint16_t {
    const float v = fmaxf(h2f(u), 0.f);
    return f2h(v * v);
  };
  auto sq2 = [&](unsigned w) -> unsigned {
    return (unsigned)sq((uint16_t)(w & 0xffffu)) | ((unsigned)sq((uint16_t)(w >> 16)) << 16);
  };
  constexpr int kStep = 8 * 256;  // halves per workgroup access round
  for (int r = blockIdx.x; r < M; r += gridDim.x) {
    uint16_t *row = Y + (int64_t)r * ldy;
    if (VEC) {
      for (int c0 = 8 * threadIdx.x; c0 < N; c0 += 4 * kStep) {
        uint4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (c0 + j * kStep < N) v[j] = *reinterpret_cast<const uint4 *>(row + c0 + j * kStep);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (c0 + j * kStep < N)
            *reinterpret_cast<uint4 *>(row + c0 + j * kStep) =
                make_uint4(sq2(v[j].x), sq2(v[j].y), sq2(v[j].z), sq2(v[j].w));
      }
    } else {
      for (int c = threadIdx.x; c < N; c += 256) row[c] = sq(row[c]);
    }
  }
}

bool launch_relusq_half(const GemmProb &p, int M, hipStream_t st) {
  const bool vec = p.N % 8 == 0 && p.ldy % 8 == 0 && reinterpret_cast<uintptr_t>(p.Y) % 16 == 0;
  const int grid = M < 4096 ? M : 4096;
  uint16_t *y = static_cast<uint16_t *>(p.Y);
  if (vec) relusq_half_kernel<true><<<grid, 256, 0, st>>>(y, p.ldy, p.N, M);
  else relusq_half_kernel<false><<<grid, 256, 0, st>>>(y, p.ldy, p.N, M);
  return hipGetLastError() == hipSuccess;
}

}  // namespace

bool lt_eligible(const GemmProb &p) {
  return !p.a32 && (p.epi == GEPI_F32 || p.epi == GEPI_F16 || p.epi == GEPI_ADD_F32 || (p.epi == GEPI_RELUSQ && !p.bf));
}

bool lt_gemm(const GemmProb &p, int M, hipStream_t st) { return lt_gemm_batched(p, 1, 0, 0, 0, M, st); }

bool lt_gemm_batched(const GemmProb &p, int batch, int64_t sa, int64_t sw, int64_t sy, int M, hipStream_t st) {
  if (!lt_eligible(p) || M <= 0 || batch < 1) return false;
  // relu^2 (half) runs as the plain half product (same plan) and the in-place pass
  const bool relusq = p.epi == GEPI_RELUSQ;
  const LtKey k{M, p.N, p.K, relusq ? (int)GEPI_F16 : p.epi, p.bf ? 1 : 0, p.lda, p.ldw, p.ldy,
                batch, batch > 1 ? sa : 0, batch > 1 ? sw : 0, batch > 1 ? sy : 0};
  const LtPlan *pl = lt_plan(k, st);
  if (!pl) return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  const float alpha = 1.f, beta = p.epi == GEPI_ADD_F32 ? 1.f : 0.f;
  if (hipblasLtMatmul(g_lt[dev].h, pl->desc, &alpha, p.W, pl->lw, p.A, pl->la, &beta, p.Y, pl->ly, p.Y, pl->ly,
                      &pl->algo, nullptr, 0, st) != HIPBLAS_STATUS_SUCCESS)
    return false;
  // a pass that fails to launch leaves the plain product in Y: returning false
  // has the caller's own kernels recompute the problems into Y
  for (int b = 0; relusq && b < batch; ++b) {
    GemmProb q = p;
    q.Y = static_cast<uint16_t *>(p.Y) + b * sy;
    if (!launch_relusq_half(q, M, st)) return false;
  }
  return true;
}

}  // namespace rwkv7
