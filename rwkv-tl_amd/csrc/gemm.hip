// fp16 MFMA GEMM for prefill and batched decode: Y = epi(A W^T).
//
// A is [M, K] f16 (activations, row stride lda), W is [N, K] f16 (weights in
// the checkpoint's [out, in] orientation, row stride ldw): both operands are
// K-contiguous, which is what v_mfma_f32_16x16x32_f16 wants in every lane
// (8 consecutive k of one row). Accumulation is fp32.
//
// At the sizes of prefill and batched decode (M = B*T up to a few hundred) the
// product is neither MFMA- nor HBM-bound: a workgroup's time is the latency of
// its one round of loads, its products and its epilogue (MFMA-busy and fetch
// counters at the 0.4B prefill: under 0.05 of the MFMA pipes' cycles, ~1 TB/s
// of fetch). So the kernel is built around issuing every load of a workgroup
// as early as possible:
//   * workgroup tile: BM rows x 64 columns; wave w owns columns [16w, 16w+16)
//     and all BM rows (BM/16 accumulators);
//   * each wave streams its 16-row strip of W straight into registers, a chunk
//     (4 k-steps of 32) ahead of its use, double-buffered in registers;
//   * the A tile is staged through LDS in chunks of 128 k, double-buffered, and
//     shared by the 4 waves;
//   * split-K: when the tiles alone cannot fill the GPU (N = 1024 at small M
//     gives 16 tiles), the K range of each tile is split over S workgroups
//     (S a power of two). Each writes its fp32 partial tile to the workspace;
//     the last of the S to finish (a per-tile arrival counter, reset by that
//     workgroup) sums the S partials in split order, so the result does not
//     depend on which workgroup came last, and applies the epilogue.
//
// A may also be f32 (GemmProb::a32): each A fragment is then split into its
// 16-bit hi part and 16-bit remainder (split_hi_lo) and multiplied by the same
// W fragment twice, which keeps the activations at fp32-grade precision for
// the cost of the second MFMA (the MFMA pipes are nearly idle at these sizes)
// and of A's doubled bytes, which lengthen each workgroup's load round.
//
// One launch runs a group of up to 8 problems that share M and A's rows (the
// r/k/v projections and the four LoRA first steps of one layer, for instance).
// Reference counterparts: fused_rkv_gemm, ffn_h, ffn_v, out_mm
// (src/rwkv_tl/kernels/gemm.py:215-305) and the torch LoRA matmuls of prefill
// (demo/_rwkv7_base.py:243-269).
#include "rwkv7_kernels.h"

namespace rwkv7 {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxProb = 8;
constexpr int kBN = 64;       // columns per workgroup tile
constexpr int kKC = 128;      // k per staged A chunk (4 k-steps)
constexpr int kLdsPadH = 8;   // halves of padding per A row in LDS
constexpr int kMaxSplit = 16;

struct GemmGroup {
  GemmProb p[kMaxProb];
  int wg_begin[kMaxProb + 1];  // first workgroup of each problem
  int splits[kMaxProb];        // S of each problem
  int kslice[kMaxProb];        // k per split (multiple of kKC)
  int64_t part_off[kMaxProb];  // floats into part
  int ctr_off[kMaxProb];       // counters into ctr
  int nprob, M, m_tiles;
  float *part;
  unsigned *ctr;
};

RWKV7_DEV void store_epi(const GemmProb &P, int row, int col, float v) {
  const int64_t o = (int64_t)row * P.ldy + col;
  // 16-bit outputs in the operands' format (half, or bfloat16 if P.bf)
  auto st16 = [&](float x) { reinterpret_cast<uint16_t *>(P.Y)[o] = P.bf ? f2b(x) : f2h(x); };
  switch (P.epi) {
    case GEPI_F32: reinterpret_cast<float *>(P.Y)[o] = v; break;
    case GEPI_F16: st16(v); break;
    case GEPI_RELUSQ: {
      const float q = fmaxf(v, 0.f);
      st16(q * q);
      break;
    }
    case GEPI_ADD_F32: reinterpret_cast<float *>(P.Y)[o] += v; break;
    case GEPI_TANH_F16: st16(tanhf(v)); break;
    case GEPI_SIGM_F16: st16(sigmoidf_(v)); break;
    case GEPI_RELUSQ_F32: {
      const float q = fmaxf(v, 0.f);
      reinterpret_cast<float *>(P.Y)[o] = q * q;
      break;
    }
    case GEPI_TANH_F32: reinterpret_cast<float *>(P.Y)[o] = tanhf(v); break;
    default: reinterpret_cast<float *>(P.Y)[o] = sigmoidf_(v); break;
  }
}

// Split-K hand-off shared by both kernels. Each of the workgroup's `nhold`
// holder waves (index `hold`, or -1 for a wave holding nothing) owns MB float4
// per lane. Returns false for every workgroup but the last of the S; the last
// gets the split-ordered sum in acc. Partials go out with device-scope (sc1)
// stores, which complete only once visible to every CU; each wave waits for
// its own (an asm with a memory clobber keeps every store before it), then one
// thread counts the workgroup in, and the last workgroup reads the partials
// with device-scope loads. No cache write-back or invalidation is involved.
template <int MB>
RWKV7_DEV bool splitk_arrive(floatx4 (&acc)[MB], float *pbase, int S, int split, int nhold, int hold,
                             unsigned *ctr, int *s_last) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int nbytes = S * nhold * MB * 64 * 16;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(pbase, 0, nbytes, 0x00020000);
  if (hold >= 0) {
    const int my = ((split * nhold + hold) * MB * 64 + lane) * 16;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc[mb]), rs, my + mb * 64 * 16, 0, 16);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old == (unsigned)(S - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = last;
  }
  __syncthreads();
  if (!*s_last) return false;
  if (hold < 0) return true;
  // NB splits per batch of loads (16 float4 per lane in flight), summed in
  // split order; indices past S are clamped and their values dropped
  constexpr int NB = MB >= 16 ? 1 : 16 / MB;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += NB) {
    floatx4 q[NB][MB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int sp = s0 + b < S ? s0 + b : S - 1;
      const int at = ((sp * nhold + hold) * MB * 64 + lane) * 16;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        q[b][mb] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, at + mb * 64 * 16, 0, 16));
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const bool use = s0 + b < S;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] += use ? q[b][mb] : floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  return true;
}

// The work unit of one tiled-GEMM workgroup (gemm_kernel, gemm_pf_kernel).
// Workgroup order: a unit u = (n-tile, split) reads one W slice; its m-tiles
// get indices 8 apart, so they run on the same XCD (workgroups are dealt
// round-robin over the 8 XCDs) and all but the first find W in that L2.
struct TileUnit {
  int pi, S, split, tile, m0, n0, kb, ke, nch;
  bool live;  // false for the padding of the last group of 8 units
};
template <int BM>
RWKV7_DEV TileUnit tile_unit(const GemmGroup &g) {
  TileUnit w;
  const int bx = blockIdx.x;
  w.pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProb; ++i) w.pi += (i < g.nprob && bx >= g.wg_begin[i]);
  const GemmProb &P = g.p[w.pi];
  w.S = g.splits[w.pi];
  const int local = bx - g.wg_begin[w.pi];
  const int mtl = g.m_tiles;
  const int u = local / (8 * mtl) * 8 + (local & 7);
  const int mt = local % (8 * mtl) / 8;
  w.live = u < (P.N + kBN - 1) / kBN * w.S;
  w.split = u & (w.S - 1);
  const int nt = u / w.S;
  w.tile = nt * mtl + mt;
  w.m0 = mt * BM;
  w.n0 = nt * kBN;
  w.kb = w.split * g.kslice[w.pi];
  w.ke = min(P.K, w.kb + g.kslice[w.pi]);
  w.nch = (w.ke - w.kb + kKC - 1) / kKC;  // chunks of this split
  return w;
}

// W of k-step ks (a 32-wide k block) for the wave's 16-column strip: lane ->
// row n0 + 16 wv + (lane & 15), 8 k at 32 ks + 8 (lane >> 4). In fragment
// order the strip (clamped to the padded rows) is one contiguous KiB per
// k-step; k-steps past the padded K are clamped (out-of-range k meets a zero A,
// out-of-range rows are never stored).
struct WStrip {
  const uint16_t *base;
  int K, nksf1, wmul, kmul, lane;
  RWKV7_DEV uint4 load(int kstep) const {
    const int k = 32 * kstep + 8 * (lane >> 4);
    const int ks = min(kstep, nksf1);
    const int64_t off = (int64_t)ks * wmul + (k < K - 8 ? k : K - 8) * kmul;
    return *reinterpret_cast<const uint4 *>(base + off);
  }
};
RWKV7_DEV WStrip w_strip(const GemmProb &P, int n0, int wv, int lane) {
  WStrip s;
  const bool frag = P.Wf != nullptr;
  const int wn = n0 + wv * 16 + (lane & 15);
  const int nstrip = (P.N + 15) / 16, strip = min(n0 / 16 + wv, nstrip - 1);
  s.base = frag ? P.Wf + ((int64_t)strip * P.nksf * 64 + lane) * 8 : P.W + (int64_t)(wn < P.N ? wn : P.N - 1) * P.ldw;
  s.K = P.K;
  s.nksf1 = P.nksf - 1;
  s.wmul = frag ? 512 : 0;
  s.kmul = frag ? 0 : 1;
  s.lane = lane;
  return s;
}

// Split-K hand-off (when S > 1) and epilogue of a workgroup's tile: lane holds
// rows 4 (lane >> 4) + {0..3} of column (lane & 15) of each 16-row block.
// With use_yres (add epilogue only) yres holds the Y values of those
// elements, loaded before the products, so the epilogue stores without a read
// round trip.
template <int MB>
RWKV7_DEV void tile_store_y(const GemmGroup &g, const TileUnit &w, floatx4 (&acc)[MB], int *s_last, bool use_yres,
                            const float (&yres)[MB][4]) {
  const GemmProb &P = g.p[w.pi];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int col = w.n0 + wv * 16 + (lane & 15);
  if (w.S > 1) {
    float *pbase = g.part + g.part_off[w.pi] + (int64_t)w.tile * w.S * 4 * MB * 256;
    if (!splitk_arrive<MB>(acc, pbase, w.S, w.split, 4, wv, g.ctr + g.ctr_off[w.pi] + w.tile, s_last)) return;
  }
  if (col >= P.N) return;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = w.m0 + mb * 16 + (lane >> 4) * 4 + r;
      if (row >= g.M) continue;
      if (use_yres) reinterpret_cast<float *>(P.Y)[(int64_t)row * P.ldy + col] = yres[mb][r] + acc[mb][r];
      else store_epi(P, row, col, acc[mb][r]);
    }
  }
}

template <int MB>
RWKV7_DEV void tile_store(const GemmGroup &g, const TileUnit &w, floatx4 (&acc)[MB], int *s_last) {
  float none[MB][4];
  tile_store_y<MB>(g, w, acc, s_last, false, none);
}

// The Y values tile_store's add epilogue accumulates into (addresses clamped
// into the output; rows and columns past it are never stored).
template <int MB>
RWKV7_DEV void load_yres(const GemmGroup &g, const TileUnit &w, float (&y)[MB][4]) {
  const GemmProb &P = g.p[w.pi];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int col = min(w.n0 + wv * 16 + (lane & 15), P.N - 1);
  const float *Y = reinterpret_cast<const float *>(P.Y);
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) y[mb][r] = Y[(int64_t)min(w.m0 + mb * 16 + (lane >> 4) * 4 + r, g.M - 1) * P.ldy + col];
}

// One 8-element A piece in registers: 16 bytes of 16-bit values, or 32 bytes of
// f32 (A32) that store_piece splits into the hi and lo planes of LDS.
template <bool A32>
struct APiece {
  uint4 v[A32 ? 2 : 1];
};
template <bool A32>
RWKV7_DEV APiece<A32> load_piece(const GemmProb &P, int rc, int kc) {
  APiece<A32> a;
  if constexpr (A32) {
    const uint4 *q = reinterpret_cast<const uint4 *>(reinterpret_cast<const float *>(P.A) + (int64_t)rc * P.lda + kc);
    a.v[0] = q[0];
    a.v[1] = q[1];
  } else {
    a.v[0] = *reinterpret_cast<const uint4 *>(P.A + (int64_t)rc * P.lda + kc);
  }
  return a;
}
// Stores a piece (zeros when !live) at hi[off] and, for A32, its remainder at lo[off].
template <bool BF, bool A32>
RWKV7_DEV void store_piece(const APiece<A32> &a, bool live, uint16_t *hi, uint16_t *lo, int off) {
  if constexpr (A32) {
    uint4 h = make_uint4(0, 0, 0, 0), l = make_uint4(0, 0, 0, 0);
    if (live) split_hi_lo<BF>(a.v[0], a.v[1], h, l);
    *reinterpret_cast<uint4 *>(hi + off) = h;
    *reinterpret_cast<uint4 *>(lo + off) = l;
  } else {
    *reinterpret_cast<uint4 *>(hi + off) = live ? a.v[0] : make_uint4(0, 0, 0, 0);
  }
}

template <int BM, bool BF, bool A32>
__global__ __launch_bounds__(256) void gemm_kernel(GemmGroup g) {
  constexpr int MB = BM / 16;                // 16-row blocks
  constexpr int kRowH = kKC + kLdsPadH;      // halves per LDS row
  constexpr int kAPer = BM * (kKC / 8) / 256;  // 8-element A pieces per thread per chunk
  constexpr int NP = A32 ? 2 : 1;            // LDS planes of A: hi (and lo)
  __shared__ __align__(16) uint16_t s_a[2][NP][BM][kRowH];
  __shared__ int s_last;

  const TileUnit U = tile_unit<BM>(g);
  if (!U.live) return;
  const GemmProb &P = g.p[U.pi];
  const int m0 = U.m0, kb = U.kb, ke = U.ke, nch = U.nch;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int M = g.M, K = P.K;

  // A staging: piece idx -> row idx >> 4, 16-byte column idx & 15. Loads are
  // unconditional (row and k clamped into range) and masked after arrival, so
  // the compiler can count outstanding loads exactly.
  APiece<A32> a_reg[kAPer];
  auto load_a = [&](int c) {
    const int k0 = kb + c * kKC;
#pragma unroll
    for (int u = 0; u < kAPer; ++u) {
      const int idx = t + 256 * u;
      const int r = m0 + (idx >> 4), k = k0 + 8 * (idx & 15);
      const int rc = r < M ? r : M - 1, kc = k < K - 8 ? k : K - 8;
      a_reg[u] = load_piece<A32>(P, rc, kc);
    }
  };
  auto store_a = [&](int c, int buf) {
    const int k0 = kb + c * kKC;
#pragma unroll
    for (int u = 0; u < kAPer; ++u) {
      const int idx = t + 256 * u;
      const int r = m0 + (idx >> 4), k = k0 + 8 * (idx & 15);
      const int off = (idx >> 4) * kRowH + 8 * (idx & 15);
      store_piece<BF, A32>(a_reg[u], r < M && k < ke, &s_a[buf][0][0][0], &s_a[buf][NP - 1][0][0], off);
    }
  };
  // W fragments of chunk c: k-steps kb/32 + 4c + j (see WStrip)
  const WStrip ws = w_strip(P, U.n0, wv, lane);
  const int kb32 = kb / 32;
  auto load_w = [&](int c, uint4 (&dst)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j] = ws.load(kb32 + 4 * c + j);
  };

  floatx4 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf, const uint4 (&w)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int pl = 0; pl < NP; ++pl) {
          const uint4 afrag =
              *reinterpret_cast<const uint4 *>(&s_a[buf][pl][mb * 16 + (lane & 15)][32 * j + 8 * (lane >> 4)]);
          acc[mb] = mfma16<BF>(afrag, w[j], acc[mb]);
        }
      }
    }
  };

  // Chunk loop, unrolled by two so the register double buffers of W have
  // fixed names. Every load is unconditional (addresses clamped) so the
  // compiler counts outstanding loads exactly; an odd chunk count gets one
  // padding chunk whose products are skipped.
  const int nch2 = (nch + 1) & ~1;
  uint4 w0[4], w1[4];
  load_a(0);
  load_w(0, w0);
  load_w(1, w1);
  // the residual of an add epilogue, with the first loads
  const bool add = P.epi == GEPI_ADD_F32;
  float yres[MB][4];
  if (add) load_yres<MB>(g, U, yres);
  store_a(0, 0);
  __syncthreads();
  // (scheduling barriers keep each chunk's A loads ahead of the W loads issued
  // after its products, so storing A to LDS waits for A alone)
  for (int c = 0; c < nch2; c += 2) {
    // chunk c (A in buffer 0, W in w0)
    load_a(c + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(0, w0);
    load_w(c + 2, w0);
    __builtin_amdgcn_sched_barrier(0);
    store_a(c + 1, 1);
    __syncthreads();
    // chunk c + 1 (A in buffer 1, W in w1)
    load_a(c + 2);
    __builtin_amdgcn_sched_barrier(0);
    if (c + 1 < nch) compute(1, w1);
    load_w(c + 3, w1);
    __builtin_amdgcn_sched_barrier(0);
    store_a(c + 2, 0);
    __syncthreads();
  }

  tile_store_y<MB>(g, U, acc, &s_last, add, yres);
}

// Prefetch-all variant of gemm_kernel for splits of at most NC chunks (every
// prefill GEMM at M <= 256 after plan_splits): all A chunks and all W chunks of
// the split are issued before the first product, so a workgroup waits for one
// memory round trip instead of one per chunk pair (the tiles are latency-bound
// at these sizes, not bandwidth-bound). Same tiling, unit order, split-K
// hand-off and epilogue as gemm_kernel.
template <int BM, int NC, bool BF, bool A32>
__global__ __launch_bounds__(256) void gemm_pf_kernel(GemmGroup g) {
  constexpr int MB = BM / 16;
  constexpr int kRowH = kKC + kLdsPadH;
  constexpr int kAPer = BM * (kKC / 8) / 256;
  constexpr int NP = A32 ? 2 : 1;
  __shared__ __align__(16) uint16_t s_a[NC][NP][BM][kRowH];
  __shared__ int s_last;

  const TileUnit U = tile_unit<BM>(g);
  if (!U.live) return;
  const GemmProb &P = g.p[U.pi];
  const int m0 = U.m0, kb = U.kb, ke = U.ke, nch = U.nch;  // nch <= NC
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int M = g.M, K = P.K;

  // A pieces (row idx >> 4, 16-byte column idx & 15), loads clamped into range
  // and masked when stored; a chunk past the split re-reads the split's last
  // chunk (an L2 hit) and is never multiplied.
  APiece<A32> a_reg[NC][kAPer];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k0 = kb + (c < nch ? c : nch - 1) * kKC;
#pragma unroll
    for (int q = 0; q < kAPer; ++q) {
      const int idx = t + 256 * q;
      const int r = m0 + (idx >> 4), k = k0 + 8 * (idx & 15);
      const int rc = r < M ? r : M - 1, kc = k < K - 8 ? k : K - 8;
      a_reg[c][q] = load_piece<A32>(P, rc, kc);
    }
  }
  const WStrip ws = w_strip(P, U.n0, wv, lane);
  const int kb32 = kb / 32;
  uint4 wr[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int cc = c < nch ? c : nch - 1;
#pragma unroll
    for (int j = 0; j < 4; ++j) wr[c][j] = ws.load(kb32 + 4 * cc + j);
  }
  // the residual of an add epilogue, after the weights
  const bool add = P.epi == GEPI_ADD_F32;
  float yres[MB][4];
  if (add) load_yres<MB>(g, U, yres);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k0 = kb + c * kKC;
#pragma unroll
    for (int q = 0; q < kAPer; ++q) {
      const int idx = t + 256 * q;
      const int r = m0 + (idx >> 4), k = k0 + 8 * (idx & 15);
      const int off = (idx >> 4) * kRowH + 8 * (idx & 15);
      store_piece<BF, A32>(a_reg[c][q], r < M && k < ke, &s_a[c][0][0][0], &s_a[c][NP - 1][0][0], off);
    }
  }
  __syncthreads();

  floatx4 acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (c < nch) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
          for (int pl = 0; pl < NP; ++pl) {
            const uint4 afrag =
                *reinterpret_cast<const uint4 *>(&s_a[c][pl][mb * 16 + (lane & 15)][32 * j + 8 * (lane >> 4)]);
            acc[mb] = mfma16<BF>(afrag, wr[c][j], acc[mb]);
          }
        }
      }
    }
  }

  tile_store_y<MB>(g, U, acc, &s_last, add, yres);
}

// ---------------------------------------------------------------------------
// Large-M path (long prefills, see big_fits): the product is MFMA-bound, so
// the workgroup tile is large enough that each byte staged through LDS feeds
// many products. Problems with a plain epilogue (and half relu^2) run in
// hipBLASLt instead when it has an algorithm for them (gemm_lt.hip: ~1.7x
// faster on these shapes); this kernel keeps the bf16 relu^2 and the tanh /
// sigmoid epilogues, and the narrow problems (N < 256: the LoRA first steps)
// of a group whose wide problems take this path. BM x BN tile (256 x 256, or 128 x 128 where the larger tiles
// leave CUs idle), 8 waves as 2 (rows) x 4 (columns), each wave a (BM/2) x
// (BN/4) block of 16x16 accumulators; K in stages of 32.
//
// Operands go global -> LDS directly (global_load_lds_dwordx4: each lane's
// 16 bytes land at the wave's LDS base + 16 lane), into a ring of kBigNB
// stage buffers, kBigNB - 1 stages ahead of the products: a CU keeps ~96 KB
// of loads in flight, which is what hides the L2 / HBM latency at this
// arithmetic intensity (one stage ahead in registers reached ~0.2 of the MFMA
// peak). LDS holds both operands in fragment order: a 16-row x 32-k block is
// the 1 KiB that one v_mfma_f32_16x16x32_f16 operand reads (lane l <-> row
// l % 16, k 8 (l / 16) .. +8), so a block is one DMA instruction per wave
// (4 lanes per 64 contiguous bytes of a row, or one contiguous KiB when W
// comes from the fragment arena) and every fragment read is 64 lanes x 16
// consecutive bytes, free of bank conflicts.
//
// Synchronisation per stage: each wave waits for its own DMAs of the stage
// (vmcnt), then a bare s_barrier (no memory fence: that would wait for every
// DMA in flight) makes all of the stage visible and retires the buffer the
// next DMA overwrites.
//
// Workgroups are dealt round-robin over the 8 XCDs; consecutive tiles are
// given to one XCD so they share its L2, and inside a problem the tiles are
// ordered kBigGroupM row blocks at a time, column by column, so the ~32 tiles
// an XCD runs at once read 4 A strips and 8 W strips rather than 1 and 32
// (measured 3-5% faster on the 1.5B FFN shapes; groups of 1, 2, 8 and 16
// were not better).
// ---------------------------------------------------------------------------
constexpr int kBigBK = 32;  // k per stage
constexpr int kBigNB = 4;   // stage buffers (kBigNB - 1 stages in flight)
constexpr int kBigGroupM = 4;  // row blocks per group of the tile order

struct BigGroup {
  GemmProb p[kMaxProb];
  int tile_begin[kMaxProb + 1];  // first tile of each problem
  int tiles_n[kMaxProb];         // column tiles of each problem
  int nprob, M, m_tiles, tiles;
};

// NW waves as a 2 x (NW / 2) grid over the tile.
template <int BM, int BN, int NW, bool BF>
RWKV7_DEV void gemm_big_tile(const BigGroup &g) {
  constexpr int SA = BM / 16, SB = BN / 16;  // 16-row strips of A and W in a tile = blocks per stage
  constexpr int PERS = (SA + SB) / NW;       // blocks each wave loads per stage
  constexpr int GN = NW / 2;                 // waves along the columns
  constexpr int WM = BM / 32, WN = BN / (16 * GN);  // 16x16 tiles per wave (rows, columns)
  static_assert((SA + SB) % NW == 0 && SA % PERS == 0, "a wave loads whole blocks of one operand");
  // s_waitcnt with vmcnt = (kBigNB - 2) stages of this wave's DMAs (6-bit
  // field: bits 3..0 and 15..14), expcnt and lgkmcnt untouched
  constexpr int kVm = (kBigNB - 2) * PERS;
  static_assert(kVm < 64, "vmcnt field");
  constexpr int kWaitImm = 0x0F70 | (kVm & 15) | ((kVm >> 4) << 14);
  __shared__ __align__(16) u32x4 lds[kBigNB][SA + SB][64];

  // wv in a scalar register: each wave's DMA operands (buffer, LDS address)
  // derive from it
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // tile of this workgroup: XCD x = blockIdx % 8 takes tiles [x * per, (x+1) * per)
  const int per = (g.tiles + 7) / 8;
  const int tile = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (tile >= g.tiles) return;
  // the problem of this tile, selected field by field with a uniform index
  // (indexing the argument array at run time would copy it to scratch)
  GemmProb P = g.p[0];
  int tb = g.tile_begin[0], tn = g.tiles_n[0];
#pragma unroll
  for (int i = 1; i < kMaxProb; ++i) {
    if (i < g.nprob && tile >= g.tile_begin[i]) {
      P = g.p[i];
      tb = g.tile_begin[i];
      tn = g.tiles_n[i];
    }
  }
  // grouped order inside a problem: kBigGroupM row blocks at a time, column
  // by column, so the tiles one XCD runs at once share few A and W strips
  const int local = tile - tb;
  const int grp = local / (kBigGroupM * tn), in = local % (kBigGroupM * tn);
  const int gm = min(kBigGroupM, g.m_tiles - grp * kBigGroupM);
  const int m0 = (grp * kBigGroupM + in % gm) * BM, n0 = in / gm * BN;
  const int M = g.M, N = P.N, K = P.K;

  // Block b of a stage (A strips 0 .. SA - 1, then W strips): wave wv loads
  // blocks wv * PERS .. +PERS, all of one operand; lane l the piece of row
  // 16 strip + l % 16 at k 8 (l / 16) of the stage. Rows past M or N are
  // clamped (their products are never stored). Offsets in halfs from `base`.
  const bool isA = wv * PERS < SA;
  const int sb0 = isA ? wv * PERS : wv * PERS - SA;
  const bool wfrag = !isA && P.Wf != nullptr;
  const uint16_t *base = isA ? P.A : wfrag ? P.Wf : P.W;
  // the operand as a buffer resource: a lane's piece is a 32-bit byte offset,
  // the stage a scalar one
  const int64_t rows = isA ? M : wfrag ? (int64_t)(N + 15) / 16 * 16 : N;
  const int64_t ld = isA ? P.lda : wfrag ? (int64_t)P.nksf * 32 : P.ldw;
  const int64_t nbytes = rows * ld * 2;  // integer clamp: the descriptor words stay in scalar registers
  const i32x4 rsrc = buffer_words(base, nbytes > 0x7fffffff ? 0x7fffffff : (int)nbytes);
  const int stage_b = 2 * (wfrag ? 512 : kBigBK);  // bytes per stage (one block in fragment order)
  unsigned off[PERS];
#pragma unroll
  for (int u = 0; u < PERS; ++u) {
    const int strip = sb0 + u;
    if (isA) off[u] = 2u * (unsigned)(min(m0 + 16 * strip + (lane & 15), M - 1) * (int)P.lda + 8 * (lane >> 4));
    else if (wfrag) off[u] = 2u * (unsigned)(min(n0 / 16 + strip, (N + 15) / 16 - 1) * P.nksf * 512 + 8 * lane);
    else off[u] = 2u * (unsigned)(min(n0 + 16 * strip + (lane & 15), N - 1) * (int)P.ldw + 8 * (lane >> 4));
  }
  const int nst = K / kBigBK;
  // DMA of stage st (clamped: past the last stage the last one is reloaded into
  // a buffer nobody reads again, which keeps the vmcnt bookkeeping uniform)
  auto issue = [&](int st, int buf) __attribute__((always_inline)) {
    const unsigned s2 = (unsigned)(st < nst ? st : nst - 1) * stage_b;
#pragma unroll
    for (int u = 0; u < PERS; ++u)
      dma16(rsrc, lds_addr(&lds[buf][wv * PERS + u][0]), off[u], s2);
  };

  const int wm = wv / GN, wn = wv % GN;  // this wave's block of the tile
  floatx4 acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int q = 0; q < WN; ++q) acc[i][q] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](int st, int buf) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kWaitImm);  // this wave's DMAs of stage st have landed
    // everyone's have, and every read of buffer (st - 1) % NB is complete (the
    // lgkmcnt wait); the memory clobber keeps the compiler from moving LDS
    // reads or DMAs across the barrier
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(st + kBigNB - 1, (buf + kBigNB - 1) % kBigNB);
    u32x4 bf[WN];
#pragma unroll
    for (int q = 0; q < WN; ++q) bf[q] = lds[buf][SA + wn * WN + q][lane];
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const u32x4 af = lds[buf][wm * WM + i][lane];
#pragma unroll
      for (int q = 0; q < WN; ++q) acc[i][q] = mfma16<BF>(af, bf[q], acc[i][q]);
    }
  };
#pragma unroll
  for (int b = 0; b < kBigNB - 1; ++b) issue(b, b);
  int st = 0;
  for (; st + kBigNB <= nst; st += kBigNB) {
#pragma unroll
    for (int b = 0; b < kBigNB; ++b) step(st + b, b);
  }
#pragma unroll
  for (int b = 0; b < kBigNB; ++b)
    if (st + b < nst) step(st + b, b);
  // drain the clamped DMAs before the workgroup's LDS can be reused
  __builtin_amdgcn_s_waitcnt(0x0F70);

  // Epilogue: the activation applied in registers under one uniform branch,
  // then stores. Every accumulator index is a compile-time constant: a
  // per-element switch made the unrolled loop too large to unroll, and the
  // dynamic indexing that remained put the whole accumulator array in
  // scratch memory, written back on every iteration of the stage loop.
  const int epi = P.epi;
  auto map = [&](auto fn) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int q = 0; q < WN; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][q][r] = fn(acc[i][q][r]);
  };
  if (epi == GEPI_RELUSQ || epi == GEPI_RELUSQ_F32) map([](float v) { v = fmaxf(v, 0.f); return v * v; });
  else if (epi == GEPI_TANH_F16 || epi == GEPI_TANH_F32) map([](float v) { return tanhf(v); });
  else if (epi == GEPI_SIGM_F16 || epi == GEPI_SIGM_F32) map([](float v) { return sigmoidf_(v); });
  const bool add = epi == GEPI_ADD_F32;
  const bool f32 = add || epi == GEPI_F32 || epi == GEPI_RELUSQ_F32 || epi == GEPI_TANH_F32 || epi == GEPI_SIGM_F32;
  float *yf = static_cast<float *>(P.Y);
  uint16_t *yh = static_cast<uint16_t *>(P.Y);
  // lane holds rows 4 (lane >> 4) + {0..3} of column lane & 15 of each 16x16 tile
#pragma unroll
  for (int q = 0; q < WN; ++q) {
    const int col = n0 + 16 * (wn * WN + q) + (lane & 15);
#pragma unroll
    for (int i = 0; i < WM; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + 16 * (wm * WM + i) + 4 * (lane >> 4) + r;
        if (row < M && col < N) {
          const int64_t o = (int64_t)row * P.ldy + col;
          const float v = acc[i][q][r];
          if (add) yf[o] += v;
          else if (f32) yf[o] = v;
          else yh[o] = P.bf ? f2b(v) : f2h(v);
        }
      }
    }
  }
}

__global__ __launch_bounds__(512) void gemm_big_kernel_256(BigGroup g) { gemm_big_tile<256, 256, 8, false>(g); }
__global__ __launch_bounds__(512) void gemm_big_kernel_128(BigGroup g) { gemm_big_tile<128, 128, 8, false>(g); }
__global__ __launch_bounds__(512) void gemm_big_kernel_256_bf(BigGroup g) { gemm_big_tile<256, 256, 8, true>(g); }
__global__ __launch_bounds__(512) void gemm_big_kernel_128_bf(BigGroup g) { gemm_big_tile<128, 128, 8, true>(g); }

// The large-M kernel reads A and W through buffer resources, whose byte
// offsets are 32-bit: an operand extent must stay below 2^31 bytes. W (or its
// fragment copy) is one extent, so a problem whose W spans 2 GiB or more goes
// to the 64-bit-addressed tiled kernels; A is cut into row blocks of at most
// big_rows_per_launch(lda) rows, one launch each (A and Y rebased).
constexpr int64_t kBufMax = 0x7fffffff;
static bool big_w_addressable(const GemmProb &p) {
  const int64_t rows = p.Wf ? (int64_t)(p.N + 15) / 16 * 16 : p.N;
  const int64_t ld = p.Wf ? (int64_t)p.nksf * 32 : p.ldw;
  return rows * ld * 2 <= kBufMax;
}
static int big_rows_per_launch(int64_t lda) {
  const int64_t rows = kBufMax / (2 * lda) / 256 * 256;  // whole 256-row tiles
  return (int)(rows < (int64_t)1 << 30 ? rows : (int64_t)1 << 30);
}

// Problems of the large-M path: K a multiple of 64, at least 256 columns, and
// enough 128 x 128 tiles for two workgroups per CU (measured: at M = 512 the
// 32-row tiled kernels with split-K are 2-3x faster; at M = 4096 this path is
// ~2x faster than them).
static bool big_fits(const GemmProb &p, int M, int cus) {
  return !p.a32 && p.K % kBigBK == 0 && p.N >= 256 &&
         (int64_t)((M + 127) / 128) * ((p.N + 127) / 128) >= 2 * cus && big_w_addressable(p) &&
         big_rows_per_launch(p.lda) >= 256;
}

// Bytes per output element of an epilogue.
static int epi_out_bytes(int epi) {
  return epi == GEPI_F32 || epi == GEPI_ADD_F32 || epi == GEPI_RELUSQ_F32 || epi == GEPI_TANH_F32 ||
                 epi == GEPI_SIGM_F32
             ? 4
             : 2;
}

int gemm_big_min_rows(int N) {
  if (N < 256) return 0x7fffffff;
  const int cus = mk_cus() > 0 ? mk_cus() : 256;
  const int nt = (N + 127) / 128, mt = (2 * cus + nt - 1) / nt;
  return (mt - 1) * 128 + 1;
}

#define RWKV7_TRY_GEMM(expr)         \
  do {                               \
    const int rc_ = (expr);          \
    if (rc_ != RWKV7_OK) return rc_; \
  } while (0)

// Runs a group of problems that all fit the large-M path.
static int launch_big(const GemmProb *probs, int nprob, int M, int cus, hipStream_t st) {
  BigGroup g;
  g.nprob = nprob;
  g.M = M;
  // 256 x 256 tiles when they alone give every CU a workgroup, else 128 x 128
  auto count = [&](int bt) {
    int t = 0;
    for (int i = 0; i < nprob; ++i) t += (M + bt - 1) / bt * ((probs[i].N + bt - 1) / bt);
    return t;
  };
  const int BT = count(256) >= cus ? 256 : 128;
  g.m_tiles = (M + BT - 1) / BT;
  int t = 0;
  for (int i = 0; i < kMaxProb; ++i) {
    g.tile_begin[i] = t;
    if (i < nprob) {
      g.p[i] = probs[i];
      g.tiles_n[i] = (probs[i].N + BT - 1) / BT;
      t += g.m_tiles * g.tiles_n[i];
    } else {
      g.p[i] = probs[0];
      g.tiles_n[i] = 1;
    }
  }
  g.tile_begin[kMaxProb] = t;
  g.tiles = t;
  const int grid = (t + 7) / 8 * 8;
  const bool bf = probs[0].bf != 0;
  if (BT == 256) {
    if (bf) gemm_big_kernel_256_bf<<<grid, 512, 0, st>>>(g);
    else gemm_big_kernel_256<<<grid, 512, 0, st>>>(g);
  } else {
    if (bf) gemm_big_kernel_128_bf<<<grid, 512, 0, st>>>(g);
    else gemm_big_kernel_128<<<grid, 512, 0, st>>>(g);
  }
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

// ---------------------------------------------------------------------------
// Skinny path, M <= 32 (batched decode, short prefill). One workgroup of 4
// waves per 16-column strip of W (and per split of K, see below); the waves
// split the strip's k-steps, each loading its W fragments and the A fragments
// of the live rows straight from memory (A is small and stays in L2) in
// batches of KB k-steps, all in flight before the first product. Loads are
// exact: no k-step is loaded twice and rows past M are not loaded (their MFMA
// rows compute zeros that are never stored). The 4 per-wave accumulators are
// summed through LDS in wave order.
//
// A CU streams about 30 GB/s of loads, so a strip whose W and A run past
// ~64 KB (K = 4096) is also split over S workgroups; the last to arrive sums
// the S partials in split order (the protocol of the tiled kernel below).
// ---------------------------------------------------------------------------
constexpr int kSkW = 4;           // waves per workgroup
constexpr int kSkinnyMaxM = 32;   // M up to this runs the skinny path
// with f32 A only up to 8 rows: from 9 rows the 16-row tiles are faster
// (measured: 0.4B prefill 1 x 32 1.37 vs 1.68 ms, decode B = 32 1.28 vs
// 1.59 ms/step, the 1.5B shape at B = 32 2.08 vs 3.24 and B = 16 1.77 vs
// 2.18 ms/step; at 2 and 4 rows the skinny strips are 5-7 % faster)
constexpr int kA32SkinnyMaxM = 8;

struct SkinnyGroup {
  GemmProb p[kMaxProb];
  int wg_begin[kMaxProb + 1];  // first workgroup of each problem
  int splits[kMaxProb];        // S of each problem (power of two)
  int64_t part_off[kMaxProb];  // floats into part
  int ctr_off[kMaxProb];
  int nprob, M;
  float *part;
  unsigned *ctr;
};

template <int MB, bool BF, bool A32>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(SkinnyGroup g) {
  constexpr int KB = MB == 1 ? 8 : 5;
  __shared__ __align__(16) float4 red[kSkW][MB][64];
  __shared__ int s_last;
  const int bx = blockIdx.x;
  int pi = 0;
#pragma unroll
  for (int i = 1; i < kMaxProb; ++i) pi += (i < g.nprob && bx >= g.wg_begin[i]);
  const GemmProb &P = g.p[pi];
  const int S = g.splits[pi];
  const int local = bx - g.wg_begin[pi];
  const int split = local & (S - 1), strip = local / S;
  const int n0 = strip * 16;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int M = g.M, N = P.N, K = P.K;
  // k-steps of this split, then of this wave
  const int nks = (K + 31) / 32;
  const int sps = (nks + S - 1) / S;
  const int s0 = split * sps, s1 = min(nks, s0 + sps);
  const int per = (s1 - s0 + kSkW - 1) / kSkW;
  const int ks0 = s0 + wv * per, ks1 = min(s1, ks0 + per);
  // W fragment of k-step ks: fragment order reads block (strip, ks), one
  // contiguous KiB per wave; row-major reads 8 k of row n0 + lane % 16
  const bool frag = P.Wf != nullptr;
  const int wn = n0 + (lane & 15);
  const uint16_t *wbase = frag ? P.Wf + ((int64_t)strip * P.nksf * 64 + lane) * 8
                               : P.W + (int64_t)(wn < N ? wn : N - 1) * P.ldw;
  auto woff = [&](int ks) -> int64_t {
    const int k = 32 * ks + 8 * (lane >> 4);
    return frag ? (int64_t)ks * 512 : (int64_t)(k < K - 8 ? k : K - 8);
  };
  int arow[MB];  // A row of each 16-row block (clamped)
  bool alive[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = mb * 16 + (lane & 15);
    alive[mb] = r < M;
    arow[mb] = r < M ? r : M - 1;
  }
  floatx4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int kb = ks0; kb < ks1; kb += KB) {
    const int cnt = min(KB, ks1 - kb);  // wave-uniform
    uint4 wf[KB];
    APiece<A32> af[KB][MB];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      wf[j] = make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int h = 0; h < (A32 ? 2 : 1); ++h) af[j][mb].v[h] = make_uint4(0, 0, 0, 0);
      if (j < cnt) {
        const int k = 32 * (kb + j) + 8 * (lane >> 4);
        const int kc = k < K - 8 ? k : K - 8;
        wf[j] = ld_stream(reinterpret_cast<const uint4 *>(wbase + woff(kb + j)));
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          if (alive[mb] && k < K) af[j][mb] = load_piece<A32>(P, arow[mb], kc);
      }
    }
    // every load of the batch is issued before the first product waits
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (j < cnt) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          if constexpr (A32) {
            uint4 hi, lo;
            split_hi_lo<BF>(af[j][mb].v[0], af[j][mb].v[1], hi, lo);
            acc[mb] = mfma16<BF>(hi, wf[j], acc[mb]);
            acc[mb] = mfma16<BF>(lo, wf[j], acc[mb]);
          } else {
            acc[mb] = mfma16<BF>(af[j][mb].v[0], wf[j], acc[mb]);
          }
        }
      }
    }
  }
  // cross-wave sum in wave order; wave 0 holds the strip's result
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) red[wv][mb][lane] = make_float4(acc[mb][0], acc[mb][1], acc[mb][2], acc[mb][3]);
  __syncthreads();
  if (wv == 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      floatx4 o = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < kSkW; ++w) {
        const float4 q = red[w][mb][lane];
        o += floatx4{q.x, q.y, q.z, q.w};
      }
      acc[mb] = o;
    }
  }
  if (S > 1) {
    float *pbase = g.part + g.part_off[pi] + (int64_t)strip * S * MB * 256;
    if (!splitk_arrive<MB>(acc, pbase, S, split, 1, wv == 0 ? 0 : -1, g.ctr + g.ctr_off[pi] + strip, &s_last))
      return;
  }
  const int col = n0 + (lane & 15);
  if (wv != 0 || col >= N) return;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = mb * 16 + (lane >> 4) * 4 + r;
      if (row < M) store_epi(P, row, col, acc[mb][r]);
    }
  }
}

// Splits of a skinny strip: enough that one workgroup moves at most ~64 KB
// of W and A, ~128 KB above 16 rows (measured: with 17..32 rows the larger
// cap is 4-5% faster, with up to 16 rows 2% slower).
static int skinny_splits(int M, int K, bool can_split, bool a32) {
  if (!can_split) return 1;
  const int64_t per_k = 16 * 2 + (int64_t)(M < 16 ? M : 16) * (a32 ? 4 : 2) * ((M + 15) / 16);  // bytes per unit of k
  const int64_t cap = M > 16 ? 128 * 1024 : 64 * 1024;
  int S = 1;
  while (S < kMaxSplit && (int64_t)K / S * per_k > cap && K / (2 * S) >= 256) S *= 2;
  return S;
}

static int launch_skinny(const GemmProb *probs, int nprob, int M, hipStream_t st, float *part, unsigned *ctr,
                         int64_t part_cap) {
  SkinnyGroup g;
  g.nprob = nprob;
  g.M = M;
  g.part = part;
  g.ctr = ctr;
  const int MB = (M + 15) / 16;
  // splits per problem, then halved (largest strips x splits first) until the
  // partial tiles and arrival counters fit the workspace
  int split[kMaxProb] = {};
  for (int i = 0; i < nprob; ++i)
    split[i] = skinny_splits(M, probs[i].K, part != nullptr && ctr != nullptr, probs[i].a32 != 0);
  for (;;) {
    int64_t need_fl = 0;
    int need_ctr = 0, worst = -1;
    int64_t worst_units = 0;
    for (int i = 0; i < nprob; ++i) {
      const int strips = (probs[i].N + 15) / 16;
      if (split[i] == 1) continue;
      need_fl += (int64_t)strips * split[i] * MB * 256;
      need_ctr += strips;
      if ((int64_t)strips * split[i] > worst_units) worst_units = (int64_t)strips * split[i], worst = i;
    }
    if ((need_fl * 4 <= part_cap && need_ctr <= kGemmCounters) || worst < 0) break;
    split[worst] /= 2;
  }
  int wgs = 0, ctrs = 0;
  int64_t pfl = 0;
  for (int i = 0; i < kMaxProb; ++i) {
    g.wg_begin[i] = wgs;
    if (i < nprob) {
      const int strips = (probs[i].N + 15) / 16;
      const int S = split[i];
      g.p[i] = probs[i];
      g.splits[i] = S;
      g.part_off[i] = pfl;
      g.ctr_off[i] = ctrs;
      wgs += strips * S;
      if (S > 1) {
        pfl += (int64_t)strips * S * MB * 256;
        ctrs += strips;
      }
    } else {
      g.p[i] = probs[0];
      g.splits[i] = 1;
      g.part_off[i] = 0;
      g.ctr_off[i] = 0;
    }
  }
  g.wg_begin[kMaxProb] = wgs;
  if (pfl * 4 > part_cap || ctrs > kGemmCounters) return RWKV7_EWORKSPACE;
  const bool bf = probs[0].bf != 0, a32 = probs[0].a32 != 0;
  const int variant = (MB == 1 ? 0 : 4) | (bf ? 2 : 0) | (a32 ? 1 : 0);
  switch (variant) {
    case 0: gemm_skinny_kernel<1, false, false><<<wgs, 256, 0, st>>>(g); break;
    case 1: gemm_skinny_kernel<1, false, true><<<wgs, 256, 0, st>>>(g); break;
    case 2: gemm_skinny_kernel<1, true, false><<<wgs, 256, 0, st>>>(g); break;
    case 3: gemm_skinny_kernel<1, true, true><<<wgs, 256, 0, st>>>(g); break;
    case 4: gemm_skinny_kernel<2, false, false><<<wgs, 256, 0, st>>>(g); break;
    case 5: gemm_skinny_kernel<2, false, true><<<wgs, 256, 0, st>>>(g); break;
    case 6: gemm_skinny_kernel<2, true, false><<<wgs, 256, 0, st>>>(g); break;
    default: gemm_skinny_kernel<2, true, true><<<wgs, 256, 0, st>>>(g); break;
  }
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

// Row tile of the tiled path: 32 rows up to M = 256 (the tiles alone then
// cover the GPU and W, re-read per row tile, comes from L2), 64 beyond
// (measured at M = 512 to 4096: 128-row tiles leave too few workgroups per CU
// to hide the chunk loads; 32-row tiles re-read W too often).
//
// f32 A (a32) up to kA32Bm16MaxM rows: 16-row tiles, so a workgroup's f32 A
// chunk takes the bytes (and registers) a 32-row 16-bit chunk takes and the
// prefetch-all kernel can hold 8 chunks without extra K splits; beyond,
// 32-row tiles (measured against 64: 0.4B prefill 1 x 512 3.66 vs 4.36 ms,
// 1 x 1024 6.29 vs 6.62 ms, 1 x 1536 8.67 vs 9.51 ms -- a 64-row f32 tile
// doubles both the A bytes per workgroup and the MFMAs per W fragment).
constexpr int kA32Bm16MaxM = 256;
static int bm_for(int M, bool a32 = false) {
  if (a32) return M <= kA32Bm16MaxM ? 16 : 32;
  return M <= 256 ? 32 : 64;
}

// Splits of a tiled problem: K is split (power of two, each split keeping at
// least two 128-wide chunks) until the group has a workgroup per CU and no
// workgroup streams more than ~256 KB of W and A (measured: a 128 KB cap,
// i.e. twice the splits, made prefill at T = 128 to 512 2-8% slower).
//
// f32 A (a32) at 32-row tiles: also split until a split holds at most 4
// chunks, the most whose f32 A pieces and W fragments the prefetch-all kernel
// keeps in registers at once. f32 A tiles take ~70 KB of LDS in the
// prefetch-all kernel, so two workgroups share a CU: splitting stops before a
// second round of workgroups (measured against splitting up to four per CU:
// the 1.5B shape's B=64 decode 2.65 vs 3.04 ms/step, 0.4B prefill 16 x 16
// 2.38 vs 2.51 ms; 1 x 128 unchanged).
static void plan_splits(const GemmProb *probs, int nprob, int M, int cus, bool can_split, int *S, int *kslice) {
  const int BM = bm_for(M, probs[0].a32 != 0);
  const int m_tiles = (M + BM - 1) / BM;
  int tiles = 0;
  for (int i = 0; i < nprob; ++i) tiles += m_tiles * ((probs[i].N + kBN - 1) / kBN);
  for (int i = 0; i < nprob; ++i) {
    const int K = probs[i].K;
    const bool a32 = probs[i].a32 != 0;
    int s = 1;
    if (can_split) {
      auto bytes = [&](int sp) { return (int64_t)(2 * kBN + (a32 ? 4 : 2) * BM) * ((K + sp - 1) / sp); };
      auto too_long = [&](int sp) { return a32 && BM == 32 && (K + sp - 1) / sp > 4 * kKC; };
      while (s < kMaxSplit && K / (2 * s) >= 2 * kKC &&
             (tiles * s < cus || bytes(s) > 256 * 1024 || too_long(s)) &&
             (int64_t)tiles * 2 * s <= (a32 ? 2 : 4) * cus)
        s *= 2;
    }
    S[i] = s;
    kslice[i] = ((K + s - 1) / s + kKC - 1) / kKC * kKC;
  }
}

int64_t gemm_ws_bytes(int M, int cus) {
  // partial tiles of BM x 64 floats; the tiled plan keeps tiles x S <= 4 cus,
  // the skinny one at most 16 splits of 16-column strips of 32 rows
  const int64_t tiled = (int64_t)4 * cus * bm_for(M) * kBN * 4;
  const int64_t skinny = (int64_t)4 * cus * 32 * 16 * 4;
  return tiled > skinny ? tiled : skinny;
}

// b follows a as the next problem of a strided batch: one shape and
// epilogue, A, W and Y later by positive strides (elements), Y not
// overlapping a's M rows.
static bool batch_next(const GemmProb &a, const GemmProb &b, int M, int64_t *sa, int64_t *sw, int64_t *sy) {
  if (a.N != b.N || a.K != b.K || a.epi != b.epi || a.bf != b.bf || a.lda != b.lda || a.ldw != b.ldw ||
      a.ldy != b.ldy)
    return false;
  const int ysz = epi_out_bytes(a.epi);
  const int64_t yb = static_cast<const char *>(b.Y) - static_cast<const char *>(a.Y);
  *sa = b.A - a.A;
  *sw = b.W - a.W;
  *sy = yb / ysz;
  return *sa > 0 && *sw > 0 && yb % ysz == 0 && *sy >= (int64_t)M * a.ldy;
}

// Problems of the large-M path over row blocks whose A extents stay below
// 2^31 bytes (big_rows_per_launch), A and Y rebased per block. With lt, each
// problem goes to hipBLASLt first (plain epilogues, half relu^2), consecutive
// problems of one shape at uniform strides as one strided-batched call (r, k,
// v of the prefill: 3 x 38.6 -> 100.9 us per call at the 1.5B shape, measured
// alone); the others, and any it declines, run in one launch of the large-M
// kernel per block.
static int launch_large_m(const GemmProb *probs, int n, int M, int cus, hipStream_t st, bool lt) {
  int rows = M;
  for (int i = 0; i < n; ++i) rows = min(rows, big_rows_per_launch(probs[i].lda));
  for (int r0 = 0; r0 < M; r0 += rows) {
    GemmProb blk[kMaxProb];
    int nk = 0;
    const int mr = min(rows, M - r0);
    auto rebased = [&](int i) {
      GemmProb b = probs[i];
      b.A = probs[i].A + (int64_t)r0 * probs[i].lda;
      b.Y = static_cast<char *>(probs[i].Y) + (int64_t)r0 * probs[i].ldy * epi_out_bytes(probs[i].epi);
      return b;
    };
    for (int i = 0; i < n;) {
      int cnt = 1;
      int64_t sa = 0, sw = 0, sy = 0;
      if (lt && i + 1 < n && batch_next(probs[i], probs[i + 1], M, &sa, &sw, &sy)) {
        int64_t a2, w2, y2;
        cnt = 2;
        while (i + cnt < n && batch_next(probs[i + cnt - 1], probs[i + cnt], M, &a2, &w2, &y2) && a2 == sa &&
               w2 == sw && y2 == sy)
          ++cnt;
      }
      if (cnt > 1 && lt_gemm_batched(rebased(i), cnt, sa, sw, sy, mr, st)) {
        i += cnt;
        continue;
      }
      for (int j = i; j < i + cnt; ++j) {
        const GemmProb b = rebased(j);
        if (!lt || !lt_gemm(b, mr, st)) blk[nk++] = b;
      }
      i += cnt;
    }
    if (nk > 0) RWKV7_TRY_GEMM(launch_big(blk, nk, mr, cus, st));
  }
  return RWKV7_OK;
}

// Checks shapes and launches one group. Every problem needs K % 8 == 0, K >= 8
// and 16-byte aligned rows (lda, ldw multiples of 8). part/ctr: split-K
// workspace (gemm_ws_bytes(M) bytes and kGemmCounters zeroed counters); with
// part == nullptr no problem is split.
int launch_gemm_group(const GemmProb *probs, int nprob, int M, hipStream_t st, float *part, unsigned *ctr) {
  if (nprob < 1 || nprob > kMaxProb || M <= 0) return RWKV7_ESHAPE;
  const int cus = mk_cus();
  if (cus <= 0) return RWKV7_ELAUNCH;
  GemmGroup g;
  const int BM = bm_for(M, probs[0].a32 != 0);
  g.M = M;
  g.m_tiles = (M + BM - 1) / BM;
  g.nprob = nprob;
  g.part = part;
  g.ctr = ctr;
  int S[kMaxProb], ks[kMaxProb];
  for (int i = 0; i < nprob; ++i) {
    const GemmProb &p = probs[i];
    if (p.K < 8 || p.N <= 0 || p.K % 8 || p.lda % 8 || p.ldw % 8) return RWKV7_ESHAPE;
    if (!p.A || !p.W || !p.Y) return RWKV7_EINVAL;
    if (p.bf != probs[0].bf || p.a32 != probs[0].a32) return RWKV7_EINVAL;  // one operand format per launch
  }
  const bool bf = probs[0].bf != 0, a32 = probs[0].a32 != 0;
  if (M <= (a32 ? kA32SkinnyMaxM : kSkinnyMaxM))
    return launch_skinny(probs, nprob, M, st, part, ctr, gemm_ws_bytes(M, cus));
  {
    // problems the large-M path takes run there; the rest (LoRA widths) below
    GemmProb big[kMaxProb], rest[kMaxProb];
    int nb = 0, nr = 0;
    for (int i = 0; i < nprob; ++i) {
      if (big_fits(probs[i], M, cus)) big[nb++] = probs[i];
      else rest[nr++] = probs[i];
    }
    if (nb > 0) {
      RWKV7_TRY_GEMM(launch_large_m(big, nb, M, cus, st, true));
      if (nr == 0) return RWKV7_OK;
      // The group's narrow problems at the same M (the LoRA first steps beside
      // r/k/v: N = 64..256, too few tiles for big_fits alone) join the
      // large-M kernel as well, 128 x 128 tiles in one launch (measured on the
      // 1.5B 4 x 1024 prefill: 21.4 -> 20.6 ms against the tiled kernels).
      bool fit = true;
      for (int i = 0; i < nr; ++i)
        fit = fit && rest[i].K % kBigBK == 0 && big_w_addressable(rest[i]) && big_rows_per_launch(rest[i].lda) >= 256;
      if (fit) return launch_large_m(rest, nr, M, cus, st, false);
      probs = rest;
      nprob = nr;
    }
  }
  plan_splits(probs, nprob, M, cus, part != nullptr && ctr != nullptr, S, ks);
  int wgs = 0, ctrs = 0;
  int64_t pfl = 0;
  for (int i = 0; i < kMaxProb; ++i) {
    g.wg_begin[i] = wgs;
    if (i < nprob) {
      const int tiles = g.m_tiles * ((probs[i].N + kBN - 1) / kBN);
      const int units = (probs[i].N + kBN - 1) / kBN * S[i];
      g.p[i] = probs[i];
      g.splits[i] = S[i];
      g.kslice[i] = ks[i];
      g.part_off[i] = pfl;
      g.ctr_off[i] = ctrs;
      wgs += (units + 7) / 8 * 8 * g.m_tiles;
      if (S[i] > 1) {
        pfl += (int64_t)tiles * S[i] * BM * kBN;
        ctrs += tiles;
      }
    } else {
      g.p[i] = probs[0];
      g.splits[i] = 1;
      g.kslice[i] = kKC;
      g.part_off[i] = 0;
      g.ctr_off[i] = 0;
    }
  }
  g.wg_begin[kMaxProb] = wgs;
  if (pfl * 4 > gemm_ws_bytes(M, cus) || ctrs > kGemmCounters) return RWKV7_EWORKSPACE;
  // every split of at most 8 chunks (4 with f32 A): the prefetch-all kernel
  int ncmax = 1;
  for (int i = 0; i < nprob; ++i) ncmax = max(ncmax, ks[i] / kKC);
  const int nc = ncmax == 1 ? 1 : ncmax == 2 ? 2 : ncmax <= 4 ? 4 : ncmax <= 8 ? 8 : 0;
  if ((BM == 32 || BM == 16) && nc > 0 && !(a32 && BM == 32 && nc > 4)) {
#define RWKV7_PF(NC)                                                                          \
  if (BM == 16) {                                                                             \
    if (bf) gemm_pf_kernel<16, NC, true, true><<<wgs, 256, 0, st>>>(g);                       \
    else gemm_pf_kernel<16, NC, false, true><<<wgs, 256, 0, st>>>(g);                         \
  } else if (bf) {                                                                            \
    if (a32) gemm_pf_kernel<32, NC < 4 ? NC : 4, true, true><<<wgs, 256, 0, st>>>(g);        \
    else gemm_pf_kernel<32, NC, true, false><<<wgs, 256, 0, st>>>(g);                         \
  } else {                                                                                    \
    if (a32) gemm_pf_kernel<32, NC < 4 ? NC : 4, false, true><<<wgs, 256, 0, st>>>(g);       \
    else gemm_pf_kernel<32, NC, false, false><<<wgs, 256, 0, st>>>(g);                        \
  }
    switch (nc) {
      case 1: RWKV7_PF(1) break;
      case 2: RWKV7_PF(2) break;
      case 4: RWKV7_PF(4) break;
      default: RWKV7_PF(8) break;
    }
#undef RWKV7_PF
    RWKV7_CHECK_LAUNCH();
    return RWKV7_OK;
  }
  // the row tiles bm_for picks: 16 (f32 A only), 32 or 64 rows
  if (BM == 16) {
    if (bf) gemm_kernel<16, true, true><<<wgs, 256, 0, st>>>(g);
    else gemm_kernel<16, false, true><<<wgs, 256, 0, st>>>(g);
    RWKV7_CHECK_LAUNCH();
    return RWKV7_OK;
  }
  const int variant = (BM == 32 ? 0 : 4) | (bf ? 2 : 0) | (a32 ? 1 : 0);
  switch (variant) {
    case 0: gemm_kernel<32, false, false><<<wgs, 256, 0, st>>>(g); break;
    case 1: gemm_kernel<32, false, true><<<wgs, 256, 0, st>>>(g); break;
    case 2: gemm_kernel<32, true, false><<<wgs, 256, 0, st>>>(g); break;
    case 3: gemm_kernel<32, true, true><<<wgs, 256, 0, st>>>(g); break;
    case 4: gemm_kernel<64, false, false><<<wgs, 256, 0, st>>>(g); break;
    case 5: gemm_kernel<64, false, true><<<wgs, 256, 0, st>>>(g); break;
    case 6: gemm_kernel<64, true, false><<<wgs, 256, 0, st>>>(g); break;
    default: gemm_kernel<64, true, true><<<wgs, 256, 0, st>>>(g); break;
  }
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

}  // namespace rwkv7
