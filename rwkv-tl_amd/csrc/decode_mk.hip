// One-token decode of one sequence as a single persistent kernel.
//
// A kernel launch costs ~1.6 us even when empty (graph replay on MI355X), and
// one RWKV7 layer is a chain of five dependent all-to-all stages:
//   P1  LN1 + token shift + r/k/v projections + LoRA first step   (3C+sumR rows)
//   P2  per head: LoRA second step, gates, L2 norm, wkv7, GroupNorm, gate
//   P3  o-projection + residual                                    (C rows)
//   P4  LN2 + token shift + FFN key + relu^2                       (F rows)
//   P5  FFN value + residual                                       (C rows, K=F)
// so decode is a chain of 5L+1 stages, each moving a few MiB of weights. Here
// the whole token runs in one launch with one workgroup per CU. Every stage's
// rows are split evenly over the workgroups; a workgroup issues the loads of
// its weight slice BEFORE waiting for the stage's input vector, so weight
// streaming overlaps the hand-off latency. Inputs are exchanged through global
// memory as 64-bit words {tag:32, value:32} written and read with device-scope
// (sc1) accesses: the consumer polls the data words themselves, so a hand-off
// costs one memory round trip and needs no atomics or cache maintenance. The
// tag is unique per (launch, stage), so words left over from older stages or
// launches never match.
//
// Every wait is bounded: past ~1 s a waiter raises a per-launch abort word and
// gives up, and every other waiter then gives up within a few polls, so a
// launch always terminates (its output is then garbage and an error counter is
// set). The grid must be resident all at once: one 512-thread workgroup per
// CU, grid = CU count.
//
// Reference counterparts: RWKV7Base.decode / make_TMIX / make_CMIX
// (demo/_rwkv7_base.py:74-87,153-206,285-290) and the captured decode graph
// (demo/cuda_graph.py:111-128).
#include "rwkv7_kernels.h"

#define RWKV7_DEV_HOST_INLINE __host__ __device__ inline

namespace rwkv7 {

constexpr int kT = 512;        // threads per workgroup
constexpr int kW = kT / 64;    // waves per workgroup
constexpr int kRMax = 4;       // max rows per wave in P1 / P4 (the RM template bound)
constexpr int kSpinLimit = 1 << 21;

// sync words (the first 256 bytes of the exchange region)
enum { SY_EPOCH = 0, SY_ABORT = 16, SY_ERRORS = 32 };

RWKV7_DEV unsigned ld_u32(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RWKV7_DEV void st_u32(unsigned *p, unsigned v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RWKV7_DEV uint64_t ld_u64(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RWKV7_DEV void publish(uint64_t *p, unsigned tag, float v) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __builtin_bit_cast(unsigned, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

struct MkCtx {
  unsigned *sync;
  unsigned epoch;
  unsigned nph;
  RWKV7_DEV unsigned tag(int phase) const {
    return (unsigned)(((uint64_t)epoch * nph + (uint64_t)phase) % 0xFFFFFFFFull) + 1u;
  }
  RWKV7_DEV bool aborted() const { return ld_u32(sync + SY_ABORT) == epoch + 1u; }
  RWKV7_DEV void abort() const {
    st_u32(sync + SY_ABORT, epoch + 1u);
    __hip_atomic_fetch_add(sync + SY_ERRORS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
};

// Waits until every word src[idx(i)] (i < n, i.e. the entries this thread
// handles: i = threadIdx.x + kT * j) carries `tag`, storing the values into
// dst[i]. Ends with a workgroup barrier.
template <int NPT, typename Idx>
RWKV7_DEV void poll_vec(const MkCtx &cx, const uint64_t *src, int n, unsigned tag, float *dst, Idx idx) {
  unsigned pending = 0;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
    if ((int)threadIdx.x + kT * j < n) pending |= 1u << j;
  int spins = 0;
  while (pending) {
    uint64_t w[NPT];
#pragma unroll
    for (int j = 0; j < NPT; ++j)
      if (pending & (1u << j)) w[j] = ld_u64(src + idx(threadIdx.x + kT * j));
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      if ((pending & (1u << j)) && (unsigned)(w[j] >> 32) == tag) {
        dst[threadIdx.x + kT * j] = __builtin_bit_cast(float, (unsigned)w[j]);
        pending &= ~(1u << j);
      }
    }
    if (pending) {
      ++spins;
      if ((spins & 63) == 0 && cx.aborted()) break;
      if (spins > kSpinLimit) {
        cx.abort();
        break;
      }
    }
  }
  __syncthreads();
}

// acc + sum_e w[e] * x[e] for 8 f16 weights and 8 f32 inputs in LDS.
RWKV7_DEV float dot8(const uint4 &w, const float *x, float acc) {
  float wf[8];
  h8_to_f(w, wf);
  const float4 u = reinterpret_cast<const float4 *>(x)[0], v = reinterpret_cast<const float4 *>(x)[1];
  acc = fmaf(wf[0], u.x, acc); acc = fmaf(wf[1], u.y, acc);
  acc = fmaf(wf[2], u.z, acc); acc = fmaf(wf[3], u.w, acc);
  acc = fmaf(wf[4], v.x, acc); acc = fmaf(wf[5], v.y, acc);
  acc = fmaf(wf[6], v.z, acc); acc = fmaf(wf[7], v.w, acc);
  return acc;
}

struct Ident {
  RWKV7_DEV int operator()(int i) const { return i; }
};

// Sum over the 512 threads; every thread gets the result.
RWKV7_DEV float block_sum(float v, float *red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kW; ++i) s += red[i];
  return s;
}

// out[c] = LN(x)[c] for c < C (x, out in LDS; out may alias x).
RWKV7_DEV void ln_lds(const float *x, float *out, const float *w, const float *b, int C, float *red) {
  float s = 0.f;
  for (int c = threadIdx.x; c < C; c += kT) s += x[c];
  const float mean = block_sum(s, red) / (float)C;
  float q = 0.f;
  for (int c = threadIdx.x; c < C; c += kT) {
    const float d = x[c] - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(block_sum(q, red) / (float)C + kLnEps);
  __syncthreads();
  for (int c = threadIdx.x; c < C; c += kT) out[c] = (x[c] - mean) * rstd * w[c] + b[c];
  __syncthreads();
}

// Floats of the stage-input region: the polled FFN hidden vector, P2's inputs,
// or up to 4 per-segment mixed vectors of P1.
RWKV7_DEV_HOST_INLINE int mk_nin(int C, int F, int SR) {
  int n = F > 192 + SR ? F : 192 + SR;
  return n > 4 * C ? n : 4 * C;
}

struct MkArgs {
  const char *layers;
  int64_t lbytes, o_rkv, o_l2, o_o, o_fk, o_fv, o_vec;
  const uint16_t *emb, *head;
  const float *ln_out;
  int L, C, H, F, V, rv, rw, ra, rg;
  uint16_t *tmix_x;
  float *rnn;
  uint16_t *cmix_x;
  const int64_t *tok;
  uint16_t *logits;
  uint64_t *x_ex, *proj_ex, *core_ex, *hid_ex;
  unsigned *sync;
};

// Loads this wave's rows of W (row stride ld halfs) for a wave-per-row stage:
// wave w owns rows r0 + w + kW * i (i < RM) below r1; lane l holds the
// 16-byte chunks l + 64 * c of each row.
template <int RM, int CPL>
RWKV7_DEV void load_rows(const uint16_t *W, int64_t ld, int r0, int r1, int K, uint4 (&wreg)[RM][CPL]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nch = K >> 3;
#pragma unroll
  for (int i = 0; i < RM; ++i) {
    const int r = r0 + wv + kW * i;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int j = lane + 64 * c;
      wreg[i][c] = (r < r1 && j < nch) ? ld_stream(reinterpret_cast<const uint4 *>(W + (int64_t)r * ld) + j)
                                       : make_uint4(0, 0, 0, 0);
    }
  }
}

// Rows split along K over several waves (P3, P5): wave w works on row
// r0 + w / ks, K-part w % ks; lane chunks j = part*per + lane + 64*c.
template <int NC>
RWKV7_DEV void load_split(const uint16_t *W, int64_t ld, int r0, int nrow, int ks, int K, uint4 (&wreg)[NC]) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nch = K >> 3, per = (nch + ks - 1) / ks;
  const int row = wv / ks, part = wv % ks;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int jj = lane + 64 * c;
    const int j = part * per + jj;
    wreg[c] = (row < nrow && jj < per && j < nch)
                  ? ld_stream(reinterpret_cast<const uint4 *>(W + (int64_t)(r0 + row) * ld) + j)
                  : make_uint4(0, 0, 0, 0);
  }
}

// Partial dot of the split rows with x (LDS f32, K values); partial sums are
// combined through red[] and row results returned to threads t < nrow.
template <int NC>
RWKV7_DEV float dot_split(const uint4 (&wreg)[NC], const float *x, int nrow, int ks, int K, float *red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int nch = K >> 3, per = (nch + ks - 1) / ks;
  const int part = wv % ks;
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int jj = lane + 64 * c;
    const int j = part * per + jj;
    if (jj < per && j < nch) {
      acc = dot8(wreg[c], x + 8 * j, acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) red[wv] = acc;
  __syncthreads();
  float out = 0.f;
  if ((int)threadIdx.x < nrow) {
    for (int p = 0; p < ks; ++p) out += red[threadIdx.x * ks + p];
  }
  __syncthreads();
  return out;
}

// Loads vec[c] for this thread's elements c = threadIdx.x + kT * i (i < CPL).
template <int CPL>
RWKV7_DEV void ld_own(float (&dst)[CPL], const float *src, int C) {
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = threadIdx.x + kT * i;
    dst[i] = c < C ? src[c] : 0.f;
  }
}
template <int CPL>
RWKV7_DEV void ld_own16(float (&dst)[CPL], const uint16_t *src, int C) {
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = threadIdx.x + kT * i;
    dst[i] = c < C ? h2f(src[c]) : 0.f;
  }
}

// Polls this thread's own elements c = threadIdx.x + kT * i of a tagged vector
// into registers (no barrier).
template <int CPL>
RWKV7_DEV void poll_own(const MkCtx &cx, const uint64_t *src, int n, unsigned tag, float (&dst)[CPL]) {
  unsigned pending = 0;
#pragma unroll
  for (int i = 0; i < CPL; ++i)
    if ((int)threadIdx.x + kT * i < n) pending |= 1u << i;
    else dst[i] = 0.f;
  int spins = 0;
  while (pending) {
    uint64_t w[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i)
      if (pending & (1u << i)) w[i] = ld_u64(src + threadIdx.x + kT * i);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      if ((pending & (1u << i)) && (unsigned)(w[i] >> 32) == tag) {
        dst[i] = __builtin_bit_cast(float, (unsigned)w[i]);
        pending &= ~(1u << i);
      }
    }
    if (pending) {
      ++spins;
      if ((spins & 63) == 0 && cx.aborted()) break;
      if (spins > kSpinLimit) {
        cx.abort();
        break;
      }
    }
  }
}

// LayerNorm of a vector held as this thread's own elements (block reductions).
template <int CPL>
RWKV7_DEV void ln_own(float (&x)[CPL], const float (&w)[CPL], const float (&b)[CPL], int C, float *red) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) s += x[i];
  const float mean = block_sum(s, red) / (float)C;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i)
    if ((int)threadIdx.x + kT * i < C) {
      const float d = x[i] - mean;
      q += d * d;
    }
  const float rstd = rsqrtf(block_sum(q, red) / (float)C + kLnEps);
#pragma unroll
  for (int i = 0; i < CPL; ++i) x[i] = (x[i] - mean) * rstd * w[i] + b[i];
}

// RM: rows per wave in P1/P4; CPL: 16-byte chunks per lane of a C-long row
// (also this thread's share of a C-long vector); NC5: chunks per lane of the
// K-split rows of P3/P5; NPTH: hidden-vector words polled per thread; NL2:
// LoRA second-step chunks per thread.
template <int RM, int CPL, int NC5, int NPTH, int NL2>
__global__ __launch_bounds__(kT) void decode_mk_kernel(MkArgs a) {
  extern __shared__ __align__(16) float smem[];
  const int C = a.C, F = a.F, H = a.H, L = a.L;
  const int SR = a.rv + a.rw + a.ra + a.rg;
  const int G = gridDim.x, g = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;

  float *s_x = smem;             // [C]  mixed input of P4 / normalised input of the head
  float *s_ln1 = s_x + C;        // [C]  LN1 output (kept to P3 for the shift state)
  float *s_ln2 = s_ln1 + C;      // [C]  LN2 output (kept to P5)
  float *s_spare = s_ln2 + C;    // [C]
  const int nin = mk_nin(C, F, SR);
  float *s_in = s_spare + C;     // [nin] polled stage inputs / P1 segment mixes
  float *s_red = s_in + nin;     // [64]
  float *s_own = s_red + 64;     // [16] this workgroup's rows of the residual
  float *s_vf = s_own + 16;      // [64] v_first of the head this workgroup owns
  float *s_core = s_vf + 64;     // [8][64] r w k v a b g y
  float *s_lora = s_core + 8 * 64;  // [512]
  float *s_d = s_lora + 512;        // [4][64] LoRA second-step results
  (void)s_spare;

  MkCtx cx;
  cx.sync = a.sync;
  cx.epoch = ld_u32(a.sync + SY_EPOCH);
  cx.nph = 5u * L + 1u;

  const int N1 = 3 * C + SR;
  const int p1a = (int)((int64_t)N1 * g / G), p1b = (int)((int64_t)N1 * (g + 1) / G);
  const int p4a = (int)((int64_t)F * g / G), p4b = (int)((int64_t)F * (g + 1) / G);
  const int owa = (int)((int64_t)C * g / G), owb = (int)((int64_t)C * (g + 1) / G);
  const int nown = owb - owa;
  const int ks = nown > 0 ? (kW / nown > 0 ? kW / nown : 1) : 1;

  int64_t token = a.tok[0];
  token = token < 0 ? 0 : token >= a.V ? a.V - 1 : token;
  const uint16_t *erow = a.emb + token * C;
  if (t < nown) s_own[t] = h2f(erow[owa + t]);

  // rows of the stacked P1 matrix fall in 7 segments: r, k, v, LoRA v, w, a, g
  const int e0 = C, e1 = 2 * C, e2 = 3 * C, e3 = e2 + a.rv, e4 = e3 + a.rw, e5 = e4 + a.ra;
  auto seg_of = [=](int r) {
    return (r >= e0) + (r >= e1) + (r >= e2) + (r >= e3) + (r >= e4) + (r >= e5);
  };
  auto seg_mu = [](int sgm) {  // vector-block index of each segment's mix
    return sgm == 0 ? RWKV7_V_X_R : sgm == 1 ? RWKV7_V_X_K : sgm <= 3 ? RWKV7_V_X_V
         : sgm == 4 ? RWKV7_V_X_W : sgm == 5 ? RWKV7_V_X_A : RWKV7_V_X_G;
  };
  const int seg0 = seg_of(p1a), nseg = seg_of(p1b - 1) - seg0 + 1;

  // P2 thread roles: 8 threads per channel c2 of the head; thread sub2 takes the
  // 16-byte chunks sub2, sub2+8, ... of the channel's [v|w|a|g] LoRA row
  const int c2 = t >> 3, sub2 = t & 7;
  const int nch2 = SR >> 3;
  const int b1 = a.rv >> 3, b2 = (a.rv + a.rw) >> 3, b3 = (a.rv + a.rw + a.ra) >> 3;  // gate bounds in chunks

  // ---- prefetched operands (each issued one stage ahead of its use) -----------
  uint4 w1[RM][CPL];               // P1 rows
  float ln1w[CPL], ln1b[CPL], prv1[CPL], mu1[4][CPL];
  uint4 w2[NL2];                   // P2 LoRA second-step chunks
  float4 S0 = make_float4(0.f, 0.f, 0.f, 0.f), S1 = S0;  // P2 state rows
  float gv[8];                     // P2 per-channel vectors
  uint4 w3[NC5];                   // P3 rows
  uint4 w4[RM][CPL];               // P4 rows
  float ln2w[CPL], ln2b[CPL], prv2[CPL], mu4[CPL];
  uint4 w5[NC5];                   // P5 rows

  auto prefetch_p1 = [&](int l) {
    const char *Lp = a.layers + (int64_t)l * a.lbytes;
    const float *vec = reinterpret_cast<const float *>(Lp + a.o_vec);
    load_rows<RM, CPL>(reinterpret_cast<const uint16_t *>(Lp + a.o_rkv), C, p1a, p1b, C, w1);
    ld_own<CPL>(ln1w, vec + RWKV7_V_LN1_W * C, C);
    ld_own<CPL>(ln1b, vec + RWKV7_V_LN1_B * C, C);
    ld_own16<CPL>(prv1, a.tmix_x + (int64_t)l * C, C);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (q < nseg) ld_own<CPL>(mu1[q], vec + (int64_t)seg_mu(seg0 + q) * C, C);
  };

  prefetch_p1(0);
  float xo[CPL];
  ld_own16<CPL>(xo, erow, C);

  for (int l = 0; l < L; ++l) {
    const char *Lp = a.layers + (int64_t)l * a.lbytes;
    const float *vec = reinterpret_cast<const float *>(Lp + a.o_vec);
    const int ph = 5 * l;

    // ---------------- P1: LN1 + shift + [r;k;v;LoRA1] ------------------------
    {
      if (l > 0) poll_own<CPL>(cx, a.x_ex, C, cx.tag(ph - 1), xo);
      // stage-ahead prefetch: P2 (head workgroups) and P3
      if (g < H) {
        const uint4 *row = reinterpret_cast<const uint4 *>(
            reinterpret_cast<const uint16_t *>(Lp + a.o_l2) + (int64_t)(g * kN + c2) * SR);
#pragma unroll
        for (int i = 0; i < NL2; ++i) w2[i] = sub2 + 8 * i < nch2 ? row[sub2 + 8 * i] : make_uint4(0, 0, 0, 0);
        const float4 *Sp = reinterpret_cast<const float4 *>(
            a.rnn + (((int64_t)l * H + g) * kN + (t >> 3)) * kN + (t & 7) * 8);
        S0 = Sp[0];
        S1 = Sp[1];
        if (t < 64) {
          const int ch = g * kN + t;
          const int idx[8] = {RWKV7_V_V0, RWKV7_V_W0, RWKV7_V_A0, RWKV7_V_K_K,
                              RWKV7_V_K_A, RWKV7_V_R_K, RWKV7_V_LNX_W, RWKV7_V_LNX_B};
#pragma unroll
          for (int j = 0; j < 8; ++j) gv[j] = vec[idx[j] * C + ch];
        }
      }
      ln_own<CPL>(xo, ln1w, ln1b, C, s_red);
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = t + kT * i;
        if (c < C) {
          s_ln1[c] = xo[i];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (q < nseg) s_in[q * C + c] = xo[i] + mu1[q][i] * (prv1[i] - xo[i]);
        }
      }
      __syncthreads();
      const unsigned tg = cx.tag(ph);
#pragma unroll
      for (int i = 0; i < RM; ++i) {
        const int r = p1a + wv + kW * i;
        if (r >= p1b) break;
        const float *xs = s_in + (seg_of(r) - seg0) * C;
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int j = lane + 64 * c;
          if (j < (C >> 3)) acc = dot8(w1[i][c], xs + 8 * j, acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) publish(a.proj_ex + r, tg, acc);
      }
      // stage-ahead prefetch: P3 (small; issued here to keep it out of P1's registers)
      load_split<NC5>(reinterpret_cast<const uint16_t *>(Lp + a.o_o), C, owa, nown, ks, C, w3);
      // P2 / P3 poll into s_in, which still holds the segment mixes other waves read
      __syncthreads();
    }

    // ---------------- P2: per-head core (workgroups 0..H-1) -------------------
    if (g < H) {
      const int h = g;
      poll_vec<2>(cx, a.proj_ex, 192 + SR, cx.tag(ph), s_in, [&](int i) {
        return i < 192 ? (i >> 6) * C + h * kN + (i & 63) : 3 * C + (i - 192);
      });
      for (int i = t; i < SR; i += kT) {
        float x = s_in[192 + i];
        if (i >= a.rv && i < a.rv + a.rw) x = tanhf(x);
        else if (i >= a.rv + a.rw + a.ra) x = sigmoidf_(x);
        s_lora[i] = x;
      }
      __syncthreads();
      float *s_r = s_core, *s_w = s_core + 64, *s_k = s_core + 128, *s_v = s_core + 192;
      float *s_a = s_core + 256, *s_b = s_core + 320, *s_g = s_core + 384, *s_y = s_core + 448;
      {  // LoRA second step from the prefetched chunks; per-gate partial sums joined
         // across the channel's 8 lanes
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NL2; ++i) {
          const int cj = sub2 + 8 * i;
          if (cj < nch2) {
            const float p = dot8(w2[i], s_lora + 8 * cj, 0.f);
            const int q = (cj >= b1) + (cj >= b2) + (cj >= b3);
            acc[0] += q == 0 ? p : 0.f;
            acc[1] += q == 1 ? p : 0.f;
            acc[2] += q == 2 ? p : 0.f;
            acc[3] += q == 3 ? p : 0.f;
          }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float v = sum4(acc[q]);
          v += dpp<kDppHalfMirror>(v);
          if (sub2 == 0) s_d[q * 64 + c2] = v;
        }
      }
      __syncthreads();
      if (t < 64) {
        const float r = s_in[t], k = s_in[64 + t];
        float v = s_in[128 + t];
        if (l == 0) {
          s_vf[t] = v;
        } else {
          v = v + sigmoidf_(gv[0] + s_d[t]) * (s_vf[t] - v);
        }
        const float w = expf(-sigmoidf_(gv[1] + s_d[64 + t]) / 1.6487212707001282f);
        const float ag = sigmoidf_(gv[2] + s_d[128 + t]);
        const float kk = k * gv[3];
        const float kn = k + gv[4] * (k * ag - k);
        const float nrm = sqrtf(wave_sum(kk * kk));
        const float kh = kk / fmaxf(nrm, 1e-12f);
        const float rk = wave_sum(r * kn * gv[5]);
        s_r[t] = r; s_w[t] = w; s_k[t] = kn; s_v[t] = v;
        s_a[t] = kh; s_b[t] = -kh * ag; s_g[t] = s_d[192 + t];
        if (t == 0) s_red[32] = rk;
      }
      __syncthreads();
      {
        const int row = t >> 3, j0 = (t & 7) * 8;
        float Sv[8] = {S0.x, S0.y, S0.z, S0.w, S1.x, S1.y, S1.z, S1.w};
        float sa = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sa = fmaf(Sv[e], s_a[j0 + e], sa);
        sa = sum4(sa);
        sa += dpp<kDppHalfMirror>(sa);
        const float vi = s_v[row];
        float y = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = j0 + e;
          Sv[e] = Sv[e] * s_w[j] + sa * s_b[j] + vi * s_k[j];
          y = fmaf(Sv[e], s_r[j], y);
        }
        y = sum4(y);
        y += dpp<kDppHalfMirror>(y);
        float4 *Sp = reinterpret_cast<float4 *>(a.rnn + (((int64_t)l * H + h) * kN + row) * kN + j0);
        Sp[0] = make_float4(Sv[0], Sv[1], Sv[2], Sv[3]);
        Sp[1] = make_float4(Sv[4], Sv[5], Sv[6], Sv[7]);
        if ((t & 7) == 0) s_y[row] = y;
      }
      __syncthreads();
      if (t < 64) {
        const int ch = h * kN + t;
        const float y = s_y[t];
        const float mean = wave_sum(y) * (1.f / kN);
        const float d = y - mean;
        const float var = wave_sum(d * d) * (1.f / kN);
        const float yn = d * rsqrtf(var + kGnEps) * gv[6] + gv[7];
        publish(a.core_ex + ch, cx.tag(ph + 1), (yn + s_red[32] * s_v[t]) * s_g[t]);
      }
    }

    // ---------------- P3: o-projection + residual -----------------------------
    {
      poll_vec<4>(cx, a.core_ex, C, cx.tag(ph + 1), s_in, Ident());
      // stage-ahead prefetch: P4
      load_rows<RM, CPL>(reinterpret_cast<const uint16_t *>(Lp + a.o_fk), C, p4a, p4b, C, w4);
      ld_own<CPL>(ln2w, vec + RWKV7_V_LN2_W * C, C);
      ld_own<CPL>(ln2b, vec + RWKV7_V_LN2_B * C, C);
      ld_own<CPL>(mu4, vec + RWKV7_V_FFN_X_K * C, C);
      ld_own16<CPL>(prv2, a.cmix_x + (int64_t)l * C, C);
      const float d = dot_split<NC5>(w3, s_in, nown, ks, C, s_red);
      const unsigned tg = cx.tag(ph + 2);
      if (t < nown) {
        s_own[t] += d;
        publish(a.x_ex + owa + t, tg, s_own[t]);
        // every reader of this layer's time-mix shift state is done (all of P2's inputs arrived)
        a.tmix_x[(int64_t)l * C + owa + t] = f2h(s_ln1[owa + t]);
      }
    }

    // ---------------- P4: LN2 + shift + FFN key + relu^2 ----------------------
    {
      poll_own<CPL>(cx, a.x_ex, C, cx.tag(ph + 2), xo);
      // stage-ahead prefetch: P5
      load_split<NC5>(reinterpret_cast<const uint16_t *>(Lp + a.o_fv), F, owa, nown, ks, F, w5);
      ln_own<CPL>(xo, ln2w, ln2b, C, s_red);
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = t + kT * i;
        if (c < C) {
          s_ln2[c] = xo[i];
          s_x[c] = xo[i] + mu4[i] * (prv2[i] - xo[i]);
        }
      }
      __syncthreads();
      const unsigned tg = cx.tag(ph + 3);
#pragma unroll
      for (int i = 0; i < RM; ++i) {
        const int r = p4a + wv + kW * i;
        if (r >= p4b) break;
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int j = lane + 64 * c;
          if (j < (C >> 3)) acc = dot8(w4[i][c], s_x + 8 * j, acc);
        }
        acc = wave_sum(acc);
        const float q = fmaxf(acc, 0.f);
        if (lane == 0) publish(a.hid_ex + r, tg, q * q);
      }
    }

    // ---------------- P5: FFN value + residual --------------------------------
    {
      poll_vec<NPTH>(cx, a.hid_ex, F, cx.tag(ph + 3), s_in, Ident());
      if (l + 1 < L) prefetch_p1(l + 1);  // stage-ahead prefetch: next layer's P1
      const float d = dot_split<NC5>(w5, s_in, nown, ks, F, s_red);
      const unsigned tg = cx.tag(ph + 4);
      if (t < nown) {
        s_own[t] += d;
        publish(a.x_ex + owa + t, tg, s_own[t]);
        a.cmix_x[(int64_t)l * C + owa + t] = f2h(s_ln2[owa + t]);
      }
    }
  }

  // ---------------- head: ln_out + logits ---------------------------------------
  {
    const int ha = (int)((int64_t)a.V * g / G), hb = (int)((int64_t)a.V * (g + 1) / G);
    float low[CPL], lob[CPL];
    ld_own<CPL>(low, a.ln_out, C);
    ld_own<CPL>(lob, a.ln_out + C, C);
    uint4 wh[4][CPL];
    auto load_head = [&](int r0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int j = lane + 64 * c;
          wh[i][c] = (r0 + i < hb && j < (C >> 3))
                         ? ld_stream(reinterpret_cast<const uint4 *>(a.head + (int64_t)(r0 + i) * C) + j)
                         : make_uint4(0, 0, 0, 0);
        }
    };
    load_head(ha + wv * 4);
    poll_own<CPL>(cx, a.x_ex, C, cx.tag(5 * L - 1), xo);
    ln_own<CPL>(xo, low, lob, C, s_red);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = t + kT * i;
      if (c < C) s_x[c] = xo[i];
    }
    __syncthreads();
    for (int r0 = ha + wv * 4; r0 < hb; r0 += kW * 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int j = lane + 64 * c;
          if (j < (C >> 3)) acc = dot8(wh[i][c], s_x + 8 * j, acc);
        }
        acc = wave_sum(acc);
        if (lane == i && r0 + i < hb) a.logits[r0 + i] = f2h(acc);
      }
      if (r0 + kW * 4 < hb) load_head(r0 + kW * 4);
    }
  }
  // all workgroups have read the epoch and passed their last wait on it
  if (g == 0 && t == 0) st_u32(a.sync + SY_EPOCH, cx.epoch + 1u);
}

// ---- host side --------------------------------------------------------------

// Chunks per lane of the K-split P3/P5 rows for workgroup count G.
static int mk_nc5(const rwkv7_dims &d, int G) {
  const int C = d.n_embd, F = d.n_ffn;
  int nown = (C + G - 1) / G;
  if (nown < 1) nown = 1;
  const int ks = kW / nown > 0 ? kW / nown : 1;
  const int per = ((F >> 3) + ks - 1) / ks;
  return (per + 63) / 64;
}

// Template instance for these sizes: 0 = <2,2,4,8,5>; -1 if none fits.
static int mk_variant(const rwkv7_dims &d, int G) {
  const int cpl = ((d.n_embd >> 3) + 63) / 64, nc5 = mk_nc5(d, G), npth = (d.n_ffn + kT - 1) / kT;
  const int nl2 = ((d.rank_w + d.rank_a + d.rank_v + d.rank_g) / 8 + 7) / 8;  // P2 chunks per thread
  const int n1 = 3 * d.n_embd + d.rank_w + d.rank_a + d.rank_v + d.rank_g;
  const int rm = ((n1 + G - 1) / G + kW - 1) / kW > ((d.n_ffn + G - 1) / G + kW - 1) / kW
                     ? ((n1 + G - 1) / G + kW - 1) / kW
                     : ((d.n_ffn + G - 1) / G + kW - 1) / kW;
  if (rm <= 2 && cpl <= 2 && nc5 <= 4 && npth <= 8 && nl2 <= 5) return 0;
  // The wider instances (n_embd 2048) exceed the register file and spill to
  // scratch; those models decode one sequence through the GEMV kernels instead.
  return -1;
}

static int g_cus = 0;

int mk_cus() {
  if (g_cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return 0;
    g_cus = p.multiProcessorCount;
  }
  return g_cus;
}

int64_t mk_lds_bytes(int C, int F, int SR) {
  const int nin = mk_nin(C, F, SR);
  return (int64_t)(4 * C + nin + 64 + 16 + 64 + 8 * 64 + 512 + 256) * 4;
}

// Exchange region: sync words, then x (C), proj (3C+SR), core (C), hid (F) as u64.
int64_t mk_exchange_bytes(int C, int F, int SR) {
  return 256 + (int64_t)(C + 3 * C + SR + C + F) * 8;
}


bool mk_supported(const rwkv7_dims &d, int G) {
  const int C = d.n_embd, F = d.n_ffn, SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g;
  if (G < 1) return false;
  const int N1 = 3 * C + SR;
  const int c8 = C >> 3;
  if (C > 2048 || (c8 + 63) / 64 > 4) return false;
  if ((N1 + G - 1) / G > kRMax * kW || (F + G - 1) / G > kRMax * kW) return false;
  if ((C + G - 1) / G > 16) return false;
  if (mk_variant(d, G) < 0) return false;
  if (F > 8192 || 192 + SR > 8192) return false;

  // P1 keeps the mixed input of every row segment a workgroup touches (<= 4)
  const int e[6] = {C, 2 * C, 3 * C, 3 * C + d.rank_v, 3 * C + d.rank_v + d.rank_w,
                    3 * C + d.rank_v + d.rank_w + d.rank_a};
  auto seg = [&](int r) {
    int s = 0;
    for (int i = 0; i < 6; ++i) s += r >= e[i];
    return s;
  };
  for (int g = 0; g < G; ++g) {
    const int r0 = (int)((int64_t)N1 * g / G), r1 = (int)((int64_t)N1 * (g + 1) / G);
    if (r1 <= r0 || seg(r1 - 1) - seg(r0) + 1 > 4) return false;
  }
  return mk_lds_bytes(C, F, SR) <= 160 * 1024;
}

int launch_decode_mk(const rwkv7_model &m, const rwkv7_layer_layout &lay, const rwkv7_state &s,
                     const int64_t *tok, void *logits, char *xreg, hipStream_t st) {
  const rwkv7_dims &d = m.dims;
  const int SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g;
  const int G = mk_cus();
  const int C = d.n_embd, F = d.n_ffn;
  MkArgs a;
  a.layers = static_cast<const char *>(m.layers);
  a.lbytes = lay.bytes;
  a.o_rkv = lay.w_rkv;
  a.o_l2 = lay.w_lora2;
  a.o_o = lay.w_o;
  a.o_fk = lay.w_fk;
  a.o_fv = lay.w_fv;
  a.o_vec = lay.vec;
  a.emb = static_cast<const uint16_t *>(m.emb);
  a.head = static_cast<const uint16_t *>(m.head);
  a.ln_out = static_cast<const float *>(m.ln_out);
  a.L = d.n_layer;
  a.C = C;
  a.H = d.n_head;
  a.F = F;
  a.V = d.vocab;
  a.rv = d.rank_v;
  a.rw = d.rank_w;
  a.ra = d.rank_a;
  a.rg = d.rank_g;
  a.tmix_x = static_cast<uint16_t *>(s.tmix_x);
  a.rnn = static_cast<float *>(s.rnn);
  a.cmix_x = static_cast<uint16_t *>(s.cmix_x);
  a.tok = tok;
  a.logits = static_cast<uint16_t *>(logits);
  a.sync = reinterpret_cast<unsigned *>(xreg);
  uint64_t *ex = reinterpret_cast<uint64_t *>(xreg + 256);
  a.x_ex = ex;
  a.proj_ex = a.x_ex + C;
  a.core_ex = a.proj_ex + 3 * C + SR;
  a.hid_ex = a.core_ex + C;
  const int64_t lds = mk_lds_bytes(C, F, SR);
  const int variant = mk_variant(d, G);
  const void *fn = (const void *)decode_mk_kernel<2, 2, 4, 8, 5>;
  if (variant < 0) return RWKV7_ESHAPE;
  static int64_t lds_set = 0;  // largest dynamic LDS size already allowed
  if (lds > lds_set) {
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return RWKV7_ELAUNCH;
    lds_set = lds;
  }
  decode_mk_kernel<2, 2, 4, 8, 5><<<G, kT, lds, st>>>(a);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

}  // namespace rwkv7
