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
// the whole token runs in one launch with one workgroup per CU; every stage's
// rows are split evenly over the workgroups and exchanged through global memory
// as 64-bit words {tag:32, value:32}, written and read with device-scope (sc1)
// accesses. The consumer polls the data words themselves, so a hand-off costs
// one memory round trip and needs no atomics or cache maintenance; the tag is
// unique per (launch, stage), so words left over from older stages or launches
// never match.
//
// Wave roles. Vector-memory loads of one wave complete in issue order, so a
// wave that polls hand-off words while weight loads are in flight waits for
// those loads on every poll. The workgroup therefore splits the two jobs:
//   * wave 7 (the comm wave) never issues a weight load; it probes each
//     stage's input vector (one word, offset per workgroup) and, once the
//     probe sees the vector arriving, tells the other waves through an LDS
//     flag;
//   * waves 0..6 (math waves) stream weights into registers a stage or more
//     ahead of their use and compute; a worker issues all of a layer's
//     remaining weight loads right after its P1 publish, so they are old by
//     the time its next poll waits behind them.
// After the probe every wave reads one slice of the vector (8 readers, one
// read round), and leaves the LayerNorm partials (mean, M2) of its slice in
// LDS; the stage's threads combine the 8 pairs. The roles meet at the same
// sequence of workgroup barriers (listed above comm_worker). Every output row
// belongs to one math wave, so apart from the per-head core (P2) and the
// LayerNorm partials no stage needs a cross-wave reduction.
//
// Every wait is bounded: past ~1 s a waiting wave raises a per-launch abort
// word and gives up, every other waiting wave then gives up within a few polls,
// and barriers never wait on memory, so a launch always terminates. A
// workgroup that gave up (or found the launch aborted) publishes nothing
// more, writes no more state, and writes NaN logits; the launch's first worker
// counts the aborted launch in an error word that the host reads
// (rwkv7_workspace_errors). State layers updated before the failure stay
// updated. The grid must be resident all at once: one 512-thread workgroup
// per CU, grid = CU count; the host checks the occupancy for this kernel
// before choosing it.
//
// Reference counterparts: RWKV7Base.decode / make_TMIX / make_CMIX
// (demo/_rwkv7_base.py:74-87,153-206,285-290) and the captured decode graph
// (demo/cuda_graph.py:111-128).
#include <atomic>
#include <type_traits>

#include "rwkv7_kernels.h"

#define RWKV7_DEV_HOST_INLINE __host__ __device__ inline

namespace rwkv7 {

constexpr int kT = 512;          // threads per workgroup
constexpr int kW = kT / 64;      // waves per workgroup
constexpr int kNComm = 1;        // comm waves (the last ones)
constexpr int kMW = kW - kNComm; // math waves 0..kMW-1
constexpr int kMT = kMW * 64;    // math threads
constexpr int kHB = 4;           // head rows per batch
constexpr int kHRing = 3;        // head batches in flight
constexpr int kSpinLimit = 1 << 21;
// timeline points (diagnostic build): workers 0 P1 input ready, 1 P1 published,
// 2 P3 input ready, 3 P3 published, 4 P4 input ready, 5 P4 published, 6 P5
// input ready, 7 P5 published; head workgroups 8 P2 input ready, 9 P2 published
RWKV7_TL_BUFFER(tl_decode);
constexpr int kRep = 8;          // replicas of each broadcast hand-off vector
constexpr int kHidProbe = 4096;  // probe stride of the FFN hidden vector
constexpr int kXProbe = 1024;    // probe stride of the x vectors
static_assert(kRep < 64, "lanes 0..kRep of a wave publish a value and its state");

// 32-bit sync words at the start of the exchange region (byte offsets 0, 16
// and 32): launch epoch, abort word (epoch + 1 while the launch with that
// epoch is aborted), count of aborted launches. Then kMaxG start words (one per
// workgroup: epoch + 1 once it started), then the hand-off vectors.
enum { SY_EPOCH = 0, SY_ABORT = 4, SY_ERRORS = 8 };
constexpr int kSyncBytes = 256;
constexpr int kMaxG = 1024;

// s_waitcnt vmcnt(0), leaving the export and LDS counters alone
RWKV7_DEV void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Keeps the instruction scheduler from moving anything across this point:
// placed after a prefetch so its loads are issued there, not sunk next to
// their first use.
RWKV7_DEV void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

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

// Tags are 32-bit and wrap: tag = epoch * nph + 1 + phase (mod 2^32). A slot
// is rewritten by every launch, so a stale word is at most one launch old
// (or a few, after aborted launches), and two tags of one slot collide only
// k launches apart with k * nph = 0 (mod 2^32), i.e. never in practice. The
// first launch on a zeroed workspace uses tags 1..nph, never 0.
struct MkCtx {
  unsigned *sync;
  unsigned *fail;  // LDS word: nonzero once a wave of this workgroup gave up a wait
  unsigned epoch;
  unsigned tag0;  // epoch * nph + 1
  int pskew;      // probe offset of this workgroup (even)
  RWKV7_DEV unsigned tag(int phase) const { return tag0 + (unsigned)phase; }
  RWKV7_DEV bool aborted() const { return ld_u32(sync + SY_ABORT) == epoch + 1u; }
  RWKV7_DEV bool failed() const {
    return __hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u;
  }
  RWKV7_DEV void give_up() const { __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
  RWKV7_DEV void abort() const {
    st_u32(sync + SY_ABORT, epoch + 1u);
    give_up();
  }
};

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
  // hand-off words; x, proj, core and hid have kRep replicas of C, 3C+SR, C
  // and F words
  uint64_t *x_ex, *proj_ex, *core_ex, *hid_ex;
  unsigned *sync;
  unsigned *started;  // [kMaxG] start words
  // int8 weights (the Q8 instance): per-layer arenas and their sections, the
  // head and its row scales
  const char *layers_q;
  int64_t q_lbytes, q_rkv, q_o, q_fk, q_fv, q_scale;
  const uint16_t *head_q;  // int8 rows of C bytes, addressed in 16-bit units
  const float *head_qs;
};

// Row ranges and roles, computed identically by every wave of a workgroup.
struct MkGeom {
  int C, F, H, L, SR, G, g;
  int p1a, p1b;      // rows of the stacked [r;k;v;LoRA1] matrix (P1)
  int p4a, p4b;      // rows of the FFN key matrix (P4)
  int owa, nown;     // channels whose residual this workgroup owns (P3, P5)
  int seg0, nseg;    // P1 row segments touched (see seg_of)
  int ha, hb;        // head rows
  bool head;         // this workgroup runs the per-head core of head g (P2)
  int e[6];          // P1 segment starts: k, v, LoRA v, w, a, g
  RWKV7_DEV int seg_of(int r) const {
    return (r >= e[0]) + (r >= e[1]) + (r >= e[2]) + (r >= e[3]) + (r >= e[4]) + (r >= e[5]);
  }
};

RWKV7_DEV int seg_mu(int sgm) {  // vector-block index of each P1 segment's mix
  return sgm == 0 ? RWKV7_V_X_R : sgm == 1 ? RWKV7_V_X_K : sgm <= 3 ? RWKV7_V_X_V
       : sgm == 4 ? RWKV7_V_X_W : sgm == 5 ? RWKV7_V_X_A : RWKV7_V_X_G;
}

// LDS layout (floats). Each stage input has its own buffer, so the comm wave
// fills the next stage's input while the math waves read the current one.
struct MkLds {
  float *x1;      // [C]  P1 input x (and the head's input)
  float *ln1;     // [C]  LN1(x): the time-mix shift state written in P3
  float *mix;     // [4][C] P1 segment mixes; the head's normalised input
  float *p2;      // [192 + SR] P2 input: r, k, v of the head, activated LoRA1
  float *gsum;    // [5][64] LoRA second-step dots: v, w, a, g (two halves)
  float *core;    // [7][64] r w k a b y v of the head (P2)
  float *core_in; // [C]  P3 input
  float *x4;      // [C]  P4 input x'
  float *ln2;     // [C]  LN2(x'): the channel-mix shift state written in P5
  float *mix4;    // [C]  P4 mix
  float *hid;     // [F]  P5 input
  unsigned *pubs; // count of math-wave publish steps (the comm waves' start signal)
  unsigned *xflag; // tag of the x vector the comm wave's probe saw arriving (a start hint)
  unsigned *fail;  // a wave of this workgroup gave up a wait (see MkCtx)
  unsigned *ep;    // the launch epoch, read once by thread 0
  float *xst;     // [2][kW][2] (mean, M2) of each wave's slice of x (P1 input), x' (P4 input)
};

RWKV7_DEV_HOST_INLINE int64_t mk_lds_floats(int C, int F, int SR) {
  return (int64_t)10 * C + (192 + SR) + 5 * 64 + 7 * 64 + F + 8 + 4 * kW;
}

RWKV7_DEV MkLds mk_lds(float *smem, int C, int F, int SR) {
  MkLds s;
  s.x1 = smem;
  s.ln1 = s.x1 + C;
  s.mix = s.ln1 + C;
  s.core_in = s.mix + 4 * C;
  s.x4 = s.core_in + C;
  s.ln2 = s.x4 + C;
  s.mix4 = s.ln2 + C;
  s.hid = s.mix4 + C;
  s.p2 = s.hid + F;
  s.gsum = s.p2 + 192 + SR;
  s.core = s.gsum + 5 * 64;
  s.pubs = reinterpret_cast<unsigned *>(s.core + 7 * 64);
  s.xflag = s.pubs + 1;
  s.fail = s.pubs + 2;
  s.ep = s.pubs + 3;
  s.xst = s.core + 7 * 64 + 8;
  return s;
}

// ---- math-wave helpers --------------------------------------------------------

// acc + sum_e w[e] * x[e] for 8 16-bit weights (F16T<BF>) and 8 f32 inputs.
template <bool BF>
RWKV7_DEV float dot8r(const uint4 &w, const float (&x)[8], float acc) {
  float wf[8];
  F16T<BF>::to_f8(w, wf);
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = fmaf(wf[e], x[e], acc);
  return acc;
}

// Dot of one row held by the wave (lane l has chunks l + 64c) with x in LDS;
// the wave-uniform result. Every LDS read of the row is issued before the
// first FMA (a sched_barrier keeps the compiler from interleaving them, which
// would cost one LDS round trip per chunk); a chunk past the row (zero
// weights, see load_row) reads a valid x chunk instead. Two accumulators
// halve the dependent FMA chain.
template <bool BF, int NC>
RWKV7_DEV float row_dot(const uint4 (&w)[NC], const float *x, int nch) {
  const int lane = threadIdx.x & 63;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  float4 xa[NC], xb[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    int j = lane + 64 * c;
    j = j < nch ? j : nch - 1;
    xa[c] = x4[2 * j];
    xb[c] = x4[2 * j + 1];
  }
  sched_fence();
  float acc[2] = {0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    float wf[8];
    F16T<BF>::to_f8(w[c], wf);
    float a = acc[c & 1];
    a = fmaf(wf[0], xa[c].x, a); a = fmaf(wf[1], xa[c].y, a);
    a = fmaf(wf[2], xa[c].z, a); a = fmaf(wf[3], xa[c].w, a);
    a = fmaf(wf[4], xb[c].x, a); a = fmaf(wf[5], xb[c].y, a);
    a = fmaf(wf[6], xb[c].z, a); a = fmaf(wf[7], xb[c].w, a);
    acc[c & 1] = a;
  }
  return wave_sum(acc[0] + acc[1]);
}

// The same for an int8 row: lane l has chunks l + 64c of 16 weights, each
// dotted with 16 inputs; the row's scale is applied by the caller.
template <int NC>
RWKV7_DEV float row_dot_q8(const uint4 (&w)[NC], const float *x, int nch) {
  const int lane = threadIdx.x & 63;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  float4 xs[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    int j = lane + 64 * c;
    j = j < nch ? j : nch - 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) xs[c][q] = x4[4 * j + q];
  }
  sched_fence();
  float acc[2] = {0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const unsigned wd[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float a = acc[q & 1];
      a = fmaf((float)(int)(signed char)(wd[q] & 0xFF), xs[c][q].x, a);
      a = fmaf((float)(int)(signed char)((wd[q] >> 8) & 0xFF), xs[c][q].y, a);
      a = fmaf((float)(int)(signed char)((wd[q] >> 16) & 0xFF), xs[c][q].z, a);
      a = fmaf((float)(int)(signed char)(wd[q] >> 24), xs[c][q].w, a);
      acc[q & 1] = a;
    }
  }
  return wave_sum(acc[0] + acc[1]);
}

// acc + sum_e q[e] * x[e] for 16 int8 weights and 16 f32 inputs in registers.
RWKV7_DEV float dot16r_q8(const uint4 &w, const float (&x)[16], float acc) {
  const unsigned wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = fmaf((float)(int)(signed char)(wd[q] & 0xFF), x[4 * q], acc);
    acc = fmaf((float)(int)(signed char)((wd[q] >> 8) & 0xFF), x[4 * q + 1], acc);
    acc = fmaf((float)(int)(signed char)((wd[q] >> 16) & 0xFF), x[4 * q + 2], acc);
    acc = fmaf((float)(int)(signed char)(wd[q] >> 24), x[4 * q + 3], acc);
  }
  return acc;
}

// Loads row r of W (row stride ld halfs, nch 16-byte chunks) as lane chunks.
template <int NC>
RWKV7_DEV void load_row(const uint16_t *W, int64_t ld, int r, bool valid, int nch, uint4 (&w)[NC]) {
  const int lane = threadIdx.x & 63;
  const uint4 *row = reinterpret_cast<const uint4 *>(W + (int64_t)r * ld);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int j = lane + 64 * c;
    w[c] = (valid && j < nch) ? ld_stream(row + j) : make_uint4(0, 0, 0, 0);
  }
}

// ---- x hand-offs: every wave reads one slice ------------------------------------

// Mean and M2 (sum of squared deviations) of this wave's slice
// x[w*XS, (w+1)*XS) (XS <= 128: at most two values per lane), into st[0..1].
RWKV7_DEV void slice_stats(const float *x, int w, int XS, float *st) {
  const int lane = threadIdx.x & 63;
  const int i0 = lane, i1 = lane + 64;
  const float a = x[w * XS + (i0 < XS ? i0 : 0)], b = x[w * XS + (i1 < XS ? i1 : 0)];
  const float na = i0 < XS ? 1.f : 0.f, nb = i1 < XS ? 1.f : 0.f;
  const float mean = wave_sum(na * a + nb * b) / (float)XS;
  const float da = a - mean, db = b - mean;
  const float m2 = wave_sum(na * da * da + nb * db * db);
  if (lane == 0) {
    st[0] = mean;
    st[1] = m2;
  }
}

// LayerNorm mean and 1/std of a C-vector from its kW equal slices' (mean, M2)
// (pairwise-combination formula: M2 = sum M2_w + XS * sum (mean_w - mean)^2).
// st is 16-byte aligned: the kW pairs are read as kW / 2 float4 in one batch.
RWKV7_DEV float2 combine_stats(const float *st, int C, float inv_c) {
  const float XS = (float)(C / kW);
  float4 q[kW / 2];
#pragma unroll
  for (int i = 0; i < kW / 2; ++i) q[i] = reinterpret_cast<const float4 *>(st)[i];
  float mean = 0.f;
#pragma unroll
  for (int i = 0; i < kW / 2; ++i) mean += q[i].x + q[i].z;
  mean *= 1.f / kW;
  float m2 = 0.f;
#pragma unroll
  for (int i = 0; i < kW / 2; ++i) {
    const float d0 = q[i].x - mean, d1 = q[i].z - mean;
    m2 += (q[i].y + XS * d0 * d0) + (q[i].w + XS * d1 * d1);
  }
  return make_float2(mean, rsqrtf(m2 * inv_c + kLnEps));
}

// ---- comm wave ------------------------------------------------------------------

// ---- comm waves -----------------------------------------------------------------

// 16-byte device-scope (sc1) loads through a buffer resource: two tagged words
// per load, and reads past the end of the resource return zero.
RWKV7_DEV __amdgpu_buffer_rsrc_t words_rsrc(const uint64_t *p, int64_t nwords) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t *>(p), 0, (int)(nwords * 8), 0x00020000);
}
RWKV7_DEV uint4 ld_pair(__amdgpu_buffer_rsrc_t r, int word) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, word * 8, 0, /*sc1*/ 16);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Spins until the launch is aborted or the spin limit is hit (then aborts it).
struct SpinBound {
  const MkCtx &cx;
  int spins = 0;
  RWKV7_DEV explicit SpinBound(const MkCtx &c) : cx(c) {}
  // bounded: false once this workgroup gave up or the launch is aborted
  RWKV7_DEV bool keep_waiting() {
    ++spins;
    if (cx.failed()) return false;
    if ((spins & 1023) == 0 && cx.aborted()) {
      cx.give_up();
      return false;
    }
    if (spins > kSpinLimit) {
      cx.abort();
      return false;
    }
    return true;
  }
};

// Probe phase: polls one pair in every `probe` words (lane l of wave cw takes
// stride 64 cw + l) until those carry the tag.
template <typename Idx>
RWKV7_DEV void probe_wait(const MkCtx &cx, int cw, __amdgpu_buffer_rsrc_t r, int n, int probe, unsigned tag,
                          Idx idx) {
  SpinBound sb(cx);
  const int p0 = 64 * cw + (threadIdx.x & 63);
  const int nq = (n + probe - 1) / probe;
  // the probed word of each stride, shifted per workgroup so that the
  // readers of one replica do not all poll the same few lines
  int pq = probe * p0 + cx.pskew % probe;
  pq = pq < n ? pq : probe * p0;
  bool waiting = p0 < nq;
  while (waiting) {
    asm volatile("" ::: "memory");  // re-read every round
    const uint4 v = ld_pair(r, idx(pq));
    if (v.y == tag) waiting = false;
    else if (!sb.keep_waiting()) break;
    else __builtin_amdgcn_s_sleep(1);  // only while some lane still waits
  }
}

// Reads until every word idx(i), i < n, of the buffer `r` carries `tag`,
// handing each value to put(i, v). idx must map each even i and i + 1 to
// consecutive, 16-byte aligned words; lane l of wave cw handles the pairs
// p = 64 cw + l + 64 kNComm j (j < NJ), i = 2p. A round is one 16-byte load per
// pair; D rounds stay in flight (re-issued unconditionally, so the compiler's
// load counting stays exact), checked oldest first, at most 16 loads per lane.
// Poll traffic slows every hand-off on the chip, so callers start this only
// after a sparse probe (probe_wait, here or in the workgroup's comm wave, which
// then raises an LDS flag) and use D = 1.
template <int NJ, int D, typename Idx, typename Put>
RWKV7_DEV void read_all(const MkCtx &cx, int cw, __amdgpu_buffer_rsrc_t r, int n, unsigned tag, Idx idx, Put put) {
  static_assert(NJ * D <= 16 && NJ <= 16, "at most 16 loads per lane in flight");
  SpinBound sb(cx);
  int p0 = 64 * cw + (threadIdx.x & 63);
  asm volatile("" : "+v"(p0));  // per-call addresses: keep them out of the layer loop
  constexpr int kStep = 64 * kNComm;
  const int np = n >> 1;
  unsigned pending = 0;
  int addr[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int p = p0 + kStep * j;
    if (p < np) pending |= 1u << j;
    addr[j] = idx(p < np ? 2 * p : 0);
  }
  uint4 buf[D][NJ];
#pragma unroll
  for (int d = 0; d < D; ++d)
#pragma unroll
    for (int j = 0; j < NJ; ++j) buf[d][j] = ld_pair(r, addr[j]);
  // Straight-line body: every buffer is checked and re-issued each pass, so at
  // each check exactly (D - 1) * NJ younger loads are in flight.
  while (true) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (((pending >> j) & 1) && buf[d][j].y == tag && buf[d][j].w == tag) {
          const int i = 2 * (p0 + kStep * j);
          put(i, __builtin_bit_cast(float, buf[d][j].x));
          put(i + 1, __builtin_bit_cast(float, buf[d][j].z));
          pending &= ~(1u << j);
        }
      }
      asm volatile("" ::: "memory");  // re-read every round
#pragma unroll
      for (int j = 0; j < NJ; ++j) buf[d][j] = ld_pair(r, addr[j]);
    }
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0 || !sb.keep_waiting()) break;
  }
}

// Waits (LDS spin, bounded) until *flag == tag. Only a start hint: the reads
// that follow check every word's tag themselves.
RWKV7_DEV void wait_flag(const MkCtx &cx, const unsigned *flag, unsigned tag) {
  SpinBound sb(cx);
  while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != tag) {
    __builtin_amdgcn_s_sleep(1);
    if (!sb.keep_waiting()) break;
  }
}

struct Ident {
  RWKV7_DEV int operator()(int i) const { return i; }
};

// Waits (LDS spin, bounded by the launch's abort word) until the math waves
// of this workgroup have completed `target` publish steps.
RWKV7_DEV void wait_local(const MkCtx &cx, const unsigned *pubs, unsigned target) {
  SpinBound sb(cx);
  while (__hip_atomic_load(pubs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
    __builtin_amdgcn_s_sleep(1);
    if (!sb.keep_waiting()) break;
  }
}

// Workgroup roles. Workgroups 0..H-1 (head workgroups) run only the
// per-head core P2 of head g; the others (workers) run P1, P3, P4, P5 and the
// logits, each stage's rows split evenly over the workers. A head workgroup
// thus streams only its own head's operands (LoRA second-step rows, wkv state)
// and nothing delays its hand-offs, which sit on the critical path.
//
// Barrier schedules (one line per workgroup barrier; the comm and math waves
// of a workgroup execute the same sequence):
//   head, per layer:    HA  P2 input in p2
//                       B2b gates in core (each LoRA part's wave finishes its gate)
//                       B2c wkv outputs in core
//   worker, per layer:  A1  P1 input in x1
//                       B1  P1 mixes in mix
//                       A3  P3 input in core_in
//                       A4  P4 input in x4
//                       B4  P4 mix in mix4
//                       A5  P5 input in hid
//   worker, after:      AH  head input in x1
//                       BH  normalised head input in mix
// Worker math waves count their publish steps in s.pubs (kMW per P1, P3, P4,
// P5); the comm wave starts reading a vector the workers produce only after
// its own workgroup's share is out.

// NJF: pairs per lane of one of the kW slices of the FFN hidden vector (every
// wave of the workgroup reads one slice).
template <int NJF, bool BF>
RWKV7_DEV void comm_worker(const MkArgs &a, const MkGeom &m, const MkLds &s, const MkCtx &cx) {
  const int lane = threadIdx.x & 63;
  const int C = m.C, F = m.F, L = m.L;
  int64_t token = a.tok[0];
  token = token < 0 ? 0 : token >= a.V ? a.V - 1 : token;
  const uint16_t *erow = a.emb + token * C;
  // this wave's slice of x (the math waves load and read the others); its
  // LayerNorm partial statistics go to xst
  static_assert(kNComm == 1, "the comm wave holds slice kMW");
  const int XS = C / kW;
  for (int i = lane; i < XS; i += 64) s.x1[kMW * XS + i] = F16T<BF>::to_f(erow[kMW * XS + i]);
  slice_stats(s.x1, kMW, XS, s.xst + 2 * kMW);
  auto to = [](float *d) { return [d](int i, float v) { d[i] = v; }; };
  const int rp = m.g % kRep;  // the replica this workgroup reads
  const __amdgpu_buffer_rsrc_t r_xall = words_rsrc(a.x_ex + (int64_t)rp * C, C);
  const __amdgpu_buffer_rsrc_t r_x = words_rsrc(a.x_ex + (int64_t)rp * C + kMW * XS, XS);
  // x hand-offs: this wave probes the whole vector, tells the math waves (each
  // reads one slice) through xflag, then reads slice kMW
  auto poll_x = [&](unsigned tag, float *x, float *st) {
    probe_wait(cx, 0, r_xall, C, kXProbe, tag, Ident());
    if (lane == 0) __hip_atomic_store(s.xflag, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    read_all<1, 1>(cx, 0, r_x, XS, tag, Ident(), to(x + kMW * XS));
    slice_stats(x, kMW, XS, st + 2 * kMW);
  };
  const __amdgpu_buffer_rsrc_t r_core = words_rsrc(a.core_ex + (int64_t)rp * C, C);
  const __amdgpu_buffer_rsrc_t r_cs = words_rsrc(a.core_ex + (int64_t)rp * C + kMW * (C / kW), C / kW);
  const int FS = F / kW;  // words of one hidden-vector slice
  const __amdgpu_buffer_rsrc_t r_hid = words_rsrc(a.hid_ex + (int64_t)rp * F + (int64_t)kMW * FS, FS);
  const __amdgpu_buffer_rsrc_t r_hidall = words_rsrc(a.hid_ex + (int64_t)rp * F, F);
  unsigned pubs = 0;  // publish steps of the math waves seen so far
  for (int l = 0; l < L; ++l) {
    const int ph = 5 * l;
    __syncthreads();  // A1
    __syncthreads();  // B1
    pubs += kMW;
    // the head workgroups' outputs: one probe pair per head first
    probe_wait(cx, 0, r_core, C, 16 * kN, cx.tag(ph + 1), Ident());
    if (lane == 0) __hip_atomic_store(s.xflag, cx.tag(ph + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    read_all<1, 1>(cx, 0, r_cs, XS, cx.tag(ph + 1), Ident(), to(s.core_in + kMW * XS));
    __syncthreads();  // A3
    pubs += kMW;
    wait_local(cx, s.pubs, pubs);
    poll_x(cx.tag(ph + 2), s.x4, s.xst + 2 * kW);
    __syncthreads();  // A4
    __syncthreads();  // B4
    pubs += kMW;
    wait_local(cx, s.pubs, pubs);
    // the last slice of the hidden vector (the math waves read the others)
    probe_wait(cx, 0, r_hidall, F, kHidProbe, cx.tag(ph + 3), Ident());
    if (lane == 0) __hip_atomic_store(s.xflag, cx.tag(ph + 3), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    read_all<NJF, 1>(cx, 0, r_hid, FS, cx.tag(ph + 3), Ident(), to(s.hid + kMW * FS));
    __syncthreads();  // A5
    pubs += kMW;
    wait_local(cx, s.pubs, pubs);
    poll_x(cx.tag(ph + 4), s.x1, s.xst);
  }
  __syncthreads();  // AH
  __syncthreads();  // BH
}

// Word of P2 input element i of head h in a proj replica: r, k, v of the head
// (i < 192), then the whole LoRA first step.
struct HeadWord {
  int C, h;
  RWKV7_DEV int operator()(int i) const { return i < 192 ? (i >> 6) * C + h * kN + (i & 63) : 3 * C + (i - 192); }
};
RWKV7_DEV HeadWord head_word(int C, int h) { return HeadWord{C, h}; }

// Wave w's slice of the P2 input (every wave of a head workgroup reads one),
// activated on arrival: tanh for the w LoRA, sigmoid for the g LoRA.
RWKV7_DEV void head_read(const MkCtx &cx, const MkArgs &a, const MkLds &s, int h, int w, unsigned tag) {
  const int C = a.C, n = 192 + a.rv + a.rw + a.ra + a.rg;
  const int rv = a.rv, rwa = a.rv + a.rw, rwaa = a.rv + a.rw + a.ra;
  const int S = ((n + kW - 1) / kW + 1) & ~1;  // even slice length
  const int i0 = w * S, m = n - i0 < S ? n - i0 : S;
  if (m <= 0) return;
  const __amdgpu_buffer_rsrc_t r = words_rsrc(a.proj_ex + (int64_t)(h % kRep) * (3 * C + n - 192), 3 * C + n - 192);
  const HeadWord hw = head_word(C, h);
  read_all<1, 1>(cx, 0, r, m, tag, [&](int li) { return hw(i0 + li); },
                 [&](int li, float v) {
                   const int j = i0 + li - 192;
                   if (j >= rv && j < rwa) v = tanhf(v);
                   else if (j >= rwaa) v = sigmoidf_(v);
                   s.p2[i0 + li] = v;
                 });
}

RWKV7_DEV void comm_head(const MkArgs &a, const MkGeom &m, const MkLds &s, const MkCtx &cx) {
  const int C = m.C, SR = m.SR, L = m.L;
  const int h = m.g;
  const __amdgpu_buffer_rsrc_t r_proj = words_rsrc(a.proj_ex + (int64_t)(h % kRep) * (3 * C + SR), 3 * C + SR);
  for (int l = 0; l < L; ++l) {
    // r, k, v of this head and the whole LoRA first step: a sparse probe
    // (this poll starts a whole layer before its data), then every wave reads
    // one slice (see head_read)
    probe_wait(cx, 0, r_proj, 192 + SR, 512, cx.tag(5 * l), head_word(C, h));
    if ((threadIdx.x & 63) == 0)
      __hip_atomic_store(s.xflag, cx.tag(5 * l), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    head_read(cx, a, s, h, kMW, cx.tag(5 * l));
    __syncthreads();  // HA
    __syncthreads();  // B2b
    __syncthreads();  // B2c
  }
}

// ---- math waves -----------------------------------------------------------------

// Per-head core of head g for every layer: LoRA second step, gates, L2 norm,
// wkv7, GroupNorm, output gate (demo/rwkv7_torch.py:92-120). NL2: LoRA
// second-step chunks per thread.
template <int NL2, bool BF>
RWKV7_DEV void math_head(const MkArgs &a, const MkGeom &m, const MkLds &s, const MkCtx &cx, int wv) {
  int mt = threadIdx.x, lane = mt & 63;
  auto refresh = [&]() {
    asm volatile("" : "+v"(mt));
    lane = mt & 63;
  };
  const int C = m.C, H = m.H, SR = m.SR, L = m.L, g = m.g;
  const int nch2 = SR >> 3;
  // LoRA second step: wave q < 5 computes part q (v, w, a, first and second
  // half of g) for channel lane; part q covers chunks [p2s(q), p2s(q + 1)) of
  // the channel's [v|w|a|g] row
  const int b1 = a.rv >> 3, b2 = (a.rv + a.rw) >> 3, b3 = (a.rv + a.rw + a.ra) >> 3;
  const int b4 = b3 + (nch2 - b3 + 1) / 2;
  auto p2s = [&](int q) { return q == 0 ? 0 : q == 1 ? b1 : q == 2 ? b2 : q == 3 ? b3 : q == 4 ? b4 : nch2; };
  // this wave's LoRA second-step part (waves 0..4), fixed for the launch
  const int js = wv < 5 ? p2s(wv) : 0, je = wv < 5 ? p2s(wv + 1) : 0;
  uint4 w2[NL2];
  float4 S4[4];
  float gv[8];
  auto pre_p2 = [&](int l) {
    const char *Lp = a.layers + (int64_t)l * a.lbytes;
    if (wv < 5) {
      const uint4 *row = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(Lp + a.o_l2) +
                                                         (int64_t)(g * kN + lane) * SR);
      if (je > js) {
#pragma unroll
        for (int i = 0; i < NL2; ++i) w2[i] = ld_stream(row + (js + i < je ? js + i : je - 1));
      }
    }
    if (mt < 4 * kN) {
      const float4 *Sp = reinterpret_cast<const float4 *>(a.rnn + (((int64_t)l * H + g) * kN + (mt >> 2)) * kN) +
                         (mt & 3) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) S4[e] = Sp[e];
    }
    if (wv < 3) {  // the gate vectors (waves 0..2 finish the v, w and a parts)
      const float *vec = reinterpret_cast<const float *>(Lp + a.o_vec);
      const int idx[8] = {RWKV7_V_V0, RWKV7_V_W0, RWKV7_V_A0, RWKV7_V_K_K,
                          RWKV7_V_K_A, RWKV7_V_R_K, RWKV7_V_LNX_W, RWKV7_V_LNX_B};
#pragma unroll
      for (int j = 0; j < 8; ++j) gv[j] = vec[idx[j] * C + g * kN + lane];
    }
    sched_fence();
  };
  float vfirst = 0.f;  // v of layer 0 for channel g*64 + lane (wave 0)
  float *s_r = s.core, *s_w = s.core + 64, *s_k = s.core + 128, *s_a = s.core + 192, *s_b = s.core + 256,
        *s_y = s.core + 320;
  pre_p2(0);
  for (int l = 0; l < L; ++l) {
    wait_flag(cx, s.xflag, cx.tag(5 * l));  // the comm wave's probe saw the P2 input arriving
    head_read(cx, a, s, g, wv, cx.tag(5 * l));
    __syncthreads();  // HA
    RWKV7_TL(tl_decode, l, 8);
    wait_vm0();       // this layer's operands (issued a layer ago)
    refresh();
    if (wv < 5) {  // LoRA second step, part wv of channel lane
      // every LDS read issued before the first FMA; a chunk past the part
      // gets zero weights and reads the part's first chunk
      const float4 *x4 = reinterpret_cast<const float4 *>(s.p2 + 192);
      float4 xa[NL2], xb[NL2];
#pragma unroll
      for (int i = 0; i < NL2; ++i) {
        const int c = js + i < je ? js + i : js;
        xa[i] = x4[2 * c];
        xb[i] = x4[2 * c + 1];
      }
      sched_fence();
      float acc[2] = {0.f, 0.f};
#pragma unroll
      for (int i = 0; i < NL2; ++i) {
        float wf[8];
        F16T<BF>::to_f8(js + i < je ? w2[i] : make_uint4(0, 0, 0, 0), wf);
        float t = acc[i & 1];
        t = fmaf(wf[0], xa[i].x, t); t = fmaf(wf[1], xa[i].y, t);
        t = fmaf(wf[2], xa[i].z, t); t = fmaf(wf[3], xa[i].w, t);
        t = fmaf(wf[4], xb[i].x, t); t = fmaf(wf[5], xb[i].y, t);
        t = fmaf(wf[6], xb[i].z, t); t = fmaf(wf[7], xb[i].w, t);
        acc[i & 1] = t;
      }
      const float d = acc[0] + acc[1];
      // each part's wave finishes its own gates for channel t = lane
      const int t = lane;
      if (wv == 0) {  // v, mixed with layer 0's v
        float v = s.p2[128 + t];
        if (l == 0) vfirst = v;
        else v = v + sigmoidf_(gv[0] + d) * (vfirst - v);
        s.core[384 + t] = v;
        s_r[t] = s.p2[t];
      } else if (wv == 1) {  // decay
        s_w[t] = expf(-sigmoidf_(gv[1] + d) / 1.6487212707001282f);
      } else if (wv == 2) {  // a, the normalised key kk and the key with its a-mix
        const float r = s.p2[t], k = s.p2[64 + t];
        const float ag = sigmoidf_(gv[2] + d);
        const float kk = k * gv[3];
        const float kn = k + gv[4] * (k * ag - k);
        // kk / max(|kk|, 1e-12) = kk * rsqrt(max(|kk|^2, 1e-24)); both sums in lockstep
        const float2 sums = wave_sum2(kk * kk, r * kn * gv[5]);
        const float kh = kk * rsqrtf(fmaxf(sums.x, 1e-24f));
        const float rk = sums.y;
        s_k[t] = kn; s_a[t] = kh; s_b[t] = -kh * ag;
        if (t == 0) s.gsum[0] = rk;
      } else {  // the two halves of the output gate's dot
        s.gsum[wv * kN + t] = d;
      }
    }
    __syncthreads();  // B2b
    // wkv7: 4 threads per state row, 16 columns each; the new state is written
    // back only after the core output is published (wave 0 publishes first)
    const int row = mt >> 2, j0 = (mt & 3) * 16;
    float Sv[16];
    if (mt < 4 * kN) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        Sv[4 * e] = S4[e].x; Sv[4 * e + 1] = S4[e].y; Sv[4 * e + 2] = S4[e].z; Sv[4 * e + 3] = S4[e].w;
      }
      float av[16], wv16[16], bv[16], kv[16], rv16[16];
      auto ld16 = [&](float (&d)[16], const float *src) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float4 q = reinterpret_cast<const float4 *>(src + j0)[e];
          d[4 * e] = q.x; d[4 * e + 1] = q.y; d[4 * e + 2] = q.z; d[4 * e + 3] = q.w;
        }
      };
      ld16(av, s_a);
      ld16(wv16, s_w);
      ld16(bv, s_b);
      ld16(kv, s_k);
      ld16(rv16, s_r);
      const float vi = s.core[384 + row];
      float sa = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) sa = fmaf(Sv[e], av[e], sa);
      sa = sum4(sa);
      float y = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        Sv[e] = Sv[e] * wv16[e] + sa * bv[e] + vi * kv[e];
        y = fmaf(Sv[e], rv16[e], y);
      }
      y = sum4(y);
      if ((mt & 3) == 0) s_y[row] = y;
      // GroupNorm partials of this wave's 16 rows (each row's y is in 4 lanes)
      const float m16 = wave_sum(y) * (1.f / (4 * 16));
      const float dy = y - m16;
      const float m2 = wave_sum(dy * dy) * 0.25f;
      if (lane == 0) {
        s.gsum[8 + 2 * wv] = m16;
        s.gsum[9 + 2 * wv] = m2;
      }
    }
    __syncthreads();  // B2c
    // inputs of this layer arrived (a wave that gave up set fail before HA)
    const bool ok = !cx.failed();
    if (wv == 0 && ok) {
      // GroupNorm of the head from the 4 waves' (mean, M2) over 16 rows each
      float mean = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) mean += s.gsum[8 + 2 * w];
      mean *= 0.25f;
      float m2 = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float dm = s.gsum[8 + 2 * w] - mean;
        m2 += s.gsum[9 + 2 * w] + 16.f * dm * dm;
      }
      const float y = s_y[lane];
      const float v = s.core[384 + lane], rk = s.gsum[0];
      const float gate = s.gsum[3 * kN + lane] + s.gsum[4 * kN + lane];
      const float yn = (y - mean) * rsqrtf(m2 * (1.f / kN) + kGnEps) * gv[6] + gv[7];
      const float out = (yn + rk * v) * gate;
#pragma unroll
      for (int rp = 0; rp < kRep; ++rp) publish(a.core_ex + (int64_t)rp * C + g * kN + lane, cx.tag(5 * l + 1), out);
      RWKV7_TL(tl_decode, l, 9);
    }
    if (mt < 4 * kN && ok) {
      float4 *Sp = reinterpret_cast<float4 *>(a.rnn + (((int64_t)l * H + g) * kN + row) * kN + j0);
#pragma unroll
      for (int e = 0; e < 4; ++e) Sp[e] = make_float4(Sv[4 * e], Sv[4 * e + 1], Sv[4 * e + 2], Sv[4 * e + 3]);
    }
    // next layer's operands: a whole layer to arrive
    refresh();
    if (l + 1 < L) pre_p2(l + 1);
  }
}

// P1, P3, P4, P5 and the logits on the worker workgroups. CPL: 16-byte chunks
// per lane of a C-long row; RM: P1/P4 rows per math wave; NC5: chunks per lane
// of an F-long row; VPL: elements per math thread of a C-vector; NHB: head
// batches.
//
// Weight schedule: right after publishing P1, a worker issues every load of
// the rest of the layer (P3, P4, P5 rows and vectors, next layer's P1 rows and
// vectors). They stream while the head workgroups run P2 (the layer's longest
// wait), and a single vmcnt(0) at the start of P3 covers them all, so the
// later hand-offs of the layer run with no weight traffic in flight.
template <int CPL, int RM, int NC5, int VPL, int NHB, bool Q8, bool BF>
RWKV7_DEV void math_worker(const MkArgs &a, const MkGeom &m, const MkLds &s, const MkCtx &cx, int wv) {
  // Math threads are 0..kMT-1. refresh() passes the thread index through an
  // empty asm at each stage, so per-thread addresses are recomputed there
  // instead of being hoisted out of the layer loop into ~100 live registers.
  int mt = threadIdx.x, lane = mt & 63;
  auto refresh = [&]() {
    asm volatile("" : "+v"(mt));
    lane = mt & 63;
  };
  const int C = m.C, F = m.F, L = m.L;
  const int nchC = C >> 3, nchF = F >> 3;
  // Weight rows: f16 (8 per 16-byte chunk) or int8 (16 per chunk, with an
  // f32 scale per row). CW / N5: chunks per lane of a C-long / F-long row;
  // wchC / wchF: chunks of a row; wld: row stride of a C-long row in halfs.
  constexpr int CW = Q8 ? (CPL + 1) / 2 : CPL;
  constexpr int N5 = Q8 ? (NC5 + 1) / 2 : NC5;
  const int wchC = Q8 ? C >> 4 : nchC, wchF = Q8 ? F >> 4 : nchF;
  const int wldC = Q8 ? C >> 1 : C, wldF = Q8 ? F >> 1 : F;

  uint4 w1[RM][CW];
  float v1w[VPL], v1b[VPL], mu1[4][VPL];
  uint16_t pv1[VPL];
  uint4 w3[CW];
  uint4 w4[RM][CW];
  float v4w[VPL], v4b[VPL], mu4[VPL];
  uint16_t pv4[VPL];
  uint4 w5[N5];
  uint4 wh[kHRing][kHB][CW];
  float hlw[VPL], hlb[VPL];
  float q1s[RM], q3s = 1.f, q4s[RM], q5s = 1.f;  // int8 row scales
  float hqs[kHRing][kHB];

  auto layer_ptr = [&](int l) { return a.layers + (int64_t)l * a.lbytes; };
  auto qlayer = [&](int l) { return a.layers_q + (int64_t)l * a.q_lbytes; };
  // the matrix rows a stage streams, and their scales (int8) in the order of
  // the layout's scale section: P1 rows, o rows, FFN key rows, FFN value rows
  auto wbase = [&](int l, int64_t o16, int64_t o8) {
    return reinterpret_cast<const uint16_t *>(Q8 ? qlayer(l) + o8 : layer_ptr(l) + o16);
  };
  auto qscale = [&](int l, int row) { return reinterpret_cast<const float *>(qlayer(l) + a.q_scale)[row]; };
  const int N1 = 3 * C + m.SR;
  // a row's dot product, scale included
  auto rdot = [&](const auto &w, const float *x, int nch, float sc) {
    if constexpr (Q8) return row_dot_q8(w, x, nch) * sc;
    else return row_dot<BF>(w, x, nch);
  };
  auto vec_ptr = [&](int l) { return reinterpret_cast<const float *>(layer_ptr(l) + a.o_vec); };
  // Vector loads are unconditional (index clamped; elements past C are never
  // used): a load under a branch makes the compiler wait for it inside the
  // branch (converting it there, or at the join), which stalls the prefetch
  // behind every load issued before it.
  auto ld_vec = [&](float (&d)[VPL], const float *src) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = mt + kMT * i;
      d[i] = src[c < C ? c : C - 1];
    }
  };
  auto ld_vec16 = [&](uint16_t (&d)[VPL], const uint16_t *src) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = mt + kMT * i;
      d[i] = src[c < C ? c : C - 1];
    }
  };
  auto pre_p1 = [&](int l) {
    const uint16_t *W = wbase(l, a.o_rkv, a.q_rkv);
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      const int r = m.p1a + wv + kMW * i;
      load_row<CW>(W, wldC, r, r < m.p1b, wchC, w1[i]);
      if constexpr (Q8) q1s[i] = qscale(l, r < N1 ? r : N1 - 1);
    }
    const float *vec = vec_ptr(l);
    ld_vec(v1w, vec + RWKV7_V_LN1_W * C);
    ld_vec(v1b, vec + RWKV7_V_LN1_B * C);
    ld_vec16(pv1, a.tmix_x + (int64_t)l * C);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (q < m.nseg) ld_vec(mu1[q], vec + (int64_t)seg_mu(m.seg0 + q) * C);
    sched_fence();
  };
  auto pre_p3 = [&](int l) {
    const uint16_t *W = wbase(l, a.o_o, a.q_o);
    load_row<CW>(W, wldC, m.owa + wv, wv < m.nown, wchC, w3);
    if constexpr (Q8) q3s = qscale(l, N1 + (m.owa + wv < C ? m.owa + wv : C - 1));
    sched_fence();
  };
  auto pre_p4 = [&](int l) {
    const uint16_t *W = wbase(l, a.o_fk, a.q_fk);
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      const int r = m.p4a + wv + kMW * i;
      load_row<CW>(W, wldC, r, r < m.p4b, wchC, w4[i]);
      if constexpr (Q8) q4s[i] = qscale(l, N1 + C + (r < F ? r : F - 1));
    }
    const float *vec = vec_ptr(l);
    ld_vec(v4w, vec + RWKV7_V_LN2_W * C);
    ld_vec(v4b, vec + RWKV7_V_LN2_B * C);
    ld_vec(mu4, vec + RWKV7_V_FFN_X_K * C);
    ld_vec16(pv4, a.cmix_x + (int64_t)l * C);
    sched_fence();
  };
  auto pre_p5 = [&](int l) {
    const uint16_t *W = wbase(l, a.o_fv, a.q_fv);
    load_row<N5>(W, wldF, m.owa + wv, wv < m.nown, wchF, w5);
    if constexpr (Q8) q5s = qscale(l, N1 + C + F + (m.owa + wv < C ? m.owa + wv : C - 1));
    sched_fence();
  };
  // head rows of this wave: a contiguous range, kHB rows per batch
  const int hr0 = m.ha + (int)((int64_t)(m.hb - m.ha) * wv / kMW);
  const int hr1 = m.ha + (int)((int64_t)(m.hb - m.ha) * (wv + 1) / kMW);
  // Head loads are unconditional (rows and chunks clamped into range, unused
  // lanes later multiply by a zero input) so that the unrolled head loop issues
  // a fixed number of loads and the compiler's load counting stays exact.
  auto pre_head = [&](int b, uint4 (&dst)[kHB][CW]) {
#pragma unroll
    for (int k = 0; k < kHB; ++k) {
      int r = hr0 + kHB * b + k;
      r = r < m.hb ? r : m.hb - 1;
      const uint4 *row = reinterpret_cast<const uint4 *>((Q8 ? a.head_q : a.head) + (int64_t)r * wldC);
      if constexpr (Q8) hqs[b % kHRing][k] = a.head_qs[r];
#pragma unroll
      for (int c = 0; c < CW; ++c) {
        const int j = lane + 64 * c;
        dst[k][c] = ld_stream(row + (j < wchC ? j : wchC - 1));
      }
    }
    sched_fence();
  };
  auto count_publish = [&]() {  // this wave's publishes of the stage are issued
    if (lane == 0) __hip_atomic_fetch_add(s.pubs, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };

  float xown = 0.f;  // residual of channel owa + wv (waves wv < nown)
  const float inv_c = 1.f / (float)C;
  // materialises values loaded above (one wait for the whole batch) so the
  // compiler does not sink the loads into the conditional code that uses them
  auto keep_v = [](float (&v)[VPL]) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) asm volatile("" ::"v"(v[i]));
  };
  // x hand-offs: this wave reads slice wv of x (the comm wave slice kMW) and
  // leaves the slice's LayerNorm partial statistics in xst
  const int XS = C / kW;
  const __amdgpu_buffer_rsrc_t r_xs = words_rsrc(a.x_ex + (int64_t)(m.g % kRep) * C + wv * XS, XS);
  const __amdgpu_buffer_rsrc_t r_cso = words_rsrc(a.core_ex + (int64_t)(m.g % kRep) * C + wv * XS, XS);
  auto poll_x = [&](unsigned tag, float *x, float *st) {
    wait_flag(cx, s.xflag, tag);  // the comm wave's probe saw the vector arriving
    read_all<1, 1>(cx, 0, r_xs, XS, tag, Ident(), [&](int i, float v) { x[wv * XS + i] = v; });
    slice_stats(x, wv, XS, st + 2 * wv);
  };
  {
    int64_t token = a.tok[0];
    token = token < 0 ? 0 : token >= a.V ? a.V - 1 : token;
    const uint16_t *erow = a.emb + token * C;
    for (int i = lane; i < XS; i += 64) s.x1[wv * XS + i] = F16T<BF>::to_f(erow[wv * XS + i]);
    slice_stats(s.x1, wv, XS, s.xst + 2 * wv);
  }
  pre_p1(0);
  wait_vm0();
  for (int l = 0; l < L; ++l) {
    const int ph = 5 * l;
    // ---------------- P1: LN1 + shift + [r;k;v;LoRA1] ------------------------
    __syncthreads();  // A1
    RWKV7_TL(tl_decode, l, 0);
    refresh();
    {
      const float2 st = combine_stats(s.xst, C, inv_c);
      float xv[VPL];  // read up front (index clamped), not one LDS round trip per element
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = mt + kMT * i;
        xv[i] = s.x1[c < C ? c : C - 1];
      }
      keep_v(xv);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = mt + kMT * i;
        if (c < C) {
          const float ln = (xv[i] - st.x) * st.y * v1w[i] + v1b[i];
          const float prv = F16T<BF>::to_f(pv1[i]);
          s.ln1[c] = ln;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (q < m.nseg) s.mix[q * C + c] = ln + mu1[q][i] * (prv - ln);
        }
      }
      if (l == 0 && wv < m.nown) xown = s.x1[m.owa + wv];
    }
    __syncthreads();  // B1
    {
      const bool ok = !cx.failed();
      const unsigned tg = cx.tag(ph);
#pragma unroll
      for (int i = 0; i < RM; ++i) {
        const int r = m.p1a + wv + kMW * i;
        if (r < m.p1b) {
          const float d = rdot(w1[i], s.mix + (m.seg_of(r) - m.seg0) * C, wchC, Q8 ? q1s[i] : 1.f);
          if (lane < kRep && ok) publish(a.proj_ex + (int64_t)lane * (3 * C + m.SR) + r, tg, d);
        }
      }
    }
    count_publish();
    RWKV7_TL(tl_decode, l, 1);
    // every load of the rest of the layer, issued while the head workgroups wait
    // for their input (that hand-off is slow anyway) and compute
    refresh();
    pre_p3(l);
    pre_p4(l);
    pre_p5(l);
    if (l + 1 < L) pre_p1(l + 1);
    wait_flag(cx, s.xflag, cx.tag(ph + 1));
    read_all<1, 1>(cx, 0, r_cso, XS, cx.tag(ph + 1), Ident(), [&](int i, float v) { s.core_in[wv * XS + i] = v; });
    __syncthreads();  // A3
    RWKV7_TL(tl_decode, l, 2);
    wait_vm0();
    // ---------------- P3: o-projection + residual -----------------------------
    refresh();
    if (wv < m.nown && !cx.failed()) {
      const float d = rdot(w3, s.core_in, wchC, q3s);
      xown += d;
      const int c = m.owa + wv;
      if (lane < kRep) publish(a.x_ex + (int64_t)lane * C + c, cx.tag(ph + 2), xown);
      // every reader of this layer's time-mix shift state is done (all of P2's inputs arrived)
      if (lane == kRep) a.tmix_x[(int64_t)l * C + c] = F16T<BF>::from_f(s.ln1[c]);
    }
    count_publish();
    RWKV7_TL(tl_decode, l, 3);
    poll_x(cx.tag(ph + 2), s.x4, s.xst + 2 * kW);
    __syncthreads();  // A4
    RWKV7_TL(tl_decode, l, 4);
    // ---------------- P4: LN2 + shift + FFN key + relu^2 ----------------------
    refresh();
    {
      const float2 st = combine_stats(s.xst + 2 * kW, C, inv_c);
      float xv[VPL];
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = mt + kMT * i;
        xv[i] = s.x4[c < C ? c : C - 1];
      }
      keep_v(xv);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = mt + kMT * i;
        if (c < C) {
          const float ln = (xv[i] - st.x) * st.y * v4w[i] + v4b[i];
          s.ln2[c] = ln;
          s.mix4[c] = ln + mu4[i] * (F16T<BF>::to_f(pv4[i]) - ln);
        }
      }
    }
    __syncthreads();  // B4
    {
      const bool ok = !cx.failed();
      const unsigned tg = cx.tag(ph + 3);
#pragma unroll
      for (int i = 0; i < RM; ++i) {
        const int r = m.p4a + wv + kMW * i;
        if (r < m.p4b) {
          const float q = fmaxf(rdot(w4[i], s.mix4, wchC, Q8 ? q4s[i] : 1.f), 0.f);
          if (lane < kRep && ok) publish(a.hid_ex + (int64_t)lane * F + r, tg, q * q);
        }
      }
    }
    count_publish();
    RWKV7_TL(tl_decode, l, 5);
    {
      // every wave reads one slice of the hidden vector (the math waves are
      // idle until it is complete, and 8 readers cut its round trips)
      const int FS = F / kW;
      const __amdgpu_buffer_rsrc_t r = words_rsrc(a.hid_ex + (int64_t)(m.g % kRep) * F + (int64_t)wv * FS, FS);
      wait_flag(cx, s.xflag, cx.tag(ph + 3));  // the comm wave's probe saw it arriving
      read_all<NC5 / 2, 1>(cx, 0, r, FS, cx.tag(ph + 3), Ident(),
                            [&](int i, float v) { s.hid[wv * FS + i] = v; });
    }
    __syncthreads();  // A5
    RWKV7_TL(tl_decode, l, 6);
    // ---------------- P5: FFN value + residual --------------------------------
    refresh();
    if (wv < m.nown && !cx.failed()) {
      const float d = rdot(w5, s.hid, wchF, q5s);
      xown += d;
      const int c = m.owa + wv;
      if (lane < kRep) publish(a.x_ex + (int64_t)lane * C + c, cx.tag(ph + 4), xown);
      if (lane == kRep) a.cmix_x[(int64_t)l * C + c] = F16T<BF>::from_f(s.ln2[c]);
    }
    count_publish();
    RWKV7_TL(tl_decode, l, 7);
    poll_x(cx.tag(ph + 4), s.x1, s.xst);
  }

  // ---------------- head: ln_out + logits ---------------------------------------
  refresh();
  const bool glob_abort = cx.aborted();  // issued before the head rows, used after them
  ld_vec(hlw, a.ln_out);
  ld_vec(hlb, a.ln_out + C);
#pragma unroll
  for (int b = 0; b < kHRing; ++b) pre_head(b, wh[b]);
  __syncthreads();  // AH
  {
    const float2 st = combine_stats(s.xst, C, inv_c);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = mt + kMT * i;
      if (c < C) s.mix[c] = (s.x1[c] - st.x) * st.y * hlw[i] + hlb[i];
    }
  }
  __syncthreads();  // BH
  const bool bad = cx.failed() || glob_abort;
  constexpr int XE = Q8 ? 16 : 8;  // inputs per weight chunk
  float xr[CW][XE];
#pragma unroll
  for (int c = 0; c < CW; ++c) {
    const int j = lane + 64 * c;
#pragma unroll
    for (int e = 0; e < XE; ++e) xr[c][e] = j < wchC ? s.mix[XE * j + e] : 0.f;
  }
  float out = 0.f;  // lane k: logit of row hr0 + k
#pragma unroll
  for (int b = 0; b < NHB; ++b) {
    uint4 (&cur)[kHB][CW] = wh[b % kHRing];
#pragma unroll
    for (int k = 0; k < kHB; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < CW; ++c) {
        if constexpr (Q8) acc = dot16r_q8(cur[k][c], xr[c], acc);
        else acc = dot8r<BF>(cur[k][c], xr[c], acc);
      }
      acc = wave_sum(acc);
      if constexpr (Q8) acc *= hqs[b % kHRing][k];
      if (lane == kHB * b + k) out = acc;
    }
    if (b + kHRing < NHB) pre_head(b + kHRing, cur);
  }
  // NaN logits if this workgroup's input did not arrive or the launch was aborted
  if (hr0 + lane < hr1) a.logits[hr0 + lane] = bad ? F16T<BF>::kNaN : F16T<BF>::from_f(out);
}

// One workgroup per CU by construction (2 waves per SIMD): telling the
// compiler so keeps its scheduler from trading prefetch distance for an
// occupancy this kernel never runs at.
template <int CPL, int RM, int NC5, int VPL, int NL2, int NHB, bool Q8, bool BF>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_mk_kernel(MkArgs a) {
  extern __shared__ __align__(16) float smem[];
  MkGeom m;
  m.C = a.C;
  m.F = a.F;
  m.H = a.H;
  m.L = a.L;
  m.SR = a.rv + a.rw + a.ra + a.rg;
  m.G = gridDim.x;
  m.g = blockIdx.x;
  m.head = m.g < m.H;
  // worker rows: split over the G - H workers
  const int Gw = m.G - m.H, gw = m.head ? 0 : m.g - m.H;
  const int N1 = 3 * m.C + m.SR;
  auto part = [&](int n, int i) { return (int)((int64_t)n * i / Gw); };
  m.p1a = part(N1, gw);
  m.p1b = m.head ? m.p1a : part(N1, gw + 1);
  m.p4a = part(m.F, gw);
  m.p4b = m.head ? m.p4a : part(m.F, gw + 1);
  m.owa = part(m.C, gw);
  m.nown = m.head ? 0 : part(m.C, gw + 1) - m.owa;
  m.ha = part(a.V, gw);
  m.hb = m.head ? m.ha : part(a.V, gw + 1);
  m.e[0] = m.C;
  m.e[1] = 2 * m.C;
  m.e[2] = 3 * m.C;
  m.e[3] = m.e[2] + a.rv;
  m.e[4] = m.e[3] + a.rw;
  m.e[5] = m.e[4] + a.ra;
  m.seg0 = m.seg_of(m.p1a);
  m.nseg = m.p1b > m.p1a ? m.seg_of(m.p1b - 1) - m.seg0 + 1 : 0;
  const MkLds s = mk_lds(smem, m.C, m.F, m.SR);

  // One thread reads the epoch and the abort word, so every wave of the
  // workgroup takes the same view of the launch; a launch whose abort word is
  // already set for its epoch does no work (every wait gives up at once).
  if (threadIdx.x == 0) {
    const unsigned e = ld_u32(a.sync + SY_EPOCH);
    const unsigned ab = ld_u32(a.sync + SY_ABORT);
    *s.pubs = 0u;
    *s.xflag = 0u;
    *s.ep = e;
    *s.fail = ab == e + 1u ? 1u : 0u;
    st_u32(a.started + m.g, e + 1u);
  }
  __syncthreads();
  MkCtx cx;
  cx.sync = a.sync;
  cx.fail = s.fail;
  cx.epoch = __builtin_amdgcn_readfirstlane(*s.ep);
  cx.tag0 = cx.epoch * (5u * m.L + 1u) + 1u;
  cx.pskew = (m.g / kRep) * 34;

  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (m.head) {
    if (wv >= kMW) comm_head(a, m, s, cx);
    else math_head<NL2, BF>(a, m, s, cx, wv);
  } else {
    if (wv >= kMW) comm_worker<NC5 / 2, BF>(a, m, s, cx);
    else math_worker<CPL, RM, NC5, VPL, NHB, Q8, BF>(a, m, s, cx, wv);
  }
  // The next launch's epoch. In a launch that completed, this worker ends only
  // after every workgroup has published (its logits need the last layer's x,
  // which needs every worker's P5 and every head's core), so every workgroup
  // read the epoch already. An aborted launch is counted, and the epoch is
  // advanced only once every workgroup recorded its start (bounded wait).
  if (m.g == m.H && threadIdx.x == 0) {
    if (cx.aborted()) {
      __hip_atomic_fetch_add(a.sync + SY_ERRORS, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int spins = 0;
      for (int g = 0; g < m.G; ++g)
        while (ld_u32(a.started + g) != cx.epoch + 1u && ++spins < kSpinLimit) __builtin_amdgcn_s_sleep(1);
    }
    st_u32(a.sync + SY_EPOCH, cx.epoch + 1u);
  }
}

// ---- host side --------------------------------------------------------------

// The compiled instances: CPL 2, RM 3, NC5 8, VPL 3, NL2 8, NHB 10; variant
// v = q8 + 2 bf: matrices streamed as 16-bit or int8 (q8), 16-bit data in
// IEEE half or bfloat16 (bf).
constexpr int kCPL = 2, kRM = 3, kNC5 = 8, kVPL = 3, kNL2 = 8, kNHB = 10;
constexpr int kMkVariants = 4;
#define RWKV7_MK_INSTANCE(Q8, BF) decode_mk_kernel<kCPL, kRM, kNC5, kVPL, kNL2, kNHB, Q8, BF>
static const void *mk_instance(int v) {
  switch (v) {
    case 0: return (const void *)RWKV7_MK_INSTANCE(false, false);
    case 1: return (const void *)RWKV7_MK_INSTANCE(true, false);
    case 2: return (const void *)RWKV7_MK_INSTANCE(false, true);
    default: return (const void *)RWKV7_MK_INSTANCE(true, true);
  }
}

static int cdiv(int a, int b) { return (a + b - 1) / b; }

// Per-device facts, filled on first use with that device current: the CU
// count, the largest dynamic LDS size already allowed for the kernel, and
// whether a grid of one workgroup per CU with a given LDS size fits at once.
constexpr int kMaxDevices = 64;
struct MkDevice {
  std::atomic<int> cus{0};
  std::atomic<int64_t> lds_allowed[kMkVariants] = {};   // per instance variant
  std::atomic<int64_t> resident_lds[kMkVariants] = {};  // largest LDS size found co-resident
};
static MkDevice g_mk_dev[kMaxDevices];

static MkDevice *mk_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  return &g_mk_dev[dev];
}

int mk_cus() {
  MkDevice *d = mk_device();
  if (!d) return 0;
  int n = d->cus.load(std::memory_order_relaxed);
  if (n == 0) {
    int dev = 0;
    hipDeviceProp_t p;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) return 0;
    n = p.multiProcessorCount;
    d->cus.store(n, std::memory_order_relaxed);
  }
  return n;
}

static int64_t mk_lds_bytes(int C, int F, int SR) { return mk_lds_floats(C, F, SR) * 4; }

// Exchange region: sync words, start words, then x (kRep x C), proj (3C+SR),
// core (kRep x C), hid (kRep x F) as u64.
int64_t mk_exchange_bytes(int C, int F, int SR) {
  return kSyncBytes + 4 * kMaxG + (int64_t)(kRep * C + kRep * (3 * C + SR) + kRep * C + kRep * F) * 8;
}

// Allows the kernel its dynamic LDS on the current device and checks that a
// grid of one workgroup per CU can be resident at once (the occupancy of this
// kernel instance with that LDS is at least one workgroup per CU).
static bool mk_prepare(int64_t lds, int v) {
  MkDevice *d = mk_device();
  if (!d || v < 0 || v >= kMkVariants) return false;
  const void *fn = mk_instance(v);
  if (lds > d->lds_allowed[v].load(std::memory_order_relaxed)) {
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) return false;
    d->lds_allowed[v].store(lds, std::memory_order_relaxed);
  }
  if (lds <= d->resident_lds[v].load(std::memory_order_relaxed)) return true;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kT, (size_t)lds) != hipSuccess || per_cu < 1)
    return false;
  d->resident_lds[v].store(lds, std::memory_order_relaxed);
  return true;
}

bool mk_supported(const rwkv7_dims &d, int G) {
  const int C = d.n_embd, F = d.n_ffn, H = d.n_head, V = d.vocab;
  const int SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g;
  const int Gw = G - H;  // worker workgroups
  if (C != H * kN || Gw < 1) return false;
  const int N1 = 3 * C + SR;
  // every worker owns at least one residual channel and one P1 row, so each
  // worker's end implies every workgroup has published
  if (C < Gw || N1 < Gw || F < Gw || V < Gw) return false;
  if (cdiv(C >> 3, 64) > kCPL || cdiv(F >> 3, 64) > kNC5) return false;
  if (cdiv(cdiv(N1, Gw), kMW) > kRM || cdiv(cdiv(F, Gw), kMW) > kRM) return false;
  if (cdiv(C, Gw) > kMW) return false;  // one residual channel per math wave
  if (cdiv(C, kMT) > kVPL) return false;
  // P2 parts (v, w, a, two halves of g), at most kNL2 chunks each, one wave each
  {
    const int cv = d.rank_v >> 3, cw = d.rank_w >> 3, ca = d.rank_a >> 3, cg = d.rank_g >> 3;
    if (cv > kNL2 || cw > kNL2 || ca > kNL2 || (cg + 1) / 2 > kNL2 || kMW < 5) return false;
  }
  const int cj = 2 * 64 * kNComm;  // words per round: one pair per lane and slot
  // x, core and hidden-vector slices: one read round of at most one (x, core)
  // or NC5 / 2 (hidden) pairs per lane; the P2 input in kW even slices of at
  // most 128 words
  if (C / kW > cj || cdiv(F / kW, cj) > kNC5 / 2 || ((192 + SR + kW - 1) / kW + 1) / 2 > 64) return false;
  if (F % (2 * kW)) return false;  // hidden-vector slices of whole 16-byte pairs
  if (C % (2 * kW) || C / kW > 128) return false;  // x slices: whole pairs, <= 2 values per lane
  if (H > 64 * kNComm) return false;  // one probe lane per head
  const int hrows = cdiv(cdiv(V, Gw), kMW);
  if (hrows > kHB * kNHB || hrows > 64) return false;
  // P1 keeps the mixed input of every row segment a worker touches (<= 4)
  if (G > kMaxG) return false;
  const int e[6] = {C, 2 * C, 3 * C, 3 * C + d.rank_v, 3 * C + d.rank_v + d.rank_w,
                    3 * C + d.rank_v + d.rank_w + d.rank_a};
  auto seg = [&](int r) {
    int s = 0;
    for (int i = 0; i < 6; ++i) s += r >= e[i];
    return s;
  };
  for (int g = 0; g < Gw; ++g) {
    const int r0 = (int)((int64_t)N1 * g / Gw), r1 = (int)((int64_t)N1 * (g + 1) / Gw);
    if (seg(r1 - 1) - seg(r0) + 1 > 4) return false;
  }
  return mk_lds_bytes(C, F, SR) <= 160 * 1024;
}

static int mk_variant(const rwkv7_model &m) {
  return (mk_int8(m) ? 1 : 0) + ((m.flags & RWKV7_MODEL_BF16) ? 2 : 0);
}

bool mk_usable(const rwkv7_model &m) {
  const rwkv7_dims &d = m.dims;
  const int G = mk_cus();
  if (G < 1 || !mk_supported(d, G)) return false;
  const int SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g;
  return mk_prepare(mk_lds_bytes(d.n_embd, d.n_ffn, SR), mk_variant(m));
}

bool mk_int8(const rwkv7_model &m) {
  return (m.flags & RWKV7_MODEL_INT8_DECODE) && m.layers_q != nullptr && m.head_q != nullptr;
}

int launch_decode_mk(const rwkv7_model &m, const rwkv7_layer_layout &lay, const rwkv7_state &s,
                     const int64_t *tok, void *logits, char *xreg, hipStream_t st) {
  const rwkv7_dims &d = m.dims;
  const int SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g;
  const int G = mk_cus();
  const int C = d.n_embd, F = d.n_ffn;
  const int variant = mk_variant(m);
  if (!mk_usable(m)) return RWKV7_ESHAPE;
  MkArgs a;
  a.layers_q = static_cast<const char *>(m.layers_q);
  a.q_lbytes = lay.q_bytes;
  a.q_rkv = lay.q_rkv;
  a.q_o = lay.q_o;
  a.q_fk = lay.q_fk;
  a.q_fv = lay.q_fv;
  a.q_scale = lay.q_scale;
  a.head_q = static_cast<const uint16_t *>(m.head_q);
  a.head_qs = m.head_q ? reinterpret_cast<const float *>(static_cast<const char *>(m.head_q) +
                                                         ((int64_t)d.vocab * C + 255) / 256 * 256)
                       : nullptr;
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
  a.started = reinterpret_cast<unsigned *>(xreg + kSyncBytes);
  uint64_t *ex = reinterpret_cast<uint64_t *>(xreg + kSyncBytes + 4 * kMaxG);
  a.x_ex = ex;
  a.proj_ex = a.x_ex + (int64_t)kRep * C;
  a.core_ex = a.proj_ex + (int64_t)kRep * (3 * C + SR);
  a.hid_ex = a.core_ex + (int64_t)kRep * C;
  const int64_t lds = mk_lds_bytes(C, F, SR);
  switch (variant) {
    case 0: RWKV7_MK_INSTANCE(false, false)<<<G, kT, lds, st>>>(a); break;
    case 1: RWKV7_MK_INSTANCE(true, false)<<<G, kT, lds, st>>>(a); break;
    case 2: RWKV7_MK_INSTANCE(false, true)<<<G, kT, lds, st>>>(a); break;
    default: RWKV7_MK_INSTANCE(true, true)<<<G, kT, lds, st>>>(a); break;
  }
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

}  // namespace rwkv7

RWKV7_TL_READER(rwkv7_timeline_read_decode, rwkv7::tl_decode);
