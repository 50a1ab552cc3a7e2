// A step of a few rows -- B sequences x T tokens, M = B T <= 16 (batched
// decode, short prefills) -- as one persistent kernel.
//
// The multi-launch path runs such a step as ~7-10 dependent launches per layer
// (LayerNorm + shift, GEMM groups, the per-head core, ...), each a few us of
// launch ramp and one memory round trip for a few MB of weights. Here the
// whole step runs in one grid of one workgroup per CU and every layer is five
// stages joined by grid-wide hand-offs:
//   P1  LN1 + token shift + [r; k; v; LoRA first steps]   16-row blocks of
//       the [3C+sumR, C] matrix, one block per workgroup
//   P2  per (sequence, head): LoRA second steps, gates, L2 norm, the wkv7 scan
//       over the sequence's T tokens, GroupNorm, bonus, output gate
//   P3  o-projection + residual                            C/16 blocks
//   P4  LN2 + shift + FFN key + relu^2                     F/16 blocks
//   P5  FFN value + residual                               C/16 blocks x 4
//       K-quarters; quarter 0 adds the other three's partial tiles, handed
//       over as tagged words ({value, tag} as one 64-bit store / load, polled
//       directly), in a fixed order
// then (decode) LN_out and the head, V/16 blocks.
//
// Matrix stages run on MFMA (v_mfma_f32_16x16x32_f16): a block is 16 weight
// rows of the fragment arena (one contiguous KiB per 16 x 32 fragment), the A
// operand is the M activation rows (padded to 16) staged in LDS as f32, and
// the 8 waves of the workgroup split K and sum their 16 x 16 tiles in LDS.
// Each A fragment is split in registers into its 16-bit part and the 16-bit
// remainder (split_hi_lo) and both are multiplied by the weight fragment, so
// the activations keep fp32-grade precision; the hand-off payloads (residual
// rows, per-head outputs, FFN hidden rows) are f32.
//
// Hand-offs. P2 -> P3, P3 -> P4, P4 -> P5 and P5 -> next P1 (the residual
// rows x, the per-head outputs, the FFN hidden rows): the producer of a block
// writes its payload with device-scope (sc1) stores, waits until they are
// acknowledged (s_waitcnt vmcnt(0)), then a workgroup barrier, then stores the
// block's flag word = the stage's tag; a consumer polls the flags it needs
// with device-scope loads and then reads the payload with device-scope loads.
// This relies on the gfx942/gfx950 behaviour the split-K GEMM relies on: a
// store issued with sc1 is acknowledged only once it reached the device's
// coherence point beyond every XCD's L2, and sc1 loads are not served from a
// stale L2 line. P1 -> P2 (the projections, small per reader) and the P5
// partial tiles: tagged words, {value, tag} stored and loaded as one 64-bit
// device-scope access (single-copy atomic), which the consumer polls directly
// -- no acknowledgement wait, flag or separate read; measured, this pays for
// small payloads but not for the 32-64 KB ones, whose reads it doubles. Tags
// are unique per (launch, layer, stage); a buffer is rewritten only after
// every reader of its previous contents has published a later stage that the
// writer waited for.
//
// Every wait is bounded; past the spin limit the waiting workgroup raises the
// launch's abort word, every other waiter gives up within a few polls, and the
// launch writes NaN logits and no state for unfinished work, as the batch-1
// persistent kernel does (decode_mk.hip); an aborted launch is counted in the
// workspace error word (rwkv7_workspace_errors).
//
// Reference counterparts: RWKV7Base.decode / prefill with a batched state
// (demo/_rwkv7_base.py:74-98) and the captured graphs of short steps
// (demo/cuda_graph.py:111-148).
#include <atomic>

#include "rwkv7_kernels.h"

namespace rwkv7 {
namespace {

constexpr int kRT = 512;             // threads per workgroup
constexpr int kRW = kRT / 64;        // waves
constexpr int kRSpin = 1 << 21;      // polls before a wait gives up
constexpr int kRMaxC = 1024;         // A tiles of C columns live in LDS
constexpr int kRLdX = kRMaxC + 4;    // floats per LDS row of xs (padding spreads the 16 rows over the banks)
constexpr int kRLdA = kRMaxC + 8;    // halves per row of the second LDS region (P2 scratch)
constexpr int kRMaxG = 1024;
// timeline points (diagnostic build), per layer, from the first block of each
// stage a workgroup runs: P1 0 start, 1 input x ready, 2 statistics, 3 products
// done; P2 4 start, 5 done; P3 6 start, 7 input ready, 8 published; P4 9 start,
// 10 input ready, 11 statistics, 12 products done, 13 published; P5 14 start,
// 15 input ready, 16 products done, 17 published
RWKV7_TL_BUFFER(tl_rows);
// P2 keeps the activated LoRA first steps (f32 [16][552]), the second steps
// and gates of up to 16 tokens (f32 [16][256 + 512] + 16) in the xs and
// scratch regions
static_assert(16 * 552 * 4 + (16 * (256 + 512) + 16) * 4 <= 16 * kRLdX * 4 + 16 * kRLdA * 2, "P2 scratch");

// sync words (byte offsets 0, 16): epoch, abort; then kRMaxG start words
enum { RS_EPOCH = 0, RS_ABORT = 4 };
constexpr int kRSyncBytes = 256;

struct RkArgs {
  const char *layers, *frag;
  int64_t lbytes, fbytes, o_l2, o_vec, f_rkv, f_l1[4], f_o, f_fk, f_fv;
  const uint16_t *emb, *head_frag;
  const float *ln_out;
  int L, C, H, F, V, rv, rw, ra, rg, SR;
  uint16_t *tmix_x;
  float *rnn;
  uint16_t *cmix_x;
  const int64_t *tok;
  uint16_t *logits;  // [B, V] or null
  int B, T, M, G;
  unsigned *sync, *started, *errors;
  unsigned *fl[5];   // per-stage flags: P2 units, P3 blocks, P4 blocks, P5 blocks (fl[0] unused: P1 hands off tagged words)
  uint64_t *proj;    // [M, 3C + SR] f32 as tagged words
  float *core;       // [M, C]
  float *x;          // [M, C]
  float *hid;        // [M, F]
  uint64_t *part;    // [C/16, 4, 256] FFN-value partial tiles of K-quarters 1..3 (tagged words)
  float *vfirst;     // [M, C]
};

RWKV7_DEV unsigned rld(const unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RWKV7_DEV void rst(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RWKV7_DEV void rst_f(float *p, float v) { rst(reinterpret_cast<unsigned *>(p), __builtin_bit_cast(unsigned, v)); }
RWKV7_DEV float rld_f(const float *p) { return __builtin_bit_cast(float, rld(reinterpret_cast<const unsigned *>(p))); }

// 16-byte device-scope loads through a buffer resource (reads past the end
// return zero)
RWKV7_DEV __amdgpu_buffer_rsrc_t rrsrc(const void *p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}
typedef unsigned u32x4r __attribute__((ext_vector_type(4)));
RWKV7_DEV u32x4r rld16(__amdgpu_buffer_rsrc_t r, int byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, /*sc1*/ 16);
}
// The same load as four floats (whole-vector bit cast: a bit cast of one
// element of an ext-vector lvalue is not what it reads in this compiler)
RWKV7_DEV floatx4 rld16f(__amdgpu_buffer_rsrc_t r, int byte_off) { return __builtin_bit_cast(floatx4, rld16(r, byte_off)); }

struct RkCtx {
  unsigned *sync;
  unsigned *fail;  // LDS: nonzero once this workgroup gave up
  unsigned epoch, tag0;
  RWKV7_DEV unsigned tag(int l, int st) const { return tag0 + 5u * (unsigned)l + (unsigned)st; }
  RWKV7_DEV bool failed() const {
    return __hip_atomic_load(fail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u;
  }
  RWKV7_DEV bool aborted() const { return rld(sync + RS_ABORT) == epoch + 1u; }
  RWKV7_DEV void give_up() const { __hip_atomic_store(fail, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
};

// Wave 0 polls flags[idx(i)], i < n, until all carry `tag` (bounded); then
// the workgroup barrier. Returns false if this workgroup gave up.
template <typename Idx>
RWKV7_DEV bool wait_flags(const RkCtx &cx, const unsigned *flags, int n, unsigned tag, Idx idx) {
  if ((threadIdx.x >> 6) == 0 && !cx.failed()) {
    const int lane = threadIdx.x & 63;
    int spins = 0;
    for (;;) {
      bool ok = true;
      for (int i = lane; i < n; i += 64) ok = ok && rld(flags + idx(i)) == tag;
      if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
      ++spins;
      if ((spins & 1023) == 0 && cx.aborted()) {
        if (lane == 0) cx.give_up();
        break;
      }
      if (spins > kRSpin) {
        if (lane == 0) {
          rst(cx.sync + RS_ABORT, cx.epoch + 1u);
          cx.give_up();
        }
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  return !cx.failed();
}

// Publishes a block: the payload stores of every thread are acknowledged
// before one thread stores the flag.
RWKV7_DEV void publish_flag(const RkCtx &cx, unsigned *flag, unsigned tag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0 && !cx.failed()) rst(flag, tag);
}

// Tagged words: a value and the tag of the (launch, layer, stage) that wrote
// it, stored and loaded as one 64-bit device-scope access (single-copy
// atomic), so a reader that sees the tag also sees the value.
RWKV7_DEV void st64f(uint64_t *p, float v, unsigned tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | __builtin_bit_cast(unsigned, v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
RWKV7_DEV unsigned tag_of(uint64_t w) { return (unsigned)(w >> 32); }
RWKV7_DEV float val_f(uint64_t w) { return __builtin_bit_cast(float, (unsigned)w); }
typedef unsigned u32x2r __attribute__((ext_vector_type(2)));
RWKV7_DEV uint64_t rld8(__amdgpu_buffer_rsrc_t r, int byte_off) {
  const u32x2r v = __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, /*sc1*/ 16);
  return ((uint64_t)v[1] << 32) | v[0];
}

// N tagged words at byte offsets off(i) of r, each read again until its tag
// equals `tag` (bounded like wait_flags; a thread that gives up raises the
// abort word or follows another workgroup's).
template <int N, typename Off>
RWKV7_DEV void read_words(const RkCtx &cx, __amdgpu_buffer_rsrc_t r, unsigned tag, Off off, uint64_t (&w)[N]) {
  unsigned pend = (1u << N) - 1u;
#pragma unroll
  for (int i = 0; i < N; ++i) w[i] = rld8(r, off(i));
  int spins = 0;
  for (;;) {
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (((pend >> i) & 1u) && tag_of(w[i]) == tag) pend &= ~(1u << i);
    if (pend == 0 || cx.failed()) break;
    ++spins;
    if ((spins & 1023) == 0 && cx.aborted()) {
      cx.give_up();
      break;
    }
    if (spins > kRSpin) {
      rst(cx.sync + RS_ABORT, cx.epoch + 1u);
      cx.give_up();
      break;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if ((pend >> i) & 1u) w[i] = rld8(r, off(i));
  }
}

struct RkLds {
  float *xs;        // [16][kRLdX] the stage's input rows, then its MFMA A operand (f32)
  uint16_t *A;      // [16][kRLdA] second region, P2 scratch (with xs)
  float *red;       // [kRW][256] per-wave partial tiles
  float *stat;      // [16][4] LN mean, rstd of each row
  float *u;         // P2 scratch
  uint16_t *sst;    // [16][C] the layer's old shift states (f16)
  int *tok;         // [16] embedding row offsets of the step's tokens
  uint16_t *shs1, *shs2;  // [16][16] this workgroup's 16 columns of the new time-/channel-mix shift states
  unsigned *fail, *ep;
};

// LN statistics (mean, 1/std) of the M <= 16 rows of xs: 32 threads per row
// (rows 2w and 2w + 1 on wave w), each holding C / 32 <= 32 of the row's
// values in registers for the two-pass variance.
RWKV7_DEV void row_stats(const RkLds &s, int M, int C) {
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int m = 2 * wv + (lane >> 5), l32 = lane & 31;
  const bool live = m < M;
  float4 v[8];
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int c = 4 * l32 + 128 * j;
    v[j] = live && c < C ? *reinterpret_cast<const float4 *>(s.xs + m * kRLdX + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    acc += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  acc = sum16(acc);
  const float sum = lane < 32 ? lane_value(acc, 0) + lane_value(acc, 16) : lane_value(acc, 32) + lane_value(acc, 48);
  const float mean = sum / (float)C;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (4 * l32 + 128 * j < C) {
      const float d0 = v[j].x - mean, d1 = v[j].y - mean, d2 = v[j].z - mean, d3 = v[j].w - mean;
      q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    }
  }
  q = sum16(q);
  const float sq = lane < 32 ? lane_value(q, 0) + lane_value(q, 16) : lane_value(q, 32) + lane_value(q, 48);
  if (live && l32 == 0) {
    s.stat[4 * m] = mean;
    s.stat[4 * m + 1] = rsqrtf(sq / (float)C + kLnEps);
  }
}

// The B shift-state rows of a layer ([B][C] f16) into LDS (sst), eight
// halves per load, by waves 1..7 (wave 0 polls; see load_block), up to five
// loads in flight per thread.
RWKV7_DEV void load_state(const RkLds &s, const uint16_t *state, int B, int C) {
  if (threadIdx.x < 64) return;
  const int tid = threadIdx.x - 64, nt = kRT - 64;
  const uint4 *src = reinterpret_cast<const uint4 *>(state);
  uint4 *dst = reinterpret_cast<uint4 *>(s.sst);
  const int n = B * C / 8;
  for (int i0 = tid; i0 < n; i0 += 5 * nt) {
    uint4 v[5];
#pragma unroll
    for (int j = 0; j < 5; ++j) v[j] = i0 + j * nt < n ? src[i0 + j * nt] : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 5; ++j)
      if (i0 + j * nt < n) dst[i0 + j * nt] = v[j];
  }
}

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
// Two floats as packed halves, round to nearest even (v_cvt_pk_f16_f32; the
// same bits as two single conversions).
RWKV7_DEV unsigned pack_h2(float lo, float hi) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2v{lo, hi}, f16x2v));
}

// xs[m][k] <- ln(m) + mu[k] (prev(m) - ln(m)) for rows m < M, in place (f32),
// with ln(m) = LayerNorm of row m (statistics from row_stats) and prev(m) =
// ln(m - 1) within a sequence, the f16 shift state (sst) for its first token.
// Rows M..15 are left as they are: they only reach output rows that are never
// stored. Thread t < C / 2 owns columns 2t, 2t + 1 of every row (LN weight,
// bias and mix from load_mix, loaded before the stage's wait) and walks the
// rows in order, keeping ln(m - 1) in registers, so the in-place update never
// overwrites a value another thread still reads. With c0 >= 0, columns
// [c0, c0 + 16) of each sequence's last LayerNorm row -- the new shift state
// -- also go to slice ([B][16] f16, LDS).
struct MixVec {
  float2 w, b, u;  // LN weight, LN bias, mix of this thread's 2 columns
};
RWKV7_DEV MixVec load_mix(const float *lw, const float *lb, const float *mu, int C) {
  const int k = 2 * (threadIdx.x % (C / 2));
  MixVec v;
  v.w = *reinterpret_cast<const float2 *>(lw + k);
  v.b = *reinterpret_cast<const float2 *>(lb + k);
  v.u = *reinterpret_cast<const float2 *>(mu + k);
  return v;
}

RWKV7_DEV void build_mix(const RkLds &s, const RkArgs &a, int C, const MixVec &mv, uint16_t *slice, int c0) {
  if ((int)threadIdx.x >= C / 2) return;
  const int M = a.M, T = a.T;
  const int k = 2 * threadIdx.x;
  const float2 w = mv.w, bias = mv.b, u = mv.u;
  const bool shift_cols = c0 >= 0 && k >= c0 && k < c0 + 16;
  float2 p = make_float2(0.f, 0.f);
  int t = 0, b = 0;
  for (int m = 0; m < M; ++m) {
    float2 *xp = reinterpret_cast<float2 *>(s.xs + m * kRLdX + k);
    const float2 x = *xp;
    const float2 st = *reinterpret_cast<const float2 *>(s.stat + 4 * m);  // mean, 1/std
    const float nm = -st.x * st.y;
    const float2 ln = make_float2(fmaf(fmaf(x.x, st.y, nm), w.x, bias.x), fmaf(fmaf(x.y, st.y, nm), w.y, bias.y));
    if (t == 0) {
      const unsigned sv = *reinterpret_cast<const unsigned *>(s.sst + b * C + k);
      p = make_float2(h2f((uint16_t)(sv & 0xFFFFu)), h2f((uint16_t)(sv >> 16)));
    }
    *xp = make_float2(fmaf(u.x, p.x - ln.x, ln.x), fmaf(u.y, p.y - ln.y, ln.y));
    if (t == T - 1 && shift_cols) *reinterpret_cast<unsigned *>(slice + b * 16 + (k - c0)) = pack_h2(ln.x, ln.y);
    p = ln;
    if (++t == T) t = 0, ++b;
  }
}

// The weights of one 16-row block, spread over waves 1..7 (wave 0 polls the
// hand-off flags and issues no load before a wait: its poll results would
// queue behind them): wave w >= 1 takes k-steps w - 1, w - 1 + 7, ... of the
// block's nks <= 35 (fragment k-step k at wf + (k0step + k) 512 halves).
// Loaded ahead of a stage's wait, used by block_mma after it.
constexpr int kWW = kRW - 1;  // weight-loading waves
struct WBlock {
  uint4 w[5];
};
RWKV7_DEV WBlock load_block(const uint16_t *wf, int k0step, int nks) {
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  WBlock b;
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const int kj = wv - 1 + kWW * j;
    b.w[j] = wv > 0 && kj < nks ? ld_stream(reinterpret_cast<const uint4 *>(wf + (int64_t)(k0step + kj) * 512) + lane)
                                : make_uint4(0, 0, 0, 0);
  }
  return b;
}

// The block times the A tile (xs columns 32 k .. 32 k + 31 for k-step k, f32,
// each fragment split into its f16 part and f16 remainder: two MFMAs).
// Returns the wave's partial 16 x 16 tile (zero on wave 0), rows = A rows,
// columns = the block's weight rows.
RWKV7_DEV floatx4 block_mma(const RkLds &s, const WBlock &wb, int nks) {
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
  if (wv == 0) return acc;
#pragma unroll
  for (int j = 0; j < 5; ++j) {
    const int kj = wv - 1 + kWW * j;
    if (kj < nks) {
      const float *ap = s.xs + (lane & 15) * kRLdX + 32 * kj + 8 * (lane >> 4);
      uint4 hi, lo;
      split_hi_lo<false>(*reinterpret_cast<const uint4 *>(ap), *reinterpret_cast<const uint4 *>(ap + 4), hi, lo);
      acc = mfma16<false>(hi, wb.w[j], acc);
      acc = mfma16<false>(lo, wb.w[j], acc);
    }
  }
  return acc;
}

// Sum of the waves' tiles: thread t < 256 gets D[m][n], m = 4 ((t & 63) >> 4)
// + (t >> 6), n = t & 15 (rows of A, rows of the weight block).
RWKV7_DEV float reduce_tile(const RkLds &s, const floatx4 &acc, int *m_out, int *n_out) {
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  *reinterpret_cast<float4 *>(&s.red[wv * 256 + 4 * lane]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  __syncthreads();
  const int t = threadIdx.x & 255;
  const int l = t & 63, r = t >> 6;
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < kRW; ++w) v += s.red[w * 256 + 4 * l + r];
  *m_out = 4 * (l >> 4) + r;
  *n_out = l & 15;
  return v;
}

// Reads columns [c0, c0 + K) of an [M][ld] f32 buffer (device-scope) into xs
// rows 0..M-1 (K <= kRMaxC), zero rows M..15 when zero_rest; every load of
// the thread (at most 8) in flight before the first LDS store.
RWKV7_DEV void read_rows(const RkLds &s, const float *src, int ld, int c0, int K, int M, bool zero_rest) {
  const __amdgpu_buffer_rsrc_t r = rrsrc(src, (int64_t)M * ld * 4);
  const int q = K / 4;  // 16-byte pieces per row
  const int rows = zero_rest ? 16 : M;
  floatx4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = threadIdx.x + j * kRT, m = i / q, p = i - m * q;
    v[j] = m < M ? rld16f(r, 4 * (m * ld + c0 + 4 * p)) : floatx4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = threadIdx.x + j * kRT, m = i / q, p = i - m * q;
    if (m < rows) *reinterpret_cast<floatx4 *>(&s.xs[m * kRLdX + 4 * p]) = v[j];
  }
}
// The [M][C] f32 residual rows x into xs.
RWKV7_DEV void read_x(const RkLds &s, const float *x, int M, int C) { read_rows(s, x, C, 0, C, M, false); }

RWKV7_DEV int64_t clamp_tok(int64_t id, int V) { return id < 0 ? 0 : id >= V ? V - 1 : id; }

// The embedding rows of the step's tokens (layer 0 input) into xs; thread ->
// column, the M row loads issued together. s.tok: the rows' offsets in emb.
RWKV7_DEV void embed_rows(const RkLds &s, const RkArgs &a) {
  const int C = a.C, M = a.M;
  if (threadIdx.x < 16) s.tok[threadIdx.x] = threadIdx.x < M ? (int)clamp_tok(a.tok[threadIdx.x], a.V) * C : 0;
  __syncthreads();
  int id[16];
#pragma unroll
  for (int m = 0; m < 16; ++m) id[m] = s.tok[m];
  for (int k = threadIdx.x; k < C; k += kRT) {
    float v[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) v[m] = m < M ? h2f(a.emb[id[m] + k]) : 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m)
      if (m < M) s.xs[m * kRLdX + k] = v[m];
  }
}

// The residual input of row m, column c at layer l: the embedding row at
// layer 0, else the hand-off vector x.
RWKV7_DEV float residual_in(const RkArgs &a, int l, int m, int c) {
  if (l > 0) return rld_f(a.x + (int64_t)m * a.C + c);
  return h2f(a.emb[clamp_tok(a.tok[m], a.V) * a.C + c]);
}

// This workgroup's 16-column slice of a new shift state (LDS [B][16] f16,
// from build_mix) into columns [c0, c0 + 16) of layer l of a state arena.
RWKV7_DEV void store_shift_slice(const RkArgs &a, const uint16_t *slice, uint16_t *arena, int l, int c0) {
  if ((int)threadIdx.x < a.B * 8) {
    const int b = threadIdx.x >> 3, c = 2 * (threadIdx.x & 7);
    *reinterpret_cast<unsigned *>(arena + ((int64_t)l * a.B + b) * a.C + c0 + c) =
        *reinterpret_cast<const unsigned *>(slice + b * 16 + c);
  }
}

// ---- P2: one (sequence, head) unit over its T tokens --------------------------
// Gates of every token first (they do not depend on the state), then the
// sequential wkv7 scan, then GroupNorm and the output of every token:
//   A1  thread t < SR: LoRA first-step column t of the T tokens, activated,
//       into LDS as f16 [T][kLoraLd]; wave w: r, k, v (and v_first) of its
//       tokens w, w + 8 into registers -- every load of the unit in flight
//   A2  LoRA second steps on MFMA: [T x R] activations times the head's
//       [R x 16] weight tiles (4 gates x 4 channel tiles, two per wave), the
//       weights read from the row-major [C, SR] arena before the unit's wait
//   A3  gates, one wave per token, lane = channel
//   B   wkv7 over the T tokens, thread t -> state row t >> 3, key columns
//       8 (t & 7) .. +8 (no barrier between tokens: a thread's rows depend
//       only on the precomputed gates)
//   C   GroupNorm over the head, bonus, output gate, one wave per token
// Per token this is the one-token core's arithmetic (tmix.hip,
// tmix_decode_kernel), the LoRA activations multiplied as f16 parts and f16
// remainders.
constexpr int kLoraLd = 512 + 40;  // floats per LDS LoRA row: SR <= 512, a zeroed 32-wide tail, 16-byte rows
RWKV7_DEV void p2_unit(const RkArgs &a, const RkLds &s, const RkCtx &cx, int l, int b, int h) {
  const int t = threadIdx.x, wv = t >> 6, lane = t & 63;
  const int C = a.C, SR = a.SR, T = a.T;
  const int N1 = 3 * C + SR;
  const char *Lp = a.layers + (int64_t)l * a.lbytes;
  const float *vec = reinterpret_cast<const float *>(Lp + a.o_vec);
  const uint16_t *l2 = reinterpret_cast<const uint16_t *>(Lp + a.o_l2);
  float *s_l32 = s.u;                                              // [16][kLoraLd] f32
  float *s_d = s.u + 16 * kLoraLd;                                 // [T][4][64] LoRA second steps v w a g
  float *s_g = s_d + 16 * 256;                                     // [T][8][64] r w kn v kh b g y
  float *s_rk = s_g + 16 * 512;                                    // [T]
  const int ch = h * kN + lane;
  // loads that do not depend on this layer's hand-offs: the wkv state rows,
  // the wave's LoRA second-step weight fragments and the channel's vectors --
  // before the wait on waves 1..7, after it on wave 0 (the polling wave,
  // whose poll results would queue behind them)
  float S[8];
  float4 *Sp = reinterpret_cast<float4 *>(a.rnn + ((((int64_t)l * a.B + b) * a.H + h) * kN + (t >> 3)) * kN + (t & 7) * 8);
  // wave w: (gate, channel tile) pairs w and w + 8: gate = pair >> 2, tile = pair & 3
  int goff[2], grank[2];
  uint4 wq[2][4];
  float v_v0, v_w0, v_a0, v_kk, v_ka, v_rk, v_lw, v_lb;
  auto prefetch = [&]() {
    const float4 u0 = Sp[0], u1 = Sp[1];
    S[0] = u0.x, S[1] = u0.y, S[2] = u0.z, S[3] = u0.w, S[4] = u1.x, S[5] = u1.y, S[6] = u1.z, S[7] = u1.w;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int q = (wv + kRW * e) >> 2, tile = (wv + kRW * e) & 3;
      goff[e] = q == 0 ? 0 : q == 1 ? a.rv : q == 2 ? a.rv + a.rw : a.rv + a.rw + a.ra;
      grank[e] = q == 0 ? a.rv : q == 1 ? a.rw : q == 2 ? a.ra : a.rg;
      const uint16_t *wrow = l2 + (int64_t)(h * kN + 16 * tile + (lane & 15)) * SR + goff[e];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int k = 32 * ks + 8 * (lane >> 4);
        wq[e][ks] = k < grank[e] ? *reinterpret_cast<const uint4 *>(wrow + k) : make_uint4(0, 0, 0, 0);
      }
    }
    v_v0 = vec[RWKV7_V_V0 * C + ch], v_w0 = vec[RWKV7_V_W0 * C + ch], v_a0 = vec[RWKV7_V_A0 * C + ch];
    v_kk = vec[RWKV7_V_K_K * C + ch], v_ka = vec[RWKV7_V_K_A * C + ch], v_rk = vec[RWKV7_V_R_K * C + ch];
    v_lw = vec[RWKV7_V_LNX_W * C + ch], v_lb = vec[RWKV7_V_LNX_B * C + ch];
  };
  prefetch();
  // A1: the P1 outputs of this unit, tagged words (each read again until it
  // carries this layer's P1 tag), all in flight at once: the LoRA first steps
  // as 16-byte chunks (columns j, j + 1 of token m; chunk i = t + kRT c,
  // c < 5: T SR / 2 <= 5 kRT), then r, k, v of the wave's tokens
  float pr[2], pk[2], pv[2], pf[2];
  {
    const __amdgpu_buffer_rsrc_t rp = rrsrc(a.proj + (int64_t)b * T * N1, (int64_t)T * N1 * 8);
    const int cpt = SR / 2, nch = T * cpt;
    const unsigned tg = cx.tag(l, 0);
    auto coff = [&](int c) {
      const int i = t + kRT * c, m = i / cpt;
      return 8 * (m * N1 + 3 * C + 2 * (i - m * cpt));
    };
    auto woff = [&](int i) { return 8 * ((wv + kRW * (i / 3)) * N1 + (i % 3) * C + ch); };
    u32x4r ck[5];
    uint64_t w[6];
    unsigned pend = 0;
#pragma unroll
    for (int c = 0; c < 5; ++c)
      if (t + kRT * c < nch) {
        ck[c] = rld16(rp, coff(c));
        pend |= 1u << c;
      }
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      w[i] = 0;
      if (wv + kRW * (i / 3) < T) {
        w[i] = rld8(rp, woff(i));
        pend |= 32u << i;
      }
    }
    int spins = 0;
    for (;;) {
#pragma unroll
      for (int c = 0; c < 5; ++c) {
        if (((pend >> c) & 1u) && ck[c][1] == tg && ck[c][3] == tg) {
          pend &= ~(1u << c);
          const int i = t + kRT * c, m = i / cpt, j = 2 * (i - m * cpt);
          // (the elements go through scalars: a bit cast of an ext-vector
          // element lvalue reads element 0 in this compiler)
          const unsigned u0 = ck[c][0], u1 = ck[c][2];
          float x0 = __builtin_bit_cast(float, u0), x1 = __builtin_bit_cast(float, u1);
          // tanh on the w group, sigmoid on the g group (j and j + 1 share a group: ranks are even)
          if (j >= a.rv && j < a.rv + a.rw) x0 = tanhf(x0), x1 = tanhf(x1);
          else if (j >= a.rv + a.rw + a.ra) x0 = sigmoidf_(x0), x1 = sigmoidf_(x1);
          *reinterpret_cast<float2 *>(&s_l32[m * kLoraLd + j]) = make_float2(x0, x1);
        }
      }
#pragma unroll
      for (int i = 0; i < 6; ++i)
        if (((pend >> (5 + i)) & 1u) && tag_of(w[i]) == tg) pend &= ~(32u << i);
      if (pend == 0 || cx.failed()) break;
      ++spins;
      if ((spins & 1023) == 0 && cx.aborted()) {
        cx.give_up();
        break;
      }
      if (spins > kRSpin) {
        rst(cx.sync + RS_ABORT, cx.epoch + 1u);
        cx.give_up();
        break;
      }
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int c = 0; c < 5; ++c)
        if ((pend >> c) & 1u) ck[c] = rld16(rp, coff(c));
#pragma unroll
      for (int i = 0; i < 6; ++i)
        if ((pend >> (5 + i)) & 1u) w[i] = rld8(rp, woff(i));
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      pr[e] = val_f(w[3 * e]);
      pk[e] = val_f(w[3 * e + 1]);
      pv[e] = val_f(w[3 * e + 2]);
      const int m = wv + kRW * e;
      pf[e] = l > 0 && m < T ? rld_f(a.vfirst + (int64_t)(b * T + m) * C + ch) : 0.f;
    }
  }
  if (t < 32)  // the zero tail past the last group (a partial k-step of a rank-16 group reads into it)
    for (int m = 0; m < T; ++m) s_l32[m * kLoraLd + SR + t] = 0.f;
  __syncthreads();
  const bool ok = !cx.failed();
#pragma unroll
  for (int e = 0; e < 2; ++e) {  // A2
    const int q = (wv + kRW * e) >> 2, tile = (wv + kRW * e) & 3;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (32 * ks < grank[e]) {
        const float *ap = &s_l32[(lane & 15) * kLoraLd + goff[e] + 32 * ks + 8 * (lane >> 4)];
        uint4 hi, lo;
        split_hi_lo<false>(*reinterpret_cast<const uint4 *>(ap), *reinterpret_cast<const uint4 *>(ap + 4), hi, lo);
        acc = mfma16<false>(hi, wq[e][ks], acc);
        acc = mfma16<false>(lo, wq[e][ks], acc);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * (lane >> 4) + r;
      if (m < T) s_d[m * 256 + q * 64 + 16 * tile + (lane & 15)] = acc[r];
    }
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 2; ++e) {  // A3
    const int m = wv + kRW * e;
    if (m >= T) break;
    const int mg = b * T + m;
    const float *d = s_d + m * 256;
    const float r = pr[e], k = pk[e];
    float v = pv[e];
    if (l == 0) {
      rst_f(a.vfirst + (int64_t)mg * C + ch, v);
    } else {
      v = v + sigmoidf_(v_v0 + d[lane]) * (pf[e] - v);
    }
    const float w = expf(-sigmoidf_(v_w0 + d[64 + lane]) / 1.6487212707001282f);
    const float ag = sigmoidf_(v_a0 + d[128 + lane]);
    const float kk = k * v_kk;
    const float kn = k + v_ka * (k * ag - k);
    const float nrm = sqrtf(wave_sum(kk * kk));
    const float kh = kk / fmaxf(nrm, 1e-12f);
    const float rk = wave_sum(r * kn * v_rk);
    float *gm = s_g + m * 512;
    gm[lane] = r;
    gm[64 + lane] = w;
    gm[128 + lane] = kn;
    gm[192 + lane] = v;
    gm[256 + lane] = kh;
    gm[320 + lane] = -kh * ag;
    gm[384 + lane] = d[192 + lane];
    if (lane == 0) s_rk[m] = rk;
  }
  __syncthreads();
  {  // B
    const int i = t >> 3, j0 = (t & 7) * 8;
    for (int m = 0; m < T; ++m) {
      float *gm = s_g + m * 512;
      float sa = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sa = fmaf(S[e], gm[256 + j0 + e], sa);
      sa = sum4(sa);
      sa += dpp<kDppHalfMirror>(sa);
      const float vi = gm[192 + i];
      float y = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = j0 + e;
        S[e] = S[e] * gm[64 + j] + sa * gm[320 + j] + vi * gm[128 + j];
        y = fmaf(S[e], gm[j], y);
      }
      y = sum4(y);
      y += dpp<kDppHalfMirror>(y);
      if ((t & 7) == 0) gm[448 + i] = y;
    }
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 2; ++e) {  // C
    const int m = wv + kRW * e;
    if (m >= T) break;
    const int mg = b * T + m;
    const float *gm = s_g + m * 512;
    const float y = gm[448 + lane];
    const float mean = wave_sum(y) * (1.f / kN);
    const float dy = y - mean;
    const float var = wave_sum(dy * dy) * (1.f / kN);
    const float yn = dy * rsqrtf(var + kGnEps) * v_lw + v_lb;
    const float out = (yn + s_rk[m] * gm[192 + lane]) * gm[384 + lane];
    if (ok) rst_f(a.core + (int64_t)mg * C + ch, out);
  }
  if (ok && !cx.failed()) {
    Sp[0] = make_float4(S[0], S[1], S[2], S[3]);
    Sp[1] = make_float4(S[4], S[5], S[6], S[7]);
  }
  __syncthreads();
}

__global__ __launch_bounds__(kRT) void rows_mk_kernel(RkArgs a) {
  extern __shared__ __align__(16) char rsmem[];
  const int C = a.C, F = a.F, M = a.M, L = a.L, G = a.G, SR = a.SR;
  const int g = blockIdx.x;
  RkLds s;
  s.xs = reinterpret_cast<float *>(rsmem);                       // 16 kRLdX floats
  s.A = reinterpret_cast<uint16_t *>(rsmem + 16 * kRLdX * 4);    // 16 kRLdA halves
  s.red = reinterpret_cast<float *>(rsmem + 16 * kRLdX * 4 + 16 * kRLdA * 2);
  s.stat = s.red + kRW * 256;
  s.fail = reinterpret_cast<unsigned *>(s.stat + 64);
  s.ep = s.fail + 1;
  s.tok = reinterpret_cast<int *>(s.fail + 16);
  s.shs1 = reinterpret_cast<uint16_t *>(s.fail + 32);
  s.shs2 = s.shs1 + 256;
  s.sst = s.shs2 + 256;
  s.u = s.xs;  // P2 scratch: xs and the second region (contiguous)
  if (threadIdx.x == 0) {
    const unsigned e = rld(a.sync + RS_EPOCH);
    *s.ep = e;
    *s.fail = rld(a.sync + RS_ABORT) == e + 1u ? 1u : 0u;
    rst(a.started + g, e + 1u);
  }
  __syncthreads();
  RkCtx cx;
  cx.sync = a.sync;
  cx.fail = s.fail;
  cx.epoch = __builtin_amdgcn_readfirstlane(*s.ep);
  cx.tag0 = cx.epoch * (5u * (unsigned)L + 1u) + 1u;

  const int N1 = 3 * C + SR;
  const int nP1 = N1 / 16, nP2 = a.B * a.H, nP3 = C / 16, nP4 = F / 16, nP5 = C / 16;
  const int nksC = C / 32, nksF = F / 32, nksQ = F / 128;  // k-steps: K = C, the fv strip, a quarter
  // P1 row segments r, k, v, then the LoRA first steps v, w, a, g (ends e0..e5, N1)
  const int e0 = C, e1 = 2 * C, e2 = 3 * C, e3 = e2 + a.rv, e4 = e3 + a.rw, e5 = e4 + a.ra;
  // Workgroup g < C/16 keeps columns [16 g, 16 g + 16) of the new shift states
  // in LDS and stores them into the State once no workgroup reads the old
  // values any more: the time-mix state of layer l after its P4 wait (every
  // o-projection block read every (sequence, head) unit's output, and every
  // unit read its P1 blocks), the channel-mix state of layer l after the P1
  // wait of layer l + 1 (or the last wait).
  const bool slice_owner = g < nP3;
  auto ident = [](int i) { return i; };

  for (int l = 0; l < L; ++l) {
    const char *Lp = a.layers + (int64_t)l * a.lbytes;
    const char *Fp = a.frag + (int64_t)l * a.fbytes;
    const float *vec = reinterpret_cast<const float *>(Lp + a.o_vec);
    // ---------------- P1 ----------------
    for (int b1 = g; b1 < nP1; b1 += G) {
      if (b1 == g) RWKV7_TL(tl_rows, l, 0);
      const int row0 = 16 * b1;
      const int sg = row0 < e0 ? 0 : row0 < e1 ? 1 : row0 < e2 ? 2 : row0 < e3 ? 3 : row0 < e4 ? 4 : row0 < e5 ? 5 : 6;
      const int mu = sg == 0 ? RWKV7_V_X_R : sg == 1 ? RWKV7_V_X_K : sg <= 3 ? RWKV7_V_X_V
                   : sg == 4 ? RWKV7_V_X_W : sg == 5 ? RWKV7_V_X_A : RWKV7_V_X_G;
      // r, k, v: strips of the [3C, C] arena; LoRA groups v, w, a, g: their own arenas
      const int64_t foff = sg < 3 ? a.f_rkv + (int64_t)b1 * nksC * 1024
                         : (sg == 3 ? a.f_l1[0] : sg == 4 ? a.f_l1[1] : sg == 5 ? a.f_l1[2] : a.f_l1[3]) +
                               (int64_t)((row0 - (sg == 3 ? e2 : sg == 4 ? e3 : sg == 5 ? e4 : e5)) / 16) * nksC * 1024;
      // before the wait: weights and old shift states (waves 1..7), the mix
      // vectors (wave 0 loads its own after the wait)
      const WBlock wb = load_block(reinterpret_cast<const uint16_t *>(Fp + foff), 0, nksC);
      load_state(s, a.tmix_x + (int64_t)l * a.B * C, a.B, C);
      const float *lw1 = vec + RWKV7_V_LN1_W * C, *lb1 = vec + RWKV7_V_LN1_B * C, *mu1 = vec + mu * C;
      MixVec mv{};
      if (threadIdx.x >= 64) mv = load_mix(lw1, lb1, mu1, C);
      if (l == 0) {
        embed_rows(s, a);
      } else {
        wait_flags(cx, a.fl[4], nP5, cx.tag(l - 1, 4), ident);
        if (b1 == g) RWKV7_TL(tl_rows, l, 1);
        read_x(s, a.x, M, C);
      }
      if (threadIdx.x < 64) mv = load_mix(lw1, lb1, mu1, C);
      __syncthreads();
      // the channel-mix state of the last layer (every FFN-value block of it has published)
      if (l > 0 && b1 == g && slice_owner && !cx.failed()) store_shift_slice(a, s.shs2, a.cmix_x, l - 1, 16 * g);
      row_stats(s, M, C);
      if (b1 == g) RWKV7_TL(tl_rows, l, 2);
      __syncthreads();
      // blocks 0 .. C/16 - 1 also write 16 columns each of the new time-mix shift state
      build_mix(s, a, C, mv, s.shs1, b1 == g && slice_owner ? 16 * g : -1);
      __syncthreads();
      const floatx4 acc = block_mma(s, wb, nksC);
      if (b1 == g) RWKV7_TL(tl_rows, l, 3);
      int m, n;
      const float v = reduce_tile(s, acc, &m, &n);
      if (threadIdx.x < 256 && m < M && !cx.failed()) st64f(a.proj + (int64_t)m * N1 + row0 + n, v, cx.tag(l, 0));
      __syncthreads();
    }
    // ---------------- P2 ----------------
    for (int u = g; u < nP2; u += G) {
      if (u == g) RWKV7_TL(tl_rows, l, 4);
      const int b = u / a.H, h = u % a.H;
      p2_unit(a, s, cx, l, b, h);
      if (u == g) RWKV7_TL(tl_rows, l, 5);
      publish_flag(cx, a.fl[1] + u, cx.tag(l, 1));
    }
    // ---------------- the shift states ----------------
    // Once every (sequence, head) unit has published, every P1 block of this
    // layer has been read, so no workgroup reads the old time-mix state of
    // this layer (P1) or the old channel-mix state of the last one (P4) again.

    // ---------------- P3 ----------------
    for (int b3 = g; b3 < nP3; b3 += G) {
      if (b3 == g) RWKV7_TL(tl_rows, l, 6);
      const WBlock wb = load_block(reinterpret_cast<const uint16_t *>(Fp + a.f_o) + (int64_t)b3 * nksC * 512, 0, nksC);
      // the residual of this thread's output (final since this workgroup's P1
      // wait), loaded and stored by threads 256..511 (not the polling wave)
      const int t = threadIdx.x & 255;
      const int mr = 4 * ((t & 63) >> 4) + (t >> 6), cr = 16 * b3 + (t & 15);
      const float res = threadIdx.x >= 256 && mr < M ? residual_in(a, l, mr, cr) : 0.f;
      wait_flags(cx, a.fl[1], nP2, cx.tag(l, 1), ident);
      if (b3 == g) RWKV7_TL(tl_rows, l, 7);
      read_rows(s, a.core, C, 0, C, M, true);
      __syncthreads();
      const floatx4 acc = block_mma(s, wb, nksC);
      int m, n;
      const float v = reduce_tile(s, acc, &m, &n);
      if (threadIdx.x >= 256 && m < M && !cx.failed()) rst_f(a.x + (int64_t)m * C + 16 * b3 + n, res + v);
      publish_flag(cx, a.fl[2] + b3, cx.tag(l, 2));
      if (b3 == g) RWKV7_TL(tl_rows, l, 8);
    }
    // ---------------- P4 ----------------
    for (int b4 = g; b4 < nP4; b4 += G) {
      if (b4 == g) RWKV7_TL(tl_rows, l, 9);
      const WBlock wb = load_block(reinterpret_cast<const uint16_t *>(Fp + a.f_fk) + (int64_t)b4 * nksC * 512, 0, nksC);
      load_state(s, a.cmix_x + (int64_t)l * a.B * C, a.B, C);
      const float *lw2 = vec + RWKV7_V_LN2_W * C, *lb2 = vec + RWKV7_V_LN2_B * C, *mu2 = vec + RWKV7_V_FFN_X_K * C;
      MixVec mv{};
      if (threadIdx.x >= 64) mv = load_mix(lw2, lb2, mu2, C);
      wait_flags(cx, a.fl[2], nP3, cx.tag(l, 2), ident);
      if (b4 == g) RWKV7_TL(tl_rows, l, 10);
      read_x(s, a.x, M, C);
      if (threadIdx.x < 64) mv = load_mix(lw2, lb2, mu2, C);
      __syncthreads();
      // the time-mix state of this layer (every o-projection block has published)
      if (b4 == g && slice_owner && !cx.failed()) store_shift_slice(a, s.shs1, a.tmix_x, l, 16 * g);
      row_stats(s, M, C);
      if (b4 == g) RWKV7_TL(tl_rows, l, 11);
      __syncthreads();
      // blocks 0 .. C/16 - 1 also write 16 columns each of the new channel-mix shift state
      build_mix(s, a, C, mv, s.shs2, b4 == g && slice_owner ? 16 * g : -1);
      __syncthreads();
      const floatx4 acc = block_mma(s, wb, nksC);
      if (b4 == g) RWKV7_TL(tl_rows, l, 12);
      int m, n;
      float v = reduce_tile(s, acc, &m, &n);
      v = fmaxf(v, 0.f);
      v = v * v;
      if (threadIdx.x < 256 && m < M && !cx.failed()) rst_f(a.hid + (int64_t)m * F + 16 * b4 + n, v);
      publish_flag(cx, a.fl[3] + b4, cx.tag(l, 3));
      if (b4 == g) RWKV7_TL(tl_rows, l, 13);
    }
    // ---------------- P5 ----------------
    for (int u5 = g; u5 < 4 * nP5; u5 += G) {
      if (u5 == g) RWKV7_TL(tl_rows, l, 14);
      const int b5 = u5 >> 2, q = u5 & 3;
      const int Kq = F / 4;
      const WBlock wb =
          load_block(reinterpret_cast<const uint16_t *>(Fp + a.f_fv) + (int64_t)b5 * nksF * 512, q * nksQ, nksQ);
      const int f0 = q * (nP4 / 4);
      wait_flags(cx, a.fl[3], nP4 / 4, cx.tag(l, 3), [f0](int i) { return f0 + i; });
      if (u5 == g) RWKV7_TL(tl_rows, l, 15);
      // the residual (the o-projection output, final: the P4 blocks waited for it)
      const int t = threadIdx.x & 255;
      const int mr = 4 * ((t & 63) >> 4) + (t >> 6), cr = 16 * b5 + (t & 15);
      const float res = mr < M ? rld_f(a.x + (int64_t)mr * C + cr) : 0.f;
      read_rows(s, a.hid, F, q * Kq, Kq, M, true);
      __syncthreads();
      const floatx4 acc = block_mma(s, wb, nksQ);
      if (u5 == g) RWKV7_TL(tl_rows, l, 16);
      int m, n;
      const float v = reduce_tile(s, acc, &m, &n);
      // split-K hand-off: quarters 1..3 store their partial tiles as tagged
      // words and go on; quarter 0 reads them (each word re-read until it
      // carries this layer's tag), adds them in the order 0, 1, 2, 3 and the
      // residual, and publishes the block
      if (q != 0) {
        if (threadIdx.x < 256 && !cx.failed()) st64f(a.part + ((int64_t)b5 * 4 + q) * 256 + threadIdx.x, v, cx.tag(l, 4));
        __syncthreads();
      } else {
        if (threadIdx.x < 256 && m < M && !cx.failed()) {
          const __amdgpu_buffer_rsrc_t rq = rrsrc(a.part + (int64_t)b5 * 4 * 256, 4 * 256 * 8);
          uint64_t pw[3];
          read_words<3>(cx, rq, cx.tag(l, 4), [](int i) { return 8 * ((1 + i) * 256 + (int)threadIdx.x); }, pw);
          const float sum = ((v + val_f(pw[0])) + val_f(pw[1])) + val_f(pw[2]);
          if (!cx.failed()) rst_f(a.x + (int64_t)m * C + 16 * b5 + n, res + sum);
        }
        publish_flag(cx, a.fl[4] + b5, cx.tag(l, 4));
        if (u5 == g) RWKV7_TL(tl_rows, l, 17);
      }
    }
  }
  // ---------------- the channel-mix state of the last layer, the head ----------------
  const int nb = a.logits ? a.V / 16 : 0;
  WBlock wb = g < nb ? load_block(a.head_frag + (int64_t)g * nksC * 512, 0, nksC) : WBlock{};
  const bool done = wait_flags(cx, a.fl[4], nP5, cx.tag(L - 1, 4), ident);
  if (slice_owner && done) store_shift_slice(a, s.shs2, a.cmix_x, L - 1, 16 * g);
  if (a.logits) {
    const int B = a.B, T = a.T;
    // LN_out of each sequence's last token into A rows 0..B-1
    const __amdgpu_buffer_rsrc_t rx = rrsrc(a.x, (int64_t)a.M * C * 4);
    const int n = B * C / 4;
    floatx4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = threadIdx.x + j * kRT, bb = (4 * i) / C, k = 4 * i - bb * C;
      v[j] = i < n ? rld16f(rx, 4 * ((bb * T + T - 1) * C + k)) : floatx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = threadIdx.x + j * kRT, bb = (4 * i) / C, k = 4 * i - bb * C;
      if (i < n) *reinterpret_cast<floatx4 *>(&s.xs[bb * kRLdX + k]) = v[j];
    }
    __syncthreads();
    row_stats(s, B, C);
    __syncthreads();
    // LN_out in place (f32): thread t < C / 2 owns columns 2t, 2t + 1
    if ((int)threadIdx.x < C / 2) {
      const int k = 2 * threadIdx.x;
      const float w0 = a.ln_out[k], w1 = a.ln_out[k + 1], b0 = a.ln_out[C + k], b1 = a.ln_out[C + k + 1];
      for (int m = 0; m < B; ++m) {
        const float mean = s.stat[4 * m], rs = s.stat[4 * m + 1];
        float2 *xp = reinterpret_cast<float2 *>(s.xs + m * kRLdX + k);
        const float2 x = *xp;
        *xp = make_float2((x.x - mean) * rs * w0 + b0, (x.y - mean) * rs * w1 + b1);
      }
    }
    __syncthreads();
    for (int hb = g; hb < nb; hb += G) {
      // the next block's weights in flight while this one is multiplied
      const WBlock nxt = hb + G < nb ? load_block(a.head_frag + (int64_t)(hb + G) * nksC * 512, 0, nksC) : wb;
      const floatx4 acc = block_mma(s, wb, nksC);
      int m, n;
      const float v = reduce_tile(s, acc, &m, &n);
      if (threadIdx.x < 256 && m < B) a.logits[(int64_t)m * a.V + 16 * hb + n] = done ? f2h(v) : (uint16_t)0x7E00u;
      __syncthreads();
      wb = nxt;
    }
  }
  // The next launch's epoch, stored by workgroup 0 once every workgroup has
  // read this launch's (some workgroups own no block of any stage and would
  // otherwise be able to start after the store and wait on the next launch's
  // tags). A workgroup that never starts while the others run (the grid did
  // not fit at once) cannot be waited for: the bounded wait gives up, the
  // launch counts as aborted.
  if (g == 0 && threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int spins = 0;
    bool all = false;
    while (!all && spins++ < kRSpin) {
      bool ok = true;
      for (int w = lane; w < G; w += 64) ok = ok && rld(a.started + w) == cx.epoch + 1u;
      all = __builtin_amdgcn_ballot_w64(!ok) == 0;
      if (!all) __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) {
      if (!all || cx.aborted() || cx.failed())
        __hip_atomic_fetch_add(a.errors, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      rst(a.sync + RS_EPOCH, cx.epoch + 1u);
    }
  }
}

constexpr int64_t rows_lds_bytes() {
  return 16 * kRLdX * 4 + 16 * kRLdA * 2 + kRW * 256 * 4 + 64 * 4 + 128 + 2 * 256 * 2 + 16 * kRMaxC * 2;
}

// Per device, checked once with that device current: 1 when the kernel's
// dynamic LDS is allowed and a grid of one workgroup per CU fits at once, -1
// when not, 0 before the check.
std::atomic<int> g_rows_resident[64];

}  // namespace

int64_t rows_exchange_bytes(const rwkv7_dims &d) {
  const int64_t C = d.n_embd, F = d.n_ffn, H = d.n_head, SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g;
  const int64_t M = 16;
  auto al = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  int64_t o = kRSyncBytes + al(4 * kRMaxG);
  o += al(4 * 16 * H) + al(4 * (C / 16)) + al(4 * (F / 16)) + al(4 * (C / 16));
  o += al(M * (3 * C + SR) * 8);      // proj
  o += al(M * C * 4);                 // core
  o += al(M * C * 4);                 // x
  o += al(M * F * 4);                 // hid
  o += al((C / 16) * 4 * 256 * 8);    // part
  o += al(M * C * 4);                 // vfirst
  return o;
}

static bool rows_supported(const rwkv7_model &m, int B, int T) {
  const rwkv7_dims &d = m.dims;
  const int C = d.n_embd, F = d.n_ffn;
  if (!m.layers_frag || !m.head_frag || (m.flags & (RWKV7_MODEL_BF16 | RWKV7_MODEL_MULTI_LAUNCH_DECODE))) return false;
  if (B < 1 || T < 1 || B * T > 16) return false;
  if (C > kRMaxC || C % 64 || F % 128 || F > 4 * kRMaxC || d.vocab % 16) return false;
  const int r[4] = {d.rank_v, d.rank_w, d.rank_a, d.rank_g};
  for (int x : r)
    if (x % 16 || x > 128) return false;  // 16-row P1 blocks; P2 holds at most four k-steps per gate
  if (d.rank_w + d.rank_a + d.rank_v + d.rank_g > 320) return false;  // P2 reads 16 x SR / 2 <= 5 kRT chunks
  const int G = mk_cus();
  return G >= C / 16 && G <= kRMaxG;  // workgroup g < C/16 owns P1 and P4 block g
}

// The dynamic LDS is allowed and the grid of one workgroup per CU fits at once
// (checked once per device).
bool rows_usable(const rwkv7_model &m, int B, int T) {
  if (!rows_supported(m, B, T)) return false;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  int r = g_rows_resident[dev].load(std::memory_order_relaxed);
  if (r == 0) {
    const int64_t lds = rows_lds_bytes();
    int per_cu = 0;
    const bool fits =
        hipFuncSetAttribute((const void *)rows_mk_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) ==
            hipSuccess &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)rows_mk_kernel, kRT, (size_t)lds) ==
            hipSuccess &&
        per_cu >= 1;
    r = fits ? 1 : -1;
    g_rows_resident[dev].store(r, std::memory_order_relaxed);
  }
  return r == 1;
}

int launch_rows_mk(const rwkv7_model &m, const rwkv7_layer_layout &lay, const rwkv7_state &s, const int64_t *tok,
                   int T, void *logits, char *xreg, unsigned *errors, hipStream_t st) {
  if (!rows_usable(m, s.batch, T)) return RWKV7_ESHAPE;
  const rwkv7_dims &d = m.dims;
  RkArgs a;
  a.layers = static_cast<const char *>(m.layers);
  a.frag = static_cast<const char *>(m.layers_frag);
  a.lbytes = lay.bytes;
  a.fbytes = lay.frag_bytes;
  a.o_l2 = lay.w_lora2;
  a.o_vec = lay.vec;
  a.f_rkv = lay.f_rkv;
  for (int i = 0; i < 4; ++i) a.f_l1[i] = lay.f_l1[i];
  a.f_o = lay.f_o;
  a.f_fk = lay.f_fk;
  a.f_fv = lay.f_fv;
  a.emb = static_cast<const uint16_t *>(m.emb);
  a.head_frag = static_cast<const uint16_t *>(m.head_frag);
  a.ln_out = static_cast<const float *>(m.ln_out);
  a.L = d.n_layer;
  a.C = d.n_embd;
  a.H = d.n_head;
  a.F = d.n_ffn;
  a.V = d.vocab;
  a.rv = d.rank_v;
  a.rw = d.rank_w;
  a.ra = d.rank_a;
  a.rg = d.rank_g;
  a.SR = d.rank_w + d.rank_a + d.rank_v + d.rank_g;
  a.tmix_x = static_cast<uint16_t *>(s.tmix_x);
  a.rnn = static_cast<float *>(s.rnn);
  a.cmix_x = static_cast<uint16_t *>(s.cmix_x);
  a.tok = tok;
  a.logits = static_cast<uint16_t *>(logits);
  a.B = s.batch;
  a.T = T;
  a.M = s.batch * T;
  a.G = mk_cus();
  const int64_t C = a.C, F = a.F, H = a.H, SR = a.SR, M = 16;
  auto al = [](int64_t x) { return (x + 255) & ~int64_t(255); };
  char *p = xreg;
  a.sync = reinterpret_cast<unsigned *>(p);
  p += kRSyncBytes;
  a.started = reinterpret_cast<unsigned *>(p);
  p += al(4 * kRMaxG);
  const int64_t nfl[5] = {0, 16 * H, C / 16, F / 16, C / 16};
  for (int i = 0; i < 5; ++i) {
    a.fl[i] = reinterpret_cast<unsigned *>(p);
    p += al(4 * nfl[i]);
  }
  a.proj = reinterpret_cast<uint64_t *>(p);
  p += al(M * (3 * C + SR) * 8);
  a.core = reinterpret_cast<float *>(p);
  p += al(M * C * 4);
  a.x = reinterpret_cast<float *>(p);
  p += al(M * C * 4);
  a.hid = reinterpret_cast<float *>(p);
  p += al(M * F * 4);
  a.part = reinterpret_cast<uint64_t *>(p);
  p += al((C / 16) * 4 * 256 * 8);
  a.vfirst = reinterpret_cast<float *>(p);
  p += al(M * C * 4);
  a.errors = errors;
  rows_mk_kernel<<<a.G, kRT, rows_lds_bytes(), st>>>(a);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

}  // namespace rwkv7

RWKV7_TL_READER(rwkv7_timeline_read_rows, rwkv7::tl_rows);
