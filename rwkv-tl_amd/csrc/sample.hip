// Token sampling on the device: repetition penalty, greedy argmax,
// temperature, top-k, top-p and the random draw for each row of logits, in
// one launch (semantics of demo/sampling.py:13-70).
//
// One 1024-thread workgroup per row; thread t holds logits [64 t, 64 t + 64)
// (f16 or f32 in memory, f32 in registers; V <= 65536), so the row is read
// from HBM once.
//
// * Thresholds. top-k keeps x >= the k-th largest value (ties kept, as
//   torch.topk's cutoff with `>=`); top-p keeps x >= the largest value y whose
//   inclusive mass sum_{x_j >= y} p_j exceeds top_p (the token at which the
//   descending cumulative mass first passes top_p is the last one kept, as in
//   sampling.py:62-68). Both are "largest value y with weight(x >= y) > W"
//   and are found exactly, without sorting: one pass of 256 equal-width bins
//   over [min, max] (the bin index is a monotone function of x), then radix
//   passes of up to 8 bits over the order-preserving integer key of x inside
//   the chosen bin, until one value remains.
// * Mass. exp(x - max) is summed in 64-bit fixed point (scale 2^40), so every
//   sum is exact and the result does not depend on summation order.
// * Draw. One Philox4x32-10 block (Salmon et al., "Parallel random numbers:
//   as easy as 1, 2, 3", SC'11) per row: key = seed, counter = (offset, row,
//   0). Its first 64 bits r pick target = floor(Z r / 2^64) in [0, Z), and the
//   token is the first index (vocabulary order) whose inclusive prefix of kept
//   mass exceeds target: inverse-CDF sampling of the kept distribution.
#include "rwkv7_common.h"

namespace rwkv7 {
namespace {

typedef unsigned long long u64;

constexpr int kSmpThreads = 1024;
constexpr int kSmpWaves = kSmpThreads / kWave;
constexpr int kSmpE = 64;                      // logits per thread
constexpr int kSmpMaxV = kSmpThreads * kSmpE;  // 65536
constexpr float kFix = 1099511627776.0f;       // 2^40
constexpr float kInf = __builtin_inff();
constexpr int kCandCap = 4096;                 // LDS candidates of a threshold's bin

struct SampleArgs {
  const void *logits;
  int64_t ld;
  int V;
  float temp, top_p, pen;
  int top_k;
  uint32_t seed_lo, seed_hi, off_lo, off_hi;
  uint32_t *seen;
  int64_t seen_ld;
  int update_seen;
  int64_t *out;
  float *probs;
  int64_t probs_ld;
};

struct SampleLds {
  u64 hist[256];
  u64 wu[kSmpWaves];
  float wa[kSmpWaves], wb[kSmpWaves];
  int wi[kSmpWaves];
  u64 cross_above;
  int cross_bin;
  int ncand;
  float cand[kCandCap];
};

RWKV7_DEV uint32_t okey(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
RWKV7_DEV float okey_inv(uint32_t k) { return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k); }

RWKV7_DEV u64 shfl_xor64(u64 v, int m) {
  const int lo = __shfl_xor((int)(uint32_t)v, m), hi = __shfl_xor((int)(uint32_t)(v >> 32), m);
  return (u64)(uint32_t)lo | ((u64)(uint32_t)hi << 32);
}
RWKV7_DEV u64 shfl_up64(u64 v, int d) {
  const int lo = __shfl_up((int)(uint32_t)v, d), hi = __shfl_up((int)(uint32_t)(v >> 32), d);
  return (u64)(uint32_t)lo | ((u64)(uint32_t)hi << 32);
}
RWKV7_DEV u64 shfl_down64(u64 v, int d) {
  const int lo = __shfl_down((int)(uint32_t)v, d), hi = __shfl_down((int)(uint32_t)(v >> 32), d);
  return (u64)(uint32_t)lo | ((u64)(uint32_t)hi << 32);
}

// The compiler would otherwise keep per-element values (64 u64 weights, 64
// keys) live from one pass to the next instead of recomputing them from the 64
// logits, which overflows the 128 VGPRs of a 1024-thread workgroup: each pass
// reads its constants through this opaque copy.
RWKV7_DEV float opaque(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

RWKV7_DEV u64 mass(float x, float m) { return (u64)(__expf(x - m) * kFix); }

RWKV7_DEV bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// Block (max value, lowest index among ties); every thread gets the result.
RWKV7_DEV void block_argmax(float &v, int &i, SampleLds &s) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    const float ov = __shfl_xor(v, m);
    const int oi = __shfl_xor(i, m);
    if (better(ov, oi, v, i)) v = ov, i = oi;
  }
  const int w = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) s.wa[w] = v, s.wi[w] = i;
  __syncthreads();
  v = s.wa[0], i = s.wi[0];
  for (int j = 1; j < kSmpWaves; ++j)
    if (better(s.wa[j], s.wi[j], v, i)) v = s.wa[j], i = s.wi[j];
  __syncthreads();
}

RWKV7_DEV void block_minmax(float &lo, float &hi, SampleLds &s) {
#pragma unroll
  for (int m = 1; m < kWave; m <<= 1) {
    lo = fminf(lo, __shfl_xor(lo, m));
    hi = fmaxf(hi, __shfl_xor(hi, m));
  }
  const int w = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) s.wa[w] = lo, s.wb[w] = hi;
  __syncthreads();
  lo = s.wa[0], hi = s.wb[0];
  for (int j = 1; j < kSmpWaves; ++j) lo = fminf(lo, s.wa[j]), hi = fmaxf(hi, s.wb[j]);
  __syncthreads();
}

// Exclusive prefix of x over the block in thread order, and the block total.
RWKV7_DEV u64 block_excl_scan(u64 x, u64 &total, SampleLds &s) {
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  u64 inc = x;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const u64 o = shfl_up64(inc, d);
    if (lane >= d) inc += o;
  }
  if (lane == kWave - 1) s.wu[w] = inc;
  __syncthreads();
  u64 base = 0, tot = 0;
  for (int j = 0; j < kSmpWaves; ++j) {
    const u64 o = s.wu[j];
    base += j < w ? o : 0ull;
    tot += o;
  }
  __syncthreads();
  total = tot;
  return base + inc - x;
}

// Over s.hist, the largest bin b with above + sum_{b' >= b} hist[b'] > W.
// Sets s.cross_bin = b (-1 if none) and s.cross_above = above + sum_{b' > b}.
RWKV7_DEV void find_cross(SampleLds &s, u64 above, u64 W) {
  if (threadIdx.x < kWave) {
    const int L = threadIdx.x;
    const u64 h[4] = {s.hist[4 * L], s.hist[4 * L + 1], s.hist[4 * L + 2], s.hist[4 * L + 3]};
    const u64 own = (h[0] + h[1]) + (h[2] + h[3]);
    u64 suf = own;  // sum over bins >= 4 L
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const u64 o = shfl_down64(suf, d);
      if (L + d < kWave) suf += o;
    }
    // suf does not increase with L, so the lanes that pass form a prefix
    const u64 mask = __ballot(above + suf > W);
    if (mask == 0) {
      if (L == 0) s.cross_bin = -1;
    } else if (L == 63 - __clzll(mask)) {
      u64 acc = above + suf - own;  // <= W: the lane above failed
      int b = 4 * L;
      for (int j = 3; j >= 0; --j) {
        if (acc + h[j] > W) {
          b = 4 * L + j;
          break;
        }
        acc += h[j];
      }
      s.cross_bin = b;
      s.cross_above = acc;
    }
  }
  __syncthreads();
}

// Largest value y among the elements x >= lo (lo > -inf; hi their maximum) with
// sum over x >= y of wt(x) > W, where wt(x) = 1 (MASS false) or mass(x, m).
// If the total is <= W, lo. Each thread holds E elements (-inf: none).
//
// One pass of 256 equal-width bins over [lo, hi] picks the bin that holds y;
// its elements are copied to LDS (when there are at most kCandCap of them),
// and radix passes of up to 8 bits over their order-preserving keys narrow the
// key range to one value. A larger bin is narrowed the same way straight from
// the registers.
template <bool MASS, int E>
RWKV7_DEV float select_gt(const float (&l)[E], float lo, float hi, float m, u64 W, SampleLds &s) {
  auto wt = [](float x, float mm) -> u64 { return MASS ? mass(x, mm) : 1ull; };
  if (!(lo < hi)) return lo;
  // pass 0: equal-width bins over [lo, hi]
  const float scale = fminf(256.f / (hi - lo), 3.0e38f);  // finite, so (lo - lo) * scale == 0
  auto lbin = [](float x, float o, float sc) { return (int)fminf(255.f, (x - o) * sc); };
  for (int i = threadIdx.x; i < 256; i += kSmpThreads) s.hist[i] = 0;
  if (threadIdx.x == 0) s.ncand = 0;
  __syncthreads();
  {
    const float mo = opaque(m);
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (l[e] > -kInf && l[e] >= lo) atomicAdd(&s.hist[lbin(l[e], lo, scale)], wt(l[e], mo));
  }
  __syncthreads();
  find_cross(s, 0, W);
  const int b0 = s.cross_bin;
  if (b0 < 0) return lo;
  u64 above = s.cross_above;
  // the elements of bin b0: their range, and a copy in LDS
  float nlo = kInf, nhi = -kInf;
  {
    const float lo2 = opaque(lo), sc2 = opaque(scale);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (l[e] > -kInf && l[e] >= lo2 && lbin(l[e], lo2, sc2) == b0) {
        nlo = fminf(nlo, l[e]), nhi = fmaxf(nhi, l[e]);
        const int slot = atomicAdd(&s.ncand, 1);
        if (slot < kCandCap) s.cand[slot] = l[e];
      }
    }
  }
  block_minmax(nlo, nhi, s);  // its barriers order the copy and the cross_bin reads before what follows
  const int ncand = s.ncand;
  const bool from_lds = ncand <= kCandCap;  // block-uniform
  // radix passes over the keys in [kl, kh]: the elements of bin b0
  uint32_t kl = okey(nlo), kh = okey(nhi);
  while (kl != kh) {
    const int top = 31 - __clz(kl ^ kh);  // highest differing bit
    const int sh = max(0, top - 7);
    const uint32_t dmask = (1u << (top - sh + 1)) - 1u;
    for (int i = threadIdx.x; i < 256; i += kSmpThreads) s.hist[i] = 0;
    __syncthreads();
    const float zero = opaque(0.f), mo = opaque(m);
    if (from_lds) {
      for (int i = threadIdx.x; i < ncand; i += kSmpThreads) {
        const float x = s.cand[i];
        const uint32_t k = okey(x);
        if (k >= kl && k <= kh) atomicAdd(&s.hist[(k >> sh) & dmask], wt(x, mo));
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const uint32_t k = okey(l[e] + zero);  // + 0 keeps the value (no -0 is left)
        if (l[e] > -kInf && k >= kl && k <= kh) atomicAdd(&s.hist[(k >> sh) & dmask], wt(l[e], mo));
      }
    }
    __syncthreads();
    find_cross(s, above, W);
    const int b = s.cross_bin;
    above = s.cross_above;
    __syncthreads();
    if (b < 0) break;  // unreachable: above <= W < above + weight([kl, kh]) holds here
    const uint32_t keep_hi = top == 31 ? 0u : (0xffffffffu << (top + 1));
    const uint32_t nl = (kl & keep_hi) | ((uint32_t)b << sh);
    const uint32_t nh = nl | ((1u << sh) - 1u);
    kl = max(kl, nl);
    kh = min(kh, nh);
  }
  return okey_inv(kl);
}

RWKV7_DEV void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const u64 p0 = (u64)0xD2511F53u * c[0], p1 = (u64)0xCD9E8D57u * c[2];
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    c[0] = n0, c[1] = (uint32_t)p1, c[2] = n2, c[3] = (uint32_t)p0;
    k0 += 0x9E3779B9u, k1 += 0xBB67AE85u;
  }
}

// Logits 8..8c+7 of this thread's 64, as f32 (-inf past V). VEC: rows
// 16-byte aligned and V % 8 == 0, so each 8-logit chunk is whole 16-byte
// loads or wholly past V. FMT: 0 half, 1 f32, 2 bfloat16.
template <bool VEC, int FMT>
RWKV7_DEV void load8(const void *row_ptr, int i0, int V, float *f) {
  constexpr bool F32 = FMT == 1, BF = FMT == 2;
  if (VEC) {
    if (F32) {
      const float4 *p = reinterpret_cast<const float4 *>(static_cast<const float *>(row_ptr) + i0);
      const float4 u = i0 < V ? p[0] : make_float4(-kInf, -kInf, -kInf, -kInf);
      const float4 v = i0 < V ? p[1] : make_float4(-kInf, -kInf, -kInf, -kInf);
      f[0] = u.x, f[1] = u.y, f[2] = u.z, f[3] = u.w, f[4] = v.x, f[5] = v.y, f[6] = v.z, f[7] = v.w;
    } else {
      const uint32_t ninf2 = BF ? 0xff80ff80u : 0xfc00fc00u;  // two 16-bit -inf
      const uint4 u = i0 < V ? *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(row_ptr) + i0)
                             : make_uint4(ninf2, ninf2, ninf2, ninf2);
      F16T<BF>::to_f8(u, f);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0 + j;
      f[j] = i >= V  ? -kInf
             : F32 ? static_cast<const float *>(row_ptr)[i]
                   : F16T<BF>::to_f(static_cast<const uint16_t *>(row_ptr)[i]);
    }
  }
}

// Temperature-scaled sampling of one row from the E values each thread holds
// (-inf: none), the threads' values in vocabulary order thread by thread;
// idx(e) is the vocabulary index of this thread's e-th value. Top-k, top-p,
// the kept mass and the draw as described at the top; pr (optional) receives
// the kept distribution at the indices held. Returns the token on the one
// thread that draws it, -1 on the others.
// The top-p threshold when at most kWave values are kept: the largest kept
// value y with sum_{x >= y} mass(x) > W is the value at the first position
// of the descending order whose running mass exceeds W (a tie group's
// members share the value, so where in the group that position falls does
// not matter). The kept values are compacted to LDS, and wave 0 sorts them
// (bitonic, one per lane), forms the running masses and picks that value.
// Returns false (and does nothing else) when more values are kept.
template <int E>
RWKV7_DEV bool top_p_in_wave(const float (&l)[E], float m, float top_p, float &thr, SampleLds &s) {
  int own = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) own += l[e] > -kInf;
  u64 total;
  int at = (int)block_excl_scan((u64)own, total, s);
  if (total > (u64)kWave) return false;  // block-uniform
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (l[e] > -kInf) s.cand[at++] = l[e];
  __syncthreads();
  if (threadIdx.x < kWave) {
    const int L = threadIdx.x;
    float v = L < (int)total ? s.cand[L] : -kInf;
    const float mo = opaque(m);
    u64 z = v > -kInf ? mass(v, mo) : 0ull;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) z += shfl_xor64(z, d);
    const u64 W = (u64)((double)top_p * (double)z);
#pragma unroll
    for (int k = 2; k <= kWave; k <<= 1) {  // descending bitonic sort over the lanes
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        const float o = __shfl_xor(v, j);
        const bool take_max = ((L & j) == 0) == ((L & k) == 0);
        v = take_max ? fmaxf(v, o) : fminf(v, o);
      }
    }
    u64 c = v > -kInf ? mass(v, mo) : 0ull;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const u64 o = shfl_up64(c, d);
      if (L >= d) c += o;
    }
    const u64 pass = __ballot(c > W);  // nonzero: the last lane holds z > W
    const int first = __ffsll((unsigned long long)pass) - 1;
    const float y = __shfl(v, first);
    if (L == 0) s.wa[0] = y;
  }
  __syncthreads();
  thr = s.wa[0];
  __syncthreads();
  return true;
}

// FLOOR: before the top-k selection, bound the k-th largest value from below
// by the k-th largest of the threads' maxima (a saving when every thread holds
// many values, as in the one-workgroup kernel).
template <int E, bool FLOOR, class Idx>
RWKV7_DEV int draw_tempered(float (&l)[E], Idx idx, const SampleArgs &a, int row, float *pr, SampleLds &s) {
  const int V = a.V;
  float lo = kInf, m = -kInf, tmax = -kInf;
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (l[e] > -kInf) lo = fminf(lo, l[e]), tmax = fmaxf(tmax, l[e]);
  m = tmax;
  block_minmax(lo, m, s);
  float thr = -kInf;  // tokens with x >= thr stay
  bool small = false;  // at most kWave tokens left after top-k
  if (a.top_k > 0 && a.top_k < V) {  // sampling.py:56-60
    // The k-th largest value is at least the k-th largest of the threads'
    // maxima when k threads hold values: only values from there up take part.
    float floor_k = lo;
    if (FLOOR && __syncthreads_count(tmax > -kInf) >= a.top_k) {
      float tl = tmax > -kInf ? tmax : kInf, th = tmax;
      block_minmax(tl, th, s);
      const float tv[1] = {tmax};
      floor_k = select_gt<false, 1>(tv, tl, th, m, (u64)(a.top_k - 1), s);
    }
    thr = select_gt<false, E>(l, floor_k, m, m, (u64)(a.top_k - 1), s);
    lo = thr;  // the smallest value top-k keeps
    small = a.top_k <= kWave;
  }
  if (a.top_p < 1.f) {  // sampling.py:62-68
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (l[e] < thr) l[e] = -kInf;
    float tp;
    if (small && top_p_in_wave<E>(l, m, a.top_p, tp, s)) {
      thr = tp;
    } else {
      u64 own = 0, z = 0;
      const float mo = opaque(m);
#pragma unroll
      for (int e = 0; e < E; ++e)
        if (l[e] > -kInf) own += mass(l[e], mo);
      block_excl_scan(own, z, s);
      thr = select_gt<true, E>(l, lo, m, m, (u64)((double)a.top_p * (double)z), s);
    }
  }
  u64 own = 0, z = 0;
  {
    const float m1 = opaque(m);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (l[e] < thr) l[e] = -kInf;
      if (l[e] > -kInf) own += mass(l[e], m1);
    }
  }
  const u64 excl = block_excl_scan(own, z, s);
  uint32_t c[4] = {a.off_lo, a.off_hi, (uint32_t)row, 0u};
  philox4x32_10(c, a.seed_lo, a.seed_hi);
  const u64 target = __umul64hi(z, (u64)c[0] | ((u64)c[1] << 32));  // in [0, z)
  int token = -1;  // exactly one thread finds it: z >= 2^40, since the maximum is always kept
  if (excl <= target && target < excl + own) {
    u64 acc = excl;
    const float m2 = opaque(m);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      if (l[e] > -kInf) acc += mass(l[e], m2);
      if (token < 0 && acc > target) token = idx(e);
    }
  }
  if (pr) {
    const float inv = 1.f / (float)z, m3 = opaque(m);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = idx(e);
      if (i < V) pr[i] = l[e] > -kInf ? (float)mass(l[e], m3) * inv : 0.f;
    }
  }
  return token;
}

// The whole row on one workgroup (thread t holds logits 64 t .. 64 t + 63).
// Returns the token on the thread that holds it (every thread for greedy).
template <bool VEC, int FMT>
RWKV7_DEV int sample_row(const SampleArgs &a, int row, SampleLds &s) {
  const int base = threadIdx.x * kSmpE, V = a.V;
  const void *src = static_cast<const char *>(a.logits) + (int64_t)row * a.ld * (FMT == 1 ? 4 : 2);
  float l[kSmpE];
#pragma unroll
  for (int c = 0; c < kSmpE / 8; ++c) load8<VEC, FMT>(src, base + 8 * c, V, &l[8 * c]);
  // repetition penalty (sampling.py:44-47), applied once per seen token
  if (a.seen && a.pen != 1.f) {
    const uint32_t *sr = a.seen + (int64_t)row * a.seen_ld;
    const int nw = (V + 31) / 32;
    const uint32_t m0 = 2 * threadIdx.x < nw ? sr[2 * threadIdx.x] : 0u;
    const uint32_t m1 = 2 * threadIdx.x + 1 < nw ? sr[2 * threadIdx.x + 1] : 0u;
#pragma unroll
    for (int e = 0; e < kSmpE; ++e) {
      if (((e < 32 ? m0 : m1) >> (e & 31)) & 1u) l[e] = l[e] > 0.f ? l[e] / a.pen : l[e] * a.pen;
    }
  }
#pragma unroll
  for (int e = 0; e < kSmpE; ++e) l[e] = l[e] + 0.f;  // -0 -> +0: one key per value

  float *pr = a.probs ? a.probs + (int64_t)row * a.probs_ld : nullptr;
  if (!(a.temp > 0.f)) {
    // greedy: argmax, first index among ties (sampling.py:49-50)
    float v = -kInf;
    int vi = 0x7fffffff;
#pragma unroll
    for (int e = 0; e < kSmpE; ++e)
      if (better(l[e], base + e, v, vi)) v = l[e], vi = base + e;
    block_argmax(v, vi, s);
    const int token = vi < V ? vi : 0;  // only a row of NaNs leaves vi past V
    if (pr) {
#pragma unroll
      for (int e = 0; e < kSmpE; ++e)
        if (base + e < V) pr[base + e] = base + e == token ? 1.f : 0.f;
    }
    return threadIdx.x == 0 ? token : -1;
  }
#pragma unroll
  for (int e = 0; e < kSmpE; ++e) l[e] = l[e] / a.temp;
  return draw_tempered<kSmpE, true>(l, [base](int e) { return base + e; }, a, row, pr, s);
}

RWKV7_DEV void put_token(const SampleArgs &a, int row, int token) {
  if (token >= 0) {
    a.out[row] = token;
    if (a.update_seen) atomicOr(a.seen + (int64_t)row * a.seen_ld + token / 32, 1u << (token % 32));
  }
}

template <bool VEC, int FMT>
__global__ __launch_bounds__(kSmpThreads) void sample_kernel(SampleArgs a) {
  __shared__ SampleLds s;
  put_token(a, blockIdx.x, sample_row<VEC, FMT>(a, blockIdx.x, s));
}

// ---------------------------------------------------------------------------
// Top-k over many CUs (temperature > 0, 1 <= top_k <= kCandMax, no probs):
// every token top-k keeps is among the top_k largest of its own slice of the
// row, so the row is cut into slices of kCandSlice logits, each workgroup of
// sample_cand_kernel keeps the values of its slice >= the slice's top_k-th
// largest (ties included; exact, by the same selection as above) in index
// order, and sample_finish_kernel runs draw_tempered on those candidates,
// which hold the same values at the same vocabulary positions as the
// one-workgroup kernel would: the thresholds, the fixed-point masses, the
// draw and therefore the token are identical. A slice with more than
// kCandMax candidates (a tie group at its threshold) marks its count -1, and
// the row is sampled by sample_row instead.
// ---------------------------------------------------------------------------
constexpr int kCandSlice = 2 * kSmpThreads;  // 2 logits per thread
constexpr int kCandMax = 128;                // candidates kept per slice
constexpr int kCandSlices = kSmpMaxV / kCandSlice;
constexpr int kCandE = kCandSlices * kCandMax / kSmpThreads;  // candidates per thread in the finish

struct CandBuf {
  int *cnt;     // [B][G]: candidates of each slice, -1 when more than kCandMax
  float *val;   // [B][G][kCandMax]
  int *idx;     // [B][G][kCandMax]
  int G;
};

template <int FMT>
RWKV7_DEV float load1(const void *row_ptr, int i) {
  if (FMT == 1) return static_cast<const float *>(row_ptr)[i];
  return F16T<FMT == 2>::to_f(static_cast<const uint16_t *>(row_ptr)[i]);
}

template <int FMT>
__global__ __launch_bounds__(kSmpThreads) void sample_cand_kernel(SampleArgs a, CandBuf cb) {
  __shared__ SampleLds s;
  const int g = blockIdx.x, row = blockIdx.y, V = a.V;
  const void *src = static_cast<const char *>(a.logits) + (int64_t)row * a.ld * (FMT == 1 ? 4 : 2);
  const int i0 = g * kCandSlice + 2 * threadIdx.x;
  float l[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) l[e] = i0 + e < V ? load1<FMT>(src, i0 + e) : -kInf;
  if (a.seen && a.pen != 1.f) {  // the same operations, in the same order, as sample_row
    const uint32_t *sr = a.seen + (int64_t)row * a.seen_ld;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = i0 + e;
      if (i < V && ((sr[i >> 5] >> (i & 31)) & 1u)) l[e] = l[e] > 0.f ? l[e] / a.pen : l[e] * a.pen;
    }
  }
#pragma unroll
  for (int e = 0; e < 2; ++e) l[e] = (l[e] + 0.f) / a.temp;
  float lo = kInf, hi = -kInf;
#pragma unroll
  for (int e = 0; e < 2; ++e)
    if (l[e] > -kInf) lo = fminf(lo, l[e]), hi = fmaxf(hi, l[e]);
  block_minmax(lo, hi, s);
  // the slice's top_k-th largest value (lo when it holds fewer values)
  const float u = select_gt<false, 2>(l, lo, hi, hi, (u64)(a.top_k - 1), s);
  bool keep[2];
  int own = 0;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    keep[e] = l[e] > -kInf && l[e] >= u;
    own += keep[e];
  }
  u64 total;
  int at = (int)block_excl_scan((u64)own, total, s);
  const int64_t slot = (int64_t)row * cb.G + g;
  if (threadIdx.x == 0) cb.cnt[slot] = total <= (u64)kCandMax ? (int)total : -1;
  if (total <= (u64)kCandMax) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      if (keep[e]) {
        cb.val[slot * kCandMax + at] = l[e];
        cb.idx[slot * kCandMax + at] = i0 + e;
        ++at;
      }
    }
  }
}

template <bool VEC, int FMT>
__global__ __launch_bounds__(kSmpThreads) void sample_finish_kernel(SampleArgs a, CandBuf cb) {
  __shared__ SampleLds s;
  __shared__ int s_off[kCandSlices + 1];
  __shared__ int s_bad;
  const int row = blockIdx.x, G = cb.G;
  if (threadIdx.x < kWave) {  // slice offsets: inclusive prefix of the counts
    const int L = threadIdx.x;
    const int c = L < G ? cb.cnt[(int64_t)row * G + L] : 0;
    int inc = c < 0 ? 0 : c;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int o = __shfl_up(inc, d);
      if (L >= d) inc += o;
    }
    const bool bad = __ballot(c < 0) != 0;
    if (L <= kCandSlices - 1) s_off[L + 1] = inc;
    if (L == 0) {
      s_off[0] = 0;
      s_bad = bad;
    }
  }
  __syncthreads();
  if (s_bad) {  // a tie group overflowed a slice: the whole row here
    put_token(a, row, sample_row<VEC, FMT>(a, row, s));
    return;
  }
  const int n = s_off[G];
  float l[kCandE];
  int ix[kCandE];
#pragma unroll
  for (int e = 0; e < kCandE; ++e) {
    const int d = kCandE * threadIdx.x + e;
    l[e] = -kInf;
    ix[e] = a.V;
    if (d < n) {
      int g = 0;
      while (g + 1 < G && s_off[g + 1] <= d) ++g;
      const int64_t at = ((int64_t)row * G + g) * kCandMax + (d - s_off[g]);
      l[e] = cb.val[at];
      ix[e] = cb.idx[at];
    }
  }
  put_token(a, row, draw_tempered<kCandE, false>(l, [&ix](int e) { return ix[e]; }, a, row, nullptr, s));
}

}  // namespace
}  // namespace rwkv7

static int64_t cand_bytes(int B, int G) {
  auto al = [](int64_t x) { return (x + 255) / 256 * 256; };
  return al((int64_t)B * G * 4) + 2 * al((int64_t)B * G * rwkv7::kCandMax * 4);
}

extern "C" int64_t rwkv7_sample_workspace_bytes(int32_t B, int32_t V) {
  using namespace rwkv7;
  if (B < 1 || V < 1 || V > kSmpMaxV) return 0;
  return cand_bytes(B, (V + kCandSlice - 1) / kCandSlice);
}

extern "C" int rwkv7_sample(const void *logits, int32_t logits_dtype, int64_t ld, int32_t B, int32_t V, const rwkv7_sampling *p,
                            uint32_t *seen, int64_t seen_ld, int32_t update_seen, int64_t *out, float *probs,
                            int64_t probs_ld, void *workspace, int64_t workspace_bytes, void *stream) {
  using namespace rwkv7;
  if (!logits || !p || !out || B < 1 || (update_seen && !seen)) return RWKV7_EINVAL;
  if (logits_dtype < 0 || logits_dtype > 2) return RWKV7_EINVAL;
  if (V < 1 || V > kSmpMaxV || ld < V || (seen && seen_ld < (V + 31) / 32) || (probs && probs_ld < V))
    return RWKV7_ESHAPE;
  SampleArgs a;
  a.logits = logits;
  a.ld = ld;
  a.V = V;
  a.temp = p->temperature;
  a.top_p = p->top_p;
  a.pen = p->repetition_penalty;
  a.top_k = p->top_k;
  a.seed_lo = (uint32_t)p->seed, a.seed_hi = (uint32_t)(p->seed >> 32);
  a.off_lo = (uint32_t)p->offset, a.off_hi = (uint32_t)(p->offset >> 32);
  a.seen = seen;
  a.seen_ld = seen_ld;
  a.update_seen = update_seen;
  a.out = out;
  a.probs = probs;
  a.probs_ld = probs_ld;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = reinterpret_cast<uintptr_t>(logits) % 16 == 0 && ld % 8 == 0 && V % 8 == 0;
  const int G = (V + kCandSlice - 1) / kCandSlice;
  const bool cand = workspace && workspace_bytes >= cand_bytes(B, G) && a.temp > 0.f && a.top_k >= 1 &&
                    a.top_k <= kCandMax && a.top_k < V && !probs && G >= 2;
  if (cand) {
    char *w = static_cast<char *>(workspace);
    const int64_t c0 = cand_bytes(B, G) - 2 * (((int64_t)B * G * kCandMax * 4 + 255) / 256 * 256);
    CandBuf cb;
    cb.cnt = reinterpret_cast<int *>(w);
    cb.val = reinterpret_cast<float *>(w + c0);
    cb.idx = reinterpret_cast<int *>(w + c0 + ((int64_t)B * G * kCandMax * 4 + 255) / 256 * 256);
    cb.G = G;
    switch (logits_dtype) {
      case 0: sample_cand_kernel<0><<<dim3(G, B), kSmpThreads, 0, st>>>(a, cb); break;
      case 1: sample_cand_kernel<1><<<dim3(G, B), kSmpThreads, 0, st>>>(a, cb); break;
      default: sample_cand_kernel<2><<<dim3(G, B), kSmpThreads, 0, st>>>(a, cb); break;
    }
    RWKV7_CHECK_LAUNCH();
    switch (logits_dtype) {
      case 0: vec ? sample_finish_kernel<true, 0><<<B, kSmpThreads, 0, st>>>(a, cb) : sample_finish_kernel<false, 0><<<B, kSmpThreads, 0, st>>>(a, cb); break;
      case 1: vec ? sample_finish_kernel<true, 1><<<B, kSmpThreads, 0, st>>>(a, cb) : sample_finish_kernel<false, 1><<<B, kSmpThreads, 0, st>>>(a, cb); break;
      default: vec ? sample_finish_kernel<true, 2><<<B, kSmpThreads, 0, st>>>(a, cb) : sample_finish_kernel<false, 2><<<B, kSmpThreads, 0, st>>>(a, cb); break;
    }
    RWKV7_CHECK_LAUNCH();
    return RWKV7_OK;
  }
  switch (logits_dtype) {
    case 0: vec ? sample_kernel<true, 0><<<B, kSmpThreads, 0, st>>>(a) : sample_kernel<false, 0><<<B, kSmpThreads, 0, st>>>(a); break;
    case 1: vec ? sample_kernel<true, 1><<<B, kSmpThreads, 0, st>>>(a) : sample_kernel<false, 1><<<B, kSmpThreads, 0, st>>>(a); break;
    default: vec ? sample_kernel<true, 2><<<B, kSmpThreads, 0, st>>>(a) : sample_kernel<false, 2><<<B, kSmpThreads, 0, st>>>(a); break;
  }
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}
