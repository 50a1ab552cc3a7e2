// Time-mix (TMIX) kernels: the wkv7 DPLR recurrence and everything fused
// around it, plus the small elementwise stages of decode and prefill.
//
// wkv7 state: S[h] is 64x64 fp32, S[h][i][j] with i the value row and j the
// key column (src/rwkv_tl/state.py:37-41). One step (demo/rwkv7_torch.py:49-64):
//   sa_i  = sum_j S_ij a_j
//   S'_ij = S_ij w_j + sa_i b_j + v_i k_j
//   y_i   = sum_j S'_ij r_j
// Rows are independent given the step's (w, a, b, k, r), so a head's rows can
// be spread over lanes and workgroups freely; every reduction is along j.
#include <type_traits>

#include "rwkv7_kernels.h"

namespace rwkv7 {

// ---------------------------------------------------------------------------
// Decode: one token per sequence, grid (H, B), 256 threads.
// LoRA second step + gates + L2 norm + wkv7 + GroupNorm + r.k.r_k bonus +
// output gate. Stands in for fused_gates / fused_l2norm_neg_kk_a / fused_dplr /
// fused_gn_rkrk (src/rwkv_tl/kernels/gates.py:315-357, dplr.py:229-270) and
// the gate multiply (demo/_rwkv7_base.py:206).
// ---------------------------------------------------------------------------


constexpr int kMaxRanks = 512;  // SR = rv + rw + ra + rg of the batched decode core

template <bool BF>
__global__ __launch_bounds__(256) void tmix_decode_kernel(TmixDecodeArgs a) {
  using T16 = F16T<BF>;
  __shared__ float s_lora[kMaxRanks];
  __shared__ float s_d[4][kN];
  __shared__ float s_r[kN], s_w[kN], s_k[kN], s_v[kN], s_a[kN], s_b[kN], s_g[kN], s_y[kN];
  __shared__ float s_rk;

  const int t = threadIdx.x;
  const int h = blockIdx.x, b = blockIdx.y;
  const int C = a.C;
  const int SR = a.rv + a.rw + a.ra + a.rg;
  const float *prow = a.proj + (int64_t)b * a.ldp;
  const float *vec = a.vec;

  for (int i = t; i < SR; i += 256) {
    float x = prow[3 * C + i];
    if (i >= a.rv && i < a.rv + a.rw) x = tanhf(x);
    else if (i >= a.rv + a.rw + a.ra) x = sigmoidf_(x);
    s_lora[i] = x;
  }
  __syncthreads();

  {  // LoRA second step: thread -> (gate q, channel c)
    const int c = t & (kN - 1), q = t >> 6;
    const int off = q == 0 ? 0 : q == 1 ? a.rv : q == 2 ? a.rv + a.rw : a.rv + a.rw + a.ra;
    const int R = q == 0 ? a.rv : q == 1 ? a.rw : q == 2 ? a.ra : a.rg;
    const uint4 *wr = reinterpret_cast<const uint4 *>(a.w_lora2 + (int64_t)(h * kN + c) * SR + off);
    float acc = 0.f;
#pragma unroll 4
    for (int r = 0; r < R; r += 8) {
      float wf[8];
      T16::to_f8(wr[r >> 3], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(wf[e], s_lora[off + r + e], acc);
    }
    s_d[q][c] = acc;
  }
  __syncthreads();

  if (t < kN) {  // gates, one lane per channel of this head
    const int ch = h * kN + t;
    const float r = prow[ch], k = prow[C + ch];
    float v = prow[2 * C + ch];
    float *vf = a.vfirst + (int64_t)b * C + ch;
    if (a.layer0) {
      *vf = v;
    } else {
      v = v + sigmoidf_(vec[RWKV7_V_V0 * C + ch] + s_d[0][t]) * (*vf - v);
    }
    const float w = expf(-sigmoidf_(vec[RWKV7_V_W0 * C + ch] + s_d[1][t]) / 1.6487212707001282f);
    const float ag = sigmoidf_(vec[RWKV7_V_A0 * C + ch] + s_d[2][t]);
    const float kk = k * vec[RWKV7_V_K_K * C + ch];
    const float kn = k + vec[RWKV7_V_K_A * C + ch] * (k * ag - k);
    const float nrm = sqrtf(wave_sum(kk * kk));
    const float kh = kk / fmaxf(nrm, 1e-12f);
    const float rk = wave_sum(r * kn * vec[RWKV7_V_R_K * C + ch]);
    s_r[t] = r; s_w[t] = w; s_k[t] = kn; s_v[t] = v;
    s_a[t] = kh; s_b[t] = -kh * ag; s_g[t] = s_d[3][t];
    if (t == 0) s_rk = rk;
    if (a.shift) a.shift[(int64_t)b * C + ch] = T16::from_f(a.xln[(int64_t)b * C + ch]);
  }
  __syncthreads();

  {  // wkv7: thread -> row i, 16 key columns
    const int i = t >> 2, j0 = (t & 3) * 16;
    float4 *Sp = reinterpret_cast<float4 *>(a.rnn + (((int64_t)b * a.H + h) * kN + i) * kN + j0);
    float S[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float4 u = Sp[q];
      S[4 * q] = u.x; S[4 * q + 1] = u.y; S[4 * q + 2] = u.z; S[4 * q + 3] = u.w;
    }
    float sa = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) sa = fmaf(S[e], s_a[j0 + e], sa);
    sa = sum4(sa);
    const float vi = s_v[i];
    float y = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = j0 + e;
      S[e] = S[e] * s_w[j] + sa * s_b[j] + vi * s_k[j];
      y = fmaf(S[e], s_r[j], y);
    }
    y = sum4(y);
#pragma unroll
    for (int q = 0; q < 4; ++q) Sp[q] = make_float4(S[4 * q], S[4 * q + 1], S[4 * q + 2], S[4 * q + 3]);
    if ((t & 3) == 0) s_y[i] = y;
  }
  __syncthreads();

  if (t < kN) {  // GroupNorm over the head + bonus + gate
    const int ch = h * kN + t;
    const float y = s_y[t];
    const float mean = wave_sum(y) * (1.f / kN);
    const float d = y - mean;
    const float var = wave_sum(d * d) * (1.f / kN);
    const float yn = d * rsqrtf(var + kGnEps) * vec[RWKV7_V_LNX_W * C + ch] + vec[RWKV7_V_LNX_B * C + ch];
    const float out = (yn + s_rk * s_v[t]) * s_g[t];
    if (a.yg16) a.yg16[(int64_t)b * C + ch] = T16::from_f(out);
    else a.yg[(int64_t)b * C + ch] = out;
  }
}

int launch_tmix_decode(const TmixDecodeArgs &a, int B, hipStream_t st) {
  // the LoRA rows are read 8 ranks (16 bytes) at a time, all ranks staged in LDS
  if (a.rv + a.rw + a.ra + a.rg > kMaxRanks || a.rv % 8 || a.rw % 8 || a.ra % 8 || a.rg % 8) return RWKV7_ESHAPE;
  if (a.bf) tmix_decode_kernel<true><<<dim3(a.H, B), 256, 0, st>>>(a);
  else tmix_decode_kernel<false><<<dim3(a.H, B), 256, 0, st>>>(a);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

constexpr int kCh = 16;

template <typename T> RWKV7_DEV float to_f(T x);
template <> RWKV7_DEV float to_f<float>(float x) { return x; }
template <> RWKV7_DEV float to_f<uint16_t>(uint16_t x) { return h2f(x); }
template <typename T> RWKV7_DEV T from_f(float x);
template <> RWKV7_DEV float from_f<float>(float x) { return x; }
template <> RWKV7_DEV uint16_t from_f<uint16_t>(float x) { return f2h(x); }
template <> RWKV7_DEV float to_f<bf16_t>(bf16_t x) { return b2f(x.bits); }
template <> RWKV7_DEV bf16_t from_f<bf16_t>(float x) { return bf16_t{f2b(x)}; }

// Four consecutive elements as float4: one 16-byte load for f32, one 8-byte
// load for f16 or bf16.
RWKV7_DEV float4 ld4_as_f(const float *p) { return *reinterpret_cast<const float4 *>(p); }
RWKV7_DEV float4 ld4_as_f(const uint16_t *p) {
  const half4 h = __builtin_bit_cast(half4, *reinterpret_cast<const uint2 *>(p));
  return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}
RWKV7_DEV float4 ld4_as_f(const bf16_t *p) {
  const uint2 u = *reinterpret_cast<const uint2 *>(p);
  return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xFFFF0000u),
                     __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xFFFF0000u));
}

// ---------------------------------------------------------------------------
// Chunked wkv7 scan (demo/rwkv7_torch.py:227-232; dplr.py:174-227). Grid
// (4 * H, B[, segments]): each workgroup owns 16 value rows of one head's fp32
// state, kept in registers: 16 lanes per row, 4 key columns per lane. The step
// inputs (w, a, b, k, r, v) of CH tokens at a time are staged through
// double-buffered LDS by a staging policy:
//   * GateStager (the model's prefill and batched decode): the gate math of
//     each token (demo/rwkv7_torch.py:203-224) from the projections -- every
//     workgroup computes all 64 channels of its head (the L2 norm of kk needs
//     them all) and writes the gated k and the mixed v of its 16 channels (and
//     v itself on layer 0) for the GroupNorm stage (all 64 when constructed
//     with quarter -1, as the chunked kernels below do);
//   * RawStager (the operator-level rwkv7_wkv7): the inputs as given.
//
// Step loop: sa = S a is a 16-lane DPP sum; S w + v k is formed while it runs,
// so the new state is one FMA past sa; the next step's inputs are read from
// LDS while the current step computes; y is left as per-lane partials in LDS
// and summed once per chunk.
//
// Segments (grid z, model path): a long sequence is cut into nseg pieces of
// seg_len tokens scanned at once. Segment 0 starts from the real state;
// segment j > 0 starts from zero and also carries the rows of its transition
// product P_t = M_1 ... M_t (M = diag(w) + a b^T, from the identity, no v k
// term), so that with S_in the state entering it, S_t = S_in P_t + S_loc_t and
// y_t = y_loc_t + S_in u_t with u_t = P_t r. It writes y_loc and u, and its
// end state and product to Send / Pend; wkv7_prefill_combine_kernel then
// chains the segments and adds S_in u_t.
// ---------------------------------------------------------------------------

// s_in[buf][vec][token][16 float4]: vec 0 w, 1 a, 2 b, 3 k, 4 r, 5 v
template <int CH>
using StageBuf = float4[6][CH][kN / 4];

// Model path: gates of each token from r, k, v and the LoRA second steps.
// Thread -> token t >> 4 of the chunk, channels 4q .. 4q+3 of the head (the
// threads of tokens past CH compute a copy of the chunk's last token and store
// nothing; every thread takes part in the 16-lane L2-norm sum).
template <int CH>
struct GateStager {
  using Args = PrefillScanArgs;
  const PrefillScanArgs &p;
  int64_t base, MC;
  int t1, quarter, st_tok, q, C;
  bool stager;
  float4 v0v, w0v, a0v, kkv, kav;
  float4 g_r, g_k, g_v, g_dv, g_dw, g_da, g_vf;
  // when set: the chunk's LoRA second steps v, w, a in LDS ([3][16][lds_ld],
  // token-major, the head's 64 channels), formed by the caller before commit
  const float *lds_d = nullptr;
  int lds_ld = 0;

  RWKV7_DEV GateStager(const PrefillScanArgs &p_, int h, int quarter_, int64_t base_, int t1_)
      : p(p_), base(base_), t1(t1_), quarter(quarter_) {
    const int t = threadIdx.x;
    C = p.C;
    MC = (int64_t)p.M * C;
    st_tok = t >> 4;
    q = t & 15;
    stager = st_tok < CH;
    const int ch0 = h * kN + 4 * q;
    const float *vec = p.vec;
    v0v = ld4_as_f(vec + RWKV7_V_V0 * C + ch0);
    w0v = ld4_as_f(vec + RWKV7_V_W0 * C + ch0);
    a0v = ld4_as_f(vec + RWKV7_V_A0 * C + ch0);
    kkv = ld4_as_f(vec + RWKV7_V_K_K * C + ch0);
    kav = ld4_as_f(vec + RWKV7_V_K_A * C + ch0);
  }
  RWKV7_DEV void fetch(int c0) {  // c0: first token of the chunk
    const int tt = c0 + st_tok;
    const int ts = tt < t1 ? tt : t1 - 1;  // clamped (its step is never run)
    const int64_t o = base + (int64_t)ts * C + 4 * q;
    g_r = ld4_as_f(p.rkv + o);
    g_k = ld4_as_f(p.rkv + MC + o);
    g_v = ld4_as_f(p.rkv + 2 * MC + o);
    if (!lds_d) {
      g_dv = ld4_as_f(p.d + o);
      g_dw = ld4_as_f(p.d + MC + o);
      g_da = ld4_as_f(p.d + 2 * MC + o);
    }
    g_vf = p.layer0 ? g_v : ld4_as_f(p.vfirst + o);
  }
  RWKV7_DEV void commit(int c0, StageBuf<CH> &dst) {
    commit_to(c0, [&](int i, int t, int qq, const float4 &x) { dst[i][t][qq] = x; });
  }
  // The six staged vectors of this thread's token and float4 go to
  // sink(vector, token, float4 index, value).
  template <class Sink>
  RWKV7_DEV void commit_to(int c0, Sink &&sink) {
    const int tt = c0 + st_tok;
    if (lds_d) {
      const int r = st_tok < CH ? st_tok : CH - 1;
      g_dv = *reinterpret_cast<const float4 *>(lds_d + r * lds_ld + 4 * q);
      g_dw = *reinterpret_cast<const float4 *>(lds_d + (CH + r) * lds_ld + 4 * q);
      g_da = *reinterpret_cast<const float4 *>(lds_d + (2 * CH + r) * lds_ld + 4 * q);
    }
    const float k4[4] = {g_k.x, g_k.y, g_k.z, g_k.w};
    const float vr[4] = {g_v.x, g_v.y, g_v.z, g_v.w}, dv[4] = {g_dv.x, g_dv.y, g_dv.z, g_dv.w};
    const float dw[4] = {g_dw.x, g_dw.y, g_dw.z, g_dw.w}, da[4] = {g_da.x, g_da.y, g_da.z, g_da.w};
    const float vf[4] = {g_vf.x, g_vf.y, g_vf.z, g_vf.w};
    const float pv0[4] = {v0v.x, v0v.y, v0v.z, v0v.w}, pw0[4] = {w0v.x, w0v.y, w0v.z, w0v.w};
    const float pa0[4] = {a0v.x, a0v.y, a0v.z, a0v.w}, pkk[4] = {kkv.x, kkv.y, kkv.z, kkv.w};
    const float pka[4] = {kav.x, kav.y, kav.z, kav.w};
    float w[4], kn[4], v[4], kk[4], ag[4];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = p.layer0 ? vr[e] : vr[e] + sigmoidf_(pv0[e] + dv[e]) * (vf[e] - vr[e]);
      w[e] = expf(-sigmoidf_(pw0[e] + dw[e]) / 1.6487212707001282f);
      ag[e] = sigmoidf_(pa0[e] + da[e]);
      kk[e] = k4[e] * pkk[e];
      kn[e] = k4[e] + pka[e] * (k4[e] * ag[e] - k4[e]);
      ss += kk[e] * kk[e];
    }
    const float inv = 1.f / fmaxf(sqrtf(sum16(ss)), 1e-12f);
    float a[4], b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = kk[e] * inv;
      b[e] = -a[e] * ag[e];
    }
    if (!stager) return;
    sink(0, st_tok, q, make_float4(w[0], w[1], w[2], w[3]));
    sink(1, st_tok, q, make_float4(a[0], a[1], a[2], a[3]));
    sink(2, st_tok, q, make_float4(b[0], b[1], b[2], b[3]));
    sink(3, st_tok, q, make_float4(kn[0], kn[1], kn[2], kn[3]));
    sink(4, st_tok, q, g_r);
    sink(5, st_tok, q, make_float4(v[0], v[1], v[2], v[3]));
    // this workgroup's 16 channels of the values GroupNorm needs
    if (tt < t1 && (quarter < 0 || (q >> 2) == quarter)) {
      const int64_t o = base + (int64_t)tt * C + 4 * q;
      *reinterpret_cast<float4 *>(p.kn_out + o) = make_float4(kn[0], kn[1], kn[2], kn[3]);
      *reinterpret_cast<float4 *>(p.v_out + o) = make_float4(v[0], v[1], v[2], v[3]);
      if (p.layer0) *reinterpret_cast<float4 *>(p.vfirst + o) = g_v;
    }
  }
  RWKV7_DEV void put_y(int64_t o, float y) { p.y[o] = y; }
  RWKV7_DEV void record(int, int, int, const float4 &) {}
};

// Operator level: w, a, b, k, r, v as given ([B, T, H, 64]; f16 or bf16, w
// also f32; every operand f32 for the training forward).
// Thread -> token t >> 4, float4 q = t & 15 of the head's 64 channels.
template <int CH, typename TI, typename TW, typename TY>
struct RawStager {
  using Args = ScanArgs<TI, TW, TY>;
  const Args &p;
  int64_t base;
  int t1, st_tok, q, C;
  bool stager;
  float4 g[6];

  int64_t hbase;  // this head's slab of the optional state history

  RWKV7_DEV RawStager(const Args &p_, int h, int, int64_t base_, int t1_) : p(p_), base(base_), t1(t1_) {
    C = p.H * kN;
    hbase = ((int64_t)blockIdx.y * p.H + h) * p.T * (kN * kN);
    st_tok = threadIdx.x >> 4;
    q = threadIdx.x & 15;
    stager = st_tok < CH;
  }
  RWKV7_DEV void fetch(int c0) {
    const int tt = c0 + st_tok;
    const int ts = tt < t1 ? tt : t1 - 1;
    const int64_t o = base + (int64_t)ts * C + 4 * q;
    g[0] = ld4_as_f(p.w + o);
    g[1] = ld4_as_f(p.a + o);
    g[2] = ld4_as_f(p.b + o);
    g[3] = ld4_as_f(p.k + o);
    g[4] = ld4_as_f(p.r + o);
    g[5] = ld4_as_f(p.v + o);
  }
  RWKV7_DEV void commit(int c0, StageBuf<CH> &dst) {
    commit_to(c0, [&](int i, int t, int qq, const float4 &x) { dst[i][t][qq] = x; });
  }
  template <class Sink>
  RWKV7_DEV void commit_to(int, Sink &&sink) {
    if (!stager) return;
#pragma unroll
    for (int i = 0; i < 6; ++i) sink(i, st_tok, q, g[i]);
  }
  RWKV7_DEV void put_y(int64_t o, float y) { p.y[o] = from_f<TY>(y); }
  // state entering token tt: row `row`, key columns 4 lc .. 4 lc + 3
  RWKV7_DEV void record(int tt, int row, int lc, const float4 &S) {
    if (p.hist) *reinterpret_cast<float4 *>(p.hist + hbase + (int64_t)tt * (kN * kN) + row * kN + 4 * lc) = S;
  }
};

// SEG: launched with more than one segment (GateStager only). CH: tokens
// staged per chunk (16; 1 for single-token steps, whose small LDS lets four
// workgroups share a CU).
template <bool SEG, int CH, class St>
__global__ __launch_bounds__(256) void dplr_scan_kernel(typename St::Args p, int seg_len, int nseg) {
  __shared__ StageBuf<CH> s_in[2];
  __shared__ float s_yp[CH][16][17];  // per-lane partial y: [step][row][lane], padded
  __shared__ float s_up[SEG ? CH : 1][16][17];  // the same for u (segments after the first)

  const int t = threadIdx.x;
  const int h = blockIdx.x >> 2, quarter = blockIdx.x & 3, bi = blockIdx.y;
  const int seg = blockIdx.z;
  const bool tail = SEG && seg > 0;  // block-uniform
  const int H = p.H, T = p.T, C = H * kN;
  const int t0 = seg * seg_len, t1 = min(T, t0 + seg_len), Tl = t1 - t0;
  const int row = quarter * 16 + (t >> 4);
  const int lc = t & 15;  // owns key columns 4*lc .. 4*lc+3
  const int64_t base = (int64_t)bi * T * C + (int64_t)h * kN;  // token 0, channel 0 of the head
  St st(p, h, quarter, base, t1);

  float4 *Sp = reinterpret_cast<float4 *>(p.S + (((int64_t)bi * H + h) * kN + row) * kN) + lc;
  float4 S = tail ? make_float4(0.f, 0.f, 0.f, 0.f) : *Sp;
  // rows of the transition product, from the identity (tail segments only)
  float4 P = make_float4(0.f, 0.f, 0.f, 0.f);
  if (lc == (row >> 2)) {
    const int e = row & 3;
    P = make_float4(e == 0, e == 1, e == 2, e == 3);
  }

  st.fetch(t0);
  st.commit(t0, s_in[0]);
  __syncthreads();
  const int nch = (Tl + CH - 1) / CH;
  for (int c = 0; c < nch; ++c) {
    const int buf = c & 1;
    if (c + 1 < nch) st.fetch(t0 + (c + 1) * CH);
    const int steps = min(CH, Tl - c * CH);
    const float *vrow = reinterpret_cast<const float *>(&s_in[buf][5][0][0]) + row;
    struct In {
      float4 w, a, b, k, r;
      float v;
    };
    auto load_in = [&](In &x, int sp) {
      x.w = s_in[buf][0][sp][lc];
      x.a = s_in[buf][1][sp][lc];
      x.b = s_in[buf][2][sp][lc];
      x.k = s_in[buf][3][sp][lc];
      x.r = s_in[buf][4][sp][lc];
      x.v = vrow[sp * kN];
    };
    auto step = [&](const In &x, int sp) {
      st.record(t0 + c * CH + sp, row, lc, S);
      float p0 = S.x * x.a.x, p1 = S.z * x.a.z;
      p0 = fmaf(S.y, x.a.y, p0);
      p1 = fmaf(S.w, x.a.w, p1);
      float4 pre;
      pre.x = fmaf(S.x, x.w.x, x.v * x.k.x);
      pre.y = fmaf(S.y, x.w.y, x.v * x.k.y);
      pre.z = fmaf(S.z, x.w.z, x.v * x.k.z);
      pre.w = fmaf(S.w, x.w.w, x.v * x.k.w);
      const float sa = sum16(p0 + p1);
      S.x = fmaf(sa, x.b.x, pre.x);
      S.y = fmaf(sa, x.b.y, pre.y);
      S.z = fmaf(sa, x.b.z, pre.z);
      S.w = fmaf(sa, x.b.w, pre.w);
      float y0 = S.x * x.r.x, y1 = S.z * x.r.z;
      y0 = fmaf(S.y, x.r.y, y0);
      y1 = fmaf(S.w, x.r.w, y1);
      s_yp[sp][t >> 4][lc] = y0 + y1;
    };
    // the same step plus the transition product's rows: P <- P (diag(w) + a b^T)
    auto step_tail = [&](const In &x, int sp) {
      float p0 = S.x * x.a.x, p1 = S.z * x.a.z;
      float q0 = P.x * x.a.x, q1 = P.z * x.a.z;
      p0 = fmaf(S.y, x.a.y, p0);
      p1 = fmaf(S.w, x.a.w, p1);
      q0 = fmaf(P.y, x.a.y, q0);
      q1 = fmaf(P.w, x.a.w, q1);
      float4 pre;
      pre.x = fmaf(S.x, x.w.x, x.v * x.k.x);
      pre.y = fmaf(S.y, x.w.y, x.v * x.k.y);
      pre.z = fmaf(S.z, x.w.z, x.v * x.k.z);
      pre.w = fmaf(S.w, x.w.w, x.v * x.k.w);
      const float2 sums = sum16x2(p0 + p1, q0 + q1);
      S.x = fmaf(sums.x, x.b.x, pre.x);
      S.y = fmaf(sums.x, x.b.y, pre.y);
      S.z = fmaf(sums.x, x.b.z, pre.z);
      S.w = fmaf(sums.x, x.b.w, pre.w);
      P.x = fmaf(sums.y, x.b.x, P.x * x.w.x);
      P.y = fmaf(sums.y, x.b.y, P.y * x.w.y);
      P.z = fmaf(sums.y, x.b.z, P.z * x.w.z);
      P.w = fmaf(sums.y, x.b.w, P.w * x.w.w);
      float y0 = S.x * x.r.x, y1 = S.z * x.r.z;
      float u0 = P.x * x.r.x, u1 = P.z * x.r.z;
      y0 = fmaf(S.y, x.r.y, y0);
      y1 = fmaf(S.w, x.r.w, y1);
      u0 = fmaf(P.y, x.r.y, u0);
      u1 = fmaf(P.w, x.r.w, u1);
      s_yp[sp][t >> 4][lc] = y0 + y1;
      if constexpr (SEG) s_up[sp][t >> 4][lc] = u0 + u1;
    };
    // two input register sets in turn: the next step's inputs are read from
    // LDS while the current step computes
    In x0, x1;
    load_in(x0, 0);
    int sp = 0;
    if (!tail) {
      for (; sp + 1 < steps; sp += 2) {
        load_in(x1, sp + 1);
        step(x0, sp);
        load_in(x0, sp + 2 < steps ? sp + 2 : sp + 1);
        step(x1, sp + 1);
      }
      if (sp < steps) step(x0, sp);
    } else if constexpr (SEG) {
      for (; sp + 1 < steps; sp += 2) {
        load_in(x1, sp + 1);
        step_tail(x0, sp);
        load_in(x0, sp + 2 < steps ? sp + 2 : sp + 1);
        step_tail(x1, sp + 1);
      }
      if (sp < steps) step_tail(x0, sp);
    }
    __syncthreads();
    {  // y (and u) of (step t >> 4, row t & 15): sums of the 16 lane partials
      const int ss = t >> 4, rr = t & 15;
      if (ss < steps) {
        float y = 0.f;
#pragma unroll
        for (int l = 0; l < 16; ++l) y += s_yp[ss][rr][l];
        const int64_t o = base + (int64_t)(t0 + c * CH + ss) * C + quarter * 16 + rr;
        st.put_y(o, y);
        if constexpr (SEG) {
          if (tail) {
            float u = 0.f;
#pragma unroll
            for (int l = 0; l < 16; ++l) u += s_up[ss][rr][l];
            p.U[o] = u;
          }
        }
      }
    }
    if (c + 1 < nch) st.commit(t0 + (c + 1) * CH, s_in[buf ^ 1]);
    __syncthreads();
  }
  if constexpr (!SEG) {
    *Sp = S;
  } else {
    const int64_t slab = (int64_t)p.B * H * kN * kN;
    const int64_t o = (((int64_t)bi * H + h) * kN + row) * kN + 4 * lc;
    *reinterpret_cast<float4 *>(p.Send + seg * slab + o) = S;
    if (tail) *reinterpret_cast<float4 *>(p.Pend + seg * slab + o) = P;
  }
}

template <typename TI, typename TW, typename TY>
int launch_wkv7_scan(const ScanArgs<TI, TW, TY> &p, hipStream_t st) {
  if (p.T <= 0 || p.B <= 0 || p.H <= 0) return RWKV7_OK;
  if (p.T == 1)
    dplr_scan_kernel<false, 1, RawStager<1, TI, TW, TY>><<<dim3(4 * p.H, p.B, 1), 256, 0, st>>>(p, p.T, 1);
  else
    dplr_scan_kernel<false, kCh, RawStager<kCh, TI, TW, TY>><<<dim3(4 * p.H, p.B, 1), 256, 0, st>>>(p, p.T, 1);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

// ---------------------------------------------------------------------------
// Backward of the wkv7 recurrence (the training path the reference plans,
// TODO.md:46-54). Forward, per head (rows i = value, columns j = key):
//   sa_i = sum_j S[i,j] a_j ;  S'[i,j] = S[i,j] w_j + sa_i b_j + v_i k_j ;
//   y_i = sum_j S'[i,j] r_j
// Reverse-time adjoint G = dL/dS', from G = dL/dS_T, for t = T-1 .. 0 with
// S = the state entering step t (recorded by the forward) and S' the one
// after it:
//   G += gy r^T ;  gr = S'^T gy ;  gv = G k ;  gk = G^T v ;  gw = diag(G^T S)
//   gsa = G b ;  gb = G^T sa ;  ga = S^T gsa ;  G <- G diag(w) + gsa a^T
// and dL/dS_0 = G at the end. Grid (H, B), 256 threads: thread -> row
// i = t / 4, key columns 16 (t % 4) .. +16; row sums are 4-lane DPP sums,
// column sums run over the 16 rows of a wave with lane shuffles and then over
// the 4 waves in LDS.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void wkv7_bwd_kernel(Wkv7BwdArgs p) {
  __shared__ float s_in[7][kN];       // r w k v a b gy of the step
  __shared__ float s_col[5][4][kN];   // per-wave column sums: gr gk gw gb ga
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int h = blockIdx.x, bi = blockIdx.y;
  const int H = p.H, T = p.T, C = H * kN;
  const int i = t >> 2, j0 = 16 * (t & 3);
  const int64_t sbase = ((int64_t)bi * H + h) * kN * kN + (int64_t)i * kN + j0;  // this thread's S piece
  const int64_t hslab = ((int64_t)bi * H + h) * (int64_t)T * kN * kN;
  float G[16], Sn[16], Sp[16];
  auto ld16 = [&](float (&d)[16], const float *src) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float4 q = reinterpret_cast<const float4 *>(src)[e];
      d[4 * e] = q.x; d[4 * e + 1] = q.y; d[4 * e + 2] = q.z; d[4 * e + 3] = q.w;
    }
  };
  ld16(Sn, p.S_T + sbase);
  if (p.gS_T) ld16(G, p.gS_T + sbase);
  else {
#pragma unroll
    for (int e = 0; e < 16; ++e) G[e] = 0.f;
  }
  const float *ins[7] = {p.r, p.w, p.k, p.v, p.a, p.b, p.gy};
  for (int tt = T - 1; tt >= 0; --tt) {
    const int64_t tok = ((int64_t)bi * T + tt) * C + (int64_t)h * kN;
    for (int e = t; e < 7 * kN; e += 256) s_in[e / kN][e % kN] = ins[e / kN][tok + e % kN];
    ld16(Sp, p.hist + hslab + (int64_t)tt * kN * kN + (int64_t)i * kN + j0);
    __syncthreads();
    const float vi = s_in[3][i], gyi = s_in[6][i];
    float sa = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) sa = fmaf(Sp[e], s_in[4][j0 + e], sa);
    sa = sum4(sa);
    float gv = 0.f, gsa = 0.f;
    float part[5][16];  // gr gk gw gb ga of this thread's columns
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = j0 + e;
      G[e] = fmaf(gyi, s_in[0][j], G[e]);
      part[0][e] = Sn[e] * gyi;
      part[1][e] = G[e] * vi;
      part[2][e] = G[e] * Sp[e];
      part[3][e] = G[e] * sa;
      gv = fmaf(G[e], s_in[2][j], gv);
      gsa = fmaf(G[e], s_in[5][j], gsa);
    }
    gv = sum4(gv);
    gsa = sum4(gsa);
#pragma unroll
    for (int e = 0; e < 16; ++e) part[4][e] = gsa * Sp[e];
    // column sums over the wave's 16 rows: lanes 4 r + c share column group c
#pragma unroll
    for (int q = 0; q < 5; ++q)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float x = part[q][e];
        x += __shfl_xor(x, 4);
        x += __shfl_xor(x, 8);
        x += __shfl_xor(x, 16);
        x += __shfl_xor(x, 32);
        part[q][e] = x;
      }
    if (lane < 4) {
#pragma unroll
      for (int q = 0; q < 5; ++q)
#pragma unroll
        for (int e = 0; e < 16; ++e) s_col[q][wv][j0 + e] = part[q][e];
    }
    if ((t & 3) == 0) p.gv[tok + i] = gv;
    // adjoint of the state entering the step
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = j0 + e;
      G[e] = fmaf(G[e], s_in[1][j], gsa * s_in[4][j]);
      Sn[e] = Sp[e];
    }
    __syncthreads();
    for (int e = t; e < 5 * kN; e += 256) {
      const int q = e / kN, j = e % kN;
      const float sum = (s_col[q][0][j] + s_col[q][1][j]) + (s_col[q][2][j] + s_col[q][3][j]);
      float *dst = q == 0 ? p.gr : q == 1 ? p.gk : q == 2 ? p.gw : q == 3 ? p.gb : p.ga;
      dst[tok + j] = sum;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    reinterpret_cast<float4 *>(p.gS0 + sbase)[e] = make_float4(G[4 * e], G[4 * e + 1], G[4 * e + 2], G[4 * e + 3]);
}

int launch_wkv7_bwd(const Wkv7BwdArgs &p, hipStream_t st) {
  if (p.T <= 0 || p.B <= 0 || p.H <= 0) return RWKV7_OK;
  wkv7_bwd_kernel<<<dim3(p.H, p.B), 256, 0, st>>>(p);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

template int launch_wkv7_scan<uint16_t, float, uint16_t>(const ScanArgs<uint16_t, float, uint16_t> &, hipStream_t);
template int launch_wkv7_scan<uint16_t, uint16_t, uint16_t>(const ScanArgs<uint16_t, uint16_t, uint16_t> &, hipStream_t);
template int launch_wkv7_scan<float, float, float>(const ScanArgs<float, float, float> &, hipStream_t);
template int launch_wkv7_scan<bf16_t, float, bf16_t>(const ScanArgs<bf16_t, float, bf16_t> &, hipStream_t);
template int launch_wkv7_scan<bf16_t, bf16_t, bf16_t>(const ScanArgs<bf16_t, bf16_t, bf16_t> &, hipStream_t);

// Chains the segments of dplr_scan_kernel (model path). Grid (4 H, B, (nseg - 1) *
// nblk): the workgroup of segment j >= 1 and 16-token block k of it forms the
// state entering j, S_in(1) = Send(0), S_in(i + 1) = S_in(i) Pend(i) + Send(i),
// adds S_in(j) u_t to y_t of its tokens, and (block 0 of the last segment)
// writes the final state. 16 rows of one head per workgroup, 4 columns per
// lane. The products are staged in LDS kPmBuf at a time with all their loads
// in flight, since they were written by other XCDs and each load is a trip to
// memory.
constexpr int kPmBuf = 3;
__global__ __launch_bounds__(256) void wkv7_prefill_combine_kernel(PrefillScanArgs p, int seg_len, int nseg) {
  __shared__ float s_row[16][kN + 4];
  __shared__ float4 s_pm[kPmBuf][kN][kN / 4];
  __shared__ float4 s_sd[kPmBuf][256];  // this thread's Send rows
  const int t = threadIdx.x;
  const int nblk = (seg_len + kCh - 1) / kCh;
  const int h = blockIdx.x >> 2, quarter = blockIdx.x & 3, bi = blockIdx.y;
  const int j = blockIdx.z / nblk + 1, blk = blockIdx.z % nblk;
  const int r16 = t >> 4, row = quarter * 16 + r16, lc = t & 15;
  const int H = p.H, C = p.C;
  const int64_t slab = (int64_t)p.B * H * kN * kN;
  const int64_t hoff = ((int64_t)bi * H + h) * kN * kN;
  auto at = [&](const float *m, int i) {
    return *reinterpret_cast<const float4 *>(m + i * slab + hoff + (int64_t)row * kN + 4 * lc);
  };
  const bool final_state = j == nseg - 1 && blk == 0;
  const int last = final_state ? j : j - 1;  // products to apply
  // this block's u loads go out first: they do not depend on the chain
  const int64_t base = (int64_t)bi * p.T * C + (int64_t)h * kN;
  const int tb = j * seg_len + blk * kCh;
  const int n = min(kCh, min(p.T, (j + 1) * seg_len) - tb);
  float4 u[kCh];
#pragma unroll
  for (int q = 0; q < kCh; ++q) {
    u[q] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q < n) u[q] = *reinterpret_cast<const float4 *>(p.U + base + (int64_t)(tb + q) * C + 4 * lc);
  }
  float4 sin = at(p.Send, 0), sin_j = sin;
  for (int g0 = 1; g0 <= last; g0 += kPmBuf) {
    const int gn = min(kPmBuf, last - g0 + 1);
    __syncthreads();  // the previous group's readers are done
#pragma unroll
    for (int b = 0; b < kPmBuf; ++b) {
      if (b < gn) {  // global to LDS: no load waits for a store
        const float4 *src = reinterpret_cast<const float4 *>(p.Pend + (g0 + b) * slab + hoff);
#pragma unroll
        for (int e = 0; e < 4; ++e) (&s_pm[b][0][0])[t + 256 * e] = src[t + 256 * e];
        s_sd[b][t] = at(p.Send, g0 + b);
      }
    }
    for (int b = 0; b < gn; ++b) {
      {
        if (g0 + b == j) sin_j = sin;
        __syncthreads();
        *reinterpret_cast<float4 *>(&s_row[r16][4 * lc]) = sin;
        __syncthreads();
        float4 acc = s_sd[b][t];
#pragma unroll 16
        for (int k = 0; k < kN; ++k) {
          const float sk = s_row[r16][k];
          const float4 pr = s_pm[b][k][lc];
          acc.x = fmaf(sk, pr.x, acc.x);
          acc.y = fmaf(sk, pr.y, acc.y);
          acc.z = fmaf(sk, pr.z, acc.z);
          acc.w = fmaf(sk, pr.w, acc.w);
        }
        sin = acc;
      }
    }
  }
  if (final_state) {
    *(reinterpret_cast<float4 *>(p.S + hoff + (int64_t)row * kN) + lc) = sin;
    sin = sin_j;  // the state entering segment j, for the outputs below
  }
  // y_t += S_in(j) u_t for the (up to) 16 tokens of this block: the 16 lanes'
  // partial dots summed through LDS, lane k finishing token k
  float part[kCh];
#pragma unroll
  for (int q = 0; q < kCh; ++q)
    part[q] = fmaf(sin.x, u[q].x, fmaf(sin.y, u[q].y, fmaf(sin.z, u[q].z, sin.w * u[q].w)));
  __syncthreads();  // s_pm readers are done: its first 16 KB take the partials
  float *red = reinterpret_cast<float *>(&s_pm[0][0][0]);  // [16 rows][16 tokens][17]
#pragma unroll
  for (int q = 0; q < kCh; ++q) red[(r16 * kCh + q) * 17 + lc] = part[q];
  __syncthreads();
  if (lc < n) {
    float tot = 0.f;
#pragma unroll
    for (int l = 0; l < 16; ++l) tot += red[(r16 * kCh + lc) * 17 + l];
    p.y[base + (int64_t)(tb + lc) * C + row] += tot;
  }
}

// Segments of the prefill scan for T tokens of B sequences of H heads
// (lengths a multiple of the 16-token staging chunk): one below 64 tokens, up
// to 4 of >= 32 tokens below 256, up to 8 of >= 64 tokens beyond (measured on
// 0.4B: more, shorter segments lose more to the chain of products than they
// gain in the scan), and no more than fit the 4 H B workgroups of one segment
// on the GPU's 256 CUs at once (a segmented workgroup takes a CU's LDS).
int prefill_segments(int T, int B, int H, int cus, int *seg_len) {
  int P = T < 64 ? 1 : T < 256 ? min(4, T / 32) : min(8, T / 64);
  P = min(P, cus / max(1, 4 * H * B));
  if (P < 2) {
    *seg_len = T;
    return 1;
  }
  int L = (T + P - 1) / P;
  L = (L + kCh - 1) / kCh * kCh;
  *seg_len = L;
  return (T + L - 1) / L;
}

// ---------------------------------------------------------------------------
// Chunked wkv7 on fp32 MFMA (the model's prefill at T >= kChunkMinT, and
// rwkv7_wkv7_chunked). Over a chunk of L = 16 tokens entered with state S0,
// with D(s, t] = prod_{m=s+1..t} diag(w_m) over the key channels (D(t, t] =
// I) and s = -1 standing for "before the chunk", the recurrence unrolls to
//   S_t   = S0 D(-1, t] + sum_{s<=t} (sig_s b_s^T + v_s k_s^T) D(s, t]
//   sig_t = S_{t-1} a_t
// which is linear in S0. With tokens as rows (Sig, V, U, Y0: 16 x 64 value
// channels; A~, R~, B^, K^, G1, G2: 16 x 64 key channels):
//   Sig = G1 S0^T + U,   G1 = T A~,   U = T Aka V,   T = (I - Aba)^-1
//   Y   = G2 S0^T + Y0,  G2 = R~ + Bbr G1,   Y0 = Bbr U + Bkr V
//   S16 = S0 diag(gam) + Sig^T B^ + V^T K^
// where a~_t = a_t D(-1, t-1], r~_t = r_t D(-1, t], b^_s = b_s D(s, 15],
// k^_s = k_s D(s, 15], gam = D(-1, 15], and the 16 x 16 token matrices are
//   Aba[t][s] = b_s^T D(s, t-1] a_t,  Aka[t][s] = k_s^T D(s, t-1] a_t  (s < t)
//   Bbr[t][s] = b_s^T D(s, t] r_t,    Bkr[t][s] = k_s^T D(s, t] r_t    (s <= t).
// Two kernels:
// 1. wkv7_chunk_prep_kernel, one workgroup per (chunk, head, sequence), all at
//    once: stages the chunk through the serial scan's staging policies, forms
//    the token matrices -- on MFMA as (a~)(b / P_s)^T etc. with the prefix
//    products P_t = D(-1, t] when every P_t of the chunk lies in [1e-30,
//    1e30], otherwise straight from products of w -- solves for T by forward
//    substitution, and writes G1, G2, B^, K^, U, Y0, V and gam as a chunk
//    record laid out in the chain kernel's MFMA operand order.
// 2. wkv7_chunk_chain_kernel, grid (4 H / NQ, B): each workgroup carries
//    16 NQ value rows of a head's state through the chunks in order; per
//    chunk and quarter, Sig and Y from S (16 x 64 by 64 x 16), then
//    S <- S diag(gam) + Sig^T B^ + V^T K^. Four waves per quarter, one
//    16-column block of the state each; the Sig and Y partials of the blocks
//    are summed through LDS in block order.
// A chunk past the end of the sequence is padded with identity steps (w = 1,
// a = b = k = r = v = 0), whose outputs are not stored.
// ---------------------------------------------------------------------------
constexpr int kCk = 16;
// Chunk record (f32). G1, G2, B^, K^: [wave][lane][kk]; U, V: [quarter][lane][kk];
// Y0: [quarter][t][i]; gam: [64]. The chain kernel's lane l of wave w (rows
// 16 q .. of the state) reads element kk of [w or q][l] as its operand of the
// kk-th MFMA step.
constexpr int kRecG1 = 0, kRecG2 = 1024, kRecBh = 2048, kRecKh = 3072, kRecU = 4096, kRecY0 = 5120,
              kRecV = 6144, kRecGam = 7168, kRecFloats = 7232;
constexpr int kPad = kN + 1;  // a padded 64-channel LDS row

// the chain kernel addresses a (sequence, head)'s records and a sequence's y
// through 32-bit buffer offsets
static bool chunk_offsets_fit(int T, int H, int ybytes) {
  return (int64_t)((T + kCk - 1) / kCk) * kRecFloats * 4 < (int64_t)INT32_MAX &&
         (int64_t)T * H * kN * ybytes < (int64_t)INT32_MAX;
}

bool prefill_chunked(int T, int, int H, int) { return T >= kChunkMinT && chunk_offsets_fit(T, H, 4); }

int64_t wkv7_chunk_rec_bytes(int B, int T, int H) {
  return (int64_t)((T + kCk - 1) / kCk) * H * B * kRecFloats * 4;
}

// D (16 x 16) += A (16 x 4) B (4 x 16), f32: lane l gives A[l % 16][l / 16]
// and B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16], r = 0..3.
RWKV7_DEV floatx4 mfma4(float a, float b, floatx4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

// The LoRA second steps of one chunk and head (PrefillScanArgs::l1), for
// ranks up to kL2Steps 32-wide k-steps each (v, w, a, g: 32, 64, 64, 128 --
// the 0.1B / 0.4B sizes; lora2_fits). Wave w owns the head's channels
// 16 w .. 16 w + 15 and multiplies the chunk's 16 rows of the four LoRA first
// steps by their second matrices on 16x16x32 MFMA -- the products and
// summation order of the GEMM group it replaces (f32 first steps as 16-bit
// hi + lo parts, lanes past a rank multiplying zeros). Every operand load is
// issued before the products (lora2_load, then the stager's own loads), so
// the step costs one memory round trip. v, w, a go to LDS ([3][16][64],
// token-major) for the gate stager; g goes to dg for the GroupNorm + gate
// stage.
constexpr int kL2Steps[4] = {1, 2, 2, 4};
constexpr int kL2Total = 9;
bool lora2_fits(int rv, int rw, int ra, int rg) {
  return rv <= 32 * kL2Steps[0] && rw <= 32 * kL2Steps[1] && ra <= 32 * kL2Steps[2] && rg <= 32 * kL2Steps[3];
}
template <bool F32>
struct Lora2Regs {
  uint4 w[kL2Total];
  uint4 a[kL2Total][F32 ? 2 : 1];
};
template <bool F32>
RWKV7_DEV Lora2Regs<F32> lora2_load(const PrefillScanArgs &p, int h, int bi, int T, int t0, int t1) {
  Lora2Regs<F32> g;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int SR = p.rv + p.rw + p.ra + p.rg;
  const int64_t arow = (int64_t)bi * T + min(t0 + (lane & 15), t1 - 1);  // A row: a token (clamped)
  const uint16_t *wrow = p.w2 + (int64_t)(h * kN + 16 * wv + (lane & 15)) * SR;  // B row: a channel
  const int rk[4] = {p.rv, p.rw, p.ra, p.rg};
  int off = 0, st = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int s = 0; s < kL2Steps[j]; ++s, ++st) {
      const int k = 32 * s + 8 * (lane >> 4);
      const int kc = off + min(k, rk[j] - 8);  // in range; lanes past the rank are zeroed at use
      g.w[st] = *reinterpret_cast<const uint4 *>(wrow + kc);
      if constexpr (F32) {
        const uint4 *a = reinterpret_cast<const uint4 *>(static_cast<const float *>(p.l1) + arow * SR + kc);
        g.a[st][0] = a[0];
        g.a[st][1] = a[1];
      } else {
        g.a[st][0] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p.l1) + arow * SR + kc);
      }
    }
    off += rk[j];
  }
  return g;
}
template <bool BF, bool F32>
RWKV7_DEV void lora2_compute(const PrefillScanArgs &p, const Lora2Regs<F32> &g, int h, int bi, int T, int t0, int t1,
                             float *s_d) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, ch = 16 * wv + (lane & 15);
  const int rk[4] = {p.rv, p.rw, p.ra, p.rg};
  const uint4 zero = make_uint4(0, 0, 0, 0);
  floatx4 acc[4];
  int st = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kL2Steps[j]; ++s, ++st) {
      if (32 * s >= rk[j]) continue;  // uniform
      const bool live = 32 * s + 8 * (lane >> 4) < rk[j];
      if constexpr (F32) {
        uint4 hi, lo;
        split_hi_lo<BF>(live ? g.a[st][0] : zero, live ? g.a[st][1] : zero, hi, lo);
        acc[j] = mfma16<BF>(hi, g.w[st], acc[j]);
        acc[j] = mfma16<BF>(lo, g.w[st], acc[j]);
      } else {
        acc[j] = mfma16<BF>(live ? g.a[st][0] : zero, g.w[st], acc[j]);
      }
    }
  }
  // acc[j][r]: token 4 (lane / 16) + r of the chunk, channel ch of the head
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = 4 * (lane >> 4) + r;
    s_d[t * kN + ch] = acc[0][r];
    s_d[(kCk + t) * kN + ch] = acc[1][r];
    s_d[(2 * kCk + t) * kN + ch] = acc[2][r];
    if (t0 + t < t1) p.dg[((int64_t)bi * T + t0 + t) * p.C + h * kN + ch] = acc[3][r];
  }
}
template <bool BF, bool F32, class St>
RWKV7_DEV void lora2_chunk(const PrefillScanArgs &p, St &st, int h, int bi, int T, int t0, int t1, float *s_d) {
  const Lora2Regs<F32> g = lora2_load<F32>(p, h, bi, T, t0, t1);
  st.fetch(t0);
  lora2_compute<BF, F32>(p, g, h, bi, T, t0, t1, s_d);
}

// L2: the model path with the LoRA second steps formed here (GateStager and
// p.l1 set); a separate instance, whose registers those products no longer
// hold, keeps three workgroups per CU for the other cases.
template <class St, bool L2>
__global__ __launch_bounds__(256) void wkv7_chunk_prep_kernel(typename St::Args p, float *rec, int T, int H) {
  // 35 KB of LDS without the LoRA steps (43 KB with them, which stage there),
  // so that four workgroups share a CU (the 1.5B-shaped 4 x 1024 prefill
  // runs 8192 of them): the stager writes its padded rows straight into s_x,
  // b^ and k^ go from registers straight into the record, and the later
  // 16 x 64 results take the rows that are dead by then -- AkaV and then G2
  // the prefix products', G1 w's, U b's and Y0 k's (each phase below ends
  // with a barrier before the next reuses a row)
  constexpr int NB = L2 ? 3 : 1;
  __shared__ float s_x[6][kCk][kPad];     // w, a (a~), b (b / P), k (k / P), r (r~), v
  __shared__ float s_bkp[NB][kCk][kPad];  // prefix products P_t = D(-1, t] (and the LoRA steps before them)
  __shared__ float s_m[4][kCk][kCk + 1];  // Aba, Aka, Bbr, Bkr
  __shared__ float s_t[kCk][kCk + 1];
  __shared__ float s_gam[kN];
  typedef float Row[kPad];
  Row *s_p = s_bkp[NB - 1];
  Row *s_akav = s_bkp[NB - 1], *s_g2 = s_bkp[NB - 1], *s_g1 = s_x[0], *s_u = s_x[2], *s_y0 = s_x[3];
  static_assert(!L2 || sizeof(s_bkp) >= 3 * kCk * kN * sizeof(float), "LoRA steps staged in s_bkp");

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int row = lane & 15, kq = lane >> 4, col = 16 * wv + row;
  const int c = blockIdx.x, h = blockIdx.y, bi = blockIdx.z;
  const int C = H * kN;
  const int t0 = c * kCk, t1 = min(T, t0 + kCk), Tl = t1 - t0;
  // this chunk's record
  float *R = rec + (((int64_t)bi * H + h) * gridDim.x + c) * kRecFloats;
  St st(p, h, -1, (int64_t)bi * T * C + (int64_t)h * kN, t1);
  bool fetched = false;
  if constexpr (L2 && std::is_same<St, GateStager<kCk>>::value) {
    {
      float *s_d = &s_bkp[0][0][0];  // free until the products below
      if (p.bf) {
        if (p.l1_f32) lora2_chunk<true, true>(p, st, h, bi, T, t0, t1, s_d);
        else lora2_chunk<true, false>(p, st, h, bi, T, t0, t1, s_d);
      } else {
        if (p.l1_f32) lora2_chunk<false, true>(p, st, h, bi, T, t0, t1, s_d);
        else lora2_chunk<false, false>(p, st, h, bi, T, t0, t1, s_d);
      }
      st.lds_d = s_d;
      st.lds_ld = kN;
      fetched = true;
      __syncthreads();
    }
  }
  if (!fetched) st.fetch(t0);
  // padded f32 rows; tokens past the end become identity steps
  st.commit_to(t0, [&](int i, int tt, int qq, float4 x) {
    if (tt >= Tl) x = i == 0 ? make_float4(1.f, 1.f, 1.f, 1.f) : make_float4(0.f, 0.f, 0.f, 0.f);
    s_x[i][tt][4 * qq] = x.x;
    s_x[i][tt][4 * qq + 1] = x.y;
    s_x[i][tt][4 * qq + 2] = x.z;
    s_x[i][tt][4 * qq + 3] = x.w;
  });
  __syncthreads();
  bool ok = true;
  if (tid < kN) {  // wave 0: prefix products P_t, and whether they stay in range
    const int j = tid;
    float P = 1.f;
#pragma unroll
    for (int t = 0; t < kCk; ++t) {
      P *= s_x[0][t][j];
      s_p[t][j] = P;
      ok = ok && P >= 1e-30f && P <= 1e30f;  // false for NaN too
    }
  } else if (tid < 2 * kN) {  // wave 1: suffix products (b^, k^, gam), exact products of w
    const int j = tid - kN;
    float Q = 1.f, bh[kCk], kh[kCk];
#pragma unroll
    for (int t = kCk - 1; t >= 0; --t) {
      bh[t] = s_x[2][t][j] * Q;
      kh[t] = s_x[3][t][j] * Q;
      Q *= s_x[0][t][j];
    }
    s_gam[j] = Q;
    // B operand of the state update, X[4 kk + kq][16 w + row], as the chain
    // kernel's thread 64 w + 16 kq + row reads it (kk = 0..3 in one float4)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int off = 4 * (64 * (j >> 4) + 16 * q + (j & 15));
      *reinterpret_cast<float4 *>(R + kRecBh + off) = make_float4(bh[q], bh[4 + q], bh[8 + q], bh[12 + q]);
      *reinterpret_cast<float4 *>(R + kRecKh + off) = make_float4(kh[q], kh[4 + q], kh[8 + q], kh[12 + q]);
    }
  }
  const bool fast = __syncthreads_and(ok);  // block-uniform
  if (!fast) {  // token matrices straight from products of w: thread (t, s)
    const int t = tid >> 4, s = tid & 15;
    float aba = 0.f, aka = 0.f, bbr = 0.f, bkr = 0.f;
    if (s <= t) {
      for (int j = 0; j < kN; ++j) {
        float d = 1.f;  // D(s, t-1]
        for (int m = s + 1; m < t; ++m) d *= s_x[0][m][j];
        const float dt = s < t ? d * s_x[0][t][j] : 1.f;  // D(s, t]
        const float bs = s_x[2][s][j], ks = s_x[3][s][j], at = s_x[1][t][j], rt = s_x[4][t][j];
        if (s < t) {
          aba = fmaf(bs * d, at, aba);
          aka = fmaf(ks * d, at, aka);
        }
        bbr = fmaf(bs * dt, rt, bbr);
        bkr = fmaf(ks * dt, rt, bkr);
      }
    }
    s_m[0][t][s] = aba;
    s_m[1][t][s] = aka;
    s_m[2][t][s] = bbr;
    s_m[3][t][s] = bkr;
    __syncthreads();
  }
  {  // a~, r~ (and b / P, k / P for the MFMA form) in place: token tid / 16, 4 channels
    const int t = tid >> 4, j0 = 4 * (tid & 15);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u;
      const float P = s_p[t][j], Pp = t > 0 ? s_p[t - 1][j] : 1.f;
      s_x[1][t][j] *= Pp;
      s_x[4][t][j] *= P;
      if (fast) {
        s_x[2][t][j] = s_x[2][t][j] / P;
        s_x[3][t][j] = s_x[3][t][j] / P;
      }
    }
  }
  __syncthreads();
  if (fast) {  // wave m: token matrix m, (a~ or r~) (b / P or k / P)^T, masked
    const int m = wv;
    const Row *X = s_x[m < 2 ? 1 : 4];
    const Row *Y = s_x[(m & 1) ? 3 : 2];
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < kN / 4; ++kk) acc = mfma4(X[row][4 * kk + kq], Y[row][4 * kk + kq], acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * kq + r, s = row;
      s_m[m][t][s] = (m < 2 ? s < t : s <= t) ? acc[r] : 0.f;
    }
    __syncthreads();
  }
  {  // AkaV, value columns 16 wv ..
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = mfma4(s_m[1][row][4 * kk + kq], s_x[5][4 * kk + kq][col], acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) s_akav[4 * kq + r][col] = acc[r];
  }
  if (tid < kCk) {  // T = (I - Aba)^-1 by forward substitution, lane = column
    const int cc = tid;
    float tc[kCk];
#pragma unroll
    for (int t = 0; t < kCk; ++t) {
      float acc = t == cc ? 1.f : 0.f;
#pragma unroll
      for (int s = 0; s < t; ++s) acc = fmaf(s_m[0][t][s], tc[s], acc);
      tc[t] = acc;
      s_t[t][cc] = acc;
    }
  }
  __syncthreads();
  {  // G1 = T A~, U = T AkaV (column block wv)
    floatx4 g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const float tv = s_t[row][4 * kk + kq];
      g = mfma4(tv, s_x[1][4 * kk + kq][col], g);
      u = mfma4(tv, s_akav[4 * kk + kq][col], u);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s_g1[4 * kq + r][col] = g[r];
      s_u[4 * kq + r][col] = u[r];
    }
  }
  __syncthreads();
  {  // G2 = R~ + Bbr G1, Y0 = Bbr U + Bkr V
    floatx4 g2, y0 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r) g2[r] = s_x[4][4 * kq + r][col];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const float bb = s_m[2][row][4 * kk + kq], bk = s_m[3][row][4 * kk + kq];
      g2 = mfma4(bb, s_g1[4 * kk + kq][col], g2);
      y0 = mfma4(bb, s_u[4 * kk + kq][col], y0);
      y0 = mfma4(bk, s_x[5][4 * kk + kq][col], y0);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s_g2[4 * kq + r][col] = g2[r];
      s_y0[4 * kq + r][col] = y0[r];
    }
  }
  __syncthreads();
  // the rest of the record, one float4 per thread and array (thread = wave
  // 64 + lane of the chain kernel's reader)
  const int w = tid >> 6;
  auto put = [&](int off, float a0, float a1, float a2, float a3) {
    *reinterpret_cast<float4 *>(R + off + 4 * tid) = make_float4(a0, a1, a2, a3);
  };
  // A operand of the chain's Sig / Y step: G[row][16 w + 4 kk + kq]
  put(kRecG1, s_g1[row][16 * w + kq], s_g1[row][16 * w + 4 + kq], s_g1[row][16 * w + 8 + kq],
      s_g1[row][16 * w + 12 + kq]);
  put(kRecG2, s_g2[row][16 * w + kq], s_g2[row][16 * w + 4 + kq], s_g2[row][16 * w + 8 + kq],
      s_g2[row][16 * w + 12 + kq]);
  // A operand of the state update (value rows 16 q + row, q = w here)
  put(kRecU, s_u[kq][16 * w + row], s_u[4 + kq][16 * w + row], s_u[8 + kq][16 * w + row],
      s_u[12 + kq][16 * w + row]);
  put(kRecV, s_x[5][kq][16 * w + row], s_x[5][4 + kq][16 * w + row], s_x[5][8 + kq][16 * w + row],
      s_x[5][12 + kq][16 * w + row]);
  {  // Y0[q][t][i] = Y0[t][16 q + i]
    const int e = 4 * tid, q = e >> 8, t = (e >> 4) & 15, i = e & 15;
    put(kRecY0, s_y0[t][16 * q + i], s_y0[t][16 * q + i + 1], s_y0[t][16 * q + i + 2], s_y0[t][16 * q + i + 3]);
  }
  if (tid < kN / 4) put(kRecGam, s_gam[4 * tid], s_gam[4 * tid + 1], s_gam[4 * tid + 2], s_gam[4 * tid + 3]);
}



// One chunk record in LDS as a chain workgroup of NQ value quarters uses it:
// G1, G2, B^, K^ of the four column blocks, then 1 KiB pieces: U, V and Y0
// ([t * 16 + i]) of each of its quarters and gam (the first 64 floats of its
// piece; the rest is what follows gam in the record, unused), one piece per
// wave (with NQ = 2 the last wave fetches gam again).
template <int NQ>
struct ChainSlot {
  float4 g[4][4][64];   // [G1, G2, B^, K^][column block][lane]
  float p5[4 * NQ][256];  // U, V, Y0 of each quarter, gam, padding
};
constexpr int kRing = 3;  // chunk records in LDS: the current one and the next two in flight

// y store of one element: a raw buffer store, dropped by the hardware when the
// offset is past the sequence (tokens of the padded last chunk), so every
// step issues the same memory operations (the wait counts below rely on it)
RWKV7_DEV void store_y(__amdgpu_buffer_rsrc_t r, unsigned off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, off, 0, 0);
}
RWKV7_DEV void store_y(__amdgpu_buffer_rsrc_t r, unsigned off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, 0);
}
RWKV7_DEV void store_y(__amdgpu_buffer_rsrc_t r, unsigned off, bf16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v.bits, r, off, 0, 0);
}

// Grid (4 H / NQ, B), 256 NQ threads: NQ value quarters (16 state rows each)
// of a head per workgroup; wave w takes quarter w / 4 of the workgroup and key
// column block w % 4. With NQ = 2 each record is fetched once for two
// quarters: at many heads the record stream is what bounds the chain.
template <typename TY, int NQ>
__global__ __launch_bounds__(256 * NQ) void wkv7_chunk_chain_kernel(float *S, const float *rec, TY *y, int T, int H) {
  static_assert(NQ == 1 || NQ == 2, "one or two quarters per workgroup");
  __shared__ float s_s[16 * NQ][kPad];  // the workgroup's state rows
  __shared__ float s_xp[NQ][4][kCk][kCk + 1], s_yp[NQ][4][kCk][kCk + 1];  // per-block Sig^T / Y partials [t][i]
  // the ring, one object per slot
  __shared__ ChainSlot<NQ> s_rec0, s_rec1, s_rec2;
  static_assert(kRing == 3, "one object per slot");
  auto slot_ref = [&](int k) -> ChainSlot<NQ> & { return k == 0 ? s_rec0 : k == 1 ? s_rec1 : s_rec2; };
  // wv in a scalar register: the DMA's LDS address derives from it
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qq = wv >> 2, cb = wv & 3;  // this wave's quarter in the workgroup, key column block
  const int row = lane & 15, kq = lane >> 4;
  const int h = blockIdx.x / (4 / NQ), bi = blockIdx.y;
  const int q = blockIdx.x % (4 / NQ) * NQ + qq;  // the quarter's value rows 16 q ..
  const int NC = (T + kCk - 1) / kCk, C = H * kN;
  // lane holds S[16 q + 4 kq + r][16 cb + row], r = 0..3 (the MFMA D layout)
  float *Sp = S + (((int64_t)bi * H + h) * kN + 16 * q) * kN;
  floatx4 st;
#pragma unroll
  for (int r = 0; r < 4; ++r) st[r] = Sp[(4 * kq + r) * kN + 16 * cb + row];
  // this (sequence, head)'s records, and this sequence's y, as buffers
  const i32x4 rr = buffer_words(rec + ((int64_t)bi * H + h) * NC * kRecFloats, NC * kRecFloats * 4);
  const __amdgpu_buffer_rsrc_t yr =
      __builtin_amdgcn_make_buffer_rsrc(y + (int64_t)bi * T * C, 0, (int)((int64_t)T * C * sizeof(TY)), 0x00020000);
  // the record piece that this wave fetches: U, V, Y0 of the workgroup's
  // quarters, then gam (repeated by the waves left over)
  const int q0 = q - qq;  // the workgroup's first quarter
  const int psrc = wv < NQ ? kRecU * 4 + (q0 + wv) * 1024 : wv < 2 * NQ ? kRecV * 4 + (q0 + wv - NQ) * 1024
                 : wv < 3 * NQ ? kRecY0 * 4 + (q0 + wv - 2 * NQ) * 1024 : kRecGam * 4;
  // Record of chunk c into a ring slot: block cb of G1, G2, B^, K^ and one
  // piece per wave (16 bytes per lane landing in lane order). Past the last
  // chunk the last one is loaded again (unused), so the count per step never
  // changes.
  constexpr int kDmaPerWave = 4 / NQ + 1;
  auto dma = [&](int c, int slot) {
    const int cc = c < NC ? c : NC - 1;
    ChainSlot<NQ> &sl = slot_ref(slot);
    const int base = cc * kRecFloats * 4;
    const int offs[4] = {kRecG1, kRecG2, kRecBh, kRecKh};
#pragma unroll
    for (int u = 0; u < 4 / NQ; ++u) {
      const int a = qq * (4 / NQ) + u;  // the waves of column block cb share its four arrays
      dma16(rr, lds_addr(&sl.g[a][cb][0]), offs[a] * 4 + (64 * cb + lane) * 16, base);
    }
    // one piece per wave into p5[wave] (past the record's end the buffer
    // returns zeros)
    dma16(rr, lds_addr(&sl.p5[wv][0]), psrc + lane * 16, base);
  };
  // Each step issues one record's DMAs and then one y store per wave; the
  // prologue pairs each record with a y store that the buffer drops. So at
  // the wait of chunk c's step exactly kVm memory operations were issued
  // after chunk c's DMAs: the y stores of the kRing - 1 steps (or prologue
  // entries) since, and the DMAs of the kRing - 2 records in between. The
  // counter counts loads and stores in issue order, so waiting for at most
  // kVm outstanding waits for chunk c's record and nothing later.
  constexpr int kVm = kDmaPerWave * (kRing - 2) + (kRing - 1);
  static_assert(kVm < 16, "vmcnt field (low bits only)");
  constexpr int kWaitRec = 0x0F70 | kVm;
#pragma unroll
  for (int c = 0; c < kRing - 1; ++c) {
    dma(c, c);
    store_y(yr, 0xFFFFFFF0u, from_f<TY>(0.f));  // past the buffer: dropped
  }
  // slot: c % kRing, a constant in the unrolled loop below, so that every
  // slot address is a constant offset
  auto step = [&](int c, int slot) {
    const ChainSlot<NQ> &sl = slot_ref(slot);
#pragma unroll
    for (int r = 0; r < 4; ++r) s_s[16 * qq + 4 * kq + r][16 * cb + row] = st[r];
    __builtin_amdgcn_s_waitcnt(kWaitRec);  // this wave's DMAs of chunk c have landed
    // everyone's have, and the state tile is in LDS: a bare barrier after the
    // LDS stores (a memory fence would also wait for the DMAs still in flight)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    dma(c + kRing - 1, (slot + kRing - 1) % kRing);  // the slot of chunk c - 1: its readers passed the barrier
    const float4 g1 = sl.g[0][cb][lane], g2 = sl.g[1][cb][lane], kh = sl.g[3][cb][lane];
    const float4 vv = reinterpret_cast<const float4 *>(sl.p5[NQ + qq])[lane];
    const float G1[4] = {g1.x, g1.y, g1.z, g1.w}, G2[4] = {g2.x, g2.y, g2.z, g2.w};
    const float V[4] = {vv.x, vv.y, vv.z, vv.w}, KH[4] = {kh.x, kh.y, kh.z, kh.w};
    // S diag(gam) + V^T K^ does not depend on Sig: formed while the Sig
    // products run
    const float gam = sl.p5[3 * NQ][16 * cb + row];
    floatx4 acc;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = st[r] * gam;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = mfma4(V[kk], KH[kk], acc);
    // Sig^T and Y over this wave's 16 key columns: D[t][i] = sum_j G[t][j] S[i][j]
    floatx4 xa = {0.f, 0.f, 0.f, 0.f}, ya = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const float sv = s_s[16 * qq + row][16 * cb + 4 * kk + kq];
      xa = mfma4(G1[kk], sv, xa);
      ya = mfma4(G2[kk], sv, ya);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s_xp[qq][cb][4 * kq + r][row] = xa[r];
      s_yp[qq][cb][4 * kq + r][row] = ya[r];
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // S <- S diag(gam) + V^T K^ + Sig^T B^ (this wave's 16 columns)
    const float4 bh = sl.g[2][cb][lane];
    const float4 u = reinterpret_cast<const float4 *>(sl.p5[qq])[lane];
    const float BH[4] = {bh.x, bh.y, bh.z, bh.w}, U[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int t = 4 * kk + kq;
      const float xv = ((s_xp[qq][0][t][row] + s_xp[qq][1][t][row]) + (s_xp[qq][2][t][row] + s_xp[qq][3][t][row])) + U[kk];
      acc = mfma4(xv, BH[kk], acc);
    }
    st = acc;
    {  // y of token t, value row 16 q + i (past the sequence: dropped by the buffer)
      const int lt = tid & 255, t = lt >> 4, i = lt & 15, tt = c * kCk + t;
      const float yv = ((s_yp[qq][0][t][i] + s_yp[qq][1][t][i]) + (s_yp[qq][2][t][i] + s_yp[qq][3][t][i])) + sl.p5[2 * NQ + qq][lt];
      const unsigned off = tt < T ? (unsigned)(((int64_t)tt * C + h * kN + 16 * q + i) * sizeof(TY)) : 0xFFFFFFF0u;
      store_y(yr, off, from_f<TY>(yv));
    }
  };
  for (int c0 = 0; c0 < NC; c0 += kRing) {
#pragma unroll
    for (int k = 0; k < kRing; ++k)
      if (c0 + k < NC) step(c0 + k, k);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // the clamped DMAs land before the workgroup's LDS is reused
#pragma unroll
  for (int r = 0; r < 4; ++r) Sp[(4 * kq + r) * kN + 16 * cb + row] = st[r];
}

template <class St, typename TY>
static int launch_chunked(const typename St::Args &p, float *S, TY *y, float *rec, int B, int T, int H,
                          hipStream_t st) {
  if (!rec) return RWKV7_EWORKSPACE;
  const int nc = (T + kCk - 1) / kCk;
  if constexpr (std::is_same<St, GateStager<kCk>>::value) {
    if (p.l1) wkv7_chunk_prep_kernel<St, true><<<dim3(nc, H, B), 256, 0, st>>>(p, rec, T, H);
    else wkv7_chunk_prep_kernel<St, false><<<dim3(nc, H, B), 256, 0, st>>>(p, rec, T, H);
  } else {
    wkv7_chunk_prep_kernel<St, false><<<dim3(nc, H, B), 256, 0, st>>>(p, rec, T, H);
  }
  RWKV7_CHECK_LAUNCH();
  // two value quarters per workgroup (each record fetched once for both)
  // where that still leaves a workgroup per CU
  if (2 * B * H >= (mk_cus() > 0 ? mk_cus() : 256))
    wkv7_chunk_chain_kernel<TY, 2><<<dim3(2 * H, B), 512, 0, st>>>(S, rec, y, T, H);
  else
    wkv7_chunk_chain_kernel<TY, 1><<<dim3(4 * H, B), 256, 0, st>>>(S, rec, y, T, H);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

template <typename TI, typename TW, typename TY>
int launch_wkv7_chunked(const ScanArgs<TI, TW, TY> &p, float *rec, hipStream_t st) {
  if (p.T <= 0 || p.B <= 0 || p.H <= 0) return RWKV7_OK;
  if (!chunk_offsets_fit(p.T, p.H, (int)sizeof(TY))) return RWKV7_ESHAPE;
  return launch_chunked<RawStager<kCk, TI, TW, TY>, TY>(p, p.S, p.y, rec, p.B, p.T, p.H, st);
}
template int launch_wkv7_chunked<uint16_t, float, uint16_t>(const ScanArgs<uint16_t, float, uint16_t> &, float *,
                                                            hipStream_t);
template int launch_wkv7_chunked<uint16_t, uint16_t, uint16_t>(const ScanArgs<uint16_t, uint16_t, uint16_t> &,
                                                               float *, hipStream_t);
template int launch_wkv7_chunked<bf16_t, float, bf16_t>(const ScanArgs<bf16_t, float, bf16_t> &, float *,
                                                        hipStream_t);
template int launch_wkv7_chunked<bf16_t, bf16_t, bf16_t>(const ScanArgs<bf16_t, bf16_t, bf16_t> &, float *,
                                                         hipStream_t);
template int launch_wkv7_chunked<float, float, float>(const ScanArgs<float, float, float> &, float *, hipStream_t);

int launch_wkv7_prefill(const PrefillScanArgs &p, hipStream_t st) {
  if (p.T <= 0 || p.B <= 0 || p.H <= 0) return RWKV7_OK;
  if (p.C != p.H * kN) return RWKV7_ESHAPE;
  const int cus = mk_cus() > 0 ? mk_cus() : 256;
  if (prefill_chunked(p.T, p.B, p.H, cus))
    return launch_chunked<GateStager<kCk>, float>(p, p.S, p.y, p.rec, p.B, p.T, p.H, st);
  int seg_len;
  const int nseg = prefill_segments(p.T, p.B, p.H, cus, &seg_len);
  if (nseg > 1 && (!p.U || !p.Send || !p.Pend)) return RWKV7_EWORKSPACE;
  if (p.T == 1)
    dplr_scan_kernel<false, 1, GateStager<1>><<<dim3(4 * p.H, p.B, 1), 256, 0, st>>>(p, seg_len, nseg);
  else if (nseg == 1)
    dplr_scan_kernel<false, kCh, GateStager<kCh>><<<dim3(4 * p.H, p.B, 1), 256, 0, st>>>(p, seg_len, nseg);
  else
    dplr_scan_kernel<true, kCh, GateStager<kCh>><<<dim3(4 * p.H, p.B, nseg), 256, 0, st>>>(p, seg_len, nseg);
  RWKV7_CHECK_LAUNCH();
  if (nseg > 1) {
    const int nblk = (seg_len + kCh - 1) / kCh;
    wkv7_prefill_combine_kernel<<<dim3(4 * p.H, p.B, (nseg - 1) * nblk), 256, 0, st>>>(p, seg_len, nseg);
    RWKV7_CHECK_LAUNCH();
  }
  return RWKV7_OK;
}

// ---------------------------------------------------------------------------
// Prefill elementwise stages. Rows m = b * T + t of the [M, C] activations.
// ---------------------------------------------------------------------------

// Block-wide sum over 256 threads (4 waves); all threads get the result.
RWKV7_DEV float block_sum256(float v, float *scratch4) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch4[w] = v;
  __syncthreads();
  return (scratch4[0] + scratch4[1]) + (scratch4[2] + scratch4[3]);
}

constexpr int kMaxCPer = 16;  // C <= 4096
// Loop over the C/256 per-thread elements with a compile-time bound so the
// per-thread arrays stay in registers.
#define RWKV7_UNROLL_N(i) _Pragma("unroll") for (int i = 0; i < kMaxCPer; ++i) if (i < n)

// Token shift of prefill (demo/rwkv7_torch.py:189-197, 251-254): prev[t] =
// LN(x0[t-1]) and prev[0] = state; the state becomes LN(x0[T-1]). The
// workgroup that holds row t = 0 is the only one that touches that
// sequence's state (or that state's column slice): it reads it and then
// writes the new value, so there is no cross-workgroup hazard.
//
// Two regimes, by the number of rows M:
// * few rows (decode, short prefills): latency-bound, so every load is issued
//   up front and a row's output columns are split over `ncs` workgroups;
//   each reads the whole row for the statistics but only its slice of the
//   LayerNorm and mix vectors (the 6 mix vectors are most of a row's bytes),
//   so more CUs share the row's traffic;
// * many rows (long prefills): bound by the bytes moved into CUs, so a
//   workgroup takes R consecutive rows and loads the LayerNorm and mix
//   vectors once for all of them; a row's normalised predecessor is the
//   previous row's result, kept in registers.
// Statistics: two-pass mean / variance per row (as ln_row), the rows needed at
// once sharing two block reductions.
RWKV7_DEV void block_sum3(float &a, float &b, float &c, float (*red)[4]) {
  a = wave_sum(a);
  b = wave_sum(b);
  c = wave_sum(c);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = a;
    red[1][w] = b;
    red[2][w] = c;
  }
  __syncthreads();
  a = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
  b = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  c = (red[2][0] + red[2][1]) + (red[2][2] + red[2][3]);
}

// The mix vector (row of a.mu) of output slot j: stored order, or with RKV
// (LnShiftArgs::mix_order 1) r, k, v, w, a, g. A compile-time choice: a
// run-time select of the row made the row kernel wait for its vector loads
// one at a time.
template <bool RKV>
constexpr int mix_row(int j) {
  return !RKV ? j : j == 1 ? 2 : j == 2 ? 3 : j == 3 ? 1 : j;
}

// A mixed value into the output: f32, or the model's 16-bit format.
RWKV7_DEV void store_mix(const LnShiftArgs &a, int64_t i, float v) {
  if (a.out_f32) static_cast<float *>(a.out)[i] = v;
  else static_cast<uint16_t *>(a.out)[i] = f_to_u16(v, a.bf);
}

// One row per workgroup, every load up front (measured faster than the
// kernel below for C <= 1024 below 1024 rows).
template <int NP>
__global__ __launch_bounds__(256) void ln_shift_row_kernel(LnShiftArgs a) {
  __shared__ float red[2][3][4];
  const int m = blockIdx.x;
  const int t = m % a.T, b = m / a.T;
  const int C = a.C, tid = threadIdx.x;
  const bool has_prev = t > 0, has_last = t == 0 && a.T > 1;
  const float *rc = a.x0 + (int64_t)m * C;
  const float *rp = a.x0 + (int64_t)(has_prev ? m - 1 : m) * C;
  const float *rl = a.x0 + (int64_t)(has_last ? m + a.T - 1 : m) * C;
  uint16_t *sh = a.shift + (int64_t)b * C;
  float xc[NP], xp[NP], xl[NP], lw[NP], lb[NP], mu[6][NP];
  uint16_t st[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int c = tid + 256 * i;
    xc[i] = rc[c];
    xp[i] = rp[c];
    xl[i] = rl[c];
    lw[i] = a.ln_w[c];
    lb[i] = a.ln_b[c];
    st[i] = sh[c];
  }
#pragma unroll
  for (int j = 0; j < 6; ++j)
#pragma unroll
    for (int i = 0; i < NP; ++i) mu[j][i] = a.mu[(int64_t)(j < a.n_mix ? j : 0) * C + tid + 256 * i];

  float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    s0 += xc[i];
    s1 += xp[i];
    s2 += xl[i];
  }
  block_sum3(s0, s1, s2, red[0]);
  const float invC = 1.f / (float)C;
  const float m0 = s0 * invC, m1 = s1 * invC, m2 = s2 * invC;
  float q0 = 0.f, q1 = 0.f, q2 = 0.f;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    q0 += (xc[i] - m0) * (xc[i] - m0);
    q1 += (xp[i] - m1) * (xp[i] - m1);
    q2 += (xl[i] - m2) * (xl[i] - m2);
  }
  block_sum3(q0, q1, q2, red[1]);
  const float r0 = rsqrtf(q0 * invC + kLnEps), r1 = rsqrtf(q1 * invC + kLnEps), r2 = rsqrtf(q2 * invC + kLnEps);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    xc[i] = (xc[i] - m0) * r0 * lw[i] + lb[i];
    xp[i] = has_prev ? (xp[i] - m1) * r1 * lw[i] + lb[i] : u16_to_f(st[i], a.bf);
  }
  for (int j = 0; j < a.n_mix; ++j) {
    const int64_t o = ((int64_t)j * a.M + m) * C;
#pragma unroll
    for (int i = 0; i < NP; ++i) store_mix(a, o + tid + 256 * i, xc[i] + mu[j][i] * (xp[i] - xc[i]));
  }
  if (t == 0) {
#pragma unroll
    for (int i = 0; i < NP; ++i)
      sh[tid + 256 * i] = f_to_u16(has_last ? (xl[i] - m2) * r2 * lw[i] + lb[i] : xc[i], a.bf);
  }
}

template <int NP, bool RKV>
__global__ __launch_bounds__(256) void ln_shift_kernel(LnShiftArgs a, int R, int ncs) {
  __shared__ float red[2][3][4];
  const int C = a.C, tid = threadIdx.x, T = a.T;
  // this workgroup's output columns: blocks i0 .. i0 + per of the NP
  // 256-column blocks (column tid + 256 i)
  const int per = NP / ncs, i0 = blockIdx.y * per;
  auto mine = [&](int i) { return i >= i0 && i < i0 + per; };
  const int m0 = blockIdx.x * R, m1 = min(a.M, m0 + R);
  // Row m's inputs: the row, its predecessor unless already normalised, and
  // for t = 0 of a multi-token sequence its last token (the new state) and
  // the old state. Loaded before the vectors below and at the end of the
  // previous row, so that no wait separates them from other loads.
  float xc[NP], xp[NP], xl[NP];
  uint16_t st[NP];
  auto load_row = [&](int m, bool have_prev) {
    const int t = m % T, b = m / T;
    const bool need_p = t > 0 && !have_prev, need_l = t == 0 && T > 1;
    const float *rc = a.x0 + (int64_t)m * C;
    const float *rp = a.x0 + (int64_t)(need_p ? m - 1 : m) * C;
    const float *rl = a.x0 + (int64_t)(need_l ? m + T - 1 : m) * C;
    const uint16_t *sh = a.shift + (int64_t)b * C;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int c = tid + 256 * i;
      xc[i] = rc[c];
      xp[i] = need_p ? rp[c] : 0.f;
      xl[i] = need_l ? rl[c] : 0.f;
      st[i] = t == 0 && mine(i) ? sh[c] : (uint16_t)0;
    }
  };
  load_row(m0, false);
  float lw[NP], lb[NP], mu[6][NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    lw[i] = lb[i] = 0.f;
#pragma unroll
    for (int j = 0; j < 6; ++j) mu[j][i] = 0.f;
    if (mine(i)) {
      const int c = tid + 256 * i;
      lw[i] = a.ln_w[c];
      lb[i] = a.ln_b[c];
#pragma unroll
      for (int j = 0; j < 6; ++j)
        if (j < a.n_mix) mu[j][i] = a.mu[(int64_t)mix_row<RKV>(j) * C + c];
    }
  }
  const float invC = 1.f / (float)C;
  float prev[NP];  // LN of the row before m (this slice), once computed
  bool have_prev = false;
  for (int m = m0; m < m1; ++m) {
    const int t = m % T, b = m / T;
    const bool need_p = t > 0 && !have_prev, need_l = t == 0 && T > 1;
    uint16_t *sh = a.shift + (int64_t)b * C;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      s0 += xc[i];
      s1 += xp[i];
      s2 += xl[i];
    }
    block_sum3(s0, s1, s2, red[0]);
    const float mc = s0 * invC, mp = s1 * invC, ml = s2 * invC;
    float q0 = 0.f, q1 = 0.f, q2 = 0.f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      q0 += (xc[i] - mc) * (xc[i] - mc);
      q1 += (xp[i] - mp) * (xp[i] - mp);
      q2 += (xl[i] - ml) * (xl[i] - ml);
    }
    block_sum3(q0, q1, q2, red[1]);
    const float rc0 = rsqrtf(q0 * invC + kLnEps), rp0 = rsqrtf(q1 * invC + kLnEps), rl0 = rsqrtf(q2 * invC + kLnEps);
    float xn[NP], pv[NP], ns[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      xn[i] = (xc[i] - mc) * rc0 * lw[i] + lb[i];
      pv[i] = t == 0 ? u16_to_f(st[i], a.bf) : need_p ? (xp[i] - mp) * rp0 * lw[i] + lb[i] : prev[i];
      ns[i] = need_l ? (xl[i] - ml) * rl0 * lw[i] + lb[i] : xn[i];
    }
    if (m + 1 < m1) load_row(m + 1, true);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      if (!mine(i)) continue;
      const int c = tid + 256 * i;
#pragma unroll
      for (int j = 0; j < 6; ++j)
        if (j < a.n_mix) store_mix(a, ((int64_t)j * a.M + m) * C + c, xn[i] + mu[j][i] * (pv[i] - xn[i]));
      if (t == 0) sh[c] = f_to_u16(ns[i], a.bf);
      prev[i] = xn[i];
    }
    have_prev = true;
  }
}

// The many-rows regime of ln_shift_kernel with each thread on NP consecutive
// columns (NP a multiple of 4), so that every load and store is a vector
// access: 16 bytes per lane for f32 rows and vectors, 8 or 16 for the 16-bit
// mix rows and shift states (ln_shift_kernel's column-strided layout stores
// the six 16-bit mix rows two bytes per lane, 6 NP stores per thread and row).
template <int NP, bool RKV>
__global__ __launch_bounds__(256) void ln_shift_vec_kernel(LnShiftArgs a, int R) {
  static_assert(NP % 4 == 0, "whole float4 pieces per thread");
  constexpr int NV = NP / 4;
  __shared__ float red[2][3][4];
  const int C = a.C, tid = threadIdx.x, T = a.T, c0 = NP * tid;
  const int m0 = blockIdx.x * R, m1 = min(a.M, m0 + R);
  auto ld = [&](const float *row, float (&d)[NP]) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const float4 q = reinterpret_cast<const float4 *>(row + c0)[v];
      d[4 * v] = q.x;
      d[4 * v + 1] = q.y;
      d[4 * v + 2] = q.z;
      d[4 * v + 3] = q.w;
    }
  };
  float xc[NP], xp[NP], xl[NP];
  uint32_t st[NP / 2];  // the old shift state, two 16-bit values per word
  auto load_row = [&](int m, bool have_prev) {
    const int t = m % T, b = m / T;
    ld(a.x0 + (int64_t)m * C, xc);
#pragma unroll
    for (int i = 0; i < NP; ++i) xp[i] = xl[i] = 0.f;
    if (t > 0 && !have_prev) ld(a.x0 + (int64_t)(m - 1) * C, xp);
    if (t == 0 && T > 1) ld(a.x0 + (int64_t)(m + T - 1) * C, xl);
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      uint2 u = make_uint2(0u, 0u);
      if (t == 0) u = reinterpret_cast<const uint2 *>(a.shift + (int64_t)b * C + c0)[v];
      st[2 * v] = u.x;
      st[2 * v + 1] = u.y;
    }
  };
  load_row(m0, false);
  float lw[NP], lb[NP], mu[6][NP];
  ld(a.ln_w, lw);
  ld(a.ln_b, lb);
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    if (j < a.n_mix) ld(a.mu + (int64_t)mix_row<RKV>(j) * C, mu[j]);
    else
#pragma unroll
      for (int i = 0; i < NP; ++i) mu[j][i] = 0.f;
  }
  const float invC = 1.f / (float)C;
  float prev[NP];  // LN of the row before m, once computed
  bool have_prev = false;
  for (int m = m0; m < m1; ++m) {
    const int t = m % T, b = m / T;
    const bool need_p = t > 0 && !have_prev, need_l = t == 0 && T > 1;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      s0 += xc[i];
      s1 += xp[i];
      s2 += xl[i];
    }
    block_sum3(s0, s1, s2, red[0]);
    const float mc = s0 * invC, mp = s1 * invC, ml = s2 * invC;
    float q0 = 0.f, q1 = 0.f, q2 = 0.f;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      q0 += (xc[i] - mc) * (xc[i] - mc);
      q1 += (xp[i] - mp) * (xp[i] - mp);
      q2 += (xl[i] - ml) * (xl[i] - ml);
    }
    block_sum3(q0, q1, q2, red[1]);
    const float rc0 = rsqrtf(q0 * invC + kLnEps), rp0 = rsqrtf(q1 * invC + kLnEps), rl0 = rsqrtf(q2 * invC + kLnEps);
    float xn[NP], pv[NP], ns[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const uint16_t sv = (uint16_t)(st[i >> 1] >> (16 * (i & 1)));
      xn[i] = (xc[i] - mc) * rc0 * lw[i] + lb[i];
      pv[i] = t == 0 ? u16_to_f(sv, a.bf) : need_p ? (xp[i] - mp) * rp0 * lw[i] + lb[i] : prev[i];
      ns[i] = need_l ? (xl[i] - ml) * rl0 * lw[i] + lb[i] : xn[i];
    }
    if (m + 1 < m1) load_row(m + 1, true);
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      if (j >= a.n_mix) continue;
      float o[NP];
#pragma unroll
      for (int i = 0; i < NP; ++i) o[i] = xn[i] + mu[j][i] * (pv[i] - xn[i]);
      const int64_t base = ((int64_t)j * a.M + m) * C + c0;
      if (a.out_f32) {
        float4 *dst = reinterpret_cast<float4 *>(static_cast<float *>(a.out) + base);
#pragma unroll
        for (int v = 0; v < NV; ++v) dst[v] = make_float4(o[4 * v], o[4 * v + 1], o[4 * v + 2], o[4 * v + 3]);
      } else {
        uint32_t w[NP / 2];
#pragma unroll
        for (int i = 0; i < NP / 2; ++i)
          w[i] = (uint32_t)f_to_u16(o[2 * i], a.bf) | ((uint32_t)f_to_u16(o[2 * i + 1], a.bf) << 16);
        uint16_t *dst = static_cast<uint16_t *>(a.out) + base;
        if constexpr (NP % 8 == 0) {
#pragma unroll
          for (int v = 0; v < NP / 8; ++v)
            reinterpret_cast<uint4 *>(dst)[v] = make_uint4(w[4 * v], w[4 * v + 1], w[4 * v + 2], w[4 * v + 3]);
        } else {
#pragma unroll
          for (int v = 0; v < NV; ++v) reinterpret_cast<uint2 *>(dst)[v] = make_uint2(w[2 * v], w[2 * v + 1]);
        }
      }
    }
    if (t == 0) {
      uint2 *sh = reinterpret_cast<uint2 *>(a.shift + (int64_t)b * C + c0);
#pragma unroll
      for (int v = 0; v < NV; ++v)
        sh[v] = make_uint2((uint32_t)f_to_u16(ns[4 * v], a.bf) | ((uint32_t)f_to_u16(ns[4 * v + 1], a.bf) << 16),
                           (uint32_t)f_to_u16(ns[4 * v + 2], a.bf) | ((uint32_t)f_to_u16(ns[4 * v + 3], a.bf) << 16));
    }
#pragma unroll
    for (int i = 0; i < NP; ++i) prev[i] = xn[i];
    have_prev = true;
  }
}

int launch_ln_shift(const LnShiftArgs &a, hipStream_t st) {
  if (a.C % 256 || a.C > 256 * kMaxCPer || a.n_mix < 1 || a.n_mix > 6 || a.M <= 0 || a.T <= 0) return RWKV7_ESHAPE;
  const int np = a.C / 256;
  // about two workgroups per CU: many rows share a workgroup, few rows are
  // split over column slices (a power of two dividing np); rows of at most
  // 1024 columns below that take one workgroup each (measured: 0.4B prefill
  // 1 x 128 1.88 ms against 1.93 with column slices, 1 x 512 3.39 against
  // 3.43 with the same grid)
  const int want = 2 * (mk_cus() > 0 ? mk_cus() : 256);
  int R = 1, ncs = 1;
  if (a.M >= 2 * want) R = min(8, a.M / want);
  else
    while (ncs * 2 <= np && np % (ncs * 2) == 0 && (int64_t)a.M * ncs < want) ncs *= 2;
  const bool rkv = a.mix_order != 0;  // only the two other kernels take this order
  const bool row_kernel = R == 1 && np <= 4 && !rkv;
  const dim3 grid((a.M + R - 1) / R, row_kernel ? 1 : ncs);
  // the vector form at C = 1024 and 2048 (the 0.4B and 1.5B widths; at 4096
  // its registers would leave one wave per SIMD)
  if (R > 1 && (np == 4 || np == 8)) {
    if (np == 4) {
      if (rkv) ln_shift_vec_kernel<4, true><<<grid, 256, 0, st>>>(a, R);
      else ln_shift_vec_kernel<4, false><<<grid, 256, 0, st>>>(a, R);
    } else {
      if (rkv) ln_shift_vec_kernel<8, true><<<grid, 256, 0, st>>>(a, R);
      else ln_shift_vec_kernel<8, false><<<grid, 256, 0, st>>>(a, R);
    }
    RWKV7_CHECK_LAUNCH();
    return RWKV7_OK;
  }
  switch (np) {
#define RWKV7_LNS_CASE(n)                                                   \
  case n:                                                                   \
    if (row_kernel) ln_shift_row_kernel<n><<<grid, 256, 0, st>>>(a);        \
    else if (rkv) ln_shift_kernel<n, true><<<grid, 256, 0, st>>>(a, R, ncs); \
    else ln_shift_kernel<n, false><<<grid, 256, 0, st>>>(a, R, ncs);        \
    break;
    RWKV7_LNS_CASE(1) RWKV7_LNS_CASE(2) RWKV7_LNS_CASE(3) RWKV7_LNS_CASE(4)
    RWKV7_LNS_CASE(5) RWKV7_LNS_CASE(6) RWKV7_LNS_CASE(7) RWKV7_LNS_CASE(8)
    RWKV7_LNS_CASE(9) RWKV7_LNS_CASE(10) RWKV7_LNS_CASE(11) RWKV7_LNS_CASE(12)
    RWKV7_LNS_CASE(13) RWKV7_LNS_CASE(14) RWKV7_LNS_CASE(15) RWKV7_LNS_CASE(16)
#undef RWKV7_LNS_CASE
    default: return RWKV7_ESHAPE;
  }
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}


// GroupNorm + r.k.r_k bonus + gate (demo/rwkv7_torch.py:234-242).
__global__ __launch_bounds__(256) void gn_gate_kernel(GnGateArgs a) {
  const int C = a.C, H = C / kN;
  const int gh = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int m = gh / H, h = gh % H;
  if (m >= a.M) return;
  const int ch = h * kN + (threadIdx.x & 63);
  const int64_t o = (int64_t)m * C + ch;
  const float y = a.y[o];
  const float mean = wave_sum(y) * (1.f / kN);
  const float d = y - mean;
  const float var = wave_sum(d * d) * (1.f / kN);
  const float yn = d * rsqrtf(var + kGnEps) * a.vec[RWKV7_V_LNX_W * C + ch] + a.vec[RWKV7_V_LNX_B * C + ch];
  const float rk = wave_sum(a.r[o] * a.kn[o] * a.vec[RWKV7_V_R_K * C + ch]);
  const float out = (yn + rk * a.v[o]) * a.g[o];
  if (a.out_f32) static_cast<float *>(a.out)[o] = out;
  else static_cast<uint16_t *>(a.out)[o] = f_to_u16(out, a.bf);
}

int launch_gn_gate(const GnGateArgs &a, hipStream_t st) {
  const int waves = a.M * (a.C / kN);
  gn_gate_kernel<<<(waves + 3) / 4, 256, 0, st>>>(a);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

// ---------------------------------------------------------------------------
// Small utility kernels.
// ---------------------------------------------------------------------------

// x0[m] = emb[tok[m]] as f32 (F.embedding, demo/rwkv7_torch.py:173-175).
__global__ void embed_kernel(const int64_t *tok, const uint16_t *emb, float *x0, int C, int V, int bf) {
  const int m = blockIdx.x;
  int64_t id = tok[m];
  id = id < 0 ? 0 : id >= V ? V - 1 : id;
  const uint16_t *row = emb + id * C;
  for (int c = threadIdx.x; c < C; c += blockDim.x) x0[(int64_t)m * C + c] = u16_to_f(row[c], bf);
}

int launch_embed(const int64_t *tok, const uint16_t *emb, float *x0, int M, int C, int V, int bf, hipStream_t st) {
  embed_kernel<<<M, 256, 0, st>>>(tok, emb, x0, C, V, bf);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

// out[i] = f16(LN(x[row_i])) with row_i = i * stride + offset (gathers the
// last token of each sequence before the LM head).
__global__ __launch_bounds__(256) void ln_rows_kernel(const void *x, int x_f32, const float *w,
                                                      const float *bvec, void *out, int out_f32,
                                                      int C, int stride, int offset, int bf) {
  __shared__ float scratch4[4];
  const int i = blockIdx.x;
  const int64_t src = (int64_t)i * stride + offset;
  const int n = C >> 8;
  float v[kMaxCPer];
  float s = 0.f;
  RWKV7_UNROLL_N(q) {
    const int c = threadIdx.x + 256 * q;
    v[q] = x_f32 ? reinterpret_cast<const float *>(x)[src * C + c]
                 : u16_to_f(reinterpret_cast<const uint16_t *>(x)[src * C + c], bf);
    s += v[q];
  }
  const float mean = block_sum256(s, scratch4) / (float)C;
  float qv = 0.f;
  RWKV7_UNROLL_N(q) {
    const float d = v[q] - mean;
    qv += d * d;
  }
  const float rstd = rsqrtf(block_sum256(qv, scratch4) / (float)C + kLnEps);
  RWKV7_UNROLL_N(q) {
    const int c = threadIdx.x + 256 * q;
    const float y = (v[q] - mean) * rstd * w[c] + bvec[c];
    if (out_f32) reinterpret_cast<float *>(out)[(int64_t)i * C + c] = y;
    else reinterpret_cast<uint16_t *>(out)[(int64_t)i * C + c] = f_to_u16(y, bf);
  }
}

int launch_ln_rows(const void *x, int x_f32, const float *w, const float *b, void *out, int out_f32,
                   int rows, int C, int stride, int offset, int bf, hipStream_t st) {
  if (C % 256 || C > 256 * kMaxCPer) return RWKV7_ESHAPE;
  ln_rows_kernel<<<rows, 256, 0, st>>>(x, x_f32, w, b, out, out_f32, C, stride, offset, bf);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

// Token-shift lerps for one vector (src/rwkv_tl/kernels/lerp.py:140-198).
__global__ void lerp_kernel(const uint16_t *x, const uint16_t *prev, const float *mu, int n_mix,
                            uint16_t *out, uint16_t *x_copy, int C, int bf) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const float xv = u16_to_f(x[c], bf), pv = u16_to_f(prev[c], bf);
  for (int j = 0; j < n_mix; ++j) out[(int64_t)j * C + c] = f_to_u16(xv + mu[(int64_t)j * C + c] * (pv - xv), bf);
  if (x_copy) x_copy[c] = x[c];  // after this thread's read of prev[c]
}

int launch_lerp(const uint16_t *x, const uint16_t *prev, const float *mu, int n_mix, uint16_t *out,
                uint16_t *x_copy, int C, int bf, hipStream_t st) {
  lerp_kernel<<<(C + 255) / 256, 256, 0, st>>>(x, prev, mu, n_mix, out, x_copy, C, bf);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

// Copies f32 -> 16-bit (decode: the channel-mix token-shift state update
// after the FFN key GEMV has read the old state).
__global__ void store_f16_kernel(const float *src, uint16_t *dst, int n, int bf) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = f_to_u16(src[i], bf);
}

int launch_store_f16(const float *src, uint16_t *dst, int n, int bf, hipStream_t st) {
  store_f16_kernel<<<(n + 255) / 256, 256, 0, st>>>(src, dst, n, bf);
  RWKV7_CHECK_LAUNCH();
  return RWKV7_OK;
}

}  // namespace rwkv7
