// C ABI of librwkv7_hip.so: layouts, workspace sizing, the decode and prefill
// step sequencers and the operator-level entry points. Host code only; the
// kernels live in gemv.hip, tmix.hip and gemm.hip.
#include <stdlib.h>
#include <string.h>

#include "rwkv7_kernels.h"

namespace rwkv7 {

// ---- layouts -------------------------------------------------------------

static int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

static int check_dims(const rwkv7_dims *d) {
  if (!d) return RWKV7_EINVAL;
  const int C = d->n_embd;
  if (d->n_layer < 1 || C < 256 || C % 256 || C > 4096 || d->n_head * kN != C) return RWKV7_ESHAPE;
  if (d->n_ffn < 256 || d->n_ffn % 256 || d->n_ffn > 8192 || d->vocab < 1) return RWKV7_ESHAPE;
  const int r[4] = {d->rank_w, d->rank_a, d->rank_v, d->rank_g};
  int sr = 0;
  for (int i = 0; i < 4; ++i) {
    if (r[i] < 8 || r[i] % 8) return RWKV7_ESHAPE;
    sr += r[i];
  }
  if (sr > 512) return RWKV7_ESHAPE;
  return RWKV7_OK;
}

static int sum_ranks(const rwkv7_dims &d) { return d.rank_w + d.rank_a + d.rank_v + d.rank_g; }

// bytes of an [N, K] matrix in fragment order (N, K padded to 16, 32)
static int64_t frag_bytes(int64_t N, int64_t K) { return ((N + 15) / 16 * 16) * ((K + 31) / 32 * 32) * 2; }

static void layout_of(const rwkv7_dims &d, rwkv7_layer_layout *o) {
  const int64_t C = d.n_embd, F = d.n_ffn, SR = sum_ranks(d);
  int64_t off = 0;
  o->w_rkv = off;
  off += 3 * C * C * 2;
  o->w_lora1 = off;  // contiguous with w_rkv (3*C*C*2 is a multiple of 256)
  off = align256(off + SR * C * 2);
  o->w_lora2 = off;
  off = align256(off + C * SR * 2);
  o->w_o = off;
  off = align256(off + C * C * 2);
  o->w_fk = off;
  off = align256(off + F * C * 2);
  o->w_fv = off;
  off = align256(off + C * F * 2);
  o->vec = off;
  off = align256(off + int64_t(RWKV7_NVEC) * C * 4);
  o->bytes = off;
  // fragment arena
  const int64_t R[4] = {d.rank_v, d.rank_w, d.rank_a, d.rank_g};
  off = 0;
  o->f_rkv = off;
  off = align256(off + frag_bytes(3 * C, C));
  for (int g = 0; g < 4; ++g) {
    o->f_l1[g] = off;
    off = align256(off + frag_bytes(R[g], C));
  }
  for (int g = 0; g < 4; ++g) {
    o->f_l2[g] = off;
    off = align256(off + frag_bytes(C, R[g]));
  }
  o->f_o = off;
  off = align256(off + frag_bytes(C, C));
  o->f_fk = off;
  off = align256(off + frag_bytes(F, C));
  o->f_fv = off;
  off = align256(off + frag_bytes(C, F));
  o->frag_bytes = off;
  // int8 arena
  off = 0;
  o->q_rkv = off;
  off = align256(off + (3 * C + SR) * C);
  o->q_o = off;
  off = align256(off + C * C);
  o->q_fk = off;
  off = align256(off + F * C);
  o->q_fv = off;
  off = align256(off + C * F);
  o->q_scale = off;
  off = align256(off + (3 * C + SR + C + F + C) * 4);
  o->q_bytes = off;
}

// Workspace of the one-sequence decode path (GEMV kernels).
struct DecodeWs {
  float *x0, *xln, *proj, *vfirst, *yg, *xln2, *hid;
};
// The workspace starts with the persistent decode kernel's exchange region
// (synchronisation words and tagged hand-off vectors); it must be zero when the
// workspace is first used and is only ever touched by that kernel.
static int64_t exchange_bytes(const rwkv7_dims &d) {
  return align256(mk_exchange_bytes(d.n_embd, d.n_ffn, sum_ranks(d)));
}
// Then the GEMM split-K arrival counters (zero between launches), then the
// path's own buffers.
static unsigned *gemm_counters(const rwkv7_dims &d, char *base) {
  return reinterpret_cast<unsigned *>(base + exchange_bytes(d));
}
// Then the exchange region of the persistent few-row kernel (zero before
// first use, only ever touched by that kernel).
static char *rows_exchange(const rwkv7_dims &d, char *base) {
  return base + exchange_bytes(d) + align256((int64_t)kGemmCounters * 4);
}
static int64_t fixed_bytes(const rwkv7_dims &d) {
  return exchange_bytes(d) + align256((int64_t)kGemmCounters * 4) + align256(rows_exchange_bytes(d));
}

static int64_t decode_ws(const rwkv7_dims &d, char *base, DecodeWs *w) {
  const int64_t C = d.n_embd, F = d.n_ffn, SR = sum_ranks(d);
  int64_t off = fixed_bytes(d);
  auto take = [&](int64_t bytes) {
    char *p = base ? base + off : nullptr;
    off = align256(off + bytes);
    return reinterpret_cast<float *>(p);
  };
  DecodeWs t;
  t.x0 = take(C * 4);
  t.xln = take(C * 4);
  t.proj = take((3 * C + SR) * 4);
  t.vfirst = take(C * 4);
  t.yg = take(C * 4);
  t.xln2 = take(C * 4);
  t.hid = take(F * 4);
  if (w) *w = t;
  return off;
}

// Workspace of the batched path (M = B * T rows). The GEMM operands xmix, l1,
// yg, hid and headin are f32 when the step runs with f32 activations
// (batch_a32), else 16-bit; their buffers are sized for f32 either way.
struct BatchWs {
  float *x0, *rkv, *d, *vfirst, *kv, *y, *part;  // kv: gated k, mixed v [2][M][C]
  float *proj1;  // one-token steps: r, k, v, raw LoRA first steps [M, 3C+SR]
  void *xmix, *l1, *yg, *hid, *headin;
  float *U, *Send, *Pend;  // segmented scan of long sequences (null with one segment)
  float *rec;              // chunk records of the chunked scan (prefill_chunked)
};
static int64_t batch_ws(const rwkv7_dims &d, int64_t B, int64_t T, char *base, BatchWs *w) {
  const int64_t C = d.n_embd, F = d.n_ffn, SR = sum_ranks(d), M = B * T;
  int64_t off = fixed_bytes(d);
  auto take = [&](int64_t bytes) {
    char *p = base ? base + off : nullptr;
    off = align256(off + bytes);
    return p;
  };
  BatchWs t;
  t.x0 = reinterpret_cast<float *>(take(M * C * 4));
  t.xmix = take(6 * M * C * 4);
  t.rkv = reinterpret_cast<float *>(take(3 * M * C * 4));
  t.l1 = take(M * SR * 4);
  t.d = reinterpret_cast<float *>(take(4 * M * C * 4));
  t.vfirst = reinterpret_cast<float *>(take(M * C * 4));
  t.kv = reinterpret_cast<float *>(take(2 * M * C * 4));
  t.y = reinterpret_cast<float *>(take(M * C * 4));
  t.yg = take(M * C * 4);
  t.hid = take(M * F * 4);
  t.headin = take(B * C * 4);
  t.proj1 = T == 1 ? reinterpret_cast<float *>(take(M * (3 * C + SR) * 4)) : nullptr;
  const int cus = mk_cus() > 0 ? mk_cus() : 256;
  t.part = reinterpret_cast<float *>(take(gemm_ws_bytes((int)(M > B ? M : B), cus)));
  int seg_len;
  const int64_t nseg = prefill_segments((int)T, (int)B, d.n_head, cus, &seg_len);
  t.U = t.Send = t.Pend = t.rec = nullptr;
  if (prefill_chunked((int)T, (int)B, d.n_head, cus)) {
    t.rec = reinterpret_cast<float *>(take(wkv7_chunk_rec_bytes((int)B, (int)T, d.n_head)));
  } else if (nseg > 1) {
    const int64_t slab = nseg * B * d.n_head * (int64_t)RWKV7_HEAD_SIZE * RWKV7_HEAD_SIZE * 4;
    t.U = reinterpret_cast<float *>(take(M * C * 4));
    t.Send = reinterpret_cast<float *>(take(slab));
    t.Pend = reinterpret_cast<float *>(take(slab));
  }
  if (w) *w = t;
  return off;
}

#define RWKV7_TRY(expr)            \
  do {                             \
    int rc_ = (expr);              \
    if (rc_ != RWKV7_OK) return rc_; \
  } while (0)

// One token for one sequence through the GEMV kernels.
static int decode_one(const rwkv7_model &m, const rwkv7_state &s, const int64_t *tok, void *logits,
                      char *ws, hipStream_t st) {
  const rwkv7_dims &d = m.dims;
  const int C = d.n_embd, F = d.n_ffn, H = d.n_head, SR = sum_ranks(d);
  rwkv7_layer_layout lay;
  layout_of(d, &lay);
  DecodeWs w;
  decode_ws(d, ws, &w);
  const int bf = (m.flags & RWKV7_MODEL_BF16) ? 1 : 0;
  RWKV7_TRY(launch_embed(tok, static_cast<const uint16_t *>(m.emb), w.x0, 1, C, d.vocab, bf, st));
  for (int l = 0; l < d.n_layer; ++l) {
    const char *L = static_cast<const char *>(m.layers) + (int64_t)l * lay.bytes;
    const float *vec = reinterpret_cast<const float *>(L + lay.vec);
    uint16_t *tshift = static_cast<uint16_t *>(s.tmix_x) + (int64_t)l * C;
    uint16_t *cshift = static_cast<uint16_t *>(s.cmix_x) + (int64_t)l * C;
    float *rnn = static_cast<float *>(s.rnn) + (int64_t)l * H * kN * kN;

    GemvArgs g = {};
    g.W = reinterpret_cast<const uint16_t *>(L + lay.w_rkv);
    g.ldw = C;
    g.N = 3 * C + SR;
    g.K = C;
    g.x = w.x0;
    g.ln_w = vec + RWKV7_V_LN1_W * C;
    g.ln_b = vec + RWKV7_V_LN1_B * C;
    g.prev = tshift;
    g.mu = vec;
    const int ends[7] = {C, 2 * C, 3 * C, 3 * C + d.rank_v, 3 * C + d.rank_v + d.rank_w,
                         3 * C + d.rank_v + d.rank_w + d.rank_a, 3 * C + SR};
    const int mus[7] = {RWKV7_V_X_R, RWKV7_V_X_K, RWKV7_V_X_V, RWKV7_V_X_V,
                        RWKV7_V_X_W, RWKV7_V_X_A, RWKV7_V_X_G};
    memcpy(g.seg_end, ends, sizeof ends);
    memcpy(g.seg_mu, mus, sizeof mus);
    g.xln_out = w.xln;
    g.y = w.proj;
    g.bf = bf;
    RWKV7_TRY((launch_gemv<PRO_TMIX, EPI_F32>(g, st)));

    TmixDecodeArgs t;
    t.proj = w.proj;
    t.ldp = 3 * C + SR;
    t.w_lora2 = reinterpret_cast<const uint16_t *>(L + lay.w_lora2);
    t.vec = vec;
    t.vfirst = w.vfirst;
    t.rnn = rnn;
    t.xln = w.xln;
    t.shift = tshift;
    t.yg = w.yg;
    t.C = C;
    t.H = H;
    t.rv = d.rank_v;
    t.rw = d.rank_w;
    t.ra = d.rank_a;
    t.rg = d.rank_g;
    t.layer0 = l == 0;
    t.yg16 = nullptr;
    t.bf = bf;
    RWKV7_TRY(launch_tmix_decode(t, 1, st));

    GemvArgs o = {};
    o.W = reinterpret_cast<const uint16_t *>(L + lay.w_o);
    o.ldw = C;
    o.N = C;
    o.K = C;
    o.x = w.yg;
    o.y = w.x0;
    o.bf = bf;
    RWKV7_TRY((launch_gemv<PRO_F32, EPI_RESID>(o, st)));

    GemvArgs fk = {};
    fk.W = reinterpret_cast<const uint16_t *>(L + lay.w_fk);
    fk.ldw = C;
    fk.N = F;
    fk.K = C;
    fk.x = w.x0;
    fk.ln_w = vec + RWKV7_V_LN2_W * C;
    fk.ln_b = vec + RWKV7_V_LN2_B * C;
    fk.prev = cshift;
    fk.mu = vec + RWKV7_V_FFN_X_K * C;
    fk.xln_out = w.xln2;
    fk.y = w.hid;
    fk.bf = bf;
    RWKV7_TRY((launch_gemv<PRO_CMIX, EPI_RELUSQ>(fk, st)));
    RWKV7_TRY(launch_store_f16(w.xln2, cshift, C, bf, st));

    GemvArgs fv = {};
    fv.W = reinterpret_cast<const uint16_t *>(L + lay.w_fv);
    fv.ldw = F;
    fv.N = C;
    fv.K = F;
    fv.x = w.hid;
    fv.y = w.x0;
    fv.bf = bf;
    RWKV7_TRY((launch_gemv<PRO_F32, EPI_RESID>(fv, st)));
  }
  if (logits) {
    const float *lo = static_cast<const float *>(m.ln_out);
    GemvArgs hd = {};
    hd.W = static_cast<const uint16_t *>(m.head);
    hd.ldw = C;
    hd.N = d.vocab;
    hd.K = C;
    hd.x = w.x0;
    hd.ln_w = lo;
    hd.ln_b = lo + C;
    hd.y = logits;
    hd.bf = bf;
    RWKV7_TRY((launch_gemv<PRO_LN, EPI_F16>(hd, st)));
  }
  return RWKV7_OK;
}

// The batched path runs with f32 activations -- every GEMM operand produced
// in f32 and multiplied as two 16-bit parts (GemmProb::a32) -- when no GEMM of
// the step would take the large-M path: below gemm_big_min_rows of the
// widest layer matrix. Above it (long prefills, where the products are
// MFMA-bound and the large-M kernel streams 16-bit operands by LDS DMA) the
// activations are rounded to the model's 16-bit format.
static bool batch_a32(const rwkv7_dims &d, int M) { return M < gemm_big_min_rows(d.n_ffn > d.n_embd ? d.n_ffn : d.n_embd); }

// B sequences x T tokens through the MFMA GEMM path; logits (optional) of the
// last token of each sequence.
static int run_batched(const rwkv7_model &m, const rwkv7_state &s, const int64_t *tok, int T,
                       void *logits, char *ws, hipStream_t st) {
  const rwkv7_dims &d = m.dims;
  const int B = s.batch;
  const int C = d.n_embd, F = d.n_ffn, H = d.n_head, SR = sum_ranks(d);
  const int M = B * T;
  const int64_t MC = (int64_t)M * C;
  const int rv = d.rank_v, rw = d.rank_w, ra = d.rank_a, rg = d.rank_g;
  rwkv7_layer_layout lay;
  layout_of(d, &lay);
  BatchWs w;
  batch_ws(d, B, T, ws, &w);
  unsigned *ctr = gemm_counters(d, ws);
  const int bf = (m.flags & RWKV7_MODEL_BF16) ? 1 : 0;
  const int a32 = batch_a32(d, M) ? 1 : 0;
  const int esz = a32 ? 4 : 2;  // bytes per element of the GEMM operands
  const int cus = mk_cus() > 0 ? mk_cus() : 256;  // as launch_wkv7_prefill decides
  // every GEMM of the step runs on the model's 16-bit format, with f32 A if a32
  auto gemm = [&](GemmProb *p, int n, int rows) {
    for (int i = 0; i < n; ++i) {
      p[i].bf = bf;
      p[i].a32 = a32;
    }
    return launch_gemm_group(p, n, rows, st, w.part, ctr);
  };
  // element offset into an operand buffer, as the uint16_t pointer GemmProb
  // holds for A (at) and as an output pointer (out_at)
  auto at = [&](void *base, int64_t elems) {
    return reinterpret_cast<const uint16_t *>(static_cast<char *>(base) + elems * esz);
  };
  auto out_at = [&](void *base, int64_t elems) { return static_cast<void *>(static_cast<char *>(base) + elems * esz); };
  const int epi_relusq = a32 ? GEPI_RELUSQ_F32 : GEPI_RELUSQ;
  const int epi_plain = a32 ? GEPI_F32 : GEPI_F16;
  const int epi_tanh = a32 ? GEPI_TANH_F32 : GEPI_TANH_F16;
  const int epi_sigm = a32 ? GEPI_SIGM_F32 : GEPI_SIGM_F16;
  RWKV7_TRY(launch_embed(tok, static_cast<const uint16_t *>(m.emb), w.x0, M, C, d.vocab, bf, st));
  for (int l = 0; l < d.n_layer; ++l) {
    const char *L = static_cast<const char *>(m.layers) + (int64_t)l * lay.bytes;
    const float *vec = reinterpret_cast<const float *>(L + lay.vec);
    const uint16_t *wrkv = reinterpret_cast<const uint16_t *>(L + lay.w_rkv);
    const uint16_t *wl1 = reinterpret_cast<const uint16_t *>(L + lay.w_lora1);
    const uint16_t *wl2 = reinterpret_cast<const uint16_t *>(L + lay.w_lora2);
    uint16_t *tshift = static_cast<uint16_t *>(s.tmix_x) + (int64_t)l * B * C;
    uint16_t *cshift = static_cast<uint16_t *>(s.cmix_x) + (int64_t)l * B * C;
    float *rnn = static_cast<float *>(s.rnn) + (int64_t)l * B * H * kN * kN;

    LnShiftArgs ls = {w.x0, vec + RWKV7_V_LN1_W * C, vec + RWKV7_V_LN1_B * C, vec + RWKV7_V_X_R * C,
                      6, w.xmix, tshift, C, T, M};
    ls.bf = bf;
    ls.out_f32 = a32;
    // 16-bit operands (the large-M path): r, k, v at one stride, for one
    // strided-batched GEMM call (with f32 activations the stored order
    // measured ~1 % faster at 0.4B 1 x 512)
    ls.mix_order = a32 ? 0 : 1;
    RWKV7_TRY(launch_ln_shift(ls, st));
    const int64_t sk = a32 ? 2 : 1, sv = a32 ? 3 : 2, sw = a32 ? 1 : 3;  // slots of k, v, w
    const uint16_t *xr = at(w.xmix, 0), *xk = at(w.xmix, sk * MC), *xv = at(w.xmix, sv * MC),
                   *xw = at(w.xmix, sw * MC), *xa = at(w.xmix, 4 * MC), *xg = at(w.xmix, 5 * MC);
    if (T == 1) {
      // one token per sequence: r, k, v and the raw LoRA first steps into one
      // [M, 3C+SR] f32 matrix, then the fused per-head kernel (LoRA second
      // steps, gates, wkv7, GroupNorm, gate) writes the o-projection input
      const int64_t ldp = 3 * C + SR;
      float *proj = w.proj1;
      GemmProb g1[7] = {
          {xr, wrkv, proj, C, C, ldp, C, C, GEPI_F32},
          {xk, wrkv + (int64_t)C * C, proj + C, C, C, ldp, C, C, GEPI_F32},
          {xv, wrkv + 2 * (int64_t)C * C, proj + 2 * C, C, C, ldp, C, C, GEPI_F32},
          {xv, wl1, proj + 3 * C, C, C, ldp, rv, C, GEPI_F32},
          {xw, wl1 + (int64_t)rv * C, proj + 3 * C + rv, C, C, ldp, rw, C, GEPI_F32},
          {xa, wl1 + (int64_t)(rv + rw) * C, proj + 3 * C + rv + rw, C, C, ldp, ra, C, GEPI_F32},
          {xg, wl1 + (int64_t)(rv + rw + ra) * C, proj + 3 * C + rv + rw + ra, C, C, ldp, rg, C, GEPI_F32},
      };
      const char *Fl = m.layers_frag ? static_cast<const char *>(m.layers_frag) + (int64_t)l * lay.frag_bytes : nullptr;
      auto frag = [&](GemmProb &p, int64_t off, int64_t strip0) {
        if (!Fl) return;
        p.nksf = (p.K + 31) / 32;
        p.Wf = reinterpret_cast<const uint16_t *>(Fl + off) + strip0 * p.nksf * 512;
      };
      frag(g1[0], lay.f_rkv, 0);
      frag(g1[1], lay.f_rkv, C / 16);
      frag(g1[2], lay.f_rkv, 2 * C / 16);
      for (int g = 0; g < 4; ++g) frag(g1[3 + g], lay.f_l1[g], 0);
      RWKV7_TRY(gemm(g1, 7, M));
      TmixDecodeArgs td;
      td.proj = proj;
      td.ldp = ldp;
      td.w_lora2 = wl2;
      td.vec = vec;
      td.vfirst = w.vfirst;
      td.rnn = rnn;
      td.xln = nullptr;
      td.shift = nullptr;  // ln_shift wrote the shift state
      td.yg = a32 ? static_cast<float *>(w.yg) : nullptr;
      td.yg16 = a32 ? nullptr : static_cast<uint16_t *>(w.yg);
      td.C = C;
      td.H = H;
      td.rv = rv;
      td.rw = rw;
      td.ra = ra;
      td.rg = rg;
      td.layer0 = l == 0;
      td.bf = bf;
      RWKV7_TRY(launch_tmix_decode(td, B, st));
      GemmProb go = {at(w.yg, 0), reinterpret_cast<const uint16_t *>(L + lay.w_o), w.x0, C, C, C, C, C, GEPI_ADD_F32};
      frag(go, lay.f_o, 0);
      RWKV7_TRY(gemm(&go, 1, M));
      LnShiftArgs lc = {w.x0, vec + RWKV7_V_LN2_W * C, vec + RWKV7_V_LN2_B * C, vec + RWKV7_V_FFN_X_K * C,
                        1, w.xmix, cshift, C, T, M};
      lc.bf = bf;
      lc.out_f32 = a32;
      RWKV7_TRY(launch_ln_shift(lc, st));
      GemmProb gk = {at(w.xmix, 0), reinterpret_cast<const uint16_t *>(L + lay.w_fk), w.hid, C, C, F, F, C, epi_relusq};
      frag(gk, lay.f_fk, 0);
      RWKV7_TRY(gemm(&gk, 1, M));
      GemmProb gv = {at(w.hid, 0), reinterpret_cast<const uint16_t *>(L + lay.w_fv), w.x0, F, F, C, C, F, GEPI_ADD_F32};
      frag(gv, lay.f_fv, 0);
      RWKV7_TRY(gemm(&gv, 1, M));
      continue;
    }
    GemmProb g1[7] = {
        {xr, wrkv, w.rkv, C, C, C, C, C, GEPI_F32},
        {xk, wrkv + (int64_t)C * C, w.rkv + MC, C, C, C, C, C, GEPI_F32},
        {xv, wrkv + 2 * (int64_t)C * C, w.rkv + 2 * MC, C, C, C, C, C, GEPI_F32},
        {xv, wl1, w.l1, C, C, SR, rv, C, epi_plain},
        {xw, wl1 + (int64_t)rv * C, out_at(w.l1, rv), C, C, SR, rw, C, epi_tanh},
        {xa, wl1 + (int64_t)(rv + rw) * C, out_at(w.l1, rv + rw), C, C, SR, ra, C, epi_plain},
        {xg, wl1 + (int64_t)(rv + rw + ra) * C, out_at(w.l1, rv + rw + ra), C, C, SR, rg, C, epi_sigm},
    };
    // fragment-order copies (16 x 32 blocks) when the model has them
    const char *Fl = m.layers_frag ? static_cast<const char *>(m.layers_frag) + (int64_t)l * lay.frag_bytes : nullptr;
    auto frag = [&](GemmProb &p, int64_t off, int64_t strip0) {
      if (!Fl) return;
      p.nksf = (p.K + 31) / 32;
      p.Wf = reinterpret_cast<const uint16_t *>(Fl + off) + strip0 * p.nksf * 512;
    };
    frag(g1[0], lay.f_rkv, 0);
    frag(g1[1], lay.f_rkv, C / 16);
    frag(g1[2], lay.f_rkv, 2 * C / 16);
    for (int g = 0; g < 4; ++g) frag(g1[3 + g], lay.f_l1[g], 0);
    RWKV7_TRY(gemm(g1, 7, M));
    GemmProb g2[4] = {
        {at(w.l1, 0), wl2, w.d, SR, SR, C, C, rv, GEPI_F32},
        {at(w.l1, rv), wl2 + rv, w.d + MC, SR, SR, C, C, rw, GEPI_F32},
        {at(w.l1, rv + rw), wl2 + rv + rw, w.d + 2 * MC, SR, SR, C, C, ra, GEPI_F32},
        {at(w.l1, rv + rw + ra), wl2 + rv + rw + ra, w.d + 3 * MC, SR, SR, C, C, rg, GEPI_F32},
    };
    for (int g = 0; g < 4; ++g) frag(g2[g], lay.f_l2[g], 0);
    PrefillScanArgs sc = {rnn, w.rkv, w.d, vec, w.vfirst, w.y, w.kv, w.kv + MC, B, T, H, C, M, l == 0,
                          w.U, w.Send, w.Pend, w.rec};
    if (prefill_chunked(T, B, H, cus) && lora2_fits(rv, rw, ra, rg)) {
      // the chunked scan's prep kernel forms the LoRA second steps itself
      sc.l1 = w.l1;
      sc.w2 = wl2;
      sc.dg = w.d + 3 * MC;
      sc.rv = rv;
      sc.rw = rw;
      sc.ra = ra;
      sc.rg = rg;
      sc.l1_f32 = a32;
      sc.bf = bf;
    } else {
      RWKV7_TRY(gemm(g2, 4, M));
    }
    RWKV7_TRY(launch_wkv7_prefill(sc, st));
    GnGateArgs gn = {w.y, w.rkv, w.kv, w.kv + MC, w.d + 3 * MC, vec, w.yg, C, M};
    gn.bf = bf;
    gn.out_f32 = a32;
    RWKV7_TRY(launch_gn_gate(gn, st));
    GemmProb go = {at(w.yg, 0), reinterpret_cast<const uint16_t *>(L + lay.w_o), w.x0, C, C, C, C, C, GEPI_ADD_F32};
    frag(go, lay.f_o, 0);
    RWKV7_TRY(gemm(&go, 1, M));

    LnShiftArgs lc = {w.x0, vec + RWKV7_V_LN2_W * C, vec + RWKV7_V_LN2_B * C, vec + RWKV7_V_FFN_X_K * C,
                      1, w.xmix, cshift, C, T, M};
    lc.bf = bf;
    lc.out_f32 = a32;
    RWKV7_TRY(launch_ln_shift(lc, st));
    GemmProb gk = {at(w.xmix, 0), reinterpret_cast<const uint16_t *>(L + lay.w_fk), w.hid, C, C, F, F, C, epi_relusq};
    frag(gk, lay.f_fk, 0);
    RWKV7_TRY(gemm(&gk, 1, M));
    GemmProb gv = {at(w.hid, 0), reinterpret_cast<const uint16_t *>(L + lay.w_fv), w.x0, F, F, C, C, F, GEPI_ADD_F32};
    frag(gv, lay.f_fv, 0);
    RWKV7_TRY(gemm(&gv, 1, M));
  }
  if (logits) {
    // B rows: the head GEMM always takes f32 A (B is far below the large-M path)
    const float *lo = static_cast<const float *>(m.ln_out);
    RWKV7_TRY(launch_ln_rows(w.x0, 1, lo, lo + C, w.headin, 1, B, C, T, T - 1, bf, st));
    GemmProb gh = {static_cast<const uint16_t *>(w.headin), static_cast<const uint16_t *>(m.head), logits, C, C,
                   d.vocab, d.vocab, C, GEPI_F16};
    if (m.head_frag) {
      gh.Wf = static_cast<const uint16_t *>(m.head_frag);
      gh.nksf = (C + 31) / 32;
    }
    gh.bf = bf;
    gh.a32 = 1;
    RWKV7_TRY(launch_gemm_group(&gh, 1, B, st, w.part, ctr));
  }
  return RWKV7_OK;
}

static int check_model_state(const rwkv7_model *m, const rwkv7_state *s) {
  if (!m || !s) return RWKV7_EINVAL;
  RWKV7_TRY(check_dims(&m->dims));
  if (!m->layers || !m->emb || !m->head || !m->ln_out) return RWKV7_EINVAL;
  if (!s->tmix_x || !s->rnn || !s->cmix_x || s->batch < 1) return RWKV7_EINVAL;
  return RWKV7_OK;
}

// The one-launch persistent kernel serves batch-1 steps that produce logits,
// for the sizes it was compiled for and when its grid fits on the device at
// once; the model flag RWKV7_MODEL_MULTI_LAUNCH_DECODE selects the
// multi-launch path instead.
static bool use_persistent_decode(const rwkv7_model &m, int batch, bool logits) {
  if (batch != 1 || !logits || (m.flags & RWKV7_MODEL_MULTI_LAUNCH_DECODE)) return false;
  return mk_usable(m);
}

// Batched decode steps and prefills of B sequences x T tokens with B T <= 16
// run as the one-launch few-row kernel when it serves the model (half
// precision, fragment arenas, no multi-launch flag) and its grid fits; batch-1
// decode has its own kernel above.
static bool use_rows_kernel(const rwkv7_model &m, int batch, int T) { return rows_usable(m, batch, T); }

static int run_rows(const rwkv7_model &m, const rwkv7_state &s, const int64_t *tok, int T, void *logits, char *ws,
                    hipStream_t st) {
  rwkv7_layer_layout lay;
  layout_of(m.dims, &lay);
  // the aborted-launch counter shared with the batch-1 kernel (workspace byte 32)
  return launch_rows_mk(m, lay, s, tok, T, logits, rows_exchange(m.dims, ws), reinterpret_cast<unsigned *>(ws + 32),
                        st);
}

}  // namespace rwkv7

using namespace rwkv7;

extern "C" {

int rwkv7_abi_version(void) { return RWKV7_ABI_VERSION; }

const char *rwkv7_strerror(int code) {
  switch (code) {
    case RWKV7_OK: return "ok";
    case RWKV7_EINVAL: return "invalid argument (null pointer or bad enum value)";
    case RWKV7_ESHAPE: return "unsupported shape";
    case RWKV7_EWORKSPACE: return "workspace too small";
    case RWKV7_ELAUNCH: return "kernel launch failed";
    default: return "unknown error";
  }
}

int rwkv7_layer_layout_get(const rwkv7_dims *dims, rwkv7_layer_layout *out) {
  RWKV7_TRY(check_dims(dims));
  if (!out) return RWKV7_EINVAL;
  layout_of(*dims, out);
  return RWKV7_OK;
}

int64_t rwkv7_head_q_scale_offset(const rwkv7_dims *dims) {
  if (check_dims(dims) != RWKV7_OK) return -1;
  return align256((int64_t)dims->vocab * dims->n_embd);
}

int64_t rwkv7_workspace_bytes(const rwkv7_dims *dims, int32_t batch, int32_t seq_len) {
  if (check_dims(dims) != RWKV7_OK || batch < 1 || seq_len < 1) return -1;
  const int64_t a = decode_ws(*dims, nullptr, nullptr);
  const int64_t b = batch_ws(*dims, batch, seq_len, nullptr, nullptr);
  return a > b ? a : b;
}

int rwkv7_decode_launches(const rwkv7_model *model, int32_t batch, int32_t with_logits) {
  if (!model || check_dims(&model->dims) != RWKV7_OK || batch < 1) return -1;
  const rwkv7_dims *dims = &model->dims;
  if (use_persistent_decode(*model, batch, with_logits != 0) || (batch > 1 && use_rows_kernel(*model, batch, 1)))
    return 1;
  // decode_one: embed, 6 per layer, head GEMV; run_batched with one token:
  // embed, 7 per layer (LayerNorm + shift, projections, per-head core,
  // o-projection, LayerNorm + shift, FFN key, FFN value), final LayerNorm and
  // head GEMM
  if (batch == 1) return 1 + 6 * dims->n_layer + (with_logits ? 1 : 0);
  return 1 + 7 * dims->n_layer + (with_logits ? 2 : 0);
}

int rwkv7_step_f32_activations(const rwkv7_model *model, int32_t batch, int32_t seq_len) {
  if (!model || check_dims(&model->dims) != RWKV7_OK || batch < 1 || seq_len < 1) return -1;
  if (seq_len == 1 && use_persistent_decode(*model, batch, true)) return 1;  // fp32 activations throughout
  if (use_rows_kernel(*model, batch, seq_len)) return 1;                     // f32 rows, hi/lo MFMA
  return batch_a32(model->dims, batch * seq_len) ? 1 : 0;
}

int rwkv7_decode(const rwkv7_model *model, const rwkv7_state *state, const int64_t *tokens, void *logits,
                 void *workspace, int64_t workspace_bytes, void *stream) {
  RWKV7_TRY(check_model_state(model, state));
  if (!tokens || !workspace) return RWKV7_EINVAL;
  if (workspace_bytes < rwkv7_workspace_bytes(&model->dims, state->batch, 1)) return RWKV7_EWORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // int8 weights exist only for the persistent batch-1 kernel: a batch-1
  // decode with the flag set that cannot run it is an error, not an f16
  // fallback (batched decode reads the f16 arenas, as documented)
  if ((model->flags & RWKV7_MODEL_INT8_DECODE) && state->batch == 1 &&
      (!mk_int8(*model) || !use_persistent_decode(*model, 1, logits != nullptr)))
    return RWKV7_ESHAPE;
  if (state->batch == 1) {
    if (use_persistent_decode(*model, 1, logits != nullptr)) {
      rwkv7_layer_layout lay;
      layout_of(model->dims, &lay);
      return launch_decode_mk(*model, lay, *state, tokens, logits, static_cast<char *>(workspace), st);
    }
    return decode_one(*model, *state, tokens, logits, static_cast<char *>(workspace), st);
  }
  if (use_rows_kernel(*model, state->batch, 1))
    return run_rows(*model, *state, tokens, 1, logits, static_cast<char *>(workspace), st);
  return run_batched(*model, *state, tokens, 1, logits, static_cast<char *>(workspace), st);
}

int rwkv7_workspace_errors(const void *workspace, int64_t workspace_bytes, uint32_t *count, void *stream) {
  if (!workspace || !count) return RWKV7_EINVAL;
  if (workspace_bytes < 64) return RWKV7_EWORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (hipStreamSynchronize(st) != hipSuccess) return RWKV7_ELAUNCH;
  uint32_t v = 0;
  if (hipMemcpy(&v, static_cast<const char *>(workspace) + 32, 4, hipMemcpyDeviceToHost) != hipSuccess)
    return RWKV7_ELAUNCH;
  *count = v;
  return RWKV7_OK;
}

int rwkv7_prefill(const rwkv7_model *model, const rwkv7_state *state, const int64_t *tokens, int32_t seq_len,
                  void *workspace, int64_t workspace_bytes, void *stream) {
  RWKV7_TRY(check_model_state(model, state));
  if (!tokens || !workspace) return RWKV7_EINVAL;
  if (seq_len < 1) return RWKV7_ESHAPE;
  if (workspace_bytes < rwkv7_workspace_bytes(&model->dims, state->batch, seq_len)) return RWKV7_EWORKSPACE;
  if (use_rows_kernel(*model, state->batch, seq_len))
    return run_rows(*model, *state, tokens, seq_len, nullptr, static_cast<char *>(workspace),
                    static_cast<hipStream_t>(stream));
  return run_batched(*model, *state, tokens, seq_len, nullptr, static_cast<char *>(workspace),
                     static_cast<hipStream_t>(stream));
}

// The scan instance for the operand formats of an operator-level call: 16-bit
// r, k, v, a, b (half or bfloat16), w 16-bit or f32, y in r's format.
extern "C++" template <class Run>
static int wkv7_dispatch(float *S, const void *r, const void *w, int32_t w_is_f32, const void *k, const void *v,
                         const void *a, const void *b, void *y, int32_t B, int32_t T, int32_t H, int32_t bf16,
                         Run run) {
  if (bf16) {
    auto bp = [](const void *q) { return static_cast<const bf16_t *>(q); };
    bf16_t *yb = static_cast<bf16_t *>(y);
    if (w_is_f32) {
      ScanArgs<bf16_t, float, bf16_t> p = {S, bp(r), bp(k), bp(v), bp(a), bp(b), static_cast<const float *>(w),
                                           yb, B, T, H};
      return run(p);
    }
    ScanArgs<bf16_t, bf16_t, bf16_t> p = {S, bp(r), bp(k), bp(v), bp(a), bp(b), bp(w), yb, B, T, H};
    return run(p);
  }
  auto hp = [](const void *q) { return static_cast<const uint16_t *>(q); };
  uint16_t *y16 = static_cast<uint16_t *>(y);
  if (w_is_f32) {
    ScanArgs<uint16_t, float, uint16_t> p = {S, hp(r), hp(k), hp(v), hp(a), hp(b), static_cast<const float *>(w),
                                             y16, B, T, H};
    return run(p);
  }
  ScanArgs<uint16_t, uint16_t, uint16_t> p = {S, hp(r), hp(k), hp(v), hp(a), hp(b), hp(w), y16, B, T, H};
  return run(p);
}

int rwkv7_wkv7(float *S, const void *r, const void *w, int32_t w_is_f32, const void *k, const void *v,
               const void *a, const void *b, void *y, int32_t B, int32_t T, int32_t H, int32_t bf16,
               void *stream) {
  if (!S || !r || !w || !k || !v || !a || !b || !y) return RWKV7_EINVAL;
  if (B < 1 || T < 1 || H < 1) return RWKV7_ESHAPE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return wkv7_dispatch(S, r, w, w_is_f32, k, v, a, b, y, B, T, H, bf16,
                       [&](const auto &p) { return launch_wkv7_scan(p, st); });
}

int64_t rwkv7_wkv7_chunked_workspace_bytes(int32_t B, int32_t T, int32_t H) {
  if (B < 1 || T < 1 || H < 1) return 0;
  return wkv7_chunk_rec_bytes(B, T, H);
}

int rwkv7_wkv7_chunked(float *S, const void *r, const void *w, int32_t w_is_f32, const void *k, const void *v,
                       const void *a, const void *b, void *y, int32_t B, int32_t T, int32_t H, int32_t bf16,
                       void *workspace, int64_t workspace_bytes, void *stream) {
  if (!S || !r || !w || !k || !v || !a || !b || !y || !workspace) return RWKV7_EINVAL;
  if (B < 1 || T < 1 || H < 1) return RWKV7_ESHAPE;
  if (workspace_bytes < wkv7_chunk_rec_bytes(B, T, H)) return RWKV7_EWORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  float *rec = static_cast<float *>(workspace);
  return wkv7_dispatch(S, r, w, w_is_f32, k, v, a, b, y, B, T, H, bf16,
                       [&](const auto &p) { return launch_wkv7_chunked(p, rec, st); });
}

int rwkv7_wkv7_f32(float *S, const float *r, const float *w, const float *k, const float *v, const float *a,
                   const float *b, float *y, float *hist, int32_t B, int32_t T, int32_t H, void *stream) {
  if (!S || !r || !w || !k || !v || !a || !b || !y) return RWKV7_EINVAL;
  if (B < 1 || T < 1 || H < 1) return RWKV7_ESHAPE;
  ScanArgs<float, float, float> p = {S, r, k, v, a, b, w, y, B, T, H, hist};
  return launch_wkv7_scan(p, static_cast<hipStream_t>(stream));
}

int rwkv7_wkv7_backward(const float *hist, const float *S_T, const float *r, const float *w, const float *k,
                        const float *v, const float *a, const float *b, const float *gy, const float *gS_T,
                        float *gS0, float *gr, float *gw, float *gk, float *gv, float *ga, float *gb, int32_t B,
                        int32_t T, int32_t H, void *stream) {
  if (!hist || !S_T || !r || !w || !k || !v || !a || !b || !gy || !gS0 || !gr || !gw || !gk || !gv || !ga || !gb)
    return RWKV7_EINVAL;
  if (B < 1 || T < 1 || H < 1) return RWKV7_ESHAPE;
  Wkv7BwdArgs p = {hist, S_T, r, w, k, v, a, b, gy, gS_T, gS0, gr, gw, gk, gv, ga, gb, B, T, H};
  return launch_wkv7_bwd(p, static_cast<hipStream_t>(stream));
}

int rwkv7_layernorm(const void *x, int32_t x_is_f32, const float *weight, const float *bias, float *y, int32_t M,
                    int32_t C, int32_t bf16, void *stream) {
  if (!x || !weight || !bias || !y) return RWKV7_EINVAL;
  if (M < 1) return RWKV7_ESHAPE;
  return launch_ln_rows(x, x_is_f32, weight, bias, y, 1, M, C, 1, 0, bf16 ? 1 : 0, static_cast<hipStream_t>(stream));
}

int rwkv7_lerp(const void *x, const void *prev, const float *mu, int32_t n_mix, void *out, void *x_copy, int32_t C,
               int32_t bf16, void *stream) {
  if (!x || !prev || !mu || !out) return RWKV7_EINVAL;
  if ((n_mix != 1 && n_mix != 6) || C < 1) return RWKV7_ESHAPE;
  return launch_lerp(static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(prev), mu, n_mix,
                     static_cast<uint16_t *>(out), static_cast<uint16_t *>(x_copy), C, bf16 ? 1 : 0,
                     static_cast<hipStream_t>(stream));
}

int rwkv7_gemv_f16(const float *x, const void *W, int64_t ldw, float *y, int32_t N, int32_t K, int32_t bf16,
                   void *stream) {
  if (!x || !W || !y) return RWKV7_EINVAL;
  if (N < 1 || K < 256 || K % 256 || K > 8192 || ldw < K || ldw % 8) return RWKV7_ESHAPE;
  GemvArgs g = {};
  g.W = static_cast<const uint16_t *>(W);
  g.ldw = ldw;
  g.N = N;
  g.K = K;
  g.x = x;
  g.y = y;
  g.bf = bf16 ? 1 : 0;
  return launch_gemv<PRO_F32, EPI_F32>(g, static_cast<hipStream_t>(stream));
}

int rwkv7_gemm_f16(const void *A, int64_t lda, const void *W, int64_t ldw, void *Y, int64_t ldy, int32_t M, int32_t N,
                   int32_t K, int32_t epi, int32_t bf16, void *stream) {
  if (!A || !W || !Y) return RWKV7_EINVAL;
  if (epi < 0 || epi > GEPI_SIGM_F32 || (bf16 & ~(RWKV7_GEMM_BF16 | RWKV7_GEMM_A_F32))) return RWKV7_EINVAL;
  if (M < 1 || N < 1 || K < 8 || lda < K || ldw < K || ldy < N) return RWKV7_ESHAPE;
  GemmProb p = {static_cast<const uint16_t *>(A), static_cast<const uint16_t *>(W), Y, lda, ldw, ldy, N, K, epi};
  p.bf = (bf16 & RWKV7_GEMM_BF16) ? 1 : 0;
  p.a32 = (bf16 & RWKV7_GEMM_A_F32) ? 1 : 0;
  return launch_gemm_group(&p, 1, M, static_cast<hipStream_t>(stream), nullptr, nullptr);
}

static const uint16_t *h16(const void *p) { return static_cast<const uint16_t *>(p); }
static uint16_t *h16(void *p) { return static_cast<uint16_t *>(p); }
static hipStream_t hs(void *s) { return static_cast<hipStream_t>(s); }

int rwkv7_w_gate(const void *x, const void *w0, void *out, int32_t C, int32_t bf16, void *stream) {
  if (!x || !w0 || !out) return RWKV7_EINVAL;
  if (C < 1) return RWKV7_ESHAPE;
  return launch_w_gate(h16(x), h16(w0), h16(out), C, bf16 ? 1 : 0, hs(stream));
}

int rwkv7_v_gate(const void *v, const void *v_first, const void *v0, const void *v12, void *out, int32_t C,
                 int32_t bf16, void *stream) {
  if (!v || !v_first || !v0 || !v12 || !out) return RWKV7_EINVAL;
  if (C < 1) return RWKV7_ESHAPE;
  return launch_v_gate(h16(v), h16(v_first), h16(v0), h16(v12), h16(out), C, bf16 ? 1 : 0, hs(stream));
}

int rwkv7_a_kk_k(const void *a0, const void *a_x, const void *k, const void *k_k, const void *k_a, void *a_out,
                 void *kk_out, void *k_out, int32_t C, int32_t bf16, void *stream) {
  if (!a0 || !a_x || !k || !k_k || !k_a || !a_out || !kk_out || !k_out) return RWKV7_EINVAL;
  if (C < 1) return RWKV7_ESHAPE;
  return launch_a_kk_k(h16(a0), h16(a_x), h16(k), h16(k_k), h16(k_a), h16(a_out), h16(kk_out), h16(k_out), C,
                       bf16 ? 1 : 0, hs(stream));
}

int rwkv7_gates(const rwkv7_gates_io *io, int32_t rank_v, int32_t rank_w, int32_t rank_a, int32_t rank_g, int32_t C,
                int32_t bf16, void *stream) {
  if (!io) return RWKV7_EINVAL;
  const void *ins[16] = {io->vr, io->wr, io->ar, io->gr, io->v2t, io->w2t, io->a2t, io->g2t,
                         io->v,  io->v_first, io->k, io->v0, io->w0, io->a0, io->k_k, io->k_a};
  const void *outs[6] = {io->v_out, io->w_out, io->a_out, io->kk_out, io->k_out, io->g_out};
  for (const void *p : ins)
    if (!p) return RWKV7_EINVAL;
  for (const void *p : outs)
    if (!p) return RWKV7_EINVAL;
  if (C < 1 || rank_v < 1 || rank_w < 1 || rank_a < 1 || rank_g < 1) return RWKV7_ESHAPE;
  return launch_gates(*io, rank_v, rank_w, rank_a, rank_g, C, bf16 ? 1 : 0, hs(stream));
}

int rwkv7_rank_gemv(const void *xv, const void *xw, const void *xa, const void *xg, const void *W, void *out,
                    int32_t rank_v, int32_t rank_w, int32_t rank_a, int32_t rank_g, int32_t C, int32_t bf16,
                    void *stream) {
  if (!xv || !xw || !xa || !xg || !W || !out) return RWKV7_EINVAL;
  if (C < 8 || C % 8 || rank_v < 1 || rank_w < 1 || rank_a < 1 || rank_g < 1) return RWKV7_ESHAPE;
  return launch_rank_gemv(h16(xv), h16(xw), h16(xa), h16(xg), h16(W), h16(out), rank_v, rank_w, rank_a, rank_g, C,
                          bf16 ? 1 : 0, hs(stream));
}

int rwkv7_l2norm_neg_kk_a(const void *kk, const void *a, void *kk_norm, void *b, int32_t H, int32_t bf16,
                          void *stream) {
  if (!kk || !a || !kk_norm || !b) return RWKV7_EINVAL;
  if (H < 1) return RWKV7_ESHAPE;
  return launch_l2norm(h16(kk), h16(a), h16(kk_norm), h16(b), H, bf16 ? 1 : 0, hs(stream));
}

int rwkv7_gn_rkrk(const void *y, const void *r, const void *k, const void *v, const void *r_k, const void *ln_w,
                  const void *ln_b, void *out, int32_t H, int32_t bf16, void *stream) {
  if (!y || !r || !k || !v || !r_k || !ln_w || !ln_b || !out) return RWKV7_EINVAL;
  if (H < 1) return RWKV7_ESHAPE;
  return launch_gn_rkrk(h16(y), h16(r), h16(k), h16(v), h16(r_k), h16(ln_w), h16(ln_b), h16(out), H, bf16 ? 1 : 0,
                        hs(stream));
}

}  // extern "C"
