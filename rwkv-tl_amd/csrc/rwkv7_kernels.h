// Internal interface between the host sequencer (model.hip) and the kernel
// translation units (gemv.hip, tmix.hip, gemm.hip). Not part of the C ABI.
#pragma once

#include "rwkv7_common.h"

namespace rwkv7 {

// Kernel argument blocks and launchers, shared by every translation unit.
enum { PRO_F32 = 0, PRO_TMIX = 1, PRO_CMIX = 2, PRO_LN = 3, PRO_F16 = 4 };
enum { EPI_F32 = 0, EPI_RESID = 1, EPI_RELUSQ = 2, EPI_F16 = 3 };
struct GemvArgs {
  const uint16_t *W;
  int64_t ldw;
  int N, K;
  const void *x;
  const float *ln_w;
  const float *ln_b;
  const uint16_t *prev;
  const float *mu;
  int seg_end[7];
  int seg_mu[7];
  float *xln_out;
  void *y;
  int bf;  // W, a 16-bit x, prev and a 16-bit y are bfloat16 (else half)
};
template <int PRO, int EPI> int launch_gemv(const GemvArgs &a, hipStream_t st);

// One token per sequence, grid (H, B): LoRA second step, gates, L2 norm,
// wkv7, GroupNorm, bonus and output gate. proj f32 [B, ldp] holds r, k, v
// and the raw LoRA first steps; the gated output goes to yg (f32) or, if
// yg16 is set, to yg16 (f16, the A operand of the batched o-projection).
// shift (with xln) receives the time-mix shift state; null when the caller
// already wrote it.
struct TmixDecodeArgs {
  const float *proj;
  int64_t ldp;
  const uint16_t *w_lora2;
  const float *vec;
  float *vfirst;
  float *rnn;
  const float *xln;
  uint16_t *shift;
  float *yg;
  int C, H, rv, rw, ra, rg, layer0;
  uint16_t *yg16;
  int bf;  // w_lora2, shift and yg16 are bfloat16 (else half)
};
int launch_tmix_decode(const TmixDecodeArgs &a, int B, hipStream_t st);

template <typename TI, typename TW, typename TY>
struct ScanArgs {
  float *S;
  const TI *r, *k, *v, *a, *b;
  const TW *w;
  TY *y;
  int B, T, H;
  // optional: f32 [B, H, T, 64, 64] receives the state entering each step
  // (what the backward scan needs)
  float *hist;
};
template <typename TI, typename TW, typename TY>
int launch_wkv7_scan(const ScanArgs<TI, TW, TY> &p, hipStream_t st);

// Backward of the wkv7 recurrence (reverse-time adjoint scan), all f32:
// from the gradient of y (and optionally of the final state) to the gradients
// of r, w, k, v, a, b and of the initial state.
struct Wkv7BwdArgs {
  const float *hist;                  // [B, H, T, 64, 64] state entering each step
  const float *S_T;                   // [B, H, 64, 64] state after the last step
  const float *r, *w, *k, *v, *a, *b; // [B, T, H, 64]
  const float *gy;                    // [B, T, H, 64]
  const float *gS_T;                  // [B, H, 64, 64] or null (zero)
  float *gS0;                         // [B, H, 64, 64]
  float *gr, *gw, *gk, *gv, *ga, *gb; // [B, T, H, 64]
  int B, T, H;
};
int launch_wkv7_bwd(const Wkv7BwdArgs &p, hipStream_t st);

struct LnShiftArgs {
  const float *x0;
  const float *ln_w, *ln_b;
  const float *mu;
  int n_mix;
  void *out;  // [n_mix][M][C]: f32 if out_f32, else 16-bit
  uint16_t *shift;
  int C, T, M;
  int bf;       // the 16-bit out and shift are bfloat16 (else half)
  int out_f32;  // out is f32 (the GEMMs then take it as f32 A)
  // output slot order of six mixes: 0 as the mix vectors are stored (r, w,
  // k, v, a, g), 1 r, k, v, w, a, g (r, k, v at one stride: one batched GEMM)
  int mix_order = 0;
};
int launch_ln_shift(const LnShiftArgs &a, hipStream_t st);

// Prefill time-mix core: gates of every token fused into the wkv7 scan.
// rkv f32 [3][M][C] (r, k, v), d f32 [4][M][C] (LoRA second steps v, w, a, g),
// vfirst f32 [M][C] (written on layer 0, read after), outputs y, kn_out (the
// gated k) and v_out (the mixed v), f32 [M][C]; M = B * T, rows b * T + t.
// Long sequences are scanned in nseg segments of seg_len tokens at once
// (prefill_segments); segments after the first start from a zero state and
// also carry their transition product, and a second kernel chains the
// segments. U [M, C], Send and Pend [nseg, B, H, 64, 64] (f32) are workspace
// for that; unused (may be null) when nseg == 1.
struct PrefillScanArgs {
  float *S;
  const float *rkv, *d, *vec;
  float *vfirst, *y, *kn_out, *v_out;
  int B, T, H, C, M, layer0;
  float *U, *Send, *Pend;
  // chunk records of the chunked scan (wkv7_chunk_rec_bytes), read when
  // prefill_chunked(T, B, H, cus)
  float *rec;
  // LoRA second steps inside the chunked scan (when l1 is set; d is then
  // not read): l1 [M, rv+rw+ra+rg] the LoRA first steps after their
  // activations (f32 if l1_f32, else 16-bit), w2 [C, rv+rw+ra+rg] their
  // second matrices (16-bit; bfloat16 if bf). The chunk prep kernel forms the
  // v, w, a steps of its chunk and head on MFMA and writes the g step to dg
  // [M, C] for the GroupNorm + gate stage.
  const void *l1 = nullptr;
  const uint16_t *w2 = nullptr;
  float *dg = nullptr;
  int rv = 0, rw = 0, ra = 0, rg = 0, l1_f32 = 0, bf = 0;
};
int prefill_segments(int T, int B, int H, int cus, int *seg_len);
int launch_wkv7_prefill(const PrefillScanArgs &p, hipStream_t st);

// Chunked wkv7 (16-token chunks on fp32 MFMA, tmix.hip): bytes of the chunk
// records for B sequences of T tokens and H heads, and the operator-level
// launch (the same arguments as launch_wkv7_scan, no state history).
// prefill_chunked: the model's prefill takes the chunked scan for sequences
// of at least kChunkMinT tokens (measured on MI355X against the serial scan,
// whose four workgroups per head each compute the head's gate math: 0.4B
// 1 x 128 and 1 x 512 and the 1.5B-shaped 4 x 1024 faster; 0.4B 1 x 32 and
// 1 x 64 slower).
constexpr int kChunkMinT = 128;
bool prefill_chunked(int T, int B, int H, int cus);
// the chunked scan's prep kernel can form the LoRA second steps of these
// ranks itself (PrefillScanArgs::l1)
bool lora2_fits(int rv, int rw, int ra, int rg);
int64_t wkv7_chunk_rec_bytes(int B, int T, int H);
template <typename TI, typename TW, typename TY>
int launch_wkv7_chunked(const ScanArgs<TI, TW, TY> &p, float *rec, hipStream_t st);

struct GnGateArgs {
  const float *y, *r, *kn, *v, *g, *vec;
  void *out;  // [M][C]: f32 if out_f32, else 16-bit
  int C, M;
  int bf;  // a 16-bit out is bfloat16 (else half)
  int out_f32;
};
int launch_gn_gate(const GnGateArgs &a, hipStream_t st);

// bf: the 16-bit operands are bfloat16 (else half)
int launch_embed(const int64_t *tok, const uint16_t *emb, float *x0, int M, int C, int V, int bf, hipStream_t st);
int launch_ln_rows(const void *x, int x_f32, const float *w, const float *b, void *out, int out_f32,
                   int rows, int C, int stride, int offset, int bf, hipStream_t st);
int launch_lerp(const uint16_t *x, const uint16_t *prev, const float *mu, int n_mix, uint16_t *out,
                uint16_t *x_copy, int C, int bf, hipStream_t st);
int launch_store_f16(const float *src, uint16_t *dst, int n, int bf, hipStream_t st);

enum {
  GEPI_F32 = 0,
  GEPI_F16 = 1,
  GEPI_RELUSQ = 2,
  GEPI_ADD_F32 = 3,
  GEPI_TANH_F16 = 4,
  GEPI_SIGM_F16 = 5,
  // the same activations stored as f32
  GEPI_RELUSQ_F32 = 6,
  GEPI_TANH_F32 = 7,
  GEPI_SIGM_F32 = 8,
};
struct GemmProb {
  const uint16_t *A, *W;
  void *Y;
  int64_t lda, ldw, ldy;
  int N, K, epi;
  // optional: W in fragment order (16 x 32 blocks, include/rwkv7_hip.h), with
  // nksf blocks per 16-row strip; nullptr reads the row-major W
  const uint16_t *Wf;
  int nksf;
  // A, W and the 16-bit outputs are bfloat16 (else IEEE half); one value for
  // every problem of a launch
  int bf;
  // A is f32 (lda in floats), multiplied as its 16-bit hi part plus the 16-bit
  // remainder (split_hi_lo: two MFMAs per weight fragment), so the product
  // has fp32-grade activations; one value for every problem of a launch, and
  // such problems never take the large-M path (gemm_big_min_rows)
  int a32;
};
// The fewest rows M at which an N-column problem may take the large-M path
// (whose operands stream global -> LDS as 16-bit words): callers that want
// f32 activations (a32) keep M below this for every N of a group.
int gemm_big_min_rows(int N);
// Split-K workspace: gemm_ws_bytes(M, cus) bytes of partial tiles and
// kGemmCounters arrival counters that start at zero (every launch leaves them
// at zero). With part == nullptr no problem is split.
constexpr int kGemmCounters = 1024;
int64_t gemm_ws_bytes(int M, int cus);
int launch_gemm_group(const GemmProb *probs, int nprob, int M, hipStream_t st, float *part, unsigned *ctr);
// Large-M problems with 16-bit operands and a plain epilogue (f32, 16-bit or
// add into f32), or relu^2 into half (a half product, then an in-place pass),
// through hipBLASLt (gemm_lt.hip); lt_gemm returns false when it did
// not run the problem (no algorithm, library unavailable), and the caller then
// runs its own kernel.
bool lt_eligible(const GemmProb &p);
bool lt_gemm(const GemmProb &p, int M, hipStream_t st);
// `batch` problems like p whose A, W and Y follow at strides sa, sw (16-bit
// elements) and sy (elements of Y), as one strided-batched call.
bool lt_gemm_batched(const GemmProb &p, int batch, int64_t sa, int64_t sw, int64_t sy, int M, hipStream_t st);

// Operator-level time-mix stages (ops.hip); bf: the 16-bit operands are
// bfloat16 (else IEEE half).
int launch_w_gate(const uint16_t *x, const uint16_t *w0, uint16_t *out, int C, int bf, hipStream_t st);
int launch_v_gate(const uint16_t *v, const uint16_t *vf, const uint16_t *v0, const uint16_t *v12, uint16_t *out,
                  int C, int bf, hipStream_t st);
int launch_a_kk_k(const uint16_t *a0, const uint16_t *ax, const uint16_t *k, const uint16_t *k_k,
                  const uint16_t *k_a, uint16_t *a_out, uint16_t *kk_out, uint16_t *k_out, int C, int bf,
                  hipStream_t st);
int launch_gates(const rwkv7_gates_io &io, int rv, int rw, int ra, int rg, int C, int bf, hipStream_t st);
int launch_rank_gemv(const uint16_t *xv, const uint16_t *xw, const uint16_t *xa, const uint16_t *xg,
                     const uint16_t *W, uint16_t *out, int rv, int rw, int ra, int rg, int C, int bf,
                     hipStream_t st);
int launch_l2norm(const uint16_t *kk, const uint16_t *a, uint16_t *kn, uint16_t *b, int H, int bf, hipStream_t st);
int launch_gn_rkrk(const uint16_t *y, const uint16_t *r, const uint16_t *k, const uint16_t *v, const uint16_t *r_k,
                   const uint16_t *lw, const uint16_t *lb, uint16_t *out, int H, int bf, hipStream_t st);

// One-token, one-sequence decode as a single persistent kernel (decode_mk.hip).
int mk_cus();
bool mk_supported(const rwkv7_dims &d, int G);
// mk_supported on the current device's CU count, and the grid of the kernel
// instance for the model's formats (int8 or 16-bit matrices; half or bfloat16)
// fits there all at once (checked once per device)
bool mk_usable(const rwkv7_model &m);
// the model asks for int8 decode and has the int8 arenas
bool mk_int8(const rwkv7_model &m);
int64_t mk_exchange_bytes(int C, int F, int SR);
int launch_decode_mk(const rwkv7_model &m, const rwkv7_layer_layout &lay, const rwkv7_state &s,
                     const int64_t *tok, void *logits, char *xreg, hipStream_t st);

// A step of B sequences x T tokens with B T <= 16 (batched decode, short
// prefills) as a single persistent kernel (rows_mk.hip). xreg: its exchange
// region, rows_exchange_bytes(dims), zero before first use and only ever
// touched by that kernel; errors: the workspace's aborted-launch counter.
int64_t rows_exchange_bytes(const rwkv7_dims &d);
// the model's formats and sizes are ones the kernel serves (half precision,
// fragment arenas present, no multi-launch flag), B T <= 16, and its grid fits
// on the current device at once
bool rows_usable(const rwkv7_model &m, int B, int T);
int launch_rows_mk(const rwkv7_model &m, const rwkv7_layer_layout &lay, const rwkv7_state &s, const int64_t *tok,
                   int T, void *logits, char *xreg, unsigned *errors, hipStream_t st);

}  // namespace rwkv7
