/*
 * rwkv7_hip.h -- C ABI of librwkv7_hip.so, the MI355X (gfx950) RWKV7 inference library.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream handle
 * (hipStream_t passed as void*; NULL is the legacy default stream). Nothing in
 * the library allocates or frees device memory, creates streams or events, or
 * synchronises the host (except rwkv7_workspace_errors, a status query): the
 * caller owns every buffer, so the calls can be captured in a HIP graph. One
 * exception: a GEMM past the large-M threshold with 16-bit operands and a
 * plain epilogue (long prefills) runs in hipBLASLt, whose handle -- created
 * once per device, on the first such call made outside a graph capture (a
 * call under capture runs the library's own kernel) -- holds memory of its
 * own until the process ends. Each function returns 0 on success or one of the
 * RWKV7_E* codes below (argument errors are detected on the host before any
 * launch; launch failures return RWKV7_ELAUNCH).
 *
 * Element types: "f16" is IEEE binary16, "f32" binary32, "i64" int64. All
 * arrays are dense row-major with the shapes stated. The RWKV7 head size N is
 * 64. Citations name the yuyi2439/rwkv-tl interface each entry point stands
 * in for (path:line in that repository).
 */
#ifndef RWKV7_HIP_H
#define RWKV7_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RWKV7_ABI_VERSION 11
#define RWKV7_HEAD_SIZE 64

enum {
  RWKV7_OK = 0,
  RWKV7_EINVAL = 1,    /* null pointer, bad enum value */
  RWKV7_ESHAPE = 2,    /* a dimension the kernels do not support */
  RWKV7_EWORKSPACE = 3,/* workspace smaller than rwkv7_workspace_bytes() */
  RWKV7_ELAUNCH = 4    /* a kernel launch returned a HIP error */
};

/* Model sizes. n_head * 64 == n_embd. Ranks are the LoRA widths of the w, a,
 * v and g gates (src/rwkv_tl/weight.py:77-91; demo/_rwkv7_base.py:131-137). */
typedef struct rwkv7_dims {
  int32_t n_layer, n_embd, n_head, n_ffn, vocab;
  int32_t rank_w, rank_a, rank_v, rank_g;
} rwkv7_dims;

/* Per-layer fp32 vectors, each [n_embd], stored consecutively in the layer's
 * vector block in this order (src/rwkv_tl/weight.py:66-126). r_k is the
 * [n_head, 64] tensor flattened. */
enum {
  RWKV7_V_LN1_W = 0, RWKV7_V_LN1_B, RWKV7_V_X_R, RWKV7_V_X_W, RWKV7_V_X_K,
  RWKV7_V_X_V, RWKV7_V_X_A, RWKV7_V_X_G, RWKV7_V_W0, RWKV7_V_A0, RWKV7_V_V0,
  RWKV7_V_K_K, RWKV7_V_K_A, RWKV7_V_R_K, RWKV7_V_LNX_W, RWKV7_V_LNX_B,
  RWKV7_V_LN2_W, RWKV7_V_LN2_B, RWKV7_V_FFN_X_K, RWKV7_NVEC
};

/* Byte offsets inside one layer's weight arena. All f16 matrices are
 * [out, in] (the checkpoint's own orientation):
 *   w_rkv   [3C, C]   receptance, key, value rows stacked
 *   w_lora1 [Rv+Rw+Ra+Rg, C]   v1^T, w1^T, a1^T, g1^T (the first LoRA steps)
 *   w_lora2 [C, Rv+Rw+Ra+Rg]   row c = (v2[:,c], w2[:,c], a2[:,c], g2[:,c])
 *   w_o     [C, C]
 *   w_fk    [F, C]    ffn.key
 *   w_fv    [C, F]    ffn.value
 *   vec     [RWKV7_NVEC, C] f32
 * w_lora1 immediately follows w_rkv, so the two form one [3C+sumR, C] matrix.
 * Replaces the per-tensor attributes of RWKV7ATTWeight / RWKV7FFNWeight
 * (src/rwkv_tl/weight.py:18-126) with one contiguous arena per layer. */
/* Fragment order, an optional second copy of the matrices that prefill and
 * batched decode multiply (MFMA GEMMs). A matrix W [N, K] is padded with zeros
 * to N' = 16*ceil(N/16) rows and K' = 32*ceil(K/32) columns and cut into
 * blocks of 16 rows x 32 columns; block (s, j), s < N'/16, j < K'/32, is the
 * 1024 bytes at byte offset ((s * K'/32) + j) * 1024, and inside it the 16
 * bytes at 16*l (l = 0..63) hold W[16 s + l % 16][32 j + 8 (l / 16) .. +8):
 * exactly the B operand of one 64-lane v_mfma_f32_16x16x32_f16, so one wave
 * load of a block reads one contiguous KiB. Offsets inside a layer's
 * fragment arena (gates in the order v, w, a, g, as w_lora1):
 *   f_rkv    [3C, C]       receptance, key, value rows stacked
 *   f_l1[g]  [R_g, C]      first LoRA steps
 *   f_l2[g]  [C, R_g]      second LoRA steps (K = R_g)
 *   f_o [C, C], f_fk [F, C], f_fv [C, F]
 * frag_bytes is the fragment arena size, a multiple of 256. */
/* Int8 arena, an optional third copy for batch-1 decode with int8 weights
 * (RWKV7_MODEL_INT8_DECODE): the matrices the decode streams, symmetric per
 * row, W[n, :] ~ scale[n] * q[n, :] with q int8 in [-127, 127] and scale f32:
 *   q_rkv [3C+SR, C]   the rows of w_rkv and w_lora1
 *   q_o [C, C], q_fk [F, C], q_fv [C, F]
 *   q_scale f32 [3C+SR + C + F + C]: the rows' scales in that order
 * q_bytes is the int8 arena size, a multiple of 256. The LoRA second steps
 * and the vectors stay in the f16 arena. */
typedef struct rwkv7_layer_layout {
  int64_t w_rkv, w_lora1, w_lora2, w_o, w_fk, w_fv, vec;
  int64_t bytes; /* arena size, a multiple of 256 */
  int64_t f_rkv, f_l1[4], f_l2[4], f_o, f_fk, f_fv;
  int64_t frag_bytes;
  int64_t q_rkv, q_o, q_fk, q_fv, q_scale;
  int64_t q_bytes;
} rwkv7_layer_layout;

/* Device-side model. Layer i's arena starts at layers + i * layout.bytes.
 * layers_frag and head_frag are optional (NULL: the GEMMs read the row-major
 * arenas); when set, layer i's fragment arena starts at
 * layers_frag + i * layout.frag_bytes and head_frag holds the head [V, C] in
 * fragment order. The two copies must hold the same weights. */
typedef struct rwkv7_model {
  rwkv7_dims dims;
  const void *layers; /* L consecutive layer arenas */
  const void *emb;    /* f16 [V, C], LayerNorm ln0 already applied (weight.py:175) */
  const void *head;   /* f16 [V, C] */
  const void *ln_out; /* f32 [2, C]: weight, bias */
  const void *layers_frag; /* optional: L fragment arenas */
  const void *head_frag;   /* optional: head in fragment order */
  uint32_t flags;          /* RWKV7_MODEL_* path choices, 0 for the defaults */
  const void *layers_q;    /* optional: L int8 arenas (layers_q + i * layout.q_bytes) */
  const void *head_q;      /* optional: head int8 [V, C], then f32 scales [V] at byte
                              offset rwkv7_head_q_scale_offset(dims) */
} rwkv7_model;

/* rwkv7_model.flags: run every step on the multi-launch paths (one launch
 * per stage) instead of the persistent kernels: batch-1 decode on the GEMV
 * kernels instead of the one-token kernel, and steps of B sequences x T tokens
 * with B T <= 16 (batched decode, short prefills) on the MFMA GEMMs instead of
 * the few-row kernel. */
#define RWKV7_MODEL_MULTI_LAUNCH_DECODE 1u
/* rwkv7_model.flags: batch-1 decode streams the int8 arenas (layers_q,
 * head_q; both required) in the persistent kernel, dequantising in the dot
 * products: half the weight bytes of the f16 decode. The weight-only
 * quantisation the reference plans inside its hand-written decode GEMV
 * (TODO.md:58-63). Prefill and batched decode still read the f16 arenas.
 * A batch-1 decode that cannot run that kernel (no logits requested, the
 * multi-launch flag, a device without the grid) fails with RWKV7_ESHAPE
 * rather than running on f16 weights. */
#define RWKV7_MODEL_INT8_DECODE 2u
/* rwkv7_model.flags: every 16-bit value the library reads or writes is
 * bfloat16 instead of IEEE half -- the matrices of the layer and fragment
 * arenas, emb, head, the state's tmix_x / cmix_x, logits and the f16 scratch
 * operands of the MFMA GEMMs (which then run v_mfma_f32_16x16x32_bf16); the
 * bf16 model of demo/rwkv7_bf16.py:18-27. The vectors section stays fp32,
 * arithmetic and the wkv state stay fp32. */
#define RWKV7_MODEL_BF16 4u

/* Recurrent state of `batch` independent sequences, layer-major arenas
 * (src/rwkv_tl/state.py:35-44 plus a leading batch dimension):
 *   tmix_x f16 [L, B, C]        time-mix token shift
 *   rnn    f32 [L, B, H, 64, 64] wkv state S[h, value row, key column]
 *   cmix_x f16 [L, B, C]        channel-mix token shift
 * Updated in place by decode and prefill. */
typedef struct rwkv7_state {
  void *tmix_x;
  void *rnn;
  void *cmix_x;
  int32_t batch;
} rwkv7_state;

/* ---- library ---------------------------------------------------------- */

int rwkv7_abi_version(void);
const char *rwkv7_strerror(int code);

/* Fills *out for `dims`. Returns RWKV7_ESHAPE for unsupported sizes
 * (n_embd != 64 * n_head, n_embd % 256, n_ffn % 256, ranks % 8, sum of ranks
 * > 512). */
int rwkv7_layer_layout_get(const rwkv7_dims *dims, rwkv7_layer_layout *out);

/* Byte offset of the f32 row scales inside the int8 head (after V * C bytes,
 * rounded up to 256), or -1 for unsupported dims. */
int64_t rwkv7_head_q_scale_offset(const rwkv7_dims *dims);

/* Bytes of scratch that rwkv7_decode / rwkv7_prefill need for `batch`
 * sequences of `seq_len` tokens (seq_len 1 for decode). The workspace must be
 * zero-filled once after allocation: its first regions hold the hand-off words
 * of the persistent kernels and are kept consistent by every later call.
 * One workspace must not be used by two calls that can run concurrently. */
int64_t rwkv7_workspace_bytes(const rwkv7_dims *dims, int32_t batch, int32_t seq_len);

/* Number of persistent-kernel launches on `workspace` that were aborted
 * (32-bit word at byte 32 of the workspace, cumulative; the caller may zero
 * it). Synchronises `stream` first. A launch aborts when one of its grid-wide
 * hand-offs waits longer than about a second (its workgroups were not all
 * resident, e.g. beside another process's kernels) or when its abort word was
 * set before it started; it then writes NaN into the logits of every row whose
 * inputs did not arrive and stops writing state, so the State holds the layers
 * completed before the failure. No counterpart in the reference (its CUDA
 * graphs have no grid-wide waits). */
int rwkv7_workspace_errors(const void *workspace, int64_t workspace_bytes, uint32_t *count, void *stream);

/* ---- model steps ------------------------------------------------------ */

/* One decode step for every sequence of `state`: tokens i64 [B] (device),
 * logits f16 [B, V] (device). Equivalent of RWKV7Base.decode
 * (demo/_rwkv7_base.py:74-87) / RWKV7Torch.decode (demo/rwkv7_torch.py:150-158),
 * batched. Token ids outside [0, V) are clamped into range. One sequence runs
 * as the one-token persistent kernel, 2..16 sequences as the few-row
 * persistent kernel, where the device fits their grids (else, and with
 * RWKV7_MODEL_MULTI_LAUNCH_DECODE, one launch per stage). */
int rwkv7_decode(const rwkv7_model *model, const rwkv7_state *state,
                 const int64_t *tokens, void *logits, void *workspace,
                 int64_t workspace_bytes, void *stream);

/* Number of kernel launches one rwkv7_decode call makes for `batch`
 * sequences of `model` (with_logits: whether logits are requested), or -1 for
 * unsupported dims. 1 means the step is one persistent kernel, so a graph
 * replay gains nothing over a direct call. The reference has no counterpart:
 * its CUDAGraph wrapper (demo/cuda_graph.py:61-235) always captures; this
 * lets the HIP-graph wrapper skip capture where it cannot help. */
int rwkv7_decode_launches(const rwkv7_model *model, int32_t batch, int32_t with_logits);

/* 1 if a step of batch x seq_len tokens (seq_len 1: a decode step with
 * logits) keeps every activation at fp32-grade precision (the batch-1
 * kernels compute in fp32; the few-row kernel and the batched GEMMs multiply
 * f32 activations as 16-bit parts plus 16-bit remainders), 0 if its GEMM
 * operands are rounded to the model's 16-bit format (the large-M path of
 * long prefills, where the products are MFMA-bound), -1 for bad arguments.
 * The reference has no counterpart (its fp16 model rounds every operand). */
int rwkv7_step_f32_activations(const rwkv7_model *model, int32_t batch, int32_t seq_len);

/* One batch-1 decode step, as rwkv7_decode, that allocates nothing and takes
 * no workspace. It has no counterpart in the reference; it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The persistent decode kernel's
 * exchange region lives in a static device array of
 * RWKV7_NOALLOC_SCRATCH_BYTES (1 MiB) that each GPU holds until the process
 * ends; calls that overlap on one GPU race on it. Returns RWKV7_EWORKSPACE
 * when the model's exchange region exceeds that size (0.4B needs 0.6 MB), and
 * RWKV7_ESHAPE when state->batch != 1, model->flags asks for the multi-launch
 * path, or the persistent kernel does not fit the device. An aborted launch
 * (see rwkv7_workspace_errors) shows only as NaN logits here. */
#define RWKV7_NOALLOC_SCRATCH_BYTES (1 << 20)
int rwkv7_decode_noalloc(const rwkv7_model *model, const rwkv7_state *state,
                         const int64_t *tokens, void *logits, void *stream);

/* Prefill seq_len tokens per sequence: tokens i64 [B, T] (device). Updates
 * state in place and produces no logits, like RWKV7Base.prefill
 * (demo/_rwkv7_base.py:89-98) / RWKV7Torch.prefill (demo/rwkv7_torch.py:160-171).
 * B x T <= 16 rows run as the few-row persistent kernel where the device fits
 * its grid (not with RWKV7_MODEL_MULTI_LAUNCH_DECODE). */
int rwkv7_prefill(const rwkv7_model *model, const rwkv7_state *state,
                  const int64_t *tokens, int32_t seq_len, void *workspace,
                  int64_t workspace_bytes, void *stream);

/* ---- operator level ---------------------------------------------------- */

/* Every operator below that takes 16-bit operands takes them in one format
 * per call: IEEE half, or bfloat16 when its bf16 argument is nonzero -- the
 * reference's two kernel namespaces, rwkv_tl.kernels.fp16 and .bf16
 * (src/rwkv_tl/kernels/fp16.py:13-30, bf16.py:13-30), which bind the same
 * kernels to float16 and bfloat16. "f16" in the comments below means that
 * 16-bit format; arithmetic is fp32 in both. */

/* DPLR (wkv7) recurrence over B sequences of T tokens and H heads:
 *   S[h] <- S[h] diag(w_t) + (S[h] a_t) b_t^T + v_t k_t^T ;  y_t = S[h] r_t
 * S f32 [B, H, 64, 64] (in place); r, k, v, a, b f16 [B, T, H, 64];
 * w f32 or f16 [B, T, H, 64] (w_is_f32 selects); y f16 [B, T, H, 64].
 * Stands in for fused_dplr (T=1) and fused_dplr_T
 * (src/rwkv_tl/kernels/dplr.py:256-285), where A = a, B = b. */
int rwkv7_wkv7(float *S, const void *r, const void *w, int32_t w_is_f32,
               const void *k, const void *v, const void *a, const void *b,
               void *y, int32_t B, int32_t T, int32_t H, int32_t bf16, void *stream);

/* rwkv7_wkv7 by the chunked algorithm: 16-token chunks whose transfer
 * matrices are formed on fp32 MFMA, all chunks at once, then one pass per
 * head that carries the state across the chunks. Same arguments and results
 * (to fp32 rounding; the state within 1e-5 relative of the serial scan at the
 * survey's C2 sizes), plus a device workspace of at least
 * rwkv7_wkv7_chunked_workspace_bytes(B, T, H) bytes (28,928 per 16 tokens of
 * each sequence and head). The chunked form of fused_dplr_T
 * (src/rwkv_tl/kernels/dplr.py:272-285), which the reference runs as a
 * chunked scan (dplr.py:174-227). */
int64_t rwkv7_wkv7_chunked_workspace_bytes(int32_t B, int32_t T, int32_t H);
int rwkv7_wkv7_chunked(float *S, const void *r, const void *w, int32_t w_is_f32,
                       const void *k, const void *v, const void *a, const void *b,
                       void *y, int32_t B, int32_t T, int32_t H, int32_t bf16,
                       void *workspace, int64_t workspace_bytes, void *stream);

/* The same recurrence with every operand f32 (S, r, w, k, v, a, b, y), for
 * training. When hist != NULL it receives the state entering each step, f32
 * [B, H, T, 64, 64], which rwkv7_wkv7_backward reads. Forward half of the DPLR
 * backward the reference plans (TODO.md:46-54: save the per-step states,
 * register_autograd on the DPLR op). */
int rwkv7_wkv7_f32(float *S, const float *r, const float *w, const float *k,
                   const float *v, const float *a, const float *b, float *y,
                   float *hist, int32_t B, int32_t T, int32_t H, void *stream);

/* Gradients of rwkv7_wkv7_f32 (reverse-time adjoint scan), all f32: given
 * hist (its recorded states), S_T (the state it left), its inputs, gy = dL/dy
 * [B, T, H, 64] and gS_T = dL/dS_T [B, H, 64, 64] (NULL: zero), writes
 * gS0 = dL/dS_0 and gr, gw, gk, gv, ga, gb [B, T, H, 64]. The DPLR backward of
 * the reference's training plan (TODO.md:46-54); the reference has no kernel
 * for it. */
int rwkv7_wkv7_backward(const float *hist, const float *S_T, const float *r,
                        const float *w, const float *k, const float *v,
                        const float *a, const float *b, const float *gy,
                        const float *gS_T, float *gS0, float *gr, float *gw,
                        float *gk, float *gv, float *ga, float *gb, int32_t B,
                        int32_t T, int32_t H, void *stream);

/* LayerNorm over the last dimension (eps 1e-5): x f32 or f16 [M, C]
 * (x_is_f32), weight/bias f32 [C], y f32 [M, C]. Stands in for LNWeight
 * (src/rwkv_tl/weight.py:14-15). */
int rwkv7_layernorm(const void *x, int32_t x_is_f32, const float *weight,
                    const float *bias, float *y, int32_t M, int32_t C, int32_t bf16,
                    void *stream);

/* Token-shift lerps x + mu_i (prev - x), i < n_mix (1 or 6), all f16 [C]
 * except mu f32 [n_mix, C]; out f16 [n_mix, C]. If x_copy != NULL it receives
 * x after every read of prev (x_copy may alias prev). Stands in for
 * fused_lerp6, fused_lerp6_copy and fused_lerp1_copy
 * (src/rwkv_tl/kernels/lerp.py:140-198). */
int rwkv7_lerp(const void *x, const void *prev, const float *mu, int32_t n_mix,
               void *out, void *x_copy, int32_t C, int32_t bf16, void *stream);

/* y = x W^T for one vector: x f32 [K], W f16 [N, K] (row stride ldw elements),
 * y f32 [N]. K % 256 == 0. Stands in for the decode projections
 * (demo/_rwkv7_base.py:87,206,290; kernels/gemm.py:215-262 at T=1). */
int rwkv7_gemv_f16(const float *x, const void *W, int64_t ldw, float *y,
                   int32_t N, int32_t K, int32_t bf16, void *stream);

/* y[n] = scale[n] * sum_k x[k] Q[n, k]: Q int8 [N, K] (row stride ldq bytes,
 * ldq % 16 == 0, Q and x 16-byte aligned), scale f32 [N], x and y f32.
 * 16 <= K <= 8192, K % 16 == 0. Weight-only int8 GEMV with the dequant fused
 * into the kernel: the quantisation step the reference plans for its
 * hand-written GEMV (TODO.md:58-63), which has no kernel there yet. */
int rwkv7_gemv_i8(const float *x, const void *Q, int64_t ldq, const float *scale,
                  float *y, int32_t N, int32_t K, void *stream);

/* y[n] = sum_k x[k] lut[n][code(n, k)]: any4 weights -- per row a table lut
 * f16 [N, 16] and one 4-bit code per weight, codes u8 [N, K/2] (row stride
 * ldc bytes, ldc % 8 == 0, codes 8-byte and x 16-byte aligned; byte j holds
 * column 2j in its low nibble and 2j+1 in its high nibble), x and y f32.
 * 16 <= K <= 8192, K % 16 == 0. The "any4" weight-only format the reference
 * names beside int8 for its quantised GEMV (TODO.md:58-63); it has no kernel
 * there. */
int rwkv7_gemv_any4(const float *x, const void *codes, int64_t ldc, const void *lut,
                    float *y, int32_t N, int32_t K, void *stream);

/* Y = epi(A W^T): A f16 [M, K] (row stride lda), W f16 [N, K] (ldw), fp32
 * accumulation. epi: 0 store f32, 1 store f16, 2 relu^2 store f16,
 * 3 add into f32 Y, 4 tanh store f16, 5 sigmoid store f16, 6 relu^2 store
 * f32, 7 tanh store f32, 8 sigmoid store f32. Y row stride ldy. K % 8 == 0.
 * bf16 is a flag word: RWKV7_GEMM_BF16 (A, W and 16-bit outputs are
 * bfloat16) and RWKV7_GEMM_A_F32 (A is f32, lda in floats, multiplied as its
 * 16-bit part plus the 16-bit remainder, two MFMAs per weight fragment:
 * fp32-grade activations). Stands in for fused_rkv_gemm / ffn_h / ffn_v /
 * out_mm (src/rwkv_tl/kernels/gemm.py:215-305). */
#define RWKV7_GEMM_BF16 1
#define RWKV7_GEMM_A_F32 2
int rwkv7_gemm_f16(const void *A, int64_t lda, const void *W, int64_t ldw,
                   void *Y, int64_t ldy, int32_t M, int32_t N, int32_t K,
                   int32_t epi, int32_t bf16, void *stream);

/* ---- time-mix stage operators (f16 in and out, fp32 arithmetic) --------- */

/* out[i] = exp(-sigmoid(w0[i] + x[i]) / sqrt(e)), i < C.
 * Replaces fused_w_gate (src/rwkv_tl/kernels/gates.py:287-291). */
int rwkv7_w_gate(const void *x, const void *w0, void *out, int32_t C, int32_t bf16, void *stream);

/* out = v + sigmoid(v0 + v12) * (v_first - v), [C].
 * Replaces fused_v_gate (gates.py:293-297). */
int rwkv7_v_gate(const void *v, const void *v_first, const void *v0, const void *v12, void *out,
                 int32_t C, int32_t bf16, void *stream);

/* a = sigmoid(a0 + a_x), kk = k * k_k, k' = k + k_a * (k * a - k), [C].
 * Replaces fused_a_kk_k (gates.py:299-313). */
int rwkv7_a_kk_k(const void *a0, const void *a_x, const void *k, const void *k_k, const void *k_a,
                 void *a_out, void *kk_out, void *k_out, int32_t C, int32_t bf16, void *stream);

/* Operands of rwkv7_gates, all f16: rank inputs vr [Rv], wr [Rw], ar [Ra],
 * gr [Rg] (first-step results, before activation); second-step matrices
 * v2t [C, Rv], w2t [C, Rw], a2t [C, Ra], g2t [C, Rg]; vectors [C]. */
typedef struct rwkv7_gates_io {
  const void *vr, *wr, *ar, *gr;
  const void *v2t, *w2t, *a2t, *g2t;
  const void *v, *v_first, *k, *v0, *w0, *a0, *k_k, *k_a;
  void *v_out, *w_out, *a_out, *kk_out, *k_out, *g_out;
} rwkv7_gates_io;

/* LoRA second steps with their activations (tanh for w, sigmoid for g) and
 * the gate math: v' = v + sigmoid(v0 + v2t vr) (v_first - v),
 * w = exp(-sigmoid(w0 + w2t tanh(wr)) / sqrt(e)), a = sigmoid(a0 + a2t ar),
 * kk = k k_k, k' = k + k_a (k a - k), g = g2t sigmoid(gr).
 * Replaces fused_gates (gates.py:125-213,315-357). */
int rwkv7_gates(const rwkv7_gates_io *io, int32_t rank_v, int32_t rank_w, int32_t rank_a, int32_t rank_g,
                int32_t C, int32_t bf16, void *stream);

/* Packed LoRA first steps: out = [v1t; w1t; a1t; g1t] @ (xv | xw | xa | xg),
 * W [Rv+Rw+Ra+Rg, C], inputs [C], out [Rv+Rw+Ra+Rg]; C % 8 == 0.
 * Replaces fused_rank_gemv (gates.py:215-285). */
int rwkv7_rank_gemv(const void *xv, const void *xw, const void *xa, const void *xg, const void *W, void *out,
                    int32_t rank_v, int32_t rank_w, int32_t rank_a, int32_t rank_g, int32_t C, int32_t bf16,
                    void *stream);

/* Per head h < H over its 64 channels: kk_norm = kk / max(||kk||, 1e-12),
 * b = -kk_norm * a; all [H, 64].
 * Replaces fused_l2norm_neg_kk_a (src/rwkv_tl/kernels/dplr.py:45-71,229-235). */
int rwkv7_l2norm_neg_kk_a(const void *kk, const void *a, void *kk_norm, void *b, int32_t H, int32_t bf16,
                          void *stream);

/* Per head: GroupNorm of y (biased variance, eps 64e-5) * ln_w + ln_b, plus
 * (sum over the head of r * k * r_k) * v; y, r, k, v, r_k [H, 64], ln_w,
 * ln_b and out [H * 64].
 * Replaces fused_gn_rkrk (dplr.py:73-124,237-254). */
int rwkv7_gn_rkrk(const void *y, const void *r, const void *k, const void *v, const void *r_k,
                  const void *ln_w, const void *ln_b, void *out, int32_t H, int32_t bf16, void *stream);

/* ---- sampling ---------------------------------------------------------- */

/* Parameters of one sampling call (demo/sampling.py:13-70). */
typedef struct rwkv7_sampling {
  float temperature;        /* <= 0: greedy argmax, first index among ties */
  int32_t top_k;            /* <= 0 or >= V: no top-k filter */
  float top_p;              /* >= 1: no nucleus filter */
  float repetition_penalty; /* 1: none; else seen tokens' logits x -> x > 0 ? x / p : x * p */
  uint64_t seed;            /* Philox4x32-10 key */
  uint64_t offset;          /* counter of this draw (one per call; the row is the second counter word) */
} rwkv7_sampling;

/* Sample one token per row of logits [B, V] (logits_dtype: 0 f16, 1 f32,
 * 2 bf16; row stride ld elements, V <= 65536), into out i64 [B]. In order: repetition penalty on the tokens
 * whose bit is set in seen u32 [B, seen_ld] (bit t % 32 of word t / 32;
 * NULL: none), greedy argmax if temperature <= 0, else division by the
 * temperature, top-k (keep x >= the k-th largest), top-p (keep the tokens
 * whose descending-order cumulative probability, excluding their own, is
 * <= top_p) and one draw from the kept distribution, computed in 64-bit fixed
 * point and drawn by inverse CDF in vocabulary order with Philox4x32-10
 * (key = seed, counter = (offset, row, 0)). update_seen sets the sampled
 * token's bit in seen. probs f32 [B, probs_ld] (optional) receives the kept
 * distribution (one-hot when greedy). No host sync. With a workspace of at
 * least rwkv7_sample_workspace_bytes(B, V) bytes, a call with temperature >
 * 0, 1 <= top_k <= 128 and no probs spreads each row over V / 2048
 * workgroups (each keeps the candidates of its slice of the row, a second
 * launch draws from them) and draws the same token as without it; otherwise
 * (workspace NULL) one workgroup per row does all of it.
 * Stands in for sample_logits (demo/sampling.py:13-70) as called by
 * RWKV7Model.generate (demo/_rwkv7_abc.py:41-72), with the draw of
 * torch.multinomial replaced by the counter-based one above. */
int64_t rwkv7_sample_workspace_bytes(int32_t B, int32_t V);
int rwkv7_sample(const void *logits, int32_t logits_dtype, int64_t ld, int32_t B, int32_t V, const rwkv7_sampling *params,
                 uint32_t *seen, int64_t seen_ld, int32_t update_seen, int64_t *out, float *probs,
                 int64_t probs_ld, void *workspace, int64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV7_HIP_H */
