// Device-side helpers shared by the RWKV7 gfx950 kernels.
//
// Wavefronts are 64 lanes. Reductions use DPP lane permutes inside a 16-lane
// row and v_readlane across rows, so no reduction touches LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rwkv7_hip.h"

#define RWKV7_DEV __device__ __forceinline__

namespace rwkv7 {

constexpr int kWave = 64;
constexpr int kN = RWKV7_HEAD_SIZE;  // head size
constexpr float kLnEps = 1e-5f;      // F.layer_norm default (src/rwkv_tl/weight.py:15)
constexpr float kGnEps = 64e-5f;     // GroupNorm eps (demo/rwkv7_torch.py:114)
// exp(-sigmoid(z) / sqrt(e)) decay (demo/rwkv7_torch.py:101-104); 1/sqrt(e) as float.
constexpr float kInvSqrtE = 0.60653065971263342f;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// ---- stage timeline (diagnostic builds) -----------------------------------
// `build_hip.py --timeline` defines RWKV7_TIMELINE and builds a separate
// library (librwkv7_hip_timeline.so): thread 0 of a workgroup of a persistent
// kernel then records the 100 MHz real-time counter at named points of every
// layer into that kernel's device array, [layer][workgroup][point], which
// rwkv7_timeline_read_* copies to the host (bench.py --timeline). The product
// build compiles every stamp away.
constexpr int kTlLayers = 32, kTlGroups = 1024, kTlPoints = 24;
#ifdef RWKV7_TIMELINE
#define RWKV7_TL_BUFFER(name) __device__ unsigned long long name[kTlLayers * kTlGroups * kTlPoints]
#define RWKV7_TL(buf, layer, pt)                                                                           \
  do {                                                                                                     \
    if (threadIdx.x == 0 && (layer) < kTlLayers && blockIdx.x < kTlGroups)                               \
      buf[((int64_t)(layer) * kTlGroups + blockIdx.x) * kTlPoints + (pt)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define RWKV7_TL_READER(fn, buf)                                                                  \
  extern "C" int fn(void *host, int64_t bytes) {                                                  \
    if (!host || bytes < (int64_t)sizeof(buf)) return RWKV7_EINVAL;                               \
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(buf), sizeof(buf), 0, hipMemcpyDeviceToHost) ==   \
                   hipSuccess                                                                      \
               ? RWKV7_OK                                                                          \
               : RWKV7_ELAUNCH;                                                                    \
  }
#else
#define RWKV7_TL_BUFFER(name) static_assert(true, "")
#define RWKV7_TL(buf, layer, pt) \
  do {                           \
  } while (0)
#define RWKV7_TL_READER(fn, buf) static_assert(true, "")
#endif

// ---- lane permutes ------------------------------------------------------

template <int CTRL>
RWKV7_DEV float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <- 7-i within each 8
constexpr int kDppMirror = 0x140;     // lane i <- 15-i within each 16

// Sum over groups of 4 consecutive lanes; every lane gets its group's sum.
RWKV7_DEV float sum4(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  return v;
}

// Sum over each 16-lane row; every lane of the row gets the row sum.
RWKV7_DEV float sum16(float v) {
  v = sum4(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return v;
}

// Two independent 16-lane row sums, reduced in lockstep.
RWKV7_DEV float2 sum16x2(float a, float b) {
  a += dpp<kDppXor1>(a);
  b += dpp<kDppXor1>(b);
  a += dpp<kDppXor2>(a);
  b += dpp<kDppXor2>(b);
  a += dpp<kDppHalfMirror>(a);
  b += dpp<kDppHalfMirror>(b);
  a += dpp<kDppMirror>(a);
  b += dpp<kDppMirror>(b);
  return make_float2(a, b);
}

// Sum over the whole wave; the result is wave-uniform.
RWKV7_DEV float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

RWKV7_DEV float wave_sum(float v) {
  v = sum16(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

// Two independent wave sums, reduced in lockstep (one latency chain for both).
RWKV7_DEV float2 wave_sum2(float a, float b) {
  a += dpp<kDppXor1>(a);
  b += dpp<kDppXor1>(b);
  a += dpp<kDppXor2>(a);
  b += dpp<kDppXor2>(b);
  a += dpp<kDppHalfMirror>(a);
  b += dpp<kDppHalfMirror>(b);
  a += dpp<kDppMirror>(a);
  b += dpp<kDppMirror>(b);
  return make_float2((lane_value(a, 0) + lane_value(a, 16)) + (lane_value(a, 32) + lane_value(a, 48)),
                     (lane_value(b, 0) + lane_value(b, 16)) + (lane_value(b, 32) + lane_value(b, 48)));
}

// ---- conversions ----------------------------------------------------------

RWKV7_DEV void h8_to_f(const uint4 &u, float f[8]) {
  half8 h = __builtin_bit_cast(half8, u);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
}

RWKV7_DEV uint4 f_to_h8(const float f[8]) {
  half8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (_Float16)f[i];
  return __builtin_bit_cast(uint4, h);
}

RWKV7_DEV float h2f(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }
RWKV7_DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// bfloat16: the upper half of an fp32 (widening is exact); narrowing rounds
// to nearest even (v_cvt_pk_bf16_f32).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
RWKV7_DEV float b2f(uint16_t u) { return __builtin_bit_cast(float, (uint32_t)u << 16); }
RWKV7_DEV uint16_t f2b(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// The 16-bit storage format of a model's weights, shift states and logits:
// IEEE half (BF = false) or bfloat16 (BF = true). Arithmetic is fp32 either way.
template <bool BF>
struct F16T {
  static RWKV7_DEV float to_f(uint16_t u) { return BF ? b2f(u) : h2f(u); }
  static RWKV7_DEV uint16_t from_f(float f) { return BF ? f2b(f) : f2h(f); }
  static RWKV7_DEV void to_f8(const uint4 &u, float f[8]) {
    if constexpr (BF) {
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
        f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xFFFF0000u);
      }
    } else {
      h8_to_f(u, f);
    }
  }
  static constexpr uint16_t kNaN = BF ? 0x7FC0u : 0x7E00u;
};

// A bfloat16 element as a distinct type, for templates that take the element
// type (the operator-level wkv7 scan).
struct bf16_t {
  uint16_t bits;
};

// The same chosen at run time (small elementwise kernels).
RWKV7_DEV float u16_to_f(uint16_t u, int bf) { return bf ? b2f(u) : h2f(u); }
RWKV7_DEV uint16_t f_to_u16(float f, int bf) { return bf ? f2b(f) : f2h(f); }
RWKV7_DEV void u16x8_to_f(const uint4 &u, float f[8], int bf) {
  if (bf) F16T<true>::to_f8(u, f);
  else F16T<false>::to_f8(u, f);
}

// 16x16x32 MFMA on 16-bit operands of format F16T<BF> (8 per lane, any
// 16-byte type), fp32 accumulation.
template <bool BF, class T>
RWKV7_DEV floatx4 mfma16(const T &a, const T &b, const floatx4 &c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
}

// Eight f32 values (two 16-byte words, in order) as two MFMA operands of
// format F16T<BF>: hi = each value rounded to 16 bits, lo = the remainder
// x - hi (exact in fp32) rounded to 16 bits. hi + lo carries 22 significant
// bits for IEEE half (16 for bfloat16), so two MFMAs against the same 16-bit
// weights multiply f32 activations to about fp32 precision; for half, a
// remainder below the smallest subnormal (|x| < 2^-13) is lost, an absolute
// error under 2^-25.
template <bool BF>
RWKV7_DEV void split_hi_lo(const uint4 &a, const uint4 &b, uint4 &hi, uint4 &lo) {
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x0 = __builtin_bit_cast(float, w[2 * i]), x1 = __builtin_bit_cast(float, w[2 * i + 1]);
    const uint16_t h0 = F16T<BF>::from_f(x0), h1 = F16T<BF>::from_f(x1);
    const uint16_t l0 = F16T<BF>::from_f(x0 - F16T<BF>::to_f(h0)), l1 = F16T<BF>::from_f(x1 - F16T<BF>::to_f(h1));
    h[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
    l[i] = (uint32_t)l0 | ((uint32_t)l1 << 16);
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

RWKV7_DEV float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }

// Weight streams are read exactly once per step: load them non-temporally so
// they do not evict the small activation vectors every wave re-reads.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
RWKV7_DEV uint4 ld_stream(const uint4 *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Buffer descriptor of `bytes` bytes at p (both wave-uniform), in scalar
// registers: base address, stride 0, the byte count (accesses past it are
// dropped, loads read zeros), 32-bit data format.
RWKV7_DEV i32x4 buffer_words(const void *p, int bytes) {
  const uint64_t a = (uint64_t)p;
  return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a), __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)),
               __builtin_amdgcn_readfirstlane(bytes), 0x00020000};
}

// LDS DMA: each lane's 16 bytes at voff + soff of the buffer land at
// lds + 16 lane (rsrc, lds and soff wave-uniform). Issued as inline assembly,
// so that the compiler does not track it: it would otherwise wait for every
// DMA in flight before any LDS access whose alias information it has lost
// (most accesses of an unrolled loop, and every access of a multi-buffered
// array), which serialises a ring of prefetches; and a builtin DMA whose
// operands it cannot prove uniform becomes a loop over lanes. The caller
// waits for these loads with counts of its own (s_waitcnt vmcnt) and orders
// LDS reads after them with a barrier that clobbers memory. M0 carries the
// LDS address; the gfx9 LDS instructions that the compiler emits do not read
// M0, and one wait state separates its write from the DMA.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
RWKV7_DEV void dma16(i32x4 rsrc, uint32_t lds, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane((int)lds)), "v"(voff), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory", "m0");
}
#pragma clang diagnostic pop
RWKV7_DEV uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)p; }

}  // namespace rwkv7

#define RWKV7_CHECK_LAUNCH()                                    \
  do {                                                          \
    if (hipGetLastError() != hipSuccess) return RWKV7_ELAUNCH;  \
  } while (0)
