// Hand-off latency probe, in the diagnostic build only (RWKV7_TIMELINE;
// bench.py --hops). The persistent decode kernels move every stage's output
// through 64-bit {tag, value} words written with device-scope (sc1) stores
// and polled with device-scope loads; this probe times that mechanism alone.
// G workgroups of one wave run at once; lane 0 of workgroup g and of its
// partner g ^ x play ping-pong: in round i each stores {tag0 + i, g} to its
// own word, then polls the partner's word until it carries round i or i + 1
// (the partner can be one round ahead, never two). Every poll loop is bounded
// (kProbeSpin polls; a workgroup that gives up counts it and stops), so the
// grid always drains. Workgroups are dispatched round-robin over the XCDs, so
// x = 1 pairs workgroups on different XCDs and x = 8 on the same one; the
// probe records each workgroup's XCC id to show it.
#include "rwkv7_kernels.h"

#ifdef RWKV7_TIMELINE

namespace rwkv7 {
namespace {

constexpr int kProbeWarm = 8;        // rounds before the timed ones
constexpr int kProbeSpin = 1 << 22;  // polls before a workgroup gives up
constexpr int kProbeStride = 16;     // words between two workgroups' words (128 bytes)

__global__ __launch_bounds__(64) void hop_probe_kernel(uint64_t *words, int x, unsigned tag0, int rounds,
                                                       unsigned long long *out) {
  const int g = blockIdx.x;
  if (threadIdx.x != 0) return;
  // XCC_ID (hardware register 20), bits 0..3
  const unsigned xcc = __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11));
  uint64_t *mine = words + (int64_t)kProbeStride * g;
  const uint64_t *theirs = words + (int64_t)kProbeStride * (g ^ x);
  unsigned long long t0 = 0, t1 = 0, errs = 0;
  for (int i = 0; i < rounds; ++i) {
    if (i == kProbeWarm) t0 = __builtin_amdgcn_s_memrealtime();
    const unsigned tag = tag0 + (unsigned)i;
    __hip_atomic_store(mine, ((uint64_t)tag << 32) | (unsigned)g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the partner's round index (a zeroed word reads as an index past the last round)
    int spins = 0;
    for (;;) {
      const unsigned r = (unsigned)(__hip_atomic_load(theirs, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >> 32) - tag0;
      if (r >= (unsigned)i && r < (unsigned)rounds) break;
      if (++spins > kProbeSpin) {
        ++errs;
        break;
      }
    }
    if (errs) break;
  }
  t1 = __builtin_amdgcn_s_memrealtime();
  out[3 * g] = errs ? 0ull : t1 - t0;
  out[3 * g + 1] = errs;
  out[3 * g + 2] = xcc;
}

}  // namespace
}  // namespace rwkv7

// words: u64 [16 G], zeroed; out: u64 [3 G] per workgroup: real-time-counter
// ticks (100 MHz) of rounds kProbeWarm .. rounds - 1, polls given up, XCC id.
// tag0 + rounds must not wrap past 2^32 (tags are compared as offsets from
// tag0, so any tag0 works on a zeroed buffer).
extern "C" int rwkv7_probe_hops(uint64_t *words, int32_t G, int32_t x, int32_t rounds, uint32_t tag0,
                                uint64_t *out, void *stream) {
  if (!words || !out) return RWKV7_EINVAL;
  if (G < 2 || G > 4096 || x < 1 || G % (2 * x) != 0 || rounds <= rwkv7::kProbeWarm || rounds > (1 << 20))
    return RWKV7_ESHAPE;
  if (tag0 == 0 || (uint64_t)tag0 + (uint64_t)rounds >= (1ull << 32)) return RWKV7_EINVAL;
  rwkv7::hop_probe_kernel<<<G, 64, 0, static_cast<hipStream_t>(stream)>>>(
      words, x, tag0, rounds, reinterpret_cast<unsigned long long *>(out));
  return hipGetLastError() == hipSuccess ? RWKV7_OK : RWKV7_ELAUNCH;
}

#endif  // RWKV7_TIMELINE
