// rwkv7_decode_noalloc: one batch-1 decode step that allocates nothing.
//
// Callers that cannot allocate (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc) cannot provide the workspace that
// rwkv7_decode takes. The only scratch the persistent decode kernel needs is
// its exchange region (sync words, start words and the tagged hand-off
// vectors, mk_exchange_bytes: 0.6 MB for the 0.4B model); here it lives in a
// file-scope device array, `scratch`, of kNoAllocScratchBytes. Every GPU the
// library runs on holds its own copy until the process ends.
//
// In host code `scratch` names a host-side stand-in, not a device address, so
// the kernel is never handed that name: the first call on each device (with
// that device current) resolves the device copy's address with
// hipGetSymbolAddress and keeps it per device.
//
// The array is zero when the code object is loaded, which is the state the
// exchange region needs before its first launch. It keeps the last call's
// contents; those stay valid for the next launch of the same model sizes (the
// launch epoch and tags continue), but not for other sizes (another layout of
// the hand-off words, other tags). So the array's last 256 bytes hold the
// signature of the sizes the region is laid out for, and every call first
// runs a small kernel that compares it on the device and clears the region
// when it differs. The check lives on the device, not in host memory, so it
// holds however calls are mixed: a call captured into a HIP graph carries
// its own check, and a replay that lays the region out for its sizes is seen
// by the next eager call of other sizes. Calls that overlap on one GPU race on
// the shared array.
#include <atomic>

#include "rwkv7_kernels.h"

namespace rwkv7 {

constexpr int64_t kNoAllocScratchBytes = RWKV7_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
// the last 256 bytes of `scratch`: the layout signature (u64) and an arrival
// counter of the check kernel (u32, zero between launches)
constexpr int64_t kTailBytes = 256;
constexpr int64_t kRegionMax = kNoAllocScratchBytes - kTailBytes;
constexpr int kCheckGrid = 64;
std::atomic<void *> g_ptr[kMaxDevices];  // device address of each device's `scratch`

uint64_t sizes_signature(const rwkv7_dims &d, int G) {
  uint64_t h = 1469598103934665603ull;  // FNV-1a over the fields that shape the region and its tags
  const int32_t f[7] = {d.n_layer, d.n_embd, d.n_ffn, d.rank_w + d.rank_a + d.rank_v + d.rank_g, d.n_head, G, 1};
  for (int32_t v : f) {
    for (int b = 0; b < 4; ++b) {
      h ^= (uint64_t)((v >> (8 * b)) & 0xFF);
      h *= 1099511628211ull;
    }
  }
  return h | 1ull;  // never 0 (the value of a region never laid out)
}

// Clears the first n16 16-byte words of the region unless the stored
// signature equals sig, then records sig. Every workgroup reads the stored
// signature before it counts itself in, and only the last to arrive writes the
// new one, so all workgroups see the same old value; the decode kernel runs
// after this launch has finished (same stream), so it sees the cleared region.
__global__ __launch_bounds__(256) void check_clear_kernel(uint4 *p, int64_t n16, uint64_t *sigw, unsigned *arrived,
                                                          uint64_t sig) {
  __shared__ int differs;
  if (threadIdx.x == 0)
    differs = __hip_atomic_load(sigw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != sig;
  __syncthreads();
  if (differs) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
      p[i] = make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(arrived, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (old == gridDim.x - 1) {
      __hip_atomic_store(arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (differs) __hip_atomic_store(sigw, sig, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace
}  // namespace rwkv7

using namespace rwkv7;

extern "C" int rwkv7_decode_noalloc(const rwkv7_model *model, const rwkv7_state *state, const int64_t *tokens,
                                    void *logits, void *stream) {
  if (!model || !state || !tokens || !logits) return RWKV7_EINVAL;
  if (!model->layers || !model->emb || !model->head || !model->ln_out) return RWKV7_EINVAL;
  if (!state->tmix_x || !state->rnn || !state->cmix_x) return RWKV7_EINVAL;
  rwkv7_layer_layout lay;
  const int rc = rwkv7_layer_layout_get(&model->dims, &lay);
  if (rc != RWKV7_OK) return rc;
  if (state->batch != 1 || (model->flags & RWKV7_MODEL_MULTI_LAUNCH_DECODE)) return RWKV7_ESHAPE;
  const rwkv7_dims &d = model->dims;
  if ((model->flags & RWKV7_MODEL_INT8_DECODE) && !mk_int8(*model)) return RWKV7_EINVAL;
  if (!mk_usable(*model)) return RWKV7_ESHAPE;
  const int64_t need = mk_exchange_bytes(d.n_embd, d.n_ffn, d.rank_w + d.rank_a + d.rank_v + d.rank_g);
  if (need > kRegionMax) return RWKV7_EWORKSPACE;

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RWKV7_ELAUNCH;
  void *ptr = g_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return RWKV7_ELAUNCH;
    g_ptr[dev].store(ptr, std::memory_order_release);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  char *base = static_cast<char *>(ptr);
  check_clear_kernel<<<kCheckGrid, 256, 0, st>>>(reinterpret_cast<uint4 *>(base), (need + 15) / 16,
                                                  reinterpret_cast<uint64_t *>(base + kRegionMax),
                                                  reinterpret_cast<unsigned *>(base + kRegionMax + 8),
                                                  sizes_signature(d, mk_cus()));
  RWKV7_CHECK_LAUNCH();
  return launch_decode_mk(*model, lay, *state, tokens, logits, base, st);
}
