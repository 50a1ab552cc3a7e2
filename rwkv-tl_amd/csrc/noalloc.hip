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
// launch epoch and tags continue), and a call with different sizes (another
// layout of the hand-off words, other tags) clears the region first with a
// fill kernel on the caller's stream. Calls that overlap on one GPU race on the
// shared array.
#include <atomic>

#include "rwkv7_kernels.h"

namespace rwkv7 {

constexpr int64_t kNoAllocScratchBytes = RWKV7_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
struct NoAllocDevice {
  std::atomic<void *> ptr{nullptr};     // device address of this device's `scratch`
  std::atomic<uint64_t> sizes{0};       // signature of the sizes the region was last laid out for
};
NoAllocDevice g_noalloc[kMaxDevices];

uint64_t sizes_signature(const rwkv7_dims &d, int G) {
  uint64_t h = 1469598103934665603ull;  // FNV-1a over the fields that shape the region and its tags
  const int32_t f[7] = {d.n_layer, d.n_embd, d.n_ffn, d.rank_w + d.rank_a + d.rank_v + d.rank_g, d.n_head, G, 1};
  for (int32_t v : f) {
    for (int b = 0; b < 4; ++b) {
      h ^= (uint64_t)((v >> (8 * b)) & 0xFF);
      h *= 1099511628211ull;
    }
  }
  return h | 1ull;  // never 0 (the "not laid out yet" value)
}

__global__ void clear_kernel(uint4 *p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
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
  if (need > kNoAllocScratchBytes) return RWKV7_EWORKSPACE;

  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RWKV7_ELAUNCH;
  NoAllocDevice &nd = g_noalloc[dev];
  void *ptr = nd.ptr.load(std::memory_order_acquire);
  if (!ptr) {
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return RWKV7_ELAUNCH;
    nd.ptr.store(ptr, std::memory_order_release);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t sig = sizes_signature(d, mk_cus());
  if (nd.sizes.load(std::memory_order_relaxed) != sig) {
    const int64_t n16 = (need + 15) / 16;
    clear_kernel<<<(int)((n16 + 255) / 256 < 1024 ? (n16 + 255) / 256 : 1024), 256, 0, st>>>(
        static_cast<uint4 *>(ptr), n16);
    RWKV7_CHECK_LAUNCH();
    nd.sizes.store(sig, std::memory_order_relaxed);
  }
  return launch_decode_mk(*model, lay, *state, tokens, logits, static_cast<char *>(ptr), st);
}
