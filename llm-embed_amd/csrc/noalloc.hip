// lle_embed_packed_noalloc: lle_embed_packed_async's forward for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// Every activation buffer of the forward (residual stream, f16 copies, Q / K / V^T heads,
// attention output, GeGLU output, split-K partials, packed-row tables) is carved from one
// fixed device array, `scratch`, instead of the model's grow-only workspace. Its device address
// is resolved once per device with hipGetSymbolAddress at set-up (lle_init, or the first call
// on a device) and kept per device; host code never passes the array's own name to a kernel
// or a copy (in host code it is a host-side stand-in, not a device address).
//
// Every call on one device shares that device's array: calls that overlap on one GPU race
// (serialise them on one stream, or finish one before the next starts). No kernel of the
// forward reads a workspace byte before writing it in the same call, so nothing needs
// clearing between calls.
#include <mutex>

#include "lle_internal.h"

namespace lle {
namespace {

constexpr size_t kScratchBytes = (size_t)LLE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};  // device address of `scratch`, per device

}  // namespace

int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(LLE_EINVAL, "device ordinal out of range for the scratch table");
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_ptr[device]) return LLE_OK;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return fail(LLE_EDEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  g_ptr[device] = p;
  return LLE_OK;
}

}  // namespace lle

extern "C" int32_t lle_embed_packed_noalloc(lle_model* m, const int32_t* d_ids, const int32_t* d_seq_off, int32_t B,
                                            int32_t T, int32_t L, int32_t out_dim, float* d_out, void* stream) {
  using namespace lle;
  if (!m) return fail(LLE_EINVAL, "null model");
  const int dev = model_device(m);
  if (dev < 0 || dev >= kMaxDevices) return fail(LLE_EINVAL, "model device out of range for the scratch table");
  void* p = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    p = g_ptr[dev];
  }
  if (!p) {  // a device the library was not initialised on: set up now, with it current
    LLE_HIP(hipSetDevice(dev));
    const int rc = noalloc_setup(dev);
    if (rc) return rc;
    std::lock_guard<std::mutex> lk(g_mu);
    p = g_ptr[dev];
  }
  return embed_packed_scratch(m, d_ids, d_seq_off, B, T, L, out_dim, d_out, (hipStream_t)stream, p, kScratchBytes);
}
