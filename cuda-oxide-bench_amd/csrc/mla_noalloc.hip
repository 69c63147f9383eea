// Allocation-free MLA decode: mx_mla_decode with its split partials in a
// library-owned device array instead of a caller workspace.
//
// This translation unit holds nothing but that array and the entry point,
// so the array lives in a code object of its own: processes that only call
// the other entry points never reserve it, and with the HIP runtime's
// deferred code-object loading a GPU holds it from the first call of
// mx_mla_decode_noalloc there until the process ends.
//
// `scratch` is a host-side stand-in for the array in host code, not a
// device address: its device address is looked up once per device (with
// that device current) and only that address is passed on.  Every call on
// one GPU shares that GPU's array, so calls that overlap on one GPU race;
// the decode writes every partial before its merge reads it, so nothing
// needs clearing between calls.
#include "mx_common.h"

namespace mx {
namespace mla_noalloc {

static __device__ __align__(256) unsigned char scratch[MX_MLA_SCRATCH_BYTES];

static std::once_flag scratch_once[kMaxDevices];
static void* scratch_dev[kMaxDevices];
static hipError_t scratch_rc[kMaxDevices];

// Device address of this device's `scratch`, looked up on the first call.
static int scratch_ptr(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MX_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxDevices) return MX_ERR_UNSUPPORTED;
  std::call_once(scratch_once[dev], [dev] {
    void* p = nullptr;
    scratch_rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    scratch_dev[dev] = scratch_rc[dev] == hipSuccess ? p : nullptr;
  });
  if (scratch_rc[dev] != hipSuccess || !scratch_dev[dev]) return MX_ERR_LAUNCH;
  *out = scratch_dev[dev];
  return MX_OK;
}

}  // namespace mla_noalloc
}  // namespace mx

extern "C" int mx_mla_decode_noalloc(const void* Q, const void* KV, void* O, int B, int H, int T, int d_latent,
                                     int d_rope, float scale, void* stream) {
  const size_t need = mx_mla_decode_workspace(B, H, T, d_latent);
  // No split (or invalid sizes): mx_mla_decode validates and runs without a workspace.
  if (need == 0) return mx_mla_decode(Q, KV, O, B, H, T, d_latent, d_rope, scale, nullptr, 0, stream);
  // Every other argument is checked, and nothing enqueued, by a call without
  // the workspace: it can only fail for the missing workspace.
  if (const int e = mx_mla_decode(Q, KV, O, B, H, T, d_latent, d_rope, scale, nullptr, 0, stream);
      e != MX_ERR_WORKSPACE)
    return e == MX_OK ? MX_ERR_LAUNCH : e;
  if (need > (size_t)MX_MLA_SCRATCH_BYTES) return MX_ERR_WORKSPACE;
  void* ws = nullptr;
  if (const int e = mx::mla_noalloc::scratch_ptr(&ws)) return e;
  return mx_mla_decode(Q, KV, O, B, H, T, d_latent, d_rope, scale, ws, need, stream);
}
