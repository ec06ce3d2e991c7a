// Allocation-free module-level forward: cvn_converse2d_fwd_f32 with its workspace (the transfer table
// and, on the multi-pass routes, the spectra between passes) placed in a file-scope device array of
// CVN_NOALLOC_SCRATCH_BYTES instead of a caller buffer, for callers that cannot allocate device memory.
//
// In host code `scratch` names a host-side stand-in for the array, not a device address: its device
// address is obtained once per device with hipGetSymbolAddress (each device holds its own copy) and
// only that address is ever handed to kernels.  Calls on one device share the array, so calls that
// overlap on one device race; the forward writes every byte it later reads, so nothing needs clearing
// between calls.
#include <atomic>

#include "cvn_common.h"

namespace {

constexpr size_t kScratchBytes = CVN_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::atomic<void*> g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// Device address of `scratch` on the current device, looked up on the first call per device.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return cvn::fail(CVN_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return cvn::fail(CVN_ERR_UNSUPPORTED, "device index %d above %d", dev, kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return cvn::fail(CVN_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return CVN_OK;
}

}  // namespace

extern "C" int cvn_converse2d_fwd_noalloc_f32(const float* x, int64_t B, int64_t C, int64_t H, int64_t W,
                                              const float* psf, int64_t psf_batch, int kh, int kw,
                                              const float* bias, float eps, int scale, int pad, int pad_mode,
                                              int act, float* out, cvn_stream_t stream) {
  const size_t need = cvn_converse2d_fwd_workspace(B, C, H, W, psf_batch, kh, kw, scale, pad);
  if (need == 0)  // invalid or unsupported geometry: the forward reports why before launching anything
    return cvn_converse2d_fwd_f32(x, B, C, H, W, psf, psf_batch, kh, kw, bias, eps, scale, pad, pad_mode, act,
                                  out, nullptr, 0, stream);
  if (need > kScratchBytes)
    return cvn::fail(CVN_ERR_UNSUPPORTED,
                     "this call needs %zu bytes of scratch; the allocation-free forward holds %zu "
                     "(use cvn_converse2d_fwd_f32 with a caller workspace)",
                     need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != CVN_OK) return rc;
  return cvn_converse2d_fwd_f32(x, B, C, H, W, psf, psf_batch, kh, kw, bias, eps, scale, pad, pad_mode, act, out,
                                ws, kScratchBytes, stream);
}
