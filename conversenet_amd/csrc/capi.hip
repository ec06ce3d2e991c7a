// Library-wide C-ABI entry points: version, error string, cache no-op, calibration copy kernel.
#include <algorithm>

#include "cvn_common.h"

namespace cvn {
std::string& last_error_slot() {
  static thread_local std::string s;
  return s;
}

// 16-byte grid-stride copy with a scalar tail; used to calibrate HBM byte counters and to measure
// the attainable HBM bandwidth.  Stores are non-temporal (streaming), as in the library's kernels
// whose outputs are not read back by the same launch.
typedef float copy_f32x4 __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(256) k_copy(const copy_f32x4* __restrict__ src, copy_f32x4* __restrict__ dst,
                                              int64_t n4, const float* __restrict__ src1,
                                              float* __restrict__ dst1, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride)
    __builtin_nontemporal_store(src[i], &dst[i]);
  for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst1[i] = src1[i];
}
}  // namespace cvn

using namespace cvn;

extern "C" const char* cvn_version(void) { return "conversenet_amd 0.1 (gfx950)"; }

extern "C" const char* cvn_last_error(void) { return last_error_slot().c_str(); }

extern "C" int cvn_clear_cache(void) { return CVN_OK; }

extern "C" int cvn_copy_f32(const float* src, float* dst, int64_t n, cvn_stream_t stream) {
  if (n < 0 || (n > 0 && (!src || !dst))) return fail(CVN_ERR_ARG, "bad copy arguments");
  if (n == 0) return CVN_OK;
  if (((uintptr_t)src | (uintptr_t)dst) & 15) return fail(CVN_ERR_ARG, "copy needs 16-byte aligned buffers");
  const int64_t n4 = n / 4;
  const int64_t blocks = std::min<int64_t>((n4 + 255) / 256 + 1, 256 * 64);
  hipLaunchKernelGGL(k_copy, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const copy_f32x4*)src, (copy_f32x4*)dst, n4, src, dst, n);
  return check_launch("copy");
}
