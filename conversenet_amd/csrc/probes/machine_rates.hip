// Machine-rate probes for the kernels' design (not part of libcvn_hip.so): fp32 VALU issue rate
// against the number of waves per SIMD, whether fp32 MFMA and VALU work overlap, and the LDS
// throughput and bank structure for 32- and 64-bit accesses.  Every loop is bounded; nothing is read
// out of bounds (LDS indices wrap inside the 64 KB the launch allocates).
//
// Build and run (one MI355X):
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         -o machine_rates conversenet_amd/csrc/probes/machine_rates.hip && ./machine_rates
#include <hip/hip_runtime.h>

#include <cstdio>

typedef float v4f __attribute__((ext_vector_type(4)));

// CH independent FMA chains per lane, 128 FMAs per iteration; the dynamic LDS allocation of the
// launch limits residency to one block per CU, so blockDim / 256 waves share each SIMD.
template <int CH>
__global__ void k_valu(float* out, int iters, float s) {
  extern __shared__ float pad_lds[];
  float a[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) a[i] = s * (threadIdx.x + i);
  const float x = s * threadIdx.x, y = s + threadIdx.x;
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int r = 0; r < 128 / CH; ++r)
#pragma unroll
      for (int i = 0; i < CH; ++i) a[i] = __builtin_fmaf(a[i], x, y);
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) t += a[i];
  if (t == 12345.f) pad_lds[threadIdx.x] = t;
  out[blockIdx.x * blockDim.x + threadIdx.x] = t;
}

// MODE 0: 128 FMAs per iteration; 1: four 16x16x4 fp32 MFMAs (independent accumulators);
// 2: both in every wave; 3: even waves FMAs, odd waves MFMAs.
template <int MODE>
__global__ void __launch_bounds__(1024) k_mix(float* out, int iters, float s) {
  const int tid = threadIdx.x, wave = tid >> 6;
  float a[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = s * (tid + i);
  v4f acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = (v4f){0.f, 0.f, 0.f, 0.f};
  const float x = s * tid, y = s + tid;
  const bool do_valu = MODE == 0 || MODE == 2 || (MODE == 3 && (wave & 1) == 0);
  const bool do_mfma = MODE == 1 || MODE == 2 || (MODE == 3 && (wave & 1) == 1);
  for (int it = 0; it < iters; ++it) {
    if (do_mfma) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, acc[i], 0, 0, 0);
    }
    if (do_valu) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int i = 0; i < 16; ++i) a[i] = __builtin_fmaf(a[i], x, y);
    }
  }
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) t += a[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) t += acc[i].x + acc[i].y + acc[i].z + acc[i].w;
  out[blockIdx.x * 1024 + tid] = t;
}

// LDS: lane address = base + lane * stride (in W-byte words), wrapped into 64 KB
template <int W, bool WR>
__global__ void k_lds(float* out, int iters, int stride) {
  extern __shared__ __align__(16) float2 L2[];
  float* L = (float*)L2;
  float4* L4 = (float4*)L2;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < 16384; i += blockDim.x) L[i] = i;
  __syncthreads();
  float acc = 0.f;
  const int base = wave * 37;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int idx = (base + lane * stride + r * 1024) % (65536 / W);
      if constexpr (WR) {
        if constexpr (W == 16) L4[idx] = make_float4(acc, acc, acc, acc);
        else if constexpr (W == 8) L2[idx] = make_float2(acc, acc);
        else L[idx] = acc;
        acc += 1.f;
      } else {
        if constexpr (W == 16) {
          const float4 v = L4[idx];
          acc += v.x * v.y + v.z * v.w;
        } else if constexpr (W == 8) {
          const float2 v = L2[idx];
          acc += v.x * v.y;
        } else {
          acc += L[idx];
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  }
  __syncthreads();
  out[blockIdx.x * blockDim.x + tid] = acc + L[tid];
}

int main() {
  float* out;
  if (hipMalloc(&out, 4096 * 1024 * sizeof(float)) != hipSuccess) return 1;
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  auto timeit = [&](auto launch) {
    launch();
    (void)hipEventRecord(e0);
    launch();
    (void)hipEventRecord(e1);
    (void)hipEventSynchronize(e1);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    return ms;
  };
  (void)hipFuncSetAttribute((const void*)k_valu<16>, hipFuncAttributeMaxDynamicSharedMemorySize, 100 * 1024);
  const int iters = 2000;
  printf("fp32 VALU FMA issue (16 independent chains per lane, one block per CU):\n");
  for (int wps : {1, 2, 4}) {
    const float ms = timeit([&] {
      hipLaunchKernelGGL(k_valu<16>, dim3(256 * 4), dim3(256 * wps), 100 * 1024, 0, out, iters, 1e-3f);
    });
    printf("  %d waves per SIMD: %.3f ns per wave instruction per SIMD\n", wps,
           ms * 1e6 / (4.0 * wps * iters * 128));
  }
  printf("fp32 MFMA 16x16x4 and VALU FMA (1024 blocks of 1024 threads, 4000 iterations):\n");
  const char* names[4] = {"VALU only", "MFMA only", "both in every wave", "split across waves"};
  for (int m = 0; m < 4; ++m) {
    const float ms = timeit([&] {
      switch (m) {
        case 0: hipLaunchKernelGGL(k_mix<0>, dim3(1024), dim3(1024), 0, 0, out, 4000, 1e-3f); break;
        case 1: hipLaunchKernelGGL(k_mix<1>, dim3(1024), dim3(1024), 0, 0, out, 4000, 1e-3f); break;
        case 2: hipLaunchKernelGGL(k_mix<2>, dim3(1024), dim3(1024), 0, 0, out, 4000, 1e-3f); break;
        default: hipLaunchKernelGGL(k_mix<3>, dim3(1024), dim3(1024), 0, 0, out, 4000, 1e-3f); break;
      }
    });
    printf("  %-20s %.3f ms\n", names[m], ms);
  }
  printf("LDS, ns per wave instruction per CU (1024 threads, 4 blocks per CU), lane stride in words:\n");
  printf("  stride  read32  read64  write32  write64  read128  write128\n");
  for (int s : {1, 2, 3, 4, 8, 16, 32, 33, 267}) {
    auto run = [&](auto kern) {
      const float ms = timeit([&] { hipLaunchKernelGGL(kern, dim3(1024), dim3(1024), 65536, 0, out, iters, s); });
      return ms * 1e6 / (4.0 * 16 * iters * 8);
    };
    printf("  %6d  %6.3f  %6.3f  %7.3f  %7.3f  %7.3f  %8.3f\n", s, run(k_lds<4, false>), run(k_lds<8, false>),
           run(k_lds<4, true>), run(k_lds<8, true>), run(k_lds<16, false>), run(k_lds<16, true>));
  }
  printf("status: %s\n", hipGetErrorString(hipGetLastError()));
  return 0;
}
