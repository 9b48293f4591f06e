// MFMA throughput probe for the roofline discussion (bench.py --mfma-ceiling).
//
// Every wavefront issues `iters` rounds of eight independent
// v_mfma_f32_16x16x32_f16 (eight accumulators, operands held in registers), so
// the stream has no memory traffic and no dependent-MFMA stalls.  A workgroup
// is 256 threads (one wavefront per SIMD); launching `waves_per_simd` times
// the CU count of workgroups puts that many wavefronts on every SIMD.  The
// measured rate is the practical ceiling a kernel at that occupancy can reach
// with fp16 MFMA, against the 2.5 PFLOP/s dense spec figure.
#include <hip/hip_runtime.h>

typedef _Float16 probe_h8 __attribute__((ext_vector_type(8)));
typedef float probe_f4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void mfma_probe_kernel(const probe_h8* __restrict__ in,
                                                         float* __restrict__ out, int iters) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  const probe_h8 a0 = in[(4 * t) & 4095];
  const probe_h8 a1 = in[(4 * t + 1) & 4095];
  const probe_h8 b0 = in[(4 * t + 2) & 4095];
  const probe_h8 b1 = in[(4 * t + 3) & 4095];
  probe_f4 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = probe_f4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; i += 4) {
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc[i], 0, 0, 0);
      acc[i + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b0, acc[i + 1], 0, 0, 0);
      acc[i + 2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b1, acc[i + 2], 0, 0, 0);
      acc[i + 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc[i + 3], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  out[t] = s;  // keeps the products live
}

// in: 4096 x 8 fp16 values; out: blocks * 256 floats.  Returns a hipError_t.
extern "C" __attribute__((visibility("default"))) int dflash_probe_mfma(const void* in, void* out,
                                                                       int blocks, int iters,
                                                                       void* stream) {
  if (!in || !out || blocks < 1 || iters < 1) return static_cast<int>(hipErrorInvalidValue);
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const probe_h8*>(in),
                     static_cast<float*>(out), iters);
  return static_cast<int>(hipGetLastError());
}
