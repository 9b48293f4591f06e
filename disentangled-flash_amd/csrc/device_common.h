// Device helpers shared by the attention kernels of libdflash (gfx950).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <stdint.h>

namespace dflash {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;               // wavefronts per workgroup
constexpr int kThreads = kWaves * 64;

// ---------------------------------------------------------------------------
// MFMA wrappers.  A operand: lane l holds row l%16, k-slice l/16.  B operand:
// lane l holds column l%16, the same k-slice.  C/D: lane l holds column l%16,
// rows 4*(l/16) + r for r in 0..3.  The order of k inside a slice is the same
// for A and B, so the products pair up whatever the hardware order is.
// ---------------------------------------------------------------------------
template <typename T>
struct Mma;

template <>
struct Mma<_Float16> {
  using frag = half8_t;
  static constexpr int K = 32;     // k per instruction
  static constexpr int PER = 8;    // elements of one lane's k-slice
  __device__ static f32x4_t run(frag a, frag b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mma<__bf16> {
  using frag = bf16x8_t;
  static constexpr int K = 32;
  static constexpr int PER = 8;
  __device__ static f32x4_t run(frag a, frag b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mma<float> {
  using frag = float;
  static constexpr int K = 4;
  static constexpr int PER = 1;
  __device__ static f32x4_t run(frag a, frag b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));


// Workgroup barrier that orders LDS traffic only.  __syncthreads() also waits
// for every outstanding global load (vmcnt(0)), which would force the
// next-tile prefetch to land at the first barrier; here global loads stay in
// flight and are waited for where their registers are used.
__device__ inline void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Physical workgroup n runs on XCD n % 8.  Renumber so that the query blocks
// of one (b, h) - which share K, V and the relative tables - land on the same
// XCD and hit the same L2.
__device__ inline int xcd_logical_block(int n, int total) {
  constexpr int kXcds = 8;
  int per = total / kXcds;
  int rem = total % kXcds;
  int xcd = n % kXcds;
  int idx = n / kXcds;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// Four consecutive elements of T: one 8-byte (16-bit T) or 16-byte (fp32) access.
template <typename T>
using Quad = T __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));


// Host: raise a kernel's dynamic LDS limit once per device (the attribute
// persists), instead of on every launch.
template <auto Kernel>
inline hipError_t ensure_dynamic_lds(int bytes) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  const uint64_t bit = dev < 64 ? (uint64_t{1} << dev) : 0;
  if (bit != 0 && (done.load(std::memory_order_acquire) & bit) != 0) return hipSuccess;
  err = hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (err == hipSuccess && bit != 0) done.fetch_or(bit, std::memory_order_release);
  return err;
}

}  // namespace dflash
