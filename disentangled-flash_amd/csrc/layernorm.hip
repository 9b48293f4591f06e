// Fused residual add + LayerNorm for the DeBERTa encoder layer outputs
// (DebertaV2SelfOutput / DebertaV2Output: LayerNorm(dense(x) + input),
// _reference.py:108-112, 482-485).
//
// One wavefront per row.  The sum dense + residual is rounded to the
// activation dtype first, exactly as the separate elementwise add of the
// reference produces it, then normalised in fp32 with a two-pass mean /
// variance over the values held in registers:
//
//   s = T(x + r);  y = T((s - mean(s)) * rsqrt(var(s) + eps) * gamma + beta)
//
// HBM traffic per row: read x and r, write y (3 * H * sizeof(T) bytes), which
// replaces the add's read-read-write plus the LayerNorm's read-write.  Rows
// made of 16-byte chunks with 16-byte aligned pointers take the wide kernel
// (16-byte accesses); others the 4-element one.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dflash.h"

namespace dflash {
namespace {

constexpr int kRowsPerBlock = 4;  // one wavefront per row

template <typename T>
struct Vec4 {
  typedef T type __attribute__((ext_vector_type(4)));
};

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// VPL = number of 4-element chunks per lane (H <= 256 * VPL).
template <typename T, int VPL, bool HAS_R>
__global__ __launch_bounds__(64 * kRowsPerBlock) void add_layernorm_kernel(
    const T* __restrict__ x, const T* __restrict__ r, const T* __restrict__ gamma,
    const T* __restrict__ beta, T* __restrict__ y, int rows, int hidden, float eps) {
  using V = typename Vec4<T>::type;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wavefronts exit together
  const int64_t base = static_cast<int64_t>(row) * hidden;
  const int nvec = hidden >> 2;

  float s[VPL][4];
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (v < nvec) {
      const V a = *reinterpret_cast<const V*>(x + base + 4 * v);
      V b{};
      if constexpr (HAS_R) b = *reinterpret_cast<const V*>(r + base + 4 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s[k][e] = HAS_R ? static_cast<float>(static_cast<T>(static_cast<float>(a[e]) +
                                                            static_cast<float>(b[e])))
                        : static_cast<float>(a[e]);
        sum += s[k][e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) s[k][e] = 0.0f;
    }
  }
  const float inv_h = 1.0f / static_cast<float>(hidden);
  const float mean = wave_sum(sum) * inv_h;
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    if (lane + 64 * k < nvec) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = s[k][e] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = rsqrtf(wave_sum(sq) * inv_h + eps);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (v < nvec) {
      const V g = *reinterpret_cast<const V*>(gamma + 4 * v);
      const V bb = *reinterpret_cast<const V*>(beta + 4 * v);
      V out;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        out[e] = static_cast<T>((s[k][e] - mean) * rstd * static_cast<float>(g[e]) +
                                static_cast<float>(bb[e]));
      *reinterpret_cast<V*>(y + base + 4 * v) = out;
    }
  }
}

// Wide variant: 16-byte loads, LANES lanes per row (32 or 64, so 8 or 4 rows
// per 256-thread block), CH 16-byte chunks per lane.  Used when a row is a
// whole number of 16-byte chunks and every pointer is 16-byte aligned; with
// 32 lanes per row the reductions stay inside a half-wavefront.
template <typename T>
struct Vec16 {
  static constexpr int N = 16 / sizeof(T);
  typedef T type __attribute__((ext_vector_type(16 / sizeof(T))));
};

template <int LANES>
__device__ inline float group_sum(float v) {
#pragma unroll
  for (int m = LANES / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

template <typename T, int LANES, int CH, bool HAS_R>
__global__ __launch_bounds__(256) void add_layernorm_wide_kernel(
    const T* __restrict__ x, const T* __restrict__ r, const T* __restrict__ gamma,
    const T* __restrict__ beta, T* __restrict__ y, int rows, int hidden, float eps) {
  using V = typename Vec16<T>::type;
  constexpr int N = Vec16<T>::N;
  const int sub = threadIdx.x % LANES;
  const int row = blockIdx.x * (256 / LANES) + threadIdx.x / LANES;
  if (row >= rows) return;  // whole lane groups exit together
  const int64_t base = static_cast<int64_t>(row) * hidden;
  const int nvec = hidden / N;

  V a[CH];
  V b[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int v = sub + LANES * k;
    if (v < nvec) {
      a[k] = *reinterpret_cast<const V*>(x + base + N * v);
      if constexpr (HAS_R) b[k] = *reinterpret_cast<const V*>(r + base + N * v);
    }
  }
  float s[CH][N];
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const bool live = sub + LANES * k < nvec;
#pragma unroll
    for (int e = 0; e < N; ++e) {
      if constexpr (HAS_R) {
        s[k][e] = live ? static_cast<float>(static_cast<T>(static_cast<float>(a[k][e]) +
                                                           static_cast<float>(b[k][e])))
                       : 0.0f;
      } else {
        s[k][e] = live ? static_cast<float>(a[k][e]) : 0.0f;
      }
      sum += s[k][e];
    }
  }
  const float inv_h = 1.0f / static_cast<float>(hidden);
  const float mean = group_sum<LANES>(sum) * inv_h;
  float sq = 0.0f;
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    if (sub + LANES * k < nvec) {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float d = s[k][e] - mean;
        sq += d * d;
      }
    }
  }
  const float rstd = rsqrtf(group_sum<LANES>(sq) * inv_h + eps);
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int v = sub + LANES * k;
    if (v < nvec) {
      const V g = *reinterpret_cast<const V*>(gamma + N * v);
      const V bb = *reinterpret_cast<const V*>(beta + N * v);
      V out;
#pragma unroll
      for (int e = 0; e < N; ++e)
        out[e] = static_cast<T>((s[k][e] - mean) * rstd * static_cast<float>(g[e]) +
                                static_cast<float>(bb[e]));
      *reinterpret_cast<V*>(y + base + N * v) = out;
    }
  }
}

template <typename T, int LANES, int CH>
int launch_ln_wide(const void* x, const void* r, const void* gamma, const void* beta, void* y,
                   int rows, int hidden, float eps, hipStream_t stream) {
  constexpr int kRows = 256 / LANES;
  const int blocks = (rows + kRows - 1) / kRows;
  if (r != nullptr)
    hipLaunchKernelGGL((add_layernorm_wide_kernel<T, LANES, CH, true>), dim3(blocks), dim3(256),
                       0, stream, static_cast<const T*>(x), static_cast<const T*>(r),
                       static_cast<const T*>(gamma), static_cast<const T*>(beta),
                       static_cast<T*>(y), rows, hidden, eps);
  else
    hipLaunchKernelGGL((add_layernorm_wide_kernel<T, LANES, CH, false>), dim3(blocks), dim3(256),
                       0, stream, static_cast<const T*>(x), static_cast<const T*>(r),
                       static_cast<const T*>(gamma), static_cast<const T*>(beta),
                       static_cast<T*>(y), rows, hidden, eps);
  return static_cast<int>(hipGetLastError());
}

// Rows of up to 32 * 4 chunks use 32 lanes, longer rows 64 (<= 64 * 8 chunks,
// i.e. hidden <= 4096 for 16-bit types and <= 2048 for fp32).  Returns
// kWideUnfit when the shape does not fit the wide kernel.
constexpr int kWideUnfit = -1000;

template <typename T>
int dispatch_ln_wide(const void* x, const void* r, const void* gamma, const void* beta, void* y,
                     int rows, int hidden, float eps, hipStream_t stream) {
  constexpr int N = Vec16<T>::N;
  if (hidden % N != 0) return kWideUnfit;
  const int nvec = hidden / N;
  if (nvec <= 32) return launch_ln_wide<T, 32, 1>(x, r, gamma, beta, y, rows, hidden, eps, stream);
  if (nvec <= 64) return launch_ln_wide<T, 32, 2>(x, r, gamma, beta, y, rows, hidden, eps, stream);
  if (nvec <= 96) return launch_ln_wide<T, 32, 3>(x, r, gamma, beta, y, rows, hidden, eps, stream);
  if (nvec <= 128) return launch_ln_wide<T, 32, 4>(x, r, gamma, beta, y, rows, hidden, eps, stream);
  if (nvec <= 192) return launch_ln_wide<T, 64, 3>(x, r, gamma, beta, y, rows, hidden, eps, stream);
  if (nvec <= 256) return launch_ln_wide<T, 64, 4>(x, r, gamma, beta, y, rows, hidden, eps, stream);
  if (nvec <= 512) return launch_ln_wide<T, 64, 8>(x, r, gamma, beta, y, rows, hidden, eps, stream);
  return kWideUnfit;
}

template <typename T, int VPL>
int launch_ln(const void* x, const void* r, const void* gamma, const void* beta, void* y,
              int rows, int hidden, float eps, hipStream_t stream) {
  const int blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (r != nullptr)
    hipLaunchKernelGGL((add_layernorm_kernel<T, VPL, true>), dim3(blocks), dim3(64 * kRowsPerBlock),
                       0, stream, static_cast<const T*>(x), static_cast<const T*>(r),
                       static_cast<const T*>(gamma), static_cast<const T*>(beta),
                       static_cast<T*>(y), rows, hidden, eps);
  else
    hipLaunchKernelGGL((add_layernorm_kernel<T, VPL, false>), dim3(blocks),
                       dim3(64 * kRowsPerBlock), 0, stream, static_cast<const T*>(x),
                       static_cast<const T*>(r), static_cast<const T*>(gamma),
                       static_cast<const T*>(beta), static_cast<T*>(y), rows, hidden, eps);
  return static_cast<int>(hipGetLastError());
}

template <typename T>
int dispatch_ln(const void* x, const void* r, const void* gamma, const void* beta, void* y,
                int rows, int hidden, float eps, hipStream_t stream) {
  const int vpl = (hidden + 255) / 256;
  switch (vpl) {
    case 1: return launch_ln<T, 1>(x, r, gamma, beta, y, rows, hidden, eps, stream);
    case 2: return launch_ln<T, 2>(x, r, gamma, beta, y, rows, hidden, eps, stream);
    case 3: return launch_ln<T, 3>(x, r, gamma, beta, y, rows, hidden, eps, stream);
    case 4: return launch_ln<T, 4>(x, r, gamma, beta, y, rows, hidden, eps, stream);
    case 5:
    case 6: return launch_ln<T, 6>(x, r, gamma, beta, y, rows, hidden, eps, stream);
    case 7:
    case 8: return launch_ln<T, 8>(x, r, gamma, beta, y, rows, hidden, eps, stream);
    default: return launch_ln<T, 16>(x, r, gamma, beta, y, rows, hidden, eps, stream);
  }
}

}  // namespace
}  // namespace dflash

using namespace dflash;

extern "C" int dflash_add_layernorm_fwd(const void* x, const void* residual, const void* gamma,
                                        const void* beta, void* out, int rows, int hidden,
                                        float eps, int dtype, void* stream) {
  if (rows < 0 || hidden < 4 || hidden % 4 != 0 || hidden > 4096) return DFLASH_ERR_SHAPE;
  if (rows == 0) return DFLASH_OK;  // nothing to do; empty tensors may carry null pointers
  if (!x || !gamma || !beta || !out) return DFLASH_ERR_NULL;  // residual NULL: LayerNorm(x)
  const int esize = dtype == DFLASH_DTYPE_FP32 ? 4 : 2;
  const uintptr_t addr_or = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(residual) |
                            reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta) |
                            reinterpret_cast<uintptr_t>(out);
  if (addr_or % (4 * esize) != 0) return DFLASH_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (addr_or % 16 == 0) {
    int rc = kWideUnfit;
    switch (dtype) {
      case DFLASH_DTYPE_FP16: rc = dispatch_ln_wide<_Float16>(x, residual, gamma, beta, out, rows, hidden, eps, s); break;
      case DFLASH_DTYPE_BF16: rc = dispatch_ln_wide<__bf16>(x, residual, gamma, beta, out, rows, hidden, eps, s); break;
      case DFLASH_DTYPE_FP32: rc = dispatch_ln_wide<float>(x, residual, gamma, beta, out, rows, hidden, eps, s); break;
      default: return DFLASH_ERR_DTYPE;
    }
    if (rc != kWideUnfit) return rc;
  }
  switch (dtype) {
    case DFLASH_DTYPE_FP16: return dispatch_ln<_Float16>(x, residual, gamma, beta, out, rows, hidden, eps, s);
    case DFLASH_DTYPE_BF16: return dispatch_ln<__bf16>(x, residual, gamma, beta, out, rows, hidden, eps, s);
    case DFLASH_DTYPE_FP32: return dispatch_ln<float>(x, residual, gamma, beta, out, rows, hidden, eps, s);
    default: return DFLASH_ERR_DTYPE;
  }
}
