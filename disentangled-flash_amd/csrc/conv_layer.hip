// Tail of the DeBERTa-v2 ConvLayer after the first encoder layer
// (ConvLayer.forward, _reference.py:536-566; called by the encoder loop at
// deberta.py:272-273), fused into one pass per row.
//
// The convolution itself (Conv1d, kernel 3, padding 1, one group) runs as a
// single library GEMM before this kernel: z = x . [W_0; W_1; W_2]^T over the
// [B*L, hidden] input rows, so z[row] holds the three taps' products
// z_k[row] = W_k . x[row] side by side.  Output row (b, l) of the
// convolution is then z_0[l-1] + z_1[l] + z_2[l+1] + bias, with the taps that
// fall outside the sequence dropped (zero padding).  Per element this kernel
// reproduces the rounding steps of the module in the activation dtype T:
//
//   c = T(conv)                    (the convolution output tensor)
//   c = 0 where the mask removes the position  (bool: !m; numeric: m != 1)
//   a = T(act(c))                  (gelu = exact erf form, tanh or relu)
//   s = T(residual + a)
//   y = T(LayerNorm(s)) with fp32 statistics
//   out = T(y * T(m))
//
// HBM traffic per row: the three z slices it reads (3 * hidden * sizeof(Z)),
// the residual and the output; z rows are each read once over the launch.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dflash.h"

namespace dflash {
namespace {

constexpr int kConvRowsPerBlock = 4;  // one wavefront per row

__device__ inline float conv_wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

template <typename T>
struct Four {
  typedef T type __attribute__((ext_vector_type(4)));
};

__device__ inline float apply_act(float x, int act) {
  switch (act) {
    case DFLASH_ACT_GELU: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    case DFLASH_ACT_TANH: return tanhf(x);
    default: return fmaxf(x, 0.0f);  // DFLASH_ACT_RELU
  }
}

// VPL = 4-element chunks per lane (hidden <= 256 * VPL).
template <typename T, typename Z, int VPL>
__global__ __launch_bounds__(64 * kConvRowsPerBlock) void conv_tail_kernel(
    const Z* __restrict__ z, const T* __restrict__ residual, const T* __restrict__ bias,
    const T* __restrict__ gamma, const T* __restrict__ beta, const int64_t* __restrict__ mask,
    T* __restrict__ y, int rows, int length, int hidden, float eps, int act) {
  using TV = typename Four<T>::type;
  using ZV = typename Four<Z>::type;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kConvRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wavefronts exit together
  const int l = row % length;
  const int nvec = hidden >> 2;
  const int64_t zs = 3 * static_cast<int64_t>(hidden);
  const Z* zc = z + row * zs + hidden;  // centre tap of this row
  const int64_t m = mask[row];
  const bool keep = m == 1;
  const float mscale = static_cast<float>(static_cast<T>(static_cast<float>(m)));

  float s[VPL][4];
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (v < nvec) {
      const TV bv = *reinterpret_cast<const TV*>(bias + 4 * v);
      const TV rv = *reinterpret_cast<const TV*>(residual + row * static_cast<int64_t>(hidden) + 4 * v);
      const ZV c1 = *reinterpret_cast<const ZV*>(zc + 4 * v);
      ZV c0 = ZV{0, 0, 0, 0};
      ZV c2 = ZV{0, 0, 0, 0};
      if (l > 0) c0 = *reinterpret_cast<const ZV*>(zc - zs - hidden + 4 * v);
      if (l + 1 < length) c2 = *reinterpret_cast<const ZV*>(zc + zs + hidden + 4 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float conv = static_cast<float>(c0[e]) + static_cast<float>(c1[e]) +
                           static_cast<float>(c2[e]) + static_cast<float>(bv[e]);
        const float c = keep ? static_cast<float>(static_cast<T>(conv)) : 0.0f;
        const float a = static_cast<float>(static_cast<T>(apply_act(c, act)));
        s[k][e] = static_cast<float>(static_cast<T>(static_cast<float>(rv[e]) + a));
        sum += s[k][e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) s[k][e] = 0.0f;
    }
  }
  const float inv_h = 1.0f / static_cast<float>(hidden);
  const float mean = conv_wave_sum(sum) * inv_h;
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
  const float rstd = rsqrtf(conv_wave_sum(sq) * inv_h + eps);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + 64 * k;
    if (v < nvec) {
      const TV g = *reinterpret_cast<const TV*>(gamma + 4 * v);
      const TV bb = *reinterpret_cast<const TV*>(beta + 4 * v);
      TV out;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const T normed = static_cast<T>((s[k][e] - mean) * rstd * static_cast<float>(g[e]) +
                                        static_cast<float>(bb[e]));
        out[e] = static_cast<T>(static_cast<float>(normed) * mscale);
      }
      *reinterpret_cast<TV*>(y + row * static_cast<int64_t>(hidden) + 4 * v) = out;
    }
  }
}

template <typename T, typename Z, int VPL>
int launch_conv_tail(const void* z, const void* residual, const void* bias, const void* gamma,
                     const void* beta, const int64_t* mask, void* out, int rows, int length,
                     int hidden, float eps, int act, hipStream_t stream) {
  const int blocks = (rows + kConvRowsPerBlock - 1) / kConvRowsPerBlock;
  hipLaunchKernelGGL((conv_tail_kernel<T, Z, VPL>), dim3(blocks), dim3(64 * kConvRowsPerBlock), 0,
                     stream, static_cast<const Z*>(z), static_cast<const T*>(residual),
                     static_cast<const T*>(bias), static_cast<const T*>(gamma),
                     static_cast<const T*>(beta), mask, static_cast<T*>(out), rows, length, hidden,
                     eps, act);
  return static_cast<int>(hipGetLastError());
}

template <typename T, typename Z>
int dispatch_conv_tail(const void* z, const void* residual, const void* bias, const void* gamma,
                       const void* beta, const int64_t* mask, void* out, int rows, int length,
                       int hidden, float eps, int act, hipStream_t stream) {
#define DFLASH_CONV_CASE(V)                                                                    \
  case V:                                                                                      \
    return launch_conv_tail<T, Z, V>(z, residual, bias, gamma, beta, mask, out, rows, length, \
                                     hidden, eps, act, stream);
  switch ((hidden + 255) / 256) {
    DFLASH_CONV_CASE(1)
    DFLASH_CONV_CASE(2)
    DFLASH_CONV_CASE(3)
    DFLASH_CONV_CASE(4)
    case 5:
    DFLASH_CONV_CASE(6)
    case 7:
    DFLASH_CONV_CASE(8)
    default:
      return launch_conv_tail<T, Z, 16>(z, residual, bias, gamma, beta, mask, out, rows, length,
                                        hidden, eps, act, stream);
  }
#undef DFLASH_CONV_CASE
}

}  // namespace
}  // namespace dflash

using namespace dflash;

extern "C" int dflash_conv_layer_tail_fwd(const void* z, int z_dtype, const void* residual,
                                          const void* conv_bias, const void* gamma,
                                          const void* beta, const int64_t* mask, void* out,
                                          int B, int L, int hidden, float eps, int act, int dtype,
                                          void* stream) {
  if (B < 0 || L < 0 || hidden < 4 || hidden % 4 != 0 || hidden > 4096) return DFLASH_ERR_SHAPE;
  if (act != DFLASH_ACT_GELU && act != DFLASH_ACT_TANH && act != DFLASH_ACT_RELU)
    return DFLASH_ERR_SHAPE;
  const int64_t rows = static_cast<int64_t>(B) * L;
  if (rows > 0x7fffffff / 4) return DFLASH_ERR_TOO_LARGE;
  if (rows == 0) return DFLASH_OK;  // nothing to do; empty tensors may carry null pointers
  if (!z || !residual || !conv_bias || !gamma || !beta || !mask || !out) return DFLASH_ERR_NULL;
  const int esize = dtype == DFLASH_DTYPE_FP32 ? 4 : 2;
  const int zsize = z_dtype == DFLASH_DTYPE_FP32 ? 4 : 2;
  if (z_dtype != DFLASH_DTYPE_FP32 && z_dtype != dtype) return DFLASH_ERR_DTYPE;
  const uintptr_t t_or = reinterpret_cast<uintptr_t>(residual) |
                         reinterpret_cast<uintptr_t>(conv_bias) | reinterpret_cast<uintptr_t>(gamma) |
                         reinterpret_cast<uintptr_t>(beta) | reinterpret_cast<uintptr_t>(out);
  if (t_or % (4 * esize) != 0 || reinterpret_cast<uintptr_t>(z) % (4 * zsize) != 0 ||
      reinterpret_cast<uintptr_t>(mask) % 8 != 0)
    return DFLASH_ERR_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int r = static_cast<int>(rows);
  switch (dtype) {
    case DFLASH_DTYPE_FP16:
      return z_dtype == DFLASH_DTYPE_FP32
                 ? dispatch_conv_tail<_Float16, float>(z, residual, conv_bias, gamma, beta, mask, out, r, L, hidden, eps, act, s)
                 : dispatch_conv_tail<_Float16, _Float16>(z, residual, conv_bias, gamma, beta, mask, out, r, L, hidden, eps, act, s);
    case DFLASH_DTYPE_BF16:
      return z_dtype == DFLASH_DTYPE_FP32
                 ? dispatch_conv_tail<__bf16, float>(z, residual, conv_bias, gamma, beta, mask, out, r, L, hidden, eps, act, s)
                 : dispatch_conv_tail<__bf16, __bf16>(z, residual, conv_bias, gamma, beta, mask, out, r, L, hidden, eps, act, s);
    case DFLASH_DTYPE_FP32:
      return dispatch_conv_tail<float, float>(z, residual, conv_bias, gamma, beta, mask, out, r, L, hidden, eps, act, s);
    default:
      return DFLASH_ERR_DTYPE;
  }
}
