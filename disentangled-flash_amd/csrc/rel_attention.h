// Launcher of the 16-bit in-kernel-relative attention kernel (rel_attention.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dflash {

struct RelParams {
  const void* q;
  const void* k;
  const void* v;
  int64_t sb, sh, sl;        // element strides of q/k/v: batch, head, position
  const void* pos_key;       // [H, S, D]
  const void* pos_query;     // [H, S, D]
  const int32_t* lut;        // delta_to_local [2L-1]
  const uint8_t* mask;       // [B, L], nonzero = kept
  void* out;                 // [B, L, H*D]
  int B, H, L, S;
  int nqb;                   // query blocks per (b, h), set by the launcher
  float scale_log2;          // log2(e) / sqrt(d * factor)
  int has_c2p, has_p2c;
};

// fp16 / bf16, D in {32, 64, 128}; arguments already validated by the caller.
int launch_rel_attention_16bit(const RelParams& prm, int D, int dtype, hipStream_t stream);

}  // namespace dflash
