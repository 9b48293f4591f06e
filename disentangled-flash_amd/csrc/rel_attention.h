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
  // Key splits (1 = none).  With splits > 1 each workgroup walks split_tiles
  // key tiles and writes unnormalised partial rows to part (fp32 [splits, B,
  // L, H, D], then {base, sum} pairs [splits, B, L, H]); a merge kernel
  // combines them.
  int splits;
  int split_tiles;
  float* part;
  // Query rows per wavefront of the unsplit form: 32 (default) or 16
  // (rel_attention_qw); fp32 at d = 128 always runs 16.
  int qw;
  // fp32 only: 1 = products on the bf16 matrix unit in three parts
  // (fp32_precision="fast"), 0 = IEEE fp32 MFMA.
  int fast;
  // 1 = pos_key / pos_query are the precomputed c2p / p2c tables [B, H, L, S]
  // (the reference op's contract) instead of the relative rows [H, S, D].
  // Unsplit, QW = 32 (d <= 64) or 16 (d = 128), IEEE fp32.
  int table;
  // First group of the launch, groups numbered h * B + b (the table form's
  // last slice, b = B - 1 and h = H - 1, may run as a launch of its own); 0
  // otherwise.
  int bh0;
};

// fp16 / bf16 / fp32, D in {32, 64, 128}; arguments already validated by the
// caller.  prm.splits / split_tiles / part select the split-key form (with its
// merge; 16-bit types only).
int launch_rel_attention(const RelParams& prm, int D, int dtype, hipStream_t stream);

// Key splits for a launch of B*H query-block rows that would leave the GPU
// underfilled (fewer workgroups than two per CU), and the workspace bytes they
// need; 1 and 0 when no split pays.
int rel_attention_splits(int B, int H, int L, int D, int cus, int* split_tiles);
size_t rel_attention_workspace_bytes(int splits, int B, int H, int L, int D);

// Query rows per wavefront for an unsplit launch (32 or 16) on a device with
// `cus` CUs, from the measured per-shape table in rel_attention.hip.
// `has_c2p`: the c2p term is computed (the 32-row d = 128 tile pays only then).
int rel_attention_qw(int B, int H, int L, int D, int cus, bool has_c2p);

}  // namespace dflash
