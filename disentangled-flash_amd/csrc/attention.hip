// C-ABI entry points of the fused DeBERTa-v2/v3 disentangled attention
// (include/dflash.h).  All of them run the per-delta relative-window kernel of
// rel_attention.hip:
//   * dflash_attention_fwd - the reference op's contract (kernel.py:368-438):
//     head-major Q/K/V [B, H, L, D] and precomputed c2p / p2c tables
//     [B, H, L, S]; the kernel's relative windows are read from the tables
//     (its table form) instead of computed;
//   * dflash_attention_rel_fwd (and the split and allocation-free variants) -
//     Q/K/V read with strides from the fused projection output, the relative
//     windows computed on the matrix unit from the rows [H, S, D].
//
// Mask semantics follow kernel.py:250-261 (Hugging Face padded-row behaviour):
//   kept query & kept key           -> score
//   padded query (in range)         -> 0 for every in-range key (uniform row)
//   kept query & padded key         -> -inf
//   query past L                    -> 0 at key 0 only (row never stored)

#include <hip/hip_runtime.h>
#include <atomic>
#include <mutex>
#include <stdint.h>

#include "dflash.h"

#include "device_common.h"
#include "rel_attention.h"

namespace dflash {

// Returned by check_common for an empty batch: the entry points report success
// without launching (the reference's launch over an empty grid is a no-op too).
constexpr int kEmptyBatch = 1;

int check_common(const void* q, const void* k, const void* v, const int32_t* lut,
                 const uint8_t* mask, const void* out, int B, int H, int L, int D, int S,
                 int has_c2p, int has_p2c, int dtype) {
  if (B < 0 || H < 1 || L < 1) return DFLASH_ERR_SHAPE;
  if (B == 0) return kEmptyBatch;  // nothing to launch; empty tensors may carry null pointers
  if (!q || !k || !v || !mask || !out) return DFLASH_ERR_NULL;
  if (D != 32 && D != 64 && D != 128) return DFLASH_ERR_HEAD_DIM;
  if (dtype < DFLASH_DTYPE_FP16 || dtype > DFLASH_DTYPE_FP32) return DFLASH_ERR_DTYPE;
  if (static_cast<int64_t>(L) * D >= (int64_t{1} << 31) ||
      static_cast<int64_t>(S) * D >= (int64_t{1} << 31))
    return DFLASH_ERR_TOO_LARGE;
  if (has_c2p || has_p2c) {
    if (!lut) return DFLASH_ERR_NULL;
    if (S < 1) return DFLASH_ERR_SHAPE;
  }
  return DFLASH_OK;
}

}  // namespace dflash

using namespace dflash;

extern "C" {

int dflash_attention_fwd(const void* query, const void* key, const void* value, const void* c2p,
                         const void* p2c, const int32_t* delta_to_local,
                         const uint8_t* attention_mask, void* out, int B, int H, int L, int D,
                         int S, float score_scale_log2, int has_c2p, int has_p2c, int dtype,
                         int strict_fp32, void* stream) {
  int rc = check_common(query, key, value, delta_to_local, attention_mask, out, B, H, L, D, S,
                        has_c2p, has_p2c, dtype);
  if (rc == kEmptyBatch) return DFLASH_OK;
  if (rc != DFLASH_OK) return rc;
  if ((has_c2p && !c2p) || (has_p2c && !p2c)) return DFLASH_ERR_NULL;
  const int esize = dtype == DFLASH_DTYPE_FP32 ? 4 : 2;
  // One (b, h) slice of a table is addressed through 32-bit byte offsets of a
  // buffer resource.
  if ((has_c2p || has_p2c) && static_cast<int64_t>(L) * S * esize >= (int64_t{1} << 31))
    return DFLASH_ERR_TOO_LARGE;
  const uintptr_t addr_or = reinterpret_cast<uintptr_t>(query) |
                            reinterpret_cast<uintptr_t>(key) |
                            reinterpret_cast<uintptr_t>(value) | reinterpret_cast<uintptr_t>(out);
  if (addr_or % 16 != 0) return DFLASH_ERR_ALIGN;
  const uintptr_t tab_or = reinterpret_cast<uintptr_t>(has_c2p ? c2p : nullptr) |
                           reinterpret_cast<uintptr_t>(has_p2c ? p2c : nullptr);
  if (tab_or % esize != 0) return DFLASH_ERR_ALIGN;
  // The per-delta relative-window kernel in its table form (rel_attention.hip):
  // the windows are read from the tables instead of computed.
  RelParams rp{};
  rp.q = query;
  rp.k = key;
  rp.v = value;
  rp.sb = static_cast<int64_t>(H) * L * D;  // head-major [B, H, L, D]
  rp.sh = static_cast<int64_t>(L) * D;
  rp.sl = D;
  rp.pos_key = has_c2p ? c2p : query;
  rp.pos_query = has_p2c ? p2c : key;
  rp.lut = delta_to_local;
  rp.mask = attention_mask;
  rp.out = out;
  rp.B = B;
  rp.H = H;
  rp.L = L;
  rp.S = (has_c2p || has_p2c) ? S : 1;
  rp.scale_log2 = score_scale_log2;
  rp.has_c2p = has_c2p;
  rp.has_p2c = has_p2c;
  rp.splits = 1;
  // The table form keeps the 16-row tile at d = 128 (two workgroups per CU).
  rp.qw = D >= 128 ? 16 : 32;
  // fp32 with strict_fp32 = 0: QK and PV on the bf16x3 products (the
  // reference's TF32 mode, kernel.py:222); the windows are read, not multiplied.
  rp.fast = (dtype == DFLASH_DTYPE_FP32 && !strict_fp32) ? 1 : 0;
  rp.table = 1;
  return launch_rel_attention(rp, D, dtype, static_cast<hipStream_t>(stream));
}

}  // extern "C"

// ---- static scratch of the allocation-free entry point ----
// The split-key form keeps its partial rows (fp32) in device memory between
// the attention kernel and the merge.  dflash_attention_rel_fwd_noalloc takes
// that memory from this file-scope array instead of from the caller, so it
// calls no allocator.  Every GPU the library runs on holds its own copy for
// the life of the process.  Host code never uses the array's name as an
// address (on the host it is only a stand-in): the device address comes from
// hipGetSymbolAddress, once per device, and is kept per device.
constexpr size_t kScratchBytes = size_t{16} << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// CU count of the current device (cached per device).
int current_device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    const int known = cache[dev].load(std::memory_order_relaxed);
    if (known > 0) return known;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  if (dev < 64) cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Both relative-score entry points; splits <= 1 is the single-pass form.
int rel_forward(const void* query, const void* key, const void* value, int64_t stride_b,
                int64_t stride_h, int64_t stride_l, const void* pos_key, const void* pos_query,
                const int32_t* delta_to_local, const uint8_t* attention_mask, void* out, int B,
                int H, int L, int D, int S, float score_scale_log2, int has_c2p, int has_p2c,
                int dtype, int strict_fp32, int splits, void* workspace, size_t workspace_bytes,
                void* stream) {
  int rc = check_common(query, key, value, delta_to_local, attention_mask, out, B, H, L, D, S,
                        has_c2p, has_p2c, dtype);
  if (rc == kEmptyBatch) return DFLASH_OK;
  if (rc != DFLASH_OK) return rc;
  if ((has_c2p && !pos_key) || (has_p2c && !pos_query)) return DFLASH_ERR_NULL;
  const int esize = dtype == DFLASH_DTYPE_FP32 ? 4 : 2;
  if (stride_l < D || stride_b < 1 || stride_h < 1) return DFLASH_ERR_SHAPE;
  // The kernel addresses one (b, h) slice of Q/K/V and the relative rows through
  // 32-bit byte offsets of buffer resources: both must stay below 2^31 bytes.
  if (static_cast<int64_t>(L) * stride_l * esize >= (int64_t{1} << 31) ||
      static_cast<int64_t>(S) * D * esize >= (int64_t{1} << 31))
    return DFLASH_ERR_TOO_LARGE;
  if (((stride_b | stride_h | stride_l) * esize) % 16 != 0) return DFLASH_ERR_ALIGN;
  const uintptr_t addr_or = reinterpret_cast<uintptr_t>(query) |
                            reinterpret_cast<uintptr_t>(key) |
                            reinterpret_cast<uintptr_t>(value) |
                            reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(pos_key) |
                            reinterpret_cast<uintptr_t>(pos_query);
  if (addr_or % 16 != 0) return DFLASH_ERR_ALIGN;
  // Every dtype runs the per-delta relative-window kernel (rel_attention.hip).
  RelParams rp{};
  rp.q = query;
  rp.k = key;
  rp.v = value;
  rp.sb = stride_b;
  rp.sh = stride_h;
  rp.sl = stride_l;
  rp.pos_key = has_c2p ? pos_key : query;
  rp.pos_query = has_p2c ? pos_query : key;
  rp.lut = delta_to_local;
  rp.mask = attention_mask;
  rp.out = out;
  rp.B = B;
  rp.H = H;
  rp.L = L;
  rp.S = (has_c2p || has_p2c) ? S : 1;
  rp.scale_log2 = score_scale_log2;
  rp.has_c2p = has_c2p;
  rp.has_p2c = has_p2c;
  rp.splits = 1;
  rp.qw = rel_attention_qw(B, H, L, D, current_device_cus(), has_c2p != 0);
  rp.fast = dtype == DFLASH_DTYPE_FP32 && !strict_fp32;
  if (splits > 1 && dtype != DFLASH_DTYPE_FP32) {  // fp32 runs unsplit
    if (splits > 8) return DFLASH_ERR_SHAPE;
    const int tiles = (L + 63) / 64;
    const int st = (tiles + splits - 1) / splits;
    const int eff = (tiles + st - 1) / st;
    if (eff > 1) {
      if (!workspace) return DFLASH_ERR_NULL;
      if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return DFLASH_ERR_ALIGN;
      if (workspace_bytes < rel_attention_workspace_bytes(eff, B, H, L, D))
        return DFLASH_ERR_WORKSPACE;
      rp.splits = eff;
      rp.split_tiles = st;
      rp.part = static_cast<float*>(workspace);
    }
  }
  return launch_rel_attention(rp, D, dtype, static_cast<hipStream_t>(stream));
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (nullptr + error code on failure).
int scratch_address(void** ptr) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return static_cast<int>(err);
  if (dev < 0 || dev >= kMaxDevices) return DFLASH_ERR_SHAPE;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* addr = nullptr;
    err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return static_cast<int>(err);
    if (!addr) return DFLASH_ERR_NULL;
    g_scratch_ptr[dev] = addr;
  }
  *ptr = g_scratch_ptr[dev];
  return DFLASH_OK;
}

// In-flight guard of the scratch, per device: the stream of the last call
// that used it and an event recorded after that call's kernels.  A call from
// another stream while that event is still pending would overwrite partial
// rows the earlier call has not merged yet, so it is refused
// (DFLASH_ERR_BUSY).  Calls on one stream are ordered by the stream and always
// pass.  While a stream is being captured into a HIP graph nothing is
// recorded or queried (a captured launch runs at replay time, which only the
// caller orders).
struct ScratchUse {
  hipEvent_t done = nullptr;
  hipStream_t stream = nullptr;
  bool pending = false;
};
ScratchUse g_scratch_use[kMaxDevices];

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &status) == hipSuccess &&
         status != hipStreamCaptureStatusNone;
}

}  // namespace

extern "C" {

int dflash_attention_rel_fwd(const void* query, const void* key, const void* value,
                             int64_t stride_b, int64_t stride_h, int64_t stride_l,
                             const void* pos_key, const void* pos_query,
                             const int32_t* delta_to_local, const uint8_t* attention_mask,
                             void* out, int B, int H, int L, int D, int S,
                             float score_scale_log2, int has_c2p, int has_p2c, int dtype,
                             int strict_fp32, void* stream) {
  return rel_forward(query, key, value, stride_b, stride_h, stride_l, pos_key, pos_query,
                     delta_to_local, attention_mask, out, B, H, L, D, S, score_scale_log2,
                     has_c2p, has_p2c, dtype, strict_fp32, 1, nullptr, 0, stream);
}

int dflash_attention_rel_split_plan(int B, int H, int L, int D, int* splits,
                                    size_t* workspace_bytes) {
  if (!splits || !workspace_bytes) return DFLASH_ERR_NULL;
  if (B < 0 || H < 1 || L < 1) return DFLASH_ERR_SHAPE;
  if (D != 32 && D != 64 && D != 128) return DFLASH_ERR_HEAD_DIM;
  if (*splits > 8) return DFLASH_ERR_SHAPE;
  if (*splits <= 0) {
    *splits = rel_attention_splits(B, H, L, D, current_device_cus(), nullptr);
  } else {  // the count the split form runs for this request
    const int tiles = (L + 63) / 64;
    const int st = (tiles + *splits - 1) / *splits;
    *splits = (tiles + st - 1) / st;
  }
  *workspace_bytes = rel_attention_workspace_bytes(*splits, B, H, L, D);
  return DFLASH_OK;
}

int dflash_attention_rel_fwd_split(const void* query, const void* key, const void* value,
                                   int64_t stride_b, int64_t stride_h, int64_t stride_l,
                                   const void* pos_key, const void* pos_query,
                                   const int32_t* delta_to_local,
                                   const uint8_t* attention_mask, void* out, int B, int H,
                                   int L, int D, int S, float score_scale_log2, int has_c2p,
                                   int has_p2c, int dtype, int strict_fp32, int splits,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  return rel_forward(query, key, value, stride_b, stride_h, stride_l, pos_key, pos_query,
                     delta_to_local, attention_mask, out, B, H, L, D, S, score_scale_log2,
                     has_c2p, has_p2c, dtype, strict_fp32, splits, workspace, workspace_bytes, stream);
}

int dflash_attention_rel_fwd_noalloc(const void* query, const void* key, const void* value,
                                     int64_t stride_b, int64_t stride_h, int64_t stride_l,
                                     const void* pos_key, const void* pos_query,
                                     const int32_t* delta_to_local,
                                     const uint8_t* attention_mask, void* out, int B, int H,
                                     int L, int D, int S, float score_scale_log2, int has_c2p,
                                     int has_p2c, int dtype, int strict_fp32, int splits,
                                     void* stream) {
  if (splits < 0 || splits > 8) return DFLASH_ERR_SHAPE;
  if (B < 0 || H < 1 || L < 1) return DFLASH_ERR_SHAPE;
  if (B == 0) return DFLASH_OK;
  if (D != 32 && D != 64 && D != 128) return DFLASH_ERR_HEAD_DIM;
  int count = splits;
  if (dtype == DFLASH_DTYPE_FP32) {
    count = 1;  // the fp32 kernel has no split form
  } else if (count == 0) {
    count = rel_attention_splits(B, H, L, D, current_device_cus(), nullptr);
  } else {
    const int tiles = (L + 63) / 64;
    const int st = (tiles + count - 1) / count;
    count = (tiles + st - 1) / st;
  }
  const size_t need = rel_attention_workspace_bytes(count, B, H, L, D);
  if (need > kScratchBytes) return DFLASH_ERR_SCRATCH;
  void* ws = nullptr;
  if (count <= 1) {  // no partial rows: the scratch is not touched
    return rel_forward(query, key, value, stride_b, stride_h, stride_l, pos_key, pos_query,
                       delta_to_local, attention_mask, out, B, H, L, D, S, score_scale_log2,
                       has_c2p, has_p2c, dtype, strict_fp32, 1, nullptr, 0, stream);
  }
  int rc = scratch_address(&ws);
  if (rc != DFLASH_OK) return rc;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return static_cast<int>(err);
  hipStream_t hs = static_cast<hipStream_t>(stream);
  const bool capturing = stream_capturing(hs);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  ScratchUse& use = g_scratch_use[dev];
  if (!capturing && use.pending && use.stream != hs) {
    err = hipEventQuery(use.done);
    if (err == hipErrorNotReady) return DFLASH_ERR_BUSY;
    if (err != hipSuccess) return static_cast<int>(err);
  }
  if (!capturing && !use.done) {  // before launching: a failure here launches nothing
    err = hipEventCreateWithFlags(&use.done, hipEventDisableTiming);
    if (err != hipSuccess) return static_cast<int>(err);
  }
  rc = rel_forward(query, key, value, stride_b, stride_h, stride_l, pos_key, pos_query,
                   delta_to_local, attention_mask, out, B, H, L, D, S, score_scale_log2,
                   has_c2p, has_p2c, dtype, strict_fp32, count, ws, kScratchBytes, stream);
  if (rc != DFLASH_OK || capturing) return rc;
  err = hipEventRecord(use.done, hs);
  if (err != hipSuccess) return static_cast<int>(err);
  use.stream = hs;
  use.pending = true;
  return DFLASH_OK;
}

size_t dflash_attention_rel_noalloc_scratch_bytes(void) { return kScratchBytes; }

const char* dflash_error_string(int code) {
  switch (code) {
    case DFLASH_OK:
      return "success";
    case DFLASH_ERR_NULL:
      return "a required pointer argument is null";
    case DFLASH_ERR_SHAPE:
      return "invalid shape or stride argument";
    case DFLASH_ERR_HEAD_DIM:
      return "head dimension must be 32, 64 or 128";
    case DFLASH_ERR_DTYPE:
      return "dtype must be 0 (fp16), 1 (bf16) or 2 (fp32)";
    case DFLASH_ERR_ALIGN:
      return "tensors and strides must be 16-byte aligned";
    case DFLASH_ERR_TOO_LARGE:
      return "launch grid exceeds the device limit";
    case DFLASH_ERR_WORKSPACE:
      return "workspace smaller than dflash_attention_rel_split_plan reports";
    case DFLASH_ERR_BUSY:
      return "the static scratch is in use by a call on another stream that has not "
             "completed (dflash_attention_rel_fwd_noalloc)";
    case DFLASH_ERR_SCRATCH:
      return "the split workspace this shape needs exceeds the library's static scratch "
             "(dflash_attention_rel_noalloc_scratch_bytes)";
    default:
      return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
  }
}

int dflash_abi_version(void) { return DFLASH_ABI_VERSION; }

}  // extern "C"
