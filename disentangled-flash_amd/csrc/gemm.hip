// Dense projection GEMM with fused epilogues for the encoder layers, fp16 /
// bf16, gfx950 (CDNA4).
//
//   Y[m, n] = epilogue( sum_k X[m, k] * W[n, k] + bias[n] )
//
// X is the row-major activation [M, K], W the nn.Linear weight [N, K] (both
// K-contiguous), Y row-major [M, N].  Epilogues (applied to the sum rounded to
// the dtype first, as nn.Linear's output is):
//   kEpiBias     : Y = T(acc + bias)                         (QKV projection)
//   kEpiBiasGelu : Y = T(gelu_erf(T(acc + bias)))            (FFN intermediate,
//                  DebertaV2Intermediate = dense then ACT2FN["gelu"], the exact
//                  erf form; _reference.py:470-471)
//   kEpiBiasAdd  : Y = T(T(acc + bias) + R[m, n])            (dense + residual
//                  of DebertaV2SelfOutput / DebertaV2Output before LayerNorm,
//                  _reference.py:108-112, 482-485)
//
// Tiling.  A workgroup of WAVES_M x WAVES_N wavefronts computes a 256 x BN
// tile of Y (GemmConfig below: 256 x 192 with 4 or 8 wavefronts, 256 x 128
// with 4 wavefronts at two workgroups per CU).  K is walked in steps of 32
// through a ring of LDS stages.  Global -> LDS copies use
// global_load_lds_dwordx4: no registers, no VALU; each instruction of a
// wavefront writes 1 KB of LDS in lane order, so the LDS layout is chosen by
// which global chunk each lane fetches.  Rows of the K-step are 64 bytes; two
// rows form a 128-byte line, and the eight 16-byte chunks of a line are
// XOR-swizzled with the line index, which makes the MFMA fragment reads
// (ds_read_b128, 16 rows x one k-slice per 16 lanes) bank-conflict free.
//
// MFMA v_mfma_f32_16x16x32_{f16,bf16} with the weight as the A operand and the
// activation as B, so the accumulator of lane (c, g) holds Y[m0 + c][n0 + 4g ..
// n0 + 4g + 3]: four consecutive outputs of one row.  The epilogue stages the
// tile through LDS and writes it in coalesced 16-byte chunks.
//
// Launch order: workgroup p runs on XCD p % 8.  Each XCD takes a contiguous
// range of tiles.  When X is the larger operand (M >= N: many rows) the range
// is row-major (column blocks fastest), so the tiles of one X row block run on
// the same XCD and share its L2, and every XCD streams all of W; when W is the
// larger (few rows) it is column-major, so every XCD streams all of X and only
// its own slice of W (at 512 rows this takes the 1536-wide QKV from 26.2 to
// 17.9 us and the FFN intermediate from 28.0 to 21.6 us, bf16).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "device_common.h"
#include "dflash.h"

namespace dflash {

namespace {

typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kGemmThreads = 256;  // 4 wavefronts, 2 x 2 over the tile
constexpr int kBK = 32;            // K per stage (one MFMA k-step)

constexpr int kEpiBias = 0;
constexpr int kEpiBiasGelu = 1;
constexpr int kEpiBiasAdd = 2;

// Byte offset inside a stage's X or W tile of (row, 16-byte chunk c in 0..3).
// Two 64-byte rows form line row/2; chunk position p = 4*(row&1) + c is
// XOR-swizzled with the line index.
__device__ constexpr int swz_offset(int row, int c) {
  const int line = row >> 1;
  const int p = ((row & 1) << 2) | c;
  return line * 128 + ((p ^ (line & 7)) << 4);
}

// The inverse for the copy: LDS slot s (16 bytes, lane order) -> (row, chunk).
__device__ inline void swz_slot(int s, int& row, int& c) {
  const int line = s >> 3;
  const int p = (s & 7) ^ (line & 7);
  row = 2 * line + (p >> 2);
  c = p & 3;
}

// GELU in its erf form, 0.5 x (1 + erf(x / sqrt 2)), with erf from
// Abramowitz & Stegun, Handbook of Mathematical Functions, formula 7.1.26:
//   erf(z) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) exp(-z^2),
//   t = 1 / (1 + p z), z >= 0, |error| <= 1.5e-7.
// For x < 0 the complement 1 + erf(-|z|) = (a1 t + ...) exp(-z^2) is used
// directly, so the small values of the negative tail carry no cancellation.
// About 12 instructions against ~40 for the library erff with both of its
// branches; the difference is far below the fp16/bf16 rounding of the output.
__device__ inline float gelu_erf(float x) {
  constexpr float kP = 0.3275911f;
  constexpr float kA1 = 0.254829592f, kA2 = -0.284496736f, kA3 = 1.421413741f,
                  kA4 = -1.453152027f, kA5 = 1.061405429f;
  const float z = fabsf(x) * 0.70710678118654752440f;
  const float t = __builtin_amdgcn_rcpf(fmaf(kP, z, 1.0f));
  const float poly = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, kA5, kA4), kA3), kA2), kA1);
  const float tail = poly * __builtin_amdgcn_exp2f(-z * z * 1.44269504088896341f);  // erfc(z)
  const float phi = x >= 0.0f ? 1.0f - 0.5f * tail : 0.5f * tail;                // Phi(x)
  return x * phi;
}

// One global_load_lds_dwordx4: 16 bytes from `src` (per lane) to LDS at
// `lds_base` + 16 * lane (`lds_base` wavefront-uniform).  Kept in a __device__
// function: used directly inside the kernel body, the builtin stops clang's host
// pass from emitting the kernel's launch stub.
__device__ inline void copy16_to_lds(const void* src, unsigned char* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)lds_base, 16, 0, 0);
}

// s_barrier after this wavefront's LDS reads have returned, without the memory
// fence of __syncthreads() (which would wait for every pending copy and drain
// the pipeline).  The copies' LDS writes are published by the explicit vmcnt
// waits before it; the memory clobber keeps LDS accesses on their side.
__device__ inline void workgroup_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait until at most N of this thread's vector-memory operations are pending.
template <int N>
__device__ inline void wait_vmem() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

}  // namespace

// Tile configuration: a workgroup of WAVES_M x WAVES_N wavefronts computes a
// BM x BN tile of Y (wavefront tile BM/WAVES_M x BN/WAVES_N) through a ring of
// STAGES LDS stages; WGS workgroups per CU are budgeted for.
template <int BN_, int STAGES_, int WGS_, int WAVES_M_, int WAVES_N_, int BM_ = 256>
struct GemmConfig {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int STAGES = STAGES_;
  static constexpr int WGS = WGS_;
  static constexpr int WAVES_M = WAVES_M_;
  static constexpr int WAVES_N = WAVES_N_;
  static constexpr int THREADS = 64 * WAVES_M * WAVES_N;
  static constexpr int WM = BM / WAVES_M;
  static constexpr int WN = BN / WAVES_N;
  static constexpr int MB = WM / 16;                 // 16-row blocks per wavefront
  static constexpr int NB = WN / 16;                 // 16-column blocks per wavefront
  static constexpr int A_CHUNKS = BM * kBK / 8;      // 16-byte chunks of a stage's X tile
  static constexpr int B_CHUNKS = BN * kBK / 8;
  // Copy instructions per thread per stage.  A chunk count that is not a
  // multiple of the workgroup size leaves the last round to the first
  // wavefronts (whole wavefronts, so the counts stay wavefront-uniform).
  static constexpr int A_LOADS = (A_CHUNKS + THREADS - 1) / THREADS;
  static constexpr int B_LOADS = (B_CHUNKS + THREADS - 1) / THREADS;
  static constexpr int A_BYTES = BM * kBK * 2;
  static constexpr int STAGE_BYTES = (BM + BN) * kBK * 2;
  static constexpr int TILE_LD = BN + 8;             // epilogue staging row (elements)
  static constexpr int RING = STAGES * STAGE_BYTES;
  static constexpr int STAGING = BM * TILE_LD * 2;
  static constexpr int LDS = RING > STAGING ? RING : STAGING;
  static_assert(A_CHUNKS % 64 == 0 && B_CHUNKS % 64 == 0, "copies in whole wavefronts");
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wavefront tile of whole MFMA blocks");
  static_assert(STAGES >= 3, "the pipeline keeps STAGES - 2 stages in flight");
  static_assert((STAGES - 2) * (A_LOADS + B_LOADS) <= 63, "vmcnt range");
  // Copies a wavefront issues per stage (its last rounds may be partial).
  __device__ static constexpr int loads_of(int wave) {
    int n = 0;
    for (int j = 0; j < A_LOADS; ++j) n += (j * THREADS + wave * 64 < A_CHUNKS) ? 1 : 0;
    for (int j = 0; j < B_LOADS; ++j) n += (j * THREADS + wave * 64 < B_CHUNKS) ? 1 : 0;
    return n;
  }
};

struct GemmArgs {
  const void* x;
  const void* w;
  const void* bias;
  const void* residual;
  void* y;
  int M, N, K;
  int m_blocks, n_blocks;
  int col_major;  // tile order within an XCD's range: column blocks slowest
};

template <typename T, int EPI, typename CF>
__global__ __launch_bounds__(CF::THREADS, CF::WGS) void gemm_kernel(GemmArgs a) {
  using M = Mma<T>;
  using F = typename M::frag;
  constexpr int BN = CF::BN;
  constexpr int S = CF::STAGES;
  constexpr int MB = CF::MB;
  constexpr int NB = CF::NB;
  extern __shared__ __align__(16) unsigned char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wm = wave % CF::WAVES_M;  // wavefront row block
  const int wn = wave / CF::WAVES_M;  // wavefront column block
  constexpr int NT = CF::THREADS;

  // Tile of this workgroup (XCD-aware order, see the file comment).
  const int total = a.m_blocks * a.n_blocks;
  const int p = blockIdx.x;
  const int per_xcd = (total + 7) >> 3;
  const int t = (p & 7) * per_xcd + (p >> 3);
  if (t >= total) return;  // padding of the grid to a multiple of 8
  int mb, nb;
  if (a.col_major) {
    nb = t / a.m_blocks;
    mb = t - nb * a.m_blocks;
  } else {
    mb = t / a.n_blocks;
    nb = t - mb * a.n_blocks;
  }
  const int m_base = mb * CF::BM;
  const int n_base = nb * BN;
  const int K = a.K;

  const T* X = reinterpret_cast<const T*>(a.x);
  const T* W = reinterpret_cast<const T*>(a.w);

  // Per-thread source pointers of its copy slots (advance by kBK per stage).
  const T* asrc[CF::A_LOADS];
  const T* bsrc[CF::B_LOADS];
#pragma unroll
  for (int j = 0; j < CF::A_LOADS; ++j) {
    int row, ch;
    swz_slot(min(j * NT + tid, CF::A_CHUNKS - 1), row, ch);
    const int m = min(m_base + row, a.M - 1);  // rows past M repeat row M-1 (never stored)
    asrc[j] = X + static_cast<int64_t>(m) * K + ch * 8;
  }
#pragma unroll
  for (int j = 0; j < CF::B_LOADS; ++j) {
    int row, ch;
    swz_slot(min(j * NT + tid, CF::B_CHUNKS - 1), row, ch);
    bsrc[j] = W + static_cast<int64_t>(n_base + row) * K + ch * 8;
  }
  // LDS destinations: wavefront-uniform bases of each copy instruction; a
  // wavefront whose slots of a round lie past the tile skips that round.
  auto issue = [&](int stage, int kt) {
    unsigned char* sa = smem + stage * CF::STAGE_BYTES;
    unsigned char* sb = sa + CF::A_BYTES;
    const int koff = kt * kBK;
#pragma unroll
    for (int j = 0; j < CF::A_LOADS; ++j)
      if (CF::A_CHUNKS % NT == 0 || j * NT + wave * 64 < CF::A_CHUNKS)
        copy16_to_lds(asrc[j] + koff, sa + (j * NT + wave * 64) * 16);
#pragma unroll
    for (int j = 0; j < CF::B_LOADS; ++j)
      if (CF::B_CHUNKS % NT == 0 || j * NT + wave * 64 < CF::B_CHUNKS)
        copy16_to_lds(bsrc[j] + koff, sb + (j * NT + wave * 64) * 16);
  };

  // Lane-constant fragment offsets: X rows wm*WM + 16*i + c, W rows wn*WN + 16*i + c,
  // k-slice g.  Every fragment address is a multiple of 16 bytes; saying so
  // keeps the reads single ds_read_b128 (the library is built with unaligned
  // LDS access off, where an unproven alignment becomes byte reads).
  const int xoff = swz_offset(wm * CF::WM + c, g);
  const int woff = swz_offset(wn * CF::WN + c, g);
  auto x_frag = [&](int stage, int i) {
    return *static_cast<const F*>(__builtin_assume_aligned(
        smem + stage * CF::STAGE_BYTES + xoff + i * 16 * 64, 16));
  };
  auto w_frag = [&](int stage, int i) {
    return *static_cast<const F*>(__builtin_assume_aligned(
        smem + stage * CF::STAGE_BYTES + CF::A_BYTES + woff + i * 16 * 64, 16));
  };

  f32x4_t acc[NB][MB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Pipeline over the k-steps kt = 0 .. KT-1 with a ring of S LDS stages
  // (k-step kt in stage kt % S).  While the MFMAs of kt run from registers, the
  // fragments of kt + 1 are read from LDS and the copies of kt + 2 .. kt + S - 1
  // are in flight.  One barrier per k-step: it publishes the copies of kt + 1
  // and guarantees that every wavefront has its fragments of kt in registers,
  // so stage kt % S is refilled with k-step kt + S right after it.  Every
  // iteration issues one stage of copies (past the last k-step it re-fetches
  // k-step KT - 1 into a stage nobody reads again), so the number of copies in
  // flight is the same in every iteration and the waits are compile-time.
  const int KT = K / kBK;
#pragma unroll
  for (int s0 = 0; s0 < S; ++s0) issue(s0, min(s0, KT - 1));
  F xf[MB], wf[NB], wnext[NB];
  // Waits: copies of k-step kt + 1 are complete once at most those of
  // kt + 2 .. kt + S - 1 are pending.  The per-stage count of a wavefront is
  // one of two compile-time values (full or short last copy round).
  constexpr int kLoadsHi = CF::loads_of(0);
  constexpr int kLoadsLo = CF::loads_of(CF::WAVES_M * CF::WAVES_N - 1);
  const bool short_wave = CF::loads_of(wave) != kLoadsHi;
  auto wait_next = [&]() {
    if (short_wave) {
      wait_vmem<(S - 2) * kLoadsLo>();
    } else {
      wait_vmem<(S - 2) * kLoadsHi>();
    }
  };
  if (short_wave) {
    wait_vmem<(S - 1) * kLoadsLo>();  // k-step 0
  } else {
    wait_vmem<(S - 1) * kLoadsHi>();
  }
  workgroup_barrier();
#pragma unroll
  for (int i = 0; i < MB; ++i) xf[i] = x_frag(0, i);
#pragma unroll
  for (int i = 0; i < NB; ++i) wf[i] = w_frag(0, i);
  int stage = 0;  // stage of k-step kt
  for (int kt = 0; kt < KT; ++kt) {
    // The last iteration reads stage `next` too (harmless, unused): no branch.
    const int next = stage + 1 == S ? 0 : stage + 1;
    wait_next();
    workgroup_barrier();
    issue(stage, min(kt + S, KT - 1));
    // The next W fragments go into a second register set first (every MFMA of
    // this k-step reads the current ones); X fragment j is refilled from the
    // next stage as soon as its last MFMA has issued.
#pragma unroll
    for (int i = 0; i < NB; ++i) wnext[i] = w_frag(next, i);
#pragma unroll
    for (int j = 0; j < MB; ++j) {
#pragma unroll
      for (int i = 0; i < NB; ++i) acc[i][j] = M::run(wf[i], xf[j], acc[i][j]);
      xf[j] = x_frag(next, j);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) wf[i] = wnext[i];
    stage = next;
  }

  // ---- epilogue ----
  // 1. Registers -> LDS: lane (c, g) holds Y[m][n .. n+3] of every 16 x 16
  //    block; it adds the bias, rounds to T (as nn.Linear's output), applies
  //    GELU if asked, and writes the four values into a row-major staging tile
  //    (the LDS ring is free once every copy has landed and every wavefront
  //    is past its last fragment read).
  // 2. LDS -> HBM: the workgroup writes the 256 x BN tile in 16-byte chunks,
  //    consecutive threads along a row, adding the residual for kEpiBiasAdd
  //    with the same coalesced access.
  const T* bias = reinterpret_cast<const T*>(a.bias);
  Quad<T> bq[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i)
    bq[i] = *reinterpret_cast<const Quad<T>*>(bias + n_base + wn * CF::WN + 16 * i + 4 * g);
  wait_vmem<0>();
  workgroup_barrier();
  T* tile = reinterpret_cast<T*>(smem);
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int col = wn * CF::WN + 16 * i + 4 * g;
#pragma unroll
    for (int j = 0; j < MB; ++j) {
      const int row = wm * CF::WM + 16 * j + c;
      Quad<T> out;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const T lin = static_cast<T>(acc[i][j][r] + static_cast<float>(bq[i][r]));
        if constexpr (EPI == kEpiBiasGelu) {
          out[r] = static_cast<T>(gelu_erf(static_cast<float>(lin)));
        } else {
          out[r] = lin;
        }
      }
      *static_cast<Quad<T>*>(__builtin_assume_aligned(tile + row * CF::TILE_LD + col, 8)) = out;
    }
  }
  workgroup_barrier();
  constexpr int kRowChunks = BN / 8;  // 16-byte chunks per tile row
  typedef T Oct __attribute__((ext_vector_type(8)));
  const T* res = reinterpret_cast<const T*>(a.residual);
  T* Y = reinterpret_cast<T*>(a.y);
  const int rows = min(CF::BM, a.M - m_base);
  for (int q = tid; q < rows * kRowChunks; q += NT) {
    const int row = q / kRowChunks;
    const int ch = q - row * kRowChunks;
    Oct v = *static_cast<const Oct*>(
        __builtin_assume_aligned(tile + row * CF::TILE_LD + 8 * ch, 16));
    const int64_t off = static_cast<int64_t>(m_base + row) * a.N + n_base + 8 * ch;
    if constexpr (EPI == kEpiBiasAdd) {
      const Oct rv = *reinterpret_cast<const Oct*>(res + off);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        v[e] = static_cast<T>(static_cast<float>(v[e]) + static_cast<float>(rv[e]));
    }
    *reinterpret_cast<Oct*>(Y + off) = v;
  }
}

namespace {

// Configurations: 256 x 192 tiles at one workgroup per CU (N % 192 == 0) and
// 256 x 128 tiles at two (N % 128 == 0); for few rows, 64 x 128 tiles at three
// workgroups per CU and 64 x 64 tiles at four, which give four times the tiles
// of the 256-row forms (at 512 rows a 1536-wide projection has 96 and 192).
using CfgWide = GemmConfig<192, 5, 1, 2, 2>;
using CfgPair = GemmConfig<128, 3, 2, 2, 2>;
using CfgEight = GemmConfig<192, 5, 1, 4, 2>;
using CfgSmall = GemmConfig<128, 4, 3, 2, 2, 64>;
using CfgTiny = GemmConfig<64, 4, 4, 2, 2, 64>;

template <typename T, int EPI, typename CF>
int launch_gemm(GemmArgs args, hipStream_t stream) {
  constexpr auto* kernel = &gemm_kernel<T, EPI, CF>;
  // The dynamic LDS limit is raised once per device (the attribute persists).
  static std::atomic<uint64_t> raised{0};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return static_cast<int>(err);
  const uint64_t bit = dev < 64 ? (uint64_t{1} << dev) : 0;
  if (bit == 0 || (raised.load(std::memory_order_acquire) & bit) == 0) {
    err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, CF::LDS);
    if (err == hipSuccess && bit != 0) raised.fetch_or(bit, std::memory_order_release);
  }
  if (err != hipSuccess) return static_cast<int>(err);
  args.m_blocks = (args.M + CF::BM - 1) / CF::BM;
  args.n_blocks = args.N / CF::BN;
  // Each XCD walks a contiguous range of tiles.  Row-major ranges make every
  // XCD read the whole of W (and its own rows of X), column-major ones the
  // whole of X (and its own slice of W): take the order whose repeated operand
  // is the smaller.
  args.col_major = args.N > args.M ? 1 : 0;
  const int64_t tiles = static_cast<int64_t>(args.m_blocks) * args.n_blocks;
  const int64_t grid = ((tiles + 7) / 8) * 8;
  if (grid > 0x7fffffff) return DFLASH_ERR_TOO_LARGE;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(CF::THREADS), CF::LDS,
                     stream, args);
  return static_cast<int>(hipGetLastError());
}

// CUs of the current device (cached per device; 256 if it cannot be read).
int gemm_device_cus() {
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

// config: 0 = automatic, 1 = CfgWide, 2 = CfgPair, 3 = CfgEight, 4 = CfgSmall,
// 5 = CfgTiny.  Automatic, for grids that fill at least half the CUs
// (measured at M = 16384, fp16): CfgEight where N % 192 == 0 (QKV 71.7 us,
// hidden-wide dense 24.5 us), except the GELU epilogue, whose VALU work
// overlaps better at two workgroups per CU (CfgPair, FFN intermediate 108.5
// against 117.6 us); CfgPair for N % 128 == 0 otherwise.
template <typename T, int EPI>
int pick_config(const GemmArgs& args, int config, hipStream_t stream) {
  const bool wide_ok = args.N % CfgWide::BN == 0;
  const bool pair_ok = args.N % CfgPair::BN == 0;
  if (config == 0 && !wide_ok && !pair_ok) {
    config = 5;  // N % 64 == 0 only: the 64 x 64 tiles at every row count
  } else if (config == 0) {
    config = (wide_ok && !(EPI == kEpiBiasGelu && pair_ok)) ? 3 : 2;
    // Few rows: when the 256-row grid would give fewer tiles than half the CUs,
    // the 64-row forms (four times the tiles) are faster on the device, 64 x 64
    // up to 1024 rows and 64 x 128 above (HIP-graph timings at 512 and 2048 rows:
    // e.g. a 2304-wide projection of 512 x 768 in 7.0 against 17.6 us).
    const int bn = config == 3 ? CfgEight::BN : CfgPair::BN;
    const int64_t tiles = static_cast<int64_t>((args.M + 255) / 256) * (args.N / bn);
    if (2 * tiles < gemm_device_cus()) config = (args.M <= 1024 || !pair_ok) ? 5 : 4;
  }
  switch (config) {
    case 1:
      return wide_ok ? launch_gemm<T, EPI, CfgWide>(args, stream) : DFLASH_ERR_SHAPE;
    case 2:
      return pair_ok ? launch_gemm<T, EPI, CfgPair>(args, stream) : DFLASH_ERR_SHAPE;
    case 3:
      return wide_ok ? launch_gemm<T, EPI, CfgEight>(args, stream) : DFLASH_ERR_SHAPE;
    case 4:
      return pair_ok ? launch_gemm<T, EPI, CfgSmall>(args, stream) : DFLASH_ERR_SHAPE;
    case 5:
      return launch_gemm<T, EPI, CfgTiny>(args, stream);  // N % 64 == 0 is checked on entry
    default:
      return DFLASH_ERR_SHAPE;
  }
}

template <typename T>
int dispatch_epilogue(const GemmArgs& args, int epilogue, int config, hipStream_t stream) {
  switch (epilogue) {
    case DFLASH_GEMM_BIAS:
      return pick_config<T, kEpiBias>(args, config, stream);
    case DFLASH_GEMM_BIAS_GELU:
      return pick_config<T, kEpiBiasGelu>(args, config, stream);
    case DFLASH_GEMM_BIAS_ADD:
      return pick_config<T, kEpiBiasAdd>(args, config, stream);
    default:
      return DFLASH_ERR_SHAPE;
  }
}

}  // namespace

}  // namespace dflash

using namespace dflash;

extern "C" int dflash_linear_fwd(const void* x, const void* weight, const void* bias,
                                 const void* residual, void* y, int M, int N, int K,
                                 int epilogue, int dtype, void* stream) {
  if (M < 0 || N < 1 || K < 1) return DFLASH_ERR_SHAPE;
  if (M == 0) return DFLASH_OK;
  if (!x || !weight || !bias || !y) return DFLASH_ERR_NULL;
  if ((epilogue & 0xff) == DFLASH_GEMM_BIAS_ADD && !residual) return DFLASH_ERR_NULL;
  if (N % 64 != 0 || K % kBK != 0) return DFLASH_ERR_SHAPE;
  if (static_cast<int64_t>(M) * K >= (int64_t{1} << 31) ||
      static_cast<int64_t>(M) * N >= (int64_t{1} << 31))
    return DFLASH_ERR_TOO_LARGE;
  const uintptr_t addr_or = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                            reinterpret_cast<uintptr_t>(y) |
                            reinterpret_cast<uintptr_t>(residual);
  if (addr_or % 16 != 0 || reinterpret_cast<uintptr_t>(bias) % 8 != 0) return DFLASH_ERR_ALIGN;
  // Bits 8.. of `epilogue` select a tile configuration (0 = automatic).
  const int config = epilogue >> 8;
  epilogue &= 0xff;
  GemmArgs args{x, weight, bias, residual, y, M, N, K, 0, 0};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == DFLASH_DTYPE_FP16) return dispatch_epilogue<_Float16>(args, epilogue, config, s);
  if (dtype == DFLASH_DTYPE_BF16) return dispatch_epilogue<__bf16>(args, epilogue, config, s);
  return DFLASH_ERR_DTYPE;
}
