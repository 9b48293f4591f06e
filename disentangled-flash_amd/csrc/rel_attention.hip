// Fused DeBERTa disentangled attention with in-kernel relative scores,
// 16-bit inputs (fp16 / bf16), gfx950 (CDNA4).
//
// Scores of one (batch, head), query i, key j (kernel.py:196-345):
//
//   s(i, j) = Q_i.K_j + c2p(i, slot(i-j)) + p2c(j, slot(i-j))
//   c2p(i, s) = Q_i.Kr[s],  p2c(j, s) = K_j.Qr[s]   (each rounded to the input
//   dtype, as the reference's separate torch.matmul outputs are, kernel.py:577,583)
//
// Workgroup = 4 wavefronts = 4*QW query rows of one (b, h); every wavefront
// keeps its QW query rows in registers and walks the keys in tiles of BN.
//
// Relative scores are computed per *delta* rather than per slot: for a tile
// the deltas i-j form one contiguous range, so the wavefront builds
//
//   Cw[q][t] = Q_{i0w+q} . Kr[slot(dlo_w + t)]      (its own QW queries)
//
// and the workgroup shares
//
//   Pw[jr][t] = K_{j0+jr} . Qr[slot(dlo + t)]
//
// with MFMA, where the rows Kr[slot(.)] / Qr[slot(.)] are gathered through
// delta_to_local while they are loaded from L2.  Element (i, j) of the tile
// then sits at a window index that is a lane constant plus a compile-time
// offset, so the score gathers are LDS reads with immediate offsets and no
// lookup table is touched inside the tile.  The price is that deltas sharing
// a bucket are multiplied more than once (about 15 % more relative-score MFMA
// work than one product per slot).
//
// Layout of the score tile: S^T = K.Q^T with v_mfma_f32_16x16x32_{f16,bf16},
// so each lane holds one query column and four keys per 16x16 block; the
// probabilities are then already the B operand of O^T += V^T.P^T.
// Row sums come from the same MFMA with an all-ones A operand (d <= 64), or
// for d = 128, whose matrix unit is the busier one, from per-lane dot2 sums
// reduced over the four lane groups at the end.
//
// Global reads go through buffer resources: an offset at or past the
// resource's size returns zero, which clamps rows past L for free; lookup
// indices of deltas outside [-(L-1), L-1] are clamped to the end of the table
// and read as slot 0 (those elements are masked or belong to rows that are
// never stored).  Offsets are never negative.
//
// Mask semantics (kernel.py:250-261): kept query & kept key -> score; kept
// query & padded key -> excluded; padded query in range -> uniform over the
// in-range keys, i.e. the mean of V, which is computed separately and stored
// for those rows.  The key loop of a workgroup ends at the tile of the last
// kept key of the sequence.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <numeric>
#include <type_traits>

#include <cstdlib>

#include "device_common.h"
#include "dflash.h"
#include "rel_attention.h"

namespace dflash {

namespace {

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef short s4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4_t lds_s4_t;

constexpr int kBufferFlags = 0x00020000;  // raw buffer, gfx9 family descriptor word 3

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                           static_cast<int>(bytes), kBufferFlags);
}

__device__ inline u32x4_t load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ inline u32x2_t load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ inline uint32_t load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ inline uint8_t load1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}

// One buffer_load_dwordx4 with the LDS-direct bit: 16 bytes per lane from
// `off` to LDS at `lds_base` + 16 * lane (`lds_base` wavefront-uniform, in M0;
// M0 is restored afterwards).  Out-of-range reads store zeros.  The copy
// counts in vmcnt like any buffer load, and its LDS writes are awaited with an
// explicit vmcnt wait (wait_vmem) before the barrier that publishes them.
// Written as inline assembly so that the compiler does not track the copy:
// for the builtin it cannot tell the copy's LDS range from that of the
// transposing V reads and waits for every copy in flight before them.
__device__ inline void copy16_lds(__amdgpu_buffer_rsrc_t r, uint32_t off, unsigned char* lds_base) {
  const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_base));
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_addr), "v"(off), "s"(r)
      : "memory");
}

// Wait until at most N of this wavefront's vector-memory operations are pending.
template <int N>
__device__ inline void wait_vmem() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Compiler barrier for memory operations: keeps the buffer loads issued after
// a group of direct copies on their side, so that the vmcnt waits count them.
__device__ inline void memory_order_point() { asm volatile("" ::: "memory"); }

typedef float f32x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8_t __attribute__((ext_vector_type(8)));

// Operand traits of the kernel: one k-step is 32 deep, and a lane's operand
// fragment holds 8 consecutive k of its row or column (k = 8g .. 8g+7 for lane
// group g).  16-bit T: one v_mfma_f32_16x16x32_{f16,bf16}, fragment 16 bytes.
// fp32: eight chained v_mfma_f32_16x16x4_f32, fragment 32 bytes; element e of
// every lane's fragment feeds MFMA e, where lane (c, g) contributes k = 8g + e
// in both operands, so the eight MFMAs sum exactly the 32 products of the step.
template <typename T>
struct RelMma {
  using frag = typename Mma<T>::frag;
  __device__ static f32x4_t run(frag a, frag b, f32x4_t c) { return Mma<T>::run(a, b, c); }
};
template <>
struct RelMma<float> {
  using frag = f32x8_t;
  __device__ static f32x4_t run(frag a, frag b, f32x4_t c) {
#pragma unroll
    for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], c, 0, 0, 0);
    return c;
  }
};

// fp32 operands on the bf16 matrix unit (fp32_precision="fast"): each value is
// split into x = hi + lo with hi = bf16(x) and lo = bf16(x - hi), and the
// product a.b is a_hi.b_hi + a_hi.b_lo + a_lo.b_hi (three
// v_mfma_f32_16x16x32_bf16; the dropped a_lo.b_lo and the rounding of lo leave a
// relative error of about 2^-16 per product, against 2^-11 for TF32, the
// reference's fast mode).  The fragments are the fp32 ones (k = 8g + e in both
// operands), which is the 16-bit instruction's k layout.
struct RelMmaFast {
  using frag = f32x8_t;
  struct split_frag {
    bf16x8_t hi, lo;
  };
  __device__ static split_frag split(const f32x8_t& x) {
    split_frag s;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const __bf16 h = static_cast<__bf16>(x[e]);
      s.hi[e] = h;
      s.lo[e] = static_cast<__bf16>(x[e] - static_cast<float>(h));
    }
    return s;
  }
  __device__ static const split_frag& as_split(const split_frag& x) { return x; }
  __device__ static split_frag as_split(const f32x8_t& x) { return split(x); }
  // Operands may be fp32 fragments (split here) or fragments split once where
  // they are produced (the ones used by several products).
  template <typename A, typename B>
  __device__ static f32x4_t run(const A& a, const B& b, f32x4_t c) {
    const split_frag sa = as_split(a);
    const split_frag sb = as_split(b);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.lo, sb.hi, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.hi, sb.lo, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.hi, sb.hi, c, 0, 0, 0);
  }
};

// Strict fp32 products on the bf16 matrix unit (bf16x6): each fp32 value is
// split into x = hi + mid + lo, three bf16 parts holding its 24 significand
// bits (hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid)), and a.b
// keeps the six part products down to 2^-16 of the leading one: lo.hi, hi.lo,
// mid.mid, mid.hi, hi.mid, hi.hi (smallest first).  The dropped mid.lo,
// lo.mid and lo.lo are below 2^-24 of it, fp32's own rounding; accumulation is
// fp32.  Six v_mfma_f32_16x16x32_bf16 (96 cycles) replace eight
// v_mfma_f32_16x16x4f32 (256 cycles) per 32-deep product.
struct RelMmaExact {
  using frag = f32x8_t;
  struct split_frag {
    bf16x8_t hi, mid, lo;
  };
  __device__ static split_frag split(const f32x8_t& x) {
    split_frag s;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const __bf16 h = static_cast<__bf16>(x[e]);
      const float r = x[e] - static_cast<float>(h);
      const __bf16 m = static_cast<__bf16>(r);
      s.hi[e] = h;
      s.mid[e] = m;
      s.lo[e] = static_cast<__bf16>(r - static_cast<float>(m));
    }
    return s;
  }
  __device__ static const split_frag& as_split(const split_frag& x) { return x; }
  __device__ static split_frag as_split(const f32x8_t& x) { return split(x); }
  template <typename A, typename B>
  __device__ static f32x4_t run(const A& a, const B& b, f32x4_t c) {
    const split_frag sa = as_split(a);
    const split_frag sb = as_split(b);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.lo, sb.hi, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.hi, sb.lo, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.mid, sb.mid, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.mid, sb.hi, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.hi, sb.mid, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa.hi, sb.hi, c, 0, 0, 0);
  }
};

// Elements of T per 16-byte chunk.
template <typename T>
constexpr int kChunkElems = 16 / static_cast<int>(sizeof(T));

// One lane's operand fragment from global memory (16 or 32 bytes at `off`).
template <typename T>
__device__ inline typename RelMma<T>::frag load_frag(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 4) {
    const u32x4_t lo = load16(r, off);
    const u32x4_t hi = load16(r, off + 16);
    return __builtin_bit_cast(f32x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  } else {
    return __builtin_bit_cast(typename RelMma<T>::frag, load16(r, off));
  }
}

// The elements of one 16-byte chunk.
template <typename T>
__device__ inline auto chunk_elems(u32x4_t v) {
  typedef T V __attribute__((ext_vector_type(kChunkElems<T>)));
  return __builtin_bit_cast(V, v);
}

template <typename T>
__device__ inline typename RelMma<T>::frag ones_frag() {
  typename RelMma<T>::frag f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = static_cast<T>(1.0f);
  return f;
}

// Four fp32 accumulators -> four T values in one 8-byte LDS store.
template <typename T>
__device__ inline void store4(T* dst, f32x4_t acc) {
  Quad<T> q;
#pragma unroll
  for (int r = 0; r < 4; ++r) q[r] = static_cast<T>(acc[r]);
  *reinterpret_cast<Quad<T>*>(dst) = q;
}

// s + a + b with a, b in T: one dot2 against (1, 1) (exact products, fp32 sum).
template <typename T>
__device__ inline float add2(float s, T a, T b) {
  if constexpr (sizeof(T) == 4) {
    return s + a + b;
  } else if constexpr (__is_same(T, _Float16)) {
    const half2_t v = {a, b};
    const half2_t one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
    return __builtin_amdgcn_fdot2(v, one, s, false);
  } else {
    const bf16x2_t v = {a, b};
    const bf16x2_t one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
    return __builtin_amdgcn_fdot2_f32_bf16(v, one, s, false);
  }
}

// s + lo + hi of a packed pair of T (exact products with 1, fp32 sum).
template <typename T>
__device__ inline float sum2(float s, uint32_t packed) {
  if constexpr (__is_same(T, _Float16)) {
    const half2_t one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, packed), one, s, false);
  } else {
    const bf16x2_t one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, packed), one, s, false);
  }
}

// Key of MFMA row x within a 16-key block: x = 4a + b holds key a + 4b, so
// lane (c, g) of a 16x16 score block holds keys g + 4r (r = 0..3) and one
// gather instruction (fixed r) touches four adjacent keys.  The transposing
// reads of the V operand use the same order, so P^T and V^T pair up in the PV
// product.
__device__ constexpr int key_of(int x) { return (x & 3) * 4 + (x >> 2); }

template <int N>
struct IntC {
  static constexpr int value = N;
};

// K and V tiles copied straight from memory into LDS (buffer loads with the
// LDS-direct bit) instead of through registers: 16-bit data at d >= 64.  With
// one V buffer, V is copied after the first barrier of its tile and awaited at
// the second, so the QK phase in between must hide the copy: not in the table
// form (the wait would also wait for the table loads issued after the copy),
// and only with the p2c products in that phase (without them, C5 d = 128 c2p
// ran 79.7 against 76.9 us through registers).  A copy instruction writes 64
// consecutive 16-byte chunks, so the tiles are unpadded, with the 16-byte
// chunks of each row permuted by kv_swizzle (below) instead of a row pad.
template <typename T, int D, int VBUFS, bool TABLE, bool P2C>
constexpr bool rel_kv_direct() {
  return sizeof(T) == 2 && D >= 64 && (VBUFS == 2 || (!TABLE && P2C));
}

// Chunk permutation of row `row` of a directly copied K / V tile: logical
// 16-byte chunk x of the row sits at chunk x ^ kv_swizzle(row).  With
// row = 4a + b (bits 0-3), b = 2 b1 + b0:
//   * K fragment reads (16 bytes per lane, rows key_of(c) of a 16-key block,
//     one chunk per lane group g): the eight rows of lanes c = 0..7 (or
//     8..15), b1 fixed, land in eight different chunks of a 128-byte bank
//     window (a and b0 are in bits 0-2);
//   * V transposing reads (8 bytes per lane, rows 4a + g, four lanes per
//     32-byte pair of chunks, pair x >> 1 ^ kv_swizzle >> 1): the rows served
//     together - four (a) per 16 lanes, eight (a, b0) per 32 lanes - land in
//     different pairs (a in bits 1-2, b0 in bit 3 at d = 128; at d = 64 a row
//     is 128 bytes, so rows of different b0 already sit in different halves of
//     a 256-byte window).
// Measured at d = 128 (C5): 56 bank-conflict units per wavefront, against
// 297 with b1 in bit 3 (conflict-free for 16-lane groups only).
template <int D>
__device__ constexpr int kv_swizzle(int row) {
  const int a = (row >> 2) & 3;
  const int b0 = row & 1;
  const int b1 = (row >> 1) & 1;
  return D == 64 ? ((b0 ^ b1) | (a << 1)) : (b0 | (a << 1) | (b0 << 3));
}

// Strict fp32 on the bf16 matrix unit (bf16x6 products, RelMmaExact): at
// d <= 64, and at d = 128 without the c2p term (with it, the split fragments
// spill; measured there, C5 c2p alone ran 345 against 327 us on the fp32 MFMA,
// p2c alone 232 against 275, neither term 172 against 189).
template <typename T, int D, bool FAST, bool C2P>
constexpr bool rel_exact_fp32() {
  return sizeof(T) == 4 && !FAST && (D <= 64 || !C2P);
}
// Strict fp32 on the bf16 unit stages K and V already split into three bf16
// planes (hi, mid, lo: 6 bytes per element, 1.5 times the fp32 tile).  At
// d = 64 this fits the LDS with one V buffer (159 KB per workgroup; two fp32 V
// buffers without planes measured the same as one), at d = 128 with 512 bytes
// to spare.
template <typename T, int D, bool FAST, bool C2P>
constexpr bool rel_kv_planes3() {
  return rel_exact_fp32<T, D, FAST, C2P>();
}

template <typename T, int D, int QW, int BN, int VBUFS, bool KV_DIRECT = false, bool PLANES3 = false>
struct RelLayout {
  static constexpr int BM = kWaves * QW;                // query rows per workgroup
  static constexpr int NCC = (QW + BN - 1 + 15) / 16;   // c2p window chunks per wavefront
  static constexpr int NPC = (BM + BN - 1 + 15) / 16;   // p2c window chunks per workgroup
  static constexpr int PU = (NPC + kWaves - 1) / kWaves;  // p2c chunks per wavefront
  static constexpr int KS_LD = KV_DIRECT ? D : D + 8;   // Ks[BN][KS_LD]
  // V tile row-major, Vs[BN][VS_LD]: the row pad of 4 elements makes the
  // transposing reads of the PV operand conflict-free (two passes per
  // half-wavefront) with the staging stores at their minimum.
  static constexpr int VS_LD = KV_DIRECT ? D : D + 4;
  // Row strides (in elements) chosen for the LDS of gfx950 as measured: 32
  // four-byte banks served per half-wavefront, a 2-byte read of two lanes in
  // one dword is a broadcast.  With them the score gathers (lanes = 16 queries
  // x 4 adjacent keys) are conflict-free and the 8-byte window stores take the
  // minimum two passes per half-wavefront.
  static constexpr int CW_LD = NCC == 5 ? 88 : 16 * NCC + 4;  // Cw[wave][QW][CW_LD]
  static constexpr int PW_LD = 16 * NPC + 20;                 // Pw[BN][PW_LD]

  // Elements of T in one K tile and in one V tile buffer (three bf16 planes
  // take 1.5 times the fp32 tile).
  static constexpr int KS_SIZE = PLANES3 ? BN * KS_LD * 3 / 2 : BN * KS_LD;
  static constexpr int VT_SIZE = PLANES3 ? BN * VS_LD * 3 / 2 : BN * VS_LD;

  static constexpr size_t ks_off = 0;
  static constexpr size_t vt_off = ks_off + size_t(KS_SIZE) * sizeof(T);
  static constexpr size_t pw_off = vt_off + VBUFS * size_t(VT_SIZE) * sizeof(T);
  static constexpr size_t cw_off = pw_off + size_t(BN) * PW_LD * sizeof(T);
  static constexpr size_t bytes = cw_off + size_t(kWaves) * QW * CW_LD * sizeof(T);
};

}  // namespace

template <typename T, int D, int QW, int BN, int VBUFS, int WGS, bool C2P, bool P2C, bool SPLIT,
          bool FAST = false, bool TABLE = false, bool ROWSAFE = false>
__global__ __launch_bounds__(kThreads, WGS) void rel_attention_kernel(RelParams p) {
  static_assert(!FAST || sizeof(T) == 4, "the bf16x3 form is for fp32 data");
  static_assert(!(TABLE && SPLIT), "the table form runs unsplit");
  // Relative windows built on the matrix unit from Kr / Qr rows (MC, MP), or
  // read from precomputed c2p / p2c tables (TABLE).
  constexpr bool MC = C2P && !TABLE;
  constexpr bool MP = P2C && !TABLE;
  // fp32 on the bf16 matrix unit: bf16x3 (FAST) or bf16x6 (strict, EXACT).
  constexpr bool EXACT = rel_exact_fp32<T, D, FAST, C2P>();
  constexpr bool SPLITQ = FAST || EXACT;
  using M = std::conditional_t<FAST, RelMmaFast, std::conditional_t<EXACT, RelMmaExact, RelMma<T>>>;
  using F = typename M::frag;
  // Fragments that feed several products: split once in the fp32 forms.
  using QF = std::conditional_t<FAST, typename RelMmaFast::split_frag,
                                std::conditional_t<EXACT, typename RelMmaExact::split_frag, F>>;
  auto to_q = [](const F& x) -> QF {
    if constexpr (SPLITQ) {
      return M::split(x);
    } else {
      return x;
    }
  };
  constexpr int E16 = kChunkElems<T>;   // elements per 16-byte chunk
  constexpr bool kDirect = rel_kv_direct<T, D, VBUFS, TABLE, P2C>();
  // Strict fp32 on the bf16 unit: K and V staged as three bf16 planes (split
  // once per workgroup instead of once per reading wavefront).
  constexpr bool PL3 = rel_kv_planes3<T, D, FAST, C2P>();
  static_assert(!PL3 || EXACT, "three planes feed the bf16x6 products");
  // K and V staged split (FAST: hi, lo; PL3: hi, mid, lo planes).
  constexpr bool kPlanes = FAST || PL3;
  using LY = RelLayout<T, D, QW, BN, VBUFS, kDirect, PL3>;
  constexpr int BM = LY::BM;
  constexpr int kQB = QW / 16;          // 16-query MFMA blocks per wavefront
  constexpr int KB = BN / 16;           // 16-key blocks per tile
  constexpr int DB = D / 16;            // 16-dim blocks of the output
  constexpr int KD = D / 32;            // MFMA k-steps over the head dimension
  constexpr int CPR = D / E16;          // 16-byte chunks per K row
  constexpr int NKC = BN * CPR;                  // 16-byte K chunks per tile
  constexpr int NCH = (NKC + kThreads - 1) / kThreads;
  constexpr int NVB = NCH;                       // 16-byte V chunks per thread (as K)
  constexpr int NCC = LY::NCC;
  constexpr int PU = LY::PU;
  constexpr int NPC = LY::NPC;
  constexpr uint32_t ES = sizeof(T);
  static_assert(BN % 32 == 0 && BN <= 64, "key tile must be 32 or 64 keys");
  static_assert(LY::bytes * WGS <= 160 * 1024, "workgroups per CU fit the 160 KB of LDS");
  static_assert(QW % 16 == 0, "query rows per wavefront must be a multiple of 16");
  static_assert(NKC % kThreads == 0 || NKC < kThreads, "K tile must split evenly over the workgroup");
  static_assert(!kDirect || NKC % kThreads == 0, "direct copies: whole rounds of 64 chunks per wavefront");

  extern __shared__ __align__(16) unsigned char smem[];
  T* Ks = reinterpret_cast<T*>(smem + LY::ks_off);
  T* Vt = reinterpret_cast<T*>(smem + LY::vt_off);
  T* Pw = reinterpret_cast<T*>(smem + LY::pw_off);
  T* Cw = reinterpret_cast<T*>(smem + LY::cw_off);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  const int L = p.L;
  const int mk = xcd_logical_block(blockIdx.x, gridDim.x);
  // Key split of the split-key form (the splits of a block are neighbours).
  const int split = SPLIT ? mk % p.splits : 0;
  const int m = SPLIT ? mk / p.splits : mk;
  const int qblk = m % p.nqb;
  // Groups of query blocks in head-major order (the batch index fastest):
  // each XCD's contiguous range of groups then holds sequences of every
  // length of the batch, not a few neighbouring ones, so the XCDs finish
  // together on ragged batches (C5 valid-length cycle: d = 128 71.8 -> 53.1
  // us, d = 32 28.3 -> 21.5 us; unpadded unchanged).  A group's query blocks
  // stay on one XCD.  The last group is the last (b, h) slice either way.
  const int bh = p.bh0 + m / p.nqb;
  const int h = bh / p.B;
  const int b = bh - h * p.B;
  const int i0 = qblk * BM;
  const int i0w = i0 + wave * QW;
  const uint32_t sl_bytes = static_cast<uint32_t>(p.sl) * ES;

  // Buffer resources.  Rows past L read as zero; the bound is the end of row L-1.
  const uint32_t head_bytes = (static_cast<uint32_t>(L - 1) * static_cast<uint32_t>(p.sl) + D) * ES;
  const int64_t head_off = static_cast<int64_t>(b) * p.sb + static_cast<int64_t>(h) * p.sh;
  const auto rq = make_rsrc(reinterpret_cast<const T*>(p.q) + head_off, head_bytes);
  const auto rk = make_rsrc(reinterpret_cast<const T*>(p.k) + head_off, head_bytes);
  const auto rv = make_rsrc(reinterpret_cast<const T*>(p.v) + head_off, head_bytes);
  const auto rmask = make_rsrc(p.mask + static_cast<int64_t>(b) * L, static_cast<uint32_t>(L));
  const uint32_t rel_bytes = static_cast<uint32_t>(p.S) * D * ES;
  const auto rkr = make_rsrc(reinterpret_cast<const T*>(p.pos_key) + static_cast<int64_t>(h) * p.S * D,
                             rel_bytes);
  const auto rqr = make_rsrc(reinterpret_cast<const T*>(p.pos_query) + static_cast<int64_t>(h) * p.S * D,
                             rel_bytes);
  const auto rlut = make_rsrc(p.lut, static_cast<uint32_t>(2 * L - 1) * 4u);

  // ---- queries: fragments stay in registers (B operand of K.Q^T and Kr.Q^T) ----
  // They are loaded in the prologue, after the lookups and rows that the first
  // products wait for (loads return in issue order).
  QF qf[kQB][KD];
  bool qkept[kQB];

  // ---- padding extent (wavefront-uniform; every wavefront derives the same values) ----
  // A kept query attends to kept keys only, so the key loop of a workgroup
  // with kept queries ends at the 64-key tile holding the last kept key of the
  // sequence.  The loop always starts at key 0: the start is then known before
  // any mask byte arrives, the lookup and K/V loads of the first tiles are
  // issued without waiting for the scan, and the scan's loads are only waited
  // for at the first loop test.  (Leading padded keys are excluded by the
  // masking like any other padded key.)  A padded query in range attends
  // uniformly to all L keys: its output is the mean of V over the sequence,
  // which does not depend on the query and is computed separately (v_mean below).
  const int jstart = SPLIT ? split * p.split_tiles * BN : 0;

  // Mean of V over the L keys of (b, h) in fp32, left in LDS at vmean[0..D).
  float* vred = reinterpret_cast<float*>(smem);
  float* vmean = vred + kThreads * 8;
  auto v_mean = [&]() {
    constexpr int RG = kThreads / CPR;  // rows summed in parallel
    const int cc = tid % CPR;
    const int rg = tid / CPR;
    float acc[E16];
#pragma unroll
    for (int e = 0; e < E16; ++e) acc[e] = 0.0f;
    auto add_row = [&](u32x4_t raw) {
      const auto v = chunk_elems<T>(raw);
#pragma unroll
      for (int e = 0; e < E16; ++e) acc[e] += static_cast<float>(v[e]);
    };
    // Eight rows in flight per step; rows past L read as zero and add nothing.
    for (int j = rg; j < L; j += 8 * RG) {
      u32x4_t raw[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) raw[u] = load16(rv, static_cast<uint32_t>(j + u * RG) * sl_bytes + cc * 16);
#pragma unroll
      for (int u = 0; u < 8; ++u) add_row(raw[u]);
    }
    lds_barrier();  // LDS of the key loop no longer read
#pragma unroll
    for (int e = 0; e < E16; ++e) vred[tid * E16 + e] = acc[e];
    lds_barrier();
    if (tid < D) {
      const int col = tid / E16;
      const int e = tid % E16;
      float s = 0.0f;
      for (int r = 0; r < RG; ++r) s += vred[(r * CPR + col) * E16 + e];
      vmean[tid] = s / static_cast<float>(L);
    }
    lds_barrier();
  };

  T* outp = reinterpret_cast<T*>(p.out);
  const int64_t row_stride = static_cast<int64_t>(p.H) * D;

  // ---- per-thread offsets of the K / V tile loads (add j0 * row stride per tile) ----
  uint32_t koff[NCH];
  uint32_t kls[NCH];
#pragma unroll
  for (int n = 0; n < NCH; ++n) {
    const int t = tid + n * kThreads;
    const int r = t / CPR;
    const int cc = t - r * CPR;
    // Direct copies: LDS chunk t holds logical chunk cc ^ kv_swizzle(r) of row r.
    const int src = kDirect ? (cc ^ kv_swizzle<D>(r)) : cc;
    koff[n] = static_cast<uint32_t>(r) * sl_bytes + src * 16;
    kls[n] = static_cast<uint32_t>(r * LY::KS_LD + cc * E16);
  }
  // V chunks: the same rows and 16-byte chunks as K.
  uint32_t vls[NVB];
#pragma unroll
  for (int n = 0; n < NVB; ++n) {
    const int t = tid + n * kThreads;
    const int r = t / CPR;
    const int cc = t - r * CPR;
    vls[n] = static_cast<uint32_t>(r * LY::VS_LD + cc * E16);
  }

  // ---- relative windows ----
  // Tile at key offset j0: the wavefront's c2p window starts at delta
  // dlo_w = i0w - j0 - (BN - 1), the workgroup's p2c window at
  // dlo = i0 - j0 - (BN - 1); chunk k of a window covers deltas
  // [start + 16k, start + 16k + 15] and lane c loads the row of delta start + 16k + c.
  // The next tile's windows start BN = 16 * kSlide deltas lower, so its chunk k
  // is this tile's chunk k - kSlide:
  //   * c2p: chunks >= kSlide of the next tile are this tile's chunks < kCarry;
  //     their values (queries are fixed per wavefront) are kept in registers
  //     and only kSlide new chunks are multiplied per tile;
  //   * p2c: chunk pc belongs to wavefront pc % 4 and kSlide == 4, so every
  //     wavefront keeps its rows: per tile it loads one new chunk (pc = wave)
  //     and shifts the others up by 4 (the values depend on the keys and are
  //     recomputed).
  constexpr int kSlide = BN / 16;
  constexpr int kCarry = NCC - kSlide;
  static_assert(kSlide == kWaves, "p2c chunk ownership needs a window slide of kWaves chunks");
  static_assert(kCarry >= 0 && NPC % kWaves == 0, "window geometry");
  auto lut_c_index = [&](int j0, int ch) { return i0w - j0 - (BN - 1) + 16 * ch + c + L - 1; };
  auto lut_p_index = [&](int j0, int u) {
    return i0 - j0 - (BN - 1) + 16 * (wave + kWaves * u) + c + L - 1;
  };
  // Deltas outside [-(L-1), L-1] (index outside [0, 2L-2]) read as slot 0: the
  // unsigned min sends negative and too-large indices to 2L-1, the first
  // out-of-range entry of the buffer (a wrapped 32-bit offset is not reliably
  // out of range once the compiler folds constants into the instruction offset).
  const uint32_t lut_end = static_cast<uint32_t>(2 * L - 1);
  auto lut_load = [&](int index) {
    const uint32_t idx = min(static_cast<uint32_t>(index), lut_end);
    return static_cast<int>(load4(rlut, idx * 4u));
  };
  const uint32_t sub = (8 * g) * ES;
  auto row_frag = [&](__amdgpu_buffer_rsrc_t r, int slot, int kd) {
    return load_frag<T>(r, static_cast<uint32_t>(slot) * (D * ES) + 32 * kd * ES + sub);
  };

  int lutc[MC ? kSlide : 1];   // next tile's new c2p chunks
  int lutp = 0;                 // next tile's new p2c chunk (pc = wave)
  F crow[MC ? kSlide : 1][KD];  // rows of this tile's new c2p chunks
  Quad<T> ccar[MC && kCarry > 0 ? kCarry : 1][kQB];  // c2p values carried into chunks >= kSlide
  QF prow[MP ? PU : 1][KD];    // rows of this wavefront's p2c chunks wave + 4u
  // Fast fp32: prow is kept split; the chunk loaded at the end of a tile waits
  // here (unsplit, its load in flight) until the next tile's p2c products.
  F prow_in[SPLITQ && MP ? KD : 1];

  // ---- table form: the windows read from c2p / p2c tables [B, H, L, S] ----
  //   Cw[q][t]  = c2p[i0w + q][slot(dlo_w + t)],   Pw[jr][t] = p2c[j0 + jr][slot(dlo + t)],
  // the values the matrix unit computes in the other form (a table holds the
  // products Q.Kr / K.Qr rounded to T).  Lanes run along the delta axis, so one
  // load instruction reads consecutive slots of one or two table rows.  Element
  // e = lane + 64k of the wavefront's QW x NCW c2p window is (q, t) =
  // (e / NCW, e % NCW): t repeats with period TC_P in k while q advances by TC_R
  // per period, so a lane needs TC_P lookups per tile.  The p2c window (BN x NPW)
  // is split the same way over the workgroup's threads (e = tid + 256k).  The
  // values of tile n+1 are stored after barrier B of tile n+1 (every wavefront
  // is past its gathers of tile n then).  Its p2c values are loaded a whole tile
  // ahead, right after barrier B of tile n (lookups two tiles ahead); its c2p
  // values after the gathers of tile n (both early spill registers: 296 against
  // 153 us at C2).  `sel` picks the windows: bit 0 c2p, bit 1 p2c.
  constexpr int NCW = NCC * 16;
  constexpr int NPW = NPC * 16;
  constexpr bool TC = TABLE && C2P;
  constexpr bool TP = TABLE && P2C;
  constexpr int TC_P = TC ? NCW / std::gcd(64, NCW) : 1;
  constexpr int TC_R = TC ? 64 * TC_P / NCW : 0;
  constexpr int TC_N = TC ? QW * NCW / 64 : 1;
  constexpr int TP_P = TP ? NPW / std::gcd(kThreads, NPW) : 1;
  constexpr int TP_R = TP ? kThreads * TP_P / NPW : 0;
  constexpr int TP_N = TP ? BN * NPW / kThreads : 1;
  static_assert(!TC || (QW * NCW % 64 == 0 && TC_N % TC_P == 0), "c2p window in whole loads");
  static_assert(!TP || (BN * NPW % kThreads == 0 && TP_N % TP_P == 0), "p2c window in whole loads");
  using TW = std::conditional_t<sizeof(T) == 2, uint16_t, uint32_t>;
  const uint32_t row_bytes = static_cast<uint32_t>(p.S) * ES;  // one table row
  const int64_t tab_off = (static_cast<int64_t>(b) * p.H + h) * L * p.S;
  const auto rtc = make_rsrc(reinterpret_cast<const T*>(p.pos_key) + tab_off,
                             static_cast<uint32_t>(L) * row_bytes);
  const auto rtp = make_rsrc(reinterpret_cast<const T*>(p.pos_query) + tab_off,
                             static_cast<uint32_t>(L) * row_bytes);
  int tc_q[TC_P], tc_t[TC_P], tc_slot[TC_P];
  int tp_j[TP_P], tp_t[TP_P], tp_slot[TP_P];
#pragma unroll
  for (int pp = 0; pp < TC_P; ++pp) {
    const int e = lane + 64 * pp;
    tc_q[pp] = TC ? e / NCW : 0;
    tc_t[pp] = TC ? e % NCW : 0;
    tc_slot[pp] = 0;
  }
#pragma unroll
  for (int pp = 0; pp < TP_P; ++pp) {
    const int e = tid + kThreads * pp;
    tp_j[pp] = TP ? e / NPW : 0;
    tp_t[pp] = TP ? e % NPW : 0;
    tp_slot[pp] = 0;
  }
  TW tcv[TC_N];
  TW tpv[TP_N];
  // A lane reads rows r0 + m TC_R of one lookup's slot.  The range check of a
  // raw buffer covers voffset (and the instruction offset) but not soffset.
  // The fast form puts the row step in soffset (one address register per
  // lookup); a row past L then reads outside the (b, h) slice - inside the
  // tensor for every slice but the last, whose query blocks and key tiles
  // therefore run the ROWSAFE instance when L is not a multiple of the tile
  // (see launch_rel).  ROWSAFE carries the whole offset in voffset, so rows
  // past L read as zero; it costs address registers (spills), and runs only on
  // that one slice.
  auto load_tw = [](__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) -> TW {
    if constexpr (sizeof(T) == 2) {
      return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
    } else {
      return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    }
  };
  auto row_load = [&](__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t step) -> TW {
    if constexpr (ROWSAFE) {
      return load_tw(r, voff + step, 0);
    } else {
      return load_tw(r, voff, step);
    }
  };
  // Slots of the windows of the tile at key offset j0.  A lookup entry
  // outside [0, S) is clamped to S - 1: its value is undefined (as in the
  // reference), but its offset stays inside its table row, so that with the
  // row step in soffset (unchecked) no read leaves the tensor.
  const uint32_t slot_max = static_cast<uint32_t>(p.S - 1);
  auto table_lookups = [&](int j0, auto sel) {
    if constexpr (TC && (decltype(sel)::value & 1)) {
#pragma unroll
      for (int pp = 0; pp < TC_P; ++pp)
        tc_slot[pp] = static_cast<int>(
            min(static_cast<uint32_t>(lut_load(i0w - j0 - (BN - 1) + tc_t[pp] + L - 1)), slot_max));
    }
    if constexpr (TP && (decltype(sel)::value & 2)) {
#pragma unroll
      for (int pp = 0; pp < TP_P; ++pp)
        tp_slot[pp] = static_cast<int>(
            min(static_cast<uint32_t>(lut_load(i0 - j0 - (BN - 1) + tp_t[pp] + L - 1)), slot_max));
    }
  };
  // Window values of the tile at key offset j0 (slots from table_lookups(j0)).
  // Rows past L read as zero through the buffer bounds.
  auto table_load = [&](int j0, auto sel) {
    if constexpr (TC && (decltype(sel)::value & 1)) {
#pragma unroll
      for (int pp = 0; pp < TC_P; ++pp) {
        const uint32_t voff = static_cast<uint32_t>(tc_slot[pp]) * ES +
                              static_cast<uint32_t>(i0w + tc_q[pp]) * row_bytes;
#pragma unroll
        for (int m = 0; m < TC_N / TC_P; ++m)
          tcv[pp + TC_P * m] = row_load(rtc, voff, static_cast<uint32_t>(m * TC_R) * row_bytes);
      }
    }
    if constexpr (TP && (decltype(sel)::value & 2)) {
#pragma unroll
      for (int pp = 0; pp < TP_P; ++pp) {
        const uint32_t voff = static_cast<uint32_t>(tp_slot[pp]) * ES +
                              static_cast<uint32_t>(j0 + tp_j[pp]) * row_bytes;
#pragma unroll
        for (int m = 0; m < TP_N / TP_P; ++m)
          tpv[pp + TP_P * m] = row_load(rtp, voff, static_cast<uint32_t>(m * TP_R) * row_bytes);
      }
    }
  };
  auto table_store = [&]() {
    if constexpr (TC) {
      T* cw_w = Cw + wave * QW * LY::CW_LD;
#pragma unroll
      for (int pp = 0; pp < TC_P; ++pp) {
        T* dst = cw_w + tc_q[pp] * LY::CW_LD + tc_t[pp];
#pragma unroll
        for (int m = 0; m < TC_N / TC_P; ++m)
          dst[m * TC_R * LY::CW_LD] = __builtin_bit_cast(T, tcv[pp + TC_P * m]);
      }
    }
    if constexpr (TP) {
#pragma unroll
      for (int pp = 0; pp < TP_P; ++pp) {
        T* dst = Pw + tp_j[pp] * LY::PW_LD + tp_t[pp];
#pragma unroll
        for (int m = 0; m < TP_N / TP_P; ++m)
          dst[m * TP_R * LY::PW_LD] = __builtin_bit_cast(T, tpv[pp + TP_P * m]);
      }
    }
  };

  // ---- prefetch registers (K, V, mask of the next tile) ----
  u32x4_t pk[NCH];
  u32x4_t pv[NVB];
  uint8_t pmask = 0;
  auto prefetch_k_into = [&](int j0, u32x4_t (&dk)[NCH], uint8_t& dm) {
    const uint32_t jb = static_cast<uint32_t>(j0) * sl_bytes;
#pragma unroll
    for (int n = 0; n < NCH; ++n)
      if (NKC >= kThreads || tid < NKC) dk[n] = load16(rk, koff[n] + jb);
    dm = load1(rmask, static_cast<uint32_t>(j0 + lane));
  };
  auto prefetch_v_into = [&](int j0, u32x4_t (&dv)[NVB]) {
    const uint32_t jb = static_cast<uint32_t>(j0) * sl_bytes;
#pragma unroll
    for (int n = 0; n < NVB; ++n)
      if (NKC >= kThreads || tid < NKC) dv[n] = load16(rv, koff[n] + jb);
  };
  auto prefetch_k = [&](int j0) { prefetch_k_into(j0, pk, pmask); };
  // Direct copies of the K / V tile at key offset j0 into LDS (kDirect).
  auto copy_k = [&](int j0) {
    const uint32_t jb = static_cast<uint32_t>(j0) * sl_bytes;
#pragma unroll
    for (int n = 0; n < NCH; ++n)
      copy16_lds(rk, koff[n] + jb, smem + LY::ks_off + (n * kThreads + wave * 64) * 16);
  };
  auto copy_v = [&](int j0, T* vs) {
    const uint32_t jb = static_cast<uint32_t>(j0) * sl_bytes;
#pragma unroll
    for (int n = 0; n < NVB; ++n)
      copy16_lds(rv, koff[n] + jb, reinterpret_cast<unsigned char*>(vs) + (n * kThreads + wave * 64) * 16);
  };
  auto prefetch_v = [&](int j0) { prefetch_v_into(j0, pv); };

  // ---- staging and window helpers ----
  // K of tile n+1 is staged right after the p2c barrier of tile n (every
  // wavefront has finished reading K of tile n).  The V tile has two placements:
  //   * two buffers: V of tile n+1 goes into the other buffer at the same
  //     point, while tile n still reads its own;
  //   * one buffer: V of tile n is staged after the first barrier of tile n
  //     (every wavefront has finished PV of tile n-1) and read after the
  //     second, which halves its LDS.
  // Fast fp32: K and V are staged already split, as a bf16 hi plane followed by
  // a bf16 lo plane in the same bytes (element e of the fp32 tile at e in each
  // plane), so each value is split once per workgroup instead of once per
  // wavefront that reads it; a 16-byte chunk of 4 floats becomes 8 bytes in
  // each plane.
  auto split_chunk = [](const u32x4_t& raw, u32x2_t& hi, u32x2_t& lo) {
    const f32x4_t x = __builtin_bit_cast(f32x4_t, raw);
    bf16x4_t h, l;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = static_cast<__bf16>(x[e]);
      l[e] = static_cast<__bf16>(x[e] - static_cast<float>(h[e]));
    }
    hi = __builtin_bit_cast(u32x2_t, h);
    lo = __builtin_bit_cast(u32x2_t, l);
  };
  // Strict fp32 on the bf16 unit: the three planes of RelMmaExact (hi, mid, lo), each
  // BN rows of the tile's pitch, one after the other.
  auto split_chunk3 = [](const u32x4_t& raw, u32x2_t& hi, u32x2_t& mid, u32x2_t& lo) {
    const f32x4_t x = __builtin_bit_cast(f32x4_t, raw);
    bf16x4_t h, m, l;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = static_cast<__bf16>(x[e]);
      const float r = x[e] - static_cast<float>(h[e]);
      m[e] = static_cast<__bf16>(r);
      l[e] = static_cast<__bf16>(r - static_cast<float>(m[e]));
    }
    hi = __builtin_bit_cast(u32x2_t, h);
    mid = __builtin_bit_cast(u32x2_t, m);
    lo = __builtin_bit_cast(u32x2_t, l);
  };
  auto stage_k = [&]() {
#pragma unroll
    for (int n = 0; n < NCH; ++n)
      if (NKC >= kThreads || tid < NKC) {
        if constexpr (FAST) {
          __bf16* kh = reinterpret_cast<__bf16*>(Ks);
          u32x2_t hi, lo;
          split_chunk(pk[n], hi, lo);
          *reinterpret_cast<u32x2_t*>(kh + kls[n]) = hi;
          *reinterpret_cast<u32x2_t*>(kh + BN * LY::KS_LD + kls[n]) = lo;
        } else if constexpr (PL3) {
          __bf16* kh = reinterpret_cast<__bf16*>(Ks);
          u32x2_t hi, mid, lo;
          split_chunk3(pk[n], hi, mid, lo);
          *reinterpret_cast<u32x2_t*>(kh + kls[n]) = hi;
          *reinterpret_cast<u32x2_t*>(kh + BN * LY::KS_LD + kls[n]) = mid;
          *reinterpret_cast<u32x2_t*>(kh + 2 * BN * LY::KS_LD + kls[n]) = lo;
        } else {
          *reinterpret_cast<u32x4_t*>(Ks + kls[n]) = pk[n];
        }
      }
  };
  // Element offset in Ks of the 16-bit K fragment of key row `row` (a row
  // key_of(c) of a 16-key block), k-step kd: chunk 4 kd + g of the row.
  const int k_swz = kv_swizzle<D>(key_of(c));
  auto k_elem = [&](int row, int kd) -> int {
    if constexpr (kDirect) {
      return row * D + 8 * ((4 * kd + g) ^ k_swz);
    } else {
      return row * LY::KS_LD + 32 * kd + 8 * g;
    }
  };
  // Fast fp32: K fragment of key row `row`, k-step kd, from the split planes.
  auto k_read = [&](int row, int kd) -> QF {
    if constexpr (FAST) {
      const int off = row * LY::KS_LD + 32 * kd + 8 * g;
      const __bf16* kh = reinterpret_cast<const __bf16*>(Ks);
      return QF{*reinterpret_cast<const bf16x8_t*>(kh + off),
                *reinterpret_cast<const bf16x8_t*>(kh + BN * LY::KS_LD + off)};
    } else if constexpr (PL3) {
      const int off = row * LY::KS_LD + 32 * kd + 8 * g;
      const __bf16* kh = reinterpret_cast<const __bf16*>(Ks);
      return QF{*reinterpret_cast<const bf16x8_t*>(kh + off),
                *reinterpret_cast<const bf16x8_t*>(kh + BN * LY::KS_LD + off),
                *reinterpret_cast<const bf16x8_t*>(kh + 2 * BN * LY::KS_LD + off)};
    } else {
      return QF{};  // not used by the other instances
    }
  };
  // V rows of 16-bit T are 8-byte aligned only (VS_LD = D + 4): two 8-byte
  // stores per chunk (half a chunk = E16 / 2 elements each).
  auto stage_v = [&](T* vs) {
#pragma unroll
    for (int n = 0; n < NVB; ++n)
      if (NKC >= kThreads || tid < NKC) {
        if constexpr (FAST) {
          __bf16* vh = reinterpret_cast<__bf16*>(vs);
          u32x2_t hi, lo;
          split_chunk(pv[n], hi, lo);
          *reinterpret_cast<u32x2_t*>(vh + vls[n]) = hi;
          *reinterpret_cast<u32x2_t*>(vh + BN * LY::VS_LD + vls[n]) = lo;
        } else if constexpr (PL3) {
          __bf16* vh = reinterpret_cast<__bf16*>(vs);
          u32x2_t hi, mid, lo;
          split_chunk3(pv[n], hi, mid, lo);
          *reinterpret_cast<u32x2_t*>(vh + vls[n]) = hi;
          *reinterpret_cast<u32x2_t*>(vh + BN * LY::VS_LD + vls[n]) = mid;
          *reinterpret_cast<u32x2_t*>(vh + 2 * BN * LY::VS_LD + vls[n]) = lo;
        } else {
          *reinterpret_cast<u32x2_t*>(vs + vls[n]) = u32x2_t{pv[n][0], pv[n][1]};
          *reinterpret_cast<u32x2_t*>(vs + vls[n] + E16 / 2) = u32x2_t{pv[n][2], pv[n][3]};
        }
      }
  };

  // c2p window of a tile: the kSlide new chunks are multiplied from crow (the
  // products stay in registers until the previous tile's gathers are done),
  // the kCarry old ones come from ccar.
  Quad<T> cnew[MC ? kSlide : 1][kQB];
  auto c2p_products = [&]() {
    if constexpr (MC) {
      if constexpr (SPLITQ) {
        // Each row fragment split once for its kQB products.
#pragma unroll
        for (int ch = 0; ch < kSlide; ++ch) {
          QF cq[KD];
#pragma unroll
          for (int kd = 0; kd < KD; ++kd) cq[kd] = to_q(crow[ch][kd]);
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb) {
            f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kd = 0; kd < KD; ++kd) acc = M::run(cq[kd], qf[qb][kd], acc);
#pragma unroll
            for (int r = 0; r < 4; ++r) cnew[ch][qb][r] = static_cast<T>(acc[r]);
          }
        }
      } else {
#pragma unroll
        for (int ch = 0; ch < kSlide; ++ch)
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb) {
            f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kd = 0; kd < KD; ++kd) acc = M::run(crow[ch][kd], qf[qb][kd], acc);
#pragma unroll
            for (int r = 0; r < 4; ++r) cnew[ch][qb][r] = static_cast<T>(acc[r]);
          }
      }
    }
  };
  auto c2p_store = [&]() {
    if constexpr (MC) {
      T* cw_w = Cw + wave * QW * LY::CW_LD;
      // Queries of block qb meet window indices [16qb, 16qb + BN + 14]: chunks
      // outside [qb, qb + KB] are not stored (they are still multiplied when a
      // later tile needs them as carried chunks).
      auto needed = [](int ch, int qb) { return ch >= qb && ch <= qb + KB; };
#pragma unroll
      for (int ch = 0; ch < kSlide; ++ch)
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb)
          if (needed(ch, qb))
            *reinterpret_cast<Quad<T>*>(cw_w + (16 * qb + c) * LY::CW_LD + 16 * ch + 4 * g) =
                cnew[ch][qb];
#pragma unroll
      for (int ch = 0; ch < kCarry; ++ch)
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
          if (needed(kSlide + ch, qb))
            *reinterpret_cast<Quad<T>*>(cw_w + (16 * qb + c) * LY::CW_LD + 16 * (kSlide + ch) + 4 * g) =
                ccar[ch][qb];
          ccar[ch][qb] = cnew[ch][qb];
        }
    }
  };
  // Rows of the new c2p chunks of tile jt (lookups in lutc), then the lookups
  // of tile jt + BN.
  auto load_crow = [&](int jt) {
    if constexpr (MC) {
#pragma unroll
      for (int ch = 0; ch < kSlide; ++ch)
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) crow[ch][kd] = row_frag(rkr, lutc[ch], kd);
#pragma unroll
      for (int ch = 0; ch < kSlide; ++ch) lutc[ch] = lut_load(lut_c_index(jt + BN, ch));
    }
  };

  // ---- prologue: loads of tile 0, in the order their results are needed ----
  // Lookups first (they depend only on the block).
  table_lookups(jstart, IntC<3>{});
  int lc[MC ? NCC : 1];
  int lp[MP ? PU : 1];
  if constexpr (MC) {
#pragma unroll
    for (int ch = 0; ch < NCC; ++ch) lc[ch] = lut_load(lut_c_index(jstart, ch));
#pragma unroll
    for (int ch = 0; ch < kSlide; ++ch) lutc[ch] = lut_load(lut_c_index(jstart + BN, ch));
  }
  if constexpr (MP) {
#pragma unroll
    for (int u = 0; u < PU; ++u) lp[u] = lut_load(lut_p_index(jstart, u));
    lutp = lut_load(lut_p_index(jstart + BN, 0));
  }
  // Mask bytes: the first 512 of the sequence (for the extent), the
  // workgroup's queries and each lane's queries.  Bytes past L read as zero.
  uint8_t km[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) km[e] = load1(rmask, static_cast<uint32_t>(64 * e + lane));
  constexpr int kWgMaskLoads = (BM + 63) / 64;
  uint8_t wm[kWgMaskLoads];
#pragma unroll
  for (int n = 0; n < kWgMaskLoads; ++n)
    wm[n] = 64 * n + lane < BM ? load1(rmask, static_cast<uint32_t>(i0 + 64 * n + lane)) : 0;
  uint8_t qm[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) qm[qb] = load1(rmask, static_cast<uint32_t>(i0w + 16 * qb + c));

  // Workgroup and query flags from the mask bytes.
  bool wg_kept = false;
  bool wg_padded = false;
#pragma unroll
  for (int n = 0; n < kWgMaskLoads; ++n) {
    const bool mine = 64 * n + lane < BM;
    const bool kept = wm[n] != 0;
    wg_kept = wg_kept || __any(kept);
    wg_padded = wg_padded || __any(mine && i0 + 64 * n + lane < L && !kept);
  }
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) qkept[qb] = qm[qb] != 0;

  if (!wg_kept) {
    if (SPLIT && split > 0) return;  // split 0 stores the mean of V
    // Every query of the workgroup is padded (or past L): all rows are the mean of V.
    v_mean();
    const int row_lo = i0 + tid / (D / 4);
    for (int i = row_lo; i < min(i0 + BM, L); i += kThreads / (D / 4)) {
      const int d0 = 4 * (tid % (D / 4));
      Quad<T> q;
#pragma unroll
      for (int r = 0; r < 4; ++r) q[r] = static_cast<T>(vmean[d0 + r]);
      *reinterpret_cast<Quad<T>*>(outp + (static_cast<int64_t>(b) * L + i) * row_stride + h * D + d0) = q;
    }
    return;
  }

  // Rows of the tile-0 windows, then Q and the K/V of tile 0 (a workgroup
  // without kept queries has left before issuing them).
  table_load(jstart, IntC<3>{});
  table_lookups(jstart + BN, IntC<2>{});
  F r0[MC && kCarry > 0 ? kCarry : 1][KD];
  if constexpr (MC) {
#pragma unroll
    for (int ch = 0; ch < kSlide; ++ch)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) crow[ch][kd] = row_frag(rkr, lc[ch], kd);
#pragma unroll
    for (int ch = 0; ch < kCarry; ++ch)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) r0[ch][kd] = row_frag(rkr, lc[kSlide + ch], kd);
  }
  if constexpr (MP) {
#pragma unroll
    for (int u = 0; u < PU; ++u)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) prow[u][kd] = to_q(row_frag(rqr, lp[u], kd));
  }
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int i = i0w + 16 * qb + c;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd)
      qf[qb][kd] = to_q(load_frag<T>(rq, static_cast<uint32_t>(i) * sl_bytes + (32 * kd + 8 * g) * ES));
  }
  if constexpr (kDirect) {
    // Mask bytes first: the copies are waited for by counting the buffer
    // loads issued after them (kLoadsAfterCopies).
    pmask = load1(rmask, static_cast<uint32_t>(jstart + lane));
    memory_order_point();
    copy_k(jstart);
    if constexpr (VBUFS == 2) copy_v(jstart, Vt);
    memory_order_point();
  } else {
    prefetch_k(jstart);
    prefetch_v(jstart);
  }
  // Tile 1 (d = 64 only: d = 128 has no registers to spare here, and d = 32,
  // whose tiles are short, measured faster without it): K/V and the rows of
  // its new c2p chunks (lookups in lutc), moved into the pipeline registers
  // once tile 0 has been staged and multiplied.
  constexpr bool kEarlyTile1 = D == 64;
  u32x4_t pk1[NCH];
  u32x4_t pv1[NVB];
  uint8_t pmask1 = 0;
  F crow1[MC && kEarlyTile1 ? kSlide : 1][KD];
  if constexpr (kEarlyTile1 && kDirect) {
    pmask1 = load1(rmask, static_cast<uint32_t>(jstart + BN + lane));
  } else if constexpr (kEarlyTile1) {
    prefetch_k_into(jstart + BN, pk1, pmask1);
    if constexpr (VBUFS == 2) prefetch_v_into(jstart + BN, pv1);
  }
  if constexpr (MC && kEarlyTile1) {
#pragma unroll
    for (int ch = 0; ch < kSlide; ++ch)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) crow1[ch][kd] = row_frag(rkr, lutc[ch], kd);
  }

  // Last kept key (the loop bound) from the mask bytes loaded above.
  int klast = -1;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint64_t bits = __ballot(km[e] != 0);
    if (bits != 0) klast = 64 * e + 63 - __builtin_clzll(bits);
  }
  for (int base = 512; base < L; base += 512) {  // sequences longer than 512
#pragma unroll
    for (int e = 0; e < 8; ++e) km[e] = load1(rmask, static_cast<uint32_t>(base + 64 * e + lane));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint64_t bits = __ballot(km[e] != 0);
      if (bits != 0) klast = base + 64 * e + 63 - __builtin_clzll(bits);
    }
  }
  // A kept query's own key is kept: klast >= 0 when wg_kept.
  const int jend = SPLIT ? min(klast + 1, jstart + p.split_tiles * BN) : klast + 1;

  // ---- prologue: carried c2p chunks of tile 0 ----
  if constexpr (MC) {
#pragma unroll
    for (int ch = 0; ch < kCarry; ++ch)
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) acc = M::run(r0[ch][kd], qf[qb][kd], acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) ccar[ch][qb][r] = static_cast<T>(acc[r]);
      }
  }
  if constexpr (!kDirect) {
    stage_k();
    if constexpr (VBUFS == 2) stage_v(Vt);
  }
  uint64_t kept_cur = __ballot(pmask != 0);  // keys j0 + lane (zero past L)
  uint64_t kept_next = 0;
  c2p_products();
  c2p_store();
  if constexpr (kEarlyTile1) {
    if constexpr (!kDirect) {
#pragma unroll
      for (int n = 0; n < NCH; ++n) pk[n] = pk1[n];
    }
    pmask = pmask1;
    if constexpr (VBUFS == 2 && !kDirect) {
#pragma unroll
      for (int n = 0; n < NVB; ++n) pv[n] = pv1[n];
    }
    if constexpr (MC) {
#pragma unroll
      for (int ch = 0; ch < kSlide; ++ch) {
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) crow[ch][kd] = crow1[ch][kd];
        lutc[ch] = lut_load(lut_c_index(jstart + 2 * BN, ch));
      }
    }
  } else if constexpr (kDirect) {
    pmask = load1(rmask, static_cast<uint32_t>(jstart + BN + lane));
    load_crow(jstart + BN);
  } else {
    prefetch_k(jstart + BN);
    if constexpr (VBUFS == 2) prefetch_v(jstart + BN);
    load_crow(jstart + BN);
  }
  // Direct copies: buffer loads a wavefront issues after the K / V copies of
  // a tile and before the wait for them (at the top of the next tile): the
  // mask byte is issued before the copies, then come the c2p rows and
  // lookups of load_crow.  The prologue issues at least as many after its
  // copies.  (The table form waits for everything: its c2p table loads, issued
  // after the copies, are stored right after that barrier anyway.)  With one V buffer, V is copied after the first barrier of its
  // tile and waited for before the second; the p2c rows and lookup are
  // issued in between.
  constexpr int kLoadsAfterCopies = MC ? kSlide * (KD + 1) : 0;
  constexpr int kLoadsAfterV = MP ? KD + 1 : 0;
  static_assert(!kDirect || sizeof(T) == 2, "one buffer load per row fragment");

  // ---- accumulators ----
  f32x4_t o[DB][kQB];
  // Row sums: MFMA form (all four entries equal) or this lane's part (entry 0:
  // its keys g + 4r of every block), see kRowSumValu.
  constexpr bool kRowSumValu = D >= 128 || sizeof(T) == 4;
  f32x4_t rs[kQB];
  float row_max[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    row_max[qb] = -INFINITY;
    rs[qb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db][qb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Lane-constant LDS bases of the score gathers.  Element (qb, kb, r) of the
  // tile (query 16*qb + c, key 16*kb + g + 4*r) has c2p window index
  // 16*qb + c - (16*kb + g + 4*r) + BN - 1 in the wavefront's window, and p2c
  // index QW*wave + that in the workgroup's.
  constexpr int kMinOff = -(16 * (KB - 1) + 12);
  const T* cw_lane = Cw + (wave * QW + c) * LY::CW_LD + c - g + BN - 1 + kMinOff;
  const T* pw_lane = Pw + g * LY::PW_LD + QW * wave + c - g + BN - 1 + kMinOff;
  const float scale = p.scale_log2;
  const F ones = ones_frag<T>();
  const int v_swz = kv_swizzle<D>(4 * (c >> 2) + g);

  // Per tile: barrier B (K/V staged, previous gathers done) -> QK, p2c window;
  // barrier C (p2c window complete, K tile consumed) -> stage the next K/V,
  // gathers, softmax, PV, next c2p window.
  int vbuf = 0;
  for (int j0 = jstart; j0 < jend; j0 += BN) {
    const int jn = j0 + BN;
    if constexpr (kDirect) wait_vmem<kLoadsAfterCopies>();  // K (and V) of this tile in LDS
    lds_barrier();
    if constexpr (VBUFS == 1 && kDirect) {
      memory_order_point();
      copy_v(j0, Vt);
      memory_order_point();
    } else if constexpr (VBUFS == 1) {
      stage_v(Vt);
      prefetch_v(SPLIT && jn >= jend ? L : jn);
    }
    // Table form: windows of this tile into LDS; p2c values of the next tile,
    // p2c lookups of the one after, c2p lookups of the next.
    table_store();
    table_load(jn, IntC<2>{});
    table_lookups(jn + BN, IntC<2>{});
    table_lookups(jn, IntC<1>{});

    // ---- S^T = K . Q^T and the p2c window Pw[jr][t] = Qr[slot(dlo + t)] . K_jr ----
    f32x4_t sc[KB][kQB];
    // For d <= 64, and d = 128 on the 32-row tile (512 registers per lane), one
    // straight-line copy per wavefront index, so that the chunks a wavefront
    // skips are known at compile time and the MFMAs of the whole phase form one
    // scheduling region (d = 128, C5: 75.8 -> 72.1 us).  The 16-row d = 128
    // tile keeps one copy with runtime skips (below): with four copies it runs
    // out of its 256 registers.
    auto qk_p2c = [&](auto wave_c) {
      constexpr int W = decltype(wave_c)::value;
      // K fragments one key block ahead (two register sets), so that the
      // reads of block kb + 1 are in flight during the MFMAs of block kb.
      QF kfa[2][KD];
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        if constexpr (kPlanes) {
          kfa[0][kd] = k_read(key_of(c), kd);
        } else {
          kfa[0][kd] = to_q(*reinterpret_cast<const F*>(Ks + k_elem(key_of(c), kd)));
        }
      }
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        QF kf[KD];
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) kf[kd] = kfa[kb & 1][kd];
        if (kb + 1 < KB) {
#pragma unroll
          for (int kd = 0; kd < KD; ++kd) {
            if constexpr (kPlanes) {
              kfa[(kb + 1) & 1][kd] = k_read(16 * (kb + 1) + key_of(c), kd);
            } else {
              kfa[(kb + 1) & 1][kd] = to_q(*reinterpret_cast<const F*>(Ks + k_elem(16 * (kb + 1) + key_of(c), kd)));
            }
          }
        }
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
          f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kd = 0; kd < KD; ++kd) acc = M::run(kf[kd], qf[qb][kd], acc);
          sc[kb][qb] = acc;
        }
        if constexpr (MP) {
          // Keys of block kb meet window indices [BN - 16(kb+1), BM + BN - 2 - 16kb]:
          // chunks outside [KB-1-kb, (BM+BN-2)/16 - kb] are read by no score element.
#pragma unroll
          for (int u = 0; u < PU; ++u) {
            const int pc = W + kWaves * u;
            if (pc < KB - 1 - kb || pc > (BM + BN - 2) / 16 - kb) continue;
            f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kd = 0; kd < KD; ++kd) acc = M::run(prow[u][kd], kf[kd], acc);
            store4<T>(Pw + (16 * kb + key_of(c)) * LY::PW_LD + 16 * pc + 4 * g, acc);
          }
        }
      }
    };
    if constexpr (SPLITQ && MP) {
      if (j0 != jstart) {
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) prow[0][kd] = to_q(prow_in[kd]);
      }
    }
    if constexpr (D <= 64 || QW == 32) {
      switch (wave) {
        case 0: qk_p2c(IntC<0>{}); break;
        case 1: qk_p2c(IntC<1>{}); break;
        case 2: qk_p2c(IntC<2>{}); break;
        default: qk_p2c(IntC<3>{}); break;
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        QF kf[KD];
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) {
          if constexpr (kPlanes) {
            kf[kd] = k_read(16 * kb + key_of(c), kd);
          } else {
            kf[kd] = to_q(*reinterpret_cast<const F*>(Ks + k_elem(16 * kb + key_of(c), kd)));
          }
        }
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
          f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kd = 0; kd < KD; ++kd) acc = M::run(kf[kd], qf[qb][kd], acc);
          sc[kb][qb] = acc;
        }
        if constexpr (MP) {
#pragma unroll
          for (int u = 0; u < PU; ++u) {
            const int pc = wave + kWaves * u;
            if (pc < KB - 1 - kb || pc > (BM + BN - 2) / 16 - kb) continue;
            f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kd = 0; kd < KD; ++kd) acc = M::run(prow[u][kd], kf[kd], acc);
            store4<T>(Pw + (16 * kb + key_of(c)) * LY::PW_LD + 16 * pc + 4 * g, acc);
          }
        }
      }
    }
    if constexpr (MP) {
      // Next tile's p2c rows: shift the kept chunks up by 4, load the new one.
#pragma unroll
      for (int u = PU - 1; u > 0; --u)
#pragma unroll
        for (int kd = 0; kd < KD; ++kd) prow[u][kd] = prow[u - 1][kd];
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        if constexpr (SPLITQ) {
          prow_in[kd] = row_frag(rqr, lutp, kd);
        } else {
          prow[0][kd] = row_frag(rqr, lutp, kd);
        }
      }
      lutp = lut_load(lut_p_index(jn + BN, 0));
    }
    if constexpr (kDirect && VBUFS == 1) wait_vmem<kLoadsAfterV>();  // V of this tile in LDS
    lds_barrier();

    // ---- stage the next tile; its c2p products overlap this tile's softmax ----
    // Next-tile work runs unconditionally (no branch splits the scheduling
    // region): past the last tile the buffer loads read zeros and the LDS
    // writes land in buffers nothing reads any more.
    const T* vt_cur = Vt + (VBUFS == 2 ? vbuf * LY::VT_SIZE : 0);
    // A split's tiles past its range are redirected past L: the buffer loads
    // then return zeros without touching memory.
    const int jpre = SPLIT && jn + BN >= jend ? L : jn + BN;
    if constexpr (kDirect) {
      kept_next = __ballot(pmask != 0);
      pmask = load1(rmask, static_cast<uint32_t>(jpre + lane));
      memory_order_point();
      const int jcopy = SPLIT && jn >= jend ? L : jn;
      copy_k(jcopy);
      if constexpr (VBUFS == 2) copy_v(jcopy, Vt + (vbuf ^ 1) * LY::VT_SIZE);
      memory_order_point();
    } else {
      stage_k();
      if constexpr (VBUFS == 2) stage_v(Vt + (vbuf ^ 1) * LY::VT_SIZE);
      kept_next = __ballot(pmask != 0);
      prefetch_k(jpre);
      if constexpr (VBUFS == 2) prefetch_v(jpre);
    }
    c2p_products();

    // ---- relative scores ----
    if constexpr (C2P && P2C) {
      // All 32 reads of a query block first, then the adds: written element by
      // element, the compiler interleaved read, wait and add and left most of
      // the LDS latency exposed.
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        T cvs[KB][4], pvs[KB][4];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int off = 16 * (qb - kb) - 4 * r - kMinOff;
            cvs[kb][r] = cw_lane[16 * qb * LY::CW_LD + off];
            pvs[kb][r] = pw_lane[(16 * kb + 4 * r) * LY::PW_LD + off];
          }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[kb][qb][r] = add2<T>(sc[kb][qb][r], cvs[kb][r], pvs[kb][r]);
      }
    } else if constexpr (C2P || P2C) {
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        T vals[KB][4];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int off = 16 * (qb - kb) - 4 * r - kMinOff;
            vals[kb][r] = C2P ? cw_lane[16 * qb * LY::CW_LD + off]
                              : pw_lane[(16 * kb + 4 * r) * LY::PW_LD + off];
          }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[kb][qb][r] += static_cast<float>(vals[kb][r]);
      }
    }

    table_load(jn, IntC<1>{});

    // ---- masking (wavefront-uniform slow path: tiles with a padded key or past L) ----
    // Every row drops the padded keys.  That is the rule for kept queries; the
    // other rows are never stored from the accumulators (a padded query in
    // range takes the mean of V, a query past L is not stored), so they only
    // have to stay finite or empty, which they do: every row of a workgroup
    // with a kept query meets at least one kept key.
    constexpr uint64_t kTileBits = BN == 64 ? ~uint64_t{0} : (uint64_t{1} << (BN % 64)) - 1;
    const bool full_tile = (j0 + BN <= L) && (kept_cur & kTileBits) == kTileBits;
    if (__builtin_expect(!full_tile, 0)) {
      // (The empty asm keeps this a branch: if-converted, the selects would
      // run on every tile.)
      asm volatile("");
      const uint64_t lane_bits = kept_cur >> g;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool key_kept = (lane_bits >> (16 * kb + 4 * r)) & 1;
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb) sc[kb][qb][r] = key_kept ? sc[kb][qb][r] : -INFINITY;
        }
    }

    // PV operands (V^T through transposing reads).  For d = 128 with both
    // relative terms all of them are read before the softmax so that their LDS
    // latency hides under it (93.9 -> 89.3 us on the C5 shape); with one term,
    // or for d <= 64, that cost more registers than it saved (+2-5 %), and they
    // are read next to their MFMAs.
    // Fast fp32: the transposing read of the 16-bit path (below) on one plane
    // of the split V tile.
    auto vt_tr16 = [&](const void* tile, int ks, int db) -> u32x4_t {
      const uint16_t* base = static_cast<const uint16_t*>(tile);
      const uint16_t* p_lo = base + (32 * ks + 4 * (c >> 2) + g) * LY::VS_LD + 16 * db + 4 * (c & 3);
      const uint16_t* p_hi = p_lo + 16 * LY::VS_LD;
      const u32x2_t lo = __builtin_bit_cast(
          u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)p_lo));
      const u32x2_t hi = __builtin_bit_cast(
          u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)p_hi));
      return u32x4_t{lo[0], lo[1], hi[0], hi[1]};
    };
    // Element offset in the V tile of lane (c, g)'s 8 bytes of row `row`
    // (4 (c >> 2) + g of a 16-row group), columns 16 db + 4 (c & 3) .. + 3.
    auto v_elem = [&](int row, int db) -> int {
      if constexpr (kDirect) {
        return row * D + 8 * ((2 * db + ((c & 3) >> 1)) ^ v_swz) + 4 * (c & 1);
      } else {
        return row * LY::VS_LD + 16 * db + 4 * (c & 3);
      }
    };
    auto vt_frag = [&](int ks, int db) -> QF {
      if constexpr (FAST) {
        // The P^T key order of the 16-bit path is the fp32 one (below), so the
        // transposing reads of the two planes give the split operand directly.
        const __bf16* vh = reinterpret_cast<const __bf16*>(vt_cur);
        return QF{__builtin_bit_cast(bf16x8_t, vt_tr16(vh, ks, db)),
                  __builtin_bit_cast(bf16x8_t, vt_tr16(vh + BN * LY::VS_LD, ks, db))};
      } else if constexpr (PL3) {
        const __bf16* vh = reinterpret_cast<const __bf16*>(vt_cur);
        return QF{__builtin_bit_cast(bf16x8_t, vt_tr16(vh, ks, db)),
                  __builtin_bit_cast(bf16x8_t, vt_tr16(vh + BN * LY::VS_LD, ks, db)),
                  __builtin_bit_cast(bf16x8_t, vt_tr16(vh + 2 * BN * LY::VS_LD, ks, db))};
      } else if constexpr (sizeof(T) == 4) {
        // fp32: element e holds V[key][16db + c] for the keys of the P^T
        // operand, 32ks + g + 4e (e < 4) and 32ks + 16 + g + 4(e - 4).
        F a;
        const T* col = vt_cur + 16 * db + c;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          a[e] = col[(32 * ks + (e < 4 ? 0 : 16) + g + 4 * (e & 3)) * LY::VS_LD];
        return to_q(a);
      } else {
        // Lane c of group g supplies row 32ks + 4(c>>2) + g (+16 for the upper
        // half), columns 16db + 4(c&3) .. +3, and receives V[rows of its
        // k-slice][16db + c] -- keys g + 4e and 16 + g + 4e, the order of the P^T
        // operand.  The result is moved as whole dwords: assembling the operand
        // from its 16-bit elements was compiled into wrong code.
        const T* p_lo = vt_cur + v_elem(32 * ks + 4 * (c >> 2) + g, db);
        const T* p_hi = p_lo + 16 * LY::VS_LD;
        const u32x2_t lo = __builtin_bit_cast(
            u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)p_lo));
        const u32x2_t hi = __builtin_bit_cast(
            u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)p_hi));
        return __builtin_bit_cast(F, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
      }
    };
    constexpr bool kVtEarly = D >= 128 && !SPLIT && !TABLE && C2P && P2C && !EXACT;
    QF vt_all[kVtEarly ? BN / 32 : 1][kVtEarly ? DB : 1];
    if constexpr (kVtEarly) {
#pragma unroll
      for (int ks = 0; ks < BN / 32; ++ks)
#pragma unroll
        for (int db = 0; db < DB; ++db) vt_all[ks][db] = vt_frag(ks, db);
    }

    // ---- online softmax (exp2, stale maximum) ----
    // The exponent base only has to be common to a row and keep exp2 finite,
    // so the previous maximum is reused while no scaled score exceeds it by
    // more than kSlack; only then is the maximum reduced across lanes and the
    // accumulators rescaled.  Wavefront-uniform branch.
    constexpr float kSlack = 8.0f;
    float lane_max_s[kQB];
    bool grow = false;
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      float lane_max = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) lane_max = fmaxf(lane_max, sc[kb][qb][r]);
      lane_max_s[qb] = lane_max * scale;
      grow = grow || lane_max_s[qb] > row_max[qb] + kSlack;
    }
    // One wavefront-uniform branch for all query blocks, so that the common
    // path (no rescale) is a single scheduling region.
    if (__any(grow)) {
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        float tile_max = fmaxf(lane_max_s[qb], __shfl_xor(lane_max_s[qb], 16));
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
        const float new_max = fmaxf(row_max[qb], tile_max);
        const float old_base = row_max[qb] == -INFINITY ? 0.0f : row_max[qb];
        const float new_base = new_max == -INFINITY ? 0.0f : new_max;
        const float corr = __builtin_amdgcn_exp2f(old_base - new_base);
        row_max[qb] = new_max;
        rs[qb] *= corr;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db][qb] *= corr;
      }
    }
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      const float neg_base = row_max[qb] == -INFINITY ? 0.0f : -row_max[qb];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sc[kb][qb][r] = __builtin_amdgcn_exp2f(fmaf(sc[kb][qb][r], scale, neg_base));
    }

    // ---- O^T += V^T . P^T, row sums += 1 . P^T ----
#pragma unroll
    for (int ks = 0; ks < BN / 32; ++ks) {
      F pf[kQB];
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pf[qb][r] = static_cast<T>(sc[2 * ks][qb][r]);
          pf[qb][4 + r] = static_cast<T>(sc[2 * ks + 1][qb][r]);
        }
        // Row sums of the rounded probabilities (the values PV multiplies).
        if constexpr (kRowSumValu && sizeof(T) == 4) {
#pragma unroll
          for (int e = 0; e < 8; ++e) rs[qb][0] += pf[qb][e];
        } else if constexpr (kRowSumValu) {
          const u32x4_t pp = __builtin_bit_cast(u32x4_t, pf[qb]);
#pragma unroll
          for (int e = 0; e < 4; ++e) rs[qb][0] = sum2<T>(rs[qb][0], pp[e]);
        } else {
          rs[qb] = M::run(ones, pf[qb], rs[qb]);
        }
      }
      if constexpr (SPLITQ) {
        // P split once for its DB products; V^T comes split (from the planes,
        // or split where it is read).
        QF pq[kQB];
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) pq[qb] = to_q(pf[qb]);
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          QF a;
          if constexpr (kVtEarly) {
            a = vt_all[ks][db];
          } else {
            a = vt_frag(ks, db);
          }
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb) o[db][qb] = M::run(a, pq[qb], o[db][qb]);
        }
      } else {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          F a;
          if constexpr (kVtEarly) {
            a = vt_all[ks][db];
          } else {
            a = vt_frag(ks, db);
          }
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb) o[db][qb] = M::run(a, pf[qb], o[db][qb]);
        }
      }
    }

    // ---- next tile's c2p window (after this tile's gathers), its next rows ----
    c2p_store();
    load_crow(jn + BN);
    kept_cur = kept_next;
    vbuf ^= 1;
  }
  // The last tile's copies (of a tile past the end) land before LDS is reused.
  if constexpr (kDirect) wait_vmem<0>();

  // ---- normalise and store [B, L, H*D]; padded rows take the mean of V ----
  float row_sum[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    row_sum[qb] = rs[qb][0];
    if constexpr (kRowSumValu) {
      row_sum[qb] += __shfl_xor(row_sum[qb], 16);
      row_sum[qb] += __shfl_xor(row_sum[qb], 32);
    }
  }
  if constexpr (SPLIT) {
    // Partial rows of this key split: unnormalised O, the exponent base and
    // the row sum (the merge kernel combines the splits of kept rows).  Split 0
    // also stores the padded rows, which do not depend on the keys.
    if (split == 0 && wg_padded) v_mean();
    const int64_t rows = static_cast<int64_t>(p.B) * L * p.H;
    float* part_o = p.part;
    float2* part_ml = reinterpret_cast<float2*>(p.part + static_cast<int64_t>(p.splits) * rows * D);
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      const int i = i0w + 16 * qb + c;
      if (i >= L) continue;
      const int64_t row = (static_cast<int64_t>(split) * p.B + b) * L * p.H +
                          static_cast<int64_t>(i) * p.H + h;
      if (qkept[qb]) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
          *reinterpret_cast<f32x4_t*>(part_o + row * D + 16 * db + 4 * g) = o[db][qb];
        if (g == 0) part_ml[row] = float2{row_max[qb], row_sum[qb]};
      } else if (split == 0) {
        T* dst = outp + (static_cast<int64_t>(b) * L + i) * row_stride + h * D + 4 * g;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          Quad<T> q;
#pragma unroll
          for (int r = 0; r < 4; ++r) q[r] = static_cast<T>(vmean[16 * db + 4 * g + r]);
          *reinterpret_cast<Quad<T>*>(dst + 16 * db) = q;
        }
      }
    }
    return;
  }
  if (wg_padded) v_mean();
  if constexpr (sizeof(T) == 2 && D <= 64) {
    // Output rows through LDS: each wavefront writes its QW x D tile (row pitch
    // D + 8) into its share of the K/V buffers, then stores whole rows of the
    // head, 16 bytes per lane, instead of 8-byte pieces of 16 rows per store
    // (C2 88.8 -> 87.4 us).  d = 128 keeps the direct stores: the staged form
    // needs registers it does not have (91 -> 105 us).
    constexpr int OPITCH = D + 8;
    static_assert(kWaves * QW * OPITCH * sizeof(T) <= LY::pw_off, "output staging fits K/V");
    // Values first (the padded rows read vmean, which lies in the staging area).
    Quad<T> qv[kQB][DB];
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      const float inv = 1.0f / row_sum[qb];
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        if (qkept[qb]) {
#pragma unroll
          for (int r = 0; r < 4; ++r) qv[qb][db][r] = static_cast<T>(o[db][qb][r] * inv);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) qv[qb][db][r] = static_cast<T>(vmean[16 * db + 4 * g + r]);
        }
      }
    }
    lds_barrier();  // K/V buffers and vmean no longer read by any wavefront
    T* stg = reinterpret_cast<T*>(smem) + wave * QW * OPITCH;
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb)
#pragma unroll
      for (int db = 0; db < DB; ++db)
        *reinterpret_cast<Quad<T>*>(stg + (16 * qb + c) * OPITCH + 16 * db + 4 * g) = qv[qb][db];
    constexpr int CPRO = D / 8;                    // 16-byte chunks per output row
    constexpr int ROUNDS = QW * CPRO / 64;
    static_assert(QW * CPRO % 64 == 0, "whole rounds of chunks");
    typedef T Oct __attribute__((ext_vector_type(8)));
#pragma unroll
    for (int k = 0; k < ROUNDS; ++k) {
      const int q = lane + 64 * k;
      const int row = q / CPRO;
      const int ch = q - row * CPRO;
      const Oct v = *reinterpret_cast<const Oct*>(stg + row * OPITCH + 8 * ch);
      const int i = i0w + row;
      if (i < L)
        *reinterpret_cast<Oct*>(outp + (static_cast<int64_t>(b) * L + i) * row_stride + h * D + 8 * ch) = v;
    }
  } else {
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      const int i = i0w + 16 * qb + c;
      if (i >= L) continue;
      const float inv = 1.0f / row_sum[qb];
      T* dst = outp + (static_cast<int64_t>(b) * L + i) * row_stride + h * D + 4 * g;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        Quad<T> q;
        if (qkept[qb]) {
#pragma unroll
          for (int r = 0; r < 4; ++r) q[r] = static_cast<T>(o[db][qb][r] * inv);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) q[r] = static_cast<T>(vmean[16 * db + 4 * g + r]);
        }
        *reinterpret_cast<Quad<T>*>(dst + 16 * db) = q;
      }
    }
  }
}

namespace {

// Tile configuration: QW query rows per wavefront (32 for d <= 64, 16 for
// d = 128 to stay within 256 registers at two wavefronts per SIMD; 16 is also
// built for d <= 64, for grids that leave CUs idle, see rel_attention_qw), keys
// per tile BN, V tile buffers in LDS and workgroups per CU the registers are
// budgeted for.
template <int D>
constexpr int rel_block_n() {
  return 64;
}
// d = 128 on the 16-row tile keeps one V buffer so that two workgroups fit in
// the LDS of a CU (65 KB each instead of 82 KB): 153 -> 117 us at B=16, L=512,
// H=8, fp16; the 32-row tile (one workgroup per CU) takes two.  For d <= 64 at
// QW = 32 (two workgroups either way) both placements time the same; at
// QW = 16 one buffer lets three workgroups share a CU (48 KB each).  fp32
// (twice the LDS per element) runs one workgroup per CU with up to 512
// registers per lane: two V buffers except at d = 128 and where the three bf16
// planes of K and V need the room (strict, d = 64).
template <typename T, int D, int QW, bool FAST, bool C2P>
constexpr int rel_v_buffers() {
  if constexpr (rel_kv_planes3<T, D, FAST, C2P>() && D == 64) return 1;
  return ((D >= 128 && QW == 16) || (QW == 16 && sizeof(T) == 2)) ? 1 : 2;
}
template <typename T, int D, int QW>
constexpr int rel_workgroups_per_cu() {
  if constexpr (sizeof(T) == 4 || (D >= 128 && QW == 32)) return 1;
  return (D <= 64 && QW == 16) ? 3 : 2;
}

constexpr int kMaxKeySplits = 8;

// Merge of the key splits: per kept row (b, i, h), 4 output elements per thread,
//   o = sum_s 2^(base_s - M) O_s / sum_s 2^(base_s - M) l_s,  M = max_s base_s
// (a split that met no kept key has base -inf and l = 0, so weight 0).
template <typename T>
__global__ __launch_bounds__(256) void rel_split_merge_kernel(const float* __restrict__ part,
                                                              const uint8_t* __restrict__ mask,
                                                              T* __restrict__ out, int64_t rows,
                                                              int H, int D, int splits) {
  const int per_row = D / 4;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = t / per_row;
  if (row >= rows) return;
  if (mask[row / H] == 0) return;  // padded query: stored by split 0
  const int d0 = 4 * static_cast<int>(t - row * per_row);
  const float2* ml = reinterpret_cast<const float2*>(part + static_cast<int64_t>(splits) * rows * D);
  // All loads first (at most eight splits), then one pass.
  float2 v[kMaxKeySplits];
  f32x4_t po[kMaxKeySplits];
#pragma unroll
  for (int sp = 0; sp < kMaxKeySplits; ++sp) {
    if (sp < splits) {
      v[sp] = ml[sp * rows + row];
      po[sp] = *reinterpret_cast<const f32x4_t*>(part + (sp * rows + row) * D + d0);
    }
  }
  float base = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < kMaxKeySplits; ++sp)
    if (sp < splits) base = fmaxf(base, v[sp].x);
  float l = 0.0f;
  f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < kMaxKeySplits; ++sp) {
    if (sp < splits) {
      const float w = __builtin_amdgcn_exp2f(v[sp].x - base);
      l += w * v[sp].y;
      acc += w * po[sp];
    }
  }
  const float inv = 1.0f / l;
  Quad<T> q;
#pragma unroll
  for (int r = 0; r < 4; ++r) q[r] = static_cast<T>(acc[r] * inv);
  *reinterpret_cast<Quad<T>*>(out + row * D + d0) = q;
}

template <typename T, int D, int QW, bool C2P, bool P2C, bool FAST = false, bool TABLE = false>
int launch_rel(const RelParams& base, hipStream_t stream) {
  constexpr int BN = rel_block_n<D>();
  constexpr int VB = rel_v_buffers<T, D, QW, FAST, C2P>();
  constexpr int WGS = rel_workgroups_per_cu<T, D, QW>();
  using LY = RelLayout<T, D, QW, BN, VB, rel_kv_direct<T, D, VB, TABLE, P2C>(),
                       rel_kv_planes3<T, D, FAST, C2P>()>;
  RelParams prm = base;
  prm.nqb = (prm.L + LY::BM - 1) / LY::BM;
  // The split-key form exists for the default 16-bit tile (QW = 32 at d <= 64,
  // 16 at d = 128); fp32 never splits.
  constexpr bool kSplitBuilt = sizeof(T) == 2 && (D >= 128 ? QW == 16 : QW == 32) && !TABLE;
  constexpr auto kernel = rel_attention_kernel<T, D, QW, BN, VB, WGS, C2P, P2C, false, FAST, TABLE>;
  if (prm.splits < 1) prm.splits = 1;
  if (!kSplitBuilt && prm.splits > 1) return DFLASH_ERR_SHAPE;
  hipError_t err = hipSuccess;
  const int64_t blocks = static_cast<int64_t>(prm.nqb) * prm.B * prm.H * prm.splits;
  if (blocks > 0x7fffffff) return DFLASH_ERR_TOO_LARGE;
  if constexpr (kSplitBuilt) {
    constexpr auto split_kernel = rel_attention_kernel<T, D, QW, BN, VB, WGS, C2P, P2C, true>;
    if (prm.splits > 1) {
      err = ensure_dynamic_lds<split_kernel>(static_cast<int>(LY::bytes));
      if (err != hipSuccess) return static_cast<int>(err);
      hipLaunchKernelGGL(split_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                         LY::bytes, stream, prm);
    }
  }
  if (prm.splits <= 1) {
    err = ensure_dynamic_lds<kernel>(static_cast<int>(LY::bytes));
    if (err != hipSuccess) return static_cast<int>(err);
    // Table form with L not a multiple of the tiles: the last (b, h) slice,
    // whose rows past L would read past the end of the tables, runs the
    // ROWSAFE instance (see the kernel).
    const int64_t groups = static_cast<int64_t>(prm.B) * prm.H;
    const bool tail = TABLE && groups > 0 && (prm.L % LY::BM != 0 || prm.L % BN != 0);
    const int64_t fast_blocks = tail ? blocks - prm.nqb : blocks;
    if (fast_blocks > 0) {
      hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(fast_blocks)), dim3(kThreads), LY::bytes,
                         stream, prm);
    }
    if constexpr (TABLE) {
      if (tail) {
        constexpr auto safe_kernel =
            rel_attention_kernel<T, D, QW, BN, VB, WGS, C2P, P2C, false, FAST, TABLE, true>;
        err = ensure_dynamic_lds<safe_kernel>(static_cast<int>(LY::bytes));
        if (err != hipSuccess) return static_cast<int>(err);
        RelParams last = prm;
        last.bh0 = static_cast<int>(groups - 1);
        hipLaunchKernelGGL(safe_kernel, dim3(static_cast<unsigned>(prm.nqb)), dim3(kThreads),
                           LY::bytes, stream, last);
      }
    }
  }
  err = hipGetLastError();
  if (err != hipSuccess || prm.splits == 1) return static_cast<int>(err);
  const int64_t rows = static_cast<int64_t>(prm.B) * prm.L * prm.H;
  const int64_t threads = rows * (D / 4);
  hipLaunchKernelGGL(rel_split_merge_kernel<T>, dim3(static_cast<unsigned>((threads + 255) / 256)),
                     dim3(256), 0, stream, static_cast<const float*>(prm.part), prm.mask,
                     static_cast<T*>(prm.out), rows, prm.H, D, prm.splits);
  return static_cast<int>(hipGetLastError());
}

template <typename T, int D, int QW, bool FAST = false>
int rel_modes_qw(const RelParams& prm, hipStream_t stream) {
  if constexpr (sizeof(T) == 4 && !FAST) {
    if (prm.fast) return rel_modes_qw<T, D, QW, true>(prm, stream);
  }
  // Table form: the default tile of each head dim, 16-bit or fp32 (IEEE, or
  // the bf16x3 products of the fast form for QK and PV).
  if constexpr (QW == (D >= 128 ? 16 : 32)) {
    if (prm.table) {
      if (prm.has_c2p && prm.has_p2c) return launch_rel<T, D, QW, true, true, FAST, true>(prm, stream);
      if (prm.has_c2p) return launch_rel<T, D, QW, true, false, FAST, true>(prm, stream);
      if (prm.has_p2c) return launch_rel<T, D, QW, false, true, FAST, true>(prm, stream);
    }
  }
  if (prm.has_c2p && prm.has_p2c) return launch_rel<T, D, QW, true, true, FAST>(prm, stream);
  if (prm.has_c2p) return launch_rel<T, D, QW, true, false, FAST>(prm, stream);
  if (prm.has_p2c) return launch_rel<T, D, QW, false, true, FAST>(prm, stream);
  return launch_rel<T, D, QW, false, false, FAST>(prm, stream);
}

// 16-bit d = 128 runs QW = 32 (one workgroup per CU, 512 registers per lane)
// when prm.qw asks for it, unsplit; the split instance and fp32 keep QW = 16.
// d = 32 runs QW = 16 when prm.qw asks for it (only
// for the unsplit form: the split instances are built for QW = 32); d = 64 has
// only QW = 32 (QW = 16 measured 1.2-2.5x slower at every batch, see
// rel_attention_qw).
template <typename T, int D>
int rel_modes(const RelParams& prm, hipStream_t stream) {
  if constexpr (D >= 128 && sizeof(T) == 2) {
    if (prm.qw == 32 && prm.splits <= 1) return rel_modes_qw<T, D, 32>(prm, stream);
    return rel_modes_qw<T, D, 16>(prm, stream);
  } else if constexpr (D >= 128) {
    return rel_modes_qw<T, D, 16>(prm, stream);
  } else if constexpr (D == 32 && sizeof(T) == 2) {
    if (prm.qw == 16 && prm.splits <= 1) return rel_modes_qw<T, D, 16>(prm, stream);
    return rel_modes_qw<T, D, 32>(prm, stream);
  } else {
    return rel_modes_qw<T, D, 32>(prm, stream);
  }
}

}  // namespace

int rel_attention_splits(int B, int H, int L, int D, int cus, int* split_tiles) {
  // Split only when the unsplit grid leaves most CUs idle (at most a quarter
  // of them get a workgroup), and only up to one workgroup per CU: a workgroup
  // costs about four tiles of fixed time (start-up, pipeline fill, partial
  // rows), which only pays when the CUs it occupies would otherwise idle.
  // Each split keeps at least two key tiles; at most eight splits.
  const int bm = kWaves * (D >= 128 ? 16 : 32);
  const int64_t blocks = static_cast<int64_t>((L + bm - 1) / bm) * B * H;
  const int tiles = (L + 63) / 64;
  const int64_t n_cu = cus > 0 ? cus : 1;
  int splits = 1;
  // d = 128: the split instance runs out of registers (272 B of spills) and is
  // slower than the unsplit kernel even at B = 1 (29.3 against 26.9 us).
  if (D <= 64 && blocks > 0 && 4 * blocks <= n_cu) {
    const int64_t fit = n_cu / blocks;
    splits = static_cast<int>(fit < kMaxKeySplits ? fit : kMaxKeySplits);
    if (splits > tiles / 2) splits = tiles / 2;
    if (splits < 2) splits = 1;
  }
  const int st = (tiles + splits - 1) / splits;
  if (split_tiles) *split_tiles = st;
  return (tiles + st - 1) / st;
}

int rel_attention_qw(int B, int H, int L, int D, int cus, bool has_c2p) {
  // DFLASH_REL_QW=16 or 32 forces the tile (measurement runs only).
  static const int forced = [] {
    const char* env = std::getenv("DFLASH_REL_QW");
    return env ? std::atoi(env) : 0;
  }();
  if (forced == 16 || forced == 32) return forced;
  // d = 128 (16-bit): QW = 32 at one workgroup per CU (512 registers per lane)
  // against QW = 16 at two.  Each wavefront loads the relative rows of its own
  // c2p window, so 32 rows per wavefront halve those loads per query; the tile
  // pays with the c2p term and a grid that fills the CUs (C5, H = 8, L = 512,
  // c2p|p2c: B = 8 39.5 against 46.8 us, B = 16 76.0 against 86.9, B = 32
  // 148.8 against 166.9; B = 4 38.8 against 26.4; p2c alone 54.1 against 48.1).
  if (D >= 128) {
    const int64_t wg32 = static_cast<int64_t>((L + 127) / 128) * B * H;
    return (has_c2p && cus > 0 && wg32 >= cus) ? 32 : 16;
  }
  // Measured table (MI355X, 256 CUs, fp16, c2p|p2c; kernel time of back-to-back
  // launches, QW = 32 against QW = 16):
  //   d = 64, H = 12, L = 512, B = 1..48: QW = 32 wins everywhere (QW = 16 at
  //     three workgroups per CU is 1.2-2.5x slower: per-workgroup fixed costs
  //     double while the MFMA work per workgroup halves).
  //   d = 32, H = 16, L = 384: QW = 32 runs 19.0 us while its grid fits one
  //     round of two workgroups per CU (B <= 10, 480 workgroups) and 27.0-27.6 us
  //     at B = 11..16 (528..768); QW = 16 at three workgroups per CU runs
  //     25.1-25.4 us at B = 11..13 (528..624 workgroups of QW = 32) and
  //     28.7-29.2 us at B = 14..16.  So QW = 16 pays exactly when the QW = 32
  //     grid overflows one round by at most a quarter.
  // Grids are counted in QW = 32 workgroups (4 * 32 query rows of one (b, h)).
  if (D != 32 || cus <= 0) return 32;
  const int64_t wg32 = static_cast<int64_t>((L + 127) / 128) * B * H;
  const int64_t round = 2 * static_cast<int64_t>(cus);
  return (wg32 > round && 4 * wg32 <= 5 * round) ? 16 : 32;
}

size_t rel_attention_workspace_bytes(int splits, int B, int H, int L, int D) {
  if (splits <= 1) return 0;
  return static_cast<size_t>(splits) * B * L * H * static_cast<size_t>(D + 2) * sizeof(float);
}

int launch_rel_attention(const RelParams& prm, int D, int dtype, hipStream_t stream) {
#define DFLASH_REL_CASE(TYPE, DIM) \
  if (D == DIM) return rel_modes<TYPE, DIM>(prm, stream);
  if (dtype == DFLASH_DTYPE_FP16) {
    DFLASH_REL_CASE(_Float16, 32) DFLASH_REL_CASE(_Float16, 64) DFLASH_REL_CASE(_Float16, 128)
  } else if (dtype == DFLASH_DTYPE_BF16) {
    DFLASH_REL_CASE(__bf16, 32) DFLASH_REL_CASE(__bf16, 64) DFLASH_REL_CASE(__bf16, 128)
  } else if (dtype == DFLASH_DTYPE_FP32) {
    DFLASH_REL_CASE(float, 32) DFLASH_REL_CASE(float, 64) DFLASH_REL_CASE(float, 128)
  } else {
    return DFLASH_ERR_DTYPE;
  }
#undef DFLASH_REL_CASE
  return DFLASH_ERR_HEAD_DIM;
}

}  // namespace dflash
