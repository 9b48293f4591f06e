// Fused DeBERTa-v2/v3 disentangled attention forward for gfx950 (CDNA4).
//
// One workgroup = 4 wavefronts = 128 query rows of one (batch, head).  Each
// wavefront owns 32 query rows for the whole kernel and walks the key axis in
// tiles of BN keys:
//
//   S^T[j, i]  = K_j . Q_i                         (MFMA, keys x queries)
//   S^T[j, i] += c2p(i, slot(i-j)) + p2c(j, slot(i-j))
//   x          = S^T * log2(e) / sqrt(d * factor), factorized padding mask
//   online softmax over j (exp2), P cast to the input dtype
//   O^T[:, i] += V^T . P^T                          (MFMA, dims x queries)
//
// The score tile is kept transposed so that every lane holds one query column:
// a row max / row sum then needs 16 in-register steps and two cross-lane
// exchanges per 64 keys.
//
// Relative scores come from one of two sources:
//   * TABLE: precomputed c2p/p2c tables [B, H, L, S] in HBM (the contract of
//     the reference op, kernel.py:137-345);
//   * windowed (default): computed inside the tile.  The bucket function is
//     monotone in i-j, so a tile's deltas map to a contiguous slot range
//     [lo, hi].  Each wavefront computes its own c2p window Q_w . Kr[lo..hi]^T
//     and the workgroup computes one shared p2c window K_tile . Qr[lo..hi]^T,
//     both with MFMA into LDS, rounded to the input dtype exactly like the
//     reference's separate torch.matmul (kernel.py:577,583).  No [B,H,L,S] or
//     [B,H,L,L] tensor ever reaches HBM.
//
// Mask semantics follow kernel.py:250-261 (Hugging Face padded-row behaviour):
//   kept query & kept key           -> score
//   padded query (in range)         -> 0 for every in-range key (uniform row)
//   kept query & padded key         -> -inf
//   query past L                    -> 0 at key 0 only (row never stored)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dflash.h"

namespace dflash {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;               // wavefronts per workgroup
constexpr int kQueriesPerWave = 32;     // query rows owned by one wavefront
constexpr int kBlockM = kWaves * kQueriesPerWave;
constexpr int kThreads = kWaves * 64;
constexpr int kQB = kQueriesPerWave / 16;  // 16-row MFMA blocks per wavefront

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

// Load one lane's k-slice starting at `base` (which already points at k0 of
// the MFMA step for this lane's row/column).
template <typename T>
__device__ inline typename Mma<T>::frag load_slice(const T* base, int g) {
  if constexpr (Mma<T>::PER == 8) {
    return *reinterpret_cast<const typename Mma<T>::frag*>(base + 8 * g);
  } else {
    return base[g];
  }
}

template <typename T>
__device__ inline typename Mma<T>::frag zero_frag() {
  typename Mma<T>::frag z;
  if constexpr (Mma<T>::PER == 8) {
    for (int e = 0; e < 8; ++e) z[e] = static_cast<T>(0.0f);
  } else {
    z = 0.0f;
  }
  return z;
}

template <typename T>
__device__ inline T to_t(float x) {
  return static_cast<T>(x);
}

template <typename T>
__device__ inline float to_f(T x) {
  return static_cast<float>(x);
}

// 16-byte global/LDS chunk copy.
struct alignas(16) Chunk {
  uint32_t w[4];
};

struct Params {
  const void* q;
  const void* k;
  const void* v;
  int64_t sb, sh, sl;          // element strides of q/k/v: batch, head, position
  const void* pos_key;         // [H, S, D] (windowed) or c2p table [B, H, L, S]
  const void* pos_query;       // [H, S, D] (windowed) or p2c table [B, H, L, S]
  const int32_t* lut;          // delta_to_local [2L-1]
  const uint8_t* mask;         // [B, L], nonzero = kept
  void* out;                   // [B, L, H*D]
  int B, H, L, S;
  int nqb;                     // query blocks per (b, h)
  float scale_log2;            // log2(e) / sqrt(d * factor)
};

// Padded LDS row lengths (elements).  16-bit rows stay 16-byte aligned.
template <typename T>
constexpr int pad_of() {
  return sizeof(T) == 2 ? 8 : 4;
}
constexpr int round16(int x) { return (x + 15) / 16 * 16; }

template <typename T, int D, int BN>
struct Layout {
  static constexpr int kPad = pad_of<T>();
  static constexpr int KS_LD = D + kPad;                         // Ks[BN][KS_LD]
  static constexpr int VT_LD = BN + kPad;                        // Vt[D][VT_LD]
  static constexpr int WP_MAX = round16(kBlockM + BN - 1);       // p2c window
  static constexpr int PW_LD = WP_MAX + kPad;                    // Pw[BN][PW_LD]
  static constexpr int WC_MAX = round16(kQueriesPerWave + BN - 1);  // c2p window
  static constexpr int CW_LD = WC_MAX + kPad;                    // Cw[w][32][CW_LD]
  static constexpr int LW_N = kBlockM + BN;                      // lut window

  static constexpr size_t ks_bytes = size_t(BN) * KS_LD * sizeof(T);
  static constexpr size_t vt_bytes = size_t(D) * VT_LD * sizeof(T);
  static constexpr size_t pw_bytes = size_t(BN) * PW_LD * sizeof(T);
  static constexpr size_t cw_bytes = size_t(kWaves) * kQueriesPerWave * CW_LD * sizeof(T);
  static constexpr size_t lw_bytes = size_t(LW_N) * sizeof(int32_t);
  static constexpr size_t km_bytes = size_t(BN);

  static constexpr size_t ks_off = 0;
  static constexpr size_t vt_off = ks_off + ks_bytes;
  static constexpr size_t pw_off = vt_off + vt_bytes;
  static constexpr size_t cw_off = pw_off + pw_bytes;
  static constexpr size_t lw_off = cw_off + cw_bytes;
  static constexpr size_t km_off = lw_off + lw_bytes;

  static constexpr size_t bytes(bool windowed) {
    size_t total = ks_bytes + vt_bytes + lw_bytes + km_bytes;
    if (windowed) total += pw_bytes + cw_bytes;
    return total;
  }
};

__device__ inline int clampi(int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); }

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

template <typename T, int D, int BN, bool C2P, bool P2C, bool TABLE>
__global__ __launch_bounds__(kThreads, 2) void attention_kernel(Params p) {
  using M = Mma<T>;
  using F = typename M::frag;
  using LY = Layout<T, D, BN>;
  constexpr bool WINDOWED = (C2P || P2C) && !TABLE;
  constexpr int KB = BN / 16;          // 16-key blocks per tile
  constexpr int DB = D / 16;           // 16-dim blocks of the output
  constexpr int KD = D / M::K;         // MFMA steps over the head dimension
  constexpr int E16 = 16 / sizeof(T);  // elements per 16-byte chunk
  constexpr int CPR = D / E16;         // chunks per K/V row
  static_assert(BN % 32 == 0 || sizeof(T) == 4, "16-bit PV steps need 32-key groups");

  extern __shared__ __align__(16) unsigned char smem[];
  T* Ks = reinterpret_cast<T*>(smem + LY::ks_off);
  T* Vt = reinterpret_cast<T*>(smem + LY::vt_off);
  T* Pw = reinterpret_cast<T*>(smem + LY::pw_off);
  T* Cw = reinterpret_cast<T*>(smem + LY::cw_off);
  int32_t* Lw = reinterpret_cast<int32_t*>(smem + (WINDOWED ? LY::lw_off : LY::pw_off));
  uint8_t* Km = smem + (WINDOWED ? LY::km_off : LY::pw_off + LY::lw_bytes);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;

  const int L = p.L;
  const int H = p.H;
  const int S = p.S;
  const int m = xcd_logical_block(blockIdx.x, gridDim.x);
  const int bh = m / p.nqb;
  const int qblk = m - bh * p.nqb;
  const int b = bh / H;
  const int h = bh - b * H;
  const int i0 = qblk * kBlockM;
  const int i0w = i0 + wave * kQueriesPerWave;

  const T* qg = reinterpret_cast<const T*>(p.q) + b * p.sb + h * p.sh;
  const T* kg = reinterpret_cast<const T*>(p.k) + b * p.sb + h * p.sh;
  const T* vg = reinterpret_cast<const T*>(p.v) + b * p.sb + h * p.sh;
  const uint8_t* maskb = p.mask + static_cast<int64_t>(b) * L;

  // Q fragments stay in registers for the whole kernel.  They serve as the B
  // operand of K.Q^T and as the A operand of the c2p window product.
  F qf[kQB][KD];
  bool qkept[kQB];
  bool qin[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int i = i0w + 16 * qb + c;
    qin[qb] = i < L;
    qkept[qb] = qin[qb] && maskb[i] != 0;
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      qf[qb][kd] = qin[qb] ? load_slice<T>(qg + static_cast<int64_t>(i) * p.sl + kd * M::K, g)
                           : zero_frag<T>();
    }
  }

  f32x4_t o[DB][kQB];
  float row_max[kQB];
  float row_sum[kQB];  // per-lane partial sums; reduced across lanes at the end
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    row_max[qb] = -INFINITY;
    row_sum[qb] = 0.0f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db][qb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const T* posk = reinterpret_cast<const T*>(p.pos_key);
  const T* posq = reinterpret_cast<const T*>(p.pos_query);
  const T* c2p_rows = posk + static_cast<int64_t>(bh) * L * S;  // TABLE only
  const T* p2c_rows = posq + static_cast<int64_t>(bh) * L * S;  // TABLE only
  const T* kr = posk + static_cast<int64_t>(h) * S * D;         // windowed only
  const T* qr = posq + static_cast<int64_t>(h) * S * D;         // windowed only

  for (int j0 = 0; j0 < L; j0 += BN) {
    // Delta window of this workgroup tile and of this wavefront.
    const int dlo = i0 - (j0 + BN - 1);
    const int dlo_c = clampi(dlo, -(L - 1), L - 1);
    const int dhi_c = clampi(i0 + kBlockM - 1 - j0, -(L - 1), L - 1);
    int lo_p = 0, w_p = 0, lo_c = 0, w_c = 0;
    if constexpr (WINDOWED) {
      lo_p = p.lut[dlo_c + L - 1];
      w_p = p.lut[dhi_c + L - 1] - lo_p + 1;
      const int dlo_w = clampi(i0w - (j0 + BN - 1), -(L - 1), L - 1);
      const int dhi_w = clampi(i0w + kQueriesPerWave - 1 - j0, -(L - 1), L - 1);
      lo_c = p.lut[dlo_w + L - 1];
      w_c = p.lut[dhi_w + L - 1] - lo_c + 1;
      // A plan whose lookup table steps by more than one slot per delta breaks
      // the window precondition; clamp so LDS writes stay inside the buffers.
      w_p = min(w_p, LY::WP_MAX);
      w_c = min(w_c, LY::WC_MAX);
    }

    __syncthreads();  // the previous tile is done with every LDS buffer

    // ---- stage K (row-major), V^T, key mask and the delta -> slot window ----
    for (int t = tid; t < BN * CPR; t += kThreads) {
      const int r = t / CPR;
      const int cc = t - r * CPR;
      const int j = j0 + r;
      Chunk kv{{0u, 0u, 0u, 0u}};
      Chunk vv{{0u, 0u, 0u, 0u}};
      if (j < L) {
        kv = *reinterpret_cast<const Chunk*>(kg + static_cast<int64_t>(j) * p.sl + cc * E16);
        vv = *reinterpret_cast<const Chunk*>(vg + static_cast<int64_t>(j) * p.sl + cc * E16);
      }
      *reinterpret_cast<Chunk*>(Ks + r * LY::KS_LD + cc * E16) = kv;
      const T* ve = reinterpret_cast<const T*>(&vv);
#pragma unroll
      for (int e = 0; e < E16; ++e) Vt[(cc * E16 + e) * LY::VT_LD + r] = ve[e];
    }
    for (int t = tid; t < BN; t += kThreads) {
      const int j = j0 + t;
      Km[t] = (j < L) ? (maskb[j] != 0) : 0;
    }
    if constexpr (C2P || P2C) {
      for (int t = tid; t < kBlockM + BN - 1; t += kThreads) {
        const int d = clampi(dlo + t, -(L - 1), L - 1);
        Lw[t] = p.lut[d + L - 1] - lo_p;
      }
    }
    __syncthreads();

    // ---- relative-score windows (MFMA into LDS) ----
    if constexpr (WINDOWED) {
      if constexpr (P2C) {
        // Pw[jr][s - lo_p] = K[j0 + jr] . Qr[s], shared by the workgroup.
        const int nsc = (w_p + 15) >> 4;
        for (int item = wave; item < KB * nsc; item += kWaves) {
          const int kb = item / nsc;
          const int sc = item - kb * nsc;
          const int s = min(lo_p + 16 * sc + c, S - 1);
          f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kd = 0; kd < KD; ++kd) {
            F a = load_slice<T>(Ks + (16 * kb + c) * LY::KS_LD + kd * M::K, g);
            F bq = load_slice<T>(qr + static_cast<int64_t>(s) * D + kd * M::K, g);
            acc = M::run(a, bq, acc);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r)
            Pw[(16 * kb + 4 * g + r) * LY::PW_LD + 16 * sc + c] = to_t<T>(acc[r]);
        }
      }
      if constexpr (C2P) {
        // Cw[wave][q][s - lo_c] = Q[i0w + q] . Kr[s], private to the wavefront.
        T* cw = Cw + wave * kQueriesPerWave * LY::CW_LD;
        const int nsc = (w_c + 15) >> 4;
        for (int sc = 0; sc < nsc; ++sc) {
          const int s = min(lo_c + 16 * sc + c, S - 1);
          F bk[KD];
#pragma unroll
          for (int kd = 0; kd < KD; ++kd)
            bk[kd] = load_slice<T>(kr + static_cast<int64_t>(s) * D + kd * M::K, g);
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb) {
            f32x4_t acc{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kd = 0; kd < KD; ++kd) acc = M::run(qf[qb][kd], bk[kd], acc);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              cw[(16 * qb + 4 * g + r) * LY::CW_LD + 16 * sc + c] = to_t<T>(acc[r]);
          }
        }
      }
      __syncthreads();
    }

    // ---- S^T = K . Q^T ----
    f32x4_t sc_acc[KB][kQB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) sc_acc[kb][qb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        F a = load_slice<T>(Ks + (16 * kb + c) * LY::KS_LD + kd * M::K, g);
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) sc_acc[kb][qb] = M::run(a, qf[qb][kd], sc_acc[kb][qb]);
      }
    }

    // ---- relative scores, scale, mask, online softmax ----
    const T* cw = Cw + wave * kQueriesPerWave * LY::CW_LD;
    const int c_shift = lo_c - lo_p;
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      const int iq = 16 * qb + c;        // query row inside the wavefront
      const int i = i0w + iq;
      float tile_max = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int jr = 16 * kb + 4 * g + r;
          const int j = j0 + jr;
          float s = sc_acc[kb][qb][r];
          if constexpr (C2P || P2C) {
            const int ls = Lw[i - j - dlo];
            if constexpr (TABLE) {
              const bool ok = qin[qb] && j < L;
              if constexpr (C2P)
                if (ok) s += to_f<T>(c2p_rows[static_cast<int64_t>(i) * S + ls]);
              if constexpr (P2C)
                if (ok) s += to_f<T>(p2c_rows[static_cast<int64_t>(j) * S + ls]);
            } else {
              if constexpr (C2P) s += to_f<T>(cw[iq * LY::CW_LD + ls - c_shift]);
              if constexpr (P2C) s += to_f<T>(Pw[jr * LY::PW_LD + ls]);
            }
          }
          float x = s * p.scale_log2;
          const bool kin = j < L;
          const bool kkept = Km[jr] != 0;
          if (!(qkept[qb] && kkept)) {
            if (qin[qb]) {
              x = (!qkept[qb] && kin) ? 0.0f : -INFINITY;
            } else {
              x = (j == 0) ? 0.0f : -INFINITY;
            }
          }
          sc_acc[kb][qb][r] = x;
          tile_max = fmaxf(tile_max, x);
        }
      }
      tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 16));
      tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
      const float new_max = fmaxf(row_max[qb], tile_max);
      const float base = new_max == -INFINITY ? 0.0f : new_max;
      const float corr = __builtin_amdgcn_exp2f(row_max[qb] - base);
      row_max[qb] = new_max;
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = __builtin_amdgcn_exp2f(sc_acc[kb][qb][r] - base);
          sc_acc[kb][qb][r] = pr;
          psum += pr;
        }
      row_sum[qb] = row_sum[qb] * corr + psum;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db][qb] *= corr;
    }

    // ---- O^T += V^T . P^T ----
    if constexpr (M::PER == 8) {
#pragma unroll
      for (int ks = 0; ks < BN / 32; ++ks) {
        F pf[kQB];
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            pf[qb][r] = to_t<T>(sc_acc[2 * ks][qb][r]);
            pf[qb][4 + r] = to_t<T>(sc_acc[2 * ks + 1][qb][r]);
          }
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const T* vrow = Vt + (16 * db + c) * LY::VT_LD + 32 * ks + 4 * g;
          F a;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            a[r] = vrow[r];
            a[4 + r] = vrow[16 + r];
          }
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb) o[db][qb] = M::run(a, pf[qb], o[db][qb]);
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const float a = Vt[(16 * db + c) * LY::VT_LD + 16 * kb + 4 * g + r];
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb)
              o[db][qb] = M::run(a, sc_acc[kb][qb][r], o[db][qb]);
          }
        }
      }
    }
  }

  // ---- normalise and store [B, L, H*D] ----
  T* outp = reinterpret_cast<T*>(p.out);
  const int64_t row_stride = static_cast<int64_t>(H) * D;
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    float total = row_sum[qb];
    total += __shfl_xor(total, 16);
    total += __shfl_xor(total, 32);
    const int i = i0w + 16 * qb + c;
    if (i >= L) continue;
    const float inv = 1.0f / total;
    T* dst = outp + (static_cast<int64_t>(b) * L + i) * row_stride + h * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      T vals[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) vals[r] = to_t<T>(o[db][qb][r] * inv);
      T* d4 = dst + 16 * db + 4 * g;
      if constexpr (sizeof(T) == 2) {
        uint2 packed;
        __builtin_memcpy(&packed, vals, 8);
        *reinterpret_cast<uint2*>(d4) = packed;
      } else {
        *reinterpret_cast<float4*>(d4) = make_float4(vals[0], vals[1], vals[2], vals[3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host-side dispatch
// ---------------------------------------------------------------------------
template <typename T, int D>
constexpr int block_n() {
  return sizeof(T) == 4 ? 32 : 64;
}

template <typename T, int D, bool C2P, bool P2C, bool TABLE>
int launch(const Params& prm, hipStream_t stream) {
  constexpr int BN = block_n<T, D>();
  using LY = Layout<T, D, BN>;
  constexpr bool WINDOWED = (C2P || P2C) && !TABLE;
  const size_t lds = LY::bytes(WINDOWED);
  auto kernel = attention_kernel<T, D, BN, C2P, P2C, TABLE>;
  hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       static_cast<int>(lds));
  if (err != hipSuccess) return static_cast<int>(err);
  const int64_t blocks = static_cast<int64_t>(prm.nqb) * prm.B * prm.H;
  if (blocks > 0x7fffffff) return DFLASH_ERR_TOO_LARGE;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), lds, stream, prm);
  return static_cast<int>(hipGetLastError());
}

template <typename T, int D, bool TABLE>
int dispatch_modes(const Params& prm, int has_c2p, int has_p2c, hipStream_t stream) {
  if (has_c2p && has_p2c) return launch<T, D, true, true, TABLE>(prm, stream);
  if (has_c2p) return launch<T, D, true, false, TABLE>(prm, stream);
  if (has_p2c) return launch<T, D, false, true, TABLE>(prm, stream);
  return launch<T, D, false, false, TABLE>(prm, stream);
}

template <bool TABLE>
int dispatch(const Params& prm, int D, int dtype, int has_c2p, int has_p2c, hipStream_t stream) {
#define DFLASH_CASE(TYPE, DIM)                                                     \
  if (D == DIM) return dispatch_modes<TYPE, DIM, TABLE>(prm, has_c2p, has_p2c, stream);
  switch (dtype) {
    case DFLASH_DTYPE_FP16:
      DFLASH_CASE(_Float16, 32) DFLASH_CASE(_Float16, 64) DFLASH_CASE(_Float16, 128) break;
    case DFLASH_DTYPE_BF16:
      DFLASH_CASE(__bf16, 32) DFLASH_CASE(__bf16, 64) DFLASH_CASE(__bf16, 128) break;
    case DFLASH_DTYPE_FP32:
      DFLASH_CASE(float, 32) DFLASH_CASE(float, 64) DFLASH_CASE(float, 128) break;
    default:
      return DFLASH_ERR_DTYPE;
  }
#undef DFLASH_CASE
  return DFLASH_ERR_HEAD_DIM;
}

int check_common(const void* q, const void* k, const void* v, const int32_t* lut,
                 const uint8_t* mask, const void* out, int B, int H, int L, int D, int S,
                 int has_c2p, int has_p2c, int dtype) {
  if (!q || !k || !v || !mask || !out) return DFLASH_ERR_NULL;
  if (B < 1 || H < 1 || L < 1) return DFLASH_ERR_SHAPE;
  if (D != 32 && D != 64 && D != 128) return DFLASH_ERR_HEAD_DIM;
  if (dtype < DFLASH_DTYPE_FP16 || dtype > DFLASH_DTYPE_FP32) return DFLASH_ERR_DTYPE;
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
  (void)strict_fp32;  // fp32 always runs IEEE fp32 MFMA on gfx950
  int rc = check_common(query, key, value, delta_to_local, attention_mask, out, B, H, L, D, S,
                        has_c2p, has_p2c, dtype);
  if (rc != DFLASH_OK) return rc;
  if ((has_c2p && !c2p) || (has_p2c && !p2c)) return DFLASH_ERR_NULL;
  Params prm{};
  prm.q = query;
  prm.k = key;
  prm.v = value;
  prm.sb = static_cast<int64_t>(H) * L * D;
  prm.sh = static_cast<int64_t>(L) * D;
  prm.sl = D;
  prm.pos_key = has_c2p ? c2p : query;
  prm.pos_query = has_p2c ? p2c : key;
  prm.lut = delta_to_local;
  prm.mask = attention_mask;
  prm.out = out;
  prm.B = B;
  prm.H = H;
  prm.L = L;
  prm.S = (has_c2p || has_p2c) ? S : 1;
  prm.nqb = (L + kBlockM - 1) / kBlockM;
  prm.scale_log2 = score_scale_log2;
  return dispatch<true>(prm, D, dtype, has_c2p, has_p2c, static_cast<hipStream_t>(stream));
}

int dflash_attention_rel_fwd(const void* query, const void* key, const void* value,
                             int64_t stride_b, int64_t stride_h, int64_t stride_l,
                             const void* pos_key, const void* pos_query,
                             const int32_t* delta_to_local, const uint8_t* attention_mask,
                             void* out, int B, int H, int L, int D, int S,
                             float score_scale_log2, int has_c2p, int has_p2c, int dtype,
                             int strict_fp32, void* stream) {
  (void)strict_fp32;
  int rc = check_common(query, key, value, delta_to_local, attention_mask, out, B, H, L, D, S,
                        has_c2p, has_p2c, dtype);
  if (rc != DFLASH_OK) return rc;
  if ((has_c2p && !pos_key) || (has_p2c && !pos_query)) return DFLASH_ERR_NULL;
  const int esize = dtype == DFLASH_DTYPE_FP32 ? 4 : 2;
  if (stride_l < D || stride_b < 1 || stride_h < 1) return DFLASH_ERR_SHAPE;
  if (((stride_b | stride_h | stride_l) * esize) % 16 != 0) return DFLASH_ERR_ALIGN;
  const uintptr_t addr_or = reinterpret_cast<uintptr_t>(query) |
                            reinterpret_cast<uintptr_t>(key) |
                            reinterpret_cast<uintptr_t>(value) |
                            reinterpret_cast<uintptr_t>(out) |
                            reinterpret_cast<uintptr_t>(pos_key) |
                            reinterpret_cast<uintptr_t>(pos_query);
  if (addr_or % 16 != 0) return DFLASH_ERR_ALIGN;
  Params prm{};
  prm.q = query;
  prm.k = key;
  prm.v = value;
  prm.sb = stride_b;
  prm.sh = stride_h;
  prm.sl = stride_l;
  prm.pos_key = has_c2p ? pos_key : query;
  prm.pos_query = has_p2c ? pos_query : key;
  prm.lut = delta_to_local;
  prm.mask = attention_mask;
  prm.out = out;
  prm.B = B;
  prm.H = H;
  prm.L = L;
  prm.S = (has_c2p || has_p2c) ? S : 1;
  prm.nqb = (L + kBlockM - 1) / kBlockM;
  prm.scale_log2 = score_scale_log2;
  return dispatch<false>(prm, D, dtype, has_c2p, has_p2c, static_cast<hipStream_t>(stream));
}

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
    default:
      return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
  }
}

int dflash_abi_version(void) { return DFLASH_ABI_VERSION; }

}  // extern "C"
