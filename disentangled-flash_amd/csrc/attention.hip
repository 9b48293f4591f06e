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
// Relative scores come from precomputed c2p/p2c tables [B, H, L, S] in HBM:
// this kernel serves the reference op's contract (kernel.py:137-345) and the
// relative_mode="table" data flow.  The default path computes the relative
// scores inside the tile instead (rel_attention.hip).
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

template <typename T, int D, int BN, int QW, bool C2P, bool P2C>
__global__ __launch_bounds__(kThreads, 2) void attention_kernel(Params p) {
  using M = Mma<T>;
  using F = typename M::frag;
  using LY = Layout<T, D, BN, QW>;
  constexpr int kBlockM = LY::kBlockM;
  constexpr int kQB = QW / 16;         // 16-row MFMA blocks per wavefront
  constexpr bool REL = C2P || P2C;
  constexpr int KB = BN / 16;          // 16-key blocks per tile
  constexpr int DB = D / 16;           // 16-dim blocks of the output
  constexpr int KD = D / M::K;         // MFMA steps over the head dimension
  constexpr int E16 = 16 / sizeof(T);  // elements per 16-byte chunk
  constexpr int CPR = D / E16;         // 16-byte chunks per K row
  static_assert(BN % 32 == 0 || sizeof(T) == 4, "16-bit PV steps need 32-key groups");

  extern __shared__ __align__(16) unsigned char smem[];
  T* Ks = reinterpret_cast<T*>(smem + LY::ks_off);
  T* Vt = reinterpret_cast<T*>(smem + LY::vt_off);
  float* Kbias = reinterpret_cast<float*>(smem + LY::kb_off);
  int32_t* Lw = reinterpret_cast<int32_t*>(smem + LY::lw_off);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wavefront index as a scalar: per-wave window bounds then use scalar loads.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const int i0w = i0 + wave * QW;

  const T* qg = reinterpret_cast<const T*>(p.q) + b * p.sb + h * p.sh;
  const T* kg = reinterpret_cast<const T*>(p.k) + b * p.sb + h * p.sh;
  const T* vg = reinterpret_cast<const T*>(p.v) + b * p.sb + h * p.sh;
  const uint8_t* maskb = p.mask + static_cast<int64_t>(b) * L;
  const int sl = static_cast<int>(p.sl);  // row stride; L * sl < 2^31 is checked on the host

  // Q fragments stay in registers for the whole kernel.  In the 16x16 MFMA
  // layouts the A and B operands of a lane hold the same (row/column, k-slice),
  // so these registers serve as B of K.Q^T and as B of Kr.Q^T.
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
  const T* c2p_rows = posk + static_cast<int64_t>(bh) * L * S;  // [L, S] of this (b, h)
  const T* p2c_rows = posq + static_cast<int64_t>(bh) * L * S;

  // ---- per-thread prefetch registers for the next tile ----
  // K: 16-byte row chunks.  V: 4 keys x 4 dims blocks, transposed in registers
  // and written to V^T as 4 packed stores.  Plus one LUT entry and one mask byte.
  constexpr int NCH = (BN * CPR + kThreads - 1) / kThreads;
  constexpr int VQD = D / 4;                                   // dim quads per row
  constexpr int NVB = (BN / 4 * VQD + kThreads - 1) / kThreads;
  constexpr int NLW = (kBlockM + BN - 1 + kThreads - 1) / kThreads;
  constexpr bool K_EXACT = (BN * CPR) % kThreads == 0;
  constexpr bool V_EXACT = (BN / 4 * VQD) % kThreads == 0;
  u32x4_t pk[NCH];
  Quad<T> pv[NVB][4];
  int plut[NLW];
  uint8_t pmask_raw = 0;  // mask byte of key jt + tid % BN (row clamped to L-1)
  bool pmask_in = false;  // whether that key is inside the sequence
  auto prefetch = [&](int jt) {
#pragma unroll
    for (int n = 0; n < NCH; ++n) {
      const int t = tid + n * kThreads;
      const int r = t / CPR;
      const int cc = t - r * CPR;
      // Rows past L are read from row L-1: finite values whose scores the key
      // bias masks and whose probabilities are zero.
      const int j = min(jt + r, L - 1);
      if (K_EXACT || t < BN * CPR)
        pk[n] = *reinterpret_cast<const u32x4_t*>(kg + (j * sl + cc * E16));
    }
#pragma unroll
    for (int n = 0; n < NVB; ++n) {
      const int t = tid + n * kThreads;
      const int kq = t / VQD;
      const int dq = t - kq * VQD;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int j = min(jt + 4 * kq + rr, L - 1);
        if (V_EXACT || t < BN / 4 * VQD)
          pv[n][rr] = *reinterpret_cast<const Quad<T>*>(vg + (j * sl + 4 * dq));
      }
    }
    if constexpr (REL) {
      const int dlo_t = i0 - (jt + BN - 1);
#pragma unroll
      for (int n = 0; n < NLW; ++n) {
        const int t = tid + n * kThreads;
        const int d = clampi(dlo_t + t, -(L - 1), L - 1);
        plut[n] = p.lut[d + L - 1];
      }
    }
    const int jm = jt + (tid % BN);
    pmask_raw = maskb[min(jm, L - 1)];
    pmask_in = jm < L;
  };

  prefetch(0);
  for (int j0 = 0; j0 < L; j0 += BN) {
    lds_barrier();  // the previous tile is done with every LDS buffer

    // ---- stage the prefetched tile: K, V^T, key bias, delta -> slot window ----
#pragma unroll
    for (int n = 0; n < NCH; ++n) {
      const int t = tid + n * kThreads;
      if (K_EXACT || t < BN * CPR) {
        const int r = t / CPR;
        const int cc = t - r * CPR;
        *reinterpret_cast<u32x4_t*>(Ks + r * LY::KS_LD + cc * E16) = pk[n];
      }
    }
#pragma unroll
    for (int n = 0; n < NVB; ++n) {
      const int t = tid + n * kThreads;
      if (V_EXACT || t < BN / 4 * VQD) {
        const int kq = t / VQD;
        const int dq = t - kq * VQD;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          Quad<T> col;
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) col[rr] = pv[n][rr][e];
          *reinterpret_cast<Quad<T>*>(Vt + (4 * dq + e) * LY::VT_LD + 4 * kq) = col;
        }
      }
    }
    if (tid < BN) Kbias[tid] = (pmask_in && pmask_raw != 0) ? 0.0f : -INFINITY;
    if constexpr (REL) {
#pragma unroll
      for (int n = 0; n < NLW; ++n) {
        const int t = tid + n * kThreads;
        if (t < kBlockM + BN - 1) Lw[t] = plut[n];
      }
    }
    lds_barrier();

    auto kfrag = [&](int kb, int kd) -> F {
      return load_slice<T>(Ks + (16 * kb + c) * LY::KS_LD + kd * M::K, g);
    };

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
        const F a = kfrag(kb, kd);
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) sc_acc[kb][qb] = M::run(a, qf[qb][kd], sc_acc[kb][qb]);
      }
    }

    // Next tile's K/V/LUT/mask: issued after every load this tile consumes
    // (vector-memory counters retire in order), in flight during the softmax.
    // Unconditional (the last tile re-reads clamped rows) so that no branch
    // joins pending loads, which would force early waits on them.
    prefetch(j0 + BN);

    // ---- relative scores, scale, key bias ----
    // The local slot of (i, j) sits in the LDS window of lookups at
    //   i - j - (i0 - j0 - BN + 1) = lane_base + 16*(qb - kb) - r,
    //   lane_base = wave*QW + c - 4g + BN - 1.
    const int lane_base = wave * QW + c - 4 * g + BN - 1;
    const int32_t* lw_lane = Lw + lane_base;
    f32x4_t kbias[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      kbias[kb] = *reinterpret_cast<const f32x4_t*>(Kbias + 16 * kb + 4 * g);
    const float scale = p.scale_log2;

    auto relative = [&](int qb, int kb, int r, int ls) -> float {
      float add = 0.0f;
      const int i = i0w + 16 * qb + c;
      const int j = j0 + 16 * kb + 4 * g + r;
      const bool ok = qin[qb] && j < L;
      if constexpr (C2P)
        if (ok) add += to_f<T>(c2p_rows[static_cast<int64_t>(i) * S + ls]);
      if constexpr (P2C)
        if (ok) add += to_f<T>(p2c_rows[static_cast<int64_t>(j) * S + ls]);
      return add;
    };
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float s = sc_acc[kb][qb][r];
          if constexpr (REL) s += relative(qb, kb, r, lw_lane[16 * (qb - kb) - r]);
          sc_acc[kb][qb][r] = fmaf(s, scale, kbias[kb][r]);
        }

    // ---- padded and out-of-range query rows (rare; wavefront-uniform branch) ----
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      if (__any(!qkept[qb])) {
        if (!qkept[qb]) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int j = j0 + 16 * kb + 4 * g + r;
              // padded row: uniform over in-range keys; row past L: key 0 only
              const bool hit = qin[qb] ? (j < L) : (j == 0);
              sc_acc[kb][qb][r] = hit ? 0.0f : -INFINITY;
            }
        }
      }
    }

    // ---- online softmax ----
    // The exponent base of a row only has to be common to the row and keep
    // exp2 finite, so the previous maximum is reused while no score exceeds it
    // by more than kSlack (p <= 2^kSlack); only then are the row maxima reduced
    // across lanes and the accumulators rescaled.  Wavefront-uniform branch.
    constexpr float kSlack = 8.0f;
#pragma unroll
    for (int qb = 0; qb < kQB; ++qb) {
      float lane_max = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) lane_max = fmaxf(lane_max, sc_acc[kb][qb][r]);
      if (__any(lane_max > row_max[qb] + kSlack)) {
        float tile_max = fmaxf(lane_max, __shfl_xor(lane_max, 16));
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 32));
        const float new_max = fmaxf(row_max[qb], tile_max);
        const float old_base = row_max[qb] == -INFINITY ? 0.0f : row_max[qb];
        const float new_base = new_max == -INFINITY ? 0.0f : new_max;
        const float corr = __builtin_amdgcn_exp2f(old_base - new_base);
        row_max[qb] = new_max;
        row_sum[qb] *= corr;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db][qb] *= corr;
      }
      const float base = row_max[qb] == -INFINITY ? 0.0f : row_max[qb];
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = __builtin_amdgcn_exp2f(sc_acc[kb][qb][r] - base);
          sc_acc[kb][qb][r] = pr;
          psum += pr;
        }
      row_sum[qb] += psum;
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
          const Quad<T> lo = *reinterpret_cast<const Quad<T>*>(vrow);
          const Quad<T> hi = *reinterpret_cast<const Quad<T>*>(vrow + 16);
          F a;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            a[r] = lo[r];
            a[4 + r] = hi[r];
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
// Tile configuration per (dtype, head dim): keys per tile and query rows per
// wavefront.  d=128 halves the rows per wavefront to stay within 256 VGPRs at
// two wavefronts per SIMD.
template <typename T, int D>
constexpr int block_n() {
  return sizeof(T) == 4 ? 32 : 64;
}
template <typename T, int D>
constexpr int queries_per_wave() {
  return D >= 128 ? 16 : 32;
}

template <typename T, int D, bool C2P, bool P2C>
int launch(const Params& base, hipStream_t stream) {
  constexpr int BN = block_n<T, D>();
  constexpr int QW = queries_per_wave<T, D>();
  using LY = Layout<T, D, BN, QW>;
  Params prm = base;
  prm.nqb = (prm.L + LY::kBlockM - 1) / LY::kBlockM;
  constexpr size_t lds = LY::bytes;
  constexpr auto kernel = attention_kernel<T, D, BN, QW, C2P, P2C>;
  hipError_t err = ensure_dynamic_lds<kernel>(static_cast<int>(lds));
  if (err != hipSuccess) return static_cast<int>(err);
  const int64_t blocks = static_cast<int64_t>(prm.nqb) * prm.B * prm.H;
  if (blocks > 0x7fffffff) return DFLASH_ERR_TOO_LARGE;
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), lds, stream, prm);
  return static_cast<int>(hipGetLastError());
}

template <typename T, int D>
int dispatch_modes(const Params& prm, int has_c2p, int has_p2c, hipStream_t stream) {
  if (has_c2p && has_p2c) return launch<T, D, true, true>(prm, stream);
  if (has_c2p) return launch<T, D, true, false>(prm, stream);
  if (has_p2c) return launch<T, D, false, true>(prm, stream);
  return launch<T, D, false, false>(prm, stream);
}

int dispatch(const Params& prm, int D, int dtype, int has_c2p, int has_p2c, hipStream_t stream) {
#define DFLASH_CASE(TYPE, DIM) \
  if (D == DIM) return dispatch_modes<TYPE, DIM>(prm, has_c2p, has_p2c, stream);
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
  // The table contract runs IEEE fp32 MFMA for either precision; the fast
  // fp32 form (bf16x3) is built for the in-kernel-relative entry points.
  (void)strict_fp32;
  int rc = check_common(query, key, value, delta_to_local, attention_mask, out, B, H, L, D, S,
                        has_c2p, has_p2c, dtype);
  if (rc == kEmptyBatch) return DFLASH_OK;
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
  prm.scale_log2 = score_scale_log2;
  return dispatch(prm, D, dtype, has_c2p, has_p2c, static_cast<hipStream_t>(stream));
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
  rp.qw = rel_attention_qw(B, H, L, D, current_device_cus());
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
  if (count > 1) {
    const int rc = scratch_address(&ws);
    if (rc != DFLASH_OK) return rc;
  }
  return rel_forward(query, key, value, stride_b, stride_h, stride_l, pos_key, pos_query,
                     delta_to_local, attention_mask, out, B, H, L, D, S, score_scale_log2,
                     has_c2p, has_p2c, dtype, strict_fp32, count, ws, count > 1 ? kScratchBytes : 0,
                     stream);
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
    case DFLASH_ERR_SCRATCH:
      return "the split workspace this shape needs exceeds the library's static scratch "
             "(dflash_attention_rel_noalloc_scratch_bytes)";
    default:
      return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
  }
}

int dflash_abi_version(void) { return DFLASH_ABI_VERSION; }

}  // extern "C"
