// Gather-GEMM (forward and input-gradient) and weight-gradient kernels.
//
// Forward, output-stationary (precomputed_fwd_kernel, implicit_precomputed_gemm.py:64-126):
//   workgroup = 4 waves = 128 destination rows x BN columns.  Per kernel
//   offset k present in the tile (row masks OR-ed in LDS), the B operand
//   Bt[k] (BN x Kd slice) is staged in LDS once for all 4 waves; each wave
//   gathers the A rows of its 32 destination rows straight from HBM into
//   registers (one 16-byte load per lane per 16/32 reduction elements) and
//   accumulates 2 x BN/16 MFMA tiles in registers.  Offsets no row of a wave
//   has are skipped by that wave; offsets no row of the tile has are skipped
//   by the workgroup.  Each destination row is written exactly once: no
//   atomics, no zero-fill pass, deterministic.
// Input gradient: the same kernel over the transposed kernel map (for a
//   submanifold map, the same map with the weight offsets reversed), which
//   replaces the reference's atomic scatter (precomputed_bwd_feat_kernel :129-177).
// Weight gradient (precomputed_bwd_weight_kernel :180-230): workgroup (split,
//   k) walks its slice of map column k, compacts the valid (in, out) pairs in
//   LDS, stages 32 pairs at a time transposed (channel-major) in LDS and runs
//   MFMA with the pairs as the reduction dimension.  Per-split fp32 partials
//   are summed in a fixed order by a second kernel.
#pragma once

#include <type_traits>

#include "common.h"
#include "mfma.h"
#include "nbr_src.h"

namespace st {

constexpr int kGemmBM = 128;
constexpr int kSrcGroup = 32;  // offsets whose source rows are resolved into LDS at once
constexpr int kProbeGroup = 28;  // the same for table probes (a 3x3x3 kernel in one group)

template <typename T, int BN, typename Src, typename E>
__global__ __launch_bounds__(256) void gather_gemm_kernel(const T* __restrict__ A, Src src,
                                                          const uint32_t* __restrict__ masks, int W,
                                                          const int32_t* __restrict__ perm, const T* __restrict__ Bt,
                                                          T* __restrict__ out, int64_t n_src, int64_t n_dst, int K,
                                                          int Kd, int Nd, int vec_a, int vec_b,
                                                          E epi) {
  using F = typename Frag<T>::type;
  constexpr int VEC = Frag<T>::VEC;
  constexpr int KSTEP = Frag<T>::KSTEP;
  constexpr int KCH = sizeof(T) == 4 ? 64 : 128;  // reduction elements staged per pass
  constexpr int PITCH = KCH + VEC;                // LDS row pitch (elements), 16-byte multiple
  constexpr int NBLK = BN / 16;
  constexpr int CV = KCH / VEC;
  __shared__ __attribute__((aligned(16))) T bt_s[BN * PITCH];
  __shared__ uint32_t tmask_s[ST_MAX_KVOL / 32];
  __shared__ int32_t drow_s[kGemmBM];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * kGemmBM;
  const int n0 = blockIdx.y * BN;

  if (tid < kGemmBM) {
    const int64_t r = row0 + tid;
    drow_s[tid] = r < n_dst ? (perm ? perm[r] : (int32_t)r) : -1;
  }
  if (tid < W) tmask_s[tid] = 0;
  __syncthreads();
  if (masks) {
    for (int w = 0; w < W; ++w) {
      uint32_t v = 0;
      if (tid < kGemmBM && drow_s[tid] >= 0) v = masks[(int64_t)drow_s[tid] * W + w];
      v = wave_or(v);
      if (lane == 0 && v) atomicOr(&tmask_s[w], v);
    }
  } else if (tid < W) {
    tmask_s[tid] = (tid == W - 1 && (K & 31)) ? ((1u << (K & 31)) - 1u) : 0xFFFFFFFFu;
  }
  __syncthreads();

  // Lane (l & 31) resolves tile row wid*32 + (l & 31) (destination row
  // drow_s[...]); MFMA row c of tile m is then fetched from lane m*16 + c.
  const int32_t my_row = drow_s[wid * 32 + (lane & 31)];
  const bool my_ok = my_row >= 0;
  const typename Src::RowCtx rc = src.row(my_ok ? my_row : 0);

  v4f acc[2][NBLK];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) acc[m][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int w = 0; w < W; ++w) {
    uint32_t bits = tmask_s[w];
    while (bits) {
      const int k = w * 32 + __builtin_ctz(bits);
      bits &= bits - 1;
      int32_t s_own = my_ok ? src.get(rc, k) : -1;
      if ((int64_t)s_own >= n_src) s_own = -1;  // a caller's map entry past A: no contribution
      const int32_t s0 = __shfl(s_own, c, 64);
      const int32_t s1 = __shfl(s_own, 16 + c, 64);
      const bool wave_any = __ballot(s_own >= 0) != 0ull;
      for (int kc0 = 0; kc0 < Kd; kc0 += KCH) {
        __syncthreads();
        for (int idx = tid; idx < BN * CV; idx += 256) {
          const int nr = idx / CV, cv = idx - nr * CV;
          F f = zero_frag<T>();
          if (n0 + nr < Nd) f = load_frag<T>(Bt + ((int64_t)k * Nd + n0 + nr) * Kd, kc0 + cv * VEC, Kd, vec_b);
          *reinterpret_cast<F*>(&bt_s[nr * PITCH + cv * VEC]) = f;
        }
        __syncthreads();
        if (!wave_any) continue;
        const int kend = min(KCH, Kd - kc0);
        for (int kk = 0; kk < kend; kk += KSTEP) {
          const int col = kc0 + kk + g * VEC;
          const F a0 = s0 >= 0 ? load_frag<T>(A + (int64_t)s0 * Kd, col, Kd, vec_a) : zero_frag<T>();
          const F a1 = s1 >= 0 ? load_frag<T>(A + (int64_t)s1 * Kd, col, Kd, vec_a) : zero_frag<T>();
#pragma unroll
          for (int nb = 0; nb < NBLK; ++nb) {
            const F b = *reinterpret_cast<const F*>(&bt_s[(nb * 16 + c) * PITCH + kk + g * VEC]);
            acc[0][nb] = mfma(a0, b, acc[0][nb]);
            acc[1][nb] = mfma(a1, b, acc[1][nb]);
          }
        }
      }
    }
  }

  // per-column store epilogue (bias, optional affine map, optional ReLU)
  float em[NBLK], ea[NBLK];
#pragma unroll
  for (int nb = 0; nb < NBLK; ++nb) epi.column(n0 + nb * 16 + c, Nd, em[nb], ea[nb]);
  if constexpr (E::kReads) {
    // values first, stores after: an epilogue that reads (the residual) issues
    // all its loads before the first store, which may alias them
    float ov[2][4][NBLK];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          ov[m][r][nb] = (drow >= 0 && col < Nd) ? epi.apply(acc[m][nb][r], em[nb], ea[nb], drow, Nd, col) : 0.f;
        }
      }
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
        if (drow < 0) continue;
        T* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = from_f32<T>(ov[m][r][nb]);
        }
      }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
        if (drow < 0) continue;
        T* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = from_f32<T>(epi.apply(acc[m][nb][r], em[nb], ea[nb], drow, Nd, col));
        }
      }
  }
}

// Pipelined gather-GEMM for reduction depths known at compile time
// (Kd <= KS * KSTEP).  Per workgroup: the list of offsets present in the tile
// is built once; for offset i the B slice Bt[k_i] sits in LDS buffer i & 1
// while Bt[k_{i+1}] and the next offset's A rows are already in flight into
// registers, so global latency overlaps the MFMAs.  One barrier per offset.
// Tile row r is destination row rows[r] (the mask-sorted permutation) or r
// itself when rows is null; the map, the row masks and the hash-fly
// coordinates are indexed by destination row.
template <typename T, int BN, int KS, typename Src, typename E>
__global__ __launch_bounds__(256) void gather_gemm_pipe_kernel(
    const T* __restrict__ A, Src src, const uint32_t* __restrict__ masks, int W, const int32_t* __restrict__ rows,
    const T* __restrict__ Bt, T* __restrict__ out, int64_t n_src, int64_t n_dst, int K, int Kd, int Nd, int vec_a,
    int vec_b, E epi) {
  using F = typename Frag<T>::type;
  constexpr int VEC = Frag<T>::VEC;
  constexpr int KSTEP = Frag<T>::KSTEP;
  constexpr int KDP = KS * KSTEP;
  constexpr int PITCH = KDP + VEC;
  constexpr int NBLK = BN / 16;
  constexpr int CV = KDP / VEC;
  constexpr int BREGS = (BN * CV + 255) / 256;
  __shared__ __attribute__((aligned(16))) T bt_s[2][BN * PITCH];
  __shared__ uint32_t tmask_s[ST_MAX_KVOL / 32];
  __shared__ int32_t drow_s[kGemmBM];
  __shared__ int16_t klist_s[ST_MAX_KVOL];
  __shared__ int32_t src_s[kSrcGroup][kGemmBM];
  __shared__ int nk_s;

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int64_t row0 = (int64_t)blockIdx.x * kGemmBM;
  const int n0 = blockIdx.y * BN;

  if (tid < kGemmBM) {
    const int64_t r = row0 + tid;
    drow_s[tid] = r < n_dst ? (rows ? rows[r] : (int32_t)r) : -1;
  }
  if constexpr (Src::kTiled) {
    // the tile plan lists this tile's active offsets
    const int nkt = src.nk[blockIdx.x];
    for (int j = tid; j < nkt; j += 256) klist_s[j] = src.klist[(int64_t)blockIdx.x * src.K + j];
    if (tid == 0) nk_s = nkt;
  } else {
    if (tid < W) tmask_s[tid] = 0;
    __syncthreads();
    if (masks) {
      for (int w = 0; w < W; ++w) {
        uint32_t v = 0;
        if (tid < kGemmBM && drow_s[tid] >= 0) v = masks[(int64_t)drow_s[tid] * W + w];
        v = wave_or(v);
        if (lane == 0 && v) atomicOr(&tmask_s[w], v);
      }
    } else if (tid < W) {
      tmask_s[tid] = (tid == W - 1 && (K & 31)) ? ((1u << (K & 31)) - 1u) : 0xFFFFFFFFu;
    }
    __syncthreads();
    if (tid == 0) {
      int nk = 0;
      for (int w = 0; w < W; ++w) {
        uint32_t bits = tmask_s[w];
        while (bits) {
          klist_s[nk++] = (int16_t)(w * 32 + __builtin_ctz(bits));
          bits &= bits - 1;
        }
      }
      nk_s = nk;
    }
  }
  __syncthreads();
  const int nk = nk_s;

  // Source rows of a group of up to kSrcGroup offsets, resolved for the whole
  // tile at once (map loads / hash probes all in flight together) into LDS:
  // thread t owns tile row t & 127 and offsets (t >> 7) + 2j of the group.
  const int32_t ld_row = drow_s[tid & (kGemmBM - 1)];
  const typename Src::RowCtx rc = src.row(ld_row >= 0 ? ld_row : 0);
  auto resolve_group = [&](int g0) {
    const int ng = min(kSrcGroup, nk - g0);
    for (int j = tid >> 7; j < ng; j += 2) {
      int32_t v;
      if constexpr (Src::kTiled)
        v = src.get_tile(blockIdx.x, g0 + j, tid & (kGemmBM - 1));
      else
        v = ld_row >= 0 ? src.get(rc, klist_s[g0 + j]) : -1;
      if ((int64_t)v >= n_src) v = -1;
      src_s[j][tid & (kGemmBM - 1)] = v;
    }
  };
  auto sources = [&](int i, int32_t& s0, int32_t& s1) -> bool {
    const int j = i % kSrcGroup;
    s0 = src_s[j][wid * 32 + c];
    s1 = src_s[j][wid * 32 + 16 + c];
    return __ballot(s0 >= 0 || s1 >= 0) != 0ull;
  };
  auto load_a = [&](int32_t s0, int32_t s1, F (&a)[2][KS]) {
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const int col = j * KSTEP + g * VEC;
      a[0][j] = s0 >= 0 ? load_frag<T>(A + (int64_t)s0 * Kd, col, Kd, vec_a) : zero_frag<T>();
      a[1][j] = s1 >= 0 ? load_frag<T>(A + (int64_t)s1 * Kd, col, Kd, vec_a) : zero_frag<T>();
    }
  };
  auto load_b = [&](int k, F (&b)[BREGS]) {
#pragma unroll
    for (int j = 0; j < BREGS; ++j) {
      const int idx = tid + j * 256;
      const int nr = idx / CV, cv = idx - nr * CV;
      b[j] = zero_frag<T>();
      if (idx < BN * CV && n0 + nr < Nd)
        b[j] = load_frag<T>(Bt + ((int64_t)k * Nd + n0 + nr) * Kd, cv * VEC, Kd, vec_b);
    }
  };
  auto store_b = [&](int buf, const F (&b)[BREGS]) {
#pragma unroll
    for (int j = 0; j < BREGS; ++j) {
      const int idx = tid + j * 256;
      const int nr = idx / CV, cv = idx - nr * CV;
      if (idx < BN * CV) *reinterpret_cast<F*>(&bt_s[buf][nr * PITCH + cv * VEC]) = b[j];
    }
  };

  v4f acc[2][NBLK];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) acc[m][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  if (nk > 0) {
    F a_cur[2][KS], a_nxt[2][KS];
    F breg[BREGS];
    int32_t s0, s1;
    resolve_group(0);
    load_b(b_slice(src, klist_s[0]), breg);
    store_b(0, breg);
    __syncthreads();
    bool any_cur = sources(0, s0, s1);
    load_a(s0, s1, a_cur);
    for (int i = 0; i < nk; ++i) {
      const bool has_next = i + 1 < nk;
      bool any_nxt = false;
      if (has_next && (i + 1) % kSrcGroup == 0) {
        // every wave has read its sources of this group (they are in registers)
        __syncthreads();
        resolve_group(i + 1);
        __syncthreads();
      }
      if (has_next) {
        const int kn = b_slice(src, klist_s[i + 1]);
        int32_t t0, t1;
        any_nxt = sources(i + 1, t0, t1);
        load_a(t0, t1, a_nxt);
        load_b(kn, breg);
      }
      if (any_cur) {
        const T* bs = bt_s[i & 1];
#pragma unroll
        for (int j = 0; j < KS; ++j) {
#pragma unroll
          for (int nb = 0; nb < NBLK; ++nb) {
            const F b = *reinterpret_cast<const F*>(&bs[(nb * 16 + c) * PITCH + j * KSTEP + g * VEC]);
            acc[0][nb] = mfma(a_cur[0][j], b, acc[0][nb]);
            acc[1][nb] = mfma(a_cur[1][j], b, acc[1][nb]);
          }
        }
      }
      if (has_next) store_b((i + 1) & 1, breg);
      __syncthreads();
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int j = 0; j < KS; ++j) a_cur[m][j] = a_nxt[m][j];
      any_cur = any_nxt;
    }
  }

  // per-column store epilogue (bias, optional affine map, optional ReLU)
  float em[NBLK], ea[NBLK];
#pragma unroll
  for (int nb = 0; nb < NBLK; ++nb) epi.column(n0 + nb * 16 + c, Nd, em[nb], ea[nb]);
  if constexpr (E::kReads) {
    // values first, stores after: an epilogue that reads (the residual) issues
    // all its loads before the first store, which may alias them
    float ov[2][4][NBLK];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          ov[m][r][nb] = (drow >= 0 && col < Nd) ? epi.apply(acc[m][nb][r], em[nb], ea[nb], drow, Nd, col) : 0.f;
        }
      }
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
        if (drow < 0) continue;
        T* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = from_f32<T>(ov[m][r][nb]);
        }
      }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
        if (drow < 0) continue;
        T* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = from_f32<T>(epi.apply(acc[m][nb][r], em[nb], ea[nb], drow, Nd, col));
        }
      }
  }
}

// Row tile and column tile of a ring-kernel workgroup.  With one column tile
// the grid is the row tiles in order.  With several, the grid is 1-D over
// (row tiles rounded up to a multiple of 8) x (column tiles), and the column
// tiles of one row tile are consecutive workgroups of one XCD (the hardware
// deals workgroups to the 8 XCDs round-robin by id), so the A rows they all
// gather come into that XCD's L2 once.  Row tiles past the end are padding.
struct RingTile {
  int64_t rt;
  int ct;
};
// Row tiles run in descending order: destination rows are sorted by ascending
// offset-mask key, so the last row tiles hold the rows with the most
// neighbours (the costliest tiles); starting with them leaves the cheap tiles
// for the tail of the grid.
__device__ __forceinline__ RingTile ring_tile(int64_t n_dst, int Nd, int BN) {
  const int ncol = (Nd + BN - 1) / BN;
  const int64_t nrt = (n_dst + kGemmBM - 1) / kGemmBM;
  const int64_t b = blockIdx.x;
  if (ncol == 1) return RingTile{nrt - 1 - b, 0};
  const int64_t s = b >> 3, padded = (nrt + 7) / 8 * 8;
  return RingTile{padded - 1 - ((s / ncol) * 8 + (b & 7)), (int)(s % ncol)};
}
// Grid of the ring kernels for n_dst rows and Nd columns in BN-wide tiles.
static inline unsigned ring_grid(int64_t n_dst, int Nd, int BN) {
  const int64_t rt = (n_dst + kGemmBM - 1) / kGemmBM, ncol = (Nd + BN - 1) / BN;
  return (unsigned)(ncol == 1 ? rt : ((rt + 7) / 8) * 8 * ncol);
}

// ------------------------------------------ gather-GEMM, D-deep load ring
//
// As gather_gemm_pipe_kernel, but the A rows and the B tile of an offset are
// loaded D-1 offsets before they are used, into a ring of D register slots.
// Vector-memory loads complete in issue order, so the wait for offset i's
// loads at step i leaves the D-1 younger offsets' gathers in flight; with a
// single slot of look-ahead every step would wait out a full gather latency.
// Per step i: issue offset i+D-1's loads, store offset i's B tile into LDS
// (double-buffered), barrier, MFMAs on offset i.  Requires Kd a multiple of
// KS * KSTEP and 16-byte aligned A and Bt (every full-vector case).
template <typename T, int BN, int KS, int D, typename Src, bool LINES, typename E>
__global__ __launch_bounds__(256) void gather_gemm_ring_kernel(
    const T* __restrict__ A, Src src, const uint32_t* __restrict__ masks, int W, const int32_t* __restrict__ rows,
    const T* __restrict__ Bt, T* __restrict__ out, int64_t n_src, int64_t n_dst, int K, int Kd, int Nd, int vec_a,
    int vec_b, E epi) {
  using F = typename Frag<T>::type;
  constexpr int VEC = Frag<T>::VEC;
  constexpr int KSTEP = Frag<T>::KSTEP;
  constexpr int KDP = KS * KSTEP;
  constexpr int PITCH = KDP + VEC;
  constexpr int NBLK = BN / 16;
  constexpr int CV = KDP / VEC;
  constexpr int BREGS = (BN * CV + 255) / 256;
  // Whole-line A gathers (LINES): a row is CPR 16-byte chunks, an instruction
  // loads RPI whole rows (CPR lanes per row) and the 2 * KS instructions of a
  // step cover the wave's 32 rows; the rows pass through a per-wave LDS stage
  // (chunk ch of row r at position ch ^ (r mod CPR): conflict-free stores and
  // fragment reads) into the MFMA layout.  Fragment-shaped gathers instead
  // touch 16 cache lines per instruction for a part of each, and every line
  // twice, which backs up the L1 tag path when the rows hit in L2.
  constexpr int CPR = KDP / VEC;
  constexpr int RPI = 64 / CPR;
  static_assert(!LINES || (CPR >= 4 && CPR <= 16 && 2 * KS * RPI == 32), "whole-line gather shape");
  // offsets whose sources are resolved at once (fewer with the A stage, to keep 4 workgroups per CU;
  // a probing source resolves all of a 3x3x3 kernel's offsets in one batch)
  constexpr int SG = Src::kProbe ? kProbeGroup : (LINES ? 8 : kSrcGroup);
  // LINES: the B tile unpadded, chunk ch of row n at ch ^ bswz(n) -- the 16
  // rows one fragment read touches land on 16 distinct 4-bank groups
  constexpr int BPITCH = LINES ? KDP : PITCH;
  constexpr int BRPB = 16 / CV > 0 ? 16 / CV : 1;  // B rows per 256 bytes
  __shared__ __attribute__((aligned(16))) T bt_s[2][BN * BPITCH];
  __shared__ __attribute__((aligned(16))) T a_s[LINES ? 4 : 1][LINES ? 32 * KDP : VEC];
  __shared__ uint32_t tmask_s[ST_MAX_KVOL / 32];
  __shared__ int32_t drow_s[kGemmBM];
  __shared__ int16_t klist_s[ST_MAX_KVOL];
  __shared__ int32_t src_s[SG][kGemmBM];
  __shared__ int nk_s;
  // probing sources: the group's offsets with a source in the tile (bit j) and their list
  __shared__ uint32_t gmask_s;
  __shared__ int8_t jl_s[Src::kProbe ? SG : 1];
  __shared__ int gn_s;

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const RingTile tile = ring_tile(n_dst, Nd, BN);
  if (tile.rt * kGemmBM >= n_dst) return;  // padding of the folded grid (whole workgroup)
  const int64_t row0 = tile.rt * kGemmBM;
  const int n0 = tile.ct * BN;
  if (Src::kProbe && tid == 0) gmask_s = 0u;

  if (tid < kGemmBM) {
    const int64_t r = row0 + tid;
    drow_s[tid] = r < n_dst ? (rows ? rows[r] : (int32_t)r) : -1;
  }
  if constexpr (Src::kTiled) {
    const int nkt = src.nk[tile.rt];
    for (int j = tid; j < nkt; j += 256) klist_s[j] = src.klist[tile.rt * src.K + j];
    if (tid == 0) nk_s = nkt;
  } else {
    if (tid < W) tmask_s[tid] = 0;
    __syncthreads();
    if (masks) {
      for (int w = 0; w < W; ++w) {
        uint32_t v = 0;
        if (tid < kGemmBM && drow_s[tid] >= 0) v = masks[(int64_t)drow_s[tid] * W + w];
        v = wave_or(v);
        if (lane == 0 && v) atomicOr(&tmask_s[w], v);
      }
    } else if (tid < W) {
      tmask_s[tid] = (tid == W - 1 && (K & 31)) ? ((1u << (K & 31)) - 1u) : 0xFFFFFFFFu;
    }
    __syncthreads();
    if (tid == 0) {
      int nk = 0;
      for (int w = 0; w < W; ++w) {
        uint32_t bits = tmask_s[w];
        while (bits) {
          klist_s[nk++] = (int16_t)(w * 32 + __builtin_ctz(bits));
          bits &= bits - 1;
        }
      }
      nk_s = nk;
    }
  }
  __syncthreads();
  const int nk = nk_s;

  const int32_t ld_row = drow_s[tid & (kGemmBM - 1)];
  const typename Src::RowCtx rc = src.row(ld_row >= 0 ? ld_row : 0);
  // Sources of the group's offsets into src_s; returns how many of its offsets run.  A probing
  // source issues all its probes' first loads together (thread t: row t % 128, every other
  // offset from t / 128), then drops the offsets no row of the tile has (jl_s lists the rest).
  auto resolve_group = [&](int g0) -> int {
    const int ng = min(SG, nk - g0);
    if constexpr (Src::kProbe) {
      constexpr int PB = (SG + 1) / 2;
      const int half = tid >> 7, r = tid & (kGemmBM - 1);
      uint64_t key[PB], k0[PB];
      uint32_t slot[PB];
      bool ok[PB];
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        const int j = half + 2 * u;
        ok[u] = j < ng && ld_row >= 0 && src.prep(rc, klist_s[g0 + j], key[u], slot[u]);
      }
#pragma unroll
      for (int u = 0; u < PB; ++u) k0[u] = ok[u] ? src.keys[slot[u]] : ST_EMPTY_KEY;
      uint32_t hit[PB];
#pragma unroll
      for (int u = 0; u < PB; ++u) hit[u] = ok[u] ? find_slot_from(src.keys, src.cap, key[u], slot[u], k0[u]) : ST_NO_VAL;
      int32_t v[PB];
#pragma unroll
      for (int u = 0; u < PB; ++u) v[u] = hit[u] != ST_NO_VAL ? (int32_t)src.vals[hit[u]] : -1;
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        const int j = half + 2 * u;  // uniform across the wave
        if (j < ng) {
          const int32_t vv = (int64_t)v[u] >= n_src ? -1 : v[u];
          src_s[j][r] = vv;
          if (__ballot(vv >= 0) != 0ull && lane == 0) atomicOr(&gmask_s, 1u << j);
        }
      }
      __syncthreads();
      if (tid == 0) {
        uint32_t m = gmask_s;
        int n = 0;
        while (m) {
          jl_s[n++] = (int8_t)__builtin_ctz(m);
          m &= m - 1;
        }
        gn_s = n;
        gmask_s = 0u;  // the next group's bits come after at least one more barrier
      }
      __syncthreads();
      return gn_s;
    } else {
      // every load of the group in flight before the first is used
      constexpr int PB = (SG + 1) / 2;
      int32_t v[PB];
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        const int j = (tid >> 7) + 2 * u;  // uniform across the wave
        v[u] = -1;
        if (j < ng) {
          if constexpr (Src::kTiled)
            v[u] = src.get_tile(tile.rt, g0 + j, tid & (kGemmBM - 1));
          else
            v[u] = ld_row >= 0 ? src.get(rc, klist_s[g0 + j]) : -1;
        }
      }
#pragma unroll
      for (int u = 0; u < PB; ++u) {
        const int j = (tid >> 7) + 2 * u;
        if (j < ng) src_s[j][tid & (kGemmBM - 1)] = (int64_t)v[u] >= n_src ? -1 : v[u];
      }
      return ng;
    }
  };

  F a_ring[D][2][KS];  // LINES: a_ring[SL][v / KS][v % KS] holds instruction v's chunk
  F b_ring[D][BREGS];
  bool any_ring[D];
  v4f acc[2][NBLK];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) acc[m][nb] = v4f{0.f, 0.f, 0.f, 0.f};
  // element offset of 16-byte chunk ch of B row n
  auto bpos = [](int n, int ch) -> int {
    if constexpr (LINES)
      return n * BPITCH + (ch ^ ((n / BRPB) % CV)) * VEC;
    else
      return n * BPITCH + ch * VEC;
  };
  const int lr = lane / CPR, lc = lane % CPR;  // whole-line loader lanes: row in the instruction, chunk
  T* const a_w = a_s[LINES ? wid : 0];
  // LINES: buffer loads (the host keeps both arrays under 2 GB); missing rows read zeros
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(A, LINES ? n_src * Kd * (int64_t)sizeof(T) : 0);
  const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(Bt, LINES ? (int64_t)K * Nd * Kd * (int64_t)sizeof(T) : 0);

  // loads of offset i (its sources must be resolved) into ring slot SL
  auto issue = [&](int i, auto slot) {
    constexpr int SL = decltype(slot)::value;
    const int loc = i % SG;                          // position in the group's run list
    const int j = Src::kProbe ? jl_s[loc] : loc;     // the offset's index in the group
    if constexpr (LINES) {
      bool any = false;
#pragma unroll
      for (int v = 0; v < 2 * KS; ++v) {
        const int32_t sv = src_s[j][wid * 32 + v * RPI + lr];
        any |= sv >= 0;
        a_ring[SL][v / KS][v % KS] = load16<F>(a_rsrc, sv >= 0 ? sv * (Kd * (int)sizeof(T)) + lc * 16 : kOobOffset);
      }
      any_ring[SL] = __ballot(any) != 0ull;
    } else {
      const int32_t s0 = src_s[j][wid * 32 + c];
      const int32_t s1 = src_s[j][wid * 32 + 16 + c];
      any_ring[SL] = __ballot(s0 >= 0 || s1 >= 0) != 0ull;
      // Branch-free loads (invalid rows read row 0 and are zeroed): loads under
      // divergent branches would make the compiler drain the load queue.
      const F* ar0 = reinterpret_cast<const F*>(A + (int64_t)(s0 >= 0 ? s0 : 0) * Kd + g * VEC);
      const F* ar1 = reinterpret_cast<const F*>(A + (int64_t)(s1 >= 0 ? s1 : 0) * Kd + g * VEC);
#pragma unroll
      for (int jj = 0; jj < KS; ++jj) {
        a_ring[SL][0][jj] = ar0[jj * (KSTEP / VEC)];
        a_ring[SL][1][jj] = ar1[jj * (KSTEP / VEC)];
        if (s0 < 0) a_ring[SL][0][jj] = zero_frag<T>();
        if (s1 < 0) a_ring[SL][1][jj] = zero_frag<T>();
      }
    }
    const int k = b_slice(src, klist_s[i - loc + j]);
#pragma unroll
    for (int jb = 0; jb < BREGS; ++jb) {
      const int idx = tid + jb * 256;
      const int nr = idx / CV, cv = idx - nr * CV;
      const bool ok = idx < BN * CV && n0 + nr < Nd;
      if constexpr (LINES) {
        b_ring[SL][jb] = load16<F>(b_rsrc, ok ? ((k * Nd + n0 + nr) * Kd + cv * VEC) * (int)sizeof(T) : kOobOffset);
      } else {
        b_ring[SL][jb] = *reinterpret_cast<const F*>(Bt + ((int64_t)k * Nd + (ok ? n0 + nr : 0)) * Kd + cv * VEC);
        if (!ok) b_ring[SL][jb] = zero_frag<T>();
      }
    }
  };
  // Step i of a group of gn offsets starting at g0 (ring slot SL = i % D):
  // issue offset i + D - 1 (clamped to the group's last offset, so every step
  // issues the same loads and the compiler's load-queue accounting stays
  // exact), store offset i's B tile, barrier, MFMAs if offset i exists.
  auto step = [&](int g0, int gn, int i, auto slot) {
    constexpr int SL = decltype(slot)::value;
    constexpr int NSL = (SL + D - 1) % D;
    issue(g0 + min(i + D - 1, gn - 1), std::integral_constant<int, NSL>());
    const int buf = i & 1;
#pragma unroll
    for (int jb = 0; jb < BREGS; ++jb) {
      const int idx = tid + jb * 256;
      const int nr = idx / CV, cv = idx - nr * CV;
      if (idx < BN * CV) *reinterpret_cast<F*>(&bt_s[buf][bpos(nr, cv)]) = b_ring[SL][jb];
    }
    __syncthreads();
    if (i < gn && any_ring[SL]) {
      const T* bs = bt_s[buf];
      if constexpr (LINES) {
#pragma unroll
        for (int v = 0; v < 2 * KS; ++v) {
          const int r = v * RPI + lr;
          *reinterpret_cast<F*>(&a_w[r * KDP + (lc ^ (r & (CPR - 1))) * VEC]) = a_ring[SL][v / KS][v % KS];
        }
        // LDS operations of one wave complete in order; the fences keep the
        // compiler from moving the fragment reads above the stores.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
#pragma unroll
      for (int jj = 0; jj < KS; ++jj) {
        F a0, a1;
        if constexpr (LINES) {
          const int q = jj * (KSTEP / VEC) + g;
          a0 = *reinterpret_cast<const F*>(&a_w[c * KDP + (q ^ (c & (CPR - 1))) * VEC]);
          a1 = *reinterpret_cast<const F*>(&a_w[(16 + c) * KDP + (q ^ ((16 + c) & (CPR - 1))) * VEC]);
        } else {
          a0 = a_ring[SL][0][jj];
          a1 = a_ring[SL][1][jj];
        }
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const F b = *reinterpret_cast<const F*>(&bs[bpos(nb * 16 + c, jj * (KSTEP / VEC) + g)]);
          acc[0][nb] = mfma(a0, b, acc[0][nb]);
          acc[1][nb] = mfma(a1, b, acc[1][nb]);
        }
      }
    }
  };

  static_assert(D >= 2 && D <= 4, "ring depth 2..4");  // 2 is the one launched
  for (int g0 = 0; g0 < nk; g0 += SG) {
    if (g0 > 0) __syncthreads();  // the previous group's sources are all issued
    const int gn = resolve_group(g0);
    __syncthreads();
    if (gn == 0) continue;  // (uniform: no row of the tile has any of the group's offsets)
    issue(g0, std::integral_constant<int, 0>());
    if constexpr (D > 2) issue(g0 + min(1, gn - 1), std::integral_constant<int, 1>());
    if constexpr (D > 3) issue(g0 + min(2, gn - 1), std::integral_constant<int, 2>());
    for (int i0 = 0; i0 < gn; i0 += D) {
      step(g0, gn, i0, std::integral_constant<int, 0>());
      step(g0, gn, i0 + 1, std::integral_constant<int, 1 % D>());
      if constexpr (D > 2) step(g0, gn, i0 + 2, std::integral_constant<int, 2 % D>());
      if constexpr (D > 3) step(g0, gn, i0 + 3, std::integral_constant<int, 3 % D>());
    }
  }

  // per-column store epilogue (bias, optional affine map, optional ReLU)
  float em[NBLK], ea[NBLK];
#pragma unroll
  for (int nb = 0; nb < NBLK; ++nb) epi.column(n0 + nb * 16 + c, Nd, em[nb], ea[nb]);
  if constexpr (E::kReads) {
    // values first, stores after: an epilogue that reads (the residual) issues
    // all its loads before the first store, which may alias them
    float ov[2][4][NBLK];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          ov[m][r][nb] = (drow >= 0 && col < Nd) ? epi.apply(acc[m][nb][r], em[nb], ea[nb], drow, Nd, col) : 0.f;
        }
      }
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
        if (drow < 0) continue;
        T* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = from_f32<T>(ov[m][r][nb]);
        }
      }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
        if (drow < 0) continue;
        T* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = from_f32<T>(epi.apply(acc[m][nb][r], em[nb], ea[nb], drow, Nd, col));
        }
      }
  }
}

// ------------------------------------------- weight gradient over pair lists
//
// pairs: (in, out) int32 pairs sorted by (offset k, out); kstart[k] = first
// pair of offset k; the pair range of every offset is cut into chunks of
// `chunk` pairs (cstart[k] = first chunk of offset k, cstart[K] = total), so
// every workgroup task has the same size whatever the offset's density.
// Workgroups walk chunks with a grid stride; chunk c's C_in x C_out partial
// goes to partials[c] and the reduce kernel sums each offset's chunks in order.

// A workgroup's share of the (ordered) chunk list.  The hardware deals
// workgroups to the 8 XCDs round-robin by id; when the grid is a multiple of
// 8, XCD x takes the x-th eighth of the list and its workgroups walk it with a
// stride of their count, so the chunks running at once on an XCD are
// neighbours in the list -- in chunk order, the same output rows under every
// offset, and their input rows -- and share that XCD's L2.  (Contiguous runs
// per workgroup spread the resident workgroups over as many buckets of rows as
// there are workgroups: 43% L2 misses on config 5.)  Otherwise a plain grid
// stride.  Visit positions q0, q0 + step, ... below q1.
struct ChunkRange {
  int q0, q1, step;
};
__device__ __forceinline__ ChunkRange chunk_range(int total) {
  const int G = gridDim.x, b = blockIdx.x;
  if (G % 8 != 0) return ChunkRange{b, total, G};
  const int x = b & 7, per = G / 8;
  return ChunkRange{(int)((int64_t)x * total / 8) + (b >> 3), (int)((int64_t)(x + 1) * total / 8), per};
}

// Chunk walk and channel tile of a workgroup in a 1-D grid of G x ntiles
// workgroups: as chunk_range, with consecutive workgroups of one XCD taking
// the ntiles channel tiles of one chunk, so the rows they all read come into
// that XCD's L2 once.
struct ChunkTile {
  int q0, q1, step, tile;
};
__device__ __forceinline__ ChunkTile chunk_tile(int total, int ntiles) {
  const int b = (int)blockIdx.x, G = (int)gridDim.x / ntiles;
  if (G % 8 != 0) return ChunkTile{b / ntiles, total, G, b % ntiles};
  const int x = b & 7, s = b >> 3, per = G / 8;
  return ChunkTile{(int)((int64_t)x * total / 8) + s / ntiles, (int)((int64_t)(x + 1) * total / 8), per, s % ntiles};
}

__device__ __forceinline__ int chunk_offset(const int32_t* cstart_s, int K, int c) {
  int lo = 0, hi = K - 1;  // largest k with cstart[k] <= c
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cstart_s[mid] <= c) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// fp32: every lane gathers its own MFMA operands straight from HBM/L2
// (16 lanes read 16 consecutive channels of one pair's row), no LDS staging.
// A wave owns an MT x NT grid of 16x16 blocks; when the workgroup's channel
// tile has fewer than 4 wave tiles, waves split the chunk's pairs and sum
// through LDS at the end.
template <int MT, int NT>
__global__ __launch_bounds__(256) void wgrad_pairs_f32_kernel(const float* __restrict__ X, const float* __restrict__ dY,
                                                              const int2* __restrict__ pairs,
                                                              const int32_t* __restrict__ kstart,
                                                              const int32_t* __restrict__ cstart, const int32_t* __restrict__ chunk_order,
    int K, int chunk,
                                                              int Cin, int Cout, float* __restrict__ partials) {
  __shared__ int32_t cstart_s[ST_MAX_KVOL + 2];
  __shared__ float red_s[3][MT * NT * 4][64];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  for (int t = tid; t <= K + (chunk <= 0); t += 256) cstart_s[t] = cstart[t];  // + the size, when chosen by the list
  __syncthreads();
  const int total = cstart_s[K];

  const int MB = (Cin + 15) / 16, NB = (Cout + 15) / 16;
  const int WM = (MB + MT - 1) / MT, WN = (NB + NT - 1) / NT;
  const int wt0 = blockIdx.z * 4;
  const int nt = min(4, WM * WN - wt0);
  const int nphase = nt == 1 ? 4 : (nt == 2 ? 2 : 1);
  const int my_t = wid % (nt == 3 ? 4 : nt);
  const int phase = nt == 3 ? 0 : wid / nt;
  const bool active = my_t < nt;
  const int wt = wt0 + my_t;
  const int cm0 = (wt / WN) * MT * 16, cn0 = (wt % WN) * NT * 16;

  const ChunkRange cr = chunk_range(total);
  for (int cq = cr.q0; cq < cr.q1; cq += cr.step) {
    const int cidx = chunk_order ? chunk_order[cq] : cq;
    const int k = chunk_offset(cstart_s, K, cidx);
    const int ch = chunk > 0 ? chunk : cstart_s[K + 1];  // the plan's own size when not given
    const int p0 = kstart[k] + (cidx - cstart_s[k]) * ch;
    const int p1 = min(p0 + ch, kstart[k + 1]);
    v4f acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    if (active) {
#pragma unroll 4
      for (int q = p0 + phase * 4; q < p1; q += 4 * nphase) {
        const int p = q + g;
        int2 pr = make_int2(-1, -1);
        if (p < p1) pr = pairs[p];
        float a[MT], b[NT];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const int ch = cm0 + i * 16 + c;
          a[i] = (pr.x >= 0 && ch < Cin) ? X[(int64_t)pr.x * Cin + ch] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int ch = cn0 + j * 16 + c;
          b[j] = (pr.y >= 0 && ch < Cout) ? dY[(int64_t)pr.y * Cout + ch] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
    if (nphase > 1) {
      if (active && phase > 0) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red_s[(phase - 1) * nt + my_t][(i * NT + j) * 4 + r][lane] = acc[i][j][r];
      }
      __syncthreads();
      if (active && phase == 0) {
        for (int ph = 1; ph < nphase; ++ph)
#pragma unroll
          for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[i][j][r] += red_s[(ph - 1) * nt + my_t][(i * NT + j) * 4 + r][lane];
      }
    }
    if (active && phase == 0) {
      float* part = partials + (int64_t)cidx * Cin * Cout;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          const int col = cn0 + j * 16 + c;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = cm0 + i * 16 + g * 4 + r;
            if (row < Cin && col < Cout) part[(int64_t)row * Cout + col] = acc[i][j][r];
          }
        }
    }
    __syncthreads();
  }
}

// 16-bit: a batch of 64 pairs is staged in LDS channel-major (the MFMA
// reduction runs over pairs, which are rows in HBM), then each wave runs its
// share of the workgroup's 16x16 output blocks.
constexpr int kWpQB = 64;
template <typename T, int JB>  // JB: 16x16 output blocks per wave (4 waves x JB >= blocks of the tile)
__global__ __launch_bounds__(256) void wgrad_pairs_lds_kernel(const T* __restrict__ X, const T* __restrict__ dY,
                                                              const int2* __restrict__ pairs,
                                                              const int32_t* __restrict__ kstart,
                                                              const int32_t* __restrict__ cstart, const int32_t* __restrict__ chunk_order,
    int K, int chunk,
                                                              int Cin, int Cout, float* __restrict__ partials,
                                                              int vec_x, int vec_y) {
  using F = typename Frag<T>::type;
  constexpr int VEC = Frag<T>::VEC;
  constexpr int KSTEP = Frag<T>::KSTEP;
  constexpr int PITCH = kWpQB + 8;
  constexpr int TB = 8;  // 16x16 blocks per side of the workgroup tile (128 channels)
  __shared__ int32_t cstart_s[ST_MAX_KVOL + 2];
  __shared__ int2 pr_s[kWpQB];
  __shared__ __attribute__((aligned(16))) T xt_s[TB * 16 * PITCH];
  __shared__ __attribute__((aligned(16))) T yt_s[TB * 16 * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  for (int t = tid; t <= K + (chunk <= 0); t += 256) cstart_s[t] = cstart[t];  // + the size, when chosen by the list
  __syncthreads();
  const int total = cstart_s[K];

  const int MB = (Cin + 15) / 16, NB = (Cout + 15) / 16;
  const int nzn = (NB + TB - 1) / TB;
  const int mz = blockIdx.z / nzn, nz = blockIdx.z % nzn;
  const int mb0 = mz * TB, nb0 = nz * TB;
  const int MT = min(TB, MB - mb0), NT = min(TB, NB - nb0);
  const int nloc = MT * NT;
  const int cm0 = mb0 * 16, cn0 = nb0 * 16;
  const int CVX = (MT * 16) / VEC, CVY = (NT * 16) / VEC;

  const ChunkRange cr = chunk_range(total);
  for (int cq = cr.q0; cq < cr.q1; cq += cr.step) {
    const int cidx = chunk_order ? chunk_order[cq] : cq;
    const int k = chunk_offset(cstart_s, K, cidx);
    const int ch = chunk > 0 ? chunk : cstart_s[K + 1];  // the plan's own size when not given
    const int p0 = kstart[k] + (cidx - cstart_s[k]) * ch;
    const int p1 = min(p0 + ch, kstart[k + 1]);
    v4f acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int q0 = p0; q0 < p1; q0 += kWpQB) {
      const int nq = min(kWpQB, p1 - q0);
      if (tid < kWpQB) pr_s[tid] = tid < nq ? pairs[q0 + tid] : make_int2(-1, -1);
      __syncthreads();
      for (int idx = tid; idx < kWpQB * CVX; idx += 256) {
        const int p = idx / CVX, cv = idx - p * CVX;
        F f = zero_frag<T>();
        const int32_t i = pr_s[p].x;
        if (i >= 0) f = load_frag<T>(X + (int64_t)i * Cin, cm0 + cv * VEC, Cin, vec_x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) xt_s[(cv * VEC + e) * PITCH + p] = f[e];
      }
      for (int idx = tid; idx < kWpQB * CVY; idx += 256) {
        const int p = idx / CVY, cv = idx - p * CVY;
        F f = zero_frag<T>();
        const int32_t o = pr_s[p].y;
        if (o >= 0) f = load_frag<T>(dY + (int64_t)o * Cout, cn0 + cv * VEC, Cout, vec_y);
#pragma unroll
        for (int e = 0; e < VEC; ++e) yt_s[(cv * VEC + e) * PITCH + p] = f[e];
      }
      __syncthreads();
#pragma unroll
      for (int ps = 0; ps < kWpQB; ps += KSTEP) {
#pragma unroll
        for (int jj = 0; jj < JB; ++jj) {
          const int j = wid + 4 * jj;
          if (j < nloc) {
            const int mb = j / NT, nb = j - mb * NT;
            const F a = *reinterpret_cast<const F*>(&xt_s[(mb * 16 + c) * PITCH + ps + g * VEC]);
            const F b = *reinterpret_cast<const F*>(&yt_s[(nb * 16 + c) * PITCH + ps + g * VEC]);
            acc[jj] = mfma(a, b, acc[jj]);
          }
        }
      }
      __syncthreads();
    }
    float* part = partials + (int64_t)cidx * Cin * Cout;
#pragma unroll
    for (int jj = 0; jj < JB; ++jj) {
      const int j = wid + 4 * jj;
      if (j < nloc) {
        const int mb = j / NT, nb = j - mb * NT;
        const int col = cn0 + nb * 16 + c;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = cm0 + mb * 16 + g * 4 + r;
          if (row < Cin && col < Cout) part[(int64_t)row * Cout + col] = acc[jj][r];
        }
      }
    }
  }
}

// 16-bit, one MFMA k-step (32 pairs) per wave at a time, no workgroup barrier
// inside a chunk: the four waves take the chunk's 32-pair steps round-robin.
// Each wave stages its step's X and dY rows in its own LDS area row-major
// (pair-major, 16-byte stores straight from the gathered rows) and reads the
// MFMA fragments -- 8 pairs of one channel per lane -- with transpose LDS
// reads (tr_frag; pair p of a step lives in LDS row p, both operands take the
// same pairs per lane group).
// The wave tile is the workgroup's whole 64 x 64 channel tile (16 blocks);
// the waves' accumulators are summed through LDS once per chunk.  Requires
// C_in and C_out multiples of 64 and 16-byte aligned rows.
constexpr int kWvPitch = 80;
// MFMA operand fragment of a 32-pair step staged row-major (pitch kWvPitch
// 16-bit elements): lane (c, g) gets channel col0 + c of pairs 4g .. 4g+3 and
// 16 + 4g .. 16 + 4g+3, with two gfx950 transpose reads (ds_read_b64_tr_b16).
// Within a 16-lane group such a read hands lane l the element l mod 4 of the
// 4 elements lane 4e + l/4 addresses, for e = 0..3; so lane c addresses pair
// 16h + 4g + c/4 at channel col0 + 4 (c mod 4) and receives channel col0 + c
// of pairs 16h + 4g + e.  (Both operands take the same pairs, so the sum is the
// step's; which pairs a lane group takes only decides the banks: the two
// groups of a half-wave read rows 0-3 and 4-7 of an 8-row block, which the
// 80- and 144-element pitches put on eight distinct 32-byte bank groups --
// groups 8 rows apart, the earlier assignment, met on the same banks.)
template <typename F, typename T, int PITCH = kWvPitch>
__device__ __forceinline__ F tr_frag(const T* st, int g, int c, int col0) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef short v8s __attribute__((ext_vector_type(8)));
  using lds_v4s = __attribute__((address_space(3))) v4s;
  const T* p0 = st + (g * 4 + (c >> 2)) * PITCH + col0 + (c & 3) * 4;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p0));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p0 + 16 * PITCH));
  const v8s both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(F, both);
}

// Row pitch (16-bit elements) of a per-wave stage of rows `width` channels
// wide: the transpose reads of a fragment touch four rows at once, which land
// on distinct 32-byte bank groups when the row stride is 32 or 96 bytes
// modulo 128 (16, 48 or 80 elements).
constexpr int wave_pitch(int width) { return width == 16 ? 16 : (width == 32 ? 48 : (width == 64 ? 80 : 144)); }
// Channel tile of a workgroup: TM = 16 MB input channels x TN = 16 NB output
// channels (16, 32, 64 or 128 each; a wave computes the whole tile).  A row's
// TM channels are CPR = TM / 8 chunks of 16 bytes, so one load instruction
// covers RPI = 64 / CPR whole rows and a 32-pair step takes 32 / RPI of them.
// ONEPASS sums the four waves' tiles through LDS in one round (more LDS: two
// workgroups per CU for a 64 x 64 tile) instead of rounds of 32 rows (three).
// A 128-wide side (BIG) halves the LDS bytes per MFMA of the 64 x 64 tile --
// every staged row and every fragment read serves twice the MFMAs, the
// LDS-bound part of this kernel -- at one workgroup per CU (the 128 x 128
// accumulators take the AGPRs); its pair indices are then loaded a step ahead
// as with ONEPASS.
template <typename T, bool BUF, int MB, int NB, bool ONEPASS>  // BUF: row loads through buffer resources (X and dY under 2 GB)
__global__ __launch_bounds__(256, (MB > 4 || NB > 4) ? 1 : (ONEPASS ? 2 : 3)) void wgrad_pairs_wave_kernel(const T* __restrict__ X, const T* __restrict__ dY,
                                                               const int2* __restrict__ pairs,
                                                               const int32_t* __restrict__ kstart,
                                                               const int32_t* __restrict__ cstart, const int32_t* __restrict__ chunk_order,
    int K, int chunk,
                                                               int Cin, int Cout, int64_t n_in, int64_t n_out, float* __restrict__ partials) {
  using F = typename Frag<T>::type;
  static_assert(Frag<T>::KSTEP == 32 && Frag<T>::VEC == 8, "16-bit MFMA fragments");
  constexpr bool BIG = MB > 4 || NB > 4;
  constexpr bool PREFETCH = ONEPASS || BIG;  // pair indices one step ahead of their rows
  static_assert(!(ONEPASS && BIG), "a 128-wide tile sums in rounds");
  constexpr int TM = 16 * MB, TN = 16 * NB;
  constexpr int CPRX = TM / 8, RPIX = 64 / CPRX, NVX = 32 / RPIX;
  constexpr int CPRY = TN / 8, RPIY = 64 / CPRY, NVY = 32 / RPIY;
  constexpr int PX = wave_pitch(TM), PY = wave_pitch(TN);
  constexpr int STAGE = 32 * (PX + PY);  // elements per wave (X rows, then dY rows)
  constexpr int STAGE_BYTES = 4 * STAGE * (int)sizeof(T);
  constexpr int RP = TN + 4;            // row pitch (floats) of the per-wave tiles summed at the end
  constexpr int RH = (ONEPASS || TM < 32) ? TM : 32;  // rows summed per round
  constexpr int RED_BYTES = 4 * RH * RP * (int)sizeof(float);
  __shared__ int32_t cstart_s[ST_MAX_KVOL + 2];
  __shared__ __attribute__((aligned(16))) unsigned char lds[STAGE_BYTES > RED_BYTES ? STAGE_BYTES : RED_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  for (int t = tid; t <= K + (chunk <= 0); t += 256) cstart_s[t] = cstart[t];  // + the size, when chosen by the list
  __syncthreads();
  const int total = cstart_s[K];

  const int ntn = Cout / TN;
  const ChunkTile ct = chunk_tile(total, (Cin / TM) * ntn);
  const int cm0 = (ct.tile / ntn) * TM, cn0 = (ct.tile % ntn) * TN;
  T* xs = reinterpret_cast<T*>(lds) + wid * STAGE;
  T* ys = xs + 32 * PX;
  float* red = reinterpret_cast<float*>(lds);
  // loader lanes: lane / CPR is the row within an instruction's RPI rows, lane % CPR its chunk;
  // each lane keeps pair (lane mod 32) and takes instruction v's row index from lane v RPI + lane / CPR
  const int lrx = lane / CPRX, lcx = lane % CPRX, lry = lane / CPRY, lcy = lane % CPRY;
  const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(X, BUF ? n_in * Cin * (int64_t)sizeof(T) : 0);
  const __amdgpu_buffer_rsrc_t y_rsrc = make_rsrc(dY, BUF ? n_out * Cout * (int64_t)sizeof(T) : 0);

  for (int cq = ct.q0; cq < ct.q1; cq += ct.step) {
    const int cidx = chunk_order ? chunk_order[cq] : cq;
    const int k = chunk_offset(cstart_s, K, cidx);
    const int ch = chunk > 0 ? chunk : cstart_s[K + 1];  // the plan's own size when not given
    const int p0 = kstart[k] + (cidx - cstart_s[k]) * ch;
    const int p1 = min(p0 + ch, kstart[k + 1]);
    v4f acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    F xr[NVX], yr[NVY];
    // At two workgroups per CU (ONEPASS) the pair indices of a step are loaded
    // one step ahead of its rows, so a step's row gathers never wait for an
    // index load issued just before them; at three, the other waves hide that
    // latency and the plain order measures faster (config 5: 3.70 vs 4.05 ms).
    auto load_pairs = [&](int q) {
      const int p = q + (lane & 31);
      return p < p1 ? pairs[p] : make_int2(-1, -1);
    };
    auto load_rows = [&](int2 pr) {
      // X and dY loads interleaved (x0, y0, x1, y1, ...)
#pragma unroll
      for (int v = 0; v < (NVX > NVY ? NVX : NVY); ++v) {
        if (v < NVX) {
          const int ix = __shfl(pr.x, v * RPIX + lrx, 64);
          if constexpr (BUF)
            xr[v] = load16<F>(x_rsrc, ix >= 0 ? (ix * Cin + cm0 + lcx * 8) * (int)sizeof(T) : kOobOffset);
          else
            xr[v] = ix >= 0 ? *reinterpret_cast<const F*>(X + (int64_t)ix * Cin + cm0 + lcx * 8) : zero_frag<T>();
        }
        if (v < NVY) {
          const int iy = __shfl(pr.y, v * RPIY + lry, 64);
          if constexpr (BUF)
            yr[v] = load16<F>(y_rsrc, iy >= 0 ? (iy * Cout + cn0 + lcy * 8) * (int)sizeof(T) : kOobOffset);
          else
            yr[v] = iy >= 0 ? *reinterpret_cast<const F*>(dY + (int64_t)iy * Cout + cn0 + lcy * 8) : zero_frag<T>();
        }
      }
    };
    int q = p0 + wid * 32;
    int2 prn = load_pairs(q);
    if (q < p1) load_rows(prn);
    if constexpr (PREFETCH) prn = load_pairs(q + 128);
    for (; q < p1; q += 128) {
#pragma unroll
      for (int v = 0; v < (NVX > NVY ? NVX : NVY); ++v) {
        if (v < NVX) *reinterpret_cast<F*>(&xs[(v * RPIX + lrx) * PX + lcx * 8]) = xr[v];
        if (v < NVY) *reinterpret_cast<F*>(&ys[(v * RPIY + lry) * PY + lcy * 8]) = yr[v];
      }
      // LDS operations of one wave complete in order: the reads below see the
      // stores above; the fence keeps the compiler from moving them across.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (q + 128 < p1) {
        if constexpr (PREFETCH) {
          load_rows(prn);
          prn = load_pairs(q + 256);
        } else {
          load_rows(load_pairs(q + 128));
        }
      }
      F a[MB], b[NB];
#pragma unroll
      for (int i = 0; i < MB; ++i) a[i] = tr_frag<F, T, PX>(xs, g, c, i * 16);
#pragma unroll
      for (int j = 0; j < NB; ++j) b[j] = tr_frag<F, T, PY>(ys, g, c, j * 16);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = mfma(a[i], b[j], acc[i][j]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // sum the four waves' tiles through LDS, RH rows at a time (so the sum
    // area fits in the staging area); every thread then adds and stores
    // elements of each round's rows of the TM x TN partial, row-contiguous
    float* part = partials + (int64_t)cidx * Cin * Cout;
#pragma unroll
    for (int h = 0; h < TM / RH; ++h) {
      __syncthreads();
      float* mine = red + wid * RH * RP;
#pragma unroll
      for (int i = 0; i < RH / 16; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) mine[(i * 16 + g * 4 + r) * RP + j * 16 + c] = acc[h * (RH / 16) + i][j][r];
      __syncthreads();
      for (int e = tid; e < RH * TN; e += 256) {
        const int row = e / TN, col = e % TN;
        const float s = red[row * RP + col] + red[RH * RP + row * RP + col] + red[2 * RH * RP + row * RP + col] +
                        red[3 * RH * RP + row * RP + col];
        part[(int64_t)(cm0 + h * RH + row) * Cout + cn0 + col] = s;
      }
    }
    __syncthreads();
  }
}

// dW[k][e] = sum of partials[c][e] over offset k's chunks.  A 256-thread block
// covers 32 consecutive elements of one offset; its 8 thread groups take the
// chunks round-robin and are combined in a fixed order (deterministic).
template <typename TW>
__global__ __launch_bounds__(256) void wgrad_pairs_reduce_kernel(const float* __restrict__ partials,
                                                                 const int32_t* __restrict__ cstart, int64_t per_k,
                                                                 int K, TW* __restrict__ dW) {
  __shared__ float red[8][32];
  const int64_t blocks_per_k = (per_k + 31) / 32;
  const int64_t k = blockIdx.x / blocks_per_k;
  const int64_t e = (blockIdx.x - k * blocks_per_k) * 32 + (threadIdx.x & 31);
  const int part = threadIdx.x >> 5;
  float s = 0.f;
  if (e < per_k)
    for (int cidx = cstart[k] + part; cidx < cstart[k + 1]; cidx += 8) s += partials[(int64_t)cidx * per_k + e];
  red[part][threadIdx.x & 31] = s;
  __syncthreads();
  if (part == 0 && e < per_k) {
    float t = red[0][threadIdx.x];
#pragma unroll
    for (int j = 1; j < 8; ++j) t += red[j][threadIdx.x];
    dW[k * per_k + e] = from_f32<TW>(t);
  }
}

// Vector form of the sum above for per_k % 4 == 0 and 16-byte aligned
// partials: a workgroup sums 64 consecutive elements of one offset as 16
// lanes of float4 times 16 parts; part p takes chunks p, p + 16, ... with four
// loads in flight, and the parts are added in part order (deterministic).
// Sixteen parts keep the centre offset of a submanifold map, which owns far
// more chunks than the others, from becoming one long dependent load chain.
template <typename TW>
__global__ __launch_bounds__(256) void wgrad_pairs_reduce4_kernel(const float* __restrict__ partials,
                                                                  const int32_t* __restrict__ cstart, int64_t per_k,
                                                                  int K, TW* __restrict__ dW) {
  __shared__ float4 red[16][16];
  const int64_t blocks_per_k = (per_k + 63) / 64;
  const int64_t k = blockIdx.x / blocks_per_k;
  const int lane = threadIdx.x & 15, part = threadIdx.x >> 4;
  const int64_t e = (blockIdx.x - k * blocks_per_k) * 64 + lane * 4;
  float4 s0 = make_float4(0.f, 0.f, 0.f, 0.f), s1 = s0, s2 = s0, s3 = s0;
  if (e < per_k) {
    const float* p = partials + e;
    const int c1 = cstart[k + 1];
    int c = cstart[k] + part;
    for (; c + 48 < c1; c += 64) {
      const float4 a = *(const float4*)(p + (int64_t)c * per_k);
      const float4 b = *(const float4*)(p + (int64_t)(c + 16) * per_k);
      const float4 d = *(const float4*)(p + (int64_t)(c + 32) * per_k);
      const float4 f = *(const float4*)(p + (int64_t)(c + 48) * per_k);
      s0 += a;
      s1 += b;
      s2 += d;
      s3 += f;
    }
    for (; c < c1; c += 16) s0 += *(const float4*)(p + (int64_t)c * per_k);
  }
  red[part][lane] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (part == 0 && e < per_k) {
    float4 t = red[0][lane];
#pragma unroll
    for (int j = 1; j < 16; ++j) t += red[j][lane];
    TW* o = dW + k * per_k + e;
    o[0] = from_f32<TW>(t.x);
    o[1] = from_f32<TW>(t.y);
    o[2] = from_f32<TW>(t.z);
    o[3] = from_f32<TW>(t.w);
  }
}

constexpr int kWgQB = 32;       // pairs per MFMA batch
constexpr int kWgRows = 1024;   // map rows compacted per step (4 per thread)
constexpr int kWgTileBlk = 8;   // 16x16 blocks per workgroup sub-tile side (128 channels)

template <typename T, typename Src>
__global__ __launch_bounds__(256) void wgrad_kernel(const T* __restrict__ X, const T* __restrict__ dY, Src src,
                                                    int64_t n_in, int64_t n_out, int Cin, int Cout,
                                                    int64_t rows_per_split,
                                                    int splits, float* __restrict__ partials, int vec_x, int vec_y) {
  using F = typename Frag<T>::type;
  constexpr int VEC = Frag<T>::VEC;
  constexpr int KSTEP = Frag<T>::KSTEP;
  constexpr int PITCH = kWgQB + (sizeof(T) == 4 ? 4 : 8);
  constexpr int CH = kWgTileBlk * 16;
  __shared__ int32_t qin_s[kWgRows];
  __shared__ int32_t qout_s[kWgRows];
  __shared__ __attribute__((aligned(16))) T xt_s[CH * PITCH];
  __shared__ __attribute__((aligned(16))) T yt_s[CH * PITCH];
  __shared__ int scan_s[5];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int split = blockIdx.x, k = blockIdx.y;
  const int MB = (Cin + 15) / 16, NB = (Cout + 15) / 16;
  const int nzn = (NB + kWgTileBlk - 1) / kWgTileBlk;
  const int mz = blockIdx.z / nzn, nz = blockIdx.z % nzn;
  const int mb0 = mz * kWgTileBlk, nb0 = nz * kWgTileBlk;
  const int MT = min(kWgTileBlk, MB - mb0), NT = min(kWgTileBlk, NB - nb0);
  const int nloc = MT * NT;
  const int cm0 = mb0 * 16, cn0 = nb0 * 16;

  v4f acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int64_t o_begin = (int64_t)split * rows_per_split;
  const int64_t o_end = min(n_out, o_begin + rows_per_split);
  const int CVX = (MT * 16) / VEC, CVY = (NT * 16) / VEC;

  for (int64_t base = o_begin; base < o_end; base += kWgRows) {
    int32_t ins[4];
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t o = base + tid * 4 + j;
      ins[j] = -1;
      if (o < o_end) ins[j] = src.get(src.row(o), k);
      if ((int64_t)ins[j] >= n_in) ins[j] = -1;  // a caller's map entry past X: no contribution
      cnt += ins[j] >= 0;
    }
    int total;
    int pos = block_exclusive_scan(cnt, scan_s, &total);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (ins[j] >= 0) {
        qin_s[pos] = ins[j];
        qout_s[pos] = (int32_t)(base + tid * 4 + j);
        ++pos;
      }
    __syncthreads();
    for (int q0 = 0; q0 < total; q0 += kWgQB) {
      const int nq = min(kWgQB, total - q0);
      for (int idx = tid; idx < kWgQB * CVX; idx += 256) {
        const int p = idx / CVX, cv = idx - p * CVX;
        F f = zero_frag<T>();
        if (p < nq) f = load_frag<T>(X + (int64_t)qin_s[q0 + p] * Cin, cm0 + cv * VEC, Cin, vec_x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) xt_s[(cv * VEC + e) * PITCH + p] = f[e];
      }
      for (int idx = tid; idx < kWgQB * CVY; idx += 256) {
        const int p = idx / CVY, cv = idx - p * CVY;
        F f = zero_frag<T>();
        if (p < nq) f = load_frag<T>(dY + (int64_t)qout_s[q0 + p] * Cout, cn0 + cv * VEC, Cout, vec_y);
#pragma unroll
        for (int e = 0; e < VEC; ++e) yt_s[(cv * VEC + e) * PITCH + p] = f[e];
      }
      __syncthreads();
#pragma unroll
      for (int ps = 0; ps < kWgQB; ps += KSTEP) {
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) {
          const int j = wid + 4 * jj;
          if (j < nloc) {
            const int mb = j / NT, nb = j - mb * NT;
            const F a = *reinterpret_cast<const F*>(&xt_s[(mb * 16 + c) * PITCH + ps + g * VEC]);
            const F b = *reinterpret_cast<const F*>(&yt_s[(nb * 16 + c) * PITCH + ps + g * VEC]);
            acc[jj] = mfma(a, b, acc[jj]);
          }
        }
      }
      __syncthreads();
    }
  }

  float* part = partials + ((int64_t)k * splits + split) * (int64_t)Cin * Cout;
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    const int j = wid + 4 * jj;
    if (j < nloc) {
      const int mb = j / NT, nb = j - mb * NT;
      const int col = cn0 + nb * 16 + c;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = cm0 + mb * 16 + g * 4 + r;
        if (row < Cin && col < Cout) part[(int64_t)row * Cout + col] = acc[jj][r];
      }
    }
  }
}

template <typename T>
__global__ void wgrad_reduce_kernel(const float* __restrict__ partials, int64_t per_k, int splits, int K,
                                    T* __restrict__ dW) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= per_k * K) return;
  const int64_t k = i / per_k, e = i - k * per_k;
  const float* p = partials + k * splits * per_k + e;
  float s = 0.f;
  for (int j = 0; j < splits; ++j) s += p[(int64_t)j * per_k];
  dW[i] = from_f32<T>(s);
}

template <typename T>
__global__ void weight_prep_kernel(const T* __restrict__ w, T* __restrict__ out, int K, int Cin, int Cout, int mode) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)K * Cin * Cout;
  if (i >= total) return;
  if (mode == ST_W_TRANSPOSE) {
    // i indexes out[k][co][ci]
    const int64_t k = i / ((int64_t)Cin * Cout);
    const int64_t rem = i - k * Cin * Cout;
    const int64_t co = rem / Cin, ci = rem - co * Cin;
    out[i] = w[(k * Cin + ci) * Cout + co];
  } else if (mode == ST_W_REVERSE) {
    const int64_t k = i / ((int64_t)Cin * Cout);
    const int64_t rem = i - k * Cin * Cout;
    out[i] = w[(K - 1 - k) * Cin * Cout + rem];
  } else {
    out[i] = w[i];
  }
}

// ---------------------------------------------------------------- dispatch
//
// Typed launchers, instantiated once per dtype in gemm_{f32,f16,bf16}.hip.

// Gather-GEMM look-ahead: ST_GEMM_RING=1 selects the one-offset pipelined
// kernel instead of the two-slot ring kernel (comparison runs only).  Depth 2
// measured fastest on MI355X (config 2, bf16: 90 us vs 107 us at depth 1,
// 101 us at 3, 116 us at 4 -- deeper rings cost occupancy).
static int gemm_ring_depth() {
  static int d = -1;
  if (d < 0) {
    const char* e = getenv("ST_GEMM_RING");
    d = (e && e[0] == '1') ? 1 : 2;
  }
  return d;
}

// Whole-line A gathers staged through LDS (default); ST_GATHER_LINES=0
// selects fragment-shaped gathers straight into registers (comparison runs).
static bool gather_lines() {
  static int on = -1;
  if (on < 0) {
    const char* e = getenv("ST_GATHER_LINES");
    on = (e && e[0] == '0') ? 0 : 1;
  }
  return on == 1;
}

}  // namespace st

#include "gemm_wide.h"

namespace st {

// Whole-line kernels address A and Bt through 32-bit buffer offsets.
static bool buffer_ok(int64_t n_src, int K, int Kd, int Nd, size_t esz) {
  return n_src * Kd * (int64_t)esz < (1ll << 31) - 64 && (int64_t)K * Nd * Kd * (int64_t)esz < (1ll << 31) - 64;
}

template <typename T, int BN, int KS, typename Src, typename E>
static void launch_pipe(const T* A, int64_t n_src, const Src& src, const uint32_t* masks, int W, const int32_t* rows,
                        const T* Bt, T* out, E epi, int64_t n_dst, int K, int Kd, int Nd, int vec_a, int vec_b,
                        hipStream_t stream) {
  const dim3 grid(st_blocks(n_dst, kGemmBM), st_blocks(Nd, BN));
  const unsigned rgrid = ring_grid(n_dst, Nd, BN);
  // (IEEE fp32 keeps the register path: its MFMAs dominate and the A stage only costs occupancy there)
  if (vec_a && vec_b && Kd == KS * Frag<T>::KSTEP && gemm_ring_depth() == 2 && gather_lines() && sizeof(T) == 2 &&
      buffer_ok(n_src, K, Kd, Nd, sizeof(T)))
    gather_gemm_ring_kernel<T, BN, KS, 2, Src, true, E>
        <<<rgrid, 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst, K, Kd, Nd, vec_a, vec_b, epi);
  else if (vec_a && vec_b && Kd == KS * Frag<T>::KSTEP && gemm_ring_depth() == 2)
    gather_gemm_ring_kernel<T, BN, KS, 2, Src, false, E>
        <<<rgrid, 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst, K, Kd, Nd, vec_a, vec_b, epi);
  else
    gather_gemm_pipe_kernel<T, BN, KS, Src, E>
        <<<grid, 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst, K, Kd, Nd, vec_a, vec_b, epi);
}

template <typename T, int KS, typename Src, typename E>
static void launch_pipe_ks(const T* A, int64_t n_src, const Src& src, const uint32_t* masks, int W,
                           const int32_t* rows, const T* Bt, T* out, E epi, int64_t n_dst, int K, int Kd, int Nd, int vec_a,
                           int vec_b, hipStream_t stream) {
  constexpr int LDS128 = 2 * 128 * (KS * Frag<T>::KSTEP + Frag<T>::VEC) * (int)sizeof(T) + kSrcGroup * kGemmBM * 4;
  if (Nd <= 16)
    launch_pipe<T, 16, KS>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  else if (Nd <= 32)
    launch_pipe<T, 32, KS>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  else if (Nd <= 64 || LDS128 > 65536)  // (a 128-wide tile at KS = 4 costs occupancy more than its gathers save)
    launch_pipe<T, 64, KS>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  else if constexpr (LDS128 <= 65536)
    launch_pipe<T, 128, KS>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
}

template <typename T, typename Src, typename E>
static int launch_gather_e(const T* A, int64_t n_src, const Src& src, const uint32_t* masks, int W,
                           const int32_t* rows, const T* Bt, T* out, E epi, int64_t n_dst, int K, int Kd, int Nd,
                           hipStream_t stream) {
  constexpr int VEC = Frag<T>::VEC;
  constexpr int KSTEP = Frag<T>::KSTEP;
  if constexpr (Src::kTiled && sizeof(T) == 2) {
    if (gather_wide_mode() && wide_ok(Kd, Nd, K, sizeof(T), false, n_src, A, Bt)) {
      launch_wide<T, false, E>(A, n_src, src, rows, Bt, out, epi, n_dst, Kd, Nd, stream);
      ST_CHECK_LAUNCH();
      return ST_OK;
    }
  }
  const int vec_a = (Kd % VEC == 0) && ((uintptr_t)A % 16 == 0);
  const int vec_b = (Kd % VEC == 0) && ((uintptr_t)Bt % 16 == 0);
  const int ks = (Kd + KSTEP - 1) / KSTEP;
  if (ks == 1) {
    launch_pipe_ks<T, 1>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  } else if (ks == 2) {
    launch_pipe_ks<T, 2>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  } else if (ks <= 4) {
    launch_pipe_ks<T, 4>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  } else if constexpr (Src::kTiled) {
    return ST_ERR_UNSUPPORTED;  // deep reductions take the untiled kernels
  } else {
    // Deep reductions: the single-buffered kernel stages Bt in chunks.
    const unsigned gx = st_blocks(n_dst, kGemmBM);
    if (Nd <= 16)
      gather_gemm_kernel<T, 16, Src, E><<<dim3(gx, 1), 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst,
                                                                       K, Kd, Nd, vec_a, vec_b, epi);
    else if (Nd <= 32)
      gather_gemm_kernel<T, 32, Src, E><<<dim3(gx, 1), 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst,
                                                                       K, Kd, Nd, vec_a, vec_b, epi);
    else if (Nd <= 64)
      gather_gemm_kernel<T, 64, Src, E><<<dim3(gx, 1), 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst,
                                                                       K, Kd, Nd, vec_a, vec_b, epi);
    else
      gather_gemm_kernel<T, 128, Src, E><<<dim3(gx, st_blocks(Nd, 128)), 256, 0, stream>>>(
          A, src, masks, W, rows, Bt, out, n_src, n_dst, K, Kd, Nd, vec_a, vec_b, epi);
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

// The general store epilogue (affine map, residual, ReLU) runs on the tiled
// kernels only; everything else stores acc + bias.
template <typename T, typename Src>
static int launch_gather(const T* A, int64_t n_src, const Src& src, const uint32_t* masks, int W,
                         const int32_t* rows, const T* Bt, T* out, Epi<T> epi, int64_t n_dst, int K, int Kd, int Nd,
                         hipStream_t stream) {
  if (epi.scale || epi.shift || epi.residual || epi.relu) {
    if constexpr (Src::kTiled)
      return launch_gather_e<T, Src, Epi<T>>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, stream);
    else
      return ST_ERR_UNSUPPORTED;
  }
  return launch_gather_e<T, Src, BiasEpi<T>>(A, n_src, src, masks, W, rows, Bt, out, BiasEpi<T>{epi.bias}, n_dst,
                                              K, Kd, Nd, stream);
}

static int launch_wgrad_reduce(const float* partials, const int32_t* cstart_or_null, int64_t splits, int K,
                               int Cin, int Cout, void* dW, int dw_dtype, hipStream_t stream) {
  const int64_t per_k = (int64_t)Cin * Cout;
  const unsigned gr = st_blocks(per_k * K, 256);
  const bool vec4 = per_k % 4 == 0 && (uintptr_t)partials % 16 == 0;
#define ST_REDUCE(TW)                                                                                        \
  if (cstart_or_null && vec4)                                                                                \
    wgrad_pairs_reduce4_kernel<TW><<<(unsigned)(K * ((per_k + 63) / 64)), 256, 0, stream>>>(                 \
        partials, cstart_or_null, per_k, K, (TW*)dW);                                                        \
  else if (cstart_or_null)                                                                                   \
    wgrad_pairs_reduce_kernel<TW><<<(unsigned)(K * ((per_k + 31) / 32)), 256, 0, stream>>>(                  \
        partials, cstart_or_null, per_k, K, (TW*)dW);                                                        \
  else                                                                                                       \
    wgrad_reduce_kernel<TW><<<gr, 256, 0, stream>>>(partials, per_k, (int)splits, K, (TW*)dW);
  switch (dw_dtype) {
    case ST_F32:
    case ST_F32_BF16X3:
      ST_REDUCE(float);
      break;
    case ST_F16:
      ST_REDUCE(_Float16);
      break;
    case ST_BF16:
      ST_REDUCE(__bf16);
      break;
    default:
      return ST_ERR_UNSUPPORTED;
  }
#undef ST_REDUCE
  ST_CHECK_LAUNCH();
  return ST_OK;
}

// Weight gradient over windows of map columns for 16-bit rows whose C_in and
// C_out are multiples of 128 (a workgroup covers one 128 x 128 channel tile):
// column p of the map pairs X rows map(k, p) with dY row rows[p] (p itself
// when rows is null), so a caller can hand the columns over in any order --
// rows sorted by offset mask within slabs of their own order, with the map
// permuted to match, lets the kernel skip most offset steps without pairs
// while a slab's rows stay near each other.  A workgroup takes a window of
// rows_per_split columns and two consecutive offsets; its four waves take
// (offset, output-channel half) each, a 128 x 64 fp32 tile of dW[k] (two
// workgroups per CU).  The window is walked in 32-column steps: a step's dY
// rows are staged in LDS once for the four waves and each offset's X rows
// once for its two waves (zeros where the map has no pair; two buffers, one
// workgroup barrier a step); a wave adds X^T dY over the step, both operands
// read as transpose fragments (tr_frag), skips the MFMAs of a step in which
// its offset has no pair, and masks the dY elements of the columns without
// one, so that a non-finite dY value reaches only the offsets that pair its
// row, as in a sum over pairs.  Loads run two steps ahead: the map entries
// and rows of step s + 3 are issued before the rows of step s + 2 (the
// memory counter completes in order, so waiting on the former never waits on
// the latter), with a register set per step parity (the loop body is two
// steps, so no value still in flight is ever copied).  Against equal chunks
// of the pair list a dY row is read once per two offsets instead of once per
// pair, and the workgroups of one window run side by side on one XCD (work
// item L = (window, channel tile, offset pair) runs on XCD L / ceil(items /
// 8)), so the X rows that neighbouring offsets share come from that XCD's
// L2.  Each wave stores its tile to partials[(k * splits + window) * C_in *
// C_out ...] (the layout that wgrad_reduce_kernel sums).  Requires 16-byte
// aligned rows and X and dY addressable by 32-bit buffer offsets.
template <typename T>
__global__ __launch_bounds__(256, 2) void wgrad_window_kernel(const T* __restrict__ X, const T* __restrict__ dY,
                                                              const int32_t* __restrict__ map, int64_t ks, int64_t rs,
                                                              const int32_t* __restrict__ rows, int64_t n_in,
                                                              int64_t n_out, int K, int Cin, int Cout,
                                                              int64_t rows_per_split, int splits,
                                                              float* __restrict__ partials) {
  using F = typename Frag<T>::type;
  static_assert(Frag<T>::KSTEP == 32 && Frag<T>::VEC == 8, "16-bit MFMA fragments");
  constexpr int P = wave_pitch(128);
  constexpr int STAGE = 32 * P;  // 32 rows of 128 channels
  __shared__ __attribute__((aligned(16))) T ys_s[2 * STAGE];      // dY, two buffers
  __shared__ __attribute__((aligned(16))) T xs_s[2 * 2 * STAGE];  // X of the two offsets, two buffers
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int kpairs = (K + 1) / 2;
  const int ntn = Cout / 128, ntiles = (Cin / 128) * ntn;
  const int64_t items = (int64_t)splits * ntiles * kpairs;
  const int64_t per = (items + 7) / 8;
  const int64_t L = (int64_t)(blockIdx.x % 8) * per + blockIdx.x / 8;
  if (L >= items) return;  // uniform over the workgroup
  const int grp = (int)(L % kpairs);
  const int64_t wt = L / kpairs;
  const int tile = (int)(wt % ntiles);
  const int w = (int)(wt / ntiles);
  const int cm0 = (tile / ntn) * 128, cn0 = (tile % ntn) * 128;
  const int kw = wid >> 1, half = wid & 1;  // this wave's offset of the pair, output-channel half
  const int k = grp * 2 + kw;
  const bool kv = k < K;
  const int64_t o0 = (int64_t)w * rows_per_split;
  const int64_t o1 = min(o0 + rows_per_split, n_out);
  const int nsteps = o1 > o0 ? (int)((o1 - o0 + 31) / 32) : 0;
  const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(X, n_in * Cin * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t y_rsrc = make_rsrc(dY, n_out * Cout * (int64_t)sizeof(T));
  const int pt = half * 64 + lane;  // thread of this offset's pair of waves, 0..127

  // column (lane mod 32) of step s: its dY row (-1 past the window, and for
  // an entry of rows outside [0, n_out)) and its map entry through this
  // wave's offset (-1: none)
  auto load_row = [&](int s) -> int {
    const int64_t p = o0 + 32 * (int64_t)s + (lane & 31);
    const int r = (s < nsteps && p < o1) ? (rows ? rows[p] : (int)p) : -1;
    return (r >= 0 && r < n_out) ? r : -1;
  };
  auto load_idx = [&](int s) -> int {
    const int64_t p = o0 + 32 * (int64_t)s + (lane & 31);
    return (kv && s < nsteps && p < o1) ? map[(int64_t)k * ks + p * rs] : -1;
  };
  // this offset's X rows of a step: load v takes 16 bytes (channel chunk
  // pt mod 16) of step column pt / 16 + 8 v, whose map entry lane (column) holds
  // (each lane taking 64 bytes of its own column's row instead, no exchange:
  // 1.05 -> 1.23 ms on config 5, the loads less contiguous)
  auto load_x = [&](int idx, int row, F* xr) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int col = (pt >> 4) + 8 * v;
      const int ix = __shfl(row >= 0 ? idx : -1, col, 64);
      xr[v] = load16<F>(x_rsrc, (ix >= 0 && ix < n_in) ? (ix * Cin + cm0 + (pt & 15) * 8) * (int)sizeof(T) : kOobOffset);
    }
  };
  // the step's dY rows: 16 threads a row, step column tid / 16 + 16 v
  auto load_y = [&](int row, F* yr) {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int r = __shfl(row, (tid >> 4) + 16 * v, 64);
      yr[v] = load16<F>(y_rsrc, r >= 0 ? (r * Cout + cn0 + (tid & 15) * 8) * (int)sizeof(T) : kOobOffset);
    }
  };

  v4f acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // per step parity u: xr/yr[u] the rows of the next step s of parity u in
  // flight and pmr[u] its pair mask; at step s, idx/row[u] hold the map
  // entries and dY rows of step s + 2 (loaded at step s - 1)
  F xr[2][4], yr[2][2];
  int idx[2], row[2];
  uint64_t pmr[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    idx[u] = load_idx(u);
    row[u] = load_row(u);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    load_x(idx[u], row[u], xr[u]);
    load_y(row[u], yr[u]);
    pmr[u] = __ballot(row[u] >= 0 && idx[u] >= 0);
  }
  idx[0] = load_idx(2);
  row[0] = load_row(2);
  idx[1] = -1;  // (step 3's, loaded at step 0)
  row[1] = -1;
  // the steps rounded up to even: the extra step has no columns, so it adds
  // nothing and skips its MFMAs
  for (int s0 = 0; s0 < nsteps; s0 += 2) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int s = s0 + u;
      T* ys = ys_s + u * STAGE;
      T* xs = xs_s + (u * 2 + kw) * STAGE;
#pragma unroll
      for (int v = 0; v < 2; ++v) *reinterpret_cast<F*>(&ys[((tid >> 4) + 16 * v) * P + (tid & 15) * 8]) = yr[u][v];
#pragma unroll
      for (int v = 0; v < 4; ++v) *reinterpret_cast<F*>(&xs[((pt >> 4) + 8 * v) * P + (pt & 15) * 8]) = xr[u][v];
      // the step's stages complete for every wave; the other buffers, read in
      // the previous step, free for the next step's stores
      __syncthreads();
      const uint64_t pm = pmr[u];  // bit r (r < 32): step column r has a pair through this offset
      // step s + 3's map entries and rows first, then step s + 2's rows
      const int idx3 = load_idx(s + 3), row3 = load_row(s + 3);
      load_x(idx[u], row[u], xr[u]);
      load_y(row[u], yr[u]);
      pmr[u] = __ballot(row[u] >= 0 && idx[u] >= 0);
      // (each of idx / row[0 / 1] is set once per two steps, after its last
      // use, so no value still in flight is copied)
      idx[u ^ 1] = idx3;
      row[u ^ 1] = row3;
      if (pm) {  // uniform over the wave
        // this lane's fragment elements hold columns 4g .. 4g+3 and 16+4g .. 16+4g+3
        const uint32_t bits = (uint32_t)((pm >> (4 * g)) & 0xFu) | ((uint32_t)((pm >> (16 + 4 * g)) & 0xFu) << 4);
        uint32_t mw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          mw[e] = (((bits >> (2 * e)) & 1u) ? 0x0000FFFFu : 0u) | (((bits >> (2 * e + 1)) & 1u) ? 0xFFFF0000u : 0u);
        F b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          uint4 bw = __builtin_bit_cast(uint4, tr_frag<F, T, P>(ys, g, c, half * 64 + j * 16));
          bw.x &= mw[0];
          bw.y &= mw[1];
          bw.z &= mw[2];
          bw.w &= mw[3];
          b[j] = __builtin_bit_cast(F, bw);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const F a = tr_frag<F, T, P>(xs, g, c, i * 16);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = mfma(a, b[j], acc[i][j]);
        }
      }
    }
  }
  if (kv) {
    float* part = partials + ((int64_t)k * splits + w) * Cin * Cout;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          part[(int64_t)(cm0 + i * 16 + g * 4 + r) * Cout + cn0 + half * 64 + j * 16 + c] = acc[i][j][r];
  }
}

// Row arrays addressable by 32-bit buffer offsets.
static bool rows_fit_buffer(int64_t n_in, int Cin, int64_t n_out, int Cout, size_t esz) {
  return n_in * Cin * (int64_t)esz < (1ll << 31) - 64 && n_out * Cout * (int64_t)esz < (1ll << 31) - 64;
}

// Whether the window kernel above is taken for 16-bit maps with 128-multiple
// channel counts (ST_WGRAD_WINDOW=0 turns it off).
static bool wgrad_window_on() {
  static int mode = -1;
  if (mode < 0) {
    const char* e = getenv("ST_WGRAD_WINDOW");
    mode = (e && e[0] == '0') ? 0 : 1;
  }
  return mode == 1;
}

template <typename T, typename Src>
static int launch_wgrad(const T* X, int64_t n_in, const T* dY, const Src& src, int64_t n_out, int K, int Cin,
                        int Cout, float* partials, int64_t splits, void* dW, int dw_dtype, hipStream_t stream,
                        const int32_t* rows = nullptr) {
  constexpr int VEC = Frag<T>::VEC;
  const int vec_x = (Cin % VEC == 0) && ((uintptr_t)X % 16 == 0);
  const int vec_y = (Cout % VEC == 0) && ((uintptr_t)dY % 16 == 0);
  const int64_t rows_per_split = (n_out + splits - 1) / splits;
  const int MB = (Cin + 15) / 16, NB = (Cout + 15) / 16;
  const unsigned gz = (unsigned)(((MB + kWgTileBlk - 1) / kWgTileBlk) * ((NB + kWgTileBlk - 1) / kWgTileBlk));
  bool window = false;
  if constexpr (sizeof(T) == 2 && !Src::kTiled && !Src::kProbe)
    window = wgrad_window_on() && Cin % 128 == 0 && Cout % 128 == 0 && vec_x && vec_y &&
             rows_fit_buffer(n_in, Cin, n_out, Cout, sizeof(T));
  if (rows && !window) return ST_ERR_UNSUPPORTED;  // only the window kernel takes a column order
  if constexpr (sizeof(T) == 2 && !Src::kTiled && !Src::kProbe) {
    if (n_out > 0 && window) {
      const int64_t items = splits * (int64_t)(Cin / 128) * (Cout / 128) * ((K + 1) / 2);
      wgrad_window_kernel<T><<<(unsigned)(8 * ((items + 7) / 8)), 256, 0, stream>>>(
          X, dY, src.map, src.ks, src.rs, rows, n_in, n_out, K, Cin, Cout, rows_per_split, (int)splits, partials);
      ST_CHECK_LAUNCH();
      return launch_wgrad_reduce(partials, nullptr, splits, K, Cin, Cout, dW, dw_dtype, stream);
    }
  }
  if (n_out > 0) {
    wgrad_kernel<T, Src><<<dim3((unsigned)splits, (unsigned)K, gz), 256, 0, stream>>>(
        X, dY, src, n_in, n_out, Cin, Cout, rows_per_split, (int)splits, partials, vec_x, vec_y);
    ST_CHECK_LAUNCH();
  } else {
    const int rc = st_fill_u32((uint32_t*)partials, (int64_t)K * splits * Cin * Cout, 0u, stream);
    if (rc != ST_OK) return rc;
  }
  return launch_wgrad_reduce(partials, nullptr, splits, K, Cin, Cout, dW, dw_dtype, stream);
}

// Weight-gradient grid: up to 1024 workgroups, a multiple of 8 (one run of
// chunks per workgroup, adjacent runs per XCD; see chunk_range).
static unsigned wgrad_grid(int64_t max_chunks) {
  int64_t g = max_chunks < 1024 ? max_chunks : 1024;
  if (g >= 8) g -= g % 8;
  return (unsigned)(g > 0 ? g : 1);
}

template <int MT, int NT>
static void launch_wgrad_pairs_f32(const float* X, const float* dY, const int2* pairs, const int32_t* kstart,
                                   const int32_t* cstart, const int32_t* chunk_order, int K, int chunk,
                                   int64_t max_chunks, int Cin, int Cout, float* partials, hipStream_t stream) {
  const int MB = (Cin + 15) / 16, NB = (Cout + 15) / 16;
  const int WT = ((MB + MT - 1) / MT) * ((NB + NT - 1) / NT);
  const unsigned gx = wgrad_grid(max_chunks);
  wgrad_pairs_f32_kernel<MT, NT><<<dim3(gx, 1, (unsigned)((WT + 3) / 4)), 256, 0, stream>>>(
      X, dY, pairs, kstart, cstart, chunk_order, K, chunk, Cin, Cout, partials);
}

static int pow2_tile(int blocks) { return blocks >= 4 ? 4 : (blocks >= 2 ? 2 : 1); }



// 16-bit weight-gradient kernel: 0 = per-wave steps (default), 1 = workgroup
// LDS transpose (ST_WGRAD16=lds), 2 = per-wave steps with tiles of at most
// 64 x 64 channels (ST_WGRAD16=small); the last two for comparison runs.
static int wgrad16_mode() {
  static int mode = -1;
  if (mode < 0) {
    const char* e = getenv("ST_WGRAD16");
    mode = (e && e[0] == 'l') ? 1 : (e && e[0] == 's') ? 2 : 0;
  }
  return mode;
}

// 16-channel blocks of the per-wave weight-gradient tile for C channels: 1, 2,
// 4 or 8 (C = 16, 32, a multiple of 64, a multiple of 128), 0 when the kernel
// does not cover C.
static int wave_tile_blocks(int C) {
  if (C % 128 == 0 && wgrad16_mode() != 2) return 8;
  if (C % 64 == 0) return 4;
  if (C == 32) return 2;
  if (C == 16) return 1;
  return 0;
}

template <typename T>
int ops_wgrad_pairs(const T* X, int64_t n_in, const T* dY, int64_t n_out, const int32_t* pairs, const int32_t* kstart,
                    const int32_t* cstart, const int32_t* chunk_order, int K, int chunk, int64_t max_chunks, int Cin,
                    int Cout, float* partials, void* dW, int dw_dtype, hipStream_t stream) {
  if (max_chunks > 0) {
    if constexpr (sizeof(T) == 4) {
      const int mt = pow2_tile((Cin + 15) / 16), nt = pow2_tile((Cout + 15) / 16);
      const int2* pr = reinterpret_cast<const int2*>(pairs);
#define ST_WP(A, B)                                                                                                 \
  if (mt == A && nt == B)                                                                                           \
    launch_wgrad_pairs_f32<A, B>((const float*)X, (const float*)dY, pr, kstart, cstart, chunk_order, K, chunk,     \
                                 max_chunks, Cin, Cout, partials, stream);
      ST_WP(1, 1) ST_WP(1, 2) ST_WP(1, 4) ST_WP(2, 1) ST_WP(2, 2) ST_WP(2, 4) ST_WP(4, 1) ST_WP(4, 2) ST_WP(4, 4)
#undef ST_WP
    } else {
      constexpr int VEC = Frag<T>::VEC;
      const int vec_x = (Cin % VEC == 0) && ((uintptr_t)X % 16 == 0);
      const int vec_y = (Cout % VEC == 0) && ((uintptr_t)dY % 16 == 0);
      const int MB = (Cin + 15) / 16, NB = (Cout + 15) / 16;
      const unsigned gx = wgrad_grid(max_chunks);
      const int2* pr = reinterpret_cast<const int2*>(pairs);
      const int mode = wgrad16_mode();
      int mb = wave_tile_blocks(Cin), nb = wave_tile_blocks(Cout);
      if (mb == 8 && nb < 4) mb = 4;  // a 128-wide side only beside a side of 64 or more
      if (nb == 8 && mb < 4) nb = 4;
      if (mode != 1 && mb && nb && vec_x && vec_y) {
        const unsigned grid = gx * (unsigned)((Cin / (16 * mb)) * (Cout / (16 * nb)));
        const bool buf = rows_fit_buffer(n_in, Cin, n_out, Cout, sizeof(T));
        // A 64 x 64 tile with its cross-wave sum in 32-row rounds fits three
        // workgroups per CU.  A grid of at most two rounds at two per CU takes
        // the one-round sum instead (two per CU): a third workgroup per CU
        // would not save a round there, only slow the other two down.
        const bool onepass = grid <= 1024;
#define ST_WAVE(MB_, NB_)                                                                                         \
  if (mb == MB_ && nb == NB_) {                                                                                   \
    if (onepass && MB_ == 4 && NB_ <= 4) {                                                                        \
      if (buf)                                                                                                    \
        wgrad_pairs_wave_kernel<T, true, MB_, NB_, (MB_ <= 4 && NB_ <= 4)><<<grid, 256, 0, stream>>>(                         \
            X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin, Cout, n_in, n_out, partials);                 \
      else                                                                                                        \
        wgrad_pairs_wave_kernel<T, false, MB_, NB_, (MB_ <= 4 && NB_ <= 4)><<<grid, 256, 0, stream>>>(                        \
            X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin, Cout, n_in, n_out, partials);                 \
    } else if (buf) {                                                                                             \
      wgrad_pairs_wave_kernel<T, true, MB_, NB_, false><<<grid, 256, 0, stream>>>(                                \
          X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin, Cout, n_in, n_out, partials);                   \
    } else {                                                                                                      \
      wgrad_pairs_wave_kernel<T, false, MB_, NB_, false><<<grid, 256, 0, stream>>>(                               \
          X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin, Cout, n_in, n_out, partials);                   \
    }                                                                                                             \
  }
        ST_WAVE(1, 1) ST_WAVE(1, 2) ST_WAVE(1, 4) ST_WAVE(2, 1) ST_WAVE(2, 2) ST_WAVE(2, 4) ST_WAVE(4, 1)
        ST_WAVE(4, 2) ST_WAVE(4, 4) ST_WAVE(4, 8) ST_WAVE(8, 4) ST_WAVE(8, 8)
#undef ST_WAVE
        ST_CHECK_LAUNCH();
        return launch_wgrad_reduce(partials, cstart, 0, K, Cin, Cout, dW, dw_dtype, stream);
      }
      const unsigned gz = (unsigned)(((MB + 7) / 8) * ((NB + 7) / 8));
      const int nloc = (MB < 8 ? MB : 8) * (NB < 8 ? NB : 8);
      if (nloc <= 4)
        wgrad_pairs_lds_kernel<T, 1><<<dim3(gx, 1, gz), 256, 0, stream>>>(X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin,
                                                                          Cout, partials, vec_x, vec_y);
      else if (nloc <= 16)
        wgrad_pairs_lds_kernel<T, 4><<<dim3(gx, 1, gz), 256, 0, stream>>>(X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin,
                                                                          Cout, partials, vec_x, vec_y);
      else
        wgrad_pairs_lds_kernel<T, 16><<<dim3(gx, 1, gz), 256, 0, stream>>>(X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin,
                                                                           Cout, partials, vec_x, vec_y);
    }
    ST_CHECK_LAUNCH();
  }
  return launch_wgrad_reduce(partials, cstart, 0, K, Cin, Cout, dW, dw_dtype, stream);
}

template <typename T>
int ops_gather_map(const T* A, int64_t n_src, const int32_t* map, int64_t ks, int64_t rs, const uint32_t* masks, int W,
                   const int32_t* rows, const T* Bt, T* out, Epi<T> epi, int64_t n_dst, int K, int Kd, int Nd,
                   hipStream_t stream) {
  MapSrc src{map, ks, rs};
  return launch_gather<T>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, stream);
}

template <typename T>
int ops_gather_tiled(const T* A, int64_t n_src, const int32_t* perm, const int32_t* nk, const int16_t* klist,
                     const int32_t* tmap, const T* Bt, T* out, Epi<T> epi, int64_t n_dst, int K, int Kd, int Nd,
                     hipStream_t stream, int rev) {
  TiledSrc src{nk, klist, tmap, K, rev};
  return launch_gather<T>(A, n_src, src, nullptr, (K + 31) / 32, perm, Bt, out, epi, n_dst, K, Kd, Nd, stream);
}

template <typename CT>
static HashSrc<CT> make_hash_src(const void* coords, const int32_t* offsets, const st_lookup* lk, const uint64_t* keys,
                                 const uint32_t* vals, int64_t cap) {
  return HashSrc<CT>{(const CT*)coords, offsets,       keys,          vals,          (uint32_t)cap,
                     lk->sign,          lk->mul,       lk->div,       lk->bounds[0], lk->bounds[1],
                     lk->bounds[2],     lk->row_bounds[0], lk->row_bounds[1], lk->row_bounds[2]};
}

template <typename T>
int ops_gather_hash(const T* A, int64_t n_src, const void* coords, int coord_dtype, const int32_t* offsets,
                    const st_lookup* lk, const uint64_t* keys, const uint32_t* vals, int64_t cap, const T* Bt, T* out, Epi<T> epi,
                    int64_t n_dst, int Kd, int Nd, hipStream_t stream) {
  const int W = (lk->K + 31) / 32;
  if (coord_dtype == ST_COORD_I16)
    return launch_gather<T>(A, n_src, make_hash_src<int16_t>(coords, offsets, lk, keys, vals, cap), nullptr, W,
                            nullptr, Bt, out, epi, n_dst, lk->K, Kd, Nd, stream);
  if (coord_dtype == ST_COORD_I32)
    return launch_gather<T>(A, n_src, make_hash_src<int32_t>(coords, offsets, lk, keys, vals, cap), nullptr, W,
                            nullptr, Bt, out, epi, n_dst, lk->K, Kd, Nd, stream);
  return ST_ERR_UNSUPPORTED;
}

// Submanifold gather with the neighbours looked up in a brick index inside the
// wide kernel (16-bit types; ST_ERR_UNSUPPORTED for shapes fly_ok rejects).
template <typename T>
int ops_gather_fly(const T* A, int64_t n, const void* coords, int coord_dtype, const int32_t* offsets, int K,
                   const SubmIndex& ix, const int32_t* rows, int rev, const T* Bt, T* out, const T* bias, int Kd,
                   int Nd, hipStream_t stream) {
  if constexpr (sizeof(T) != 2) {
    return ST_ERR_UNSUPPORTED;
  } else {
    if (!fly_ok(Kd, Nd, K, sizeof(T), false, n, A, Bt)) return ST_ERR_UNSUPPORTED;
    const BiasEpi<T> epi{bias};
    if (coord_dtype == ST_COORD_I16)
      launch_wide<T, false>(A, n, FlySrc<int16_t>{(const int16_t*)coords, offsets, ix, K, rows, rev}, nullptr, Bt, out, epi, n,
                            Kd, Nd, stream);
    else if (coord_dtype == ST_COORD_I32)
      launch_wide<T, false>(A, n, FlySrc<int32_t>{(const int32_t*)coords, offsets, ix, K, rows, rev}, nullptr, Bt, out, epi, n,
                            Kd, Nd, stream);
    else
      return ST_ERR_UNSUPPORTED;
    ST_CHECK_LAUNCH();
    return ST_OK;
  }
}

template <typename T>
int ops_wgrad_map(const T* X, int64_t n_in, const T* dY, const int32_t* map, int64_t ks, int64_t rs,
                  const int32_t* rows, int64_t n_out, int K, int Cin, int Cout, float* partials, int64_t splits,
                  void* dW, int dw_dtype, hipStream_t stream) {
  MapSrc src{map, ks, rs};
  return launch_wgrad<T>(X, n_in, dY, src, n_out, K, Cin, Cout, partials, splits, dW, dw_dtype, stream, rows);
}

template <typename T>
int ops_wgrad_hash(const T* X, int64_t n_in, const T* dY, const void* coords, int coord_dtype, int64_t n_out,
                   const int32_t* offsets, const st_lookup* lk, const uint64_t* keys, const uint32_t* vals,
                   int64_t cap, int Cin, int Cout, float* partials, int64_t splits, void* dW, int dw_dtype,
                   hipStream_t stream) {
  if (coord_dtype == ST_COORD_I16)
    return launch_wgrad<T>(X, n_in, dY, make_hash_src<int16_t>(coords, offsets, lk, keys, vals, cap), n_out, lk->K,
                           Cin, Cout, partials, splits, dW, dw_dtype, stream);
  if (coord_dtype == ST_COORD_I32)
    return launch_wgrad<T>(X, n_in, dY, make_hash_src<int32_t>(coords, offsets, lk, keys, vals, cap), n_out, lk->K,
                           Cin, Cout, partials, splits, dW, dw_dtype, stream);
  return ST_ERR_UNSUPPORTED;
}

template <typename T>
int ops_weight_prep(const T* w, T* out, int K, int Cin, int Cout, int mode, hipStream_t stream) {
  const int64_t total = (int64_t)K * Cin * Cout;
  weight_prep_kernel<T><<<st_blocks(total, 256), 256, 0, stream>>>(w, out, K, Cin, Cout, mode);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // namespace st

// Declares (X = extern) or instantiates (X empty) every typed launcher for T.
#define ST_GEMM_OPS(X, T)                                                                                            \
  namespace st {                                                                                                     \
  X template int ops_gather_map<T>(const T*, int64_t, const int32_t*, int64_t, int64_t, const uint32_t*, int,        \
                                   const int32_t*, const T*, T*, Epi<T>, int64_t, int, int, int, hipStream_t);    \
  X template int ops_gather_hash<T>(const T*, int64_t, const void*, int, const int32_t*, const st_lookup*,            \
                                    const uint64_t*, const uint32_t*, int64_t, const T*, T*, Epi<T>, int64_t, int, \
                                    int,                                                                             \
                                    hipStream_t);                                                                    \
  X template int ops_wgrad_map<T>(const T*, int64_t, const T*, const int32_t*, int64_t, int64_t, const int32_t*,   \
                                  int64_t, int, int, int, float*, int64_t, void*, int, hipStream_t);               \
  X template int ops_wgrad_hash<T>(const T*, int64_t, const T*, const void*, int, int64_t, const int32_t*,           \
                                   const st_lookup*, const uint64_t*, const uint32_t*, int64_t, int, int, float*,    \
                                   int64_t, void*, int, hipStream_t);                                                \
  X template int ops_wgrad_pairs<T>(const T*, int64_t, const T*, int64_t, const int32_t*, const int32_t*,          \
                                    const int32_t*, const int32_t*, int, int, int64_t, int, int, float*, void*, int, \
                                    hipStream_t);                                                                    \
  X template int ops_weight_prep<T>(const T*, T*, int, int, int, int, hipStream_t);                                  \
  X template int ops_gather_fly<T>(const T*, int64_t, const void*, int, const int32_t*, int, const SubmIndex&,       \
                                   const int32_t*, int, const T*, T*, const T*, int, int, hipStream_t);             \
  X template int ops_gather_tiled<T>(const T*, int64_t, const int32_t*, const int32_t*, const int16_t*,              \
                                     const int32_t*, const T*, T*, Epi<T>, int64_t, int, int, int, hipStream_t,    \
                                     int);                                                                         \
  }
