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
#include "common.h"
#include "mfma.h"
#include "nbr_src.h"

namespace st {

constexpr int kGemmBM = 128;

template <typename T, int BN, typename Src>
__global__ __launch_bounds__(256) void gather_gemm_kernel(const T* __restrict__ A, Src src,
                                                          const uint32_t* __restrict__ masks, int W,
                                                          const int32_t* __restrict__ perm, const T* __restrict__ Bt,
                                                          T* __restrict__ out, int64_t n_src, int64_t n_dst, int K,
                                                          int Kd, int Nd, int vec_a, int vec_b) {
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

  // Lane (l & 31) resolves destination row wid*32 + (l & 31); MFMA row c of
  // tile m is then fetched from lane m*16 + c with a shuffle.
  const int32_t my_row = drow_s[wid * 32 + (lane & 31)];
  const typename Src::RowCtx rc = src.row(my_row >= 0 ? my_row : 0);

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
      int32_t s_own = my_row >= 0 ? src.get(rc, k) : -1;
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
        if (col < Nd) orow[col] = from_f32<T>(acc[m][nb][r]);
      }
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

template <typename T, typename Src>
static int launch_gather(const T* A, int64_t n_src, const Src& src, const uint32_t* masks, int W,
                         const int32_t* perm, const T* Bt, T* out, int64_t n_dst, int K, int Kd, int Nd,
                         hipStream_t stream) {
  constexpr int VEC = Frag<T>::VEC;
  const int vec_a = (Kd % VEC == 0) && ((uintptr_t)A % 16 == 0);
  const int vec_b = (Kd % VEC == 0) && ((uintptr_t)Bt % 16 == 0);
  const unsigned gx = st_blocks(n_dst, kGemmBM);
  if (Nd <= 16) {
    gather_gemm_kernel<T, 16, Src><<<dim3(gx, 1), 256, 0, stream>>>(A, src, masks, W, perm, Bt, out, n_src, n_dst, K, Kd,
                                                                     Nd, vec_a, vec_b);
  } else if (Nd <= 32) {
    gather_gemm_kernel<T, 32, Src><<<dim3(gx, 1), 256, 0, stream>>>(A, src, masks, W, perm, Bt, out, n_src, n_dst, K, Kd,
                                                                     Nd, vec_a, vec_b);
  } else if (Nd <= 64) {
    gather_gemm_kernel<T, 64, Src><<<dim3(gx, 1), 256, 0, stream>>>(A, src, masks, W, perm, Bt, out, n_src, n_dst, K, Kd,
                                                                     Nd, vec_a, vec_b);
  } else {
    gather_gemm_kernel<T, 128, Src><<<dim3(gx, st_blocks(Nd, 128)), 256, 0, stream>>>(
        A, src, masks, W, perm, Bt, out, n_src, n_dst, K, Kd, Nd, vec_a, vec_b);
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

template <typename T, typename Src>
static int launch_wgrad(const T* X, int64_t n_in, const T* dY, const Src& src, int64_t n_out, int K, int Cin,
                        int Cout, float* partials, int64_t splits, void* dW, int dw_dtype, hipStream_t stream) {
  constexpr int VEC = Frag<T>::VEC;
  const int vec_x = (Cin % VEC == 0) && ((uintptr_t)X % 16 == 0);
  const int vec_y = (Cout % VEC == 0) && ((uintptr_t)dY % 16 == 0);
  const int64_t rows_per_split = (n_out + splits - 1) / splits;
  const int MB = (Cin + 15) / 16, NB = (Cout + 15) / 16;
  const unsigned gz = (unsigned)(((MB + kWgTileBlk - 1) / kWgTileBlk) * ((NB + kWgTileBlk - 1) / kWgTileBlk));
  if (n_out > 0) {
    wgrad_kernel<T, Src><<<dim3((unsigned)splits, (unsigned)K, gz), 256, 0, stream>>>(
        X, dY, src, n_in, n_out, Cin, Cout, rows_per_split, (int)splits, partials, vec_x, vec_y);
  } else {
    const int rc = st_fill_u32((uint32_t*)partials, (int64_t)K * splits * Cin * Cout, 0u, stream);
    if (rc != ST_OK) return rc;
  }
  const int64_t per_k = (int64_t)Cin * Cout;
  const unsigned gr = st_blocks(per_k * K, 256);
  switch (dw_dtype) {
    case ST_F32:
      wgrad_reduce_kernel<float><<<gr, 256, 0, stream>>>(partials, per_k, (int)splits, K, (float*)dW);
      break;
    case ST_F16:
      wgrad_reduce_kernel<_Float16><<<gr, 256, 0, stream>>>(partials, per_k, (int)splits, K, (_Float16*)dW);
      break;
    case ST_BF16:
      wgrad_reduce_kernel<__bf16><<<gr, 256, 0, stream>>>(partials, per_k, (int)splits, K, (__bf16*)dW);
      break;
    default:
      return ST_ERR_UNSUPPORTED;
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // namespace st

using namespace st;

#define ST_DISPATCH_DTYPE(dt, T, ...)   \
  switch (dt) {                         \
    case ST_F32: {                      \
      using T = float;                  \
      return __VA_ARGS__;               \
    }                                   \
    case ST_F16: {                      \
      using T = _Float16;               \
      return __VA_ARGS__;               \
    }                                   \
    case ST_BF16: {                     \
      using T = __bf16;                 \
      return __VA_ARGS__;               \
    }                                   \
    default:                            \
      return ST_ERR_UNSUPPORTED;        \
  }

static int dtype_size(int dt) { return dt == ST_F32 ? 4 : 2; }

extern "C" {

int st_weight_prep(const void* w, void* out, int K, int C_in, int C_out, int mode, int dtype, st_stream_t stream) {
  if (!w || !out || K <= 0 || C_in <= 0 || C_out <= 0 || mode < 0 || mode > 2) return ST_ERR_ARG;
  const int64_t total = (int64_t)K * C_in * C_out;
  (void)dtype_size;
  ST_DISPATCH_DTYPE(dtype, T, ([&]() -> int {
                      weight_prep_kernel<T><<<st_blocks(total, 256), 256, 0, stream>>>((const T*)w, (T*)out, K, C_in,
                                                                                       C_out, mode);
                      ST_CHECK_LAUNCH();
                      return ST_OK;
                    }()));
}

int st_gather_gemm(const void* A, int64_t n_src, const int32_t* map, int64_t map_k_stride, int64_t map_r_stride,
                   const uint32_t* row_masks, int mask_words, const int32_t* perm, const void* Bt, void* out,
                   int64_t n_dst, int K, int Kd, int Nd, int dtype, st_stream_t stream) {
  if (n_src < 0 || n_dst < 0 || K <= 0 || K > ST_MAX_KVOL || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (n_dst >= (1ll << 31) || n_src >= (1ll << 31)) return ST_ERR_ARG;
  if (row_masks && mask_words != (K + 31) / 32) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!map || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  MapSrc src{map, map_k_stride, map_r_stride};
  const int W = (K + 31) / 32;
  ST_DISPATCH_DTYPE(dtype, T,
                    launch_gather<T>((const T*)A, n_src, src, row_masks, W, perm, (const T*)Bt, (T*)out, n_dst, K,
                                     Kd, Nd, stream));
}

int st_wgrad(const void* X, int64_t n_in, const void* dY, const int32_t* map, int64_t map_k_stride,
             int64_t map_r_stride, int64_t n_out, int K, int C_in, int C_out, int dtype, float* partials,
             int64_t splits, void* dW, int dw_dtype, st_stream_t stream) {
  if (n_in < 0 || n_out < 0 || K <= 0 || K > ST_MAX_KVOL || C_in <= 0 || C_out <= 0 || splits < 1 || splits > 65535)
    return ST_ERR_ARG;
  if (n_out >= (1ll << 31)) return ST_ERR_ARG;
  if (!partials || !dW || (n_out > 0 && (!X || !dY || !map))) return ST_ERR_ARG;
  MapSrc src{map, map_k_stride, map_r_stride};
  ST_DISPATCH_DTYPE(dtype, T,
                    launch_wgrad<T>((const T*)X, n_in, (const T*)dY, src, n_out, K, C_in, C_out, partials, splits,
                                    dW, dw_dtype, stream));
}

int st_hashfly_gemm(const void* A, int64_t n_src, const void* dst_coords, int coord_dtype, int64_t n_dst,
                    const int32_t* offsets, const st_lookup* lk, const uint64_t* keys, const uint32_t* vals,
                    int64_t capacity, const void* Bt, void* out, int Kd, int Nd, int dtype, st_stream_t stream) {
  if (!lk || n_src < 0 || n_dst < 0 || lk->K <= 0 || lk->K > ST_MAX_KVOL || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (lk->mul < 1 || lk->div < 1 || (lk->sign != 1 && lk->sign != -1)) return ST_ERR_ARG;
  if (capacity <= 0 || capacity >= (1ll << 31) || n_dst >= (1ll << 31)) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!dst_coords || !offsets || !keys || !vals || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  const int K = lk->K;
  const int W = (K + 31) / 32;
  ST_DISPATCH_COORD(coord_dtype, CT, {
    HashSrc<CT> src{(const CT*)dst_coords, offsets,       keys,          vals,          (uint32_t)capacity,
                    lk->sign,               lk->mul,       lk->div,       lk->bounds[0], lk->bounds[1],
                    lk->bounds[2],          lk->row_bounds[0], lk->row_bounds[1], lk->row_bounds[2]};
    ST_DISPATCH_DTYPE(dtype, T,
                      launch_gather<T>((const T*)A, n_src, src, nullptr, W, nullptr, (const T*)Bt, (T*)out, n_dst,
                                       K, Kd, Nd, stream));
  });
  return ST_OK;
}

int st_hashfly_wgrad(const void* X, int64_t n_in, const void* dY, const void* out_coords, int coord_dtype,
                     int64_t n_out,
                     const int32_t* offsets, const st_lookup* lk, const uint64_t* keys, const uint32_t* vals,
                     int64_t capacity, int C_in, int C_out, int dtype, float* partials, int64_t splits, void* dW,
                     int dw_dtype, st_stream_t stream) {
  if (!lk || n_in < 0 || n_out < 0 || lk->K <= 0 || lk->K > ST_MAX_KVOL || C_in <= 0 || C_out <= 0 || splits < 1 ||
      splits > 65535)
    return ST_ERR_ARG;
  if (lk->mul < 1 || lk->div < 1 || (lk->sign != 1 && lk->sign != -1)) return ST_ERR_ARG;
  if (capacity <= 0 || capacity >= (1ll << 31) || n_out >= (1ll << 31)) return ST_ERR_ARG;
  if (!partials || !dW || (n_out > 0 && (!X || !dY || !out_coords || !offsets || !keys || !vals)))
    return ST_ERR_ARG;
  ST_DISPATCH_COORD(coord_dtype, CT, {
    HashSrc<CT> src{(const CT*)out_coords, offsets,       keys,          vals,          (uint32_t)capacity,
                    lk->sign,               lk->mul,       lk->div,       lk->bounds[0], lk->bounds[1],
                    lk->bounds[2],          lk->row_bounds[0], lk->row_bounds[1], lk->row_bounds[2]};
    ST_DISPATCH_DTYPE(dtype, T,
                      launch_wgrad<T>((const T*)X, n_in, (const T*)dY, src, n_out, lk->K, C_in, C_out, partials,
                                      splits, dW, dw_dtype, stream));
  });
  return ST_OK;
}

}  // extern "C"
