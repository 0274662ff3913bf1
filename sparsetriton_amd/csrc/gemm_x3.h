// fp32 gather-GEMM and weight gradient on bf16 MFMA with split operands.
//
// gfx950's matrix cores run bf16 at 16x the fp32 rate.  Each fp32 operand x
// is split into bf16 parts hi = bf16(x) and lo = bf16(x - hi), so
// x = hi + lo + d with |d| <= 2^-18 |x|, and a product is taken as
//     a*b ~= ah*bh + ah*bl + al*bh           (three bf16 MFMAs)
// leaving out al*bl (<= 2^-16 |ab|).  Products are exact in the fp32
// accumulator, so every product carries a relative error of at most ~2^-15
// (3e-5) -- about 16x tighter than a TF32 product (10-bit mantissa) --
// and sums accumulate in fp32 as in the plain fp32 kernels.  Inputs,
// outputs and weights stay fp32 in HBM; the split happens in registers as
// tiles are loaded.
//
// The kernels mirror the 16-bit ones (gemm_kernels.h): the forward / input
// gradient gather-GEMM with a double-buffered B tile in LDS (hi and lo
// planes) and A rows prefetched one offset ahead; the weight gradient with
// per-wave 32-pair steps staged row-major in LDS.
#pragma once

#include "gemm_kernels.h"

namespace st {


// ------------------------------------------------------ forward / dgrad
//
// Same structure as gather_gemm_pipe_kernel: 128 destination rows per
// workgroup (a wave owns 32), BN output columns, the tile's active offsets
// in klist order, sources of up to kSrcGroup offsets resolved into LDS at
// once.  Reduction steps are 32 wide (KS steps cover Kd).
template <int BN, int KS, typename Src, typename E>
__global__ __launch_bounds__(256) void gather_gemm_x3_kernel(
    const float* __restrict__ A, Src src, const uint32_t* __restrict__ masks, int W, const int32_t* __restrict__ rows,
    const float* __restrict__ Bt, float* __restrict__ out, int64_t n_src, int64_t n_dst, int K, int Kd, int Nd,
    int vec_a, int vec_b, E epi) {
  constexpr int KDP = KS * 32;
  constexpr int PITCH = KDP + 8;  // bf16 elements per LDS row of the B tile
  constexpr int NBLK = BN / 16;
  constexpr int CV = KDP / 4;  // 4-float chunks per B row
  constexpr int BREGS = (BN * CV + 255) / 256;
  __shared__ __attribute__((aligned(16))) __bf16 bt_s[2][2][BN * PITCH];  // [buffer][hi, lo]
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
  // raw fp32 A fragments: [m][step][half] = 4 consecutive reduction elements
  auto load_a = [&](int32_t s0, int32_t s1, v4f (&a)[2][KS][2]) {
#pragma unroll
    for (int j = 0; j < KS; ++j) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int col = j * 32 + g * 8 + h * 4;
        a[0][j][h] = s0 >= 0 ? load_frag<float>(A + (int64_t)s0 * Kd, col, Kd, vec_a) : zero_frag<float>();
        a[1][j][h] = s1 >= 0 ? load_frag<float>(A + (int64_t)s1 * Kd, col, Kd, vec_a) : zero_frag<float>();
      }
    }
  };
  auto load_b = [&](int k, v4f (&b)[BREGS]) {
#pragma unroll
    for (int j = 0; j < BREGS; ++j) {
      const int idx = tid + j * 256;
      const int nr = idx / CV, cv = idx - nr * CV;
      b[j] = zero_frag<float>();
      if (idx < BN * CV && n0 + nr < Nd)
        b[j] = load_frag<float>(Bt + ((int64_t)k * Nd + n0 + nr) * Kd, cv * 4, Kd, vec_b);
    }
  };
  auto store_b = [&](int buf, const v4f (&b)[BREGS]) {
#pragma unroll
    for (int j = 0; j < BREGS; ++j) {
      const int idx = tid + j * 256;
      const int nr = idx / CV, cv = idx - nr * CV;
      if (idx < BN * CV) {
        v4bf hi, lo;
        split4(b[j], hi, lo);
        *reinterpret_cast<v4bf*>(&bt_s[buf][0][nr * PITCH + cv * 4]) = hi;
        *reinterpret_cast<v4bf*>(&bt_s[buf][1][nr * PITCH + cv * 4]) = lo;
      }
    }
  };

  v4f acc[2][NBLK];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) acc[m][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  if (nk > 0) {
    v4f a_cur[2][KS][2], a_nxt[2][KS][2];
    v4f breg[BREGS];
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
        const __bf16* bh_s = bt_s[i & 1][0];
        const __bf16* bl_s = bt_s[i & 1][1];
#pragma unroll
        for (int j = 0; j < KS; ++j) {
          v8bf ah[2], al[2];
          split8(a_cur[0][j][0], a_cur[0][j][1], ah[0], al[0]);
          split8(a_cur[1][j][0], a_cur[1][j][1], ah[1], al[1]);
#pragma unroll
          for (int nb = 0; nb < NBLK; ++nb) {
            const int off = (nb * 16 + c) * PITCH + j * 32 + g * 8;
            const v8bf bh = *reinterpret_cast<const v8bf*>(&bh_s[off]);
            const v8bf bl = *reinterpret_cast<const v8bf*>(&bl_s[off]);
            acc[0][nb] = mfma_x3(ah[0], al[0], bh, bl, acc[0][nb]);
            acc[1][nb] = mfma_x3(ah[1], al[1], bh, bl, acc[1][nb]);
          }
        }
      }
      if (has_next) store_b((i + 1) & 1, breg);
      __syncthreads();
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int j = 0; j < KS; ++j) {
          a_cur[m][j][0] = a_nxt[m][j][0];
          a_cur[m][j][1] = a_nxt[m][j][1];
        }
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
        float* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = ov[m][r][nb];
        }
      }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
        if (drow < 0) continue;
        float* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = (epi.apply(acc[m][nb][r], em[nb], ea[nb], drow, Nd, col));
        }
      }
  }
}

// ------------------------------------------------ forward / dgrad, ring
//
// gather_gemm_ring_kernel with split operands: offset i's fp32 A rows and B
// tile are loaded D-1 offsets ahead into a register ring; B is split into
// hi / lo planes when stored to LDS, A when it is used.  Requires Kd =
// KS * 32 and 16-byte aligned A and Bt.
template <int BN, int KS, int D, typename Src, bool LINES, typename E>
__global__ __launch_bounds__(256) void gather_gemm_ring_x3_kernel(
    const float* __restrict__ A, Src src, const uint32_t* __restrict__ masks, int W, const int32_t* __restrict__ rows,
    const float* __restrict__ Bt, float* __restrict__ out, int64_t n_src, int64_t n_dst, int K, int Kd, int Nd,
    E epi) {
  constexpr int KDP = KS * 32;
  constexpr int PITCH = KDP + 8;
  constexpr int NBLK = BN / 16;
  constexpr int CV = KDP / 4;
  constexpr int BREGS = (BN * CV + 255) / 256;
  // Whole-line A gathers (LINES), as in gather_gemm_ring_kernel: CPR 16-byte
  // chunks per fp32 row, RPI rows per instruction, 4 * KS instructions per
  // step, rows staged per wave in LDS (chunk ch of row r at ch ^ (r mod CPR)).
  constexpr int CPR = KDP / 4;
  constexpr int RPI = 64 / CPR;
  static_assert(!LINES || (CPR >= 8 && CPR <= 32 && 4 * KS * RPI == 32), "whole-line gather shape");
  constexpr int SG = LINES ? 8 : kSrcGroup;
  // LINES: hi / lo B planes unpadded, 8-element chunk ch of row n at ch ^ bswz(n)
  constexpr int BCH = KDP / 8;  // chunks per B row
  constexpr int BPITCH = LINES ? KDP : PITCH;
  constexpr int BRPB = 16 / BCH > 0 ? 16 / BCH : 1;
  __shared__ __attribute__((aligned(16))) __bf16 bt_s[2][2][BN * BPITCH];
  __shared__ __attribute__((aligned(16))) float a_s[LINES ? 4 : 1][LINES ? 32 * KDP : 4];
  __shared__ uint32_t tmask_s[ST_MAX_KVOL / 32];
  __shared__ int32_t drow_s[kGemmBM];
  __shared__ int16_t klist_s[ST_MAX_KVOL];
  __shared__ int32_t src_s[SG][kGemmBM];
  __shared__ int nk_s;

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const RingTile tile = ring_tile(n_dst, Nd, BN);
  if (tile.rt * kGemmBM >= n_dst) return;  // padding of the folded grid (whole workgroup)
  const int64_t row0 = tile.rt * kGemmBM;
  const int n0 = tile.ct * BN;

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
  auto resolve_group = [&](int g0) {
    // one load in flight per thread at a time: batching the group's loads measured slower here
    // (config 2 fp32: 125 -> 138 us), unlike the 16-bit ring kernel
    const int ng = min(SG, nk - g0);
    for (int j = tid >> 7; j < ng; j += 2) {
      int32_t v;
      if constexpr (Src::kTiled)
        v = src.get_tile(tile.rt, g0 + j, tid & (kGemmBM - 1));
      else
        v = ld_row >= 0 ? src.get(rc, klist_s[g0 + j]) : -1;
      if ((int64_t)v >= n_src) v = -1;
      src_s[j][tid & (kGemmBM - 1)] = v;
    }
  };

  v4f a_ring[D][2][KS][2];
  v4f b_ring[D][BREGS];
  bool any_ring[D];
  v4f acc[2][NBLK];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) acc[m][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  // element offset of 8-element chunk ch of B row n (either plane)
  auto bpos = [](int n, int ch) -> int {
    if constexpr (LINES)
      return n * BPITCH + (ch ^ ((n / BRPB) % BCH)) * 8;
    else
      return n * BPITCH + ch * 8;
  };
  const int lr = lane / CPR, lc = lane % CPR;  // whole-line loader lanes
  float* const a_w = a_s[LINES ? wid : 0];
  // LINES: buffer loads (the host keeps both arrays under 2 GB); missing rows read zeros
  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(A, LINES ? n_src * Kd * 4 : 0);
  const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(Bt, LINES ? (int64_t)K * Nd * Kd * 4 : 0);
  auto issue = [&](int i, auto slot) {
    constexpr int SL = decltype(slot)::value;
    const int j = i % SG;
    if constexpr (LINES) {
      bool any = false;
#pragma unroll
      for (int v = 0; v < 4 * KS; ++v) {
        const int32_t sv = src_s[j][wid * 32 + v * RPI + lr];
        any |= sv >= 0;
        a_ring[SL][v / (2 * KS)][(v / 2) % KS][v % 2] = load16<v4f>(a_rsrc, sv >= 0 ? sv * (Kd * 4) + lc * 16 : kOobOffset);
      }
      any_ring[SL] = __ballot(any) != 0ull;
    } else {
      const int32_t s0 = src_s[j][wid * 32 + c];
      const int32_t s1 = src_s[j][wid * 32 + 16 + c];
      any_ring[SL] = __ballot(s0 >= 0 || s1 >= 0) != 0ull;
      const v4f* ar0 = reinterpret_cast<const v4f*>(A + (int64_t)(s0 >= 0 ? s0 : 0) * Kd + g * 8);
      const v4f* ar1 = reinterpret_cast<const v4f*>(A + (int64_t)(s1 >= 0 ? s1 : 0) * Kd + g * 8);
#pragma unroll
      for (int jj = 0; jj < KS; ++jj)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          a_ring[SL][0][jj][h] = ar0[jj * 8 + h];
          a_ring[SL][1][jj][h] = ar1[jj * 8 + h];
          if (s0 < 0) a_ring[SL][0][jj][h] = zero_frag<float>();
          if (s1 < 0) a_ring[SL][1][jj][h] = zero_frag<float>();
        }
    }
    const int k = b_slice(src, klist_s[i]);
#pragma unroll
    for (int jb = 0; jb < BREGS; ++jb) {
      const int idx = tid + jb * 256;
      const int nr = idx / CV, cv = idx - nr * CV;
      const bool ok = idx < BN * CV && n0 + nr < Nd;
      if constexpr (LINES) {
        b_ring[SL][jb] = load16<v4f>(b_rsrc, ok ? ((k * Nd + n0 + nr) * Kd + cv * 4) * 4 : kOobOffset);
      } else {
        b_ring[SL][jb] = *reinterpret_cast<const v4f*>(Bt + ((int64_t)k * Nd + (ok ? n0 + nr : 0)) * Kd + cv * 4);
        if (!ok) b_ring[SL][jb] = zero_frag<float>();
      }
    }
  };
  auto step = [&](int g0, int gn, int i, auto slot) {
    constexpr int SL = decltype(slot)::value;
    constexpr int NSL = (SL + D - 1) % D;
    issue(g0 + min(i + D - 1, gn - 1), std::integral_constant<int, NSL>());
    const int buf = i & 1;
#pragma unroll
    for (int jb = 0; jb < BREGS; ++jb) {
      const int idx = tid + jb * 256;
      const int nr = idx / CV, cv = idx - nr * CV;
      if (idx < BN * CV) {
        v4bf hi, lo;
        split4_each(b_ring[SL][jb], hi, lo);
        const int o = bpos(nr, cv >> 1) + (cv & 1) * 4;
        *reinterpret_cast<v4bf*>(&bt_s[buf][0][o]) = hi;
        *reinterpret_cast<v4bf*>(&bt_s[buf][1][o]) = lo;
      }
    }
    __syncthreads();
    if (i < gn && any_ring[SL]) {
      if constexpr (LINES) {
#pragma unroll
        for (int v = 0; v < 4 * KS; ++v) {
          const int r = v * RPI + lr;
          *reinterpret_cast<v4f*>(&a_w[r * KDP + (lc ^ (r & (CPR - 1))) * 4]) =
              a_ring[SL][v / (2 * KS)][(v / 2) % KS][v % 2];
        }
        // LDS operations of one wave complete in order; the fences keep the
        // compiler from moving the fragment reads above the stores.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
#pragma unroll
      for (int jj = 0; jj < KS; ++jj) {
        // B fragments first: their LDS reads are then in flight while A is split
        v8bf bh[NBLK], bl[NBLK];
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int off = bpos(nb * 16 + c, jj * 4 + g);
          bh[nb] = *reinterpret_cast<const v8bf*>(&bt_s[buf][0][off]);
          bl[nb] = *reinterpret_cast<const v8bf*>(&bt_s[buf][1][off]);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the scheduler from sinking them to the MFMAs
        v8bf ah[2], al[2];
        if constexpr (LINES) {
          const int q = jj * 8 + g * 2;
          const float* r0 = a_w + c * KDP;
          const float* r1 = a_w + (16 + c) * KDP;
          const int z0 = c & (CPR - 1), z1 = (16 + c) & (CPR - 1);
          split8(*reinterpret_cast<const v4f*>(&r0[(q ^ z0) * 4]), *reinterpret_cast<const v4f*>(&r0[((q + 1) ^ z0) * 4]),
                 ah[0], al[0]);
          split8(*reinterpret_cast<const v4f*>(&r1[(q ^ z1) * 4]), *reinterpret_cast<const v4f*>(&r1[((q + 1) ^ z1) * 4]),
                 ah[1], al[1]);
        } else {
          split8(a_ring[SL][0][jj][0], a_ring[SL][0][jj][1], ah[0], al[0]);
          split8(a_ring[SL][1][jj][0], a_ring[SL][1][jj][1], ah[1], al[1]);
        }
        // the three products in three rounds over all 2 * NBLK accumulators, so that
        // consecutive MFMAs never feed each other (one round per product keeps
        // 2 * NBLK independent accumulations between dependent ones)
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          acc[0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[0], bh[nb], acc[0][nb], 0, 0, 0);
          acc[1][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[1], bh[nb], acc[1][nb], 0, 0, 0);
        }
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          acc[0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[0], bl[nb], acc[0][nb], 0, 0, 0);
          acc[1][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[1], bl[nb], acc[1][nb], 0, 0, 0);
        }
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          acc[0][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[0], bh[nb], acc[0][nb], 0, 0, 0);
          acc[1][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[1], bh[nb], acc[1][nb], 0, 0, 0);
        }
      }
    }
  };

  static_assert(D >= 2 && D <= 3, "ring depth 2..3");
  for (int g0 = 0; g0 < nk; g0 += SG) {
    const int gn = min(SG, nk - g0);
    if (g0 > 0) __syncthreads();
    resolve_group(g0);
    __syncthreads();
    issue(g0, std::integral_constant<int, 0>());
    if constexpr (D > 2) issue(g0 + min(1, gn - 1), std::integral_constant<int, 1>());
    for (int i0 = 0; i0 < gn; i0 += D) {
      step(g0, gn, i0, std::integral_constant<int, 0>());
      step(g0, gn, i0 + 1, std::integral_constant<int, 1 % D>());
      if constexpr (D > 2) step(g0, gn, i0 + 2, std::integral_constant<int, 2 % D>());
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
        float* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = ov[m][r][nb];
        }
      }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int32_t drow = drow_s[wid * 32 + m * 16 + g * 4 + r];
        if (drow < 0) continue;
        float* orow = out + (int64_t)drow * Nd;
#pragma unroll
        for (int nb = 0; nb < NBLK; ++nb) {
          const int col = n0 + nb * 16 + c;
          if (col < Nd) orow[col] = (epi.apply(acc[m][nb][r], em[nb], ea[nb], drow, Nd, col));
        }
      }
  }
}

// ------------------------------------------------------ weight gradient
//
// As wgrad_pairs_wave_kernel with fp32 rows: a wave stages its 32-pair step
// (X and dY rows, 64 channels each) in LDS as fp32 and splits the fragments
// as it reads them.  Requires C_in, C_out multiples of 64, 16-byte aligned.
//
// Row loads: a step's 32 rows of 64 floats (256 bytes, two cache lines) are
// read as 8 instructions of 4 whole rows each -- 16 consecutive lanes take one
// row's 16 chunks of 16 bytes -- so every load instruction touches 8 cache
// lines and uses all of each.  (Lane-per-row loads touch 64 lines for 16
// bytes each and re-reference every line 8 times, which the 32 KB L1 cannot
// hold across 8 resident waves.)  Each lane keeps its own pair index (lane
// mod 32) and takes the row index of instruction v from lane 4v + lane / 16.
//
// LDS layout: pair p's row of 64 floats is 16 chunks of 16 bytes; chunk ch is
// stored at position ch ^ swz(p & 7), swz(r) = (r & 1) << 2 | (r >> 1) & 3: a
// row store is one contiguous 256-byte span, and the fragment reads (lane
// group g takes pairs 4e + g) put the two lane groups read together on
// disjoint bank halves.
constexpr int kWvPitchF = 64;
__device__ __forceinline__ int wv_swz(int r) { return ((r & 1) << 2) | ((r >> 1) & 3); }
// LDS float index of (pair p, channel col) in the swizzled layout
__device__ __forceinline__ int wv_at(int p, int col) {
  return p * kWvPitchF + ((((col >> 2) ^ wv_swz(p & 7)) << 2) | (col & 3));
}

// bf16 plane of a 32-pair step (32 rows x 64 channels): 4-element granule q of
// row r at position q ^ f(r), f(r) = 4 * (((r >> 1) & 1) | ((r >> 2) & 2)).
// The transpose reads below touch rows 8g + 4h + {0..3}; f puts the even (and
// the odd) rows of two lane groups read together on four different granule
// groups, so each half-wave covers 64 distinct banks.
__device__ __forceinline__ int pl_at(int r, int col) {
  const int f = (((r >> 1) & 1) | ((r >> 2) & 2)) << 2;
  return r * 64 + ((((col >> 2) ^ f)) << 2) + (col & 3);
}

// MFMA operand fragment from a bf16 plane: lane (c, g) gets channel col0 + c
// of pairs 8g .. 8g+7 by two gfx950 transpose reads (ds_read_b64_tr_b16: in a
// 16-lane group, lane l receives element l mod 4 of the 4 elements lane
// 4e + l/4 addresses, e = 0..3), lane c addressing pair 8g + 4h + c/4 at
// channel col0 + 4 (c mod 4).
__device__ __forceinline__ v8bf tr_plane(const __bf16* plane, int g, int c, int col0) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef short v8s __attribute__((ext_vector_type(8)));
  using lds_v4s = __attribute__((address_space(3))) v4s;
  const int r = g * 8 + (c >> 2), col = col0 + (c & 3) * 4;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(plane + pl_at(r, col)));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(plane + pl_at(r + 4, col)));
  return __builtin_bit_cast(v8bf, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}
template <bool BUF>  // BUF: row loads through buffer resources (X and dY under 2 GB)
__global__ __launch_bounds__(256, 2) void wgrad_pairs_x3_kernel(const float* __restrict__ X,
                                                                const float* __restrict__ dY,
                                                                const int2* __restrict__ pairs,
                                                                const int32_t* __restrict__ kstart,
                                                                const int32_t* __restrict__ cstart,
                                                                const int32_t* __restrict__ chunk_order, int K, int chunk,
                                                                int Cin, int Cout, int64_t n_in, int64_t n_out,
                                                                float* __restrict__ partials) {
  constexpr int STAGE = 32 * 64;  // bf16 elements per plane (4 planes per wave: X hi, X lo, dY hi, dY lo)
  constexpr int STAGE_BYTES = 4 * 4 * STAGE * 2;
  constexpr int RP = 68;
  constexpr int RED_BYTES = 4 * 64 * RP * (int)sizeof(float);
  __shared__ int32_t cstart_s[ST_MAX_KVOL + 2];
  __shared__ __attribute__((aligned(16))) unsigned char lds[STAGE_BYTES > RED_BYTES ? STAGE_BYTES : RED_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  for (int t = tid; t <= K + (chunk <= 0); t += 256) cstart_s[t] = cstart[t];  // + the size, when chosen by the list
  __syncthreads();
  const int total = cstart_s[K];

  const int ntn = Cout / 64;
  const ChunkTile ct = chunk_tile(total, (Cin / 64) * ntn);
  const int cm0 = (ct.tile / ntn) * 64, cn0 = (ct.tile % ntn) * 64;
  __bf16* xh = reinterpret_cast<__bf16*>(lds) + wid * 4 * STAGE;
  __bf16* xl = xh + STAGE;
  __bf16* yh = xl + STAGE;
  __bf16* yl = yh + STAGE;
  float* red = reinterpret_cast<float*>(lds);
  const int lr = lane >> 4, lc = lane & 15;  // loader lanes: row lr of each 4-row group, 16-byte chunk lc
  const __amdgpu_buffer_rsrc_t x_rsrc = make_rsrc(X, BUF ? n_in * Cin * 4 : 0);
  const __amdgpu_buffer_rsrc_t y_rsrc = make_rsrc(dY, BUF ? n_out * Cout * 4 : 0);

  for (int cq = ct.q0; cq < ct.q1; cq += ct.step) {
    const int cidx = chunk_order ? chunk_order[cq] : cq;
    const int k = chunk_offset(cstart_s, K, cidx);
    const int ch = chunk > 0 ? chunk : cstart_s[K + 1];  // the plan's own size when not given
    const int p0 = kstart[k] + (cidx - cstart_s[k]) * ch;
    const int p1 = min(p0 + ch, kstart[k + 1]);
    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    v4f xr[8], yr[8];
    // pair indices one step ahead of the rows they address (no index load in
    // front of a step's row gathers)
    auto load_pairs = [&](int q) {
      const int p = q + (lane & 31);
      return p < p1 ? pairs[p] : make_int2(-1, -1);
    };
    auto load_rows = [&](int2 pr) {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int ix = __shfl(pr.x, v * 4 + lr, 64), iy = __shfl(pr.y, v * 4 + lr, 64);
        if constexpr (BUF) {
          xr[v] = load16<v4f>(x_rsrc, ix >= 0 ? (ix * Cin + cm0 + lc * 4) * 4 : kOobOffset);
          yr[v] = load16<v4f>(y_rsrc, iy >= 0 ? (iy * Cout + cn0 + lc * 4) * 4 : kOobOffset);
        } else {
          xr[v] = ix >= 0 ? *reinterpret_cast<const v4f*>(X + (int64_t)ix * Cin + cm0 + lc * 4) : zero_frag<float>();
          yr[v] = iy >= 0 ? *reinterpret_cast<const v4f*>(dY + (int64_t)iy * Cout + cn0 + lc * 4) : zero_frag<float>();
        }
      }
    };
    int q = p0 + wid * 32;
    int2 prn = load_pairs(q);
    if (q < p1) load_rows(prn);
    prn = load_pairs(q + 128);
    for (; q < p1; q += 128) {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        // split once per element as it is staged: hi = bf16(x), lo = bf16(x - hi)
        v4bf h, l;
        const int at = pl_at(v * 4 + lr, lc * 4);
        split4(xr[v], h, l);
        *reinterpret_cast<v4bf*>(&xh[at]) = h;
        *reinterpret_cast<v4bf*>(&xl[at]) = l;
        split4(yr[v], h, l);
        *reinterpret_cast<v4bf*>(&yh[at]) = h;
        *reinterpret_cast<v4bf*>(&yl[at]) = l;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (q + 128 < p1) {
        load_rows(prn);
        prn = load_pairs(q + 256);
      }
      v8bf bh[4], bl[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bh[j] = tr_plane(yh, g, c, j * 16);
        bl[j] = tr_plane(yl, g, c, j * 16);
      }
      v8bf ah[4], al[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ah[i] = tr_plane(xh, g, c, i * 16);
        al[i] = tr_plane(xl, g, c, i * 16);
      }
      // one round per product over all 16 accumulators: no MFMA waits on the one before it
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    __syncthreads();
    float* mine = red + wid * 64 * RP;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) mine[(i * 16 + g * 4 + r) * RP + j * 16 + c] = acc[i][j][r];
    __syncthreads();
    float* part = partials + (int64_t)cidx * Cin * Cout;
#pragma unroll 4
    for (int m = 0; m < 16; ++m) {
      const int e = tid + m * 256;
      const int row = e >> 6, col = e & 63;
      const float s = red[row * RP + col] + red[64 * RP + row * RP + col] + red[128 * RP + row * RP + col] +
                      red[192 * RP + row * RP + col];
      part[(int64_t)(cm0 + row) * Cout + cn0 + col] = s;
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------ launchers

template <int BN, int KS, typename Src, typename E>
static void launch_x3(const float* A, int64_t n_src, const Src& src, const uint32_t* masks, int W,
                      const int32_t* rows, const float* Bt, float* out, E epi, int64_t n_dst, int K, int Kd, int Nd,
                      int vec_a, int vec_b, hipStream_t stream) {
  const dim3 grid(st_blocks(n_dst, kGemmBM), st_blocks(Nd, BN));
  const unsigned rgrid = ring_grid(n_dst, Nd, BN);
  if (vec_a && vec_b && Kd == KS * 32 && gemm_ring_depth() == 2 && gather_lines() && buffer_ok(n_src, K, Kd, Nd, 4))
    gather_gemm_ring_x3_kernel<BN, KS, 2, Src, true, E>
        <<<rgrid, 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst, K, Kd, Nd, epi);
  else if (vec_a && vec_b && Kd == KS * 32 && gemm_ring_depth() == 2)
    gather_gemm_ring_x3_kernel<BN, KS, 2, Src, false, E>
        <<<rgrid, 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst, K, Kd, Nd, epi);
  else
    gather_gemm_x3_kernel<BN, KS, Src, E>
        <<<grid, 256, 0, stream>>>(A, src, masks, W, rows, Bt, out, n_src, n_dst, K, Kd, Nd, vec_a, vec_b, epi);
}

template <int KS, typename Src, typename E>
static void launch_x3_ks(const float* A, int64_t n_src, const Src& src, const uint32_t* masks, int W,
                         const int32_t* rows, const float* Bt, float* out, E epi, int64_t n_dst, int K, int Kd, int Nd,
                         int vec_a, int vec_b, hipStream_t stream) {
  if (Nd <= 16)
    launch_x3<16, KS>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  else if (Nd <= 32)
    launch_x3<32, KS>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  else
    launch_x3<64, KS>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
}

// Split-operand gather-GEMM for reductions up to 128 wide; deeper ones use
// the plain fp32 kernels.
template <typename Src, typename E>
static int launch_gather_x3_e(const float* A, int64_t n_src, const Src& src, const uint32_t* masks, int W,
                              const int32_t* rows, const float* Bt, float* out, E epi, int64_t n_dst, int K, int Kd,
                              int Nd, hipStream_t stream) {
  if constexpr (Src::kTiled) {
    if (gather_wide_mode() && wide_ok(Kd, Nd, K, sizeof(float), true, n_src, A, Bt)) {
      launch_wide<float, true, E>(A, n_src, src, rows, Bt, out, epi, n_dst, Kd, Nd, stream);
      ST_CHECK_LAUNCH();
      return ST_OK;
    }
  }
  const int ks = (Kd + 31) / 32;
  if (ks > 4) {
    if constexpr (Src::kTiled)
      return ST_ERR_UNSUPPORTED;
    else
      return launch_gather_e<float, Src, E>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, stream);
  }
  const int vec_a = (Kd % 4 == 0) && ((uintptr_t)A % 16 == 0);
  const int vec_b = (Kd % 4 == 0) && ((uintptr_t)Bt % 16 == 0);
  if (ks == 1)
    launch_x3_ks<1>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  else if (ks == 2)
    launch_x3_ks<2>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  else
    launch_x3_ks<4>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, vec_a, vec_b, stream);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

template <typename Src>
static int launch_gather_x3(const float* A, int64_t n_src, const Src& src, const uint32_t* masks, int W,
                            const int32_t* rows, const float* Bt, float* out, Epi<float> epi, int64_t n_dst, int K,
                            int Kd, int Nd, hipStream_t stream) {
  if (epi.scale || epi.shift || epi.residual || epi.relu) {
    if constexpr (Src::kTiled)
      return launch_gather_x3_e<Src, Epi<float>>(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd,
                                                 stream);
    else
      return ST_ERR_UNSUPPORTED;
  }
  return launch_gather_x3_e<Src, BiasEpi<float>>(A, n_src, src, masks, W, rows, Bt, out, BiasEpi<float>{epi.bias},
                                                 n_dst, K, Kd, Nd, stream);
}

}  // namespace st
