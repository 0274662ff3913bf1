// Wide-wave gather-GEMM over a tile plan (forward and input gradient).
//
// One workgroup = two waves = one 128-row destination tile x all Nd = BN
// output columns.  Wave w owns tile rows 64w .. 64w + 63 (four 16-row MFMA
// blocks) and every 16-column block.  Per active offset of the tile:
//   A  each lane loads its MFMA fragments straight from memory into
//      registers: lanes 16g .. 16g + 15 of row block m take rows
//      16m + (lane & 15) at reduction elements 32s + 8g .. +8 (16 bytes; fp32:
//      32 bytes, split into bf16 hi / lo in registers when used).  A row's
//      four lane groups cover 64 (fp32: 128) consecutive bytes.  Loads run D-1
//      offsets ahead in a register ring;
//   B  Bt[k] (BN x KD) passes through LDS, double-buffered, loaded one offset
//      ahead: stored once, read by both waves (fp32: split into hi / lo
//      planes as it is stored).
// Per offset the LDS then carries B three times (one store, two reads) and no
// A.  The four-wave ring kernels stage A through LDS as well and, with 32-row
// wave tiles, read every B fragment for half as many MFMAs: at C = 64..128
// their LDS traffic exceeds what the CU's LDS delivers in the MFMA time.
//
// Every destination row accumulates its offsets in the tile's ascending order
// with one MFMA per 32-element step (fp32: the three split products in the
// order of mfma_x3), exactly as the ring kernels do, so the two agree bitwise.
// The tile's source rows (nk x 128) are copied to LDS first, so nk <= kWideMaxK.
//
// With a FlySrc (submanifold, no kernel map) the tile is 128 rows of the given
// order (consecutive rows without one) and the prologue finds the sources itself: each thread looks its row's K
// neighbours up in the coordinates' brick index (subm_index.h), the tile's
// offset list is the union of its rows' (offsets no row of the tile has are
// never loaded), and the main loop is the same.  A row with a neighbour
// through offset k gets the same sum as from a map or a hash-table probe:
// offsets it lacks add exact zeros.
#pragma once

#include <type_traits>

#include "mfma.h"
#include "nbr_src.h"
#include "subm_index.h"

namespace st {

constexpr int kWideMaxK = 27;  // offsets whose sources a wide workgroup holds (a 3x3x3 kernel)

// Neighbours of destination row r looked up in a brick index (source rows are
// the same coordinate set's rows: out = in, stride 1).  rows (optional): the
// destination rows in tile order, a permutation of 0 .. n-1 (e.g. sorted by
// offset mask, so a tile's rows share their offsets); null = 0 .. n-1.
// rev: offset k's B slice is Bt[K - 1 - k].
template <typename CT>
struct FlySrc {
  static constexpr bool kTiled = false;
  static constexpr bool kRev = true;
  const CT* __restrict__ coords;
  const int32_t* __restrict__ offsets;  // K x 3
  SubmIndex ix;
  int K;
  const int32_t* __restrict__ rows;
  int rev;
};

// ST_GATHER_WIDE=0 keeps the four-wave kernels everywhere, =2 takes the wide one
// for every width it is built for (A/B timing); default: 128 x 128 only.
inline int gather_wide_mode() {
  static int mode = -1;
  if (mode < 0) {
    const char* e = getenv("ST_GATHER_WIDE");
    mode = (e && e[0] == '0') ? 0 : (e && e[0] == '2') ? 2 : 1;
  }
  return mode;
}

template <typename T, bool X3, int KD, int BN, int D, typename E, typename S, int TP>
__global__ __launch_bounds__(128 * TP) void gather_gemm_wide_kernel(const T* __restrict__ A, S src,
                                                                    const int32_t* __restrict__ rows,
                                                                    const T* __restrict__ Bt, T* __restrict__ out,
                                                                    int64_t n_src, int64_t n_dst, E epi) {
  static_assert(X3 == std::is_same<T, float>::value, "fp32 runs split, 16-bit types direct");
  static_assert(TP == 1 || TP == 2, "one or two tiles per workgroup");
  using L16 = typename std::conditional<X3, __bf16, T>::type;  // LDS / MFMA element
  using F16 = typename Frag<L16>::type;                          // 8 x 16-bit MFMA operand
  constexpr int NT = 128 * TP;                                   // threads
  constexpr int KSTEPS = KD / 32;
  constexpr int NBLK = BN / 16;
  constexpr int MB = 4;
  constexpr int CV = KD / 8;                       // 16-byte 16-bit chunks per B row in LDS
  constexpr int BRPB = 16 / CV > 0 ? 16 / CV : 1;  // B rows per 256 bytes
  constexpr int PLANES = X3 ? 2 : 1;
  constexpr int GCH = X3 ? KD / 4 : KD / 8;  // 16-byte global chunks per B row
  constexpr int BREGS = BN * GCH / NT;
  constexpr int AH = X3 ? 2 : 1;  // 16-byte loads per A fragment
  static_assert(KD % 32 == 0 && BN % 16 == 0 && (BN * GCH) % NT == 0, "wide tile shape");
  static_assert(D >= 2 && D <= 3, "ring depth 2..3");
  using GV = typename std::conditional<X3, v4f, F16>::type;  // one 16-byte global load

  // B, double-buffered; before the main loop a submanifold source's prologue
  // keeps its unit_rows lookup tables (8 brick words and bases per thread)
  // here too, so the buffer is sized for both
  constexpr int BT_BYTES = 2 * PLANES * BN * KD * (int)sizeof(L16);
  constexpr int LK_BYTES = S::kTiled ? 0 : 8 * NT * (int)(sizeof(unsigned long long) + sizeof(int32_t));
  __shared__ __attribute__((aligned(16))) unsigned char bt_raw[BT_BYTES > LK_BYTES ? BT_BYTES : LK_BYTES];
  auto bt_s = reinterpret_cast<L16 (*)[PLANES][BN * KD]>(bt_raw);
  __shared__ int32_t src_s[TP][kWideMaxK][kGemmBM];  // per tile: sources by list position (tiled) or offset (fly)
  __shared__ int32_t drow_s[TP][kGemmBM];
  __shared__ int16_t klist_s[TP][kWideMaxK];  // per tile's offset list (tiled)
  __shared__ int16_t uk_s[kWideMaxK];         // the workgroup's offsets: the union of its tiles'
  __shared__ int8_t pos_s[TP][kWideMaxK];     // per union offset and tile: its src_s index, -1 if absent
  __shared__ uint32_t tmask_s[TP];
  __shared__ int nk_s[TP];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = lane & 15, g = lane >> 4;
  const int hw = wid >> 1, wt = wid & 1;       // the wave's tile and its 64-row half
  const int ht = tid >> 7, r = tid & 127;      // the thread's tile and row in the prologue
  // tiles in descending order (the mask sort puts the rows with the most neighbours last); with
  // two tiles per workgroup, tiles 2p and 2p + 1
  const int64_t nrt = (n_dst + kGemmBM - 1) / kGemmBM;
  int64_t t0;
  if constexpr (TP == 1) {
    const RingTile tile = ring_tile(n_dst, BN, BN);
    t0 = tile.rt;
    if (t0 * kGemmBM >= n_dst) return;
  } else {
    t0 = 2 * ((nrt + 1) / 2 - 1 - (int64_t)blockIdx.x);
  }
  const int64_t th = t0 + ht;  // this thread's tile
  const bool tvalid = th < nrt;
  if (tid < TP) tmask_s[tid] = 0u;

  if constexpr (S::kTiled) {
    const int nkh = tvalid ? src.nk[th] : 0;
    if (r == 0) nk_s[ht] = nkh;
    {
      const int64_t gr = th * kGemmBM + r;
      drow_s[ht][r] = (tvalid && gr < n_dst) ? rows[gr] : -1;
    }
    if (r < nkh) klist_s[ht][r] = src.klist[th * src.K + r];
    {
      // the tile's sources, offset-major as the plan stores them: thread r takes row r of every offset,
      // all loads in flight together
      const int32_t* tm = src.tmap + th * (int64_t)src.K * kGemmBM + r;
      int32_t v[kWideMaxK];
#pragma unroll
      for (int j = 0; j < kWideMaxK; ++j) v[j] = j < nkh ? tm[j * kGemmBM] : -1;
#pragma unroll
      for (int j = 0; j < kWideMaxK; ++j)
        if (j < nkh) src_s[ht][j][r] = (int64_t)v[j] >= n_src ? -1 : v[j];
    }
    __syncthreads();
    if (tid < TP) {
      uint32_t m = 0u;
      for (int j = 0; j < nk_s[tid]; ++j) m |= 1u << klist_s[tid][j];
      tmask_s[tid] = m;
    }
  } else {
    // sources by offset (src_s[.][k])
    __shared__ int32_t off_s[kWideMaxK * 3];
    const int K = src.K;
    for (int j = tid; j < 3 * K; j += NT) off_s[j] = src.offsets[j];
    __syncthreads();
    const int64_t gr = th * kGemmBM + r;
    const bool live = tvalid && gr < n_dst;
    const int32_t d = live ? (src.rows ? src.rows[gr] : (int32_t)gr) : -1;
    drow_s[ht][r] = d;
    uint32_t m = 0u;
    if (live) {
      int64_t b, x, y, z;
      load_coord(src.coords, d, b, x, y, z);
      auto found = [&](int k, int32_t v) {
        v = (int64_t)v >= n_src ? -1 : v;
        src_s[ht][k][r] = v;
        m |= (v >= 0 ? 1u : 0u) << k;
      };
      if (unit_offsets(src.offsets, K))  // (uniform) the 3x3x3 kernel: 32-bit lookups, words in LDS
        unit_rows<NT>(src.ix, b, x, y, z, src.offsets, K, reinterpret_cast<unsigned long long*>(bt_raw),
                      reinterpret_cast<int32_t*>(bt_raw + 8 * NT * sizeof(unsigned long long)), found);
      else
        subm_neighbours(src.ix, b, x, y, z, off_s, K, found);
    } else {
      for (int k = 0; k < K; ++k) src_s[ht][k][r] = -1;
    }
    if (m) atomicOr(&tmask_s[ht], m);
  }
  __syncthreads();
  // the union of the tiles' offsets, ascending; per tile, where each sits in its sources
  uint32_t um = 0u;
#pragma unroll
  for (int h = 0; h < TP; ++h) um |= tmask_s[h];
  const int nk = __popc(um);
  if (tid < kWideMaxK && ((um >> tid) & 1u)) {
    const int i = __popc(um & ((1u << tid) - 1u));
    uk_s[i] = (int16_t)tid;
#pragma unroll
    for (int h = 0; h < TP; ++h) {
      const uint32_t mh = tmask_s[h];
      pos_s[h][i] = ((mh >> tid) & 1u) ? (int8_t)(S::kTiled ? __popc(mh & ((1u << tid) - 1u)) : tid) : (int8_t)-1;
    }
  }
  __syncthreads();

  const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(A, n_src * KD * (int64_t)sizeof(T));
  const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(Bt, (int64_t)src.K * BN * KD * (int64_t)sizeof(T));

  GV a_ring[D][MB][KSTEPS][AH];
  bool any_ring[D];
  GV b_reg[BREGS];
  v4f acc[MB][NBLK];
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int nb = 0; nb < NBLK; ++nb) acc[m][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  // element offset of 16-bit chunk ch of B row n (XOR swizzle: the 16 rows one fragment read
  // touches land on distinct bank groups)
  auto bpos = [](int n, int ch) -> int { return n * KD + (ch ^ ((n / BRPB) % CV)) * 8; };

  auto issue_a = [&](int i, auto slot) {
    constexpr int SL = decltype(slot)::value;
    bool any = false;
    const int si = pos_s[hw][i];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const int32_t sv = si >= 0 ? src_s[hw][si][wt * 64 + m * 16 + c] : -1;
      any |= sv >= 0;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
        for (int h = 0; h < AH; ++h) {
          const int col = s * 32 + g * 8 + h * 4;  // element
          a_ring[SL][m][s][h] =
              load16<GV>(a_rsrc, sv >= 0 ? (sv * KD + col) * (int)sizeof(T) : kOobOffset);
        }
    }
    any_ring[SL] = __ballot(any) != 0ull;
  };
  auto issue_b = [&](int i) {
    const int k = b_slice(src, uk_s[i]);
#pragma unroll
    for (int jb = 0; jb < BREGS; ++jb) {
      const int idx = tid + jb * NT;
      const int nr = idx / GCH, cv = idx - nr * GCH;
      b_reg[jb] = load16<GV>(b_rsrc, ((k * BN + nr) * KD + cv * (16 / (int)sizeof(T))) * (int)sizeof(T));
    }
  };
  auto store_b = [&](int buf) {
#pragma unroll
    for (int jb = 0; jb < BREGS; ++jb) {
      const int idx = tid + jb * NT;
      const int nr = idx / GCH, cv = idx - nr * GCH;
      if constexpr (X3) {
        v4bf hi, lo;
        split4(b_reg[jb], hi, lo);
        const int o = bpos(nr, cv >> 1) + (cv & 1) * 4;
        *reinterpret_cast<v4bf*>(&bt_s[buf][0][o]) = hi;
        *reinterpret_cast<v4bf*>(&bt_s[buf][1][o]) = lo;
      } else {
        *reinterpret_cast<F16*>(&bt_s[buf][0][bpos(nr, cv)]) = b_reg[jb];
      }
    }
  };
  auto compute = [&](int buf, auto slot) {
    constexpr int SL = decltype(slot)::value;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      F16 bh[NBLK], bl[NBLK];
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb) {
        const int off = bpos(nb * 16 + c, s * 4 + g);
        bh[nb] = *reinterpret_cast<const F16*>(&bt_s[buf][0][off]);
        if constexpr (X3) bl[nb] = *reinterpret_cast<const F16*>(&bt_s[buf][PLANES - 1][off]);
      }
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        if constexpr (X3) {
          v8bf ah, al;
          split8(a_ring[SL][m][s][0], a_ring[SL][m][s][1], ah, al);
#pragma unroll
          for (int nb = 0; nb < NBLK; ++nb) acc[m][nb] = mfma_x3(ah, al, bh[nb], bl[nb], acc[m][nb]);
        } else {
#pragma unroll
          for (int nb = 0; nb < NBLK; ++nb) acc[m][nb] = mfma(a_ring[SL][m][s][0], bh[nb], acc[m][nb]);
        }
      }
    }
  };
  // Step i (ring slot SL = i % D): B(i) into LDS buffer i & 1, loads of B(i + 1) and of A(i + D - 1)
  // (clamped to the last offset, so every step issues the same loads and the compiler's count of
  // loads in flight stays exact), barrier, MFMAs of offset i.  The barrier also orders this step's
  // B store after the other wave's reads of the same buffer two steps back.
  auto step = [&](int i, auto slot) {
    constexpr int SL = decltype(slot)::value;
    constexpr int NSL = (SL + D - 1) % D;
    store_b(i & 1);
    issue_b(min(i + 1, nk - 1));
    issue_a(min(i + D - 1, nk - 1), std::integral_constant<int, NSL>());
    __syncthreads();
    if (i < nk && any_ring[SL]) compute(i & 1, slot);
  };

  if (nk > 0) {
    issue_b(0);
    issue_a(0, std::integral_constant<int, 0>());
    if constexpr (D > 2) issue_a(min(1, nk - 1), std::integral_constant<int, 1>());
    for (int i0 = 0; i0 < nk; i0 += D) {
      step(i0, std::integral_constant<int, 0>());
      step(i0 + 1, std::integral_constant<int, 1 % D>());
      if constexpr (D > 2) step(i0 + 2, std::integral_constant<int, 2 % D>());
    }
  }

  // store epilogue: lane (c, g) holds rows 16m + 4g + r, column 16nb + c of the wave's block
  float em[NBLK], ea[NBLK];
#pragma unroll
  for (int nb = 0; nb < NBLK; ++nb) epi.column(nb * 16 + c, BN, em[nb], ea[nb]);
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int32_t drow = drow_s[hw][wt * 64 + m * 16 + g * 4 + rr];
      if (drow < 0) continue;
      float ov[NBLK];
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb) ov[nb] = epi.apply(acc[m][nb][rr], em[nb], ea[nb], drow, BN, nb * 16 + c);
      T* orow = out + (int64_t)drow * BN;
#pragma unroll
      for (int nb = 0; nb < NBLK; ++nb) orow[nb * 16 + c] = from_f32<T>(ov[nb]);
    }
}

// Whether the wide kernel takes a tiled gather.  Shapes where it measured
// faster: 16-bit 128 x 128 (config 5: 1.16 -> 0.87 ms per gather); split fp32
// with exactly one width 128 (config 3, 64 -> 128: step 0.88 -> 0.77 ms).  At
// 64 x 64 (config 2: bf16 56 vs 64 us, fp32 133 vs 148 us) and 16-bit 64 x 128 /
// 128 x 64 (config 4: step 2.20 vs 2.32 ms) the four-wave kernels stay ahead,
// their whole-line A gathers touching half as many cache lines per load.  Split
// fp32 at 128 x 128 stages 64 KB of fp32 B per offset in registers: with the
// 128 x 128 accumulators that overflows the VGPRs into AGPR copies
// (SparseResNet21D fp32 step 24.4 -> 39.8 ms with it).  Also: a
// 3x3x3-sized offset list, 16-byte aligned operands, A and Bt under 2 GB
// (32-bit buffer offsets).
inline bool wide_ok(int Kd, int Nd, int K, size_t esz, bool x3, int64_t n_src, const void* A, const void* Bt) {
  const bool built = (Kd == 64 || Kd == 128) && (Nd == 64 || Nd == 128);
  const bool faster = x3 ? ((Kd == 128) != (Nd == 128)) : (Kd == 128 && Nd == 128);
  return built && (faster || gather_wide_mode() == 2) && K <= kWideMaxK && (uintptr_t)A % 16 == 0 &&
         (uintptr_t)Bt % 16 == 0 && n_src * Kd * (int64_t)esz < (1ll << 31) - 64 &&
         (int64_t)K * Nd * Kd * (int64_t)esz < (1ll << 31) - 64;
}

// Shapes the wide kernel takes for a brick-index gather (FlySrc), where the
// alternative is a hash-table probe per (row, offset) in the four-wave
// kernels: every built width but split fp32 at 128 x 128 (the register
// overflow above); same operand limits as wide_ok.
inline bool fly_ok(int Kd, int Nd, int K, size_t esz, bool x3, int64_t n_src, const void* A, const void* Bt) {
  const bool built = (Kd == 64 || Kd == 128) && (Nd == 64 || Nd == 128);
  return built && !(x3 && Kd == 128 && Nd == 128) && K > 0 && K <= kWideMaxK && (uintptr_t)A % 16 == 0 &&
         (uintptr_t)Bt % 16 == 0 && n_src * Kd * (int64_t)esz < (1ll << 31) - 64 &&
         (int64_t)K * Nd * Kd * (int64_t)esz < (1ll << 31) - 64;
}

// Tiles per workgroup: two at 128 x 128 (16-bit), where one B slice per offset then serves 256
// rows (the B loads were a third of the address unit's work); ST_WIDE_TILES=1 / 2 overrides.
inline int wide_tiles(int Kd, int Nd, bool x3) {
  static int mode = -1;
  if (mode < 0) {
    const char* e = getenv("ST_WIDE_TILES");
    mode = (e && e[0] == '1') ? 1 : (e && e[0] == '2') ? 2 : 0;
  }
  if (mode) return mode;
  return (!x3 && Kd == 128 && Nd == 128) ? 2 : 1;
}

template <typename T, bool X3, typename E, typename S>
inline void launch_wide(const T* A, int64_t n_src, const S& src, const int32_t* rows, const T* Bt, T* out,
                        E epi, int64_t n_dst, int Kd, int Nd, hipStream_t stream) {
  const int64_t nrt = (n_dst + kGemmBM - 1) / kGemmBM;
  const int tp = wide_tiles(Kd, Nd, X3);
#define ST_WIDE(KD, BN)                                                                                           \
  if (tp == 2)                                                                                                    \
    gather_gemm_wide_kernel<T, X3, KD, BN, 2, E, S, 2><<<(unsigned)((nrt + 1) / 2), 256, 0, stream>>>(            \
        A, src, rows, Bt, out, n_src, n_dst, epi);                                                                \
  else                                                                                                            \
    gather_gemm_wide_kernel<T, X3, KD, BN, 2, E, S, 1><<<(unsigned)nrt, 128, 0, stream>>>(A, src, rows, Bt, out, \
                                                                                          n_src, n_dst, epi)
  if (Kd == 64 && Nd == 64)
    ST_WIDE(64, 64);
  else if (Kd == 64 && Nd == 128)
    ST_WIDE(64, 128);
  else if (Kd == 128 && Nd == 64)
    ST_WIDE(128, 64);
  else
    ST_WIDE(128, 128);
#undef ST_WIDE
}

}  // namespace st
