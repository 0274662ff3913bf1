// Brick index of a coordinate set (built by kmap_subm.hip) and its
// neighbour lookup, shared by the submanifold map query and the GEMMs that
// look neighbours up inside the kernel.
//
//   * bricks of 4x4x4 voxels, numbered ((b*BX + x/4)*BY + y/4)*BZ + z/4 over
//     the box [0, batches) x [0, shape);
//   * level 1: one 16-byte entry per 64 consecutive bricks -- a bit per brick
//     (occupied or not), the number of occupied bricks before the entry, and
//     the number of distinct voxels before it;
//   * level 2: one entry per occupied brick, in brick order -- a bit per
//     voxel (bit (x%4)*16 + (y%4)*4 + z%4) and the number of voxels in the
//     bricks before it;
//   * rowmap: voxel rank -> lowest row holding that voxel.
// A neighbour q resolves as: level-1 entry of q's brick, bit test, brick rank
// = entry's count + popcount below; level-2 bits and base, bit test, voxel
// rank = base + popcount below; rowmap[rank].  The result is the row a hash
// table of the coordinates returns for q (the lowest row of a repeated
// coordinate), or -1.
#pragma once

#include "common.h"

namespace st {

struct alignas(16) SubmL1 {
  unsigned long long bits;  // occupied bricks among the entry's 64
  int32_t bpre;             // occupied bricks before the entry
  int32_t v;                // distinct voxels in the entry's bricks, then voxels before the entry
};

struct SubmIndex {
  uint8_t* occ;  // one byte per brick of the box: 1 when occupied
  SubmL1* l1;
  unsigned long long* l2bits;  // per occupied brick (brick rank order)
  int32_t* l2pre;              // voxels before each occupied brick
  int32_t* rowmap;
  int32_t* tile_sums;          // per tile of kSubmTile level-1 entries: its bricks or voxels (ntiles + 1)
  int32_t* tile_pub;           // the tiles' published totals, bricks then voxels (2 x ntiles, cleared)
  // Overflow flag of an index whose rows bound is not a property of its input (the output
  // index of a strided / transposed build, sized from the kernel's candidate bound): set when
  // the occupied bricks exceed cap2 or the distinct voxels exceed nrows, after which the
  // build's later kernels return without touching the level-2 and rank arrays.  Null for the
  // index of a coordinate set, which cannot overflow (a row adds one voxel and one brick).
  int32_t* flag;
  int64_t nbricks, nw1, cap2, ntiles, nrows;
  int nb, sx, sy, sz, bx, by, bz;
};

constexpr int kSubmThreads = 256;
constexpr int kSubmTile = 256;  // level-1 entries per prefix workgroup (one per thread)
constexpr int kSubmGroup = 9;   // neighbour lookups in flight per row

__device__ __forceinline__ bool subm_in_box(const SubmIndex& ix, int64_t b, int64_t x, int64_t y, int64_t z) {
  return b >= 0 && b < ix.nb && x >= 0 && x < ix.sx && y >= 0 && y < ix.sy && z >= 0 && z < ix.sz;
}

__device__ __forceinline__ int64_t subm_brick(const SubmIndex& ix, int64_t b, int64_t x, int64_t y, int64_t z) {
  return ((b * ix.bx + (x >> 2)) * ix.by + (y >> 2)) * ix.bz + (z >> 2);
}

__device__ __forceinline__ int subm_vbit(int64_t x, int64_t y, int64_t z) {
  return (int)(((x & 3) << 4) | ((y & 3) << 2) | (z & 3));
}

__device__ __forceinline__ unsigned long long below(int bit) { return (1ull << bit) - 1ull; }

// Whether the index's overflow flag is set (a uniform scalar load; false for
// an index without one).
__device__ __forceinline__ bool subm_overflowed(const SubmIndex& ix) {
  return ix.flag && *ix.flag != 0;
}

// brick rank of an in-box coordinate whose brick is occupied
__device__ __forceinline__ int subm_brick_rank(const SubmL1& e, int64_t br) {
  return e.bpre + (int)__popcll(e.bits & below((int)(br & 63)));
}

// The rows of the coordinates (b, q) that q_of(k, qx, qy, qz) yields (false:
// none), passed to emit(k, row) in ascending k = 0 .. K-1 (row -1: no
// coordinate, outside the box or absent).  kSubmGroup lookups are in flight at
// a time, each three dependent loads (level-1 entry; level-2 bits and base;
// rowmap); G (default kSubmGroup) sets how many.
template <int G = kSubmGroup, typename Q, typename Emit>
__device__ __forceinline__ void subm_lookup(const SubmIndex& ix, int64_t b, int K, Q&& q_of, Emit&& emit) {
  for (int k0 = 0; k0 < K; k0 += G) {
    int64_t brk[G];
    int vb[G];
    bool in[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int k = k0 + j;
      in[j] = false;
      brk[j] = 0;
      vb[j] = 0;
      int64_t qx, qy, qz;
      if (k < K && q_of(k, qx, qy, qz) && subm_in_box(ix, b, qx, qy, qz)) {
        in[j] = true;
        brk[j] = subm_brick(ix, b, qx, qy, qz);
        vb[j] = subm_vbit(qx, qy, qz);
      }
    }
    SubmL1 e1[G];
#pragma unroll
    for (int j = 0; j < G; ++j) e1[j] = in[j] ? ix.l1[brk[j] >> 6] : SubmL1{0ull, 0, 0};
    unsigned long long bits[G];
    int32_t pre[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      in[j] = in[j] && ((e1[j].bits >> (brk[j] & 63)) & 1ull);
      const int r = in[j] ? subm_brick_rank(e1[j], brk[j]) : 0;
      bits[j] = in[j] ? ix.l2bits[r] : 0ull;
      pre[j] = in[j] ? ix.l2pre[r] : 0;
    }
    int32_t rr[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const bool has = in[j] && ((bits[j] >> vb[j]) & 1ull);
      rr[j] = has ? ix.rowmap[pre[j] + (int)__popcll(bits[j] & below(vb[j]))] : -1;
    }
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (k0 + j < K) emit(k0 + j, rr[j]);
  }
}

// The rows of (b, x, y, z) - off_s[k] for k = 0 .. K-1, passed to emit(k, row)
// in ascending k (row -1: outside the box or absent): subm_lookup over the
// offsets (any size; unit offsets take unit_rows).
template <int G = kSubmGroup, typename Emit>
__device__ __forceinline__ void subm_neighbours(const SubmIndex& ix, int64_t b, int64_t x, int64_t y, int64_t z,
                                                const int32_t* off_s, int K, Emit&& emit) {
  subm_lookup<G>(ix, b, K,
              [&](int k, int64_t& qx, int64_t& qy, int64_t& qz) {
                qx = x - off_s[3 * k];
                qy = y - off_s[3 * k + 1];
                qz = z - off_s[3 * k + 2];
                return true;
              },
              emit);
}

// Whether every offset component lies in [-1, 1] (uniform scalar loads).
__device__ __forceinline__ bool unit_offsets(const int32_t* __restrict__ offsets, int K) {
  bool unit = true;
  for (int t = 0; t < 3 * K; ++t) unit = unit && offsets[t] >= -1 && offsets[t] <= 1;
  return unit;
}

// The rows of (b, x, y, z) - t_k for unit offsets, k = 0 .. K-1, passed to
// emit(k, row) in ascending k (row -1: outside the box or absent) -- the
// submanifold lookup in 32-bit arithmetic.  One word per axis holds, for
// t = -1, 0, 1, the neighbour coordinate's in-box bit, which of the two bricks
// the row's neighbours span on that axis it lies in, and its position in that
// brick; the up to 8 bricks' level-2 words and bases sit in LDS (bits_s /
// pre_s, 8 x NT per workgroup of NT threads, this thread's column only); offsets are
// uniform scalar loads.  Per offset: three field extracts, an LDS read, a bit
// test and a popcount.  subm_neighbours spends ~95 VALU instructions per
// offset (64-bit coordinates, an 8-way select), which bounded the query.
template <int NT = kSubmThreads, typename Emit>
__device__ __forceinline__ void unit_rows(const SubmIndex& ix, int64_t b, int64_t x, int64_t y, int64_t z,
                                          const int32_t* __restrict__ offsets, int K,
                                          unsigned long long* __restrict__ bits_s, int32_t* __restrict__ pre_s,
                                          Emit&& emit) {
  const int tid = threadIdx.x;
  // a row more than one voxel outside the box has no neighbour in it
  const bool near = b >= 0 && b < ix.nb && x >= -1 && x <= ix.sx && y >= -1 && y <= ix.sy && z >= -1 && z <= ix.sz;
  uint32_t A[3] = {0u, 0u, 0u};
  int bb[3] = {0, 0, 0};
  if (near) {
    const int c3[3] = {(int)x, (int)y, (int)z};
    const int S3[3] = {ix.sx, ix.sy, ix.sz};
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      bb[a] = (c3[a] - 1) >> 2;  // brick of the lowest neighbour coordinate
#pragma unroll
      for (int ti = 0; ti < 3; ++ti) {  // t = ti - 1, neighbour coordinate c - t
        const int q = c3[a] - (ti - 1);
        const uint32_t f = ((q >= 0 && q < S3[a]) ? 8u : 0u) | ((uint32_t)((q >> 2) - bb[a]) << 2) | (uint32_t)(q & 3);
        A[a] |= f << (4 * ti);
      }
    }
  }
  {
    int64_t brk[8];
    bool in[8];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      const int cx = bb[0] + (s8 >> 2), cy = bb[1] + ((s8 >> 1) & 1), cz = bb[2] + (s8 & 1);
      in[s8] = near && cx >= 0 && cx < ix.bx && cy >= 0 && cy < ix.by && cz >= 0 && cz < ix.bz;
      brk[s8] = in[s8] ? ((b * ix.bx + cx) * ix.by + cy) * ix.bz + cz : 0;
    }
    // All 8 level-1 entries, then all 8 level-2 words and bases, in flight
    // together: the loads are unconditional (index 0 for a brick outside the
    // box or unoccupied, its value then dropped), and the table is stored only
    // after the last of them -- a store right after each load waited for it,
    // one round trip per brick.  An index without occupied bricks (cap2 = 0:
    // no level-2 entry to read) leaves every word 0.
    unsigned long long w2[8];
    int32_t p2[8];
    bool occ[8];
    if (ix.cap2 > 0) {  // (uniform)
      SubmL1 e1[8];
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) e1[s8] = ix.l1[in[s8] ? brk[s8] >> 6 : 0];
      int r8[8];
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) {
        occ[s8] = in[s8] && ((e1[s8].bits >> (brk[s8] & 63)) & 1ull);
        r8[s8] = occ[s8] ? subm_brick_rank(e1[s8], brk[s8]) : 0;
      }
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) {
        w2[s8] = ix.l2bits[r8[s8]];
        p2[s8] = ix.l2pre[r8[s8]];
      }
    } else {
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) {
        occ[s8] = false;
        w2[s8] = 0ull;
        p2[s8] = 0;
      }
    }
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      bits_s[s8 * NT + tid] = occ[s8] ? w2[s8] : 0ull;
      pre_s[s8 * NT + tid] = occ[s8] ? p2[s8] : 0;
    }
  }
  for (int k0 = 0; k0 < K; k0 += kSubmGroup) {
    int idx[kSubmGroup];
    // branch-free, so a group's scalar and LDS loads issue together
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) {
      const int k = k0 + j < K ? k0 + j : K - 1;
      const uint32_t fx = (A[0] >> (4 * (offsets[3 * k] + 1))) & 15u;
      const uint32_t fy = (A[1] >> (4 * (offsets[3 * k + 1] + 1))) & 15u;
      const uint32_t fz = (A[2] >> (4 * (offsets[3 * k + 2] + 1))) & 15u;
      const int s8 = (int)((fx & 4u) | ((fy & 4u) >> 1) | ((fz & 4u) >> 2));
      const int vb = (int)(((fx & 3u) << 4) | ((fy & 3u) << 2) | (fz & 3u));
      const unsigned long long w = bits_s[s8 * NT + tid];
      const int base = pre_s[s8 * NT + tid];
      const bool has = (fx & fy & fz & 8u) && ((w >> vb) & 1ull);
      idx[j] = has ? base + (int)__popcll(w & below(vb)) : -1;
    }
    int32_t rr[kSubmGroup];
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) rr[j] = idx[j] >= 0 ? ix.rowmap[idx[j]] : -1;
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j)
      if (k0 + j < K) emit(k0 + j, rr[j]);
  }
}

// Geometry of the index of n rows over [0, batches) x [0, sx) x [0, sy) x [0, sz);
// false when the box cannot be indexed (out of range, or far larger than the set:
// more than 64 bricks a row -- such sets are left to the hash table).
inline bool subm_geom(int64_t n, int64_t batches, int64_t sx, int64_t sy, int64_t sz, int64_t* nbr_out, int64_t* nw1,
                      int64_t* cap2) {
  if (n < 0 || n >= (1ll << 31)) return false;
  if (batches <= 0 || batches > 32768 || sx <= 0 || sy <= 0 || sz <= 0 || sx > 65536 || sy > 65536 || sz > 65536)
    return false;
  const int64_t nbricks = batches * ((sx + 3) / 4) * ((sy + 3) / 4) * ((sz + 3) / 4);
  if (nbricks >= (1ll << 37)) return false;
  *nbr_out = nbricks;
  *nw1 = (nbricks + 63) / 64;
  *cap2 = n < nbricks ? n : nbricks;
  // level-1 scans hold int32 counts of at most n voxels
  return nbricks <= 64 * n + (1 << 22) && *cap2 < (1ll << 31);
}

inline size_t subm_align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace bytes of the index (-1: cannot be indexed).
inline int64_t subm_workspace_bytes(int64_t n, int64_t batches, int64_t sx, int64_t sy, int64_t sz) {
  int64_t nbricks = 0, nw1 = 0, cap2 = 0;
  if (!subm_geom(n, batches, sx, sy, sz, &nbricks, &nw1, &cap2)) return -1;
  const int64_t ntiles = (nw1 + kSubmTile - 1) / kSubmTile;
  return (int64_t)(subm_align256((size_t)nbricks) + subm_align256(sizeof(int32_t) * (size_t)(ntiles + 1)) +
                   subm_align256(sizeof(int32_t) * (size_t)(2 * ntiles)) +
                   subm_align256(sizeof(SubmL1) * (size_t)nw1) +
                   subm_align256(sizeof(unsigned long long) * (size_t)cap2) +
                   subm_align256(sizeof(int32_t) * (size_t)cap2) + subm_align256(sizeof(int32_t) * (size_t)(n > 0 ? n : 1)));
}

// The index's arrays inside `workspace` (a layout subm_workspace_bytes sized); false as subm_geom.
inline bool subm_view(void* workspace, int64_t n, int64_t batches, int64_t sx, int64_t sy, int64_t sz,
                      SubmIndex* ix) {
  *ix = SubmIndex{};
  if (!subm_geom(n, batches, sx, sy, sz, &ix->nbricks, &ix->nw1, &ix->cap2)) return false;
  ix->ntiles = (ix->nw1 + kSubmTile - 1) / kSubmTile;
  ix->nrows = n;
  char* p = (char*)workspace;
  ix->occ = (uint8_t*)p;
  p += subm_align256((size_t)ix->nbricks);
  ix->tile_sums = (int32_t*)p;
  p += subm_align256(sizeof(int32_t) * (size_t)(ix->ntiles + 1));
  ix->tile_pub = (int32_t*)p;
  p += subm_align256(sizeof(int32_t) * (size_t)(2 * ix->ntiles));
  ix->l1 = (SubmL1*)p;
  p += subm_align256(sizeof(SubmL1) * (size_t)ix->nw1);
  ix->l2bits = (unsigned long long*)p;
  p += subm_align256(sizeof(unsigned long long) * (size_t)ix->cap2);
  ix->l2pre = (int32_t*)p;
  p += subm_align256(sizeof(int32_t) * (size_t)ix->cap2);
  ix->rowmap = (int32_t*)p;
  ix->nb = (int)batches;
  ix->sx = (int)sx;
  ix->sy = (int)sy;
  ix->sz = (int)sz;
  ix->bx = (int)((sx + 3) / 4);
  ix->by = (int)((sy + 3) / 4);
  ix->bz = (int)((sz + 3) / 4);
  return true;
}

}  // namespace st
