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

// Whether every offset component (off_s: K x 3) lies in [-1, 1].
__device__ __forceinline__ bool subm_unit_offsets(const int32_t* off_s, int K) {
  bool unit = true;
  for (int t = 0; t < 3 * K; ++t) unit = unit && off_s[t] >= -1 && off_s[t] <= 1;
  return unit;
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
// in ascending k (row -1: outside the box or absent).  kSubmGroup lookups are
// in flight at a time, each three dependent loads (level-1 entry; level-2
// bits and base; rowmap), all L2-resident.  With unit offsets (the 3x3x3
// kernel) the neighbours lie in the at most 2 x 2 x 2 bricks around the row,
// each looked up once.
template <int G = kSubmGroup, typename Emit>
__device__ __forceinline__ void subm_neighbours(const SubmIndex& ix, int64_t b, int64_t x, int64_t y, int64_t z,
                                                const int32_t* off_s, int K, bool unit, Emit&& emit) {
  if (unit) {
    // bricks [bx + lo, bx + hi] per axis, lo = -1 when the row sits on the brick's low face
    const int64_t bx = x >> 2, by = y >> 2, bz = z >> 2;
    const int lx = (x & 3) == 0 ? -1 : 0, ly = (y & 3) == 0 ? -1 : 0, lz = (z & 3) == 0 ? -1 : 0;
    const int hx = (x & 3) == 3 ? 1 : 0, hy = (y & 3) == 3 ? 1 : 0, hz = (z & 3) == 3 ? 1 : 0;
    int64_t brk[8];
    bool in[8];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      const int dx = lx + (s8 >> 2), dy = ly + ((s8 >> 1) & 1), dz = lz + (s8 & 1);
      const int64_t cx = bx + dx, cy = by + dy, cz = bz + dz;
      in[s8] = dx <= hx && dy <= hy && dz <= hz && b >= 0 && b < ix.nb && cx >= 0 && cx < ix.bx && cy >= 0 &&
               cy < ix.by && cz >= 0 && cz < ix.bz;
      brk[s8] = in[s8] ? ((b * ix.bx + cx) * ix.by + cy) * ix.bz + cz : 0;
    }
    SubmL1 e1[8];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) e1[s8] = in[s8] ? ix.l1[brk[s8] >> 6] : SubmL1{0ull, 0, 0};
    unsigned long long bits[8];
    int32_t pre[8];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      const bool occ = in[s8] && ((e1[s8].bits >> (brk[s8] & 63)) & 1ull);
      const int r = occ ? subm_brick_rank(e1[s8], brk[s8]) : 0;
      bits[s8] = occ ? ix.l2bits[r] : 0ull;
      pre[s8] = occ ? ix.l2pre[r] : 0;
    }
    for (int k0 = 0; k0 < K; k0 += kSubmGroup) {
      int32_t rr[kSubmGroup];
#pragma unroll
      for (int j = 0; j < kSubmGroup; ++j) {
        const int k = k0 + j;
        rr[j] = -1;
        if (k < K) {
          const int64_t qx = x - off_s[3 * k], qy = y - off_s[3 * k + 1], qz = z - off_s[3 * k + 2];
          if (subm_in_box(ix, b, qx, qy, qz)) {
            const int s8 = ((int)((qx >> 2) - bx - lx) << 2) | ((int)((qy >> 2) - by - ly) << 1) |
                           (int)((qz >> 2) - bz - lz);
            unsigned long long w = 0ull;
            int p = 0;
#pragma unroll
            for (int t8 = 0; t8 < 8; ++t8) {
              w = s8 == t8 ? bits[t8] : w;
              p = s8 == t8 ? pre[t8] : p;
            }
            const int vb = subm_vbit(qx, qy, qz);
            if ((w >> vb) & 1ull) rr[j] = ix.rowmap[p + (int)__popcll(w & below(vb))];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kSubmGroup; ++j)
        if (k0 + j < K) emit(k0 + j, rr[j]);
    }
    return;
  }
  subm_lookup<G>(ix, b, K,
              [&](int k, int64_t& qx, int64_t& qy, int64_t& qz) {
                qx = x - off_s[3 * k];
                qy = y - off_s[3 * k + 1];
                qz = z - off_s[3 * k + 2];
                return true;
              },
              emit);
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
