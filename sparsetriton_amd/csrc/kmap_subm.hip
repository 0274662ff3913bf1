// Submanifold kernel map through a compact brick index of the coordinates
// (conv.py:12-75 for out_coords == in_coords, stride 1, the query bounds equal
// to the index box), with no hash table.
//
// Index (all in the caller's workspace, sized by st_kmap_subm_workspace):
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
// rank = base + popcount below; rowmap[rank].  For config 2 (4 samples of
// 1440 x 1440 x 41, 470k voxels, 112k occupied bricks) the index is ~4 MB
// against the 64 MB of a flat bitmap with a rank prefix over the whole box,
// so the lookups hit L2.
//
// Nine short kernels (a grid-wide sync inside one cooperative kernel costs
// 36-80 us on this chip -- more than a kernel boundary):
//   clear; occupied bricks (a byte each); level-1 words + per-tile brick
//   counts; brick prefix; level-2 bits; per-tile voxel counts; voxel prefix;
//   rowmap (+ repeats, brick bases); the query.
// Level-2 bits are set by non-returning atomics (a brick's word is shared by
// a few rows); counts come from popcounts of the finished words, so no kernel
// waits on an atomic's result and no workgroup waits on another.
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
  int32_t* tile_sums;          // per tile of kSubmTile level-1 entries: its bricks or voxels
  int64_t nbricks, nw1, cap2, ntiles;
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

// brick rank of an in-box coordinate whose brick is occupied
__device__ __forceinline__ int subm_brick_rank(const SubmL1& e, int64_t br) {
  return e.bpre + (int)__popcll(e.bits & below((int)(br & 63)));
}

__global__ __launch_bounds__(kSubmThreads) void subm_clear_kernel(SubmIndex ix, int64_t n, int32_t* status) {
  const int64_t stride = (int64_t)gridDim.x * kSubmThreads;
  const int64_t t = (int64_t)blockIdx.x * kSubmThreads + threadIdx.x;
  if (status && t < ST_STATUS_WORDS) status[t] = 0;
  uint4* occ16 = reinterpret_cast<uint4*>(ix.occ);  // the byte array is padded to 16 bytes
  for (int64_t e = t; e < (ix.nbricks + 15) / 16; e += stride) occ16[e] = make_uint4(0u, 0u, 0u, 0u);
  for (int64_t e = t; e < ix.cap2; e += stride) ix.l2bits[e] = 0ull;
  for (int64_t e = t; e < n; e += stride) ix.rowmap[e] = 0x7FFFFFFF;
}

// Occupied bricks: one plain byte store per row (every writer stores the same
// 1, so no atomic is needed -- atomics on the level-1 words, shared by a
// hundred rows each, serialise).  Rows that do not pack into a key count as
// bad coordinates.
template <typename CT>
__global__ __launch_bounds__(kSubmThreads) void subm_occ_kernel(const CT* __restrict__ coords, int64_t n,
                                                                SubmIndex ix, int32_t* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * kSubmThreads + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  uint64_t key;
  if (status && !pack_key(b, x, y, z, key)) atomicAdd(&status[ST_STATUS_BAD_COORD], 1);
  if (subm_in_box(ix, b, x, y, z)) ix.occ[subm_brick(ix, b, x, y, z)] = 1;
}

// Bricks (BRICKS) or distinct voxels of level-1 entry e; the voxels of an
// entry are the popcounts of its bricks' level-2 words.
template <bool BRICKS>
__device__ __forceinline__ int subm_entry_count(const SubmIndex& ix, int64_t e) {
  const SubmL1 v = ix.l1[e];
  const int nb = (int)__popcll(v.bits);
  if (BRICKS) return nb;
  int c = 0;
  for (int j = 0; j < nb; ++j) c += (int)__popcll(ix.l2bits[v.bpre + j]);
  return c;
}

// tile_sums[t] = bricks (or voxels) of tile t's level-1 entries (one per thread)
template <bool BRICKS>
__global__ __launch_bounds__(kSubmThreads) void subm_tile_sum_kernel(SubmIndex ix) {
  __shared__ int red_s[4];
  const int tid = threadIdx.x;
  const int64_t e = (int64_t)blockIdx.x * kSubmTile + tid;
  if (BRICKS && e < ix.nw1) {
    // level-1 word e from the 64 occupancy bytes of its bricks (the array is padded to 16 bytes,
    // bytes past the last brick are zero)
    const uint4* src = reinterpret_cast<const uint4*>(ix.occ + e * 64);
    unsigned long long bits = 0ull;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (e * 64 + q * 16 >= ix.nbricks) break;
      const uint4 v = src[q];
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int bb = 0; bb < 4; ++bb)
          if ((wv[j] >> (8 * bb)) & 0xFFu) bits |= 1ull << (q * 16 + j * 4 + bb);
    }
    ix.l1[e].bits = bits;
  }
  int c = e < ix.nw1 ? subm_entry_count<BRICKS>(ix, e) : 0;
  c = wave_sum(c);
  if ((tid & 63) == 0) red_s[tid >> 6] = c;
  __syncthreads();
  if (tid == 0) ix.tile_sums[blockIdx.x] = red_s[0] + red_s[1] + red_s[2] + red_s[3];
}

// Exclusive prefix over the level-1 entries of tile blockIdx.x (one per
// thread): the sums of the tiles before it, then a scan of the tile's own
// per-entry counts, written to .bpre (BRICKS) or .v (voxels before the entry).
template <bool BRICKS>
__global__ __launch_bounds__(kSubmThreads) void subm_prefix_kernel(SubmIndex ix) {
  __shared__ int red_s[4];
  __shared__ int scan_s[8];
  const int tid = threadIdx.x, t = blockIdx.x;
  int off = 0;
  for (int j = tid; j < t; j += kSubmThreads) off += ix.tile_sums[j];
  off = wave_sum(off);
  if ((tid & 63) == 0) red_s[tid >> 6] = off;
  __syncthreads();
  off = red_s[0] + red_s[1] + red_s[2] + red_s[3];
  const int64_t e = (int64_t)t * kSubmTile + tid;
  const int c = e < ix.nw1 ? subm_entry_count<BRICKS>(ix, e) : 0;
  int total;
  const int p = off + block_exclusive_scan(c, scan_s, &total);
  if (e < ix.nw1) {
    if (BRICKS)
      ix.l1[e].bpre = p;
    else
      ix.l1[e].v = p;
  }
}

// Level-2 bits at the row's brick rank (one non-returning atomic per row: a
// level-2 word is one brick, shared by a few rows only).
template <typename CT>
__global__ __launch_bounds__(kSubmThreads) void subm_l2_kernel(const CT* __restrict__ coords, int64_t n,
                                                               SubmIndex ix) {
  const int64_t i = (int64_t)blockIdx.x * kSubmThreads + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  if (!subm_in_box(ix, b, x, y, z)) return;
  const int64_t br = subm_brick(ix, b, x, y, z);
  const int r = subm_brick_rank(ix.l1[br >> 6], br);
  __hip_atomic_fetch_or(&ix.l2bits[r], 1ull << subm_vbit(x, y, z), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Voxel rank of every row -> rowmap (lowest row of a repeated voxel); the row
// holding its brick's lowest voxel stores the brick's voxel base; rows
// repeating a coordinate count as duplicates.
template <typename CT>
__global__ __launch_bounds__(kSubmThreads) void subm_rowmap_kernel(const CT* __restrict__ coords, int64_t n,
                                                                   SubmIndex ix, int32_t* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * kSubmThreads + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  if (!subm_in_box(ix, b, x, y, z)) return;
  const int64_t br = subm_brick(ix, b, x, y, z);
  const SubmL1 e = ix.l1[br >> 6];
  const int r0 = e.bpre, r = subm_brick_rank(e, br);
  int base = e.v;  // voxels before the level-1 entry, then before the brick
  for (int j = r0; j < r; ++j) base += (int)__popcll(ix.l2bits[j]);
  const unsigned long long bits = ix.l2bits[r];
  const int vb = subm_vbit(x, y, z);
  if (!(bits & below(vb))) ix.l2pre[r] = base;
  // every row but the first to reach a voxel repeats its coordinate
  const int32_t prev = atomicMin(&ix.rowmap[base + (int)__popcll(bits & below(vb))], (int32_t)i);
  if (prev != 0x7FFFFFFF && status) atomicAdd(&status[ST_STATUS_DUPLICATE], 1);
}

// nbr[k * n + o] = row of coords[o] - t_k (in the box, present), -1 otherwise;
// kSubmGroup lookups in flight per row, each three dependent loads (level-1
// entry; level-2 bits and base; rowmap), all L2-resident.
template <typename CT>
__global__ __launch_bounds__(kSubmThreads) void subm_query_kernel(const CT* __restrict__ coords, int64_t n,
                                                                  const int32_t* __restrict__ offsets, int K,
                                                                  SubmIndex ix, int32_t* __restrict__ nbr,
                                                                  uint32_t* __restrict__ row_masks,
                                                                  int32_t* __restrict__ status) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  for (int t = threadIdx.x; t < K * 3; t += kSubmThreads) off_s[t] = offsets[t];
  __syncthreads();
  // offsets all within one voxel of the row (the 3x3x3 kernel): the row's neighbours lie in the
  // at most 2 x 2 x 2 bricks around it, each looked up once
  __shared__ int unit_s;
  if (threadIdx.x == 0) unit_s = 1;
  __syncthreads();
  for (int t = threadIdx.x; t < K * 3; t += kSubmThreads)
    if (off_s[t] < -1 || off_s[t] > 1) unit_s = 0;
  __syncthreads();
  const bool unit = unit_s != 0;
  const int64_t o = (int64_t)blockIdx.x * kSubmThreads + threadIdx.x;
  if (o >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, o, b, x, y, z);
  if (status && !(x >= 0 && x < ix.sx && y >= 0 && y < ix.sy && z >= 0 && z < ix.sz))
    atomicAdd(&status[ST_STATUS_OUT_OF_BOX], 1);
  const int W = (K + 31) >> 5;
  uint32_t mword = 0;
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
      for (int j = 0; j < kSubmGroup; ++j) {
        const int k = k0 + j;
        if (k < K) {
          nbr[(int64_t)k * n + o] = rr[j];
          if (rr[j] >= 0) mword |= 1u << (k & 31);
          if ((k & 31) == 31 || k == K - 1) {
            if (row_masks) row_masks[o * W + (k >> 5)] = mword;
            mword = 0;
          }
        }
      }
    }
    return;
  }
  for (int k0 = 0; k0 < K; k0 += kSubmGroup) {
    int64_t brk[kSubmGroup];
    int vb[kSubmGroup];
    bool in[kSubmGroup];
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) {
      const int k = k0 + j;
      in[j] = false;
      brk[j] = 0;
      vb[j] = 0;
      if (k < K) {
        const int64_t qx = x - off_s[3 * k], qy = y - off_s[3 * k + 1], qz = z - off_s[3 * k + 2];
        if (subm_in_box(ix, b, qx, qy, qz)) {
          in[j] = true;
          brk[j] = subm_brick(ix, b, qx, qy, qz);
          vb[j] = subm_vbit(qx, qy, qz);
        }
      }
    }
    SubmL1 e1[kSubmGroup];
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) e1[j] = in[j] ? ix.l1[brk[j] >> 6] : SubmL1{0ull, 0, 0};
    unsigned long long bits[kSubmGroup];
    int32_t pre[kSubmGroup];
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) {
      in[j] = in[j] && ((e1[j].bits >> (brk[j] & 63)) & 1ull);
      const int r = in[j] ? subm_brick_rank(e1[j], brk[j]) : 0;
      bits[j] = in[j] ? ix.l2bits[r] : 0ull;
      pre[j] = in[j] ? ix.l2pre[r] : 0;
    }
    int32_t rr[kSubmGroup];
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) {
      const bool has = in[j] && ((bits[j] >> vb[j]) & 1ull);
      rr[j] = has ? ix.rowmap[pre[j] + (int)__popcll(bits[j] & below(vb[j]))] : -1;
    }
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) {
      const int k = k0 + j;
      if (k < K) {
        nbr[(int64_t)k * n + o] = rr[j];
        if (rr[j] >= 0) mword |= 1u << (k & 31);
        if ((k & 31) == 31 || k == K - 1) {
          if (row_masks) row_masks[o * W + (k >> 5)] = mword;
          mword = 0;
        }
      }
    }
  }
}

static bool subm_geom(int64_t n, int64_t batches, int64_t sx, int64_t sy, int64_t sz, int64_t* nbr_out,
                      int64_t* nw1, int64_t* cap2) {
  if (batches <= 0 || batches > 32768 || sx <= 0 || sy <= 0 || sz <= 0 || sx > 65536 || sy > 65536 || sz > 65536)
    return false;
  const int64_t nbricks = batches * ((sx + 3) / 4) * ((sy + 3) / 4) * ((sz + 3) / 4);
  if (nbricks >= (1ll << 37)) return false;
  *nbr_out = nbricks;
  *nw1 = (nbricks + 63) / 64;
  *cap2 = n < nbricks ? n : nbricks;
  // a box far larger than the set (more than 64 bricks a row) is left to the hash table;
  // level-1 scans hold int32 counts of at most n voxels
  return nbricks <= 64 * n + (1 << 22) && *cap2 < (1ll << 31);
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace st

using namespace st;

extern "C" {

int st_kmap_subm_workspace(int64_t n, int64_t batches, int64_t sx, int64_t sy, int64_t sz, int64_t* bytes) {
  int64_t nbricks = 0, nw1 = 0, cap2 = 0;
  if (!bytes || n < 0 || n >= (1ll << 31) || !subm_geom(n, batches, sx, sy, sz, &nbricks, &nw1, &cap2))
    return ST_ERR_ARG;
  const int64_t ntiles = (nw1 + kSubmTile - 1) / kSubmTile;
  *bytes = (int64_t)(align256((size_t)nbricks) + align256(sizeof(int32_t) * (size_t)ntiles) +
                     align256(sizeof(SubmL1) * (size_t)nw1) +
                     align256(sizeof(unsigned long long) * (size_t)cap2) + align256(sizeof(int32_t) * (size_t)cap2) +
                     align256(sizeof(int32_t) * (size_t)(n > 0 ? n : 1)));
  return ST_OK;
}

int st_kmap_subm(const void* coords, int coord_dtype, int64_t n, const int32_t* offsets, int K, int64_t batches,
                 int64_t sx, int64_t sy, int64_t sz, void* workspace, int64_t workspace_bytes, int32_t* nbr,
                 uint32_t* row_masks, int32_t* status, st_stream_t stream) {
  int64_t need = 0;
  if (st_kmap_subm_workspace(n, batches, sx, sy, sz, &need) != ST_OK) return ST_ERR_ARG;
  if (K <= 0 || K > ST_MAX_KVOL || workspace_bytes < need) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!coords || !offsets || !workspace || !nbr) return ST_ERR_ARG;
  SubmIndex ix{};
  subm_geom(n, batches, sx, sy, sz, &ix.nbricks, &ix.nw1, &ix.cap2);
  ix.ntiles = (ix.nw1 + kSubmTile - 1) / kSubmTile;
  char* p = (char*)workspace;
  ix.occ = (uint8_t*)p;
  p += align256((size_t)ix.nbricks);
  ix.tile_sums = (int32_t*)p;
  p += align256(sizeof(int32_t) * (size_t)ix.ntiles);
  ix.l1 = (SubmL1*)p;
  p += align256(sizeof(SubmL1) * (size_t)ix.nw1);
  ix.l2bits = (unsigned long long*)p;
  p += align256(sizeof(unsigned long long) * (size_t)ix.cap2);
  ix.l2pre = (int32_t*)p;
  p += align256(sizeof(int32_t) * (size_t)ix.cap2);
  ix.rowmap = (int32_t*)p;
  ix.nb = (int)batches;
  ix.sx = (int)sx;
  ix.sy = (int)sy;
  ix.sz = (int)sz;
  ix.bx = (int)((sx + 3) / 4);
  ix.by = (int)((sy + 3) / 4);
  ix.bz = (int)((sz + 3) / 4);
  const unsigned rows = st_blocks(n, kSubmThreads);
  int64_t clear_items = ix.cap2 > n ? ix.cap2 : n;
  if ((ix.nbricks + 15) / 16 > clear_items) clear_items = (ix.nbricks + 15) / 16;
  unsigned cg = st_blocks(clear_items, kSubmThreads);
  if (cg > 4096) cg = 4096;
  subm_clear_kernel<<<cg, kSubmThreads, 0, stream>>>(ix, n, status);
  ST_DISPATCH_COORD(coord_dtype, CT, {
    const CT* c = (const CT*)coords;
    subm_occ_kernel<CT><<<rows, kSubmThreads, 0, stream>>>(c, n, ix, status);
    subm_tile_sum_kernel<true><<<(unsigned)ix.ntiles, kSubmThreads, 0, stream>>>(ix);
    subm_prefix_kernel<true><<<(unsigned)ix.ntiles, kSubmThreads, 0, stream>>>(ix);
    subm_l2_kernel<CT><<<rows, kSubmThreads, 0, stream>>>(c, n, ix);
    subm_tile_sum_kernel<false><<<(unsigned)ix.ntiles, kSubmThreads, 0, stream>>>(ix);
    subm_prefix_kernel<false><<<(unsigned)ix.ntiles, kSubmThreads, 0, stream>>>(ix);
    subm_rowmap_kernel<CT><<<rows, kSubmThreads, 0, stream>>>(c, n, ix, status);
    subm_query_kernel<CT><<<rows, kSubmThreads, 0, stream>>>(c, n, offsets, K, ix, nbr, row_masks, status);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // extern "C"
