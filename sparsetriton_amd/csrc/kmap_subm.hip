// Submanifold kernel map through a compact brick index of the coordinates
// (conv.py:12-75 for out_coords == in_coords, stride 1, the query bounds equal
// to the index box), with no hash table.  The index layout and its lookup are
// in subm_index.h.  For config 2 (4 samples of 1440 x 1440 x 41, 470k voxels,
// 112k occupied bricks) the index is ~4 MB against the 64 MB of a flat bitmap
// with a rank prefix over the whole box, so the lookups hit L2.
//
// Eight short kernels build the index (a grid-wide sync inside one
// cooperative kernel costs 36-80 us on this chip -- more than a kernel
// boundary):
//   clear; occupied bricks (a byte each); level-1 words + per-tile brick
//   counts; brick prefix (+ clearing the occupied bricks' level-2 words);
//   level-2 bits; per-tile voxel counts; voxel prefix (+ brick voxel bases);
//   rowmap (+ repeats); then the query writes the map.
// Level-2 bits are set by non-returning atomics (a brick's word is shared by
// a few rows); counts come from popcounts of the finished words, so no kernel
// waits on an atomic's result and no workgroup waits on another.
#include "outgeom.h"
#include "subm_index.h"

namespace st {

__global__ __launch_bounds__(kSubmThreads) void subm_clear_kernel(SubmIndex ix, int64_t n, int32_t* status) {
  const int64_t stride = (int64_t)gridDim.x * kSubmThreads;
  const int64_t t = (int64_t)blockIdx.x * kSubmThreads + threadIdx.x;
  if (status && t < ST_STATUS_WORDS) status[t] = 0;
  if (ix.flag && t == 0) *ix.flag = 0;
  uint4* occ16 = reinterpret_cast<uint4*>(ix.occ);  // the byte array is padded to 16 bytes
  for (int64_t e = t; e < (ix.nbricks + 15) / 16; e += stride) occ16[e] = make_uint4(0u, 0u, 0u, 0u);
  for (int64_t e = t; e < 2 * ix.ntiles; e += stride) ix.tile_pub[e] = 0;
  for (int64_t e = t; e < n; e += stride) ix.rowmap[e] = 0x7FFFFFFF;
}

// Occupied bricks: one plain byte store per row (every writer stores the same
// 1, so no atomic is needed -- atomics on the level-1 words, shared by a
// hundred rows each, serialise).  Rows that do not pack into a key count as
// bad coordinates, rows outside [0, shape) as out of the box.
template <typename CT>
__global__ __launch_bounds__(kSubmThreads) void subm_occ_kernel(const CT* __restrict__ coords, int64_t n,
                                                                SubmIndex ix, int32_t* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * kSubmThreads + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  uint64_t key;
  if (status && !pack_key(b, x, y, z, key)) atomicAdd(&status[ST_STATUS_BAD_COORD], 1);
  if (status && !(x >= 0 && x < ix.sx && y >= 0 && y < ix.sy && z >= 0 && z < ix.sz))
    atomicAdd(&status[ST_STATUS_OUT_OF_BOX], 1);
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

// Level-1 word e from the 64 occupancy bytes of its bricks (the array is padded
// to 16 bytes, bytes past the last brick are zero).
__device__ __forceinline__ unsigned long long subm_occ_bits(const SubmIndex& ix, int64_t e) {
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
  return bits;
}

// tile_sums[t] = bricks (or voxels) of tile t's level-1 entries (one per thread)
template <bool BRICKS>
__global__ __launch_bounds__(kSubmThreads) void subm_tile_sum_kernel(SubmIndex ix) {
  __shared__ int red_s[4];
  if (!BRICKS && subm_overflowed(ix)) return;
  const int tid = threadIdx.x;
  const int64_t e = (int64_t)blockIdx.x * kSubmTile + tid;
  if (BRICKS && e < ix.nw1) ix.l1[e].bits = subm_occ_bits(ix, e);
  int c = e < ix.nw1 ? subm_entry_count<BRICKS>(ix, e) : 0;
  c = wave_sum(c);
  if ((tid & 63) == 0) red_s[tid >> 6] = c;
  __syncthreads();
  if (tid == 0) ix.tile_sums[blockIdx.x] = red_s[0] + red_s[1] + red_s[2] + red_s[3];
}

// Exclusive prefix over the level-1 entries of tile blockIdx.x (one per
// thread): the sums of the tiles before it, then a scan of the tile's own
// per-entry counts, written to .bpre (BRICKS) or .v (voxels before the entry).
// BRICKS also clears the level-2 words of the entry's bricks (so only the
// words in use are cleared); voxels also write each of the entry's bricks'
// voxel base (l2pre) and, for the last entry, the distinct voxels in all to
// *voxels (optional).  An index with an overflow flag (SubmIndex::flag) sets
// it when the bricks exceed cap2 (no level-2 word past cap2 is written) or the
// voxels exceed nrows (*voxels is then 0); the voxel pass of an overflowed
// index returns at once.
// The tiles' offsets: with `scanned` the tile sums were replaced by their
// exclusive scan; otherwise each workgroup sums the tiles before its own.
// (launch_subm_level takes this kernel only above kSubmInlineTiles tiles, with
// the scan; below, subm_level_kernel does a level in one launch.)
template <bool BRICKS>
__device__ __forceinline__ void subm_entry_write(const SubmIndex& ix, int64_t e, int p, int32_t* __restrict__ voxels) {
  if (e >= ix.nw1) return;
  const SubmL1 v = ix.l1[e];
  const int nb = (int)__popcll(v.bits);
  if (BRICKS) {
    ix.l1[e].bpre = p;
    for (int j = 0; j < nb && p + j < ix.cap2; ++j) ix.l2bits[p + j] = 0ull;
    if ((int64_t)p + nb > ix.cap2 && ix.flag) atomicOr(ix.flag, 1);
  } else {
    ix.l1[e].v = p;
    int64_t q = p;
    for (int j = 0; j < nb; ++j) {
      ix.l2pre[v.bpre + j] = (int32_t)q;
      q += (int)__popcll(ix.l2bits[v.bpre + j]);
    }
    const bool over = q > ix.nrows && ix.flag;
    if (over) atomicOr(ix.flag, 1);
    if (voxels && e == ix.nw1 - 1) *voxels = over ? 0 : (int32_t)q;
  }
}

template <bool BRICKS>
__global__ __launch_bounds__(kSubmThreads) void subm_prefix_kernel(SubmIndex ix, int32_t* __restrict__ voxels,
                                                                   bool scanned) {
  __shared__ int red_s[4];
  __shared__ int scan_s[8];
  if (!BRICKS && subm_overflowed(ix)) return;
  const int tid = threadIdx.x, t = blockIdx.x;
  int off = 0;
  if (scanned) {
    off = ix.tile_sums[t];
  } else {
    for (int j = tid; j < t; j += kSubmThreads) off += ix.tile_sums[j];
    off = wave_sum(off);
    if ((tid & 63) == 0) red_s[tid >> 6] = off;
    __syncthreads();
    off = red_s[0] + red_s[1] + red_s[2] + red_s[3];
  }
  const int64_t e = (int64_t)t * kSubmTile + tid;
  const int c = e < ix.nw1 ? subm_entry_count<BRICKS>(ix, e) : 0;
  int total;
  const int p = off + block_exclusive_scan(c, scan_s, &total);
  subm_entry_write<BRICKS>(ix, e, p, voxels);
}

// Both passes of a level in one launch for indexes of at most kSubmInlineTiles
// tiles: each workgroup counts its tile's entries (BRICKS: building their
// level-1 words first), publishes the tile's total in tile_pub (flag bit 31,
// cleared by subm_clear_kernel), then adds the totals of the tiles before its
// own.  Workgroups are dispatched in index order, so every earlier tile is
// running or done and publishes within microseconds; a total still missing
// after `spin` polls is computed from the index directly (subm_tile_total),
// so the wait is bounded and the result exact either way.
constexpr int32_t kPubFlag = (int32_t)0x80000000u;

// Bricks (from the occupancy bytes: the tile's level-1 words may not be built
// yet) or voxels of tile j, summed by one thread.
template <bool BRICKS>
__device__ int subm_tile_total(const SubmIndex& ix, int64_t j) {
  int s = 0;
  const int64_t e1 = min((j + 1) * (int64_t)kSubmTile, ix.nw1);
  for (int64_t e = j * kSubmTile; e < e1; ++e) {
    if (BRICKS)
      s += (int)__popcll(subm_occ_bits(ix, e));
    else
      s += subm_entry_count<false>(ix, e);
  }
  return s;
}

template <bool BRICKS>
__global__ __launch_bounds__(kSubmThreads) void subm_level_kernel(SubmIndex ix, int32_t* __restrict__ voxels,
                                                                  int spin) {
  __shared__ int red_s[4];
  __shared__ int scan_s[8];
  if (!BRICKS && subm_overflowed(ix)) return;
  const int tid = threadIdx.x;
  const int64_t t = blockIdx.x;
  const int64_t e = t * kSubmTile + tid;
  if (BRICKS && e < ix.nw1) ix.l1[e].bits = subm_occ_bits(ix, e);
  const int c = e < ix.nw1 ? subm_entry_count<BRICKS>(ix, e) : 0;
  int total;
  const int local = block_exclusive_scan(c, scan_s, &total);
  int32_t* pub = ix.tile_pub + (BRICKS ? 0 : ix.ntiles);
  if (tid == 0) __hip_atomic_store(&pub[t], total | kPubFlag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int off = 0;
  for (int64_t j = tid; j < t; j += kSubmThreads) {
    int v = __hip_atomic_load(&pub[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int s = 0; !(v & kPubFlag) && s < spin; ++s) {
      __builtin_amdgcn_s_sleep(2);
      v = __hip_atomic_load(&pub[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    off += (v & kPubFlag) ? (v & ~kPubFlag) : subm_tile_total<BRICKS>(ix, j);
  }
  off = wave_sum(off);
  if ((tid & 63) == 0) red_s[tid >> 6] = off;
  __syncthreads();
  off = red_s[0] + red_s[1] + red_s[2] + red_s[3];
  subm_entry_write<BRICKS>(ix, e, off + local, voxels);
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

// Voxel rank of every row -> rowmap (lowest row of a repeated voxel); rows
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
  const int r = subm_brick_rank(ix.l1[br >> 6], br);
  const unsigned long long bits = ix.l2bits[r];
  const int vb = subm_vbit(x, y, z);
  // every row but the first to reach a voxel repeats its coordinate
  const int32_t prev = atomicMin(&ix.rowmap[ix.l2pre[r] + (int)__popcll(bits & below(vb))], (int32_t)i);
  if (prev != 0x7FFFFFFF && status) atomicAdd(&status[ST_STATUS_DUPLICATE], 1);
}

// LDS of a query workgroup: the unit path's brick words and bases, or the
// general path's offsets (NONE: a kernel that uses neither).
template <bool NONE = false>
struct QueryLds {
  unsigned long long bits[NONE ? 1 : 8 * kSubmThreads];
  int32_t pre[NONE ? 1 : 8 * kSubmThreads];
};
static_assert(sizeof(QueryLds<>) >= sizeof(int32_t) * ST_MAX_KVOL * 3, "offsets fit the query's LDS");

// nbr[k * n + o] = row of coords[o] - t_k (in the box, present), -1 otherwise,
// and the row's mask words (NBR = false: the mask words only).
template <typename CT, bool NBR>
__global__ __launch_bounds__(kSubmThreads) void subm_query_kernel(const CT* __restrict__ coords, int64_t n,
                                                                  const int32_t* __restrict__ offsets, int K,
                                                                  SubmIndex ix, int32_t* __restrict__ nbr,
                                                                  uint32_t* __restrict__ row_masks) {
  __shared__ QueryLds<> lds;
  const bool unit = unit_offsets(offsets, K);
  int32_t* off_s = reinterpret_cast<int32_t*>(&lds);
  if (!unit) {
    for (int t = threadIdx.x; t < K * 3; t += kSubmThreads) off_s[t] = offsets[t];
    __syncthreads();
  }
  const int64_t o = (int64_t)blockIdx.x * kSubmThreads + threadIdx.x;
  if (o >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, o, b, x, y, z);
  const int W = (K + 31) >> 5;
  uint32_t mword = 0;
  auto emit = [&](int k, int32_t v) {
    if constexpr (NBR) nbr[(int64_t)k * n + o] = v;
    if (v >= 0) mword |= 1u << (k & 31);
    if ((k & 31) == 31 || k == K - 1) {
      if (row_masks) row_masks[o * W + (k >> 5)] = mword;
      mword = 0;
    }
  };
  if (unit)
    unit_rows(ix, b, x, y, z, offsets, K, lds.bits, lds.pre, emit);
  else  // (small lookup groups: this path's registers set the kernel's occupancy)
    subm_neighbours<3>(ix, b, x, y, z, off_s, K, emit);
}

// ------------------------------------- strided / transposed output coordinates
//
// The candidates (input row i, offset k) of a strided or transposed
// convolution (outgeom.h) are deduplicated through a brick index of the
// OUTPUT box built from the candidates themselves, instead of a hash table:
// occupied bricks, level-2 bits and voxel prefix as for a coordinate set, then
// for each distinct output voxel the lowest candidate rank reaching it (an
// atomic min into the index's rowmap array).  A candidate is its coordinate's
// first occurrence when its rank is that minimum, so the outputs come out in
// the hash build's order (first occurrence in the reference's enumeration,
// kmap.py:270-278).  One thread per candidate rank: the output rows of a block
// of 256 ranks follow from a workgroup scan.  All index arrays but the ranks
// stay L2/MALL-sized (config 4: 14.2M candidates, 7.1M outputs, 5.7M bricks
// in the box).  The kernel map is then a query of each output row in the
// input coordinates' brick index (conv.py:54-59, 180-188).

// n / d for n < 2^32 as the high half of n * m, m = ceil(2^64 / d) (0 for
// d = 1): the error n * (m - 2^64 / d) / 2^64 stays below 1 - (n mod d) / d,
// so the quotient is exact.  Two integer multiplies instead of a division.
inline uint64_t fastdiv_magic(uint64_t d) { return d <= 1 ? 0ull : ~0ull / d + 1ull; }
__device__ __forceinline__ uint32_t fastdiv(uint32_t n, uint64_t m) {
  return m ? (uint32_t)__umul64hi((uint64_t)n, m) : n;
}

// Candidate ranks: n input rows, chunk offsets per chunk, ranks per chunk n * chunk.
struct Ranks {
  uint32_t n, nranks, chunk, per;
  uint64_t chunk_m, per_m;  // fastdiv_magic of chunk and per
};

inline Ranks make_ranks(const Geom& g, int64_t n, int64_t nranks) {
  Ranks r;
  r.n = (uint32_t)n;
  r.nranks = (uint32_t)nranks;
  r.chunk = (uint32_t)g.chunk;
  r.per = (uint32_t)(n * g.chunk);
  r.chunk_m = fastdiv_magic(r.chunk);
  r.per_m = fastdiv_magic(r.per);
  return r;
}

// Candidate of rank t: input row i and offset k (false past a partial last
// chunk's offsets).  Ranks are below 2^32 (checked by the caller).
__device__ __forceinline__ bool ocb_rank_cand(const Geom& g, const Ranks& rk, uint32_t t, uint32_t& i, int& k) {
  const uint32_t c = fastdiv(t, rk.per_m), r = t - c * rk.per;
  i = fastdiv(r, rk.chunk_m);
  k = (int)(c * rk.chunk + (r - i * rk.chunk));
  return k < g.K;
}

// Output coordinate of candidate rank t; false when there is none or the
// stride / range filters drop it.
template <typename CT>
__device__ __forceinline__ bool ocb_cand(const CT* __restrict__ coords, const Ranks& rk, const int32_t* off_s,
                                         const Geom& g, uint32_t t, int64_t& b, int64_t& ox, int64_t& oy,
                                         int64_t& oz) {
  uint32_t i;
  int k;
  if (t >= rk.nranks || !ocb_rank_cand(g, rk, t, i, k)) return false;
  int64_t x, y, z;
  load_coord(coords, (int64_t)i, b, x, y, z);
  return candidate(g, x, y, z, off_s[3 * k], off_s[3 * k + 1], off_s[3 * k + 2], ox, oy, oz);
}

// Voxel rank of an output coordinate inside the box whose voxel bit is set.
__device__ __forceinline__ int ocb_voxel(const SubmIndex& ox, int64_t b, int64_t x, int64_t y, int64_t z) {
  const int64_t br = subm_brick(ox, b, x, y, z);
  const int r = subm_brick_rank(ox.l1[br >> 6], br);
  return ox.l2pre[r] + (int)__popcll(ox.l2bits[r] & below(subm_vbit(x, y, z)));
}

// Occupied output bricks (plain byte stores); candidates whose batch index
// lies outside the box count into OUT_OF_BOX (the caller then falls back to
// the hash build: the index cannot hold them).
template <typename CT>
__global__ __launch_bounds__(256) void ocb_occ_kernel(const CT* __restrict__ coords, Ranks rk,
                                                      const int32_t* __restrict__ offsets, Geom g, SubmIndex ox,
                                                      int32_t* __restrict__ status) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  load_offsets(off_s, offsets, g.K);
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  int64_t b, x, y, z;
  if (!ocb_cand(coords, rk, off_s, g, t, b, x, y, z)) return;
  if (b >= 0 && b < ox.nb)
    ox.occ[subm_brick(ox, b, x, y, z)] = 1;
  else
    atomicAdd(&status[ST_STATUS_OUT_OF_BOX], 1);
}

// Level-2 voxel bits: the workgroup's candidates (256 consecutive ranks, a
// few inputs' neighbourhoods) combine their bits per brick in an LDS table
// first, then one non-returning global atomic OR per distinct brick.  One
// global atomic per candidate took 596 us on config 4 (atomics on one word
// serialise), a wave-wide OR per distinct brick 217 us.
constexpr int kL2Slots = 512;  // >= 2 x the workgroup's candidates: probing ends
template <typename CT>
__global__ __launch_bounds__(256) void ocb_l2_kernel(const CT* __restrict__ coords, Ranks rk,
                                                     const int32_t* __restrict__ offsets, Geom g, SubmIndex ox) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  __shared__ int32_t key_s[kL2Slots];
  __shared__ unsigned long long bits_s[kL2Slots];
  if (subm_overflowed(ox)) return;  // more occupied bricks than level-2 words
  for (int e = threadIdx.x; e < kL2Slots; e += 256) {
    key_s[e] = -1;
    bits_s[e] = 0ull;
  }
  load_offsets(off_s, offsets, g.K);  // (its barrier also orders the table's clearing)
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  int64_t b, x, y, z;
  if (ocb_cand(coords, rk, off_s, g, t, b, x, y, z) && b >= 0 && b < ox.nb) {
    const int64_t br = subm_brick(ox, b, x, y, z);
    const int r = subm_brick_rank(ox.l1[br >> 6], br);
    uint32_t h = ((uint32_t)r * 2654435761u) >> 23;  // 9 bits
    for (;;) {
      const int prev = atomicCAS(&key_s[h], -1, r);
      if (prev == -1 || prev == r) break;
      h = (h + 1) & (kL2Slots - 1);
    }
    atomicOr(&bits_s[h], 1ull << subm_vbit(x, y, z));
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kL2Slots; e += 256)
    if (key_s[e] >= 0)
      __hip_atomic_fetch_or(&ox.l2bits[key_s[e]], bits_s[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// rank[v] = all ones for the *total distinct output voxels; an overflowed
// index (more bricks or voxels than the candidate bound sized) is counted
// into status[ST_STATUS_OVERFLOW].
__global__ __launch_bounds__(256) void ocb_rank_clear_kernel(SubmIndex ox, const int32_t* __restrict__ total,
                                                             int32_t* __restrict__ status) {
  if (subm_overflowed(ox)) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&status[ST_STATUS_OVERFLOW], 1);
    return;
  }
  const int64_t nv = *total;
  for (int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x; v < nv; v += (int64_t)gridDim.x * 256)
    ox.rowmap[v] = -1;
}

// Lowest candidate rank per distinct output voxel.
template <typename CT>
__global__ __launch_bounds__(256) void ocb_rankmin_kernel(const CT* __restrict__ coords, Ranks rk,
                                                          const int32_t* __restrict__ offsets, Geom g,
                                                          SubmIndex ox) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  if (subm_overflowed(ox)) return;
  load_offsets(off_s, offsets, g.K);
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  int64_t b, x, y, z;
  if (!ocb_cand(coords, rk, off_s, g, t, b, x, y, z) || b < 0 || b >= ox.nb) return;
  atomicMin(reinterpret_cast<uint32_t*>(ox.rowmap) + ocb_voxel(ox, b, x, y, z), t);
}

// Whether candidate rank t is its output coordinate's first occurrence (v:
// the coordinate's voxel rank).
template <typename CT>
__device__ __forceinline__ bool ocb_first(const CT* __restrict__ coords, const Ranks& rk, const int32_t* off_s,
                                          const Geom& g, const SubmIndex& ox, uint32_t t, int64_t& b, int64_t& x,
                                          int64_t& y, int64_t& z, int& v) {
  if (!ocb_cand(coords, rk, off_s, g, t, b, x, y, z) || b < 0 || b >= ox.nb) return false;
  v = ocb_voxel(ox, b, x, y, z);
  return reinterpret_cast<const uint32_t*>(ox.rowmap)[v] == t;
}

// First occurrences per block of 256 ranks.
template <typename CT>
__global__ __launch_bounds__(256) void ocb_count_kernel(const CT* __restrict__ coords, Ranks rk,
                                                        const int32_t* __restrict__ offsets, Geom g, SubmIndex ox,
                                                        int32_t* __restrict__ block_counts) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  __shared__ int red_s[4];
  if (subm_overflowed(ox)) {  // no outputs
    if (threadIdx.x == 0) block_counts[blockIdx.x] = 0;
    return;
  }
  load_offsets(off_s, offsets, g.K);
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  int64_t b, x, y, z;
  int v;
  int c = ocb_first(coords, rk, off_s, g, ox, t, b, x, y, z, v) ? 1 : 0;
  c = wave_sum(c);
  if ((threadIdx.x & 63) == 0) red_s[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) block_counts[blockIdx.x] = red_s[0] + red_s[1] + red_s[2] + red_s[3];
}

// Output rows in rank order: block offset (scanned counts) + rank of the
// first occurrences below in the block; posmap[voxel rank] = output row.
template <typename CT>
__global__ __launch_bounds__(256) void ocb_emit_kernel(const CT* __restrict__ coords, Ranks rk,
                                                       const int32_t* __restrict__ offsets, Geom g, SubmIndex ox,
                                                       const int32_t* __restrict__ block_offsets,
                                                       CT* __restrict__ out_coords, int64_t n_out,
                                                       int32_t* __restrict__ posmap) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  __shared__ int scan_s[5];
  if (subm_overflowed(ox)) return;
  load_offsets(off_s, offsets, g.K);
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  int64_t b, x, y, z;
  int v;
  const bool first = ocb_first(coords, rk, off_s, g, ox, t, b, x, y, z, v);
  int tot;
  const int64_t pos = (int64_t)block_offsets[blockIdx.x] + block_exclusive_scan(first ? 1 : 0, scan_s, &tot);
  if (!first || pos >= n_out) return;
  posmap[v] = (int32_t)pos;
  CT* r = out_coords + pos * 4;
  r[0] = (CT)b;
  r[1] = (CT)x;
  r[2] = (CT)y;
  r[3] = (CT)z;
}

// Kernel map by query: for output row o and offset k the input coordinate
// (b, o * s - t_k), or transposed (b, (o - t_k) / s) when s divides every
// component, looked up in the input index (box [0, batches) x in_shape: the
// reference's bounds check, conv.py:54-59, 180-188; repeated coordinates
// resolve to their lowest row, as the input hash table does).  nbr and the
// output masks are written whole.  The transposed map comes from
// ocb_inverse_kernel, input-major: scattered from here, its 4-byte stores
// (14.2M on config 4) each cost a partial line (1.5 GB written per launch
// against 0.85 GB of map), and atomic ORs into its masks serialised.
constexpr int kQueryGroup = 4;  // lookups in flight per transposed query row (config 4 rows average 2 valid offsets)
inline size_t query_lds_bytes(int K) { return sizeof(int32_t) * ((size_t)(K < 32 ? K : 32) * 256 + 4 * (size_t)K); }
template <typename CT, bool TR>
__global__ __launch_bounds__(256) void strided_query_kernel(const CT* __restrict__ out_coords, int64_t n_out,
                                                            const int32_t* __restrict__ offsets, Geom g,
                                                            SubmIndex ix, int32_t* __restrict__ nbr,
                                                            uint32_t* __restrict__ out_masks) {
  __shared__ QueryLds<TR> lds;  // strided: the unit path's bricks, or the offsets
  int32_t* off_s = reinterpret_cast<int32_t*>(&lds);
  // transposed: LDS sized by K (query_lds_bytes) -- rows found [min(K, 32)][256], then per
  // offset t_k mod s on each axis (10 bits each) and floor(t_k / s) on each axis
  extern __shared__ int32_t dyn_s[];
  const int kc = g.K < 32 ? g.K : 32;
  int32_t* row_s = dyn_s;
  int32_t* tcode_s = dyn_s + kc * 256;
  int32_t* tdiv_s = tcode_s + g.K;
  if (TR) {
    for (int k = threadIdx.x; k < g.K; k += 256) {
      int code = 0;
      for (int a = 0; a < 3; ++a) {
        const int64_t t = offsets[3 * k + a];
        const int64_t td = t >= 0 ? t / g.s : -((-t + g.s - 1) / g.s);
        tdiv_s[3 * k + a] = (int32_t)td;
        code |= (int)(t - td * g.s) << (10 * a);
      }
      tcode_s[k] = code;
    }
    __syncthreads();
  }
  const bool unit = !TR && unit_offsets(offsets, g.K);
  if (!TR && !unit) load_offsets(off_s, offsets, g.K);
  const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (o >= n_out) return;
  int64_t b, x, y, z;
  load_coord(out_coords, o, b, x, y, z);
  const int K = g.K, W = (K + 31) >> 5;
  if (!TR) {  // (a kernel each: the branches' register needs differ)
    // o * s - t_k: with unit offsets the neighbours lie in the 2 x 2 x 2 bricks around o * s
    uint32_t mword = 0;
    auto emit = [&](int k, int32_t r) {
      nbr[(int64_t)k * n_out + o] = r;
      if (r >= 0) mword |= 1u << (k & 31);
      if ((k & 31) == 31 || k == K - 1) {
        out_masks[o * W + (k >> 5)] = mword;
        mword = 0;
      }
    };
    if (unit)
      unit_rows(ix, b, x * g.s, y * g.s, z * g.s, offsets, K, lds.bits, lds.pre, emit);
    else
      subm_neighbours<3>(ix, b, x * g.s, y * g.s, z * g.s, off_s, K, emit);
    return;
  }
  // (o - t_k) / s: s divides it when o and t_k agree mod s on every axis, and then it is
  // floor(o / s) - floor(t_k / s) -- one compare of residue codes per offset, 32-bit (in
  // 64-bit arithmetic, per offset, this kernel was bound by its ALU).  Few offsets qualify
  // (1 to 8 of 27 at stride 2), so the valid offsets of each 32 are compacted first and
  // looked up kQueryGroup at a time: usually one group of three dependent loads per row.
  // The rows found are staged in LDS (each thread its own column) and stored offset by
  // offset, so every store writes whole segments of a row of nbr.
  // |o| < 2^30 on every axis, else no input is near (|q| >= 2^20 > any shape)
  const bool near = x > -(1 << 30) && x < (1 << 30) && y > -(1 << 30) && y < (1 << 30) && z > -(1 << 30) &&
                    z < (1 << 30);
  int32_t xq = 0, yq = 0, zq = 0, code = -1;
  if (near) {
    int64_t q3[3];
    int rr[3];
    const int64_t c3[3] = {x, y, z};
    for (int a = 0; a < 3; ++a) {
      const int32_t c = (int32_t)c3[a];
      int32_t q;
      if (g.s_log2 >= 0) {
        q = c >> g.s_log2;
      } else {
        const int32_t s32 = (int32_t)g.s;
        q = c >= 0 ? c / s32 : -((-c + s32 - 1) / s32);
      }
      q3[a] = q;
      rr[a] = (int)(c - q * (int32_t)g.s);
    }
    xq = (int32_t)q3[0];
    yq = (int32_t)q3[1];
    zq = (int32_t)q3[2];
    code = rr[0] | (rr[1] << 10) | (rr[2] << 20);
  }
  auto q_of = [&](int k, int64_t& qx, int64_t& qy, int64_t& qz) {
    qx = xq - tdiv_s[3 * k];
    qy = yq - tdiv_s[3 * k + 1];
    qz = zq - tdiv_s[3 * k + 2];
    return subm_in_box(ix, b, qx, qy, qz);
  };
  for (int kb = 0; kb < K; kb += 32) {
    const int ke = K < kb + 32 ? K : kb + 32;
    uint32_t todo = 0, found = 0;
    for (int k = kb; k < ke; ++k) {
      int64_t qx, qy, qz;
      if (tcode_s[k] == code && q_of(k, qx, qy, qz)) todo |= 1u << (k - kb);
      row_s[(k - kb) * 256 + threadIdx.x] = -1;
    }
    while (todo) {
      int kk[kQueryGroup];
      int64_t brk[kQueryGroup];
      int vb[kQueryGroup];
      bool in[kQueryGroup];
#pragma unroll
      for (int j = 0; j < kQueryGroup; ++j) {
        in[j] = todo != 0;
        kk[j] = in[j] ? kb + __builtin_ctz(todo) : 0;
        todo &= todo - 1;  // (no-op once empty)
        int64_t qx = 0, qy = 0, qz = 0;
        if (in[j]) q_of(kk[j], qx, qy, qz);
        brk[j] = in[j] ? subm_brick(ix, b, qx, qy, qz) : 0;
        vb[j] = subm_vbit(qx, qy, qz);
      }
      SubmL1 e1[kQueryGroup];
#pragma unroll
      for (int j = 0; j < kQueryGroup; ++j) e1[j] = in[j] ? ix.l1[brk[j] >> 6] : SubmL1{0ull, 0, 0};
      unsigned long long bits[kQueryGroup];
      int32_t pre[kQueryGroup];
#pragma unroll
      for (int j = 0; j < kQueryGroup; ++j) {
        const bool occ = in[j] && ((e1[j].bits >> (brk[j] & 63)) & 1ull);
        const int r = occ ? subm_brick_rank(e1[j], brk[j]) : 0;
        bits[j] = occ ? ix.l2bits[r] : 0ull;
        pre[j] = occ ? ix.l2pre[r] : 0;
      }
#pragma unroll
      for (int j = 0; j < kQueryGroup; ++j) {
        if (!in[j]) continue;
        const bool has = (bits[j] >> vb[j]) & 1ull;
        const int32_t r = has ? ix.rowmap[pre[j] + (int)__popcll(bits[j] & below(vb[j]))] : -1;
        row_s[(kk[j] - kb) * 256 + threadIdx.x] = r;
        if (r >= 0) found |= 1u << (kk[j] - kb);
      }
    }
    for (int k = kb; k < ke; ++k) nbr[(int64_t)k * n_out + o] = row_s[(k - kb) * 256 + threadIdx.x];
    out_masks[o * W + (kb >> 5)] = found;
  }
}

// Transposed map of the brick build, input-major: invnbr[k][i] = output row
// of candidate (i, k), -1 when the filters drop it or row i is not the row the
// query resolves its coordinate to (in the box, the lowest row of a repeated
// coordinate); in_masks of the same.  Both written whole, one coalesced row of
// invnbr per offset.
template <typename CT>
__global__ __launch_bounds__(256) void ocb_inverse_kernel(const CT* __restrict__ coords, int64_t n,
                                                          const int32_t* __restrict__ offsets, Geom g, SubmIndex ox,
                                                          const int32_t* __restrict__ posmap, SubmIndex ix,
                                                          int32_t* __restrict__ invnbr,
                                                          uint32_t* __restrict__ in_masks) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  load_offsets(off_s, offsets, g.K);
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  // an overflowed output index holds no outputs: every candidate maps to none
  bool own = !subm_overflowed(ox) && subm_in_box(ix, b, x, y, z);
  if (own) {
    const int64_t br = subm_brick(ix, b, x, y, z);
    const int r = subm_brick_rank(ix.l1[br >> 6], br);
    own = ix.rowmap[ix.l2pre[r] + (int)__popcll(ix.l2bits[r] & below(subm_vbit(x, y, z)))] == (int32_t)i;
  }
  own = own && b < ox.nb;
  const int K = g.K, W = (K + 31) >> 5;
  uint32_t mword = 0;
  for (int k0 = 0; k0 < K; k0 += kSubmGroup) {
    int64_t brk[kSubmGroup];
    int vb[kSubmGroup];
    bool in[kSubmGroup];
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) {
      const int k = k0 + j;
      int64_t cx = 0, cy = 0, cz = 0;
      in[j] = own && k < K &&
              candidate(g, x, y, z, off_s[3 * k], off_s[3 * k + 1], off_s[3 * k + 2], cx, cy, cz);
      brk[j] = in[j] ? subm_brick(ox, b, cx, cy, cz) : 0;
      vb[j] = subm_vbit(cx, cy, cz);
    }
    SubmL1 e1[kSubmGroup];
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) e1[j] = in[j] ? ox.l1[brk[j] >> 6] : SubmL1{0ull, 0, 0};
    unsigned long long bits[kSubmGroup];
    int32_t pre[kSubmGroup];
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) {
      const int r = in[j] ? subm_brick_rank(e1[j], brk[j]) : 0;
      bits[j] = in[j] ? ox.l2bits[r] : 0ull;
      pre[j] = in[j] ? ox.l2pre[r] : 0;
    }
#pragma unroll
    for (int j = 0; j < kSubmGroup; ++j) {
      const int k = k0 + j;
      if (k >= K) break;
      const int32_t o = in[j] ? posmap[pre[j] + (int)__popcll(bits[j] & below(vb[j]))] : -1;
      invnbr[(int64_t)k * n + i] = o;
      if (o >= 0) mword |= 1u << (k & 31);
      if ((k & 31) == 31 || k == K - 1) {
        in_masks[i * W + (k >> 5)] = mword;
        mword = 0;
      }
    }
  }
}

// Prefix pass of an index level: above kSubmInlineTiles tiles the tile sums
// are scanned once first (the inline sum's O(ntiles^2) loads over the grid
// would outgrow the extra launch).
constexpr int64_t kSubmInlineTiles = 1024;
// Polls of a missing tile total before subm_level_kernel computes it itself
// (ST_SUBM_SPIN overrides; 0 computes every earlier tile's total directly).
static int subm_spin() {
  const char* e = getenv("ST_SUBM_SPIN");
  return e ? atoi(e) : 4096;
}

// One level of the index (bricks or voxels): the counts and prefix of its
// level-1 entries.  Up to kSubmInlineTiles tiles one launch does both
// (subm_level_kernel); above, the tile sums, their scan and the prefix run as
// three launches.
template <bool BRICKS>
int launch_subm_level(const SubmIndex& ix, int32_t* voxels, hipStream_t stream) {
  if (ix.ntiles <= kSubmInlineTiles) {
    subm_level_kernel<BRICKS><<<(unsigned)ix.ntiles, kSubmThreads, 0, stream>>>(ix, voxels, subm_spin());
    return hipGetLastError() == hipSuccess ? ST_OK : ST_ERR_HIP;
  }
  subm_tile_sum_kernel<BRICKS><<<(unsigned)ix.ntiles, kSubmThreads, 0, stream>>>(ix);
  const int rc = launch_exclusive_scan(ix.tile_sums, ix.ntiles, stream);
  if (rc != ST_OK) return rc;
  subm_prefix_kernel<BRICKS><<<(unsigned)ix.ntiles, kSubmThreads, 0, stream>>>(ix, voxels, true);
  return hipGetLastError() == hipSuccess ? ST_OK : ST_ERR_HIP;
}

// Output index geometry of a brick build: rows = the candidate bound; false
// when it cannot be indexed.
static bool ocb_geom(int64_t n, const Geom& g, int64_t batches, int64_t kernel_size, int64_t dilation,
                     int64_t* rows, int64_t* nranks, int64_t* bytes, int64_t* index_bytes = nullptr) {
  if (n <= 0 || batches <= 0 || g.s > 1024) return false;  // (residues of the query: 10 bits)
  for (int a = 0; a < 3; ++a)
    if (g.out_shape[a] < 1 || g.out_shape[a] > 32768) return false;  // every output packs into a key
  const int64_t nchunks = (g.K + g.chunk - 1) / g.chunk;
  *nranks = n * nchunks * (int64_t)g.chunk;
  if (*nranks > (1ll << 32) - 512) return false;  // every thread's 32-bit rank, padding included, fits
  *rows = n * cands_per_input(g, kernel_size, dilation);
  const int64_t ws = subm_workspace_bytes(*rows, batches, g.out_shape[0], g.out_shape[1], g.out_shape[2]);
  if (ws < 0) return false;
  // the index, the distinct-voxel count, posmap (output row per voxel rank)
  *bytes = ws + 256 + (int64_t)subm_align256(sizeof(int32_t) * (size_t)*rows);
  if (index_bytes) *index_bytes = ws;
  return true;
}

}  // namespace st

using namespace st;

extern "C" {

int st_kmap_subm_workspace(int64_t n, int64_t batches, int64_t sx, int64_t sy, int64_t sz, int64_t* bytes) {
  if (!bytes) return ST_ERR_ARG;
  const int64_t need = subm_workspace_bytes(n, batches, sx, sy, sz);
  if (need < 0) return ST_ERR_ARG;
  *bytes = need;
  return ST_OK;
}

int st_subm_index(const void* coords, int coord_dtype, int64_t n, int64_t batches, int64_t sx, int64_t sy,
                  int64_t sz, void* workspace, int64_t workspace_bytes, int32_t* status, st_stream_t stream) {
  const int64_t need = subm_workspace_bytes(n, batches, sx, sy, sz);
  if (need < 0 || workspace_bytes < need) return ST_ERR_ARG;
  if (coord_dtype < ST_COORD_I16 || coord_dtype > ST_COORD_I64) return ST_ERR_UNSUPPORTED;
  if (n == 0) return ST_OK;
  if (!coords || !workspace) return ST_ERR_ARG;
  SubmIndex ix;
  subm_view(workspace, n, batches, sx, sy, sz, &ix);
  const unsigned rows = st_blocks(n, kSubmThreads);
  int64_t clear_items = ix.cap2 > n ? ix.cap2 : n;
  if ((ix.nbricks + 15) / 16 > clear_items) clear_items = (ix.nbricks + 15) / 16;
  unsigned cg = st_blocks(clear_items, kSubmThreads);
  if (cg > 4096) cg = 4096;
  subm_clear_kernel<<<cg, kSubmThreads, 0, stream>>>(ix, n, status);
  ST_DISPATCH_COORD(coord_dtype, CT, {
    const CT* c = (const CT*)coords;
    subm_occ_kernel<CT><<<rows, kSubmThreads, 0, stream>>>(c, n, ix, status);
    if (launch_subm_level<true>(ix, nullptr, stream) != ST_OK) return ST_ERR_HIP;
    subm_l2_kernel<CT><<<rows, kSubmThreads, 0, stream>>>(c, n, ix);
    if (launch_subm_level<false>(ix, nullptr, stream) != ST_OK) return ST_ERR_HIP;
    subm_rowmap_kernel<CT><<<rows, kSubmThreads, 0, stream>>>(c, n, ix, status);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_kmap_subm_query(const void* coords, int coord_dtype, int64_t n, const int32_t* offsets, int K,
                       int64_t batches, int64_t sx, int64_t sy, int64_t sz, const void* workspace,
                       int64_t workspace_bytes, int32_t* nbr, uint32_t* row_masks, st_stream_t stream) {
  const int64_t need = subm_workspace_bytes(n, batches, sx, sy, sz);
  if (need < 0 || workspace_bytes < need || K <= 0 || K > ST_MAX_KVOL) return ST_ERR_ARG;
  if (coord_dtype < ST_COORD_I16 || coord_dtype > ST_COORD_I64) return ST_ERR_UNSUPPORTED;
  if (n == 0) return ST_OK;
  if (!coords || !offsets || !workspace || (!nbr && !row_masks)) return ST_ERR_ARG;
  SubmIndex ix;
  subm_view(const_cast<void*>(workspace), n, batches, sx, sy, sz, &ix);
  const unsigned grid = st_blocks(n, kSubmThreads);
  ST_DISPATCH_COORD(coord_dtype, CT, {
    if (nbr)
      subm_query_kernel<CT, true><<<grid, kSubmThreads, 0, stream>>>((const CT*)coords, n, offsets, K, ix, nbr,
                                                                     row_masks);
    else
      subm_query_kernel<CT, false><<<grid, kSubmThreads, 0, stream>>>((const CT*)coords, n, offsets, K, ix, nullptr,
                                                                      row_masks);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_kmap_subm(const void* coords, int coord_dtype, int64_t n, const int32_t* offsets, int K, int64_t batches,
                 int64_t sx, int64_t sy, int64_t sz, void* workspace, int64_t workspace_bytes, int32_t* nbr,
                 uint32_t* row_masks, int32_t* status, st_stream_t stream) {
  const int64_t need = subm_workspace_bytes(n, batches, sx, sy, sz);
  if (need < 0 || K <= 0 || K > ST_MAX_KVOL || workspace_bytes < need) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!coords || !offsets || !workspace || !nbr) return ST_ERR_ARG;
  const int rc = st_subm_index(coords, coord_dtype, n, batches, sx, sy, sz, workspace, workspace_bytes, status,
                               stream);
  if (rc != ST_OK) return rc;
  return st_kmap_subm_query(coords, coord_dtype, n, offsets, K, batches, sx, sy, sz, workspace, workspace_bytes, nbr,
                            row_masks, stream);
}

int st_outcoords_brick_sizes(int64_t n, const st_outgeom* gin, int64_t batches, int64_t kernel_size,
                             int64_t dilation, int64_t* workspace_bytes, int64_t* num_blocks) {
  Geom g;
  if (n < 0 || !make_geom(gin, g) || kernel_size < 1 || dilation < 1 || !workspace_bytes || !num_blocks)
    return ST_ERR_ARG;
  int64_t rows, nranks, bytes;
  if (!ocb_geom(n, g, batches, kernel_size, dilation, &rows, &nranks, &bytes)) return ST_ERR_UNSUPPORTED;
  *workspace_bytes = bytes;
  *num_blocks = (nranks + 255) / 256;
  return ST_OK;
}

int st_outcoords_brick_plan(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                            const st_outgeom* gin, int64_t batches, int64_t kernel_size, int64_t dilation,
                            void* workspace, int64_t workspace_bytes, int32_t* block_counts, int64_t num_blocks,
                            int32_t* status, st_stream_t stream) {
  Geom g;
  if (n < 0 || !make_geom(gin, g) || !offsets || !in_coords || !workspace || !block_counts || !status)
    return ST_ERR_ARG;
  int64_t rows, nranks, bytes, ixb;
  if (!ocb_geom(n, g, batches, kernel_size, dilation, &rows, &nranks, &bytes, &ixb)) return ST_ERR_UNSUPPORTED;
  if (workspace_bytes < bytes || num_blocks != (nranks + 255) / 256) return ST_ERR_ARG;
  if (coord_dtype < ST_COORD_I16 || coord_dtype > ST_COORD_I64) return ST_ERR_UNSUPPORTED;
  SubmIndex ox;
  subm_view(workspace, rows, batches, g.out_shape[0], g.out_shape[1], g.out_shape[2], &ox);
  int32_t* total = (int32_t*)((char*)workspace + ixb);
  ox.flag = total + 1;
  const Ranks rk = make_ranks(g, n, nranks);
  const unsigned grid = (unsigned)num_blocks, tiles = (unsigned)ox.ntiles;
  unsigned cg = st_blocks((ox.nbricks + 15) / 16, kSubmThreads);
  cg = cg < 1 ? 1 : (cg > 4096 ? 4096 : cg);
  subm_clear_kernel<<<cg, kSubmThreads, 0, stream>>>(ox, 0, status);
  ST_DISPATCH_COORD(coord_dtype, CT, {
    const CT* c = (const CT*)in_coords;
    ocb_occ_kernel<CT><<<grid, 256, 0, stream>>>(c, rk, offsets, g, ox, status);
    if (launch_subm_level<true>(ox, nullptr, stream) != ST_OK) return ST_ERR_HIP;
    ocb_l2_kernel<CT><<<grid, 256, 0, stream>>>(c, rk, offsets, g, ox);
    if (launch_subm_level<false>(ox, total, stream) != ST_OK) return ST_ERR_HIP;
    ocb_rank_clear_kernel<<<2048, 256, 0, stream>>>(ox, total, status);
    ocb_rankmin_kernel<CT><<<grid, 256, 0, stream>>>(c, rk, offsets, g, ox);
    ocb_count_kernel<CT><<<grid, 256, 0, stream>>>(c, rk, offsets, g, ox, block_counts);
  });
  ST_CHECK_LAUNCH();
  return launch_exclusive_scan(block_counts, num_blocks, stream);
}

int st_outcoords_brick_emit(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                            const st_outgeom* gin, int64_t batches, int64_t kernel_size, int64_t dilation,
                            void* workspace, int64_t workspace_bytes, const int32_t* block_counts,
                            int64_t num_blocks, void* out_coords, int64_t n_out, st_stream_t stream) {
  Geom g;
  if (n < 0 || n_out < 0 || !make_geom(gin, g) || !offsets || !in_coords || !workspace || !block_counts)
    return ST_ERR_ARG;
  int64_t rows, nranks, bytes, ixb;
  if (!ocb_geom(n, g, batches, kernel_size, dilation, &rows, &nranks, &bytes, &ixb)) return ST_ERR_UNSUPPORTED;
  if (workspace_bytes < bytes || num_blocks != (nranks + 255) / 256) return ST_ERR_ARG;
  if (coord_dtype < ST_COORD_I16 || coord_dtype > ST_COORD_I64) return ST_ERR_UNSUPPORTED;
  if (n_out == 0) return ST_OK;
  if (!out_coords) return ST_ERR_ARG;
  SubmIndex ox;
  subm_view(workspace, rows, batches, g.out_shape[0], g.out_shape[1], g.out_shape[2], &ox);
  ox.flag = (int32_t*)((char*)workspace + ixb) + 1;
  int32_t* posmap = (int32_t*)((char*)workspace + ixb + 256);
  ST_DISPATCH_COORD(coord_dtype, CT, {
    ocb_emit_kernel<CT><<<(unsigned)num_blocks, 256, 0, stream>>>((const CT*)in_coords, make_ranks(g, n, nranks),
                                                                  offsets, g, ox, block_counts, (CT*)out_coords,
                                                                  n_out, posmap);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_kmap_strided_query(const void* out_coords, int coord_dtype, int64_t n_out, const int32_t* offsets,
                          const st_outgeom* gin, int64_t batches, const void* in_index, int64_t in_index_bytes,
                          int64_t n_in, int32_t* nbr, uint32_t* out_masks, st_stream_t stream) {
  Geom g;
  if (n_out < 0 || n_in < 0 || !make_geom(gin, g) || !offsets) return ST_ERR_ARG;
  if (n_out >= (1ll << 31)) return ST_ERR_ARG;
  if (g.s > 1024) return ST_ERR_UNSUPPORTED;
  const int64_t need = subm_workspace_bytes(n_in, batches, g.in_shape[0], g.in_shape[1], g.in_shape[2]);
  if (need < 0 || in_index_bytes < need) return ST_ERR_ARG;
  if (coord_dtype < ST_COORD_I16 || coord_dtype > ST_COORD_I64) return ST_ERR_UNSUPPORTED;
  if (n_out == 0) return ST_OK;
  if (!out_coords || !in_index || !nbr || !out_masks) return ST_ERR_ARG;
  SubmIndex ix;
  subm_view(const_cast<void*>(in_index), n_in, batches, g.in_shape[0], g.in_shape[1], g.in_shape[2], &ix);
  ST_DISPATCH_COORD(coord_dtype, CT, {
    if (g.transposed)
      strided_query_kernel<CT, true><<<st_blocks(n_out, 256), 256, query_lds_bytes(g.K), stream>>>(
          (const CT*)out_coords, n_out, offsets, g, ix, nbr, out_masks);
    else
      strided_query_kernel<CT, false><<<st_blocks(n_out, 256), 256, 0, stream>>>((const CT*)out_coords, n_out,
                                                                                offsets, g, ix, nbr, out_masks);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_outcoords_brick_inverse(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                               const st_outgeom* gin, int64_t batches, int64_t kernel_size, int64_t dilation,
                               const void* workspace, int64_t workspace_bytes, const void* in_index,
                               int64_t in_index_bytes, int32_t* invnbr, uint32_t* in_masks, st_stream_t stream) {
  Geom g;
  if (n < 0 || !make_geom(gin, g) || !offsets || !in_coords || !workspace) return ST_ERR_ARG;
  int64_t rows, nranks, bytes, ixb;
  if (!ocb_geom(n, g, batches, kernel_size, dilation, &rows, &nranks, &bytes, &ixb)) return ST_ERR_UNSUPPORTED;
  const int64_t need = subm_workspace_bytes(n, batches, g.in_shape[0], g.in_shape[1], g.in_shape[2]);
  if (workspace_bytes < bytes || need < 0 || in_index_bytes < need) return ST_ERR_ARG;
  if (coord_dtype < ST_COORD_I16 || coord_dtype > ST_COORD_I64) return ST_ERR_UNSUPPORTED;
  if (!in_index || !invnbr || !in_masks) return ST_ERR_ARG;
  SubmIndex ox, ix;
  subm_view(const_cast<void*>(workspace), rows, batches, g.out_shape[0], g.out_shape[1], g.out_shape[2], &ox);
  ox.flag = (int32_t*)((char*)workspace + ixb) + 1;
  subm_view(const_cast<void*>(in_index), n, batches, g.in_shape[0], g.in_shape[1], g.in_shape[2], &ix);
  const int32_t* posmap = (const int32_t*)((const char*)workspace + ixb + 256);
  ST_DISPATCH_COORD(coord_dtype, CT, {
    ocb_inverse_kernel<CT><<<st_blocks(n, 256), 256, 0, stream>>>((const CT*)in_coords, n, offsets, g, ox, posmap,
                                                                 ix, invnbr, in_masks);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // extern "C"
