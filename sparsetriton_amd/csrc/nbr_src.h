// Neighbour sources for the GEMM kernels: where the row of A feeding row r
// through kernel offset k comes from.
//
//   MapSrc  : a precomputed kernel map, map[k * ks + r * rs] (-1 = none).
//   TiledSrc: a tile plan (st_tile_plan): per 128-row destination tile its
//             active offsets and, per active offset, the 128 source rows
//             stored contiguously -- the gather-GEMM's map reads become
//             coalesced 512-byte loads instead of one cache line per entry.
//   HashSrc : probe the coordinate table inside the GEMM (implicit hash-fly):
//             q = (c.xyz * mul + sign * offsets[k]) / div, kept only when the
//             division is exact and 0 <= q < bounds (on each axis whose bound
//             is > 0), then looked up.  Rows whose own c lies outside
//             [0, row_bounds) (when given) have no pairs.
//
// A source is used as  rc = src.row(r)  (once per row)  then  src.get(rc, k).
// k is uniform across the workgroup in every caller, so offsets[k] is a
// scalar load.
#pragma once

#include "common.h"

namespace st {

struct MapSrc {
  static constexpr bool kTiled = false;
  static constexpr bool kProbe = false;
  static constexpr bool kRev = false;
  const int32_t* __restrict__ map;
  int64_t ks, rs;
  typedef int64_t RowCtx;
  __device__ __forceinline__ RowCtx row(int64_t r) const { return r; }
  __device__ __forceinline__ int32_t get(const RowCtx& r, int k) const { return map[(int64_t)k * ks + r * rs]; }
};

// Tile plan of a gather-GEMM (kTileRows destination rows per tile):
// nk[t] active offsets of tile t, listed in klist[t * K + j] (ascending), and
// tmap[((int64_t)t * K + j) * kTileRows + r] = source row of the tile's row r
// through its j-th active offset (-1 = none).
constexpr int kTileRows = 128;
struct TiledSrc {
  static constexpr bool kTiled = true;
  static constexpr bool kProbe = false;
  static constexpr bool kRev = true;
  const int32_t* __restrict__ nk;
  const int16_t* __restrict__ klist;
  const int32_t* __restrict__ tmap;
  int K;
  // rev: the GEMM's B slice of offset k is Bt[K - 1 - k] (the input gradient of a
  // submanifold map that is its own transpose, with the weights as given)
  int rev = 0;
  typedef int64_t RowCtx;
  __device__ __forceinline__ RowCtx row(int64_t r) const { return r; }
  __device__ __forceinline__ int32_t get_tile(int64_t tile, int j, int r) const {
    return tmap[((int64_t)tile * K + j) * kTileRows + r];
  }
};

// Index of the B slice that multiplies the sources of offset k (sources with a
// rev member: Bt[K - 1 - k] when it is set).
template <typename Src>
__device__ __forceinline__ int b_slice(const Src& src, int k) {
  if constexpr (Src::kRev)
    return src.rev ? src.K - 1 - k : k;
  else
    return k;
}

template <typename CT>
struct HashSrc {
  static constexpr bool kTiled = false;
  static constexpr bool kRev = false;
  static constexpr bool kProbe = true;  // get() is a table probe: callers batch prep / home-slot loads / finish
  const CT* __restrict__ coords;
  const int32_t* __restrict__ offsets;
  const uint64_t* __restrict__ keys;
  const uint32_t* __restrict__ vals;
  uint32_t cap;
  int32_t sign;
  int64_t mul, div;
  int64_t bx, by, bz;
  int64_t rbx, rby, rbz;  // row bounds (checked when > 0)
  struct RowCtx {
    int64_t b, x, y, z;
    bool ok;
  };
  __device__ __forceinline__ RowCtx row(int64_t r) const {
    RowCtx c;
    load_coord(coords, r, c.b, c.x, c.y, c.z);
    c.ok = !((rbx > 0 && (c.x < 0 || c.x >= rbx)) || (rby > 0 && (c.y < 0 || c.y >= rby)) ||
             (rbz > 0 && (c.z < 0 || c.z >= rbz)));
    c.x *= mul;
    c.y *= mul;
    c.z *= mul;
    return c;
  }
  // The key of row c's neighbour through offset k and its home slot; false when it has none.
  __device__ __forceinline__ bool prep(const RowCtx& c, int k, uint64_t& key, uint32_t& slot) const {
    if (!c.ok) return false;
    int64_t qx = c.x + sign * (int64_t)offsets[3 * k];
    int64_t qy = c.y + sign * (int64_t)offsets[3 * k + 1];
    int64_t qz = c.z + sign * (int64_t)offsets[3 * k + 2];
    if (div > 1) {
      if (qx % div || qy % div || qz % div) return false;
      qx /= div;
      qy /= div;
      qz /= div;
    }
    if ((bx > 0 && (qx < 0 || qx >= bx)) || (by > 0 && (qy < 0 || qy >= by)) || (bz > 0 && (qz < 0 || qz >= bz)))
      return false;
    if (!pack_key(c.b, qx, qy, qz, key)) return false;
    slot = home_slot(key, cap);
    return true;
  }
  __device__ __forceinline__ int32_t get(const RowCtx& c, int k) const {
    uint64_t key;
    uint32_t slot;
    if (!prep(c, k, key, slot)) return -1;
    const uint32_t s = find_slot_from(keys, cap, key, slot, keys[slot]);
    return s == ST_NO_VAL ? -1 : (int32_t)vals[s];
  }
};

}  // namespace st
