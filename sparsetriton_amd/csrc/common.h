// Shared device/host helpers for the sparse-convolution HIP library (gfx950).
//
// Coordinates are rows (b, x, y, z).  Every coordinate is packed into one
// exact 64-bit key, 16 bits per component, with the same bit layout as the
// reference's flatten_coord (sparsetriton/utils/hash.py:49-54):
//     key = b << 48 | (u16)x << 32 | (u16)y << 16 | (u16)z
// A coordinate is packable when b is in [0, 32767] and x, y, z are in
// [-32768, 32767]; with b >= 0 the key's top bit is clear, so no valid key
// equals the all-ones EMPTY sentinel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/sparsetriton_amd.h"

#define ST_EMPTY_KEY 0xFFFFFFFFFFFFFFFFull
#define ST_NO_VAL 0xFFFFFFFFu

namespace st {

constexpr int kWave = 64;

// ---------------------------------------------------------------- keys/hash

__device__ __forceinline__ bool in_i16(int64_t v) { return v >= -32768 && v <= 32767; }

__device__ __forceinline__ bool pack_key(int64_t b, int64_t x, int64_t y, int64_t z, uint64_t& key) {
  if (b < 0 || b > 32767 || !in_i16(x) || !in_i16(y) || !in_i16(z)) return false;
  key = ((uint64_t)b << 48) | ((uint64_t)(uint16_t)x << 32) | ((uint64_t)(uint16_t)y << 16) |
        (uint64_t)(uint16_t)z;
  return true;
}

// 64-bit finaliser (MurmurHash3 fmix64): every input bit affects every output bit,
// so the structured (b, x, y, z) keys spread uniformly over the table.
__device__ __forceinline__ uint64_t mix64(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return k;
}

// Home slot in [0, cap): the top 32 hash bits scaled to the table size
// (multiply-shift range reduction; cap need not be a power of two).  Keys are
// spread uniformly on purpose: placing the voxels of a 4x4x4 brick in adjacent
// slots (so a row's 27 probes share cache lines) packed the dense bricks of
// config 5 into long full runs at load 0.5, and the probes for absent
// neighbours, a third of all, walked them: 12x slower queries.
__device__ __forceinline__ uint32_t home_slot(uint64_t key, uint32_t cap) {
  return (uint32_t)(((mix64(key) >> 32) * (uint64_t)cap) >> 32);
}

__device__ __forceinline__ uint32_t next_slot(uint32_t s, uint32_t cap) {
  return (s + 1 == cap) ? 0u : s + 1;
}

// Linear-probe lookup.  Returns the slot holding `key`, or ST_NO_VAL when an
// empty slot (or a full sweep of the table) proves it absent.
__device__ __forceinline__ uint32_t find_slot(const uint64_t* __restrict__ keys, uint32_t cap, uint64_t key) {
  uint32_t s = home_slot(key, cap);
  for (uint32_t step = 0; step < cap; ++step) {
    uint64_t k = keys[s];
    if (k == key) return s;
    if (k == ST_EMPTY_KEY) return ST_NO_VAL;
    s = next_slot(s, cap);
  }
  return ST_NO_VAL;
}

// find_slot continued from slot s whose key `k` the caller already loaded.
__device__ __forceinline__ uint32_t find_slot_from(const uint64_t* __restrict__ keys, uint32_t cap, uint64_t key,
                                                   uint32_t s, uint64_t k) {
  for (uint32_t step = 0; step < cap; ++step) {
    if (k == key) return s;
    if (k == ST_EMPTY_KEY) return ST_NO_VAL;
    s = next_slot(s, cap);
    k = keys[s];
  }
  return ST_NO_VAL;
}

// Insert-or-find.  Returns the slot of `key` (claimed with a 64-bit CAS if new),
// or ST_NO_VAL if the table is full.  `was_new` tells whether this call claimed it.
// A plain load precedes each CAS: probing with CAS alone measured slower.
__device__ __forceinline__ uint32_t insert_slot(uint64_t* __restrict__ keys, uint32_t cap, uint64_t key,
                                                bool& was_new) {
  uint32_t s = home_slot(key, cap);
  for (uint32_t step = 0; step < cap; ++step) {
    uint64_t k = keys[s];
    if (k == key) {
      was_new = false;
      return s;
    }
    if (k == ST_EMPTY_KEY) {
      unsigned long long old =
          atomicCAS((unsigned long long*)&keys[s], (unsigned long long)ST_EMPTY_KEY, (unsigned long long)key);
      if (old == ST_EMPTY_KEY) {
        was_new = true;
        return s;
      }
      if (old == key) {
        was_new = false;
        return s;
      }
    }
    s = next_slot(s, cap);
  }
  return ST_NO_VAL;
}

// insert_slot continued from slot s whose key `k` the caller already loaded
// (so a batch of inserts can have their first loads in flight together).
__device__ __forceinline__ uint32_t insert_slot_from(uint64_t* __restrict__ keys, uint32_t cap, uint64_t key,
                                                     uint32_t s, uint64_t k, bool& was_new) {
  for (uint32_t step = 0; step < cap; ++step) {
    if (k == key) {
      was_new = false;
      return s;
    }
    if (k == ST_EMPTY_KEY) {
      unsigned long long old =
          atomicCAS((unsigned long long*)&keys[s], (unsigned long long)ST_EMPTY_KEY, (unsigned long long)key);
      if (old == ST_EMPTY_KEY) {
        was_new = true;
        return s;
      }
      if (old == key) {
        was_new = false;
        return s;
      }
    }
    s = next_slot(s, cap);
    k = keys[s];
  }
  return ST_NO_VAL;
}

// (b, x, y, z) of a key made by pack_key
__device__ __forceinline__ void unpack_key(uint64_t key, int64_t& b, int64_t& x, int64_t& y, int64_t& z) {
  b = (int64_t)(key >> 48);
  x = (int16_t)(uint16_t)(key >> 32);
  y = (int16_t)(uint16_t)(key >> 16);
  z = (int16_t)(uint16_t)key;
}

// ------------------------------------------------------------- coordinates

template <typename CT>
__device__ __forceinline__ void load_coord(const CT* __restrict__ c, int64_t i, int64_t& b, int64_t& x, int64_t& y,
                                           int64_t& z) {
  const CT* r = c + i * 4;
  b = (int64_t)r[0];
  x = (int64_t)r[1];
  y = (int64_t)r[2];
  z = (int64_t)r[3];
}

// ------------------------------------------------------------ wave helpers

__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v |= __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Number of set lanes strictly below this lane in a 64-bit ballot.
__device__ __forceinline__ int lanes_below(uint64_t ballot) {
  const int lane = threadIdx.x & (kWave - 1);
  uint64_t below = lane == 0 ? 0ull : (ballot & (~0ull >> (64 - lane)));
  return __popcll(below);
}

// Inclusive prefix sum across the wave.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int t = __shfl_up(v, off, kWave);
    if (lane >= off) v += t;
  }
  return v;
}

// Workgroup-wide exclusive prefix of one int per thread (blockDim.x <= 1024,
// multiple of 64).  `scratch` needs blockDim.x/64 + 1 ints of LDS.
// Returns the exclusive prefix; *total receives the workgroup sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* scratch, int* total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  int inc = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    int t = __shfl_up(inc, off, kWave);
    if (lane >= off) inc += t;
  }
  if (lane == kWave - 1) scratch[wid] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < nw; ++w) {
      int t = scratch[w];
      scratch[w] = run;
      run += t;
    }
    scratch[nw] = run;
  }
  __syncthreads();
  int res = scratch[wid] + inc - v;
  *total = scratch[nw];
  __syncthreads();
  return res;
}

// In-place exclusive scan of counts[0..n) on `stream`, counts[n] = total
// (one workgroup; defined in kmap.hip).
int launch_exclusive_scan(int32_t* counts, int64_t n, hipStream_t stream);

constexpr int kPairRows = 4096;        // map rows per (row block, offset) workgroup of the pair list
constexpr int kChunkOrderMax = 16384;  // chunks whose keys one workgroup holds in LDS (uint16 each)
constexpr int kChunkOrderMaxK = 28;    // offsets of its per-(offset, bucket) count table
constexpr int kPairChunkMin = 1024;    // smallest chunk size ST_PAIR_CHUNK_AUTO picks
constexpr int kPairChunksAuto = 2048;  // ... for at most this many chunks' worth of pairs

// Chunks of an ST_PAIR_CHUNK_AUTO pair list over n rows and K offsets, at most.
inline int64_t auto_max_chunks(int64_t n, int K) {
  const int64_t by_rows = (int64_t)K * n / kPairChunkMin + K;
  return by_rows < kPairChunksAuto + K ? by_rows : kPairChunksAuto + K;
}

// Pair list of a map (count, scan + kstart / cstart, emit) and its chunk order
// (defined in kmap.hip; arguments checked by the caller).  launch_chunk_order
// returns ST_ERR_UNSUPPORTED above kChunkOrderMax chunks or kChunkOrderMaxK offsets.
int launch_pairs(const int32_t* map, int64_t ks, int64_t rs, int64_t n_out, int K, int64_t n_in,
                 int32_t* block_counts, int64_t nb, int chunk, int32_t* kstart, int32_t* cstart, int32_t* pairs,
                 hipStream_t stream);
int launch_chunk_order(const int32_t* pairs, const int32_t* kstart, const int32_t* cstart, int K, int chunk,
                       int64_t max_chunks, int64_t n_out, int32_t* order, hipStream_t stream);
int launch_chunk_keys(const int32_t* pairs, const int32_t* kstart, const int32_t* cstart, int K, int chunk,
                      int64_t max_chunks, int64_t n_out, uint32_t* keys, hipStream_t stream);

}  // namespace st

// ------------------------------------------------------------- host helpers

#define ST_DISPATCH_COORD(cd, CT, ...)            \
  switch (cd) {                                   \
    case ST_COORD_I16: {                          \
      using CT = int16_t;                         \
      __VA_ARGS__;                                \
      break;                                      \
    }                                             \
    case ST_COORD_I32: {                          \
      using CT = int32_t;                         \
      __VA_ARGS__;                                \
      break;                                      \
    }                                             \
    case ST_COORD_I64: {                          \
      using CT = int64_t;                         \
      __VA_ARGS__;                                \
      break;                                      \
    }                                             \
    default:                                      \
      return ST_ERR_UNSUPPORTED;                  \
  }


#define ST_CHECK_LAUNCH()                                    \
  do {                                                       \
    hipError_t _e = hipGetLastError();                       \
    if (_e != hipSuccess) return ST_ERR_HIP;                 \
  } while (0)

#define ST_CHECK_HIP(expr)                                   \
  do {                                                       \
    hipError_t _e = (expr);                                  \
    if (_e != hipSuccess) return ST_ERR_HIP;                 \
  } while (0)

static inline unsigned st_blocks(int64_t n, int per_block) {
  return (unsigned)((n + per_block - 1) / per_block);
}
