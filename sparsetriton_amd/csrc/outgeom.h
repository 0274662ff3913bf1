// Geometry of a strided or transposed convolution's output coordinates:
// the candidate of an (input row, offset) pair, its rank in the reference's
// enumeration order, and the bounds of the neighbour query.  Shared by the
// hash-table build (kmap.hip) and the brick-index build (kmap_subm.hip).
#pragma once

#include "common.h"

namespace st {

struct Geom {
  int K;
  int transposed;
  int chunk;   // offsets per chunk of the candidate order (K: one chunk)
  int s_log2;  // log2(s) when the stride is a power of two, else -1
  int64_t s;
  int64_t in_shape[3];
  int64_t out_shape[3];
};

// q = c / s when s divides c exactly (c of either sign); a shift and a mask
// for power-of-two strides, where a 64-bit division would cost ~100
// instructions.
__device__ __forceinline__ bool div_stride(const Geom& g, int64_t c, int64_t& q) {
  if (g.s_log2 >= 0) {
    if (c & (g.s - 1)) return false;
    q = c >> g.s_log2;
    return true;
  }
  if (c % g.s) return false;
  q = c / g.s;
  return true;
}

// Candidate output coordinate of input (x, y, z) through offset t; false when
// filtered out.  Normal conv: c = in + t must be >= 0 and divisible by the
// stride on every axis, then c / s must be <= out_shape - 1 (kmap.py:286-309).
// Transposed: c = in * s + t must lie in [0, out_shape - 1] (kmap.py:406-423).
__device__ __forceinline__ bool candidate(const Geom& g, int64_t x, int64_t y, int64_t z, int32_t tx, int32_t ty,
                                          int32_t tz, int64_t& ox, int64_t& oy, int64_t& oz) {
  if (g.transposed) {
    ox = x * g.s + tx;
    oy = y * g.s + ty;
    oz = z * g.s + tz;
  } else {
    const int64_t cx = x + tx, cy = y + ty, cz = z + tz;
    if (cx < 0 || cy < 0 || cz < 0) return false;
    if (!div_stride(g, cx, ox) || !div_stride(g, cy, oy) || !div_stride(g, cz, oz)) return false;
  }
  return ox >= 0 && oy >= 0 && oz >= 0 && ox <= g.out_shape[0] - 1 && oy <= g.out_shape[1] - 1 &&
         oz <= g.out_shape[2] - 1;
}

// The input side of the neighbour query: the reference looks the input up at
// out * s - t (= in, or in * s for transposed) and keeps it only inside
// [0, shape) (conv.py:54-59, 180-188).
__device__ __forceinline__ bool input_in_bounds(const Geom& g, int64_t x, int64_t y, int64_t z) {
  return x >= 0 && y >= 0 && z >= 0 && x < g.in_shape[0] && y < g.in_shape[1] && z < g.in_shape[2];
}

// Rank of candidate (input i, offset k) in the enumeration order: offset
// chunks of `chunk` offsets in turn, inside a chunk input-major and offset-
// minor (the reference's chunk_size loop, kmap.py:270-278; one chunk is the
// plain input-major / offset-minor order).
__device__ __forceinline__ uint32_t cand_rank(const Geom& g, int64_t n, int64_t i, int k) {
  const int c = k / g.chunk;
  return (uint32_t)((int64_t)c * n * g.chunk + i * g.chunk + (k - c * g.chunk));
}

__device__ __forceinline__ void load_offsets(int32_t* off_s, const int32_t* __restrict__ offsets, int K) {
  for (int t = threadIdx.x; t < K * 3; t += blockDim.x) off_s[t] = offsets[t];
  __syncthreads();
}

inline bool make_geom(const st_outgeom* in, Geom& g) {
  if (!in || in->K <= 0 || in->K > ST_MAX_KVOL || in->stride < 1) return false;
  g.K = in->K;
  g.transposed = in->transposed ? 1 : 0;
  g.chunk = (in->chunk <= 0 || in->chunk >= in->K) ? in->K : (int)in->chunk;
  g.s = in->stride;
  g.s_log2 = -1;
  if ((g.s & (g.s - 1)) == 0)
    for (int l = 0; l < 63; ++l)
      if (g.s == (1ll << l)) g.s_log2 = l;
  for (int a = 0; a < 3; ++a) {
    g.in_shape[a] = in->in_shape[a];
    g.out_shape[a] = in->out_shape[a];
  }
  return true;
}

inline int64_t gcd64(int64_t a, int64_t b) {
  while (b) {
    int64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

// Candidates per input that can pass the stride filter: on each axis the
// offsets j*d hit one residue class mod s at most ceil(k / (s / gcd(d, s)))
// times.
inline int64_t cands_per_input(const Geom& g, int64_t kernel_size, int64_t dilation) {
  int64_t per_axis = kernel_size;
  if (!g.transposed && g.s > 1) {
    const int64_t period = g.s / gcd64(dilation, g.s);
    per_axis = (kernel_size + period - 1) / period;
  }
  const int64_t kv = per_axis * per_axis * per_axis;
  return kv > g.K ? g.K : kv;
}

}  // namespace st
