// Pooling and upsampling of sparse tensors (nn/functional/spatial.py:26-535).
//
// Pooling: input row r goes to the output cell
//   (b, floor((x + p - k/2) / s), floor((y + p - k/2) / s), floor((z + p - k/2) / s))
// (spatial.py:104-107); the output rows are the distinct cells in ascending
// (b, x, y, z) order (the reference's torch.unique over packed keys,
// :108-110) and each is the max or the mean of its rows (:54-73, :127-128).
// Here the cells are packed into order-preserving 64-bit keys, the rows sorted
// by key (hipCUB radix sort, stable, so a cell's rows stay in input order),
// and each output reduces its contiguous run of rows in that order -- no
// float atomics, so max and mean are deterministic.  The backward gives each
// row the gradient of its one output: all of it to every row equal to the max
// (as the reference's `in == out` test, :171-176), or 1/count of it (:177-178).
//
// Upsampling (spatial.py:236-436): input row r becomes rows r * s^3 + q,
// q = (dx * s + dy) * s + dz, at (b, x s + dx, y s + dy, z s + dz) with r's
// features; the backward sums each input's s^3 output gradients.
#include <hipcub/hipcub.hpp>

#include "common.h"

namespace st {

constexpr uint64_t kPoolInvalid = ~0ull;

__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t s) { return a >= 0 ? a / s : -((-a + s - 1) / s); }

// (b, x, y, z) -> key whose unsigned order is the lexicographic signed order;
// kPoolInvalid when b is outside [0, 32767] or a spatial value outside int16.
__device__ __forceinline__ uint64_t order_key(int64_t b, int64_t x, int64_t y, int64_t z) {
  if (b < 0 || b > 32767 || !in_i16(x) || !in_i16(y) || !in_i16(z)) return kPoolInvalid;
  return ((uint64_t)b << 48) | ((uint64_t)((uint16_t)x ^ 0x8000u) << 32) | ((uint64_t)((uint16_t)y ^ 0x8000u) << 16) |
         (uint64_t)((uint16_t)z ^ 0x8000u);
}

template <typename CT>
__global__ __launch_bounds__(256) void pool_keys_kernel(const CT* __restrict__ coords, int64_t n, int k, int s, int p,
                                                        uint64_t* __restrict__ keys, int32_t* __restrict__ rows,
                                                        int32_t* __restrict__ counts) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, r, b, x, y, z);
  const int64_t sh = p - k / 2;
  const uint64_t key = order_key(b, floor_div(x + sh, s), floor_div(y + sh, s), floor_div(z + sh, s));
  keys[r] = key;
  rows[r] = (int32_t)r;
  if (key == kPoolInvalid) atomicAdd(&counts[1], 1);
}

// flag[i] = 1 where sorted position i starts a run of equal valid keys
__global__ __launch_bounds__(256) void pool_heads_kernel(const uint64_t* __restrict__ skeys, int64_t n,
                                                         int32_t* __restrict__ flags) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint64_t k = skeys[i];
  flags[i] = (k != kPoolInvalid && (i == 0 || skeys[i - 1] != k)) ? 1 : 0;
}

// pos = exclusive prefix of the head flags: output o = pos[i] for a head i.
template <typename CT>
__global__ __launch_bounds__(256) void pool_emit_kernel(const uint64_t* __restrict__ skeys,
                                                        const int32_t* __restrict__ perm,
                                                        const int32_t* __restrict__ flags,
                                                        const int32_t* __restrict__ pos, int64_t n,
                                                        int32_t* __restrict__ seg_start, int32_t* __restrict__ inv,
                                                        CT* __restrict__ out_coords, int32_t* __restrict__ counts) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint64_t k = skeys[i];
  const int32_t o = pos[i] + flags[i] - 1;  // this position's output (valid keys)
  if (k == kPoolInvalid) {
    inv[perm[i]] = -1;
    if (i == 0 || skeys[i - 1] != kPoolInvalid) {
      seg_start[pos[i]] = (int32_t)i;  // the end of the last run
      counts[0] = pos[i];
    }
    return;
  }
  inv[perm[i]] = o;
  if (flags[i]) {
    seg_start[o] = (int32_t)i;
    CT* c = out_coords + (int64_t)o * 4;
    c[0] = (CT)(int64_t)(k >> 48);
    c[1] = (CT)(int16_t)(uint16_t)(((k >> 32) & 0xFFFFu) ^ 0x8000u);
    c[2] = (CT)(int16_t)(uint16_t)(((k >> 16) & 0xFFFFu) ^ 0x8000u);
    c[3] = (CT)(int16_t)(uint16_t)((k & 0xFFFFu) ^ 0x8000u);
  }
  if (i == n - 1) {
    seg_start[o + 1] = (int32_t)n;
    counts[0] = o + 1;
  }
}

template <typename T, int V>
__device__ __forceinline__ void ld(const T* __restrict__ p, float (&v)[V]) {
  if constexpr (V == 1) {
    v[0] = (float)p[0];
  } else {
    typedef T vt __attribute__((ext_vector_type(V)));
    const vt q = *reinterpret_cast<const vt*>(p);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = (float)q[e];
  }
}

template <typename T, int V>
__device__ __forceinline__ void st_(T* __restrict__ p, const float (&v)[V]) {
  if constexpr (V == 1) {
    p[0] = (T)v[0];
  } else {
    typedef T vt __attribute__((ext_vector_type(V)));
    vt q;
#pragma unroll
    for (int e = 0; e < V; ++e) q[e] = (T)v[e];
    *reinterpret_cast<vt*>(p) = q;
  }
}

// out[o] = max or mean of the rows perm[seg_start[o] .. seg_start[o+1]), in that order
template <typename T, int V, bool MAX>
__global__ __launch_bounds__(256) void pool_forward_kernel(const T* __restrict__ feats, int C,
                                                           const int32_t* __restrict__ perm,
                                                           const int32_t* __restrict__ seg_start, int64_t n_out,
                                                           T* __restrict__ out) {
  const int nv = C / V;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_out * nv) return;
  const int64_t o = i / nv;
  const int c = (int)(i - o * nv) * V;
  const int32_t s0 = seg_start[o], s1 = seg_start[o + 1];
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = MAX ? -INFINITY : 0.f;
  for (int32_t j = s0; j < s1; ++j) {
    float v[V];
    ld<T, V>(feats + (int64_t)perm[j] * C + c, v);
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] = MAX ? fmaxf(acc[e], v[e]) : acc[e] + v[e];
  }
  if (!MAX) {
    const float inv_cnt = 1.0f / (float)(s1 - s0);
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] *= inv_cnt;
  }
  st_<T, V>(out + o * C + c, acc);
}

template <typename T, int V, bool MAX>
__global__ __launch_bounds__(256) void pool_backward_kernel(const T* __restrict__ feats, const T* __restrict__ out,
                                                            const T* __restrict__ dout, int64_t n, int C,
                                                            const int32_t* __restrict__ inv,
                                                            const int32_t* __restrict__ seg_start,
                                                            T* __restrict__ dfeats) {
  const int nv = C / V;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * nv) return;
  const int64_t r = i / nv;
  const int c = (int)(i - r * nv) * V;
  const int32_t o = inv[r];
  float g[V];
  if (o < 0) {
#pragma unroll
    for (int e = 0; e < V; ++e) g[e] = 0.f;
  } else {
    ld<T, V>(dout + (int64_t)o * C + c, g);
    if (MAX) {
      float x[V], m[V];
      ld<T, V>(feats + r * C + c, x);
      ld<T, V>(out + (int64_t)o * C + c, m);
#pragma unroll
      for (int e = 0; e < V; ++e)
        if (x[e] != m[e]) g[e] = 0.f;
    } else {
      const float inv_cnt = 1.0f / (float)(seg_start[o + 1] - seg_start[o]);
#pragma unroll
      for (int e = 0; e < V; ++e) g[e] *= inv_cnt;
    }
  }
  st_<T, V>(dfeats + r * C + c, g);
}

// Upsampling: 16-byte feature vectors, 32-bit index arithmetic whenever the
// thread count allows (I = uint32_t; a 64-bit division costs ~100
// instructions), each child's coordinate row as one vector store.
template <typename CT>
__device__ __forceinline__ void store_coord4(CT* __restrict__ p, CT b, CT x, CT y, CT z) {
  typedef CT vt __attribute__((ext_vector_type(4)));
  vt q;
  q[0] = b;
  q[1] = x;
  q[2] = y;
  q[3] = z;
  *reinterpret_cast<vt*>(p) = q;
}

template <typename T, typename CT, int V, typename I>
__global__ __launch_bounds__(256) void upsample_kernel(const T* __restrict__ feats, const CT* __restrict__ coords,
                                                       int64_t n, int C, int s, T* __restrict__ out_feats,
                                                       CT* __restrict__ out_coords) {
  // thread per (input row, vector): the vector is read once and stored into each of the row's s^3
  // children -- for a given child the lanes of a row write one whole child row
  const I nv = (I)(C / V);
  const int s3 = s * s * s;
  const I i = (I)blockIdx.x * 256 + threadIdx.x;
  if ((int64_t)i >= n * (int64_t)nv) return;
  const I r = i / nv;
  const int c = (int)(i - r * nv) * V;
  float v[V];
  ld<T, V>(feats + (int64_t)r * C + c, v);
  T* o = out_feats + (int64_t)r * s3 * C + c;
  for (int q = 0; q < s3; ++q) st_<T, V>(o + (int64_t)q * C, v);
  if (c == 0) {
    const CT* ci = coords + (int64_t)r * 4;
    const CT b = ci[0];
    const int64_t x = (int64_t)ci[1] * s, y = (int64_t)ci[2] * s, z = (int64_t)ci[3] * s;
    CT* co = out_coords + (int64_t)r * s3 * 4;
    for (int q = 0; q < s3; ++q)
      store_coord4<CT>(co + 4 * q, b, (CT)(x + q / (s * s)), (CT)(y + (q / s) % s), (CT)(z + q % s));
  }
}

template <typename T, int V, typename I>
__global__ __launch_bounds__(256) void upsample_backward_kernel(const T* __restrict__ dout, int64_t n, int C, int s,
                                                                T* __restrict__ dfeats) {
  const I nv = (I)(C / V);
  const int s3 = s * s * s;
  const I i = (I)blockIdx.x * 256 + threadIdx.x;
  if ((int64_t)i >= n * (int64_t)nv) return;
  const I r = i / nv;
  const int c = (int)(i - r * nv) * V;
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e) acc[e] = 0.f;
  for (int q = 0; q < s3; ++q) {
    float v[V];
    ld<T, V>(dout + ((int64_t)r * s3 + q) * C + c, v);
#pragma unroll
    for (int e = 0; e < V; ++e) acc[e] += v[e];
  }
  st_<T, V>(dfeats + (int64_t)r * C + c, acc);
}

// Workspace: keys, sorted keys (8 n bytes each), rows, sorted rows (perm is
// the caller's), flags and positions (4 (n + 1) bytes each), then hipCUB's
// temporary storage.
struct PoolWs {
  uint64_t *keys, *skeys;
  int32_t *rows, *flags, *pos;
  void* tmp;
  size_t tmp_bytes;
};
static size_t align256(size_t b) { return (b + 255) / 256 * 256; }
static int pool_tmp_bytes(int64_t n, size_t* bytes) {
  size_t a = 0, b = 0;
  if (hipcub::DeviceRadixSort::SortPairs(nullptr, a, (const uint64_t*)nullptr, (uint64_t*)nullptr,
                                         (const int32_t*)nullptr, (int32_t*)nullptr, (int)n) != hipSuccess)
    return ST_ERR_HIP;
  if (hipcub::DeviceScan::ExclusiveSum(nullptr, b, (const int32_t*)nullptr, (int32_t*)nullptr, (int)n) !=
      hipSuccess)
    return ST_ERR_HIP;
  *bytes = a > b ? a : b;
  return ST_OK;
}
static size_t pool_fixed_bytes(int64_t n) {
  return 2 * align256(8 * (size_t)n) + 3 * align256(4 * (size_t)(n + 1));
}
static PoolWs pool_carve(void* ws, int64_t n, size_t tmp_bytes) {
  PoolWs w;
  char* p = (char*)ws;
  w.keys = (uint64_t*)p;
  p += align256(8 * (size_t)n);
  w.skeys = (uint64_t*)p;
  p += align256(8 * (size_t)n);
  w.rows = (int32_t*)p;
  p += align256(4 * (size_t)(n + 1));
  w.flags = (int32_t*)p;
  p += align256(4 * (size_t)(n + 1));
  w.pos = (int32_t*)p;
  p += align256(4 * (size_t)(n + 1));
  w.tmp = p;
  w.tmp_bytes = tmp_bytes;
  return w;
}

static bool vec4_ok(int C, const void* a, const void* b, const void* c = nullptr, const void* d = nullptr) {
  return C % 4 == 0 && (uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0 && (uintptr_t)c % 16 == 0 &&
         (uintptr_t)d % 16 == 0;
}

template <typename T>
static void launch_pool_backward(const T* feats, const T* out, const T* dout, int64_t n, int C, const int32_t* inv,
                                 const int32_t* seg_start, int mode, bool v4, T* dfeats, hipStream_t stream) {
  const unsigned g = st_blocks(n * (C / (v4 ? 4 : 1)), 256);
  if (mode == 0) {
    if (v4)
      pool_backward_kernel<T, 4, true><<<g, 256, 0, stream>>>(feats, out, dout, n, C, inv, seg_start, dfeats);
    else
      pool_backward_kernel<T, 1, true><<<g, 256, 0, stream>>>(feats, out, dout, n, C, inv, seg_start, dfeats);
  } else {
    if (v4)
      pool_backward_kernel<T, 4, false><<<g, 256, 0, stream>>>(feats, out, dout, n, C, inv, seg_start, dfeats);
    else
      pool_backward_kernel<T, 1, false><<<g, 256, 0, stream>>>(feats, out, dout, n, C, inv, seg_start, dfeats);
  }
}

}  // namespace st

using namespace st;

#define ST_SP_DISPATCH(dt, T, ...) \
  switch (dt) {                    \
    case ST_F32:                   \
    case ST_F32_BF16X3: {          \
      using T = float;             \
      __VA_ARGS__;                 \
      break;                       \
    }                              \
    case ST_F16: {                 \
      using T = _Float16;          \
      __VA_ARGS__;                 \
      break;                       \
    }                              \
    case ST_BF16: {                \
      using T = __bf16;            \
      __VA_ARGS__;                 \
      break;                       \
    }                              \
    default:                       \
      return ST_ERR_UNSUPPORTED;   \
  }

extern "C" {

int st_pool_workspace(int64_t n, size_t* bytes) {
  if (n < 0 || n >= (1ll << 31) - 1 || !bytes) return ST_ERR_ARG;
  size_t tmp = 0;
  const int rc = pool_tmp_bytes(n > 0 ? n : 1, &tmp);
  if (rc != ST_OK) return rc;
  *bytes = pool_fixed_bytes(n > 0 ? n : 1) + tmp;
  return ST_OK;
}

int st_pool_plan(const void* coords, int coord_dtype, int64_t n, int kernel_size, int stride, int padding,
                 void* workspace, size_t workspace_bytes, int32_t* perm, int32_t* seg_start, int32_t* inv,
                 void* out_coords, int32_t* counts, st_stream_t stream) {
  if (n < 0 || n >= (1ll << 31) - 1 || kernel_size < 1 || stride < 1 || !counts) return ST_ERR_ARG;
  int rc = st_fill_u32((uint32_t*)counts, 2, 0u, stream);
  if (rc != ST_OK || n == 0) return rc;
  if (!coords || !workspace || !perm || !seg_start || !inv || !out_coords) return ST_ERR_ARG;
  size_t tmp = 0;
  rc = pool_tmp_bytes(n, &tmp);
  if (rc != ST_OK) return rc;
  if (workspace_bytes < pool_fixed_bytes(n) + tmp) return ST_ERR_ARG;
  const PoolWs w = pool_carve(workspace, n, tmp);
  const unsigned g = st_blocks(n, 256);
  ST_DISPATCH_COORD(coord_dtype, CT, {
    pool_keys_kernel<CT><<<g, 256, 0, stream>>>((const CT*)coords, n, kernel_size, stride, padding, w.keys, w.rows,
                                                counts);
    size_t tb = w.tmp_bytes;
    ST_CHECK_HIP(hipcub::DeviceRadixSort::SortPairs(w.tmp, tb, w.keys, w.skeys, w.rows, perm, (int)n, 0, 64,
                                                    stream));
    pool_heads_kernel<<<g, 256, 0, stream>>>(w.skeys, n, w.flags);
    tb = w.tmp_bytes;
    ST_CHECK_HIP(hipcub::DeviceScan::ExclusiveSum(w.tmp, tb, w.flags, w.pos, (int)n, stream));
    pool_emit_kernel<CT><<<g, 256, 0, stream>>>(w.skeys, perm, w.flags, w.pos, n, seg_start, inv, (CT*)out_coords,
                                                counts);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_pool_forward(const void* feats, int C, int dtype, const int32_t* perm, const int32_t* seg_start, int64_t n_out,
                    int mode, void* out, st_stream_t stream) {
  if (C <= 0 || n_out < 0 || (mode != 0 && mode != 1)) return ST_ERR_ARG;
  if (n_out == 0) return ST_OK;
  if (!feats || !perm || !seg_start || !out) return ST_ERR_ARG;
  const bool v4 = vec4_ok(C, feats, out);
  ST_SP_DISPATCH(dtype, T, {
    const int V = v4 ? 4 : 1;
    const unsigned g = st_blocks(n_out * (C / V), 256);
    if (mode == 0) {
      if (v4)
        pool_forward_kernel<T, 4, true><<<g, 256, 0, stream>>>((const T*)feats, C, perm, seg_start, n_out, (T*)out);
      else
        pool_forward_kernel<T, 1, true><<<g, 256, 0, stream>>>((const T*)feats, C, perm, seg_start, n_out, (T*)out);
    } else {
      if (v4)
        pool_forward_kernel<T, 4, false><<<g, 256, 0, stream>>>((const T*)feats, C, perm, seg_start, n_out, (T*)out);
      else
        pool_forward_kernel<T, 1, false><<<g, 256, 0, stream>>>((const T*)feats, C, perm, seg_start, n_out, (T*)out);
    }
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_pool_backward(const void* feats, const void* out, const void* dout, int64_t n, int C, int dtype,
                     const int32_t* inv, const int32_t* seg_start, int mode, void* dfeats, st_stream_t stream) {
  if (n < 0 || C <= 0 || (mode != 0 && mode != 1)) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!dout || !inv || !seg_start || !dfeats || (mode == 0 && (!feats || !out))) return ST_ERR_ARG;
  const bool v4 = vec4_ok(C, dout, dfeats, feats, out);
  ST_SP_DISPATCH(dtype, T,
                 launch_pool_backward<T>((const T*)feats, (const T*)out, (const T*)dout, n, C, inv, seg_start, mode,
                                         v4, (T*)dfeats, stream));
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_upsample(const void* feats, const void* coords, int coord_dtype, int64_t n, int C, int dtype, int scale,
                void* out_feats, void* out_coords, st_stream_t stream) {
  if (n < 0 || C <= 0 || scale < 1) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!feats || !coords || !out_feats || !out_coords) return ST_ERR_ARG;
  const int64_t s3 = (int64_t)scale * scale * scale;
  ST_DISPATCH_COORD(coord_dtype, CT, {
    ST_SP_DISPATCH(dtype, T, {
      constexpr int V = 16 / (int)sizeof(T);  // one 16-byte vector
      const bool vec = C % V == 0 && (uintptr_t)feats % 16 == 0 && (uintptr_t)out_feats % 16 == 0;
      const int64_t threads = n * (vec ? C / V : C);  // (input row, vector) pairs
      const unsigned g = st_blocks(threads, 256);
      const bool w32 = threads + 256 < (1ll << 32);
      if (vec && w32)
        upsample_kernel<T, CT, V, uint32_t><<<g, 256, 0, stream>>>((const T*)feats, (const CT*)coords, n, C, scale,
                                                                   (T*)out_feats, (CT*)out_coords);
      else if (vec)
        upsample_kernel<T, CT, V, int64_t><<<g, 256, 0, stream>>>((const T*)feats, (const CT*)coords, n, C, scale,
                                                                  (T*)out_feats, (CT*)out_coords);
      else if (w32)
        upsample_kernel<T, CT, 1, uint32_t><<<g, 256, 0, stream>>>((const T*)feats, (const CT*)coords, n, C, scale,
                                                                   (T*)out_feats, (CT*)out_coords);
      else
        upsample_kernel<T, CT, 1, int64_t><<<g, 256, 0, stream>>>((const T*)feats, (const CT*)coords, n, C, scale,
                                                                  (T*)out_feats, (CT*)out_coords);
    });
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_upsample_backward(const void* dout, int64_t n, int C, int dtype, int scale, void* dfeats, st_stream_t stream) {
  if (n < 0 || C <= 0 || scale < 1) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!dout || !dfeats) return ST_ERR_ARG;
  ST_SP_DISPATCH(dtype, T, {
    constexpr int V = 16 / (int)sizeof(T);  // one 16-byte vector
    const bool vec = C % V == 0 && (uintptr_t)dout % 16 == 0 && (uintptr_t)dfeats % 16 == 0;
    const int64_t threads = n * (vec ? C / V : C);
    const unsigned g = st_blocks(threads, 256);
    const bool w32 = threads + 256 < (1ll << 32);
    if (vec && w32)
      upsample_backward_kernel<T, V, uint32_t><<<g, 256, 0, stream>>>((const T*)dout, n, C, scale, (T*)dfeats);
    else if (vec)
      upsample_backward_kernel<T, V, int64_t><<<g, 256, 0, stream>>>((const T*)dout, n, C, scale, (T*)dfeats);
    else if (w32)
      upsample_backward_kernel<T, 1, uint32_t><<<g, 256, 0, stream>>>((const T*)dout, n, C, scale, (T*)dfeats);
    else
      upsample_backward_kernel<T, 1, int64_t><<<g, 256, 0, stream>>>((const T*)dout, n, C, scale, (T*)dfeats);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // extern "C"
