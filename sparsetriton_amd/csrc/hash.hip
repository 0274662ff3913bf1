// Coordinate hash table (insert / query) and the query-built kernel map.
//
// Table layout in HBM: two flat arrays of `cap` slots, keys (u64 packed
// coordinate) and vals (u32 row index).  Both are all-ones when empty, so a
// single fill clears them.  A query touches one 128-byte key line per probe
// plus one value word on a hit; at the load factor this package builds
// (<= 0.5) a hit takes ~1.5 probes and a miss ~2.5 on average.
#include "common.h"

namespace st {

template <typename T>
__global__ void fill_kernel(T* __restrict__ dst, int64_t n, T value) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += step) dst[i] = value;
}

// One thread per coordinate row (utils/hash.py:203-258 restated with exact keys).
template <typename CT>
__global__ __launch_bounds__(256) void hash_insert_kernel(const CT* __restrict__ coords, int64_t n, int64_t scale,
                                                          uint64_t* __restrict__ keys, uint32_t* __restrict__ vals,
                                                          uint32_t cap, int32_t* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  uint64_t key;
  if (!pack_key(b, x * scale, y * scale, z * scale, key)) {
    atomicAdd(&status[ST_STATUS_BAD_COORD], 1);
    return;
  }
  bool was_new = false;
  uint32_t s = insert_slot(keys, cap, key, was_new);
  if (s == ST_NO_VAL) {
    atomicAdd(&status[ST_STATUS_OVERFLOW], 1);
    return;
  }
  if (!was_new) atomicAdd(&status[ST_STATUS_DUPLICATE], 1);
  atomicMin(&vals[s], (uint32_t)i);
}

template <typename CT>
__global__ __launch_bounds__(256) void hash_query_kernel(const CT* __restrict__ coords, int64_t m,
                                                         const uint64_t* __restrict__ keys,
                                                         const uint32_t* __restrict__ vals, uint32_t cap,
                                                         int32_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  uint64_t key;
  int32_t r = -1;
  if (pack_key(b, x, y, z, key)) {
    uint32_t s = find_slot(keys, cap, key);
    if (s != ST_NO_VAL) r = (int32_t)vals[s];
  }
  out[i] = r;
}

// Kernel map by query (conv.py:12-75) through the hash table.  One thread per
// output row walks all K offsets; consecutive threads own consecutive rows, so
// each offset's column of the offset-major map is written with coalesced
// stores.  Offsets live in LDS (K <= ST_MAX_KVOL).
//
// A row's queries are independent, so they are resolved kQGroup at a time:
// the home-slot keys of all of them are loaded together, only a probe that
// meets another key at its home slot continues its chain on its own, then the
// values of the hits are loaded together.  (A submanifold map over the
// table's own coordinates takes st_kmap_subm's brick index instead.)
constexpr int kQGroup = 9;

template <typename CT>
__global__ __launch_bounds__(256) void kmap_query_kernel(const CT* __restrict__ out_coords, int64_t n_out,
                                                         const int32_t* __restrict__ offsets, int K, int64_t stride,
                                                         int64_t sx, int64_t sy, int64_t sz,
                                                         const uint64_t* __restrict__ keys,
                                                         const uint32_t* __restrict__ vals, uint32_t cap,
                                                         int32_t* __restrict__ nbr, int64_t ks, int64_t rs,
                                                         uint32_t* __restrict__ row_masks,
                                                         int32_t* __restrict__ status) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  for (int t = threadIdx.x; t < K * 3; t += blockDim.x) off_s[t] = offsets[t];
  __syncthreads();
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_out) return;
  int64_t b, x, y, z;
  load_coord(out_coords, o, b, x, y, z);
  x *= stride;
  y *= stride;
  z *= stride;
  // rows outside the bounds still get their in-bounds neighbours, but no row finds them
  // as a neighbour: the map is then not its own transpose (the caller's status tells it)
  if (status && (x < 0 || x >= sx || y < 0 || y >= sy || z < 0 || z >= sz))
    atomicAdd(&status[ST_STATUS_OUT_OF_BOX], 1);
  const int W = (K + 31) >> 5;
  uint32_t mword = 0;
  for (int k0 = 0; k0 < K; k0 += kQGroup) {
    uint64_t key[kQGroup];
    uint32_t slot[kQGroup];
    uint64_t hk[kQGroup];
#pragma unroll
    for (int j = 0; j < kQGroup; ++j) {
      const int k = k0 + j;
      bool probe = false;
      key[j] = 0;
      if (k < K) {
        const int64_t qx = x - off_s[3 * k], qy = y - off_s[3 * k + 1], qz = z - off_s[3 * k + 2];
        probe = qx >= 0 && qx < sx && qy >= 0 && qy < sy && qz >= 0 && qz < sz && pack_key(b, qx, qy, qz, key[j]);
      }
      slot[j] = probe ? home_slot(key[j], cap) : ST_NO_VAL;
      hk[j] = probe ? keys[slot[j]] : ST_EMPTY_KEY;
    }
    int32_t r[kQGroup];
#pragma unroll
    for (int j = 0; j < kQGroup; ++j) {
      if (slot[j] != ST_NO_VAL) slot[j] = find_slot_from(keys, cap, key[j], slot[j], hk[j]);
      r[j] = slot[j] != ST_NO_VAL ? (int32_t)vals[slot[j]] : -1;
    }
#pragma unroll
    for (int j = 0; j < kQGroup; ++j) {
      const int k = k0 + j;
      if (k < K) {
        nbr[(int64_t)k * ks + o * rs] = r[j];
        if (r[j] >= 0) mword |= 1u << (k & 31);
        if ((k & 31) == 31 || k == K - 1) {
          if (row_masks) row_masks[o * W + (k >> 5)] = mword;
          mword = 0;
        }
      }
    }
  }
}

}  // namespace st

using namespace st;

extern "C" {

const char* st_version(void) { return "sparsetriton_amd 0.1 gfx950"; }

int st_fill_u32(uint32_t* dst, int64_t n, uint32_t value, st_stream_t stream) {
  if (n < 0 || (n > 0 && !dst)) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  unsigned g = st_blocks(n, 256);
  if (g > 65536) g = 65536;
  fill_kernel<uint32_t><<<g, 256, 0, stream>>>(dst, n, value);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_fill_u64(uint64_t* dst, int64_t n, uint64_t value, st_stream_t stream) {
  if (n < 0 || (n > 0 && !dst)) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  unsigned g = st_blocks(n, 256);
  if (g > 65536) g = 65536;
  fill_kernel<uint64_t><<<g, 256, 0, stream>>>(dst, n, value);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_hash_insert(const void* coords, int coord_dtype, int64_t n, int64_t scale, uint64_t* keys, uint32_t* vals,
                   int64_t capacity, int32_t* status, st_stream_t stream) {
  if (n < 0 || capacity <= 0 || capacity >= (1ll << 31) || scale < 1 || !keys || !vals || !status)
    return ST_ERR_ARG;
  if (n > 0 && !coords) return ST_ERR_ARG;
  if (n >= (1ll << 31)) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  ST_DISPATCH_COORD(coord_dtype, CT,
                    hash_insert_kernel<CT><<<st_blocks(n, 256), 256, 0, stream>>>(
                        (const CT*)coords, n, scale, keys, vals, (uint32_t)capacity, status));
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_hash_query(const void* coords, int coord_dtype, int64_t m, const uint64_t* keys, const uint32_t* vals,
                  int64_t capacity, int32_t* out, st_stream_t stream) {
  if (m < 0 || capacity <= 0 || capacity >= (1ll << 31) || !keys || !vals) return ST_ERR_ARG;
  if (m > 0 && (!coords || !out)) return ST_ERR_ARG;
  if (m == 0) return ST_OK;
  ST_DISPATCH_COORD(coord_dtype, CT,
                    hash_query_kernel<CT><<<st_blocks(m, 256), 256, 0, stream>>>(
                        (const CT*)coords, m, keys, vals, (uint32_t)capacity, out));
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_kmap_query(const void* out_coords, int coord_dtype, int64_t n_out, const int32_t* offsets, int K,
                  int64_t stride, int64_t shape_x, int64_t shape_y, int64_t shape_z, const uint64_t* keys,
                  const uint32_t* vals, int64_t capacity, int32_t* nbr, int64_t nbr_k_stride, int64_t nbr_r_stride,
                  uint32_t* row_masks, int32_t* status, st_stream_t stream) {
  if (n_out < 0 || K <= 0 || K > ST_MAX_KVOL || stride < 1 || capacity <= 0 || capacity >= (1ll << 31))
    return ST_ERR_ARG;
  if (n_out >= (1ll << 31)) return ST_ERR_ARG;
  if (n_out == 0) return ST_OK;
  if (!out_coords || !offsets || !nbr || !keys || !vals) return ST_ERR_ARG;
  ST_DISPATCH_COORD(coord_dtype, CT,
                    kmap_query_kernel<CT><<<st_blocks(n_out, 256), 256, 0, stream>>>(
                        (const CT*)out_coords, n_out, offsets, K, stride, shape_x, shape_y, shape_z, keys, vals,
                        (uint32_t)capacity, nbr, nbr_k_stride, nbr_r_stride, row_masks, status));
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // extern "C"
