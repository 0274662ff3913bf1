// Coordinate hash table (insert / query) and the query-built kernel map.
//
// Table layout in HBM: two flat arrays of `cap` slots, keys (u64 packed
// coordinate) and vals (u32 row index).  Both are all-ones when empty, so a
// single fill clears them.  A query touches one 128-byte key line per probe
// plus one value word on a hit; at the load factor this package builds
// (<= 0.5) a hit takes ~1.5 probes and a miss ~2.5 on average.
#include "common.h"

#include <atomic>

namespace st {

template <typename T>
__global__ void fill_kernel(T* __restrict__ dst, int64_t n, T value) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += step) dst[i] = value;
}

// Row of an inserted key: the thread whose CAS claimed the slot stores its row
// with a plain store (one atomic per row instead of two, on unique rows); a
// repeated key counts in the status and takes the atomic-min, which
// hash_insert_fixup_kernel completes after the insert.
__device__ __forceinline__ void store_row(uint32_t* __restrict__ vals, uint32_t s, uint32_t row, bool was_new,
                                          int32_t* __restrict__ status) {
  if (was_new) {
    vals[s] = row;
  } else {
    atomicAdd(&status[ST_STATUS_DUPLICATE], 1);
    atomicMin(&vals[s], row);
  }
}

// insert_slot that claims by CAS at once instead of loading the slot first:
// one memory round trip less per row on a mostly empty table, a CAS on every
// occupied slot it passes (config 2, table at the default capacity: clear +
// insert 53.3 -> 50.4 us)
__device__ __forceinline__ uint32_t insert_slot_cas(uint64_t* __restrict__ keys, uint32_t cap, uint64_t key,
                                                    bool& was_new) {
  uint32_t s = home_slot(key, cap);
  for (uint32_t step = 0; step < cap; ++step) {
    const unsigned long long old =
        atomicCAS((unsigned long long*)&keys[s], (unsigned long long)ST_EMPTY_KEY, (unsigned long long)key);
    if (old == ST_EMPTY_KEY || old == key) {
      was_new = old == ST_EMPTY_KEY;
      return s;
    }
    s = next_slot(s, cap);
  }
  return ST_NO_VAL;
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
  uint32_t s = insert_slot_cas(keys, cap, key, was_new);
  if (s == ST_NO_VAL) {
    atomicAdd(&status[ST_STATUS_OVERFLOW], 1);
    return;
  }
  store_row(vals, s, (uint32_t)i, was_new, status);
}

// Repeated keys of an insert: the row stored by each key's slot winner may
// have landed after a smaller row's atomic-min, so when the status counts any
// repeat every row takes the atomic-min once more (probes read-only, the
// table is complete); otherwise each workgroup reads one word and returns.
template <typename CT>
__global__ __launch_bounds__(256) void hash_insert_fixup_kernel(const CT* __restrict__ coords, int64_t n,
                                                                int64_t scale, const uint64_t* __restrict__ keys,
                                                                uint32_t* __restrict__ vals, uint32_t cap,
                                                                const int32_t* __restrict__ status) {
  if (status[ST_STATUS_DUPLICATE] == 0) return;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t b, x, y, z;
    load_coord(coords, i, b, x, y, z);
    uint64_t key;
    if (!pack_key(b, x * scale, y * scale, z * scale, key)) continue;
    const uint32_t s = find_slot(keys, cap, key);
    if (s != ST_NO_VAL) atomicMin(&vals[s], (uint32_t)i);
  }
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

// ---------------------------------------------- wave-cooperative probing
//
// The alternative probe the hot-path description asks to be measured: a
// group of 16 lanes serves one key, lane j loading slot s + j of the current
// 16-slot window (one 128-byte line of keys when aligned), and one ballot
// finds the first matching or empty slot in probe order -- the same answers
// and the same table as the per-thread linear probe above.  Selected with
// ST_HASH_PROBE=wave for timing; the per-thread probe is the default because
// it measured faster (a wave then serves 64 keys with up to 9 probes of
// each row in flight, against 4 keys per wave here).
constexpr int kGroup = 16;

__device__ __forceinline__ uint32_t wrap_slot(uint64_t s, uint32_t cap) { return (uint32_t)(s % cap); }

// Bits of this lane's 16-lane group in a wave ballot.
__device__ __forceinline__ uint32_t group_bits(uint64_t ballot) {
  return (uint32_t)((ballot >> ((threadIdx.x & 63) & ~(kGroup - 1))) & 0xFFFFu);
}

// Lookup by a 16-lane group (all lanes hold the same key).
__device__ __forceinline__ uint32_t find_slot_group(const uint64_t* __restrict__ keys, uint32_t cap, uint64_t key) {
  const int j = threadIdx.x & (kGroup - 1);
  uint32_t s = home_slot(key, cap);
  for (uint32_t seen = 0; seen < cap; seen += kGroup) {
    const uint64_t k = keys[wrap_slot((uint64_t)s + j, cap)];
    const uint32_t m = group_bits(__ballot(k == key)), e = group_bits(__ballot(k == ST_EMPTY_KEY));
    if (m && (!e || __builtin_ctz(m) < __builtin_ctz(e))) return wrap_slot((uint64_t)s + __builtin_ctz(m), cap);
    if (e) return ST_NO_VAL;
    s = wrap_slot((uint64_t)s + kGroup, cap);
  }
  return ST_NO_VAL;
}

// Insert-or-find by a 16-lane group: the lowest lane whose slot holds the key
// or is empty decides; an empty slot is claimed by that lane's CAS, and a CAS
// lost to another key resumes the scan at that slot.
__device__ __forceinline__ uint32_t insert_slot_group(uint64_t* __restrict__ keys, uint32_t cap, uint64_t key,
                                                      bool& was_new) {
  const int lane = threadIdx.x & 63, j = lane & (kGroup - 1), base = lane & ~(kGroup - 1);
  uint32_t s = home_slot(key, cap);
  for (uint32_t seen = 0; seen < cap;) {
    const uint32_t sj = wrap_slot((uint64_t)s + j, cap);
    const uint64_t k = keys[sj];
    const uint32_t hit = group_bits(__ballot(k == key || k == ST_EMPTY_KEY));
    if (!hit) {
      s = wrap_slot((uint64_t)s + kGroup, cap);
      seen += kGroup;
      continue;
    }
    const int f = __builtin_ctz(hit);
    unsigned long long old = (unsigned long long)key;
    if (j == f && k == ST_EMPTY_KEY)
      old = atomicCAS((unsigned long long*)&keys[sj], (unsigned long long)ST_EMPTY_KEY, (unsigned long long)key);
    old = __shfl(old, base + f, 64);
    const uint32_t slot = wrap_slot((uint64_t)s + f, cap);
    if (old == ST_EMPTY_KEY) {
      was_new = true;
      return slot;
    }
    if (old == key) {
      was_new = false;
      return slot;
    }
    s = slot;  // lost the slot to another key: rescan from it
    seen += f;
  }
  return ST_NO_VAL;
}

// One 16-lane group per row; the group's lane 0 records the result.
template <typename CT>
__global__ __launch_bounds__(256) void hash_insert_group_kernel(const CT* __restrict__ coords, int64_t n,
                                                                int64_t scale, uint64_t* __restrict__ keys,
                                                                uint32_t* __restrict__ vals, uint32_t cap,
                                                                int32_t* __restrict__ status) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kGroup;
  const bool lead = (threadIdx.x & (kGroup - 1)) == 0;
  if (i >= n) return;  // (whole groups: n rows take n * 16 threads)
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  uint64_t key;
  if (!pack_key(b, x * scale, y * scale, z * scale, key)) {
    if (lead) atomicAdd(&status[ST_STATUS_BAD_COORD], 1);
    return;
  }
  bool was_new = false;
  const uint32_t s = insert_slot_group(keys, cap, key, was_new);
  if (!lead) return;
  if (s == ST_NO_VAL) {
    atomicAdd(&status[ST_STATUS_OVERFLOW], 1);
    return;
  }
  store_row(vals, s, (uint32_t)i, was_new, status);
}

template <typename CT>
__global__ __launch_bounds__(256) void hash_query_group_kernel(const CT* __restrict__ coords, int64_t m,
                                                               const uint64_t* __restrict__ keys,
                                                               const uint32_t* __restrict__ vals, uint32_t cap,
                                                               int32_t* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kGroup;
  if (i >= m) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  uint64_t key;
  int32_t r = -1;
  if (pack_key(b, x, y, z, key)) {
    const uint32_t s = find_slot_group(keys, cap, key);
    if (s != ST_NO_VAL) r = (int32_t)vals[s];
  }
  if ((threadIdx.x & (kGroup - 1)) == 0) out[i] = r;
}

// kmap_query_kernel with a 16-lane group per output row, its offsets in turn.
template <typename CT>
__global__ __launch_bounds__(256) void kmap_query_group_kernel(const CT* __restrict__ out_coords, int64_t n_out,
                                                               const int32_t* __restrict__ offsets, int K,
                                                               int64_t stride, int64_t sx, int64_t sy, int64_t sz,
                                                               const uint64_t* __restrict__ keys,
                                                               const uint32_t* __restrict__ vals, uint32_t cap,
                                                               int32_t* __restrict__ nbr, int64_t ks, int64_t rs,
                                                               uint32_t* __restrict__ row_masks,
                                                               int32_t* __restrict__ status) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  for (int t = threadIdx.x; t < K * 3; t += blockDim.x) off_s[t] = offsets[t];
  __syncthreads();
  const int64_t o = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kGroup;
  const bool lead = (threadIdx.x & (kGroup - 1)) == 0;
  if (o >= n_out) return;
  int64_t b, x, y, z;
  load_coord(out_coords, o, b, x, y, z);
  x *= stride;
  y *= stride;
  z *= stride;
  if (lead && status && (x < 0 || x >= sx || y < 0 || y >= sy || z < 0 || z >= sz))
    atomicAdd(&status[ST_STATUS_OUT_OF_BOX], 1);
  const int W = (K + 31) >> 5;
  uint32_t mword = 0;
  for (int k = 0; k < K; ++k) {
    const int64_t qx = x - off_s[3 * k], qy = y - off_s[3 * k + 1], qz = z - off_s[3 * k + 2];
    uint64_t key;
    int32_t r = -1;
    if (qx >= 0 && qx < sx && qy >= 0 && qy < sy && qz >= 0 && qz < sz && pack_key(b, qx, qy, qz, key)) {
      const uint32_t s = find_slot_group(keys, cap, key);
      if (s != ST_NO_VAL) r = (int32_t)vals[s];
    }
    if (lead) nbr[(int64_t)k * ks + o * rs] = r;
    if (r >= 0) mword |= 1u << (k & 31);
    if ((k & 31) == 31 || k == K - 1) {
      if (lead && row_masks) row_masks[o * W + (k >> 5)] = mword;
      mword = 0;
    }
  }
}

// 0 = per-thread probes, 1 = 16-lane group probes; set by st_hash_probe_mode (or, before the
// first call, ST_HASH_PROBE=wave).
static std::atomic<int> g_probe_mode{-1};
static bool group_probe() {
  int m = g_probe_mode.load(std::memory_order_relaxed);
  if (m < 0) {
    const char* e = getenv("ST_HASH_PROBE");
    m = (e && e[0] == 'w') ? 1 : 0;
    int expect = -1;
    g_probe_mode.compare_exchange_strong(expect, m);
    m = g_probe_mode.load(std::memory_order_relaxed);
  }
  return m == 1;
}

static unsigned group_blocks(int64_t rows) { return (unsigned)((rows * kGroup + 255) / 256); }

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

int st_hash_probe_mode(int mode) {
  const int prev = group_probe() ? 1 : 0;
  if (mode == 0 || mode == 1) g_probe_mode.store(mode, std::memory_order_relaxed);
  return prev;
}

int st_hash_insert(const void* coords, int coord_dtype, int64_t n, int64_t scale, uint64_t* keys, uint32_t* vals,
                   int64_t capacity, int32_t* status, st_stream_t stream) {
  if (n < 0 || capacity <= 0 || capacity >= (1ll << 31) || scale < 1 || !keys || !vals || !status)
    return ST_ERR_ARG;
  if (n > 0 && !coords) return ST_ERR_ARG;
  if (n >= (1ll << 31)) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (group_probe()) {
    ST_DISPATCH_COORD(coord_dtype, CT,
                      hash_insert_group_kernel<CT><<<group_blocks(n), 256, 0, stream>>>(
                          (const CT*)coords, n, scale, keys, vals, (uint32_t)capacity, status));
  } else {
    ST_DISPATCH_COORD(coord_dtype, CT,
                      hash_insert_kernel<CT><<<st_blocks(n, 256), 256, 0, stream>>>(
                          (const CT*)coords, n, scale, keys, vals, (uint32_t)capacity, status));
  }
  const unsigned fg = st_blocks(n, 256) < 256 ? st_blocks(n, 256) : 256;
  ST_DISPATCH_COORD(coord_dtype, CT,
                    hash_insert_fixup_kernel<CT><<<fg, 256, 0, stream>>>((const CT*)coords, n, scale, keys, vals,
                                                                         (uint32_t)capacity, status));
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_hash_query(const void* coords, int coord_dtype, int64_t m, const uint64_t* keys, const uint32_t* vals,
                  int64_t capacity, int32_t* out, st_stream_t stream) {
  if (m < 0 || capacity <= 0 || capacity >= (1ll << 31) || !keys || !vals) return ST_ERR_ARG;
  if (m > 0 && (!coords || !out)) return ST_ERR_ARG;
  if (m == 0) return ST_OK;
  if (group_probe()) {
    ST_DISPATCH_COORD(coord_dtype, CT,
                      hash_query_group_kernel<CT><<<group_blocks(m), 256, 0, stream>>>(
                          (const CT*)coords, m, keys, vals, (uint32_t)capacity, out));
  } else {
    ST_DISPATCH_COORD(coord_dtype, CT,
                      hash_query_kernel<CT><<<st_blocks(m, 256), 256, 0, stream>>>(
                          (const CT*)coords, m, keys, vals, (uint32_t)capacity, out));
  }
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
  if (group_probe()) {
    ST_DISPATCH_COORD(coord_dtype, CT,
                      kmap_query_group_kernel<CT><<<group_blocks(n_out), 256, 0, stream>>>(
                          (const CT*)out_coords, n_out, offsets, K, stride, shape_x, shape_y, shape_z, keys, vals,
                          (uint32_t)capacity, nbr, nbr_k_stride, nbr_r_stride, row_masks, status));
  } else {
    ST_DISPATCH_COORD(coord_dtype, CT,
                      kmap_query_kernel<CT><<<st_blocks(n_out, 256), 256, 0, stream>>>(
                          (const CT*)out_coords, n_out, offsets, K, stride, shape_x, shape_y, shape_z, keys, vals,
                          (uint32_t)capacity, nbr, nbr_k_stride, nbr_r_stride, row_masks, status));
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // extern "C"
