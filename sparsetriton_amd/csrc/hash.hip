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
__device__ __forceinline__ uint32_t insert_slot_cas_from(uint64_t* __restrict__ keys, uint32_t cap, uint64_t key,
                                                         uint32_t s, bool& was_new) {
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
__device__ __forceinline__ uint32_t insert_slot_cas(uint64_t* __restrict__ keys, uint32_t cap, uint64_t key,
                                                    bool& was_new) {
  return insert_slot_cas_from(keys, cap, key, home_slot(key, cap), was_new);
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

// ------------------------------------------------ partitioned table build
//
// The table split into segments of S consecutive slots; every row goes to
// the segment of its home slot, then one workgroup per segment builds that
// segment in LDS and writes it with coalesced stores -- instead of one
// returning 64-bit CAS per row at a random slot of a table no XCD's L2 holds
// (the CAS build runs at the memory-side atomic rate, ~11 G/s).  No global
// atomics and no fences on the common path: each pass hands its results to
// the next through a kernel boundary.
//
//   hash_bucket_kernel   a workgroup takes kBuildRows rows: their keys and
//                        segments, counted and ranked per segment in LDS,
//                        then written to the workgroup's own area grouped by
//                        segment (runs of ~kBuildRows / segments rows), with
//                        each run's count and offset packed in one word per
//                        (workgroup, segment), stored contiguously.
//   hash_segment_kernel  a workgroup per segment: the segment's slots in LDS
//                        (empty for a fresh table, else loaded), its rows
//                        gathered from every bucketing workgroup's run and
//                        inserted by LDS CAS with linear probing, the value
//                        by LDS atomic-min (the lowest row of a repeated
//                        key); rows whose probe runs past the segment's end
//                        go to the spill list; the segment stored.
//   hash_spill_kernel    the spilled rows inserted into the finished table by
//                        global CAS, as the CAS build does, each from the
//                        slot after its segment (the slots from its home to
//                        there hold other keys); returns at once when there
//                        are none.  The next build's bucketing pass resets the
//                        spill count.
// Linear probing never deletes, so a key already in the table sits behind an
// unbroken run of occupied slots from its home: the LDS probe of the same key
// (a prefix of the global probe) meets no empty slot before the segment's
// end, spills, and the global probe finds the key.  The table's key -> row
// mapping is the CAS build's; slot positions may differ (they depend on the
// insertion order in either build).
constexpr int kBuildRows = 4096;      // rows per bucketing workgroup (4 per thread)
constexpr int kBuildMaxSegs = 8192;   // the bucketing pass's LDS count table
constexpr int kBuildSlots = 2048;     // slots per segment (24 KB of LDS)
constexpr int kBuildMaxWgs = 2048;    // bucketing workgroups a segment gathers from

// Segments of kBuildSlots slots (the last one partial) and their count; false
// for tables or row counts too large for the partitioned build.
inline bool build_geom(int64_t n, int64_t cap, int64_t* S, int64_t* nseg) {
  if ((n + kBuildRows - 1) / kBuildRows > kBuildMaxWgs) return false;
  *S = kBuildSlots;
  *nseg = (cap + kBuildSlots - 1) / kBuildSlots;
  return *nseg <= kBuildMaxSegs;
}

struct BuildWs {
  int32_t* spills;     // spilled rows (zero between builds)
  uint32_t* runs;      // nwg x nseg: run of workgroup w's rows of segment s, count << 16 | offset
  uint64_t* bkeys;     // nwg x kBuildRows keys, grouped by segment per workgroup
  uint32_t* brows;     // the same for the rows
  uint64_t* skeys;     // n spilled keys
  uint32_t* srows;     // n spilled rows
  uint32_t* sfrom;     // n spilled rows' first slot to probe
  int nwg;
};

inline int64_t build_align(int64_t v) { return (v + 255) / 256 * 256; }

inline int64_t build_nwg(int64_t n) { return n > 0 ? (n + kBuildRows - 1) / kBuildRows : 1; }

inline int64_t build_ws_bytes(int64_t n, int64_t nseg) {
  const int64_t nwg = build_nwg(n), rows = nwg * kBuildRows, nn = n > 0 ? n : 1;
  return build_align(4) + build_align(4 * nseg * nwg) + build_align(8 * rows) + build_align(4 * rows) +
         build_align(8 * nn) + 2 * build_align(4 * nn);
}

inline BuildWs build_ws(void* ws, int64_t n, int64_t nseg) {
  const int64_t nwg = build_nwg(n), rows = nwg * kBuildRows, nn = n > 0 ? n : 1;
  char* p = (char*)ws;
  BuildWs w;
  w.nwg = (int)nwg;
  w.spills = (int32_t*)p;
  p += build_align(4);
  w.runs = (uint32_t*)p;
  p += build_align(4 * nseg * nwg);
  w.bkeys = (uint64_t*)p;
  p += build_align(8 * rows);
  w.brows = (uint32_t*)p;
  p += build_align(4 * rows);
  w.skeys = (uint64_t*)p;
  p += build_align(8 * nn);
  w.srows = (uint32_t*)p;
  p += build_align(4 * nn);
  w.sfrom = (uint32_t*)p;
  return w;
}

constexpr int kBucketThreads = 1024;
template <typename CT>
__global__ __launch_bounds__(kBucketThreads) void hash_bucket_kernel(const CT* __restrict__ coords, int64_t n,
                                                                     int64_t scale, uint32_t cap, uint32_t S, int nseg,
                                                                     BuildWs w, int32_t* __restrict__ status) {
  constexpr int J = kBuildRows / kBucketThreads;
  __shared__ int cnt_s[kBuildMaxSegs];
  __shared__ int scan_s[17];
  const int tid = threadIdx.x;
  if (blockIdx.x == 0 && tid == 0) *w.spills = 0;  // (read by the previous build's spill pass, which is done)
  for (int e = tid; e < nseg; e += kBucketThreads) cnt_s[e] = 0;
  const int64_t base = (int64_t)blockIdx.x * kBuildRows;
  // every row's coordinates in flight before the first LDS atomic
  int64_t cb[J], cx[J], cy[J], cz[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t i = base + j * kBucketThreads + tid;
    cb[j] = -1;
    cx[j] = cy[j] = cz[j] = 0;
    if (i < n) load_coord(coords, i, cb[j], cx[j], cy[j], cz[j]);
  }
  __syncthreads();
  uint64_t key[J];
  int seg[J], rank[J];
  int bad = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t i = base + j * kBucketThreads + tid;
    seg[j] = -1;
    key[j] = 0;
    rank[j] = 0;
    if (i < n) {
      if (pack_key(cb[j], cx[j] * scale, cy[j] * scale, cz[j] * scale, key[j])) {
        seg[j] = (int)(home_slot(key[j], cap) / S);
        rank[j] = atomicAdd(&cnt_s[seg[j]], 1);
      } else {
        ++bad;
      }
    }
  }
  bad = wave_sum(bad);
  if ((tid & 63) == 0 && bad) atomicAdd(&status[ST_STATUS_BAD_COORD], bad);
  __syncthreads();
  // the counts -> run offsets in the workgroup's area (exclusive scan over the segments, each
  // thread a contiguous range of them), published with the counts in one word per segment
  const int per = (nseg + kBucketThreads - 1) / kBucketThreads, e0 = tid * per, e1 = min(nseg, e0 + per);
  int sum = 0;
  for (int e = e0; e < e1; ++e) sum += cnt_s[e];
  int total;
  int run = block_exclusive_scan(sum, scan_s, &total);
  for (int e = e0; e < e1; ++e) {
    const int c = cnt_s[e];
    cnt_s[e] = run | (c << 16);
    run += c;
  }
  __syncthreads();
  uint32_t* runs = w.runs + (int64_t)blockIdx.x * nseg;
  for (int e = tid; e < nseg; e += kBucketThreads) runs[e] = (uint32_t)cnt_s[e];
  for (int e = tid; e < nseg; e += kBucketThreads) cnt_s[e] &= 0xFFFF;
  __syncthreads();
  const int64_t area = base;  // the workgroup's kBuildRows places
#pragma unroll
  for (int j = 0; j < J; ++j) {
    if (seg[j] < 0) continue;
    const int64_t at = area + cnt_s[seg[j]] + rank[j];
    w.bkeys[at] = key[j];
    w.brows[at] = (uint32_t)(base + j * kBucketThreads + tid);
  }
}

__global__ __launch_bounds__(256) void hash_segment_kernel(uint64_t* __restrict__ keys, uint32_t* __restrict__ vals,
                                                           uint32_t cap, uint32_t S, int fresh, BuildWs w,
                                                           int32_t* __restrict__ status) {
  __shared__ unsigned long long k_s[kBuildSlots];
  __shared__ uint32_t v_s[kBuildSlots];
  __shared__ int rs_s[kBuildMaxWgs + 1];  // where workgroup w's run starts among the segment's rows
  __shared__ int ro_s[kBuildMaxWgs];      // that run's offset in w's area
  __shared__ int scan_s[8];
  const int tid = threadIdx.x;
  const int seg = blockIdx.x;
  const uint32_t s0 = (uint32_t)seg * S;
  const uint32_t len = cap - s0 < S ? cap - s0 : S;
  for (uint32_t e = tid; e < len; e += 256) {
    k_s[e] = fresh ? ST_EMPTY_KEY : keys[s0 + e];
    v_s[e] = fresh ? ST_NO_VAL : vals[s0 + e];
  }
  const int nwg = w.nwg;
  const int per = (nwg + 255) / 256, q0 = tid * per, q1 = min(nwg, q0 + per);
  int sum = 0;
  for (int q = q0; q < q1; ++q) {
    const uint32_t v = w.runs[(int64_t)q * gridDim.x + seg];
    const int c = (int)(v >> 16);
    ro_s[q] = (int)(v & 0xFFFFu);
    rs_s[q] = c;
    sum += c;
  }
  int total;
  int run = block_exclusive_scan(sum, scan_s, &total);  // (its barriers also order the LDS stores above)
  for (int q = q0; q < q1; ++q) {
    const int c = rs_s[q];
    rs_s[q] = run;
    run += c;
  }
  if (tid == 0) rs_s[nwg] = total;
  __syncthreads();
  int dup = 0;
  // kSegBatch rows a thread at a time: their places found in LDS, then all their loads in
  // flight together, then the inserts
  constexpr int kSegBatch = 8;
  for (int r0 = 0; r0 < total; r0 += 256 * kSegBatch) {
    uint64_t key[kSegBatch];
    uint32_t row[kSegBatch];
    int64_t at[kSegBatch];
#pragma unroll
    for (int u = 0; u < kSegBatch; ++u) {
      const int r = r0 + u * 256 + tid;
      at[u] = -1;
      if (r < total) {
        // the run holding row r: the last workgroup whose run starts at or before r
        int lo = 0, hi = nwg - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (rs_s[mid] <= r)
            lo = mid;
          else
            hi = mid - 1;
        }
        at[u] = (int64_t)lo * kBuildRows + ro_s[lo] + (r - rs_s[lo]);
      }
    }
#pragma unroll
    for (int u = 0; u < kSegBatch; ++u) {
      key[u] = at[u] >= 0 ? w.bkeys[at[u]] : 0ull;
      row[u] = at[u] >= 0 ? w.brows[at[u]] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kSegBatch; ++u) {
      if (at[u] < 0) continue;
      bool placed = false;
      for (uint32_t s = home_slot(key[u], cap) - s0; s < len; ++s) {
        const unsigned long long old =
            atomicCAS(&k_s[s], (unsigned long long)ST_EMPTY_KEY, (unsigned long long)key[u]);
        if (old == ST_EMPTY_KEY || old == key[u]) {
          atomicMin(&v_s[s], row[u]);
          dup += old == key[u] ? 1 : 0;
          placed = true;
          break;
        }
      }
      if (!placed) {
        const int q = atomicAdd(w.spills, 1);
        w.skeys[q] = key[u];
        w.srows[q] = row[u];
        w.sfrom[q] = s0 + len == cap ? 0u : s0 + len;
      }
    }
  }
  dup = wave_sum(dup);
  if ((tid & 63) == 0 && dup) atomicAdd(&status[ST_STATUS_DUPLICATE], dup);
  __syncthreads();
  for (uint32_t e = tid; e < len; e += 256) {
    keys[s0 + e] = k_s[e];
    vals[s0 + e] = v_s[e];
  }
}

constexpr int kSpillGrid = 64;  // workgroups of the spill pass (a thread per spilled row, strided)
__global__ __launch_bounds__(256) void hash_spill_kernel(uint64_t* __restrict__ keys, uint32_t* __restrict__ vals,
                                                         uint32_t cap, BuildWs w, int32_t* __restrict__ status) {
  const int ns = *w.spills;
  if (ns == 0) return;
  int sdup = 0, over = 0;
  for (int q = blockIdx.x * 256 + threadIdx.x; q < ns; q += gridDim.x * 256) {
    const uint64_t key = w.skeys[q];
    const uint32_t row = w.srows[q];
    bool was_new = false;
    const uint32_t s = insert_slot_cas_from(keys, cap, key, w.sfrom[q], was_new);
    if (s == ST_NO_VAL) {
      ++over;
      continue;
    }
    atomicMin(&vals[s], row);
    sdup += was_new ? 0 : 1;
  }
  sdup = wave_sum(sdup);
  over = wave_sum(over);
  if ((threadIdx.x & 63) == 0) {
    if (sdup) atomicAdd(&status[ST_STATUS_DUPLICATE], sdup);
    if (over) atomicAdd(&status[ST_STATUS_OVERFLOW], over);
  }
}

}  // namespace st

using namespace st;

extern "C" {

int st_hash_build_workspace(int64_t n, int64_t capacity, int64_t* bytes) {
  int64_t S, nseg;
  if (n < 0 || n >= (1ll << 31) || capacity <= 0 || capacity >= (1ll << 31) || !bytes) return ST_ERR_ARG;
  if (!build_geom(n, capacity, &S, &nseg)) return ST_ERR_UNSUPPORTED;
  *bytes = build_ws_bytes(n, nseg);
  return ST_OK;
}

int st_hash_build(const void* coords, int coord_dtype, int64_t n, int64_t scale, uint64_t* keys, uint32_t* vals,
                  int64_t capacity, int fresh, void* workspace, int64_t workspace_bytes, int32_t* status,
                  st_stream_t stream) {
  int64_t S, nseg;
  if (n < 0 || n >= (1ll << 31) || capacity <= 0 || capacity >= (1ll << 31) || scale < 1 || !keys || !vals ||
      !status)
    return ST_ERR_ARG;
  if (coord_dtype < ST_COORD_I16 || coord_dtype > ST_COORD_I64) return ST_ERR_UNSUPPORTED;
  if (group_probe() || !build_geom(n, capacity, &S, &nseg)) return ST_ERR_UNSUPPORTED;
  if (!workspace || workspace_bytes < build_ws_bytes(n, nseg) || (n > 0 && !coords)) return ST_ERR_ARG;
  if (n == 0 && !fresh) return ST_OK;
  BuildWs w = build_ws(workspace, n, nseg);
  if (n > 0) {
    ST_DISPATCH_COORD(coord_dtype, CT,
                      hash_bucket_kernel<CT><<<(unsigned)w.nwg, kBucketThreads, 0, stream>>>(
                          (const CT*)coords, n, scale, (uint32_t)capacity, (uint32_t)S, (int)nseg, w, status));
  } else {
    w.nwg = 0;  // a fresh empty table: every segment stored empty
  }
  hash_segment_kernel<<<(unsigned)nseg, 256, 0, stream>>>(keys, vals, (uint32_t)capacity, (uint32_t)S,
                                                           fresh ? 1 : 0, w, status);
  if (n > 0) hash_spill_kernel<<<kSpillGrid, 256, 0, stream>>>(keys, vals, (uint32_t)capacity, w, status);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

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
