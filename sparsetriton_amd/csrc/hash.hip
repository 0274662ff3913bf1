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

// Sets the occupancy bit of every row inside the box.  With `status`, a row
// whose coordinate does not pack into a key counts as ST_STATUS_BAD_COORD and a
// row that finds its bit already set (a repeated coordinate) as
// ST_STATUS_DUPLICATE -- the bitmap path never runs the hash insert that would
// otherwise report both.
template <typename CT>
__global__ __launch_bounds__(256) void occupancy_build_kernel(const CT* __restrict__ coords, int64_t n, Occ occ,
                                                              uint64_t* __restrict__ words,
                                                              int32_t* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  uint64_t key;
  if (status && !pack_key(b, x, y, z, key)) atomicAdd(&status[ST_STATUS_BAD_COORD], 1);
  if (b < 0 || b >= occ.nb || x < 0 || x >= occ.sx || y < 0 || y >= occ.sy || z < 0 || z >= occ.sz) return;
  const uint64_t bit = 1ull << occ_bit((int)x, (int)y, (int)z);
  const unsigned long long old =
      atomicOr((unsigned long long*)&words[occ_word(occ, (int)b, (int)x, (int)y, (int)z)], bit);
  if (status && (old & bit)) atomicAdd(&status[ST_STATUS_DUPLICATE], 1);
}

// Rank index: popcount sums per 4096-word block, then per word the exclusive
// prefix within its block plus the block's offset.  Words are read and the
// prefixes written with coalesced accesses (word base + e * 256 + thread); the
// scan itself runs over 16 consecutive words per thread, staged in LDS with a
// padded layout (index i + i / 16) so the strided reads are conflict-free.
constexpr int kRankBlock = 4096;  // 256 threads x 16 words
__global__ __launch_bounds__(256) void rank_block_sums_kernel(const uint64_t* __restrict__ words, int64_t nw,
                                                              int32_t* __restrict__ sums) {
  __shared__ int part_s[4];
  const int64_t base = (int64_t)blockIdx.x * kRankBlock + threadIdx.x;
  int c = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int64_t w = base + e * 256;
    c += w < nw ? __popcll(words[w]) : 0;
  }
  c = wave_sum(c);
  if ((threadIdx.x & 63) == 0) part_s[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) sums[blockIdx.x] = part_s[0] + part_s[1] + part_s[2] + part_s[3];
}

__global__ __launch_bounds__(256) void rank_prefix_kernel(const uint64_t* __restrict__ words, int64_t nw,
                                                          const int32_t* __restrict__ sums,
                                                          int32_t* __restrict__ prefix) {
  __shared__ int pc_s[kRankBlock + kRankBlock / 16];
  __shared__ int scratch[5];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * kRankBlock;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int i = e * 256 + tid;
    const int64_t w = base + i;
    pc_s[i + (i >> 4)] = w < nw ? (int)__popcll(words[w]) : 0;
  }
  __syncthreads();
  int v[16];
  int c = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    v[j] = pc_s[tid * 17 + j];
    c += v[j];
  }
  int tot;
  int run = sums[blockIdx.x] + block_exclusive_scan(c, scratch, &tot);
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    pc_s[tid * 17 + j] = run;
    run += v[j];
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int i = e * 256 + tid;
    const int64_t w = base + i;
    if (w < nw) prefix[w] = pc_s[i + (i >> 4)];
  }
  if (blockIdx.x == gridDim.x - 1 && tid == 0) prefix[nw] = sums[blockIdx.x] + tot;
}

template <typename CT>
__global__ __launch_bounds__(256) void rank_rowmap_kernel(const CT* __restrict__ coords, int64_t n, Occ occ,
                                                          int32_t* __restrict__ rowmap) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  if (b < 0 || b >= occ.nb || x < 0 || x >= occ.sx || y < 0 || y >= occ.sy || z < 0 || z >= occ.sz) return;
  const int64_t w = occ_word(occ, (int)b, (int)x, (int)y, (int)z);
  const int bit = occ_bit((int)x, (int)y, (int)z);
  const int rank = occ.prefix[w] + (int)__popcll(occ.words[w] & ((1ull << bit) - 1ull));
  atomicMin(&rowmap[rank], (int32_t)i);
}

// Kernel map by query (conv.py:12-75).  One thread per output row walks all K
// offsets; consecutive threads own consecutive rows, so each offset's column
// of the offset-major map is written with coalesced stores.  Offsets live in
// LDS (K <= ST_MAX_KVOL).
//
// A row's queries are independent, so they are resolved kQGroup at a time in
// three rounds whose loads are all in flight together: occupancy words, then
// the home-slot keys of the candidates the bitmap lets through, then the
// values of the hits.  Only a probe that meets another key at its home slot
// continues its chain on its own.  This keeps the number of dependent memory
// round trips per row near 3 * K / kQGroup instead of ~3 * K.
constexpr int kQGroup = 9;

template <typename CT>
__global__ __launch_bounds__(256) void kmap_query_kernel(const CT* __restrict__ out_coords, int64_t n_out,
                                                         const int32_t* __restrict__ offsets, int K, int64_t stride,
                                                         int64_t sx, int64_t sy, int64_t sz,
                                                         const uint64_t* __restrict__ keys,
                                                         const uint32_t* __restrict__ vals, uint32_t cap, Occ occ,
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
    int state[kQGroup];  // 0 absent, 1 bitmap decides, 2 probe
    int64_t word[kQGroup];
    int bit[kQGroup];
#pragma unroll
    for (int j = 0; j < kQGroup; ++j) {
      const int k = k0 + j;
      state[j] = 0;
      word[j] = 0;
      bit[j] = 0;
      key[j] = 0;
      if (k < K) {
        const int64_t qx = x - off_s[3 * k], qy = y - off_s[3 * k + 1], qz = z - off_s[3 * k + 2];
        if (qx >= 0 && qx < sx && qy >= 0 && qy < sy && qz >= 0 && qz < sz && pack_key(b, qx, qy, qz, key[j]))
          state[j] = occ_locate(occ, (int)b, (int)qx, (int)qy, (int)qz, word[j], bit[j]);
      }
    }
    // pass 1: occupancy words (and, with a rank index, the words' rank prefixes)
    uint64_t w[kQGroup];
    int32_t pre[kQGroup];
    const bool ranked = occ.rowmap != nullptr;
#pragma unroll
    for (int j = 0; j < kQGroup; ++j) {
      w[j] = state[j] == 1 ? occ.words[word[j]] : 0ull;
      pre[j] = (ranked && state[j] == 1) ? occ.prefix[word[j]] : 0;
    }
    // pass 2: rows by rank for in-box hits, home-slot keys for what must be probed
    // (with no table -- keys == nullptr, rank index only -- nothing is probed)
    uint32_t slot[kQGroup];
    uint64_t hk[kQGroup];
    int32_t r[kQGroup];
#pragma unroll
    for (int j = 0; j < kQGroup; ++j) {
      const bool set = state[j] == 1 && ((w[j] >> bit[j]) & 1ull);
      const bool by_rank = ranked && set;
      r[j] = by_rank ? occ.rowmap[pre[j] + (int)__popcll(w[j] & ((1ull << bit[j]) - 1ull))] : -1;
      const bool probe = keys != nullptr && !by_rank && (state[j] == 2 || set);
      slot[j] = probe ? home_slot(key[j], cap) : ST_NO_VAL;
      hk[j] = probe ? keys[slot[j]] : ST_EMPTY_KEY;
    }
    // finish the rare chains that met another key; pass 3: values of the probed hits
#pragma unroll
    for (int j = 0; j < kQGroup; ++j) {
      if (slot[j] != ST_NO_VAL) slot[j] = find_slot_from(keys, cap, key[j], slot[j], hk[j]);
      if (slot[j] != ST_NO_VAL) r[j] = (int32_t)vals[slot[j]];
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

int st_occupancy_words(int64_t batches, int64_t sx, int64_t sy, int64_t sz, int64_t* words) {
  if (!words || batches <= 0 || batches > 32768 || sx <= 0 || sy <= 0 || sz <= 0 || sx > 65536 || sy > 65536 ||
      sz > 65536)
    return ST_ERR_ARG;
  *words = batches * ((sx + 3) / 4) * ((sy + 3) / 4) * ((sz + 3) / 4);
  return ST_OK;
}

int st_occupancy_build(const void* coords, int coord_dtype, int64_t n, uint64_t* words, int64_t batches, int64_t sx,
                       int64_t sy, int64_t sz, int32_t* status, st_stream_t stream) {
  int64_t nw = 0;
  if (st_occupancy_words(batches, sx, sy, sz, &nw) != ST_OK || !words || n < 0 || n >= (1ll << 31))
    return ST_ERR_ARG;
  if (n > 0 && !coords) return ST_ERR_ARG;
  st_occupancy o{words, batches, {sx, sy, sz}, 1};
  const Occ occ = make_occ(&o);
  unsigned g = st_blocks(nw, 256);
  if (g > 65536) g = 65536;
  fill_kernel<uint64_t><<<g, 256, 0, stream>>>(words, nw, 0ull);
  if (n > 0) {
    ST_DISPATCH_COORD(coord_dtype, CT,
                      occupancy_build_kernel<CT><<<st_blocks(n, 256), 256, 0, stream>>>((const CT*)coords, n, occ,
                                                                                         words, status));
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_occupancy_rank(const void* coords, int coord_dtype, int64_t n, const st_occupancy* occ, int32_t* prefix,
                      int32_t* rowmap, int32_t* workspace, st_stream_t stream) {
  if (!occ || !occ->words || !occ_valid(occ) || occ->scale != 1 || n < 0 || n >= (1ll << 31)) return ST_ERR_ARG;
  if (!prefix || !rowmap || !workspace || (n > 0 && !coords)) return ST_ERR_ARG;
  int64_t nw = 0;
  if (st_occupancy_words(occ->batches, occ->shape[0], occ->shape[1], occ->shape[2], &nw) != ST_OK) return ST_ERR_ARG;
  const int64_t nblk = (nw + kRankBlock - 1) / kRankBlock;
  rank_block_sums_kernel<<<(unsigned)nblk, 256, 0, stream>>>(occ->words, nw, workspace);
  if (launch_exclusive_scan(workspace, nblk, stream) != ST_OK) return ST_ERR_HIP;
  rank_prefix_kernel<<<(unsigned)nblk, 256, 0, stream>>>(occ->words, nw, workspace, prefix);
  if (n > 0) {
    unsigned g = st_blocks(n, 256);
    fill_kernel<uint32_t><<<g < 65536 ? g : 65536, 256, 0, stream>>>((uint32_t*)rowmap, n, 0x7FFFFFFFu);
    st_occupancy o = *occ;
    o.prefix = prefix;
    const Occ d = make_occ(&o);
    ST_DISPATCH_COORD(coord_dtype, CT,
                      rank_rowmap_kernel<CT><<<st_blocks(n, 256), 256, 0, stream>>>((const CT*)coords, n, d, rowmap));
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_kmap_query(const void* out_coords, int coord_dtype, int64_t n_out, const int32_t* offsets, int K,
                  int64_t stride, int64_t shape_x, int64_t shape_y, int64_t shape_z, const uint64_t* keys,
                  const uint32_t* vals, int64_t capacity, const st_occupancy* occ, int32_t* nbr,
                  int64_t nbr_k_stride, int64_t nbr_r_stride, uint32_t* row_masks, int32_t* status,
                  st_stream_t stream) {
  const bool rank_only = !keys && occ && occ->words && occ->prefix && occ->rowmap;
  if (n_out < 0 || K <= 0 || K > ST_MAX_KVOL || stride < 1 || capacity >= (1ll << 31)) return ST_ERR_ARG;
  if (!rank_only && capacity <= 0) return ST_ERR_ARG;
  if (!occ_valid(occ)) return ST_ERR_ARG;
  if (n_out >= (1ll << 31)) return ST_ERR_ARG;
  if (n_out == 0) return ST_OK;
  if (!out_coords || !offsets || !nbr || (!rank_only && (!keys || !vals))) return ST_ERR_ARG;
  ST_DISPATCH_COORD(coord_dtype, CT,
                    kmap_query_kernel<CT><<<st_blocks(n_out, 256), 256, 0, stream>>>(
                        (const CT*)out_coords, n_out, offsets, K, stride, shape_x, shape_y, shape_z, keys, vals,
                        (uint32_t)capacity, make_occ(occ), nbr, nbr_k_stride, nbr_r_stride, row_masks, status));
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // extern "C"
