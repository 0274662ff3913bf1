// Destination-row order for the gather-GEMM: rows sorted by their kernel-map
// offset bitmask.
//
// The gather-GEMM runs MFMA on 128-row tiles; a tile executes an offset if
// any of its rows has that neighbour.  In voxelisation (lexicographic) order
// neighbouring rows have different offset sets, so a tile executes far more
// offsets than its rows own (3.4x the useful work on the config-2 LiDAR
// set).  Sorting rows by the bitmask groups rows with equal or similar masks.
// For a 3x3x3 kernel (K = 27, offsets enumerated x-major with the centre at
// index 13) the key's bits are the mask's bits reordered by how many axes the
// offset leaves the centre on -- centre in bit 0, faces, edges, corners in
// the top bits: the far offsets are the rarest neighbours of surface-like
// voxel sets, and grouping rows by their rare offsets first leaves tiles with
// fewer distinct offsets (config 2: 1.36x -> 1.22x the useful MFMA rows).
// Keys wider than 32 offsets are folded into 32 bits, which still groups
// identical masks.
//
// The sort is a stable LSD radix sort, 9-bit digits, one pass per digit of
// the significant key bits (27-bit masks: 3 passes).  Each pass:
//   radix_hist_kernel    per tile (1024 elements, 4096 above 4M), a 512-bin
//                        digit histogram,
//                        stored digit-major (digit, tile);
//   radix_colscan_kernel per digit, the tile counts become each tile's
//                        exclusive prefix among the tiles, plus the digit's
//                        total;
//   radix_scatter_kernel each tile scans the 512 digit totals itself, re-reads
//                        its elements in order and writes them at offset +
//                        stable rank, the rank coming from running per-digit
//                        counters in LDS plus, inside a wave, the lanes below
//                        with the same digit (9 ballots).
#include "common.h"
#include "nbr_src.h"

#include <mutex>

namespace st {

constexpr int kRadixBits = 9;
constexpr int kRadixBins = 1 << kRadixBits;
// elements per workgroup: 256 threads x 4 up to 4M elements (enough workgroups
// to fill the chip: a tile's steps are a serial chain of LDS round trips), 256
// threads x 16 above (a smaller count table)
constexpr int kRadixTileSmall = 1024;
constexpr int kRadixTileLarge = 4096;
__host__ __device__ constexpr int radix_tile(int64_t n) { return n <= (1 << 22) ? kRadixTileSmall : kRadixTileLarge; }
constexpr int kBinsPerThread = kRadixBins / 256;

// Key bit of each offset of a 3x3x3 kernel: offsets ordered by the number of
// axes on which they leave the centre (0..3), then by index.
constexpr int off_centre_axes(int k) { return (k / 9 != 1) + (k / 3 % 3 != 1) + (k % 3 != 1); }
struct CubeKeyBits {
  uint8_t pos[27];
  constexpr CubeKeyBits() : pos{} {
    int next = 0;
    for (int a = 0; a <= 3; ++a)
      for (int k = 0; k < 27; ++k)
        if (off_centre_axes(k) == a) pos[k] = (uint8_t)next++;
  }
};
__constant__ CubeKeyBits kCubeKeyBits = CubeKeyBits();

// Sort key of row i: its mask words folded into 32 bits, for a 3x3x3 kernel
// with the bits reordered by the offset's distance from the centre.
__device__ __forceinline__ uint32_t mask_key(const uint32_t* __restrict__ masks, int W, int cube3, int64_t i) {
  uint32_t key = masks[i * W];
  for (int w = 1; w < W; ++w) {
    const uint32_t v = masks[i * W + w];
    const int r = (7 * w) & 31;
    key ^= r ? ((v << r) | (v >> (32 - r))) : v;
  }
  if (cube3) {
    const uint32_t m = key;
    key = 0;
#pragma unroll
    for (int k = 0; k < 27; ++k) key |= ((m >> k) & 1u) << kCubeKeyBits.pos[k];
  }
  return key;
}

// Keys of the first pass: computed from the masks (Keys::masks set, values =
// row ids) instead of read from the key / value buffers of the previous pass.
// With bbits > 0 the first pass also puts the row's bucket -- row * 2^bbits / n,
// a slab of the caller's row order -- above the K mask bits.
struct Keys {
  const uint32_t* keys;
  const int32_t* vals;
  const uint32_t* masks;
  int W, cube3, K, bbits;
  int64_t n;
  __device__ __forceinline__ uint32_t key(int64_t i) const {
    if (!masks) return keys[i];
    uint32_t k = mask_key(masks, W, cube3, i);
    if (bbits) k |= (uint32_t)((i << bbits) / n) << K;
    return k;
  }
  __device__ __forceinline__ int32_t val(int64_t i) const { return masks ? (int32_t)i : vals[i]; }
};

// Every thread loads its J keys before the first LDS atomic, so a tile's
// loads are all in flight together.
template <int J>
__global__ __launch_bounds__(256) void radix_hist_kernel(Keys keys, int64_t n, int shift, int64_t ntiles,
                                                         int32_t* __restrict__ hist) {
  constexpr int kTile = J * 256;
  __shared__ int h[kRadixBins];
#pragma unroll
  for (int e = 0; e < kBinsPerThread; ++e) h[threadIdx.x + e * 256] = 0;
  const int64_t base = (int64_t)blockIdx.x * kTile;
  uint32_t d[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t i = base + j * 256 + threadIdx.x;
    d[j] = i < n ? (keys.key(i) >> shift) & (kRadixBins - 1) : (uint32_t)kRadixBins;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (d[j] < (uint32_t)kRadixBins) atomicAdd(&h[d[j]], 1);
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kBinsPerThread; ++e)
    hist[(int64_t)(threadIdx.x + e * 256) * ntiles + blockIdx.x] = h[threadIdx.x + e * 256];
}

// One wave per digit: the digit's per-tile counts (a contiguous column of the
// digit-major histogram) become, in place, each tile's exclusive prefix among
// the tiles; totals[d] receives the digit's count.  The counts of 512 tiles
// are loaded at once, then scanned 64 at a time in registers.
__global__ __launch_bounds__(256) void radix_colscan_kernel(int32_t* __restrict__ hist, int64_t ntiles,
                                                            int32_t* __restrict__ totals) {
  constexpr int B = 8;
  const int lane = threadIdx.x & 63;
  const int d = blockIdx.x * 4 + (threadIdx.x >> 6);
  int32_t* col = hist + (int64_t)d * ntiles;
  int carry = 0;
  for (int64_t t0 = 0; t0 < ntiles; t0 += 64 * B) {
    int v[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int64_t t = t0 + b * 64 + lane;
      v[b] = t < ntiles ? col[t] : 0;
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const int64_t t = t0 + b * 64 + lane;
      const int inc = wave_inclusive_scan(v[b]);
      if (t < ntiles) col[t] = carry + inc - v[b];
      carry += __shfl(inc, 63, 64);
    }
  }
  if (lane == 0) totals[d] = carry;
}

// Scatter of one tile of J * 256 elements.  The tile's first output position for
// digit d is (elements of smaller digits, an exclusive scan of the digit
// totals done here) + (elements of digit d in earlier tiles, the column
// scan).  The tile's keys and values are loaded up front; then each
// 256-element step ranks its elements by digit: inside a wave from 9 ballots,
// across waves from per-wave digit counts published in LDS.  Those counts
// carry their step's tag (step + 1 in the bits above 8), so a stale entry of
// an earlier step reads as 0 and nothing is cleared, and the counts and the
// running per-digit positions alternate between two buffers by step parity,
// which leaves one barrier per step.
template <int J>
__global__ __launch_bounds__(256) void radix_scatter_kernel(Keys in, int64_t n, int shift,
                                                            int64_t ntiles, const int32_t* __restrict__ offsets,
                                                            const int32_t* __restrict__ totals,
                                                            uint32_t* __restrict__ keys_out,
                                                            int32_t* __restrict__ vals_out) {
  constexpr int kTile = J * 256;
  static_assert(kBinsPerThread == 2, "two digits per thread");
  __shared__ int run_s[2][kRadixBins];     // next output position of each digit, by step parity
  __shared__ int wcnt_s[2][4][kRadixBins];  // tagged per-wave digit counts, by step parity
  __shared__ int scan_s[8];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t base = (int64_t)blockIdx.x * kTile;
  uint32_t kk[J];
  int32_t vv[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int64_t i = base + j * 256 + tid;
    kk[j] = i < n ? in.key(i) : 0u;
    vv[j] = i < n ? in.val(i) : 0;
  }
  {
    const int d0 = 2 * tid;
    const int t0 = totals[d0], t1 = totals[d0 + 1];
    int all;
    const int ex = block_exclusive_scan(t0 + t1, scan_s, &all);
    run_s[0][d0] = ex + offsets[(int64_t)d0 * ntiles + blockIdx.x];
    run_s[0][d0 + 1] = ex + t0 + offsets[(int64_t)(d0 + 1) * ntiles + blockIdx.x];
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    wcnt_s[0][w][tid] = 0;
    wcnt_s[0][w][tid + 256] = 0;
    wcnt_s[1][w][tid] = 0;
    wcnt_s[1][w][tid + 256] = 0;
  }
  __syncthreads();
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int par = j & 1, tag = (j + 1) << 8;
    const bool ok = base + j * 256 + tid < n;
    const int d = (kk[j] >> shift) & (kRadixBins - 1);
    uint64_t same = __ballot(ok);
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
      const uint64_t bal = __ballot((d >> b) & 1);
      same &= ((d >> b) & 1) ? bal : ~bal;
    }
    // the lowest lane of each digit group publishes the group's size
    if (ok && (same & below) == 0) wcnt_s[par][wid][d] = tag | (int)__popcll(same);
    __syncthreads();
    if (ok) {
      int pos = run_s[par][d] + (int)__popcll(same & below);
      for (int w = 0; w < wid; ++w) {
        const int c = wcnt_s[par][w][d];
        pos += (c & ~255) == tag ? (c & 255) : 0;
      }
      if (keys_out) keys_out[pos] = kk[j];
      vals_out[pos] = vv[j];
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int d2 = 2 * tid + e;
      int add = 0;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int c = wcnt_s[par][w][d2];
        add += (c & ~255) == tag ? (c & 255) : 0;
      }
      run_s[par ^ 1][d2] = run_s[par][d2] + add;
    }
  }
}

// Tile plan: one workgroup per 128-row destination tile (rows in perm order).
// The union of the rows' masks gives the tile's active offsets (ascending);
// for each of them the 128 source rows are gathered from the map once and
// stored contiguously.  Source rows >= n_src are stored as -1.  Thread t
// serves row t % 128 and every other active offset from t / 128; its map
// loads are issued kPlanBatch at a time before any store, so a tile costs
// about three memory round trips (perm, mask, map) rather than one per offset.
constexpr int kPlanBatch = 16;
//
// With `skeys` (the sort's keys in sorted order, key_mode 1: the mask itself
// in the low K bits, 2: a 3x3x3 mask with its bits reordered as mask_key
// does) the tile's union comes from its rows' keys, read contiguously and
// independently of perm, instead of from each row's mask through perm.
__global__ __launch_bounds__(256) void tile_plan_kernel(const int32_t* __restrict__ map, int64_t ks, int64_t rs,
                                                        const uint32_t* __restrict__ masks, int W, int K,
                                                        const int32_t* __restrict__ perm, int64_t n_dst,
                                                        int64_t n_src, int32_t* __restrict__ tile_nk,
                                                        int16_t* __restrict__ tile_klist,
                                                        int32_t* __restrict__ tile_map,
                                                        const uint32_t* __restrict__ skeys = nullptr,
                                                        int key_mode = 0) {
  __shared__ uint32_t tmask_s[2][ST_MAX_KVOL / 32];
  __shared__ int16_t klist_s[ST_MAX_KVOL];
  __shared__ int nk_s;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int r = tid & (kTileRows - 1), half = tid >> 7;
  const int64_t tile = blockIdx.x;
  const int64_t gr = tile * kTileRows + r;
  const int32_t row = gr < n_dst ? perm[gr] : -1;
  if (skeys && key_mode) {
    uint32_t v = (half == 0 && gr < n_dst) ? skeys[gr] : 0u;
    v = wave_or(v);
    if (half == 0 && lane == 0) tmask_s[wid][0] = v;
    __syncthreads();
    if (tid == 0) {
      uint32_t kb = tmask_s[0][0] | tmask_s[1][0], m = 0u;
      if (key_mode == 2) {
        for (int k = 0; k < 27; ++k) m |= ((kb >> kCubeKeyBits.pos[k]) & 1u) << k;
      } else {
        m = K < 32 ? kb & ((1u << K) - 1u) : kb;
      }
      tmask_s[0][0] = m;
      tmask_s[1][0] = 0u;
    }
  } else if (masks) {
    // waves 0 and 1 hold the tile's 128 rows; waves 2 and 3 repeat them
    for (int w = 0; w < W; ++w) {
      uint32_t v = (half == 0 && row >= 0) ? masks[(int64_t)row * W + w] : 0u;
      v = wave_or(v);
      if (half == 0 && lane == 0) tmask_s[wid][w] = v;
    }
  } else if (tid < W) {
    tmask_s[0][tid] = (tid == W - 1 && (K & 31)) ? ((1u << (K & 31)) - 1u) : 0xFFFFFFFFu;
    tmask_s[1][tid] = 0u;
  }
  __syncthreads();
  if (tid == 0) {
    int nk = 0;
    for (int w = 0; w < W; ++w) {
      uint32_t bits = tmask_s[0][w] | tmask_s[1][w];
      while (bits) {
        klist_s[nk++] = (int16_t)(w * 32 + __builtin_ctz(bits));
        bits &= bits - 1;
      }
    }
    nk_s = nk;
    tile_nk[tile] = nk;
  }
  __syncthreads();
  const int nk = nk_s;
  for (int j = tid; j < nk; j += 256) tile_klist[tile * K + j] = klist_s[j];
  int32_t* out = tile_map + tile * K * kTileRows + r;
  for (int j0 = half; j0 < nk; j0 += 2 * kPlanBatch) {
    int32_t v[kPlanBatch];
#pragma unroll
    for (int u = 0; u < kPlanBatch; ++u) {
      const int j = j0 + 2 * u;
      v[u] = (j < nk && row >= 0) ? map[(int64_t)klist_s[j] * ks + (int64_t)row * rs] : -1;
    }
#pragma unroll
    for (int u = 0; u < kPlanBatch; ++u) {
      const int j = j0 + 2 * u;
      if (j < nk) out[(int64_t)j * kTileRows] = (int64_t)v[u] >= n_src ? -1 : v[u];
    }
  }
}

static int radix_passes(int K, int bbits = 0) {
  const int bits = K + bbits < 32 ? K + bbits : 32;
  return (bits + kRadixBits - 1) / kRadixBits;
}

}  // namespace st

extern "C" int st_kmap_sort_workspace(int64_t n, size_t* bytes) {
  if (n < 0 || n >= (1ll << 31) || !bytes) return ST_ERR_ARG;
  const int64_t tile = st::radix_tile(n), ntiles = (n + tile - 1) / tile;
  *bytes = (size_t)(st::kRadixBins * ((ntiles > 0 ? ntiles : 1) + 1)) * sizeof(int32_t);
  return ST_OK;
}

namespace st {
// LSD radix sort of rows by mask key into perm; buffers checked by the caller
// With `sorted_keys` the last pass also writes the keys in sorted order: keys_tmp + n when the
// pass count is odd, keys_tmp when even (*sorted_keys), so a caller needs no second buffer.
static int launch_sort(const uint32_t* masks, int mask_words, int K, int64_t n, uint32_t* keys_tmp,
                       int32_t* rows_tmp, int32_t* perm, int32_t* hist, hipStream_t stream, int bbits = 0,
                       const uint32_t** sorted_keys = nullptr) {
  const int64_t tile = radix_tile(n), ntiles = (n + tile - 1) / tile;
  if (K + bbits > 32) bbits = 0;
  const int passes = radix_passes(K, bbits);
  // Values ping-pong between rows_tmp and perm; start so the last pass lands in perm.
  int32_t* vbuf[2] = {(passes % 2) ? rows_tmp : perm, (passes % 2) ? perm : rows_tmp};
  uint32_t* kbuf[2] = {keys_tmp, keys_tmp + n};
  int32_t* totals = hist + kRadixBins * ntiles;
  for (int p = 0; p < passes; ++p) {
    const int shift = p * kRadixBits;
    const int in = p & 1, out = in ^ 1;
    uint32_t* kout = p + 1 < passes ? kbuf[out] : (sorted_keys ? kbuf[out] : nullptr);
    if (p + 1 == passes && sorted_keys) *sorted_keys = kbuf[out];
    // the first pass computes the keys from the masks; later ones read the previous pass's output
    const Keys ks = p == 0 ? Keys{nullptr, nullptr, masks, mask_words, K == 27, K, bbits, n}
                           : Keys{kbuf[in], vbuf[in], nullptr, 0, 0, 0, 0, 1};
    if (tile == kRadixTileSmall)
      radix_hist_kernel<kRadixTileSmall / 256><<<(unsigned)ntiles, 256, 0, stream>>>(ks, n, shift, ntiles, hist);
    else
      radix_hist_kernel<kRadixTileLarge / 256><<<(unsigned)ntiles, 256, 0, stream>>>(ks, n, shift, ntiles, hist);
    radix_colscan_kernel<<<kRadixBins / 4, 256, 0, stream>>>(hist, ntiles, totals);
    if (tile == kRadixTileSmall)
      radix_scatter_kernel<kRadixTileSmall / 256><<<(unsigned)ntiles, 256, 0, stream>>>(ks, n, shift, ntiles, hist,
                                                                                          totals, kout, vbuf[out]);
    else
      radix_scatter_kernel<kRadixTileLarge / 256><<<(unsigned)ntiles, 256, 0, stream>>>(ks, n, shift, ntiles, hist,
                                                                                          totals, kout, vbuf[out]);
  }
  return hipGetLastError() == hipSuccess ? ST_OK : ST_ERR_HIP;
}
}  // namespace st

extern "C" int st_kmap_sort_rows(const uint32_t* masks, int mask_words, int K, int64_t n, uint32_t* keys_tmp,
                                 int32_t* rows_tmp, int32_t* perm, void* workspace, size_t workspace_bytes,
                                 st_stream_t stream) {
  if (n < 0 || n >= (1ll << 31) || K <= 0 || K > ST_MAX_KVOL || mask_words != (K + 31) / 32) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!masks || !keys_tmp || !rows_tmp || !perm || !workspace) return ST_ERR_ARG;
  const int64_t tile = st::radix_tile(n), ntiles = (n + tile - 1) / tile;
  if (workspace_bytes < (size_t)(st::kRadixBins * (ntiles + 1)) * sizeof(int32_t)) return ST_ERR_ARG;
  return st::launch_sort(masks, mask_words, K, n, keys_tmp, rows_tmp, perm, (int32_t*)workspace, stream);
}

extern "C" int st_tile_plan(const int32_t* map, int64_t map_k_stride, int64_t map_r_stride, const uint32_t* row_masks,
                            int mask_words, int K, const int32_t* perm, int64_t n_dst, int64_t n_src,
                            int32_t* tile_nk, int16_t* tile_klist, int32_t* tile_map, st_stream_t stream) {
  if (K <= 0 || K > ST_MAX_KVOL || n_dst < 0 || n_dst >= (1ll << 31) || n_src < 0) return ST_ERR_ARG;
  if (row_masks && mask_words != (K + 31) / 32) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!map || !perm || !tile_nk || !tile_klist || !tile_map) return ST_ERR_ARG;
  const int64_t ntiles = (n_dst + st::kTileRows - 1) / st::kTileRows;
  st::tile_plan_kernel<<<(unsigned)ntiles, 256, 0, stream>>>(map, map_k_stride, map_r_stride, row_masks,
                                                             (K + 31) / 32, K, perm, n_dst, n_src, tile_nk,
                                                             tile_klist, tile_map);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

// ------------------------------------------------------------ whole plan

namespace {

constexpr int64_t kAlign = 256;
inline int64_t align_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct PlanScratch {
  int64_t sort_keys, sort_rows, sort_hist, pair_counts, ck_keys, ck_tmp, ck_rows, ck_hist, bytes;
};

int64_t sort_hist_bytes(int64_t n) {
  const int64_t tile = st::radix_tile(n), ntiles = (n + tile - 1) / tile;
  return (int64_t)st::kRadixBins * ((ntiles > 0 ? ntiles : 1) + 1) * (int64_t)sizeof(int32_t);
}

PlanScratch plan_scratch(int64_t n, int K, int64_t max_chunks) {
  PlanScratch s{};
  int64_t at = 0;
  s.sort_keys = at, at = align_up(at + 8 * n);
  s.sort_rows = at, at = align_up(at + 4 * n);
  s.sort_hist = at, at = align_up(at + sort_hist_bytes(n));
  const int64_t nb = (n + st::kPairRows - 1) / st::kPairRows;
  s.pair_counts = at, at = align_up(at + 4 * ((int64_t)K * nb + 1));
  s.ck_keys = s.ck_tmp = s.ck_rows = s.ck_hist = at;
  if (max_chunks > st::kChunkOrderMax || K > st::kChunkOrderMaxK) {  // chunk order by keys + radix sort
    s.ck_keys = at, at = align_up(at + 4 * max_chunks);
    s.ck_tmp = at, at = align_up(at + 8 * max_chunks);
    s.ck_rows = at, at = align_up(at + 4 * max_chunks);
    s.ck_hist = at, at = align_up(at + sort_hist_bytes(max_chunks));
  }
  s.bytes = at > 0 ? at : kAlign;
  return s;
}

bool plan_layout(int64_t n, int K, int chunk, int64_t* L) {
  if (n < 0 || n >= (1ll << 31) || K <= 0 || K > ST_MAX_KVOL || (chunk < 0 && chunk != ST_PAIR_CHUNK_AUTO))
    return false;
  if ((int64_t)K * n >= (1ll << 31)) return false;
  const int64_t tiles = (n + st::kTileRows - 1) / st::kTileRows;
  const int64_t mc = chunk > 0 ? (int64_t)K * n / chunk + K : (chunk < 0 ? st::auto_max_chunks(n, K) : 0);
  int64_t at = 0;
  L[ST_PLAN_PERM] = at, at = align_up(at + 4 * n);
  L[ST_PLAN_TILE_NK] = at, at = align_up(at + 4 * tiles);
  L[ST_PLAN_TILE_KLIST] = at, at = align_up(at + 2 * tiles * K);
  L[ST_PLAN_TILE_MAP] = at, at = align_up(at + 4 * tiles * K * st::kTileRows);
  L[ST_PLAN_PAIRS] = at, at = align_up(at + (chunk != 0 ? 8 * (int64_t)K * n : 0));
  L[ST_PLAN_KSTART] = at, at = align_up(at + (chunk != 0 ? 4 * (K + 1) : 0));
  L[ST_PLAN_CSTART] = at, at = align_up(at + (chunk != 0 ? 4 * (K + 2) : 0));
  L[ST_PLAN_CORDER] = at, at = align_up(at + 4 * mc);
  L[ST_PLAN_BYTES] = at > 0 ? at : kAlign;
  L[ST_PLAN_SCRATCH_BYTES] = plan_scratch(n, K, mc).bytes;
  L[ST_PLAN_TILES] = tiles;
  L[ST_PLAN_MAX_CHUNKS] = mc;
  return true;
}

// One side stream and a fork / join event pair per device, created on first use.
constexpr int kMaxDevices = 64;
struct SideStream {
  std::mutex mu;
  bool init = false, ok = false;
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
SideStream g_side[kMaxDevices];

}  // namespace

extern "C" int st_kmap_plans_layout(int64_t n_dst, int K, int chunk, int64_t* layout) {
  if (!layout) return ST_ERR_ARG;
  return plan_layout(n_dst, K, chunk, layout) ? ST_OK : ST_ERR_ARG;
}

extern "C" int st_kmap_plans(const int32_t* map, int64_t map_k_stride, int64_t map_r_stride, const uint32_t* row_masks,
                             int K, int64_t n_dst, int64_t n_src, int chunk, int bucket_bits, void* plan, void* scratch,
                             st_stream_t stream) {
  int64_t L[ST_PLAN_FIELDS];
  if (!plan_layout(n_dst, K, chunk, L) || n_src < 0 || bucket_bits < 0 || bucket_bits > 8) return ST_ERR_ARG;
  if (n_dst == 0 && chunk == 0) return ST_OK;
  if (!plan || !scratch || (n_dst > 0 && (!map || !row_masks))) return ST_ERR_ARG;
  const int W = (K + 31) / 32;
  char* pb = (char*)plan;
  char* sb = (char*)scratch;
  const PlanScratch S = plan_scratch(n_dst, K, L[ST_PLAN_MAX_CHUNKS]);
  int32_t* perm = (int32_t*)(pb + L[ST_PLAN_PERM]);

  SideStream* side = nullptr;
  std::unique_lock<std::mutex> lock;
  if (chunk != 0) {
    int dev = 0;
    ST_CHECK_HIP(hipGetDevice(&dev));
    if (dev >= 0 && dev < kMaxDevices) {
      SideStream& s = g_side[dev];
      lock = std::unique_lock<std::mutex>(s.mu);
      if (!s.init) {
        s.init = true;
        s.ok = hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking) == hipSuccess &&
               hipEventCreateWithFlags(&s.fork, hipEventDisableTiming) == hipSuccess &&
               hipEventCreateWithFlags(&s.join, hipEventDisableTiming) == hipSuccess;
      }
      if (s.ok) side = &s;
    }
  }
  hipStream_t ps = stream;  // the pair list's stream
  if (side) {
    ST_CHECK_HIP(hipEventRecord(side->fork, stream));
    ST_CHECK_HIP(hipStreamWaitEvent(side->stream, side->fork, 0));
    ps = side->stream;
  }
  // Everything after the fork runs inside `body`, so that the caller's stream
  // waits for the side stream on every return path: a launch error on either
  // stream must not leave pair-list kernels writing into `plan` after the
  // caller's stream has moved on.
  auto body = [&]() -> int {
    if (chunk != 0) {
      const int64_t nb = (n_dst + st::kPairRows - 1) / st::kPairRows;
      int32_t* pairs = (int32_t*)(pb + L[ST_PLAN_PAIRS]);
      int32_t* kstart = (int32_t*)(pb + L[ST_PLAN_KSTART]);
      int32_t* cstart = (int32_t*)(pb + L[ST_PLAN_CSTART]);
      int32_t* corder = (int32_t*)(pb + L[ST_PLAN_CORDER]);
      const int64_t mc = L[ST_PLAN_MAX_CHUNKS];
      int rc = st::launch_pairs(map, map_k_stride, map_r_stride, n_dst, K, n_src, (int32_t*)(sb + S.pair_counts), nb,
                                chunk, kstart, cstart, pairs, ps);
      if (rc == ST_OK) {
        if (mc <= st::kChunkOrderMax && K <= st::kChunkOrderMaxK) {
          rc = st::launch_chunk_order(pairs, kstart, cstart, K, chunk, mc, n_dst, corder, ps);
        } else {
          uint32_t* ck = (uint32_t*)(sb + S.ck_keys);
          rc = st::launch_chunk_keys(pairs, kstart, cstart, K, chunk, mc, n_dst, ck, ps);
          if (rc == ST_OK)
            rc = st::launch_sort(ck, 1, 9, mc, (uint32_t*)(sb + S.ck_tmp), (int32_t*)(sb + S.ck_rows), corder,
                                 (int32_t*)(sb + S.ck_hist), ps);
        }
      }
      if (rc != ST_OK) return rc;
    }
    if (n_dst > 0) {
      // the sorted keys give each tile's offset union when they invert to the mask (K <= 32)
      const int key_mode = W == 1 ? (K == 27 ? 2 : 1) : 0;
      const uint32_t* skeys = nullptr;
      const int rc = st::launch_sort(row_masks, W, K, n_dst, (uint32_t*)(sb + S.sort_keys),
                                     (int32_t*)(sb + S.sort_rows), perm, (int32_t*)(sb + S.sort_hist), stream,
                                     bucket_bits, key_mode ? &skeys : nullptr);
      if (rc != ST_OK) return rc;
      st::tile_plan_kernel<<<(unsigned)L[ST_PLAN_TILES], 256, 0, stream>>>(
          map, map_k_stride, map_r_stride, row_masks, W, K, perm, n_dst, n_src, (int32_t*)(pb + L[ST_PLAN_TILE_NK]),
          (int16_t*)(pb + L[ST_PLAN_TILE_KLIST]), (int32_t*)(pb + L[ST_PLAN_TILE_MAP]), skeys, key_mode);
      ST_CHECK_LAUNCH();
    }
    return ST_OK;
  };
  const int rc = body();
  if (side) {
    // the join is recorded whatever `body` returned
    const hipError_t e1 = hipEventRecord(side->join, side->stream);
    const hipError_t e2 = e1 == hipSuccess ? hipStreamWaitEvent(stream, side->join, 0) : e1;
    if (e2 != hipSuccess) {
      // the caller's stream cannot be ordered after the side stream: wait for it here
      (void)hipStreamSynchronize(side->stream);
      if (rc == ST_OK) return ST_ERR_HIP;
    }
  }
  return rc;
}
