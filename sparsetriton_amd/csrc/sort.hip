// Destination-row order for the gather-GEMM: rows sorted by their kernel-map
// offset bitmask.
//
// The gather-GEMM runs MFMA on 16/32-row slabs; a slab executes an offset if
// any of its rows has that neighbour.  In voxelisation (lexicographic) order
// neighbouring rows have different offset sets, so a slab executes far more
// offsets than each row owns (3.4x the useful work on the config-2 LiDAR
// set).  Sorting rows by the bitmask groups rows with equal or similar masks
// and brings that to 1.15x.  Keys wider than 32 offsets are folded into 32
// bits, which still groups identical masks.
//
// The sort is a stable LSD radix sort, 9-bit digits, one pass per digit of
// the significant key bits (27-bit masks: 3 passes).  Each pass:
//   radix_hist_kernel    per 4096-element tile, a 512-bin digit histogram;
//   exclusive scan       the digit-major (digit, tile) counts, scanned as one
//                        flat array, are each tile's first output position
//                        for each digit;
//   radix_scatter_kernel each tile re-reads its elements in order and writes
//                        them at offset + stable rank, the rank coming from
//                        running per-digit counters in LDS plus, inside a
//                        wave, the lanes below with the same digit (9 ballots).
#include "common.h"

namespace st {

constexpr int kRadixBits = 9;
constexpr int kRadixBins = 1 << kRadixBits;
constexpr int kRadixTile = 4096;  // elements per workgroup (256 threads x 16)
constexpr int kBinsPerThread = kRadixBins / 256;

__global__ __launch_bounds__(256) void mask_keys_kernel(const uint32_t* __restrict__ masks, int W, int64_t n,
                                                        uint32_t* __restrict__ keys, int32_t* __restrict__ rows) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t key = masks[i * W];
  for (int w = 1; w < W; ++w) {
    const uint32_t v = masks[i * W + w];
    const int r = (7 * w) & 31;
    key ^= r ? ((v << r) | (v >> (32 - r))) : v;
  }
  keys[i] = key;
  rows[i] = (int32_t)i;
}

__global__ __launch_bounds__(256) void radix_hist_kernel(const uint32_t* __restrict__ keys, int64_t n, int shift,
                                                         int64_t ntiles, int32_t* __restrict__ hist) {
  __shared__ int h[kRadixBins];
#pragma unroll
  for (int e = 0; e < kBinsPerThread; ++e) h[threadIdx.x + e * 256] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * kRadixTile;
  for (int j = 0; j < kRadixTile / 256; ++j) {
    const int64_t i = base + j * 256 + threadIdx.x;
    if (i < n) atomicAdd(&h[(keys[i] >> shift) & (kRadixBins - 1)], 1);
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < kBinsPerThread; ++e)
    hist[(int64_t)(threadIdx.x + e * 256) * ntiles + blockIdx.x] = h[threadIdx.x + e * 256];
}

__global__ __launch_bounds__(256) void radix_scatter_kernel(const uint32_t* __restrict__ keys_in,
                                                            const int32_t* __restrict__ vals_in, int64_t n, int shift,
                                                            int64_t ntiles, const int32_t* __restrict__ offsets,
                                                            uint32_t* __restrict__ keys_out,
                                                            int32_t* __restrict__ vals_out) {
  __shared__ int run_s[kRadixBins];    // elements of each digit already placed by this tile
  __shared__ int wcnt_s[4][kRadixBins];  // per-wave digit counts of the current 256-element step
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
#pragma unroll
  for (int e = 0; e < kBinsPerThread; ++e)
    run_s[tid + e * 256] = offsets[(int64_t)(tid + e * 256) * ntiles + blockIdx.x];
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  const int64_t base = (int64_t)blockIdx.x * kRadixTile;
  for (int j = 0; j < kRadixTile / 256; ++j) {
    const int64_t i = base + j * 256 + tid;
    const bool ok = i < n;
    const uint32_t key = ok ? keys_in[i] : 0u;
    const int32_t val = ok ? vals_in[i] : 0;
    const int d = (key >> shift) & (kRadixBins - 1);
    uint64_t same = __ballot(ok);
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
      const uint64_t bal = __ballot((d >> b) & 1);
      same &= ((d >> b) & 1) ? bal : ~bal;
    }
#pragma unroll
    for (int e = 0; e < kBinsPerThread; ++e)
#pragma unroll
      for (int w = 0; w < 4; ++w) wcnt_s[w][tid + e * 256] = 0;
    __syncthreads();
    // the lowest lane of each digit group publishes the group's size
    if (ok && (same & below) == 0) wcnt_s[wid][d] = (int)__popcll(same);
    __syncthreads();
    if (ok) {
      int pos = run_s[d] + (int)__popcll(same & below);
      for (int w = 0; w < wid; ++w) pos += wcnt_s[w][d];
      if (keys_out) keys_out[pos] = key;
      vals_out[pos] = val;
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < kBinsPerThread; ++e) {
      const int d2 = tid + e * 256;
      run_s[d2] += wcnt_s[0][d2] + wcnt_s[1][d2] + wcnt_s[2][d2] + wcnt_s[3][d2];
    }
  }
}

static int radix_passes(int K) {
  const int bits = K < 32 ? K : 32;
  return (bits + kRadixBits - 1) / kRadixBits;
}

}  // namespace st

extern "C" int st_kmap_sort_workspace(int64_t n, size_t* bytes) {
  if (n < 0 || n >= (1ll << 31) || !bytes) return ST_ERR_ARG;
  const int64_t ntiles = (n + st::kRadixTile - 1) / st::kRadixTile;
  *bytes = (size_t)(st::kRadixBins * (ntiles > 0 ? ntiles : 1) + 1) * sizeof(int32_t);
  return ST_OK;
}

extern "C" int st_kmap_sort_rows(const uint32_t* masks, int mask_words, int K, int64_t n, uint32_t* keys_tmp,
                                 int32_t* rows_tmp, int32_t* perm, void* workspace, size_t workspace_bytes,
                                 st_stream_t stream) {
  if (n < 0 || n >= (1ll << 31) || K <= 0 || K > ST_MAX_KVOL || mask_words != (K + 31) / 32) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!masks || !keys_tmp || !rows_tmp || !perm || !workspace) return ST_ERR_ARG;
  const int64_t ntiles = (n + st::kRadixTile - 1) / st::kRadixTile;
  if (workspace_bytes < (size_t)(st::kRadixBins * ntiles + 1) * sizeof(int32_t)) return ST_ERR_ARG;
  const int passes = st::radix_passes(K);
  // Values ping-pong between rows_tmp and perm; start so the last pass lands in perm.
  int32_t* vbuf[2] = {(passes % 2) ? rows_tmp : perm, (passes % 2) ? perm : rows_tmp};
  uint32_t* kbuf[2] = {keys_tmp, keys_tmp + n};
  int32_t* hist = (int32_t*)workspace;
  st::mask_keys_kernel<<<st_blocks(n, 256), 256, 0, stream>>>(masks, mask_words, n, kbuf[0], vbuf[0]);
  for (int p = 0; p < passes; ++p) {
    const int shift = p * st::kRadixBits;
    const int in = p & 1, out = in ^ 1;
    st::radix_hist_kernel<<<(unsigned)ntiles, 256, 0, stream>>>(kbuf[in], n, shift, ntiles, hist);
    if (st::launch_exclusive_scan(hist, st::kRadixBins * ntiles, stream) != ST_OK) return ST_ERR_HIP;
    st::radix_scatter_kernel<<<(unsigned)ntiles, 256, 0, stream>>>(kbuf[in], vbuf[in], n, shift, ntiles, hist,
                                                                   p + 1 < passes ? kbuf[out] : nullptr, vbuf[out]);
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}
