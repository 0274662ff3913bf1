// Destination-row order for the gather-GEMM: rows sorted by their kernel-map
// offset bitmask.
//
// The gather-GEMM runs MFMA on 16/32-row slabs; a slab executes an offset if
// any of its rows has that neighbour.  In voxelisation (lexicographic) order
// neighbouring rows have different offset sets, so a slab executes far more
// offsets than each row owns (3.4x the useful work on the config-2 LiDAR
// set).  A stable radix sort by the bitmask groups rows with equal or similar
// masks and brings that to 1.15x.  The sort is rocPRIM's device radix sort
// (stable, deterministic); keys wider than 32 offsets are folded into 32 bits,
// which still groups identical masks.
#include <rocprim/device/device_radix_sort.hpp>

#include "common.h"

namespace st {

__global__ __launch_bounds__(256) void mask_keys_kernel(const uint32_t* __restrict__ masks, int W, int64_t n,
                                                        uint32_t* __restrict__ keys, int32_t* __restrict__ rows) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint32_t key = masks[i * W];
  for (int w = 1; w < W; ++w) {
    const uint32_t v = masks[i * W + w];
    key ^= (v << (7 * w % 32)) | (v >> ((32 - 7 * w % 32) % 32));
  }
  keys[i] = key;
  rows[i] = (int32_t)i;
}

}  // namespace st

extern "C" int st_kmap_sort_workspace(int64_t n, size_t* bytes) {
  if (n < 0 || n >= (1ll << 31) || !bytes) return ST_ERR_ARG;
  size_t b = 0;
  hipError_t e = rocprim::radix_sort_pairs(nullptr, b, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                           (const int32_t*)nullptr, (int32_t*)nullptr, (size_t)n, 0, 32);
  if (e != hipSuccess) return ST_ERR_HIP;
  *bytes = b;
  return ST_OK;
}

extern "C" int st_kmap_sort_rows(const uint32_t* masks, int mask_words, int K, int64_t n, uint32_t* keys_tmp,
                                 int32_t* rows_tmp, int32_t* perm, void* workspace, size_t workspace_bytes,
                                 st_stream_t stream) {
  if (n < 0 || n >= (1ll << 31) || K <= 0 || K > ST_MAX_KVOL || mask_words != (K + 31) / 32) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!masks || !keys_tmp || !rows_tmp || !perm || !workspace) return ST_ERR_ARG;
  st::mask_keys_kernel<<<st_blocks(n, 256), 256, 0, stream>>>(masks, mask_words, n, keys_tmp, rows_tmp);
  ST_CHECK_LAUNCH();
  size_t b = workspace_bytes;
  const int end_bit = K < 32 ? K : 32;
  hipError_t e = rocprim::radix_sort_pairs(workspace, b, keys_tmp, keys_tmp + n, rows_tmp, perm, (size_t)n, 0,
                                           end_bit, stream);
  if (e != hipSuccess) return ST_ERR_HIP;
  return ST_OK;
}
