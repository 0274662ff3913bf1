// Sparse <-> dense conversion: the reference's to_dense (utils/to_dense.py:
// 30-282) scatters the rows of a SparseTensor into a zeroed channels-last grid
// (B, X, Y, Z, C) and, backward, gathers the grid's gradient at the same
// coordinates.  Here both move whole 16-byte chunks of a row per lane (rows
// of C channels, chunks of 16 / sizeof(T) channels when C allows it), and
// coordinates outside the grid are skipped (scatter) or read as zeros
// (gather) instead of addressing memory outside it.  As in the reference, a
// coordinate given twice keeps one of its rows (whichever store lands last).
#include "common.h"

namespace st {

// cells of the grid addressed by coordinate row r, or -1 outside it
template <typename CT>
__device__ __forceinline__ int64_t dense_cell(const CT* __restrict__ coords, int64_t r, int64_t B, int64_t sx,
                                              int64_t sy, int64_t sz) {
  const CT* p = coords + r * 4;
  const int64_t b = p[0], x = p[1], y = p[2], z = p[3];
  if (b < 0 || b >= B || x < 0 || x >= sx || y < 0 || y >= sy || z < 0 || z >= sz) return -1;
  return ((b * sx + x) * sy + y) * sz + z;
}

// 16-byte chunks of a row: chunk j of row r is thread (r * CH + j)
template <typename W, typename CT, bool SCATTER>
__global__ __launch_bounds__(256) void dense_move_kernel(const W* __restrict__ src, W* __restrict__ dst, int64_t n,
                                                         int CH, const CT* __restrict__ coords, int64_t B, int64_t sx,
                                                         int64_t sy, int64_t sz) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * CH) return;
  const int64_t r = i / CH;
  const int j = (int)(i - r * CH);
  const int64_t cell = dense_cell(coords, r, B, sx, sy, sz);
  if constexpr (SCATTER) {
    if (cell >= 0) dst[cell * CH + j] = src[i];
  } else {
    W v;
    if (cell >= 0) {
      v = src[cell * CH + j];
    } else {
      v = W{};
    }
    dst[i] = v;
  }
}

__global__ __launch_bounds__(256) void zero_words_kernel(uint4* __restrict__ p, int64_t n16, uint8_t* __restrict__ tail,
                                                         int tail_bytes) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
  if (blockIdx.x == 0 && (int)threadIdx.x < tail_bytes) tail[threadIdx.x] = 0;
}

__global__ __launch_bounds__(256) void zero_u16_kernel(uint16_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

// Row width in words W: a 16-byte vector when the row is a whole number of
// them and the buffers are aligned, else the element itself.
template <typename CT>
static int dense_move(const void* src, void* dst, int64_t n, int C, size_t esz, const CT* coords, int64_t B,
                      int64_t sx, int64_t sy, int64_t sz, bool scatter, hipStream_t stream) {
  const size_t row = (size_t)C * esz;
  const bool vec = row % 16 == 0 && (uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0;
#define ST_MOVE(Wt, CHn)                                                                                            \
  {                                                                                                                 \
    const int CH = (CHn);                                                                                           \
    const int64_t work = n * CH;                                                                                    \
    if (scatter)                                                                                                    \
      dense_move_kernel<Wt, CT, true><<<st_blocks(work, 256), 256, 0, stream>>>((const Wt*)src, (Wt*)dst, n, CH,   \
                                                                                coords, B, sx, sy, sz);             \
    else                                                                                                            \
      dense_move_kernel<Wt, CT, false><<<st_blocks(work, 256), 256, 0, stream>>>((const Wt*)src, (Wt*)dst, n, CH,  \
                                                                                 coords, B, sx, sy, sz);            \
  }
  if (vec)
    ST_MOVE(uint4, (int)(row / 16))
  else if (esz == 4)
    ST_MOVE(uint32_t, C)
  else
    ST_MOVE(uint16_t, C)
#undef ST_MOVE
  ST_CHECK_LAUNCH();
  return ST_OK;
}

// mask[r] = 1 when coords[r] (x, y, z) lies in [lo, hi] on every axis
template <typename CT>
__global__ __launch_bounds__(256) void mask_range_kernel(const CT* __restrict__ coords, int64_t n, int64_t x0,
                                                         int64_t x1, int64_t y0, int64_t y1, int64_t z0, int64_t z1,
                                                         uint8_t* __restrict__ mask) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= n) return;
  const CT* p = coords + r * 4;
  const int64_t x = p[1], y = p[2], z = p[3];
  mask[r] = (x >= x0 && x <= x1 && y >= y0 && y <= y1 && z >= z0 && z <= z1) ? 1 : 0;
}

}  // namespace st

using namespace st;

extern "C" {

int st_to_dense(const void* feats, int64_t n, int C, int dtype, const void* coords, int coord_dtype, int64_t batches,
                int64_t sx, int64_t sy, int64_t sz, void* out, st_stream_t stream) {
  if (n < 0 || C <= 0 || batches < 0 || sx < 0 || sy < 0 || sz < 0 || !out) return ST_ERR_ARG;
  if (n > 0 && (!feats || !coords)) return ST_ERR_ARG;
  if (dtype == ST_F32_BF16X3) dtype = ST_F32;
  if (dtype != ST_F32 && dtype != ST_F16 && dtype != ST_BF16) return ST_ERR_UNSUPPORTED;
  const size_t esz = dtype == ST_F32 ? 4 : 2;
  const int64_t cells = batches * sx * sy * sz;
  const int64_t bytes = cells * C * (int64_t)esz;
  if (bytes > 0) {
    if ((uintptr_t)out % 16 == 0) {
      const int64_t n16 = bytes / 16;
      int64_t g = (n16 + 255) / 256;
      g = g > 65536 ? 65536 : (g < 1 ? 1 : g);
      zero_words_kernel<<<(unsigned)g, 256, 0, stream>>>((uint4*)out, n16, (uint8_t*)out + n16 * 16,
                                                         (int)(bytes - n16 * 16));
    } else {
      int64_t g = (bytes / 2 + 255) / 256;
      g = g > 65536 ? 65536 : (g < 1 ? 1 : g);
      zero_u16_kernel<<<(unsigned)g, 256, 0, stream>>>((uint16_t*)out, bytes / 2);
    }
    ST_CHECK_LAUNCH();
  }
  if (n == 0 || cells == 0) return ST_OK;
  ST_DISPATCH_COORD(coord_dtype, CT,
                    return dense_move<CT>(feats, out, n, C, esz, (const CT*)coords, batches, sx, sy, sz, true,
                                          stream));
  return ST_OK;
}

int st_from_dense(const void* dense, int64_t batches, int64_t sx, int64_t sy, int64_t sz, int C, int dtype,
                  const void* coords, int coord_dtype, int64_t n, void* feats, st_stream_t stream) {
  if (n < 0 || C <= 0 || batches < 0 || sx < 0 || sy < 0 || sz < 0) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!feats || !coords || (!dense && batches * sx * sy * sz > 0)) return ST_ERR_ARG;
  if (dtype == ST_F32_BF16X3) dtype = ST_F32;
  if (dtype != ST_F32 && dtype != ST_F16 && dtype != ST_BF16) return ST_ERR_UNSUPPORTED;
  const size_t esz = dtype == ST_F32 ? 4 : 2;
  ST_DISPATCH_COORD(coord_dtype, CT,
                    return dense_move<CT>(dense, feats, n, C, esz, (const CT*)coords, batches, sx, sy, sz, false,
                                          stream));
  return ST_OK;
}

int st_mask_spatial_range(const void* coords, int coord_dtype, int64_t n, const int64_t* limits, uint8_t* mask,
                          st_stream_t stream) {
  if (n < 0 || !limits) return ST_ERR_ARG;
  if (n == 0) return ST_OK;
  if (!coords || !mask) return ST_ERR_ARG;
  ST_DISPATCH_COORD(coord_dtype, CT,
                    mask_range_kernel<CT><<<st_blocks(n, 256), 256, 0, stream>>>(
                        (const CT*)coords, n, limits[0], limits[1], limits[2], limits[3], limits[4], limits[5], mask));
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // extern "C"
