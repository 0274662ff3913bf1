// C entry points of the gather-GEMM and weight-gradient kernels
// (kernels in gemm_kernels.h, instantiated per dtype in gemm_{f32,f16,bf16}.hip).
#include <mutex>

#include "gemm_kernels.h"

ST_GEMM_OPS(extern, float)
ST_GEMM_OPS(extern, _Float16)
ST_GEMM_OPS(extern, __bf16)

namespace st {
int ops_gather_map_x3(const float* A, int64_t n_src, const int32_t* map, int64_t ks, int64_t rs,
                      const uint32_t* masks, int W, const int32_t* rows, const float* Bt, float* out, Epi<float> epi, int64_t n_dst,
                      int K, int Kd, int Nd, hipStream_t stream);
int ops_gather_hash_x3(const float* A, int64_t n_src, const void* coords, int coord_dtype, const int32_t* offsets,
                       const st_lookup* lk, const uint64_t* keys, const uint32_t* vals, int64_t cap, const float* Bt,
                       float* out, Epi<float> epi, int64_t n_dst, int Kd, int Nd, hipStream_t stream);
int ops_gather_tiled_x3(const float* A, int64_t n_src, const int32_t* perm, const int32_t* nk, const int16_t* klist,
                        const int32_t* tmap, const float* Bt, float* out, Epi<float> epi, int64_t n_dst, int K, int Kd, int Nd,
                        hipStream_t stream, int rev);
int ops_wgrad_pairs_x3(const float* X, int64_t n_in, const float* dY, int64_t n_out, const int32_t* pairs,
                       const int32_t* kstart, const int32_t* cstart, const int32_t* chunk_order, int K, int chunk,
                       int64_t max_chunks, int Cin, int Cout, float* partials, void* dW, int dw_dtype,
                       hipStream_t stream);
int ops_gather_fly_x3(const float* A, int64_t n, const void* coords, int coord_dtype, const int32_t* offsets, int K,
                      const SubmIndex& ix, const int32_t* rows, int rev, const float* Bt, float* out,
                      const float* bias, int Kd, int Nd, hipStream_t stream);
}  // namespace st

using namespace st;

// ST_F32_BF16X3 dispatches like ST_F32 except where a call site names its
// split-operand kernel first.
#define ST_DISPATCH_DTYPE(dt, T, ...) \
  switch (dt) {                       \
    case ST_F32:                      \
    case ST_F32_BF16X3: {             \
      using T = float;                \
      return __VA_ARGS__;             \
    }                                 \
    case ST_F16: {                    \
      using T = _Float16;             \
      return __VA_ARGS__;             \
    }                                 \
    case ST_BF16: {                   \
      using T = __bf16;               \
      return __VA_ARGS__;             \
    }                                 \
    default:                          \
      return ST_ERR_UNSUPPORTED;      \
  }

namespace st {
// out (rows x nd elements of U) = bias broadcast over the rows, or 0.
template <typename U>
__global__ __launch_bounds__(256) void fill_rows_kernel(U* __restrict__ out, int64_t n, int nd,
                                                        const U* __restrict__ bias) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    out[i] = bias ? bias[i % nd] : (U)0;
}

// out (rows x nd of T) = the epilogue of a zero sum, column by column.
template <typename T>
__global__ __launch_bounds__(256) void fill_rows_epi_kernel(T* __restrict__ out, int64_t n, int nd, Epi<T> epi) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    float mul, add;
    const int col = (int)(i % nd);
    epi.column(col, nd, mul, add);
    out[i] = (T)epi.apply(0.f, mul, add, i / nd, nd, col);
  }
}

template <typename T>
static int fill_output_epi(void* out, int64_t n_dst, int Nd, Epi<T> epi, hipStream_t stream) {
  const int64_t n = n_dst * Nd;
  const int64_t blocks = (n + 255) / 256;
  const unsigned g = (unsigned)(blocks < 65536 ? blocks : 65536);
  fill_rows_epi_kernel<T><<<g, 256, 0, stream>>>((T*)out, n, Nd, epi);
  ST_CHECK_LAUNCH();
  return ST_OK;
}
}  // namespace st

// A gather-GEMM with no source rows writes its rows as the bias alone (or
// zeros).  The kernels read a clamped row 0 for every missing source, so
// they are not launched then (an empty A may have no storage at all).
static int fill_output(void* out, int64_t n_dst, int Nd, int dtype, const void* bias, hipStream_t stream) {
  const int64_t n = n_dst * Nd;
  const int64_t blocks = (n + 255) / 256;
  const unsigned g = (unsigned)(blocks < 65536 ? blocks : 65536);
  if (dtype == ST_F16 || dtype == ST_BF16)
    st::fill_rows_kernel<uint16_t><<<g, 256, 0, stream>>>((uint16_t*)out, n, Nd, (const uint16_t*)bias);
  else
    st::fill_rows_kernel<uint32_t><<<g, 256, 0, stream>>>((uint32_t*)out, n, Nd, (const uint32_t*)bias);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

namespace st {
constexpr int kColSumBlocks = 1024;  // row ranges of the first pass (partials: kColSumBlocks x C fp32)

// Pass 1: workgroup b sums rows [b n / G, (b + 1) n / G) of Y (n x C) into
// partial[b][:] in a fixed order.  Vector path (C * sizeof(T) a multiple of
// 16 bytes, at most 256 16-byte chunks per row): a thread owns one 16-byte
// column chunk of every RPI-th row, four rows' loads in flight, and the RPI
// row phases are summed in LDS.  Otherwise a thread owns a column.
template <typename T>
__global__ __launch_bounds__(256) void colsum_partial_kernel(const T* __restrict__ Y, int64_t n, int C, int vec,
                                                             float* __restrict__ partial) {
  constexpr int VEC = 16 / (int)sizeof(T);
  typedef T vec_t __attribute__((ext_vector_type(VEC)));
  __shared__ float red[256 * VEC];
  const int G = gridDim.x, tid = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * n / G, r1 = (int64_t)(blockIdx.x + 1) * n / G;
  if (vec) {
    const int tpr = C / VEC, rpi = 256 / tpr, q = tid % tpr, sub = tid / tpr;
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    if (sub < rpi) {
      constexpr int U = 4;
      int64_t r = r0 + sub;
      for (; r + (U - 1) * rpi < r1; r += U * rpi) {
        vec_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = *reinterpret_cast<const vec_t*>(Y + (r + u * rpi) * C + q * VEC);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[e] += (float)v[u][e];
      }
      for (; r < r1; r += rpi) {
        const vec_t v = *reinterpret_cast<const vec_t*>(Y + r * C + q * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += (float)v[e];
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[tid * VEC + e] = acc[e];
    __syncthreads();
    for (int col = tid; col < C; col += 256) {
      const int cq = col / VEC, ce = col % VEC;
      float t = 0.f;
      for (int j = 0; j < rpi; ++j) t += red[(j * tpr + cq) * VEC + ce];
      partial[(int64_t)blockIdx.x * C + col] = t;
    }
  } else {
    for (int col = tid; col < C; col += 256) {
      float s = 0.f;
      int64_t r = r0;
      for (; r + 7 < r1; r += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = (float)Y[(r + u) * C + col];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
      }
      for (; r < r1; ++r) s += (float)Y[r * C + col];
      partial[(int64_t)blockIdx.x * C + col] = s;
    }
  }
}

// Pass 2: workgroup c sums column c of the G partials: thread t takes
// b = t, t + 256, ..., then a fixed-order tree over the threads.
template <typename TO>
__global__ __launch_bounds__(256) void colsum_final_kernel(const float* __restrict__ partial, int G, int C,
                                                           TO* __restrict__ out) {
  __shared__ float red[256];
  const int c = blockIdx.x, tid = threadIdx.x;
  float s = 0.f;
  for (int b = tid; b < G; b += 256) s += partial[(int64_t)b * C + c];
  red[tid] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) out[c] = from_f32<TO>(red[0]);
}

template <typename T>
static int column_sum(const T* Y, int64_t n, int C, float* partials, void* out, int out_dtype, hipStream_t stream) {
  const int G = (int)(n < kColSumBlocks ? (n > 0 ? n : 1) : kColSumBlocks);
  constexpr int VEC = 16 / (int)sizeof(T);
  const int vec = C % VEC == 0 && C / VEC <= 256 && 256 % (C / VEC) == 0 && (uintptr_t)Y % 16 == 0;
  colsum_partial_kernel<T><<<G, 256, 0, stream>>>(Y, n, C, vec, partials);
  const unsigned g2 = (unsigned)C;
  switch (out_dtype) {
    case ST_F32:
    case ST_F32_BF16X3:
      colsum_final_kernel<float><<<g2, 256, 0, stream>>>(partials, G, C, (float*)out);
      break;
    case ST_F16:
      colsum_final_kernel<_Float16><<<g2, 256, 0, stream>>>(partials, G, C, (_Float16*)out);
      break;
    case ST_BF16:
      colsum_final_kernel<__bf16><<<g2, 256, 0, stream>>>(partials, G, C, (__bf16*)out);
      break;
    default:
      return ST_ERR_UNSUPPORTED;
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}
}  // namespace st

// ------------------------------------------------ allocation-free column sum
//
// st_column_sum_noalloc keeps the column sum's partials in `scratch`, a
// library-owned device array (one copy per GPU, alive until the process
// ends), instead of a caller workspace.  In host code `scratch` names a
// host-side stand-in, not device memory: the device address comes from
// hipGetSymbolAddress, taken once per device with that device current, and
// only that address is ever handed to a kernel.
static constexpr int kNoAllocMaxDevices = 64;
static __device__ __align__(256) float scratch[st::kColSumBlocks * ST_COLUMN_SUM_NOALLOC_MAX_C];
static float* g_scratch_dev[kNoAllocMaxDevices] = {};
static std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the device's first call).
static int scratch_address(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) return ST_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return ST_ERR_HIP;
    g_scratch_dev[dev] = (float*)p;
  }
  *out = g_scratch_dev[dev];
  return ST_OK;
}

static bool lookup_ok(const st_lookup* lk) {
  return lk && lk->K > 0 && lk->K <= ST_MAX_KVOL && lk->mul >= 1 && lk->div >= 1 && (lk->sign == 1 || lk->sign == -1);
}

extern "C" {

int st_column_sum(const void* Y, int64_t n, int C, int dtype, float* partials, void* out, int out_dtype,
                  st_stream_t stream) {
  if (n < 0 || C <= 0 || !partials || !out || (n > 0 && !Y)) return ST_ERR_ARG;
  ST_DISPATCH_DTYPE(dtype, T, st::column_sum<T>((const T*)Y, n, C, partials, out, out_dtype, stream));
}

int st_column_sum_noalloc(const void* Y, int64_t n, int C, int dtype, void* out, int out_dtype,
                          st_stream_t stream) {
  if (n < 0 || C <= 0 || C > ST_COLUMN_SUM_NOALLOC_MAX_C || !out || (n > 0 && !Y)) return ST_ERR_ARG;
  if (stream) {  // the stream must run on the current device, whose copy of the array is used
    int cur = -1, sdev = -1;
    if (hipGetDevice(&cur) != hipSuccess || hipStreamGetDevice(stream, &sdev) != hipSuccess) return ST_ERR_HIP;
    if (cur != sdev) return ST_ERR_ARG;
  }
  float* partials = nullptr;
  const int rc = scratch_address(&partials);
  if (rc != ST_OK) return rc;
  // every partial row the second pass reads is written by the first: nothing to clear
  ST_DISPATCH_DTYPE(dtype, T, st::column_sum<T>((const T*)Y, n, C, partials, out, out_dtype, stream));
}

int st_weight_prep(const void* w, void* out, int K, int C_in, int C_out, int mode, int dtype, st_stream_t stream) {
  if (!w || !out || K <= 0 || C_in <= 0 || C_out <= 0 || mode < 0 || mode > 2) return ST_ERR_ARG;
  ST_DISPATCH_DTYPE(dtype, T, ops_weight_prep<T>((const T*)w, (T*)out, K, C_in, C_out, mode, stream));
}

int st_gather_gemm(const void* A, int64_t n_src, const int32_t* map, int64_t map_k_stride, int64_t map_r_stride,
                   const uint32_t* row_masks, int mask_words, const int32_t* perm, const void* Bt, const void* bias, void* out,
                   int64_t n_dst, int K, int Kd, int Nd, int dtype, st_stream_t stream) {
  if (n_src < 0 || n_dst < 0 || K <= 0 || K > ST_MAX_KVOL || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (n_dst >= (1ll << 31) || n_src >= (1ll << 31)) return ST_ERR_ARG;
  if (row_masks && mask_words != (K + 31) / 32) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!map || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  if (n_src == 0) return fill_output(out, n_dst, Nd, dtype, bias, stream);
  const int W = (K + 31) / 32;
  if (dtype == ST_F32_BF16X3)
    return ops_gather_map_x3((const float*)A, n_src, map, map_k_stride, map_r_stride, row_masks, W, perm,
                             (const float*)Bt, (float*)out, bias_epi<float>(bias), n_dst, K, Kd, Nd, stream);
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_gather_map<T>((const T*)A, n_src, map, map_k_stride, map_r_stride, row_masks, W, perm,
                                      (const T*)Bt, (T*)out, bias_epi<T>(bias), n_dst, K, Kd, Nd, stream));
}

int st_gather_gemm_tiled(const void* A, int64_t n_src, const int32_t* perm, const int32_t* tile_nk,
                         const int16_t* tile_klist, const int32_t* tile_map, const void* Bt, const void* bias, void* out,
                         int64_t n_dst, int K, int Kd, int Nd, int dtype, int flags, st_stream_t stream) {
  if (n_src < 0 || n_dst < 0 || K <= 0 || K > ST_MAX_KVOL || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (flags & ~ST_GATHER_REVERSE_K) return ST_ERR_ARG;
  const int rev = (flags & ST_GATHER_REVERSE_K) ? 1 : 0;
  if (n_dst >= (1ll << 31) || n_src >= (1ll << 31)) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!perm || !tile_nk || !tile_klist || !tile_map || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  if (n_src == 0) return fill_output(out, n_dst, Nd, dtype, bias, stream);
  if (dtype == ST_F32_BF16X3)
    return ops_gather_tiled_x3((const float*)A, n_src, perm, tile_nk, tile_klist, tile_map, (const float*)Bt,
                               (float*)out, bias_epi<float>(bias), n_dst, K, Kd, Nd, stream, rev);
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_gather_tiled<T>((const T*)A, n_src, perm, tile_nk, tile_klist, tile_map, (const T*)Bt,
                                        (T*)out, bias_epi<T>(bias), n_dst, K, Kd, Nd, stream, rev));
}

int st_gather_gemm_tiled_epilogue(const void* A, int64_t n_src, const int32_t* perm, const int32_t* tile_nk,
                                  const int16_t* tile_klist, const int32_t* tile_map, const void* Bt,
                                  const void* bias, const float* scale, const float* shift, const void* residual,
                                  int relu, void* out, int64_t n_dst, int K, int Kd, int Nd, int dtype,
                                  st_stream_t stream) {
  if (n_src < 0 || n_dst < 0 || K <= 0 || K > ST_MAX_KVOL || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (n_dst >= (1ll << 31) || n_src >= (1ll << 31)) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!perm || !tile_nk || !tile_klist || !tile_map || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  if (shift && !scale) return ST_ERR_ARG;
  if (dtype == ST_F32_BF16X3) {
    const Epi<float> epi{(const float*)bias, scale, shift, (const float*)residual, relu ? 1 : 0};
    if (n_src == 0) return fill_output_epi<float>(out, n_dst, Nd, epi, stream);
    return ops_gather_tiled_x3((const float*)A, n_src, perm, tile_nk, tile_klist, tile_map, (const float*)Bt,
                               (float*)out, epi, n_dst, K, Kd, Nd, stream, 0);
  }
  ST_DISPATCH_DTYPE(dtype, T, (n_src == 0)
                                  ? fill_output_epi<T>(out, n_dst, Nd, Epi<T>{(const T*)bias, scale, shift, (const T*)residual, relu ? 1 : 0},
                                                       stream)
                                  : ops_gather_tiled<T>((const T*)A, n_src, perm, tile_nk, tile_klist, tile_map,
                                                        (const T*)Bt, (T*)out,
                                                        Epi<T>{(const T*)bias, scale, shift, (const T*)residual, relu ? 1 : 0}, n_dst, K,
                                                        Kd, Nd, stream, 0));
}

int st_wgrad(const void* X, int64_t n_in, const void* dY, const int32_t* map, int64_t map_k_stride,
             int64_t map_r_stride, const int32_t* rows, int64_t n_out, int K, int C_in, int C_out, int dtype,
             float* partials, int64_t splits, void* dW, int dw_dtype, st_stream_t stream) {
  if (n_in < 0 || n_out < 0 || K <= 0 || K > ST_MAX_KVOL || C_in <= 0 || C_out <= 0 || splits < 1 || splits > 65535)
    return ST_ERR_ARG;
  if (n_out >= (1ll << 31)) return ST_ERR_ARG;
  if (!partials || !dW || (n_out > 0 && (!X || !dY || !map))) return ST_ERR_ARG;
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_wgrad_map<T>((const T*)X, n_in, (const T*)dY, map, map_k_stride, map_r_stride, rows, n_out, K, C_in,
                                     C_out, partials, splits, dW, dw_dtype, stream));
}

int st_wgrad_pairs(const void* X, int64_t n_in, const void* dY, int64_t n_out, const int32_t* pairs,
                   const int32_t* kstart, const int32_t* cstart, int K, int chunk, int64_t max_chunks,
                   const int32_t* chunk_order, int C_in, int C_out, int dtype, float* partials, void* dW, int dw_dtype,
                   st_stream_t stream) {
  if (K <= 0 || K > ST_MAX_KVOL || (chunk <= 0 && chunk != ST_PAIR_CHUNK_AUTO) || max_chunks < 0 ||
      max_chunks >= (1ll << 31) || C_in <= 0 ||
      C_out <= 0 || n_in < 0 || n_out < 0)
    return ST_ERR_ARG;
  if (!kstart || !cstart || !partials || !dW || (max_chunks > 0 && (!pairs || !X || !dY))) return ST_ERR_ARG;
  if (dtype == ST_F32_BF16X3)
    return ops_wgrad_pairs_x3((const float*)X, n_in, (const float*)dY, n_out, pairs, kstart, cstart, chunk_order, K,
                              chunk, max_chunks, C_in, C_out, partials, dW, dw_dtype, stream);
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_wgrad_pairs<T>((const T*)X, n_in, (const T*)dY, n_out, pairs, kstart, cstart, chunk_order, K,
                                       chunk, max_chunks, C_in, C_out, partials, dW, dw_dtype, stream));
}

int st_subm_fly_ok(int64_t n, int Kd, int Nd, int K, int dtype) {
  if (dtype != ST_BF16 && dtype != ST_F16 && dtype != ST_F32_BF16X3) return 0;
  if (n < 0) return 0;
  // the operand sizes of n rows (the wide kernel's 32-bit buffer offsets); alignment is checked
  // per call, 16 bytes being the alignment torch allocations have
  return fly_ok(Kd, Nd, K, dtype == ST_F32_BF16X3 ? 4 : 2, dtype == ST_F32_BF16X3, n, nullptr, nullptr) ? 1 : 0;
}

int st_subm_fly_gemm(const void* A, const void* coords, int coord_dtype, int64_t n, const int32_t* offsets, int K,
                     int64_t batches, int64_t sx, int64_t sy, int64_t sz, const void* index, int64_t index_bytes,
                     const int32_t* rows, const void* Bt, const void* bias, void* out, int Kd, int Nd, int dtype,
                     int flags, st_stream_t stream) {
  const int64_t need = subm_workspace_bytes(n, batches, sx, sy, sz);
  if (need < 0 || index_bytes < need || K <= 0 || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (flags & ~ST_GATHER_REVERSE_K) return ST_ERR_ARG;
  const int rev = (flags & ST_GATHER_REVERSE_K) ? 1 : 0;
  if (!st_subm_fly_ok(n, Kd, Nd, K, dtype)) return ST_ERR_UNSUPPORTED;
  if (n == 0) return ST_OK;
  if (!A || !coords || !offsets || !index || !Bt || !out) return ST_ERR_ARG;
  SubmIndex ix;
  subm_view(const_cast<void*>(index), n, batches, sx, sy, sz, &ix);
  switch (dtype) {
    case ST_F32_BF16X3:
      return ops_gather_fly_x3((const float*)A, n, coords, coord_dtype, offsets, K, ix, rows, rev, (const float*)Bt,
                               (float*)out, (const float*)bias, Kd, Nd, stream);
    case ST_BF16:
      return ops_gather_fly<__bf16>((const __bf16*)A, n, coords, coord_dtype, offsets, K, ix, rows, rev,
                                    (const __bf16*)Bt, (__bf16*)out, (const __bf16*)bias, Kd, Nd, stream);
    case ST_F16:
      return ops_gather_fly<_Float16>((const _Float16*)A, n, coords, coord_dtype, offsets, K, ix, rows, rev,
                                      (const _Float16*)Bt, (_Float16*)out, (const _Float16*)bias, Kd, Nd, stream);
    default:
      return ST_ERR_UNSUPPORTED;
  }
}

int st_hashfly_gemm(const void* A, int64_t n_src, const void* dst_coords, int coord_dtype, int64_t n_dst,
                    const int32_t* offsets, const st_lookup* lk, const uint64_t* keys, const uint32_t* vals,
                    int64_t capacity, const void* Bt, const void* bias, void* out, int Kd, int Nd, int dtype,
                    st_stream_t stream) {
  if (!lookup_ok(lk) || n_src < 0 || n_dst < 0 || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (capacity <= 0 || capacity >= (1ll << 31) || n_dst >= (1ll << 31)) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!dst_coords || !offsets || !keys || !vals || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  if (n_src == 0) return fill_output(out, n_dst, Nd, dtype, bias, stream);
  if (dtype == ST_F32_BF16X3)
    return ops_gather_hash_x3((const float*)A, n_src, dst_coords, coord_dtype, offsets, lk, keys, vals, capacity,
                              (const float*)Bt, (float*)out, bias_epi<float>(bias), n_dst, Kd, Nd, stream);
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_gather_hash<T>((const T*)A, n_src, dst_coords, coord_dtype, offsets, lk, keys, vals, capacity,
                                       (const T*)Bt, (T*)out, bias_epi<T>(bias), n_dst, Kd, Nd, stream));
}

int st_hashfly_wgrad(const void* X, int64_t n_in, const void* dY, const void* out_coords, int coord_dtype,
                     int64_t n_out, const int32_t* offsets, const st_lookup* lk, const uint64_t* keys,
                     const uint32_t* vals, int64_t capacity, int C_in, int C_out, int dtype, float* partials,
                     int64_t splits, void* dW, int dw_dtype, st_stream_t stream) {
  if (!lookup_ok(lk) || n_in < 0 || n_out < 0 || C_in <= 0 || C_out <= 0 || splits < 1 || splits > 65535)
    return ST_ERR_ARG;
  if (capacity <= 0 || capacity >= (1ll << 31) || n_out >= (1ll << 31)) return ST_ERR_ARG;
  if (!partials || !dW || (n_out > 0 && (!X || !dY || !out_coords || !offsets || !keys || !vals)))
    return ST_ERR_ARG;
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_wgrad_hash<T>((const T*)X, n_in, (const T*)dY, out_coords, coord_dtype, n_out, offsets, lk,
                                      keys, vals, capacity, C_in, C_out, partials, splits, dW, dw_dtype, stream));
}

}  // extern "C"
