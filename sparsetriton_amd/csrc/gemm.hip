// C entry points of the gather-GEMM and weight-gradient kernels
// (kernels in gemm_kernels.h, instantiated per dtype in gemm_{f32,f16,bf16}.hip).
#include "gemm_kernels.h"

ST_GEMM_OPS(extern, float)
ST_GEMM_OPS(extern, _Float16)
ST_GEMM_OPS(extern, __bf16)

namespace st {
int ops_gather_map_x3(const float* A, int64_t n_src, const int32_t* map, int64_t ks, int64_t rs,
                      const uint32_t* masks, int W, const int32_t* rows, const float* Bt, float* out, int64_t n_dst,
                      int K, int Kd, int Nd, hipStream_t stream);
int ops_gather_hash_x3(const float* A, int64_t n_src, const void* coords, int coord_dtype, const int32_t* offsets,
                       const st_lookup* lk, const uint64_t* keys, const uint32_t* vals, int64_t cap, const float* Bt,
                       float* out, int64_t n_dst, int Kd, int Nd, hipStream_t stream);
int ops_gather_tiled_x3(const float* A, int64_t n_src, const int32_t* perm, const int32_t* nk, const int16_t* klist,
                        const int32_t* tmap, const float* Bt, float* out, int64_t n_dst, int K, int Kd, int Nd,
                        hipStream_t stream);
int ops_wgrad_pairs_x3(const float* X, int64_t n_in, const float* dY, int64_t n_out, const int32_t* pairs,
                       const int32_t* kstart, const int32_t* cstart, const int32_t* chunk_order, int K, int chunk,
                       int64_t max_chunks, int Cin, int Cout, float* partials, void* dW, int dw_dtype,
                       hipStream_t stream);
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
// out[0 .. n) (16-bit units) = 0.
__global__ __launch_bounds__(256) void zero_u16_kernel(uint16_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}
}  // namespace st

// A gather-GEMM with no source rows writes zero rows.  The kernels read a
// clamped row 0 for every missing source, so they are not launched then (an
// empty A may have no storage at all).
static int zero_output(void* out, int64_t n_dst, int Nd, int dtype, hipStream_t stream) {
  const int64_t n = n_dst * Nd * ((dtype == ST_F16 || dtype == ST_BF16) ? 1 : 2);
  const int64_t blocks = (n + 255) / 256;
  st::zero_u16_kernel<<<(unsigned)(blocks < 65536 ? blocks : 65536), 256, 0, stream>>>((uint16_t*)out, n);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

static bool lookup_ok(const st_lookup* lk) {
  return lk && lk->K > 0 && lk->K <= ST_MAX_KVOL && lk->mul >= 1 && lk->div >= 1 && (lk->sign == 1 || lk->sign == -1);
}

extern "C" {

int st_weight_prep(const void* w, void* out, int K, int C_in, int C_out, int mode, int dtype, st_stream_t stream) {
  if (!w || !out || K <= 0 || C_in <= 0 || C_out <= 0 || mode < 0 || mode > 2) return ST_ERR_ARG;
  ST_DISPATCH_DTYPE(dtype, T, ops_weight_prep<T>((const T*)w, (T*)out, K, C_in, C_out, mode, stream));
}

int st_gather_gemm(const void* A, int64_t n_src, const int32_t* map, int64_t map_k_stride, int64_t map_r_stride,
                   const uint32_t* row_masks, int mask_words, const int32_t* perm, const void* Bt, void* out,
                   int64_t n_dst, int K, int Kd, int Nd, int dtype, st_stream_t stream) {
  if (n_src < 0 || n_dst < 0 || K <= 0 || K > ST_MAX_KVOL || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (n_dst >= (1ll << 31) || n_src >= (1ll << 31)) return ST_ERR_ARG;
  if (row_masks && mask_words != (K + 31) / 32) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!map || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  if (n_src == 0) return zero_output(out, n_dst, Nd, dtype, stream);
  const int W = (K + 31) / 32;
  if (dtype == ST_F32_BF16X3)
    return ops_gather_map_x3((const float*)A, n_src, map, map_k_stride, map_r_stride, row_masks, W, perm,
                             (const float*)Bt, (float*)out, n_dst, K, Kd, Nd, stream);
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_gather_map<T>((const T*)A, n_src, map, map_k_stride, map_r_stride, row_masks, W, perm,
                                      (const T*)Bt, (T*)out, n_dst, K, Kd, Nd, stream));
}

int st_gather_gemm_tiled(const void* A, int64_t n_src, const int32_t* perm, const int32_t* tile_nk,
                         const int16_t* tile_klist, const int32_t* tile_map, const void* Bt, void* out, int64_t n_dst,
                         int K, int Kd, int Nd, int dtype, st_stream_t stream) {
  if (n_src < 0 || n_dst < 0 || K <= 0 || K > ST_MAX_KVOL || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (n_dst >= (1ll << 31) || n_src >= (1ll << 31)) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!perm || !tile_nk || !tile_klist || !tile_map || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  if (n_src == 0) return zero_output(out, n_dst, Nd, dtype, stream);
  if (dtype == ST_F32_BF16X3)
    return ops_gather_tiled_x3((const float*)A, n_src, perm, tile_nk, tile_klist, tile_map, (const float*)Bt,
                               (float*)out, n_dst, K, Kd, Nd, stream);
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_gather_tiled<T>((const T*)A, n_src, perm, tile_nk, tile_klist, tile_map, (const T*)Bt,
                                        (T*)out, n_dst, K, Kd, Nd, stream));
}

int st_wgrad(const void* X, int64_t n_in, const void* dY, const int32_t* map, int64_t map_k_stride,
             int64_t map_r_stride, int64_t n_out, int K, int C_in, int C_out, int dtype, float* partials,
             int64_t splits, void* dW, int dw_dtype, st_stream_t stream) {
  if (n_in < 0 || n_out < 0 || K <= 0 || K > ST_MAX_KVOL || C_in <= 0 || C_out <= 0 || splits < 1 || splits > 65535)
    return ST_ERR_ARG;
  if (n_out >= (1ll << 31)) return ST_ERR_ARG;
  if (!partials || !dW || (n_out > 0 && (!X || !dY || !map))) return ST_ERR_ARG;
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_wgrad_map<T>((const T*)X, n_in, (const T*)dY, map, map_k_stride, map_r_stride, n_out, K, C_in,
                                     C_out, partials, splits, dW, dw_dtype, stream));
}

int st_wgrad_pairs(const void* X, int64_t n_in, const void* dY, int64_t n_out, const int32_t* pairs,
                   const int32_t* kstart, const int32_t* cstart, int K, int chunk, int64_t max_chunks,
                   const int32_t* chunk_order, int C_in, int C_out, int dtype, float* partials, void* dW, int dw_dtype,
                   st_stream_t stream) {
  if (K <= 0 || K > ST_MAX_KVOL || chunk <= 0 || max_chunks < 0 || max_chunks >= (1ll << 31) || C_in <= 0 ||
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

int st_hashfly_gemm(const void* A, int64_t n_src, const void* dst_coords, int coord_dtype, int64_t n_dst,
                    const int32_t* offsets, const st_lookup* lk, const uint64_t* keys, const uint32_t* vals,
                    int64_t capacity, const void* Bt, void* out, int Kd, int Nd, int dtype, st_stream_t stream) {
  if (!lookup_ok(lk) || n_src < 0 || n_dst < 0 || Kd <= 0 || Nd <= 0) return ST_ERR_ARG;
  if (capacity <= 0 || capacity >= (1ll << 31) || n_dst >= (1ll << 31)) return ST_ERR_ARG;
  if (n_dst == 0) return ST_OK;
  if (!dst_coords || !offsets || !keys || !vals || !Bt || !out || (n_src > 0 && !A)) return ST_ERR_ARG;
  if (n_src == 0) return zero_output(out, n_dst, Nd, dtype, stream);
  if (dtype == ST_F32_BF16X3)
    return ops_gather_hash_x3((const float*)A, n_src, dst_coords, coord_dtype, offsets, lk, keys, vals, capacity,
                              (const float*)Bt, (float*)out, n_dst, Kd, Nd, stream);
  ST_DISPATCH_DTYPE(dtype, T,
                    ops_gather_hash<T>((const T*)A, n_src, dst_coords, coord_dtype, offsets, lk, keys, vals, capacity,
                                       (const T*)Bt, (T*)out, n_dst, Kd, Nd, stream));
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
