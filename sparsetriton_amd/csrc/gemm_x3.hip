// Split-operand (3 x bf16 MFMA) fp32 gather-GEMM and weight-gradient launchers.
#include "gemm_x3.h"

namespace st {

int ops_gather_map_x3(const float* A, int64_t n_src, const int32_t* map, int64_t ks, int64_t rs,
                      const uint32_t* masks, int W, const int32_t* rows, const float* Bt, float* out, Epi<float> epi, int64_t n_dst,
                      int K, int Kd, int Nd, hipStream_t stream) {
  MapSrc src{map, ks, rs};
  return launch_gather_x3(A, n_src, src, masks, W, rows, Bt, out, epi, n_dst, K, Kd, Nd, stream);
}

int ops_gather_hash_x3(const float* A, int64_t n_src, const void* coords, int coord_dtype, const int32_t* offsets,
                       const st_lookup* lk, const uint64_t* keys, const uint32_t* vals, int64_t cap, const float* Bt,
                       float* out, Epi<float> epi, int64_t n_dst, int Kd, int Nd, hipStream_t stream) {
  const int W = (lk->K + 31) / 32;
  if (coord_dtype == ST_COORD_I16)
    return launch_gather_x3(A, n_src, make_hash_src<int16_t>(coords, offsets, lk, keys, vals, cap), nullptr, W,
                            nullptr, Bt, out, epi, n_dst, lk->K, Kd, Nd, stream);
  if (coord_dtype == ST_COORD_I32)
    return launch_gather_x3(A, n_src, make_hash_src<int32_t>(coords, offsets, lk, keys, vals, cap), nullptr, W,
                            nullptr, Bt, out, epi, n_dst, lk->K, Kd, Nd, stream);
  return ST_ERR_UNSUPPORTED;
}

int ops_gather_tiled_x3(const float* A, int64_t n_src, const int32_t* perm, const int32_t* nk, const int16_t* klist,
                        const int32_t* tmap, const float* Bt, float* out, Epi<float> epi, int64_t n_dst, int K, int Kd, int Nd,
                        hipStream_t stream, int rev) {
  TiledSrc src{nk, klist, tmap, K, rev};
  return launch_gather_x3(A, n_src, src, nullptr, (K + 31) / 32, perm, Bt, out, epi, n_dst, K, Kd, Nd, stream);
}

int ops_gather_fly_x3(const float* A, int64_t n, const void* coords, int coord_dtype, const int32_t* offsets, int K,
                      const SubmIndex& ix, const int32_t* rows, int rev, const float* Bt, float* out,
                      const float* bias, int Kd, int Nd, hipStream_t stream) {
  if (!fly_ok(Kd, Nd, K, sizeof(float), true, n, A, Bt)) return ST_ERR_UNSUPPORTED;
  const BiasEpi<float> epi{bias};
  if (coord_dtype == ST_COORD_I16)
    launch_wide<float, true>(A, n, FlySrc<int16_t>{(const int16_t*)coords, offsets, ix, K, rows, rev}, nullptr, Bt, out, epi, n,
                             Kd, Nd, stream);
  else if (coord_dtype == ST_COORD_I32)
    launch_wide<float, true>(A, n, FlySrc<int32_t>{(const int32_t*)coords, offsets, ix, K, rows, rev}, nullptr, Bt, out, epi, n,
                             Kd, Nd, stream);
  else
    return ST_ERR_UNSUPPORTED;
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int ops_wgrad_pairs_x3(const float* X, int64_t n_in, const float* dY, int64_t n_out, const int32_t* pairs,
                       const int32_t* kstart, const int32_t* cstart, const int32_t* chunk_order, int K, int chunk,
                       int64_t max_chunks, int Cin, int Cout, float* partials, void* dW, int dw_dtype,
                       hipStream_t stream) {
  const bool fits = Cin % 64 == 0 && Cout % 64 == 0 && (uintptr_t)X % 16 == 0 && (uintptr_t)dY % 16 == 0;
  if (!fits)
    return ops_wgrad_pairs<float>(X, n_in, dY, n_out, pairs, kstart, cstart, chunk_order, K, chunk, max_chunks, Cin,
                                  Cout, partials, dW, dw_dtype, stream);
  if (max_chunks > 0) {
    const unsigned gx = wgrad_grid(max_chunks);
    const unsigned grid = gx * (unsigned)((Cin / 64) * (Cout / 64));
    const int2* pr = reinterpret_cast<const int2*>(pairs);
    if (rows_fit_buffer(n_in, Cin, n_out, Cout, 4))
      wgrad_pairs_x3_kernel<true><<<grid, 256, 0, stream>>>(X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin,
                                                            Cout, n_in, n_out, partials);
    else
      wgrad_pairs_x3_kernel<false><<<grid, 256, 0, stream>>>(X, dY, pr, kstart, cstart, chunk_order, K, chunk, Cin,
                                                             Cout, n_in, n_out, partials);
    ST_CHECK_LAUNCH();
  }
  return launch_wgrad_reduce(partials, cstart, 0, K, Cin, Cout, dW, dw_dtype, stream);
}

}  // namespace st
