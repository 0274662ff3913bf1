/*
 * CPU oracle for the sparse-convolution hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
 * the checker / reported baseline; never by the product path.
 *
 * Two groups of functions:
 *
 * 1. Exact restatements (parity targets), all single-threaded and written for
 *    clarity, independent of the GPU design (sort + binary search instead of
 *    hashing):
 *      or_exact_kmap   compute_neighbor_indices semantics
 *                      (sparsetriton/nn/functional/conv/conv.py:12-75) with an
 *                      exact coordinate lookup.
 *      or_out_coords   output coordinates of a strided / transposed conv
 *                      (nn/functional/conv/kmap.py:213-444): candidates in
 *                      input-major / offset-minor order, stride + range
 *                      filters, first occurrence of each coordinate kept.
 *      or_fwd_f64 / or_dgrad_f64 / or_wgrad_f64
 *                      the three GEMMs of ConvPrecomputedNeighborGEMM
 *                      (conv/funcs/implicit_precomputed_gemm.py:64-230) in
 *                      float64 over an (n_out, K) row-major map.
 *
 * 2. A port of the reference's own algorithm (the CPU baseline and the
 *    defect ledger), fp32, OpenMP:
 *      ref_hash_build / ref_hash_query  utils/hash.py:116-299 -- 31-bit h1
 *                      probe start, 31-bit key2 stored as the key, probe
 *                      slot (h1 + 83492791*(step/8) + step) mod T, 128-probe
 *                      cap, T = int(1.5 N); inserts run sequentially in row
 *                      order (the GPU runs them in lockstep blocks, so which
 *                      colliding key wins a slot can differ).
 *      ref_kmap        conv.py:12-75 over that table, (n_out, K) row-major.
 *      ref_fwd_f32 / ref_dgrad_f32 / ref_wgrad_f32
 *                      output-stationary forward, scatter input gradient,
 *                      weight gradient by row slabs x offsets into per-thread
 *                      copies of dW (the reference's atomic-add grid; fp32
 *                      accumulation).
 *
 * Coordinates are int32 rows (b, x, y, z); offsets int32 (K, 3).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------ exact part */

static int64_t pack(int64_t b, int64_t x, int64_t y, int64_t z) {
  return (b << 48) | ((x & 0xFFFF) << 32) | ((y & 0xFFFF) << 16) | (z & 0xFFFF);
}

typedef struct {
  int64_t key;
  int64_t idx;
} kv_t;

static int cmp_kv(const void* a, const void* b) {
  const kv_t* p = (const kv_t*)a;
  const kv_t* q = (const kv_t*)b;
  if (p->key != q->key) return p->key < q->key ? -1 : 1;
  if (p->idx != q->idx) return p->idx < q->idx ? -1 : 1;
  return 0;
}

static int cmp_kv_idx(const void* a, const void* b) {
  const kv_t* p = (const kv_t*)a;
  const kv_t* q = (const kv_t*)b;
  return p->idx < q->idx ? -1 : (p->idx > q->idx ? 1 : 0);
}

/* Sorted (key, lowest idx) list of the rows of `coords` scaled by `scale`. */
static kv_t* sorted_keys(const int32_t* coords, int64_t n, int64_t scale, int64_t* n_unique) {
  kv_t* kv = (kv_t*)malloc(sizeof(kv_t) * (size_t)(n > 0 ? n : 1));
  for (int64_t i = 0; i < n; ++i) {
    const int32_t* c = coords + 4 * i;
    kv[i].key = pack(c[0], (int64_t)c[1] * scale, (int64_t)c[2] * scale, (int64_t)c[3] * scale);
    kv[i].idx = i;
  }
  qsort(kv, (size_t)n, sizeof(kv_t), cmp_kv);
  int64_t m = 0;
  for (int64_t i = 0; i < n; ++i)
    if (m == 0 || kv[m - 1].key != kv[i].key) kv[m++] = kv[i];
  *n_unique = m;
  return kv;
}

static int64_t find(const kv_t* kv, int64_t m, int64_t key) {
  int64_t lo = 0, hi = m - 1;
  while (lo <= hi) {
    int64_t mid = (lo + hi) / 2;
    if (kv[mid].key == key) return kv[mid].idx;
    if (kv[mid].key < key)
      lo = mid + 1;
    else
      hi = mid - 1;
  }
  return -1;
}

/* nbr[o*K + k] = index of in_coords row (scaled by in_scale) equal to
 * out[o]*stride - offsets[k], if 0 <= q < shape, else -1. */
int or_exact_kmap(const int32_t* in_coords, int64_t n_in, int64_t in_scale, const int32_t* out_coords,
                  int64_t n_out, const int32_t* offsets, int K, int64_t stride, int64_t sx, int64_t sy, int64_t sz,
                  int32_t* nbr) {
  int64_t m;
  kv_t* kv = sorted_keys(in_coords, n_in, in_scale, &m);
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < n_out; ++o) {
    const int32_t* c = out_coords + 4 * o;
    for (int k = 0; k < K; ++k) {
      int64_t qx = (int64_t)c[1] * stride - offsets[3 * k];
      int64_t qy = (int64_t)c[2] * stride - offsets[3 * k + 1];
      int64_t qz = (int64_t)c[3] * stride - offsets[3 * k + 2];
      int32_t r = -1;
      if (qx >= 0 && qx < sx && qy >= 0 && qy < sy && qz >= 0 && qz < sz) r = (int32_t)find(kv, m, pack(c[0], qx, qy, qz));
      nbr[o * K + k] = r;
    }
  }
  free(kv);
  return 0;
}

/* Output coordinates; returns their count (out must hold n*K rows). */
int64_t or_out_coords(const int32_t* in, int64_t n, const int32_t* offsets, int K, int64_t stride, int transposed,
                      int64_t ox_max, int64_t oy_max, int64_t oz_max, int32_t* out) {
  kv_t* cand = (kv_t*)malloc(sizeof(kv_t) * (size_t)(n * K > 0 ? n * K : 1));
  int64_t nc = 0;
  const int64_t lim[3] = {ox_max, oy_max, oz_max}; /* inclusive upper bounds (new_shape - 1) */
  for (int64_t i = 0; i < n; ++i) {
    for (int k = 0; k < K; ++k) {
      int64_t o[3];
      int ok = 1;
      for (int a = 0; a < 3; ++a) {
        int64_t v;
        if (transposed) {
          v = (int64_t)in[4 * i + 1 + a] * stride + offsets[3 * k + a];
        } else {
          v = (int64_t)in[4 * i + 1 + a] + offsets[3 * k + a];
          /* floor-mod semantics of the reference's torch `%`, then floor division */
          int64_t r = ((v % stride) + stride) % stride;
          if (r != 0) ok = 0;
          v = (v - r) / stride;
        }
        if (v < 0 || v > lim[a]) ok = 0;
        o[a] = v;
      }
      if (!ok) continue;
      cand[nc].key = pack(in[4 * i], o[0], o[1], o[2]);
      cand[nc].idx = i * K + k;
      ++nc;
    }
  }
  qsort(cand, (size_t)nc, sizeof(kv_t), cmp_kv);
  int64_t m = 0;
  for (int64_t j = 0; j < nc; ++j)
    if (m == 0 || cand[m - 1].key != cand[j].key) cand[m++] = cand[j];
  qsort(cand, (size_t)m, sizeof(kv_t), cmp_kv_idx);
  for (int64_t j = 0; j < m; ++j) {
    int64_t key = cand[j].key;
    out[4 * j] = (int32_t)(key >> 48);
    out[4 * j + 1] = (int32_t)(int16_t)((key >> 32) & 0xFFFF);
    out[4 * j + 2] = (int32_t)(int16_t)((key >> 16) & 0xFFFF);
    out[4 * j + 3] = (int32_t)(int16_t)(key & 0xFFFF);
  }
  free(cand);
  return m;
}

void or_fwd_f64(const double* X, int Cin, const double* W, int K, int Cout, const int32_t* nbr, int64_t n_out,
                double* out) {
  for (int64_t o = 0; o < n_out; ++o) {
    double* y = out + o * Cout;
    for (int j = 0; j < Cout; ++j) y[j] = 0.0;
    for (int k = 0; k < K; ++k) {
      int32_t i = nbr[o * K + k];
      if (i < 0) continue;
      const double* x = X + (int64_t)i * Cin;
      const double* w = W + (int64_t)k * Cin * Cout;
      for (int c = 0; c < Cin; ++c)
        for (int j = 0; j < Cout; ++j) y[j] += x[c] * w[c * Cout + j];
    }
  }
}

void or_dgrad_f64(const double* dY, int Cout, const double* W, int K, int Cin, const int32_t* nbr, int64_t n_out,
                  int64_t n_in, double* dX) {
  memset(dX, 0, sizeof(double) * (size_t)(n_in * Cin));
  for (int64_t o = 0; o < n_out; ++o) {
    const double* g = dY + o * Cout;
    for (int k = 0; k < K; ++k) {
      int32_t i = nbr[o * K + k];
      if (i < 0) continue;
      double* dx = dX + (int64_t)i * Cin;
      const double* w = W + (int64_t)k * Cin * Cout;
      for (int c = 0; c < Cin; ++c) {
        double s = 0.0;
        for (int j = 0; j < Cout; ++j) s += g[j] * w[c * Cout + j];
        dx[c] += s;
      }
    }
  }
}

void or_wgrad_f64(const double* X, int Cin, const double* dY, int Cout, const int32_t* nbr, int64_t n_out, int K,
                  double* dW) {
  memset(dW, 0, sizeof(double) * (size_t)K * Cin * Cout);
  for (int64_t o = 0; o < n_out; ++o) {
    const double* g = dY + o * Cout;
    for (int k = 0; k < K; ++k) {
      int32_t i = nbr[o * K + k];
      if (i < 0) continue;
      const double* x = X + (int64_t)i * Cin;
      double* dw = dW + (int64_t)k * Cin * Cout;
      for (int c = 0; c < Cin; ++c)
        for (int j = 0; j < Cout; ++j) dw[c * Cout + j] += x[c] * g[j];
    }
  }
}

/* ------------------------------------------------- reference-algorithm port */

static uint32_t ref_h1(int32_t b, int32_t x, int32_t y, int32_t z) {
  uint32_t h = ((uint32_t)b << 24) ^ ((uint32_t)x << 16) ^ ((uint32_t)y << 8) ^ (uint32_t)z;
  return h & 0x7FFFFFFFu;
}

static int32_t ref_key2(int32_t b, int32_t x, int32_t y, int32_t z) {
  uint32_t h = ((uint32_t)b * 1000003u) ^ ((uint32_t)x * 100003u) ^ ((uint32_t)y * 10007u) ^ (uint32_t)z;
  return (int32_t)(h & 0x7FFFFFFFu);
}

static uint32_t ref_slot(uint32_t h, uint32_t step, uint32_t T) {
  return (h + 83492791u * (step / 8u) + step) % T;
}

/* Returns the number of rows dropped after 128 probes. */
int64_t ref_hash_build(const int32_t* coords, int64_t n, int32_t* keys, int32_t* vals, int64_t T) {
  int64_t dropped = 0;
  for (int64_t t = 0; t < T; ++t) keys[t] = vals[t] = -1;
  for (int64_t i = 0; i < n; ++i) {
    const int32_t* c = coords + 4 * i;
    uint32_t h = ref_h1(c[0], c[1], c[2], c[3]);
    int32_t key = ref_key2(c[0], c[1], c[2], c[3]);
    int done = 0;
    for (uint32_t step = 0; step < 128 && !done; ++step) {
      uint32_t s = ref_slot(h, step, (uint32_t)T);
      if (keys[s] == -1 || keys[s] == key) {
        keys[s] = key;
        vals[s] = (int32_t)i;
        done = 1;
      }
    }
    if (!done) ++dropped;
  }
  return dropped;
}

static int32_t ref_query1(int32_t b, int32_t x, int32_t y, int32_t z, const int32_t* keys, const int32_t* vals,
                          uint32_t T) {
  uint32_t h = ref_h1(b, x, y, z) % T;
  int32_t key = ref_key2(b, x, y, z);
  for (uint32_t step = 0; step < 128; ++step) {
    uint32_t s = ref_slot(h, step, T);
    if (keys[s] == key) return vals[s];
    if (keys[s] == -1) return -1;
  }
  return -1;
}

void ref_hash_query(const int32_t* coords, int64_t m, const int32_t* keys, const int32_t* vals, int64_t T,
                    int32_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i) {
    const int32_t* c = coords + 4 * i;
    out[i] = ref_query1(c[0], c[1], c[2], c[3], keys, vals, (uint32_t)T);
  }
}

void ref_kmap(const int32_t* out_coords, int64_t n_out, const int32_t* offsets, int K, int64_t stride, int64_t sx,
              int64_t sy, int64_t sz, const int32_t* keys, const int32_t* vals, int64_t T, int32_t* nbr) {
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < n_out; ++o) {
    const int32_t* c = out_coords + 4 * o;
    for (int k = 0; k < K; ++k) {
      int64_t qx = (int64_t)c[1] * stride - offsets[3 * k];
      int64_t qy = (int64_t)c[2] * stride - offsets[3 * k + 1];
      int64_t qz = (int64_t)c[3] * stride - offsets[3 * k + 2];
      int32_t r = -1;
      if (qx >= 0 && qx < sx && qy >= 0 && qy < sy && qz >= 0 && qz < sz)
        r = ref_query1(c[0], (int32_t)qx, (int32_t)qy, (int32_t)qz, keys, vals, (uint32_t)T);
      nbr[o * K + k] = r;
    }
  }
}

/* Output coordinates as the reference builds them (kmap.py:213-444, one chunk): candidates
 * in input-major / offset-minor order (expand_coords_kernel, :11-54) -- in + t_k, kept when
 * every axis divides by the stride and divided (normal), or in * stride + t_k (transposed) --
 * then the range filter [0, new_shape) (tile.py:6-85) and filter_unique_kernel's dedup
 * (:56-97): a table of T = 2 * n * K int32 keys (key2 of the candidate, -1 empty), probe slots
 * (h1 + 83492791 * (step / 8) + step) mod T, at most 1024 steps.  A candidate is kept when its
 * CAS finds an empty slot and dropped when the slot already holds its key2, which happens for
 * its own coordinate and for any other coordinate with the same key2 whose probe sequence
 * passes that slot.  The GPU resolves candidates in lockstep blocks; this runs them one at a
 * time in order, so it keeps each coordinate's first candidate.  Returns the number kept
 * (written to out, at most n * K rows); *exhausted counts candidates that ran out of probes
 * (dropped, as the reference drops them). */
int64_t ref_out_coords(const int32_t* in, int64_t n, const int32_t* offsets, int K, int64_t stride, int transposed,
                       int64_t sx, int64_t sy, int64_t sz, int32_t* out, int64_t* exhausted) {
  const int64_t T = 2 * n * (int64_t)K;
  int32_t* keys = (int32_t*)malloc(sizeof(int32_t) * (size_t)(T > 0 ? T : 1));
  for (int64_t t = 0; t < T; ++t) keys[t] = -1;
  const int64_t lim[3] = {sx, sy, sz};
  int64_t m = 0, ex = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int32_t* c = in + 4 * i;
    for (int k = 0; k < K; ++k) {
      int64_t o[3];
      int ok = 1;
      for (int a = 0; a < 3; ++a) {
        int64_t v = transposed ? (int64_t)c[1 + a] * stride + offsets[3 * k + a] : (int64_t)c[1 + a] + offsets[3 * k + a];
        if (!transposed && stride > 1) {
          int64_t r = v % stride;
          if (r < 0) r += stride; /* torch's % is a floor modulo */
          if (r != 0) ok = 0;
          v = (v - r) / stride;   /* floor division, as //= */
        }
        if (v < 0 || v > lim[a] - 1) ok = 0;
        o[a] = v;
      }
      if (!ok) continue;
      const uint32_t h = ref_h1(c[0], (int32_t)o[0], (int32_t)o[1], (int32_t)o[2]);
      const int32_t key = ref_key2(c[0], (int32_t)o[0], (int32_t)o[1], (int32_t)o[2]);
      int kept = 0, done = 0;
      for (uint32_t step = 0; step < 1024 && !done; ++step) {
        const uint32_t sl = ref_slot(h, step, (uint32_t)T);
        if (keys[sl] == -1) {
          keys[sl] = key;
          kept = done = 1;
        } else if (keys[sl] == key) {
          done = 1;
        }
      }
      if (!done) ++ex;
      if (kept) {
        int32_t* r = out + 4 * m++;
        r[0] = c[0];
        r[1] = (int32_t)o[0];
        r[2] = (int32_t)o[1];
        r[3] = (int32_t)o[2];
      }
    }
  }
  free(keys);
  *exhausted = ex;
  return m;
}

int or_num_threads(void);

void ref_fwd_f32(const float* X, int Cin, const float* W, int K, int Cout, const int32_t* nbr, int64_t n_out,
                 float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < n_out; ++o) {
    float* y = out + o * Cout;
    for (int j = 0; j < Cout; ++j) y[j] = 0.f;
    for (int k = 0; k < K; ++k) {
      int32_t i = nbr[o * K + k];
      if (i < 0) continue;
      const float* x = X + (int64_t)i * Cin;
      const float* w = W + (int64_t)k * Cin * Cout;
      for (int c = 0; c < Cin; ++c) {
        const float xc = x[c];
        const float* wr = w + (int64_t)c * Cout;
        for (int j = 0; j < Cout; ++j) y[j] += xc * wr[j];
      }
    }
  }
}

void ref_dgrad_f32(const float* dY, int Cout, const float* W, int K, int Cin, const int32_t* nbr, int64_t n_out,
                   int64_t n_in, float* dX) {
  memset(dX, 0, sizeof(float) * (size_t)(n_in * Cin));
  /* dX[i] += dY[o] W[k]^T for every pair (the reference's input-gradient
   * kernel, implicit_precomputed_gemm.py:129-177, with its atomic adds).  W[k]
   * is transposed once to (Cout, Cin) so each pair is Cout row updates of dX[i]
   * (the product's transpose, as the reference's tl.dot of dY and W^T).  For a
   * fixed offset each input row receives from at most one output row, so the
   * scatter is race-free with the offset loop outside. */
  float* wt = (float*)malloc(sizeof(float) * (size_t)Cin * Cout);
  if (!wt) return;
  for (int k = 0; k < K; ++k) {
    const float* w = W + (int64_t)k * Cin * Cout;
    for (int c = 0; c < Cin; ++c)
      for (int j = 0; j < Cout; ++j) wt[(int64_t)j * Cin + c] = w[(int64_t)c * Cout + j];
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < n_out; ++o) {
      int32_t i = nbr[o * K + k];
      if (i < 0) continue;
      const float* g = dY + o * Cout;
      float* dx = dX + (int64_t)i * Cin;
      for (int j = 0; j < Cout; ++j) {
        const float gj = g[j];
        const float* wr = wt + (int64_t)j * Cin;
        for (int c = 0; c < Cin; ++c) dx[c] += gj * wr[c];
      }
    }
  }
  free(wt);
}

/* The reference's weight-gradient decomposition (precomputed_bwd_weight_kernel,
 * implicit_precomputed_gemm.py:180-230): its grid is (row slabs of
 * BLOCK_SIZE_N output rows) x (offsets) x (channel tiles), each program adding
 * X[nbr[slab, k]]^T dY[slab] into dW[k] with an atomic add.  Here a thread
 * takes whole row slabs (64 rows) in turn and, per slab, every offset, adding
 * into its own copy of dW (the atomic add's place); the copies are summed in
 * thread order at the end.  Each slab's dY rows stay in cache across its K
 * offsets, so dY is streamed once. */
void ref_wgrad_f32(const float* X, int Cin, const float* dY, int Cout, const int32_t* nbr, int64_t n_out, int K,
                   float* dW) {
  const int64_t nw = (int64_t)K * Cin * Cout;
  const int64_t slab = 64, nslabs = (n_out + slab - 1) / slab;
  const int nt = or_num_threads();
  float* priv = (float*)calloc((size_t)nt * (size_t)nw, sizeof(float));
  if (!priv) return;
#pragma omp parallel
  {
#ifdef _OPENMP
    float* dwt = priv + (int64_t)omp_get_thread_num() * nw;
#else
    float* dwt = priv;
#endif
#pragma omp for schedule(static)
    for (int64_t s = 0; s < nslabs; ++s) {
      const int64_t o0 = s * slab, o1 = o0 + slab < n_out ? o0 + slab : n_out;
      for (int k = 0; k < K; ++k) {
        float* dwk = dwt + (int64_t)k * Cin * Cout;
        for (int64_t o = o0; o < o1; ++o) {
          const int32_t i = nbr[o * K + k];
          if (i < 0) continue;
          const float* x = X + (int64_t)i * Cin;
          const float* g = dY + o * Cout;
          for (int c = 0; c < Cin; ++c) {
            const float xc = x[c];
            float* wr = dwk + (int64_t)c * Cout;
            for (int j = 0; j < Cout; ++j) wr[j] += xc * g[j];
          }
        }
      }
    }
  }
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e < nw; ++e) {
    float v = 0.f;
    for (int t = 0; t < nt; ++t) v += priv[(int64_t)t * nw + e];
    dW[e] = v;
  }
  free(priv);
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void or_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n);
#else
  (void)n;
#endif
}
