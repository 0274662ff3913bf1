// Per-sample batch normalisation of sparse features, with the residual add
// and ReLU of the reference's blocks fused into the same pass.
//
// The reference (nn/functional/norm.py:20-112) normalises each channel of each
// sample b (rows whose coords[:, 0] == b) by that sample's own mean and biased
// variance in training, and by the running statistics in evaluation:
//   out = (y - mean[b, c]) / sqrt(var[b, c] + eps) * w[c] + beta[c]
// and moves the running statistics towards the mean over samples of the
// per-sample statistics.  Its blocks follow it with ReLU, and the residual
// block with `relu(main + shortcut)` (nn/modules/blocks.py:21-124); here
//   out = act(bn(y) + residual)
// is one elementwise pass.
//
// Statistics are sums over a sample's rows.  They are deterministic: the
// rows are cut into G contiguous ranges, one per workgroup; in a workgroup
// each thread owns a (row group, channel vector) pair and adds its rows in
// order in registers; when the sample index changes it adds them into LDS
// slots of its wave, the wave's row groups taking turns in a fixed order, so
// every slot sees its additions in an order set by the data alone.  The
// waves' slots are then summed in a fixed order into one partial per
// workgroup, and the G partials of each (sample, channel) are summed by a
// fixed tree.  Sample counts are integers (exact under atomics).
#include "common.h"

#define ST_BN_DISPATCH(dt, T, ...) \
  switch (dt) {                    \
    case ST_F32: {                 \
      using T = float;             \
      return __VA_ARGS__;          \
    }                              \
    case ST_F16: {                 \
      using T = _Float16;          \
      return __VA_ARGS__;          \
    }                              \
    case ST_BF16: {                \
      using T = __bf16;            \
      return __VA_ARGS__;          \
    }                              \
    default:                       \
      return ST_ERR_UNSUPPORTED;   \
  }

namespace st {

constexpr int kBnLds = 16384;        // 4-byte words of per-slot sums in LDS (64 KB)
constexpr int kBnMaxBlocks = 1024;   // row ranges of a statistics pass
constexpr int kBnRowsPerBlock = 512;
constexpr int kBnUnroll = 4;         // rows whose loads are issued together

static int bn_blocks(int64_t n) {
  int64_t g = (n + kBnRowsPerBlock - 1) / kBnRowsPerBlock;
  if (g > kBnMaxBlocks) g = kBnMaxBlocks;
  return (int)(g > 0 ? g : 1);
}

// Channel vectors: V consecutive channels per thread -- 16 bytes when C allows
// it (8 16-bit or 4 fp32 channels), else 4 or 1 -- and TPR threads per row in
// column blocks of at most 256 vectors (blockIdx.y); RG = 256 / TPR rows are
// handled side by side in a workgroup.
struct BnGeom {
  int V, TPR, ncb, RG;
};
static BnGeom bn_geom(int C, size_t esz, bool aligned) {
  BnGeom g;
  g.V = 1;
  if (aligned) {
    if (esz == 2 && C % 8 == 0)
      g.V = 8;
    else if (C % 4 == 0)
      g.V = 4;
  }
  const int nv = C / g.V;
  g.TPR = nv < 256 ? nv : 256;
  g.ncb = (nv + 255) / 256;
  g.RG = 256 / g.TPR;
  return g;
}

template <typename T, int V>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float (&v)[V]) {
  if constexpr (V == 1) {
    v[0] = (float)p[0];
  } else {
    typedef T vt __attribute__((ext_vector_type(V)));
    const vt q = *reinterpret_cast<const vt*>(p);
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = (float)q[e];
  }
}

template <typename T, int V>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float (&v)[V]) {
  if constexpr (V == 1) {
    p[0] = (T)v[0];
  } else {
    typedef T vt __attribute__((ext_vector_type(V)));
    vt q;
#pragma unroll
    for (int e = 0; e < V; ++e) q[e] = (T)v[e];
    *reinterpret_cast<vt*>(p) = q;
  }
}

template <int V>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&v)[V]) {
#pragma unroll
  for (int e = 0; e < V; ++e) v[e] = p[e];
}

// Per-workgroup sums over its row range, for samples [b0, b0 + bw):
//   MODE 0: y (and, for column block 0, the rows per sample)
//   MODE 1: (y - mean)^2
//   MODE 2: g and g * xhat, g = dout masked by out > 0 when relu, xhat = (y - mean) * invstd
// partials[wg][o][bl][c], o < NOUT.  rg row groups of TPR threads.  LDS slots
// belong to waves (to a row group when TPR >= 64, which spans whole waves):
// nslot = 256 / max(TPR, 64) sets of NOUT * bw * CW floats, then (MODE 0)
// nslot * bw row counts.
__host__ __device__ inline int bn_slots(int TPR) { return 256 / (TPR > 64 ? TPR : 64); }

template <typename T, typename CT, int V, int MODE>
__global__ __launch_bounds__(256) void bn_stats_kernel(const T* __restrict__ Y, const T* __restrict__ dout,
                                                       const T* __restrict__ out, int64_t n, int C,
                                                       const CT* __restrict__ coords, int b0, int bw, int rg,
                                                       int TPR, const float* __restrict__ mean,
                                                       const float* __restrict__ invstd, int relu,
                                                       float* __restrict__ partials, int32_t* __restrict__ counts) {
  constexpr int NOUT = MODE == 2 ? 2 : 1;
  constexpr int U = kBnUnroll;
  extern __shared__ __attribute__((aligned(16))) float acc_s[];
  const int tid = threadIdx.x, q = tid % TPR, sub = tid / TPR;
  const int CW = TPR * V;            // channels of this column block
  const int per = NOUT * bw * CW;    // floats per slot
  const int nslot = bn_slots(TPR);
  // slot of this thread; its row group's turn among the row groups sharing the slot
  const int slot = TPR >= 64 ? sub : tid >> 6;
  const int turn = TPR >= 64 ? 0 : sub - (tid & ~63) / TPR;
  // a wave holds at most 64 / TPR + 2 row groups (partial ones at both ends)
  const int turns = TPR >= 64 ? 1 : 64 / TPR + 2;
  const bool with_counts = MODE == 0 && counts && blockIdx.y == 0;
  int* cnt_s = reinterpret_cast<int*>(acc_s + nslot * per);
  for (int e = tid; e < nslot * per; e += 256) acc_s[e] = 0.f;
  if (with_counts)
    for (int e = tid; e < nslot * bw; e += 256) cnt_s[e] = 0;
  __syncthreads();
  const int c = blockIdx.y * CW + q * V;
  const int G = gridDim.x;
  const int64_t r0 = (int64_t)blockIdx.x * n / G, r1 = (int64_t)(blockIdx.x + 1) * n / G;
  if (sub < rg && c < C) {
    float* mine = acc_s + slot * per + q * V;
    const bool counter = with_counts && q == 0;
    float ra[NOUT][V];
    int cur = -1, cnt = 0;
    // The row groups of a slot add in turn order: one wave's LDS accesses complete
    // in program order, and the empty asm keeps the compiler from merging the turns
    // (lanes of one instruction adding into the same word would lose updates).
    auto flush = [&]() {
      if (cur < 0) return;
      for (int j = 0; j < turns; ++j) {
        if (j == turn) {
#pragma unroll
          for (int o = 0; o < NOUT; ++o)
#pragma unroll
            for (int e = 0; e < V; ++e) mine[(o * bw + cur) * CW + e] += ra[o][e];
          if (counter) cnt_s[slot * bw + cur] += cnt;
        }
        asm volatile("" ::: "memory");
      }
    };
    for (int64_t r = r0 + sub; r < r1; r += (int64_t)U * rg) {
      // loads of U rows first (rows past the range read the range's first row and are dropped)
      int bq[U];
      float y[U][V], gv[U][V];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t rr0 = r + (int64_t)u * rg;
        const bool live = rr0 < r1;
        const int64_t rr = live ? rr0 : r0;
        const int64_t bb = (coords ? (int64_t)coords[rr * 4] : 0) - b0;  // no coords: every row is sample 0
        bq[u] = (live && bb >= 0 && bb < bw) ? (int)bb : -1;
        load_vec<T, V>(Y + rr * C + c, y[u]);
        if constexpr (MODE == 2) {
          load_vec<T, V>(dout + rr * C + c, gv[u]);
          if (relu) {
            float ov[V];
            load_vec<T, V>(out + rr * C + c, ov);
#pragma unroll
            for (int e = 0; e < V; ++e)
              if (!(ov[e] > 0.f)) gv[u][e] = 0.f;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int b = bq[u];
        if (b < 0) continue;
        if (b != cur) {
          flush();
          cur = b;
          cnt = 0;
#pragma unroll
          for (int o = 0; o < NOUT; ++o)
#pragma unroll
            for (int e = 0; e < V; ++e) ra[o][e] = 0.f;
        }
        ++cnt;
        if constexpr (MODE == 0) {
#pragma unroll
          for (int e = 0; e < V; ++e) ra[0][e] += y[u][e];
        } else {
          float m[V];
          load_f32<V>(mean + (int64_t)(b0 + b) * C + c, m);
          if constexpr (MODE == 1) {
#pragma unroll
            for (int e = 0; e < V; ++e) {
              const float d = y[u][e] - m[e];
              ra[0][e] += d * d;
            }
          } else {
            float is[V];
            load_f32<V>(invstd + (int64_t)(b0 + b) * C + c, is);
#pragma unroll
            for (int e = 0; e < V; ++e) {
              ra[0][e] += gv[u][e];
              ra[1][e] += gv[u][e] * ((y[u][e] - m[e]) * is[e]);
            }
          }
        }
      }
    }
    flush();
  }
  __syncthreads();
  // slots summed in order; one partial per workgroup
  for (int e = tid; e < per; e += 256) {
    float s = 0.f;
    for (int j = 0; j < nslot; ++j) s += acc_s[j * per + e];
    const int cc = e % CW, ob = e / CW;
    const int ch = blockIdx.y * CW + cc;
    if (ch < C) partials[((int64_t)blockIdx.x * NOUT * bw + ob) * C + ch] = s;
  }
  if (with_counts)
    for (int bl = tid; bl < bw; bl += 256) {
      int t = 0;
      for (int j = 0; j < nslot; ++j) t += cnt_s[j * bw + bl];
      if (t) atomicAdd(&counts[b0 + bl], t);
    }
}

// S[o][b0 + bl][c] = sum over workgroups of partials[wg][o][bl][c] (fixed tree);
// one workgroup per (o, bl, c).  With `mean` (the MODE 0 sums, whose sample
// counts are complete by now) it also writes mean[b][c] = S / max(count[b], 1).
__global__ __launch_bounds__(256) void bn_reduce_kernel(const float* __restrict__ partials, int G, int NOUT, int bw,
                                                        int C, int b0, int B, float* __restrict__ S,
                                                        const int32_t* __restrict__ counts,
                                                        float* __restrict__ mean) {
  __shared__ float red[256];
  const int col = blockIdx.x, tid = threadIdx.x;
  const int width = NOUT * bw * C;
  float s = 0.f;
  for (int g = tid; g < G; g += 256) s += partials[(int64_t)g * width + col];
  red[tid] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) {
    const int c = col % C, ob = col / C, bl = ob % bw, o = ob / bw;
    S[((int64_t)o * B + b0 + bl) * C + c] = red[0];
    if (mean) {
      const int cnt = counts[b0 + bl];
      mean[(int64_t)(b0 + bl) * C + c] = red[0] / (float)(cnt > 1 ? cnt : 1);
    }
  }
}

// mean[b][c] = S1[b][c] / max(count[b], 1)
__global__ __launch_bounds__(256) void bn_mean_kernel(const float* __restrict__ S1, const int32_t* __restrict__ counts,
                                                      int B, int C, float* __restrict__ mean) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)B * C) return;
  const int cnt = counts[i / C];
  mean[i] = S1[i] / (float)(cnt > 1 ? cnt : 1);
}

// invstd[b][c] = 1 / sqrt(S2[b][c] / max(count[b], 1) + eps); running statistics
// (when given) move by `momentum` towards the mean over all B samples of the
// per-sample mean and biased variance (norm.py:86-90).
__global__ __launch_bounds__(256) void bn_var_kernel(const float* __restrict__ S2, const int32_t* __restrict__ counts,
                                                     const float* __restrict__ mean, int B, int C, float eps,
                                                     float momentum, float* __restrict__ running_mean,
                                                     float* __restrict__ running_var, float* __restrict__ invstd) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < (int64_t)B * C) {
    const int cnt = counts[i / C];
    const float var = S2[i] / (float)(cnt > 1 ? cnt : 1);
    invstd[i] = 1.0f / sqrtf(var + eps);
  }
  if (i < C && (running_mean || running_var)) {
    float sm = 0.f, sv = 0.f;
    for (int b = 0; b < B; ++b) {
      const int cnt = counts[b];
      const float d = (float)(cnt > 1 ? cnt : 1);
      sm += mean[(int64_t)b * C + i];
      sv += S2[(int64_t)b * C + i] / d;
    }
    if (running_mean) running_mean[i] = (1.f - momentum) * running_mean[i] + momentum * (sm / (float)B);
    if (running_var) running_var[i] = (1.f - momentum) * running_var[i] + momentum * (sv / (float)B);
  }
}

// evaluation statistics: mean = running_mean, invstd = 1 / sqrt(running_var + eps)
__global__ __launch_bounds__(256) void bn_eval_stats_kernel(const float* __restrict__ running_mean,
                                                            const float* __restrict__ running_var, int C, float eps,
                                                            float* __restrict__ mean, float* __restrict__ invstd) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= C) return;
  mean[i] = running_mean[i];
  invstd[i] = 1.0f / sqrtf(running_var[i] + eps);
}

// Elementwise passes: a workgroup covers U * RG rows (RG rows side by side,
// TPR threads x V channels each), the loads of a thread's U rows issued
// together.  per_sample = 0 takes row 0 of mean / invstd for every row
// (evaluation); rows whose sample index is outside [0, B) are written as zeros.
//   out = act((y - mean[b][c]) * invstd[b][c] * w[c] + beta[c] + residual)
template <typename T, typename CT, int V>
__global__ __launch_bounds__(256) void bn_apply_kernel(const T* __restrict__ Y, int64_t n, int C, int TPR,
                                                       const CT* __restrict__ coords, int B, int per_sample,
                                                       const float* __restrict__ mean, const float* __restrict__ invstd,
                                                       const float* __restrict__ w, const float* __restrict__ beta,
                                                       const T* __restrict__ residual, int relu, T* __restrict__ out) {
  constexpr int U = kBnUnroll;
  const int RG = 256 / TPR, q = threadIdx.x % TPR, sub = threadIdx.x / TPR;
  const int c = blockIdx.y * TPR * V + q * V;
  if (sub >= RG || c >= C) return;
  float wv[V], bv[V];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    wv[e] = w ? w[c + e] : 1.f;
    bv[e] = beta ? beta[c + e] : 0.f;
  }
  const int64_t base = (int64_t)blockIdx.x * U * RG + sub;
  int64_t bq[U];
  float y[U][V], rs[U][V];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = base + (int64_t)u * RG;
    const int64_t rr = r < n ? r : 0;
    bq[u] = (int64_t)coords[rr * 4];
    load_vec<T, V>(Y + rr * C + c, y[u]);
    if (residual) load_vec<T, V>(residual + rr * C + c, rs[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = base + (int64_t)u * RG;
    if (r >= n) break;
    const int64_t b = bq[u];
    float v[V];
    if (b < 0 || b >= B) {
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = 0.f;
    } else {
      const int64_t sb = per_sample ? b * C : 0;
      float m[V], is[V];
      load_f32<V>(mean + sb + c, m);
      load_f32<V>(invstd + sb + c, is);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        float t = (y[u][e] - m[e]) * is[e] * wv[e] + bv[e];
        if (residual) t += rs[u][e];
        if (relu) t = t > 0.f ? t : 0.f;
        v[e] = t;
      }
    }
    store_vec<T, V>(out + r * C + c, v);
  }
}

// dweight[c] = sum over samples of S_gx[b][c]; dbias[c] = sum of S_g[b][c]
__global__ __launch_bounds__(256) void bn_param_grad_kernel(const float* __restrict__ S, int B, int C,
                                                            float* __restrict__ dweight, float* __restrict__ dbias) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  float sg = 0.f, sgx = 0.f;
  for (int b = 0; b < B; ++b) {
    sg += S[(int64_t)b * C + c];
    sgx += S[(int64_t)(B + b) * C + c];
  }
  if (dweight) dweight[c] = sgx;
  if (dbias) dbias[c] = sg;
}

// Input gradient.  g = dout (masked by out > 0 under relu); dres = g.
// training: dy = w invstd (g - S_g / n_b - xhat S_gx / n_b)   (gradient through the
//           sample's mean and biased variance, which the reference's autograd takes)
// evaluation: dy = w invstd g
template <typename T, typename CT, int V>
__global__ __launch_bounds__(256) void bn_backward_kernel(const T* __restrict__ Y, const T* __restrict__ out,
                                                          const T* __restrict__ dout, int64_t n, int C, int TPR,
                                                          const CT* __restrict__ coords, int B, int training,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ invstd,
                                                          const int32_t* __restrict__ counts,
                                                          const float* __restrict__ S, const float* __restrict__ w,
                                                          int relu, T* __restrict__ dY, T* __restrict__ dres) {
  constexpr int U = kBnUnroll;
  const int RG = 256 / TPR, q = threadIdx.x % TPR, sub = threadIdx.x / TPR;
  const int c = blockIdx.y * TPR * V + q * V;
  if (sub >= RG || c >= C) return;
  float wv[V];
#pragma unroll
  for (int e = 0; e < V; ++e) wv[e] = w ? w[c + e] : 1.f;
  const int64_t base = (int64_t)blockIdx.x * U * RG + sub;
  int64_t bq[U];
  float y[U][V], g[U][V];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = base + (int64_t)u * RG;
    const int64_t rr = r < n ? r : 0;
    bq[u] = (int64_t)coords[rr * 4];
    load_vec<T, V>(dout + rr * C + c, g[u]);
    if (training) load_vec<T, V>(Y + rr * C + c, y[u]);
    if (relu) {
      float o[V];
      load_vec<T, V>(out + rr * C + c, o);
#pragma unroll
      for (int e = 0; e < V; ++e)
        if (!(o[e] > 0.f)) g[u][e] = 0.f;
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = base + (int64_t)u * RG;
    if (r >= n) break;
    if (dres) store_vec<T, V>(dres + r * C + c, g[u]);
    const int64_t b = bq[u];
    float d[V];
    if (b < 0 || b >= B) {
#pragma unroll
      for (int e = 0; e < V; ++e) d[e] = 0.f;
    } else if (training) {
      const int cnt = counts[b];
      const float inv_n = 1.0f / (float)(cnt > 1 ? cnt : 1);
      float m[V], is[V], sg[V], sgx[V];
      load_f32<V>(mean + b * C + c, m);
      load_f32<V>(invstd + b * C + c, is);
      load_f32<V>(S + b * C + c, sg);
      load_f32<V>(S + ((int64_t)B + b) * C + c, sgx);
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float xh = (y[u][e] - m[e]) * is[e];
        d[e] = wv[e] * is[e] * (g[u][e] - sg[e] * inv_n - xh * sgx[e] * inv_n);
      }
    } else {
      float is[V];
      load_f32<V>(invstd + c, is);
#pragma unroll
      for (int e = 0; e < V; ++e) d[e] = wv[e] * is[e] * g[u][e];
    }
    store_vec<T, V>(dY + r * C + c, d);
  }
}

// Statistics pass over all samples, in windows of samples that fit the LDS.
template <typename T, typename CT, int MODE, int V>
static void bn_stats_v(const T* Y, const T* dout, const T* out, int64_t n, int C, const CT* coords, int B,
                       const float* mean, const float* invstd, int relu, const BnGeom& gm, float* partials,
                       float* S, int32_t* counts, float* mean_out, hipStream_t stream) {
  constexpr int NOUT = MODE == 2 ? 2 : 1;
  const int G = bn_blocks(n);
  const int CW = gm.TPR * V;
  const int per_b = NOUT * CW + (MODE == 0 ? 1 : 0);  // words per sample per slot (+ its row count)
  const int nslot = bn_slots(gm.TPR);
  const int bw = (int64_t)B * per_b * nslot <= kBnLds ? B : kBnLds / (per_b * nslot);
  for (int b0 = 0; b0 < B; b0 += bw) {
    const int w = B - b0 < bw ? B - b0 : bw;
    const dim3 grid((unsigned)G, (unsigned)gm.ncb);
    const size_t lds = (size_t)nslot * w * per_b * 4;
    bn_stats_kernel<T, CT, V, MODE><<<grid, 256, lds, stream>>>(Y, dout, out, n, C, coords, b0, w, gm.RG, gm.TPR,
                                                                mean, invstd, relu, partials, counts);
    bn_reduce_kernel<<<(unsigned)(NOUT * w * C), 256, 0, stream>>>(partials, G, NOUT, w, C, b0, B, S, counts,
                                                                   MODE == 0 ? mean_out : nullptr);
  }
}

template <typename T, typename CT, int MODE>
static int bn_stats(const T* Y, const T* dout, const T* out, int64_t n, int C, const CT* coords, int B,
                    const float* mean, const float* invstd, int relu, const BnGeom& gm, float* partials, float* S,
                    int32_t* counts, float* mean_out, hipStream_t stream) {
  if (gm.V == 8) {
    if constexpr (sizeof(T) == 2)
      bn_stats_v<T, CT, MODE, 8>(Y, dout, out, n, C, coords, B, mean, invstd, relu, gm, partials, S, counts, mean_out,
                                 stream);
  } else if (gm.V == 4) {
    bn_stats_v<T, CT, MODE, 4>(Y, dout, out, n, C, coords, B, mean, invstd, relu, gm, partials, S, counts, mean_out,
                                 stream);
  } else {
    bn_stats_v<T, CT, MODE, 1>(Y, dout, out, n, C, coords, B, mean, invstd, relu, gm, partials, S, counts, mean_out,
                                 stream);
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

static dim3 bn_rows_grid(int64_t n, const BnGeom& gm) {
  const int64_t rows = (int64_t)kBnUnroll * gm.RG;
  return dim3((unsigned)((n + rows - 1) / rows), (unsigned)gm.ncb);
}

template <typename T, typename CT>
static int bn_forward(const T* Y, int64_t n, int C, const CT* coords, int B, const float* weight, const float* bias,
                      const T* residual, int relu, int training, float eps, float momentum, float* running_mean,
                      float* running_var, float* mean, float* invstd, int32_t* counts, float* ws, T* out,
                      hipStream_t stream) {
  const bool aligned = (uintptr_t)Y % 16 == 0 && (uintptr_t)out % 16 == 0 &&
                       (!residual || (uintptr_t)residual % 16 == 0);
  const BnGeom gm = bn_geom(C, sizeof(T), aligned);
  if (training) {
    const int64_t BC = (int64_t)B * C;
    float* S = ws;               // S1 then S2: B * C each
    float* S2 = ws + BC;
    float* partials = ws + 2 * BC;
    int rc = st_fill_u32((uint32_t*)counts, B, 0u, stream);
    if (rc != ST_OK) return rc;
    if (n == 0) {
      rc = st_fill_u32((uint32_t*)ws, 2 * BC, 0u, stream);
      if (rc != ST_OK) return rc;
      bn_mean_kernel<<<st_blocks(BC, 256), 256, 0, stream>>>(S, counts, B, C, mean);
    } else {
      // the reduce of these sums also writes the per-sample means
      rc = bn_stats<T, CT, 0>(Y, nullptr, nullptr, n, C, coords, B, nullptr, nullptr, 0, gm, partials, S, counts,
                              mean, stream);
      if (rc != ST_OK) return rc;
    }
    if (n > 0) {
      rc = bn_stats<T, CT, 1>(Y, nullptr, nullptr, n, C, coords, B, mean, nullptr, 0, gm, partials, S2, nullptr,
                              nullptr, stream);
      if (rc != ST_OK) return rc;
    }
    const int64_t th = BC > C ? BC : C;
    bn_var_kernel<<<st_blocks(th, 256), 256, 0, stream>>>(S2, counts, mean, B, C, eps, momentum, running_mean,
                                                          running_var, invstd);
  } else {
    bn_eval_stats_kernel<<<st_blocks(C, 256), 256, 0, stream>>>(running_mean, running_var, C, eps, mean, invstd);
  }
  if (n > 0) {
    const dim3 grid = bn_rows_grid(n, gm);
    const int Bv = training ? B : (1 << 30);
#define ST_BN_APPLY(V)                                                                                      \
  bn_apply_kernel<T, CT, V><<<grid, 256, 0, stream>>>(Y, n, C, gm.TPR, coords, Bv, training, mean, invstd,  \
                                                      weight, bias, residual, relu, out)
    if (gm.V == 8) {
      if constexpr (sizeof(T) == 2) ST_BN_APPLY(8);
    } else if (gm.V == 4) {
      ST_BN_APPLY(4);
    } else {
      ST_BN_APPLY(1);
    }
#undef ST_BN_APPLY
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

template <typename T, typename CT>
static int bn_backward(const T* Y, const T* out, const T* dout, int64_t n, int C, const CT* coords, int B,
                       const float* weight, int relu, int training, const float* mean, const float* invstd,
                       const int32_t* counts, float* ws, T* dY, T* dres, float* dweight, float* dbias,
                       hipStream_t stream) {
  const bool aligned = (uintptr_t)Y % 16 == 0 && (uintptr_t)out % 16 == 0 && (uintptr_t)dout % 16 == 0 &&
                       (uintptr_t)dY % 16 == 0 && (!dres || (uintptr_t)dres % 16 == 0);
  const BnGeom gm = bn_geom(C, sizeof(T), aligned);
  const int Bs = training ? B : 1;  // statistics rows: samples, or one row of per-channel sums
  const int64_t BC = (int64_t)Bs * C;
  float* S = ws;  // S_g then S_gx: Bs * C each
  float* partials = ws + 2 * BC;
  if (n == 0) {
    const int rc = st_fill_u32((uint32_t*)ws, 2 * BC, 0u, stream);
    if (rc != ST_OK) return rc;
  } else {
    // evaluation: per-channel sums over every row, as the statistics of one sample
    // (no coordinates: every row is sample 0; mean / invstd are per channel)
    const int rc = bn_stats<T, CT, 2>(Y, dout, out, n, C, training ? coords : (const CT*)nullptr, Bs, mean, invstd,
                                      relu, gm, partials, S, nullptr, nullptr, stream);
    if (rc != ST_OK) return rc;
  }
  if (dweight || dbias)
    bn_param_grad_kernel<<<st_blocks(C, 256), 256, 0, stream>>>(S, Bs, C, dweight, dbias);
  if (n > 0) {
    const dim3 grid = bn_rows_grid(n, gm);
    const int Bv = training ? B : (1 << 30);
#define ST_BN_BWD(V)                                                                                        \
  bn_backward_kernel<T, CT, V><<<grid, 256, 0, stream>>>(Y, out, dout, n, C, gm.TPR, coords, Bv, training,  \
                                                         mean, invstd, counts, S, weight, relu, dY, dres)
    if (gm.V == 8) {
      if constexpr (sizeof(T) == 2) ST_BN_BWD(8);
    } else if (gm.V == 4) {
      ST_BN_BWD(4);
    } else {
      ST_BN_BWD(1);
    }
#undef ST_BN_BWD
  }
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // namespace st

using namespace st;

extern "C" {

int st_bn_workspace(int64_t n, int C, int B, int64_t* floats) {
  if (n < 0 || C <= 0 || B <= 0 || B > ST_BN_MAX_BATCH || !floats) return ST_ERR_ARG;
  const int G = bn_blocks(n);
  const int64_t bw = B;  // a statistics pass writes at most NOUT * min(B, window) * C floats per workgroup
  *floats = 2 * (int64_t)B * C + (int64_t)G * 2 * bw * C;
  return ST_OK;
}

int st_bn_forward(const void* Y, int64_t n, int C, int dtype, const void* coords, int coord_dtype, int B,
                  const float* weight, const float* bias, const void* residual, int relu, int training, float eps,
                  float momentum, float* running_mean, float* running_var, float* mean, float* invstd,
                  int32_t* counts, float* workspace, int64_t workspace_floats, void* out, st_stream_t stream) {
  if (n < 0 || C <= 0 || B <= 0 || B > ST_BN_MAX_BATCH || !mean || !invstd) return ST_ERR_ARG;
  if (n > 0 && (!Y || !coords || !out)) return ST_ERR_ARG;
  if (training) {
    int64_t need = 0;
    st_bn_workspace(n, C, B, &need);
    if (!counts || !workspace || workspace_floats < need) return ST_ERR_ARG;
  } else if (!running_mean || !running_var) {
    return ST_ERR_ARG;
  }
  if (dtype == ST_F32_BF16X3) dtype = ST_F32;
  ST_DISPATCH_COORD(coord_dtype, CT, {
    ST_BN_DISPATCH(dtype, T,
                      bn_forward<T, CT>((const T*)Y, n, C, (const CT*)coords, B, weight, bias, (const T*)residual,
                                        relu, training, eps, momentum, running_mean, running_var, mean, invstd,
                                        counts, workspace, (T*)out, stream));
  });
}

int st_bn_backward(const void* Y, const void* out, const void* dout, int64_t n, int C, int dtype, const void* coords,
                   int coord_dtype, int B, const float* weight, int relu, int training, const float* mean,
                   const float* invstd, const int32_t* counts, float* workspace, int64_t workspace_floats, void* dY,
                   void* dres, float* dweight, float* dbias, st_stream_t stream) {
  if (n < 0 || C <= 0 || B <= 0 || B > ST_BN_MAX_BATCH || !mean || !invstd || !workspace) return ST_ERR_ARG;
  if (n > 0 && (!Y || !dout || !coords || !dY || (relu && !out))) return ST_ERR_ARG;
  if (training && !counts) return ST_ERR_ARG;
  int64_t need = 0;
  st_bn_workspace(n, C, training ? B : 1, &need);
  if (workspace_floats < need) return ST_ERR_ARG;
  if (dtype == ST_F32_BF16X3) dtype = ST_F32;
  ST_DISPATCH_COORD(coord_dtype, CT, {
    ST_BN_DISPATCH(dtype, T,
                      bn_backward<T, CT>((const T*)Y, (const T*)out, (const T*)dout, n, C, (const CT*)coords, B,
                                         weight, relu, training, mean, invstd, counts, workspace, (T*)dY, (T*)dres,
                                         dweight, dbias, stream));
  });
}

}  // extern "C"
