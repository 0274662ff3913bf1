// Output coordinates and kernel maps of strided and transposed convolution.
//
// The reference materialises all N*K candidate coordinates, filters them with
// boolean indexing and dedups them with a lossy 31-bit hash whose survivor is
// whichever CAS wins (kmap.py:213-444).  Here candidates are never stored:
// each pass recomputes them in registers from the input row (thread per input
// row, offsets in LDS), and dedup uses exact 64-bit keys in an open-addressing
// table keyed on the output coordinate.  The survivor of each coordinate is
// its first candidate in input-major / offset-minor order (atomic min of the
// candidate index), so the output order is deterministic; it is the order the
// reference produces when its CAS winners happen to be first occurrences.
//
// Because each candidate (input i, offset k) that survives the filters is
// exactly one kernel-map pair (i -> output of the candidate, offset k), the
// map in both directions falls out of the same enumeration; no N_out x K
// neighbour query is needed.
#include "outgeom.h"

namespace st {

// The read-only passes handle candidates kCandGroup offsets at a time: the
// group's keys and home slots are computed first and their first probes
// loaded together, so a thread has up to kCandGroup random loads in flight.
constexpr int kCandGroup = 9;

// Key of candidate (input (b, x, y, z), offset k), or false when filtered out;
// *bad is set when it passes the filters but cannot be packed.
__device__ __forceinline__ bool cand_key(const Geom& g, const int32_t* off_s, int64_t b, int64_t x, int64_t y,
                                         int64_t z, int k, uint64_t& key, bool& bad) {
  int64_t ox, oy, oz;
  if (!candidate(g, x, y, z, off_s[3 * k], off_s[3 * k + 1], off_s[3 * k + 2], ox, oy, oz)) return false;
  if (!pack_key(b, ox, oy, oz, key)) {
    bad = true;
    return false;
  }
  return true;
}

// Inserts stay one candidate at a time: batching their first probes (as the
// read-only passes below do) put more CAS traffic on hot slots at once and
// measured slower.
template <typename CT>
__global__ __launch_bounds__(256) void cand_insert_kernel(const CT* __restrict__ coords, int64_t n,
                                                          const int32_t* __restrict__ offsets, Geom g,
                                                          uint64_t* __restrict__ dkeys, uint32_t* __restrict__ dvals,
                                                          uint32_t dcap, int32_t* __restrict__ status) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  load_offsets(off_s, offsets, g.K);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  for (int k = 0; k < g.K; ++k) {
    uint64_t key;
    bool bad = false;
    if (!cand_key(g, off_s, b, x, y, z, k, key, bad)) {
      if (bad) atomicAdd(&status[ST_STATUS_BAD_COORD], 1);
      continue;
    }
    bool was_new;
    uint32_t s = insert_slot(dkeys, dcap, key, was_new);
    if (s == ST_NO_VAL) {
      atomicAdd(&status[ST_STATUS_OVERFLOW], 1);
      continue;
    }
    atomicMin(&dvals[s], cand_rank(g, n, i, k));
  }
}

// Number of first-occurrence candidates of input row i, with the slot of each
// one reported through the callback.
template <typename CT, typename F>
__device__ __forceinline__ int first_candidates(const CT* __restrict__ coords, int64_t n, int64_t i,
                                                const int32_t* off_s, const Geom& g, int k0, int k1,
                                                const uint64_t* __restrict__ dkeys,
                                                const uint32_t* __restrict__ dvals, uint32_t dcap, F&& on_first) {
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  int cnt = 0;
  for (int kb = k0; kb < k1; kb += kCandGroup) {
    uint64_t key[kCandGroup], first[kCandGroup];
    uint32_t slot[kCandGroup], val[kCandGroup];
    bool ok[kCandGroup];
#pragma unroll
    for (int j = 0; j < kCandGroup; ++j) {
      bool bd = false;
      ok[j] = kb + j < k1 && cand_key(g, off_s, b, x, y, z, kb + j, key[j], bd);
      slot[j] = ok[j] ? home_slot(key[j], dcap) : 0u;
      first[j] = ok[j] ? dkeys[slot[j]] : ST_EMPTY_KEY;
    }
#pragma unroll
    for (int j = 0; j < kCandGroup; ++j) {
      if (ok[j]) slot[j] = find_slot_from(dkeys, dcap, key[j], slot[j], first[j]);
      ok[j] = ok[j] && slot[j] != ST_NO_VAL;
    }
#pragma unroll
    for (int j = 0; j < kCandGroup; ++j) val[j] = ok[j] ? dvals[slot[j]] : ST_NO_VAL;
#pragma unroll
    for (int j = 0; j < kCandGroup; ++j) {
      if (!ok[j] || val[j] != cand_rank(g, n, i, kb + j)) continue;
      int64_t ob, ox, oy, oz;
      unpack_key(key[j], ob, ox, oy, oz);
      on_first(slot[j], ob, ox, oy, oz);
      ++cnt;
    }
  }
  return cnt;
}

template <typename CT>
__global__ __launch_bounds__(256) void cand_count_kernel(const CT* __restrict__ coords, int64_t n,
                                                         const int32_t* __restrict__ offsets, Geom g,
                                                         const uint64_t* __restrict__ dkeys,
                                                         const uint32_t* __restrict__ dvals, uint32_t dcap,
                                                         int32_t* __restrict__ block_counts) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  __shared__ int red[8];
  load_offsets(off_s, offsets, g.K);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int k0 = blockIdx.y * g.chunk, k1 = min(g.K, k0 + g.chunk);  // this grid row's offset chunk
  int cnt = 0;
  if (i < n)
    cnt = first_candidates(coords, n, i, off_s, g, k0, k1, dkeys, dvals, dcap,
                           [](uint32_t, int64_t, int64_t, int64_t, int64_t) {});
  cnt = wave_sum(cnt);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) {
    int t = 0;
    for (int w = 0; w < (int)(blockDim.x / kWave); ++w) t += red[w];
    block_counts[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = t;
  }
}

// In-place exclusive scan of counts[0..n); counts[n] receives the total.
// One workgroup of 1024 threads; each round covers 8192 elements, 8
// consecutive ones per thread read and written as two 16-byte vectors (a
// wave covers 2 KB contiguously), with one workgroup scan per round.
constexpr int kScanPer = 8;
// In-place exclusive scan of counts[0..n), counts[n] = total, by one workgroup.
// With `pl` set (the per-(offset, row block) pair counts of st_kmap_pairs,
// n = K * nb) it also writes the pair list's kstart / cstart: kstart[k] is the
// scanned count of (k, block 0), cstart[k] the chunks of the offsets before k.
struct PairsFinal {
  int32_t* kstart;
  int32_t* cstart;
  int64_t nb;
  int K, chunk;
};
__global__ __launch_bounds__(1024) void exclusive_scan_kernel(int32_t* __restrict__ counts, int64_t n, PairsFinal pl) {
  __shared__ int scratch[17];
  const bool vec = (reinterpret_cast<uintptr_t>(counts) & 15) == 0;
  int carry = 0;
  for (int64_t base = 0; base < n; base += (int64_t)kScanPer * 1024) {
    const int64_t j0 = base + (int64_t)threadIdx.x * kScanPer;
    const bool full = vec && j0 + kScanPer <= n;
    int v[kScanPer];
    if (full) {
      const int4 lo = *reinterpret_cast<const int4*>(counts + j0);
      const int4 hi = *reinterpret_cast<const int4*>(counts + j0 + 4);
      v[0] = lo.x, v[1] = lo.y, v[2] = lo.z, v[3] = lo.w;
      v[4] = hi.x, v[5] = hi.y, v[6] = hi.z, v[7] = hi.w;
    } else {
#pragma unroll
      for (int e = 0; e < kScanPer; ++e) v[e] = j0 + e < n ? counts[j0 + e] : 0;
    }
    int sum = 0;
#pragma unroll
    for (int e = 0; e < kScanPer; ++e) sum += v[e];
    int tot;
    int run = carry + block_exclusive_scan(sum, scratch, &tot);
    int ex[kScanPer];
#pragma unroll
    for (int e = 0; e < kScanPer; ++e) {
      ex[e] = run;
      run += v[e];
    }
    if (full) {
      *reinterpret_cast<int4*>(counts + j0) = make_int4(ex[0], ex[1], ex[2], ex[3]);
      *reinterpret_cast<int4*>(counts + j0 + 4) = make_int4(ex[4], ex[5], ex[6], ex[7]);
    } else {
#pragma unroll
      for (int e = 0; e < kScanPer; ++e)
        if (j0 + e < n) counts[j0 + e] = ex[e];
    }
    carry += tot;
  }
  if (threadIdx.x == 0) counts[n] = carry;
  if (!pl.kstart) return;
  __syncthreads();  // the scanned counts of the other threads are visible to the workgroup
  // the chunk size: the caller's, or (ST_PAIR_CHUNK_AUTO) the least power of two >= 1024 with at
  // most 2048 chunks' worth of pairs in total -- so the list has at most 2048 + K chunks
  int chunk = pl.chunk;
  if (chunk <= 0) {
    chunk = kPairChunkMin;
    while ((int64_t)chunk * kPairChunksAuto < (int64_t)carry) chunk <<= 1;
  }
  // thread k < K (K <= 512): offset k's first pair and chunk count; cstart is the scan of the latter
  const int k = threadIdx.x;
  int nch = 0;
  if (k < pl.K) {
    const int32_t s0 = counts[(int64_t)k * pl.nb], s1 = k + 1 < pl.K ? counts[(int64_t)(k + 1) * pl.nb] : carry;
    pl.kstart[k] = s0;
    nch = (s1 - s0 + chunk - 1) / chunk;
  }
  int chunks;
  const int cex = block_exclusive_scan(nch, scratch, &chunks);
  if (k < pl.K) pl.cstart[k] = cex;
  if (k == 0) {
    pl.kstart[pl.K] = carry;
    pl.cstart[pl.K] = chunks;
    if (pl.chunk <= 0) pl.cstart[pl.K + 1] = chunk;  // the size the chunks were cut at
  }
}

int launch_exclusive_scan(int32_t* counts, int64_t n, hipStream_t stream) {
  exclusive_scan_kernel<<<1, 1024, 0, stream>>>(counts, n, PairsFinal{nullptr, nullptr, 0, 0, 0});
  return hipGetLastError() == hipSuccess ? ST_OK : ST_ERR_HIP;
}

template <typename CT>
__global__ __launch_bounds__(256) void cand_emit_kernel(const CT* __restrict__ coords, int64_t n,
                                                        const int32_t* __restrict__ offsets, Geom g,
                                                        const uint64_t* __restrict__ dkeys,
                                                        const uint32_t* __restrict__ dvals,
                                                        uint32_t* __restrict__ slot_out, uint32_t dcap,
                                                        const int32_t* __restrict__ block_offsets,
                                                        CT* __restrict__ out_coords) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  __shared__ int scratch[5];
  load_offsets(off_s, offsets, g.K);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int k0 = blockIdx.y * g.chunk, k1 = min(g.K, k0 + g.chunk);
  int cnt = 0;
  if (i < n)
    cnt = first_candidates(coords, n, i, off_s, g, k0, k1, dkeys, dvals, dcap,
                           [](uint32_t, int64_t, int64_t, int64_t, int64_t) {});
  int tot;
  int pos = block_offsets[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] + block_exclusive_scan(cnt, scratch, &tot);
  if (i >= n || cnt == 0) return;
  first_candidates(coords, n, i, off_s, g, k0, k1, dkeys, dvals, dcap,
                   [&](uint32_t s, int64_t b, int64_t ox, int64_t oy, int64_t oz) {
                     CT* r = out_coords + (int64_t)pos * 4;
                     r[0] = (CT)b;
                     r[1] = (CT)ox;
                     r[2] = (CT)oy;
                     r[3] = (CT)oz;
                     slot_out[s] = (uint32_t)pos;
                     ++pos;
                   });
}

template <typename CT>
__global__ __launch_bounds__(256) void cand_map_kernel(const CT* __restrict__ coords, int64_t n,
                                                       const int32_t* __restrict__ offsets, Geom g,
                                                       const uint64_t* __restrict__ dkeys,
                                                       const uint32_t* __restrict__ slot_out, uint32_t dcap,
                                                       const uint64_t* __restrict__ in_keys,
                                                       const uint32_t* __restrict__ in_vals, uint32_t in_cap,
                                                       int64_t n_out, int32_t* __restrict__ nbr,
                                                       int32_t* __restrict__ invnbr, uint32_t* __restrict__ out_masks,
                                                       uint32_t* __restrict__ in_masks) {
  __shared__ int32_t off_s[ST_MAX_KVOL * 3];
  load_offsets(off_s, offsets, g.K);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int64_t b, x, y, z;
  load_coord(coords, i, b, x, y, z);
  if (!input_in_bounds(g, x, y, z)) return;
  if (in_keys) {
    // Only the row the input table resolves this coordinate to is a neighbour.
    const int64_t sc = g.transposed ? g.s : 1;
    uint64_t key;
    if (!pack_key(b, x * sc, y * sc, z * sc, key)) return;
    const uint32_t s = find_slot(in_keys, in_cap, key);
    if (s == ST_NO_VAL || in_vals[s] != (uint32_t)i) return;
  }
  const int W = (g.K + 31) >> 5;
  uint32_t mword = 0;
  for (int kb = 0; kb < g.K; kb += kCandGroup) {
    uint64_t key[kCandGroup], first[kCandGroup];
    uint32_t slot[kCandGroup], o[kCandGroup];
    bool ok[kCandGroup];
#pragma unroll
    for (int j = 0; j < kCandGroup; ++j) {
      bool bd = false;
      ok[j] = kb + j < g.K && cand_key(g, off_s, b, x, y, z, kb + j, key[j], bd);
      slot[j] = ok[j] ? home_slot(key[j], dcap) : 0u;
      first[j] = ok[j] ? dkeys[slot[j]] : ST_EMPTY_KEY;
    }
#pragma unroll
    for (int j = 0; j < kCandGroup; ++j) {
      if (ok[j]) slot[j] = find_slot_from(dkeys, dcap, key[j], slot[j], first[j]);
      ok[j] = ok[j] && slot[j] != ST_NO_VAL;
    }
#pragma unroll
    for (int j = 0; j < kCandGroup; ++j) o[j] = ok[j] ? slot_out[slot[j]] : ST_NO_VAL;
#pragma unroll
    for (int j = 0; j < kCandGroup; ++j) {
      const int k = kb + j;
      if (k >= g.K) break;
      if (o[j] != ST_NO_VAL && (int64_t)o[j] < n_out) {
        invnbr[(int64_t)k * n + i] = (int32_t)o[j];
        nbr[(int64_t)k * n_out + o[j]] = (int32_t)i;
        atomicOr(&out_masks[(int64_t)o[j] * W + (k >> 5)], 1u << (k & 31));
        mword |= 1u << (k & 31);
      }
      if ((k & 31) == 31 || k == g.K - 1) {
        in_masks[i * W + (k >> 5)] = mword;
        mword = 0;
      }
    }
  }
}

}  // namespace st

using namespace st;

extern "C" {

int st_outcoords_sizes(int64_t n, const st_outgeom* gin, int64_t kernel_size, int64_t dilation,
                       int64_t* dedup_capacity, int64_t* num_blocks) {
  Geom g;
  if (n < 0 || !make_geom(gin, g) || kernel_size < 1 || dilation < 1 || !dedup_capacity || !num_blocks)
    return ST_ERR_ARG;
  const int64_t kv = cands_per_input(g, kernel_size, dilation);
  // twice the candidates that can pass the filters (clamped to the 32-bit
  // slot range; a caller that overflows the table can grow it and retry)
  int64_t cap = 2 * n * kv + 64;
  if (cap > (1ll << 31) - 64) cap = (1ll << 31) - 64;
  *dedup_capacity = cap;
  *num_blocks = ((n + 255) / 256) * ((g.K + g.chunk - 1) / g.chunk);  // per (input block, offset chunk)
  return ST_OK;
}

int st_outcoords_plan(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                      const st_outgeom* gin, uint64_t* dkeys, uint32_t* dvals, int64_t dcap, int32_t* block_counts,
                      int64_t num_blocks, int32_t* status, st_stream_t stream) {
  Geom g;
  if (n < 0 || !make_geom(gin, g) || dcap <= 0 || dcap >= (1ll << 31) || !dkeys || !dvals || !block_counts ||
      !status || !offsets)
    return ST_ERR_ARG;
  const int64_t nb = (n + 255) / 256, nchunks = (g.K + g.chunk - 1) / g.chunk;
  if (num_blocks != nb * nchunks || n * nchunks * (int64_t)g.chunk >= (1ll << 32) - 1) return ST_ERR_ARG;
  if (n > 0 && !in_coords) return ST_ERR_ARG;
  if (n > 0) {
    ST_DISPATCH_COORD(coord_dtype, CT, {
      cand_insert_kernel<CT><<<(unsigned)nb, 256, 0, stream>>>((const CT*)in_coords, n, offsets, g, dkeys, dvals,
                                                               (uint32_t)dcap, status);
      cand_count_kernel<CT><<<dim3((unsigned)nb, (unsigned)nchunks), 256, 0, stream>>>(
          (const CT*)in_coords, n, offsets, g, dkeys, dvals, (uint32_t)dcap, block_counts);
    });
  }
  exclusive_scan_kernel<<<1, 1024, 0, stream>>>(block_counts, num_blocks, PairsFinal{nullptr, nullptr, 0, 0, 0});
  ST_CHECK_LAUNCH();
  return ST_OK;
}

int st_outcoords_emit(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                      const st_outgeom* gin, const uint64_t* dkeys, const uint32_t* dvals, uint32_t* slot_out,
                      int64_t dcap, const int32_t* block_counts, int64_t num_blocks, const uint64_t* in_keys,
                      const uint32_t* in_vals, int64_t in_cap, void* out_coords, int64_t n_out, int32_t* nbr,
                      int32_t* invnbr, uint32_t* out_masks, uint32_t* in_masks, st_stream_t stream) {
  Geom g;
  if (n < 0 || n_out < 0 || !make_geom(gin, g) || dcap <= 0 || dcap >= (1ll << 31) || !dkeys || !dvals ||
      !slot_out || !block_counts || !offsets)
    return ST_ERR_ARG;
  const int64_t nb = (n + 255) / 256, nchunks = (g.K + g.chunk - 1) / g.chunk;
  if (num_blocks != nb * nchunks) return ST_ERR_ARG;
  if (in_keys && (!in_vals || in_cap <= 0 || in_cap >= (1ll << 31))) return ST_ERR_ARG;
  if (n == 0 || n_out == 0) return ST_OK;
  if (!in_coords || !out_coords) return ST_ERR_ARG;
  if (nbr && (!invnbr || !out_masks || !in_masks)) return ST_ERR_ARG;
  ST_DISPATCH_COORD(coord_dtype, CT, {
    cand_emit_kernel<CT><<<dim3((unsigned)nb, (unsigned)nchunks), 256, 0, stream>>>(
        (const CT*)in_coords, n, offsets, g, dkeys, dvals, slot_out, (uint32_t)dcap, block_counts, (CT*)out_coords);
    if (nbr)
      cand_map_kernel<CT><<<(unsigned)nb, 256, 0, stream>>>(
        (const CT*)in_coords, n, offsets, g, dkeys, slot_out, (uint32_t)dcap, in_keys, in_vals, (uint32_t)in_cap,
        n_out, nbr, invnbr, out_masks, in_masks);
  });
  ST_CHECK_LAUNCH();
  return ST_OK;
}

}  // extern "C"

// ------------------------------------------------------------ map inversion

namespace st {

// One thread per output row o: every valid (k, o) -> i entry becomes
// invnbr[k][i] = o (offset-major, like the map).  For a convolution map of
// unique output coordinates each (i, k) has at most one o, so the scatter has
// no write conflicts; the in-mask bit a row's atomic OR finds already set
// reveals one, and is counted into `conflicts` (optional).
__global__ __launch_bounds__(256) void kmap_invert_kernel(const int32_t* __restrict__ nbr, int64_t ks, int64_t rs,
                                                          int64_t n_out, int K, int64_t n_in,
                                                          int32_t* __restrict__ invnbr, uint32_t* __restrict__ in_masks,
                                                          uint32_t* __restrict__ out_masks,
                                                          int32_t* __restrict__ conflicts) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n_out) return;
  const int W = (K + 31) >> 5;
  uint32_t mword = 0;
  for (int k = 0; k < K; ++k) {
    const int32_t i = nbr[(int64_t)k * ks + o * rs];
    if (i >= 0 && (int64_t)i < n_in) {
      invnbr[(int64_t)k * n_in + i] = (int32_t)o;
      const uint32_t bit = 1u << (k & 31);
      const uint32_t old = atomicOr(&in_masks[(int64_t)i * W + (k >> 5)], bit);
      if (conflicts && (old & bit)) atomicAdd(conflicts, 1);
      mword |= bit;
    }
    if ((k & 31) == 31 || k == K - 1) {
      if (out_masks) out_masks[o * W + (k >> 5)] = mword;
      mword = 0;
    }
  }
}

}  // namespace st

extern "C" int st_kmap_invert(const int32_t* nbr, int64_t nbr_k_stride, int64_t nbr_r_stride, int64_t n_out, int K,
                              int64_t n_in, int32_t* invnbr, uint32_t* in_masks, uint32_t* out_masks,
                              int32_t* conflicts, st_stream_t stream) {
  if (n_out < 0 || n_in < 0 || K <= 0 || K > ST_MAX_KVOL) return ST_ERR_ARG;
  if (n_out >= (1ll << 31) || n_in >= (1ll << 31)) return ST_ERR_ARG;
  if (n_out == 0) return ST_OK;
  if (!nbr || (n_in > 0 && (!invnbr || !in_masks))) return ST_ERR_ARG;
  st::kmap_invert_kernel<<<st_blocks(n_out, 256), 256, 0, stream>>>(nbr, nbr_k_stride, nbr_r_stride, n_out, K, n_in,
                                                                    invnbr, in_masks, out_masks, conflicts);
  ST_CHECK_LAUNCH();
  return ST_OK;
}

// ------------------------------------------------- tile-order map and pairs

namespace st {

constexpr int kPairPer = kPairRows / 256;

__device__ __forceinline__ bool pair_valid(int32_t i, int64_t n_in) { return i >= 0 && (int64_t)i < n_in; }

// counts[k * nb + b] = valid entries of offset k among rows [b*4096, b*4096+4096).
// Grid (nb, K): one workgroup per (row block, offset) reads 4096 consecutive
// entries of the offset's column, coalesced.
__global__ __launch_bounds__(256) void pairs_count_kernel(const int32_t* __restrict__ map, int64_t ks, int64_t rs,
                                                          int64_t n_out, int64_t n_in, int64_t nb,
                                                          int32_t* __restrict__ counts) {
  __shared__ int wsum_s[4];
  const int k = blockIdx.y;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int32_t* col = map + (int64_t)k * ks;
  const int64_t row0 = (int64_t)blockIdx.x * kPairRows + threadIdx.x;
  int c = 0;
#pragma unroll
  for (int j = 0; j < kPairPer; ++j) {
    const int64_t o = row0 + j * 256;
    c += (o < n_out && pair_valid(col[o * rs], n_in)) ? 1 : 0;
  }
  c = wave_sum(c);
  if (lane == 0) wsum_s[wid] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[(int64_t)k * nb + blockIdx.x] = wsum_s[0] + wsum_s[1] + wsum_s[2] + wsum_s[3];
}

// Writes the (in, out) pairs of one (row block, offset) at offsets[k * nb + b]
// + rank, the rank counting the valid rows below in row order (j, wave, lane),
// so each offset's pairs come out sorted by output row.
__global__ __launch_bounds__(256) void pairs_emit_kernel(const int32_t* __restrict__ map, int64_t ks, int64_t rs,
                                                         int64_t n_out, int64_t n_in, int64_t nb,
                                                         const int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ pairs) {
  __shared__ int cnt_s[kPairPer * 4];
  const int k = blockIdx.y;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int32_t* col = map + (int64_t)k * ks;
  const int64_t row0 = (int64_t)blockIdx.x * kPairRows + threadIdx.x;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  int32_t iv[kPairPer];
  uint64_t bal[kPairPer];
#pragma unroll
  for (int j = 0; j < kPairPer; ++j) {
    const int64_t o = row0 + j * 256;
    iv[j] = o < n_out ? col[o * rs] : -1;
    bal[j] = __ballot(pair_valid(iv[j], n_in));
    if (lane == 0) cnt_s[j * 4 + wid] = (int)__popcll(bal[j]);
  }
  __syncthreads();
  static_assert(kPairPer * 4 == 64, "one wave scans the (step, wave) counts");
  if (wid == 0) {
    const int v = cnt_s[lane];
    const int inc = wave_inclusive_scan(v);
    cnt_s[lane] = inc - v;
  }
  __syncthreads();
  const int base = offsets[(int64_t)k * nb + blockIdx.x];
#pragma unroll
  for (int j = 0; j < kPairPer; ++j) {
    if (pair_valid(iv[j], n_in)) {
      const int pos = base + cnt_s[j * 4 + wid] + (int)__popcll(bal[j] & below);
      *reinterpret_cast<int2*>(pairs + 2 * (int64_t)pos) = make_int2(iv[j], (int32_t)(row0 + j * 256));
    }
  }
}

// The same two passes for a map whose rows are contiguous (rs = 1) and whose
// columns start 16-byte aligned: 16-byte loads, a wave reading 1 KB per
// instruction.  Thread t covers rows base + 1024 q + 4 t .. + 3 for q = 0..3, so
// row order is (q, thread, element) order.  With 4-byte loads these passes
// read config 4's 768 MB map at ~3 TB/s.
__device__ __forceinline__ int4 pair_load4(const int32_t* __restrict__ col, int64_t r, int64_t n_out) {
  if (r + 4 <= n_out) return *reinterpret_cast<const int4*>(col + r);
  int4 v = make_int4(-1, -1, -1, -1);
  if (r < n_out) v.x = col[r];
  if (r + 1 < n_out) v.y = col[r + 1];
  if (r + 2 < n_out) v.z = col[r + 2];
  return v;
}

__device__ __forceinline__ uint32_t pair_bits4(int4 v, int64_t n_in) {
  return (pair_valid(v.x, n_in) ? 1u : 0u) | (pair_valid(v.y, n_in) ? 2u : 0u) | (pair_valid(v.z, n_in) ? 4u : 0u) |
         (pair_valid(v.w, n_in) ? 8u : 0u);
}

__global__ __launch_bounds__(256) void pairs_count_vec_kernel(const int32_t* __restrict__ map, int64_t ks,
                                                              int64_t n_out, int64_t n_in, int64_t nb,
                                                              int32_t* __restrict__ counts) {
  __shared__ int wsum_s[4];
  const int k = blockIdx.y;
  const int32_t* col = map + (int64_t)k * ks;
  const int64_t r0 = (int64_t)blockIdx.x * kPairRows + 4 * threadIdx.x;
  int4 v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = pair_load4(col, r0 + 1024 * q, n_out);
  int c = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) c += __popc(pair_bits4(v[q], n_in));
  c = wave_sum(c);
  if ((threadIdx.x & 63) == 0) wsum_s[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[(int64_t)k * nb + blockIdx.x] = wsum_s[0] + wsum_s[1] + wsum_s[2] + wsum_s[3];
}

__global__ __launch_bounds__(256) void pairs_emit_vec_kernel(const int32_t* __restrict__ map, int64_t ks,
                                                             int64_t n_out, int64_t n_in, int64_t nb,
                                                             const int32_t* __restrict__ offsets,
                                                             int32_t* __restrict__ pairs) {
  __shared__ int wsum_s[4][4];  // [q][wave]
  const int k = blockIdx.y;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int32_t* col = map + (int64_t)k * ks;
  const int64_t r0 = (int64_t)blockIdx.x * kPairRows + 4 * threadIdx.x;
  int4 v[4];
  uint32_t m[4];
  int ex[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    v[q] = pair_load4(col, r0 + 1024 * q, n_out);
    m[q] = pair_bits4(v[q], n_in);
    const int c = __popc(m[q]);
    const int inc = wave_inclusive_scan(c);
    ex[q] = inc - c;
    if (lane == 63) wsum_s[q][wid] = inc;
  }
  __syncthreads();
  int base = offsets[(int64_t)k * nb + blockIdx.x];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int pos = base + ex[q];
    for (int w = 0; w < wid; ++w) pos += wsum_s[q][w];
    const int32_t e[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if ((m[q] >> j) & 1u) {
        *reinterpret_cast<int2*>(pairs + 2 * (int64_t)pos) = make_int2(e[j], (int32_t)(r0 + 1024 * q + j));
        ++pos;
      }
    base += wsum_s[q][0] + wsum_s[q][1] + wsum_s[q][2] + wsum_s[q][3];
  }
}

}  // namespace st

extern "C" int st_kmap_pairs_sizes(int64_t n_out, int K, int64_t* num_blocks) {
  if (n_out < 0 || K <= 0 || K > ST_MAX_KVOL || !num_blocks) return ST_ERR_ARG;
  *num_blocks = (n_out + st::kPairRows - 1) / st::kPairRows;
  return ST_OK;
}

namespace st {
// count, scan (+ kstart / cstart), emit; arguments checked by the caller
int launch_pairs(const int32_t* map, int64_t ks, int64_t rs, int64_t n_out, int K, int64_t n_in,
                 int32_t* block_counts, int64_t nb, int chunk, int32_t* kstart, int32_t* cstart, int32_t* pairs,
                 hipStream_t stream) {
  const dim3 grid((unsigned)nb, (unsigned)K);
  const bool vec = rs == 1 && ks % 4 == 0 && (reinterpret_cast<uintptr_t>(map) & 15) == 0;
  if (nb > 0) {
    if (vec)
      pairs_count_vec_kernel<<<grid, 256, 0, stream>>>(map, ks, n_out, n_in, nb, block_counts);
    else
      pairs_count_kernel<<<grid, 256, 0, stream>>>(map, ks, rs, n_out, n_in, nb, block_counts);
  }
  exclusive_scan_kernel<<<1, 1024, 0, stream>>>(block_counts, (int64_t)K * nb, PairsFinal{kstart, cstart, nb, K, chunk});
  if (nb > 0) {
    if (vec)
      pairs_emit_vec_kernel<<<grid, 256, 0, stream>>>(map, ks, n_out, n_in, nb, block_counts, pairs);
    else
      pairs_emit_kernel<<<grid, 256, 0, stream>>>(map, ks, rs, n_out, n_in, nb, block_counts, pairs);
  }
  return hipGetLastError() == hipSuccess ? ST_OK : ST_ERR_HIP;
}
}  // namespace st

extern "C" int st_kmap_pairs(const int32_t* map, int64_t map_k_stride, int64_t map_r_stride, int64_t n_out, int K,
                             int64_t n_in, int32_t* block_counts, int64_t num_blocks, int chunk, int32_t* kstart,
                             int32_t* cstart, int32_t* pairs, int64_t pair_capacity, st_stream_t stream) {
  if (n_out < 0 || n_in < 0 || K <= 0 || K > ST_MAX_KVOL || (chunk <= 0 && chunk != ST_PAIR_CHUNK_AUTO))
    return ST_ERR_ARG;
  if (num_blocks != (n_out + st::kPairRows - 1) / st::kPairRows) return ST_ERR_ARG;
  if ((int64_t)K * n_out >= (1ll << 31) || pair_capacity < (int64_t)K * n_out) return ST_ERR_ARG;
  if (!block_counts || !kstart || !cstart || (n_out > 0 && (!map || !pairs))) return ST_ERR_ARG;
  return st::launch_pairs(map, map_k_stride, map_r_stride, n_out, K, n_in, block_counts, num_blocks, chunk, kstart,
                          cstart, pairs, stream);
}

namespace st {
// keys[c] = 9-bit bucket (row * 512 / n_out) of the output row of chunk c's
// first pair (chunks of `chunk` pairs per offset, in (offset, out) pair
// order); 511 past the last chunk, which a stable sort keeps behind the
// real chunks of that bucket.
__global__ __launch_bounds__(256) void chunk_keys_kernel(const int32_t* __restrict__ pairs,
                                                         const int32_t* __restrict__ kstart,
                                                         const int32_t* __restrict__ cstart, int K, int chunk,
                                                         int64_t max_chunks, int64_t n_out,
                                                         uint32_t* __restrict__ keys) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= max_chunks) return;
  const int total = cstart[K];
  if (chunk <= 0) chunk = cstart[K + 1];
  uint32_t key = 511u;
  if (c < total) {
    int lo = 0, hi = K - 1;  // offset of chunk c: largest k with cstart[k] <= c
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cstart[mid] <= c) lo = mid;
      else hi = mid - 1;
    }
    const int64_t p0 = kstart[lo] + (c - cstart[lo]) * (int64_t)chunk;
    const int64_t row = pairs[2 * p0 + 1];
    key = (uint32_t)(row * 512 / (n_out > 0 ? n_out : 1));
    if (key > 511u) key = 511u;
  }
  keys[c] = key;
}
}  // namespace st

extern "C" int st_kmap_pairs_chunk_keys(const int32_t* pairs, const int32_t* kstart, const int32_t* cstart, int K,
                                        int chunk, int64_t max_chunks, int64_t n_out, uint32_t* keys,
                                        st_stream_t stream) {
  if (K <= 0 || K > ST_MAX_KVOL || (chunk <= 0 && chunk != ST_PAIR_CHUNK_AUTO) || max_chunks < 0 ||
      max_chunks >= (1ll << 31))
    return ST_ERR_ARG;
  if (max_chunks == 0) return ST_OK;
  if (!pairs || !kstart || !cstart || !keys) return ST_ERR_ARG;
  return st::launch_chunk_keys(pairs, kstart, cstart, K, chunk, max_chunks, n_out, keys, stream);
}

int st::launch_chunk_keys(const int32_t* pairs, const int32_t* kstart, const int32_t* cstart, int K, int chunk,
                          int64_t max_chunks, int64_t n_out, uint32_t* keys, hipStream_t stream) {
  chunk_keys_kernel<<<st_blocks(max_chunks, 256), 256, 0, stream>>>(pairs, kstart, cstart, K, chunk, max_chunks,
                                                                    n_out, keys);
  return hipGetLastError() == hipSuccess ? ST_OK : ST_ERR_HIP;
}

namespace st {
// Chunk order without a sort: the chunk keys of chunk_keys_kernel (9-bit
// bucket of the first output row) are nondecreasing within each offset's run
// of chunks, so in the stable order by key chunk c (offset k, index j in its
// run, bucket b) lands at
//   #(chunks of any run with bucket < b) + #(runs k' < k with bucket b)
//   + (j - #(run k's chunks with bucket < b)),
// the first two from a per-(run, bucket) count table scanned over runs and
// buckets, the last from a binary search in run k.  One workgroup holds the
// keys and the table in LDS (K <= kChunkOrderMaxK, up to kChunkOrderMax
// chunks); chunks past cstart[K] keep their index.  Same order as the stable
// radix sort of the keys.
constexpr int kChunkBuckets = 512;

__device__ __forceinline__ int chunk_run(const int32_t* cstart_s, int K, int c) {
  int lo = 0, hi = K - 1;  // largest k with cstart[k] <= c
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cstart_s[mid] <= c) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(1024) void chunk_order_kernel(const int32_t* __restrict__ pairs,
                                                           const int32_t* __restrict__ kstart,
                                                           const int32_t* __restrict__ cstart, int K, int chunk,
                                                           int64_t max_chunks, int64_t n_out,
                                                           int32_t* __restrict__ order) {
  __shared__ uint16_t keys_s[kChunkOrderMax];
  __shared__ int16_t cnt_s[kChunkOrderMaxK][kChunkBuckets];  // counts, then prefix over runs
  __shared__ int32_t below_s[kChunkBuckets];                  // chunks of all runs in lower buckets
  __shared__ int32_t cst_s[kChunkOrderMaxK + 2], kst_s[kChunkOrderMaxK + 1];
  __shared__ int scan_s[17];
  const int tid = threadIdx.x;
  for (int t = tid; t <= K + (chunk <= 0); t += 1024) {
    cst_s[t] = cstart[t];
    if (t <= K) kst_s[t] = kstart[t];
  }
  for (int t = tid; t < K * kChunkBuckets; t += 1024) (&cnt_s[0][0])[t] = 0;
  __syncthreads();
  const int total = cst_s[K];
  if (chunk <= 0) chunk = cst_s[K + 1];
  for (int c = tid; c < total; c += 1024) {
    const int k = chunk_run(cst_s, K, c);
    const int64_t p0 = kst_s[k] + (int64_t)(c - cst_s[k]) * chunk;
    const int64_t row = pairs[2 * p0 + 1];
    int64_t key = row * kChunkBuckets / (n_out > 0 ? n_out : 1);
    key = key > kChunkBuckets - 1 ? kChunkBuckets - 1 : key;
    keys_s[c] = (uint16_t)key;
    atomicAdd(reinterpret_cast<int*>(&cnt_s[k][key & ~1]), (key & 1) ? 0x10000 : 1);  // 16-bit halves
  }
  __syncthreads();
  // prefix over runs per bucket, then over buckets of the bucket totals
  int tot = 0;
  if (tid < kChunkBuckets)
    for (int k = 0; k < K; ++k) {
      const int v = cnt_s[k][tid];
      cnt_s[k][tid] = (int16_t)tot;
      tot += v;
    }
  int all;
  const int ex = block_exclusive_scan(tid < kChunkBuckets ? tot : 0, scan_s, &all);
  if (tid < kChunkBuckets) below_s[tid] = ex;
  __syncthreads();
  for (int64_t c = tid; c < max_chunks; c += 1024) {
    if (c >= total) {
      order[c] = (int32_t)c;
      continue;
    }
    const int k = chunk_run(cst_s, K, (int)c);
    const int key = keys_s[c];
    int lo = cst_s[k], hi = (int)c;  // first chunk of run k with bucket >= key
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if ((int)keys_s[mid] < key) lo = mid + 1;
      else hi = mid;
    }
    order[below_s[key] + cnt_s[k][key] + ((int)c - lo)] = (int32_t)c;
  }
}

int launch_chunk_order(const int32_t* pairs, const int32_t* kstart, const int32_t* cstart, int K, int chunk,
                       int64_t max_chunks, int64_t n_out, int32_t* order, hipStream_t stream) {
  if (max_chunks > kChunkOrderMax || K > kChunkOrderMaxK) return ST_ERR_UNSUPPORTED;
  if (max_chunks == 0) return ST_OK;
  chunk_order_kernel<<<1, 1024, 0, stream>>>(pairs, kstart, cstart, K, chunk, max_chunks, n_out, order);
  return hipGetLastError() == hipSuccess ? ST_OK : ST_ERR_HIP;
}
}  // namespace st

extern "C" int st_kmap_pairs_chunk_order(const int32_t* pairs, const int32_t* kstart, const int32_t* cstart, int K,
                                         int chunk, int64_t max_chunks, int64_t n_out, int32_t* order,
                                         st_stream_t stream) {
  if (K <= 0 || K > ST_MAX_KVOL || (chunk <= 0 && chunk != ST_PAIR_CHUNK_AUTO) || max_chunks < 0) return ST_ERR_ARG;
  if (max_chunks > st::kChunkOrderMax) return ST_ERR_UNSUPPORTED;
  if (max_chunks > 0 && (!pairs || !kstart || !cstart || !order)) return ST_ERR_ARG;
  return st::launch_chunk_order(pairs, kstart, cstart, K, chunk, max_chunks, n_out, order, stream);
}
