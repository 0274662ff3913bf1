/*
 * sparsetriton_amd -- C ABI of the MI355X (gfx950) sparse-convolution hot path.
 *
 * One shared library, libsparsetriton_amd.so, built with hipcc for gfx950.
 * Every entry point takes plain device pointers, 64-bit sizes, small enums
 * and the hipStream_t to enqueue on; nothing here allocates device memory,
 * synchronises the stream, or depends on torch types.  Callers own every
 * buffer (inputs, outputs, workspaces).  Return value: ST_OK (0) on success,
 * a negative ST_ERR_* code otherwise; device-side failures (full hash table,
 * unpackable coordinate, duplicate coordinate) are counted into a caller-owned
 * int32 status[ST_STATUS_WORDS] buffer instead of being dropped.
 *
 * Reference interfaces replaced (paths relative to the reference tree):
 *   HashTable.insert / build_hash_table_kernel ... sparsetriton/utils/hash.py:193-258, 516-544
 *   HashTable.query / query_hash_table_kernel ..... sparsetriton/utils/hash.py:261-366, 546-580
 *   compute_neighbor_indices ...................... sparsetriton/nn/functional/conv/conv.py:12-75
 *   _build_out_coords_normal / _transposed ......... sparsetriton/nn/functional/conv/kmap.py:213-444
 *   ConvPrecomputedNeighborGEMM fwd/dgrad/wgrad .... .../conv/funcs/implicit_precomputed_gemm.py:64-324
 *   ConvHashOnTheFlyImplicitGEMM fwd/dgrad/wgrad ... .../conv/funcs/implicit_hashfly_gemm.py:45-452
 */
#ifndef SPARSETRITON_AMD_H
#define SPARSETRITON_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is an opaque pointer; declared here so the header needs no HIP headers. */
typedef struct ihipStream_t* st_stream_t;

/* ------------------------------------------------------------------ enums */

enum st_status_code {
  ST_OK = 0,
  ST_ERR_ARG = -1,         /* bad size, null pointer, unsupported shape      */
  ST_ERR_HIP = -2,         /* a HIP launch or runtime call failed            */
  ST_ERR_UNSUPPORTED = -3, /* dtype / kernel volume outside what is built    */
};

enum st_coord_dtype { ST_COORD_I16 = 0, ST_COORD_I32 = 1, ST_COORD_I64 = 2 };

/* Feature dtypes.  ST_F32_BF16X3: fp32 tensors whose products are computed
 * as three bf16 MFMAs over hi/lo splits of each operand (hi*hi + hi*lo +
 * lo*hi, relative error per product <= ~2^-15, fp32 accumulation) -- the
 * matrix-core path for fp32, as TF32 is for the reference's tl.dot.  Entry
 * points without a split kernel compute ST_F32_BF16X3 in plain fp32. */
enum st_dtype { ST_F32 = 0, ST_F16 = 1, ST_BF16 = 2, ST_F32_BF16X3 = 3 };

/* Device status words, accumulated by atomics (caller zeroes them). */
enum st_status_word {
  ST_STATUS_OVERFLOW = 0,  /* inserts that found the table full               */
  ST_STATUS_BAD_COORD = 1, /* coordinates that do not pack into a 64-bit key  */
  ST_STATUS_DUPLICATE = 2, /* rows whose coordinate an earlier row already has
                              (counted by each pass that sees it: nonzero means
                              the coordinate set has repeats)                 */
  ST_STATUS_OUT_OF_BOX = 3, /* kernel-map query rows outside [0, shape)       */
  ST_STATUS_WORDS = 4,
};

/* Weight re-layouts produced by st_weight_prep from W (K, C_in, C_out). */
enum st_weight_mode {
  ST_W_TRANSPOSE = 0, /* out[k][co][ci] = W[k][ci][co]        (forward B operand)   */
  ST_W_REVERSE = 1,   /* out[k][ci][co] = W[K-1-k][ci][co]    (submanifold dgrad)   */
  ST_W_COPY = 2,      /* out = W                              (general dgrad)       */
};

/* Kernel volume limit of the kernel-map row masks (mask words = ceil(K/32)). */
#define ST_MAX_KVOL 512

/* ------------------------------------------------------------- utilities */

/* Library version string, e.g. "sparsetriton_amd 0.1 gfx950" (a utility of
 * this library: no counterpart in the reference). */
const char* st_version(void);

/* Fill n 32-bit / 64-bit words with `value` (table clears, -1 map fills; the
 * reference's torch.full calls around its kernels, utils/hash.py:428-429, 568). */
int st_fill_u32(uint32_t* dst, int64_t n, uint32_t value, st_stream_t stream);
int st_fill_u64(uint64_t* dst, int64_t n, uint64_t value, st_stream_t stream);

/* -------------------------------------------------------- coordinate hash */

/*
 * Probe style of st_hash_insert, st_hash_query and st_kmap_query: 0 = one
 * thread per key, linear probing with several keys' first loads in flight
 * (default); 1 = a 16-lane group per key, lane j loading slot s + j of a
 * 16-slot window and one ballot finding the first matching or empty slot.
 * Same table, same results; kept for timing comparisons.  mode -1 only
 * reads.  Returns the mode before the call.  No counterpart in the
 * reference, whose probes are per thread (utils/hash.py:174-299).
 */
int st_hash_probe_mode(int mode);

/*
 * Replaces HashTable.insert -> build_hash_table_kernel (utils/hash.py:193-258, 516-544).
 * Inserts the n rows of coords (n, 4) = (b, x, y, z), x/y/z multiplied by
 * `scale` (1 normally; the stride for the transposed-conv table that
 * sparse_conv3d builds from coords * s, conv.py:138-142), into an
 * open-addressing table of `capacity` slots: keys (u64, packed coordinate,
 * all-ones = empty) and vals (u32 row index, all-ones = none).  The caller
 * clears both arrays to all-ones first (st_fill_u64 / st_fill_u32).  Linear
 * probing from a 64-bit-mixed home slot; the key is claimed by a 64-bit CAS
 * and the claiming row stores its index; a repeated coordinate takes an atomic
 * min, and a second pass queued by the same call (a no-op unless the status
 * counts repeats) applies the min again after every store, so duplicate
 * coordinates resolve to the lowest row index on every run.
 */
int st_hash_insert(const void* coords, int coord_dtype, int64_t n, int64_t scale, uint64_t* keys, uint32_t* vals,
                   int64_t capacity, int32_t* status, st_stream_t stream);

/*
 * Replaces HashTable.insert -> build_hash_table_kernel (utils/hash.py:193-258,
 * 516-544), partitioned: the same insert as st_hash_insert (same keys, values,
 * lowest row of a repeated coordinate, status counts) built segment by
 * segment in LDS.  Rows are grouped by the segment of their home slot (per
 * workgroup of 4096 rows, in LDS), then one workgroup per segment of 2048
 * slots gathers its rows, inserts them by LDS CAS and stores the segment
 * with coalesced writes; rows whose probe runs past their segment are
 * inserted by global CAS, from the next segment on, after every segment is
 * stored.  Three kernels,
 * no global atomics but the spills'.  fresh = 1 builds into a table that is
 * treated as empty (no clear needed: every slot is written); fresh = 0
 * inserts into the table's current contents, as st_hash_insert does.
 * workspace (st_hash_build_workspace bytes) must be zeroed before its first
 * use; every call leaves it reusable as is.  Calls that share a workspace
 * must not overlap.  ST_ERR_UNSUPPORTED above 16.7M slots or 8.4M rows and
 * while the 16-lane probe mode is on (st_hash_probe_mode): use
 * st_hash_insert there.
 */
int st_hash_build_workspace(int64_t n, int64_t capacity, int64_t* bytes);
int st_hash_build(const void* coords, int coord_dtype, int64_t n, int64_t scale, uint64_t* keys, uint32_t* vals,
                  int64_t capacity, int fresh, void* workspace, int64_t workspace_bytes, int32_t* status,
                  st_stream_t stream);

/*
 * Replaces HashTable.query -> query_hash_table_kernel (utils/hash.py:302-366, 546-580).
 * out[i] = row index stored for coords[i], or -1 when absent.
 */
int st_hash_query(const void* coords, int coord_dtype, int64_t m, const uint64_t* keys, const uint32_t* vals,
                  int64_t capacity, int32_t* out, st_stream_t stream);

/* ------------------------------------------------------------ kernel maps */

/*
 * Replaces compute_neighbor_indices (nn/functional/conv/conv.py:12-75).
 * For every output row o and offset k:
 *   q = out_coords[o].xyz * stride - offsets[k]            (offsets: int32 (K, 3))
 *   nbr[k * nbr_k_stride + o * nbr_r_stride] = row of q in the table if
 *       0 <= q < shape (per axis) and present, else -1.
 * row_masks (n_out, ceil(K/32)) u32, optional: bit k set iff nbr[o, k] >= 0.
 * The package stores maps offset-major, (K, n_out) (nbr_k_stride = n_out,
 * nbr_r_stride = 1): every kernel that walks rows then reads and writes each
 * offset's column with coalesced accesses.
 * status (optional, ST_STATUS_WORDS int32): rows whose out_coords.xyz * stride
 * lie outside [0, shape) add to ST_STATUS_OUT_OF_BOX.  Such a row keeps its
 * in-bounds neighbours (the reference checks the neighbour only), but no row
 * finds it as a neighbour, so a submanifold map is its own transpose (offsets
 * reversed) only when this count and ST_STATUS_DUPLICATE are both zero.
 */
int st_kmap_query(const void* out_coords, int coord_dtype, int64_t n_out, const int32_t* offsets, int K,
                  int64_t stride, int64_t shape_x, int64_t shape_y, int64_t shape_z, const uint64_t* keys,
                  const uint32_t* vals, int64_t capacity, int32_t* nbr, int64_t nbr_k_stride, int64_t nbr_r_stride,
                  uint32_t* row_masks, int32_t* status, st_stream_t stream);

/*
 * Replaces compute_neighbor_indices (conv.py:12-75) with its hash table
 * (HashTable.insert + query, utils/hash.py:193-366) for the submanifold case
 * -- out_coords == in_coords, stride 1 -- with no hash table: seven short
 * kernels build a brick index of the coords over the box [0, batches) x
 * [0, shape) in `workspace` (st_kmap_subm_workspace bytes; 4x4x4-voxel
 * bricks, a bit per occupied brick and a bit per voxel of each occupied brick,
 * with rank prefixes and a rank -> lowest-row map; a few MB, so lookups stay
 * in L2) and then write, for every row o and offset k,
 *   nbr[k * n + o] = row of coords[o].xyz - offsets[k] if it lies in
 *                    [0, shape) and is present (lowest row of repeats), else -1,
 * and row_masks (n, ceil(K/32)) u32 (optional).  The same map as
 * st_kmap_query over a table of coords, bit for bit.  status (optional,
 * ST_STATUS_WORDS int32, cleared by the call) counts BAD_COORD (rows that do
 * not pack into a key), DUPLICATE (rows repeating a coordinate) and
 * OUT_OF_BOX (rows whose xyz lie outside [0, shape)).
 * st_kmap_subm_workspace returns ST_ERR_ARG when the box is far larger than
 * the set (level 1 would exceed 64 bytes a row): query a hash table instead.
 * st_kmap_subm = st_subm_index (the index alone, with the status counts) +
 * st_kmap_subm_query (the map from a built index; the index stays valid
 * while `workspace` and the coordinates are unchanged, for any offsets).
 * st_kmap_subm_query with nbr = NULL writes row_masks only (then required):
 * the input of st_kmap_sort_rows for a tile order of st_subm_fly_gemm.
 */
int st_kmap_subm_workspace(int64_t n, int64_t batches, int64_t sx, int64_t sy, int64_t sz, int64_t* bytes);
int st_kmap_subm(const void* coords, int coord_dtype, int64_t n, const int32_t* offsets, int K, int64_t batches,
                 int64_t sx, int64_t sy, int64_t sz, void* workspace, int64_t workspace_bytes, int32_t* nbr,
                 uint32_t* row_masks, int32_t* status, st_stream_t stream);
int st_subm_index(const void* coords, int coord_dtype, int64_t n, int64_t batches, int64_t sx, int64_t sy,
                  int64_t sz, void* workspace, int64_t workspace_bytes, int32_t* status, st_stream_t stream);
int st_kmap_subm_query(const void* coords, int coord_dtype, int64_t n, const int32_t* offsets, int K,
                       int64_t batches, int64_t sx, int64_t sy, int64_t sz, const void* workspace,
                       int64_t workspace_bytes, int32_t* nbr, uint32_t* row_masks, st_stream_t stream);

/* Geometry of a strided or transposed convolution's output-coordinate build. */
typedef struct st_outgeom {
  int32_t K;            /* kernel volume (offsets rows)                              */
  int32_t transposed;   /* 0: candidates (in + t_k) / stride; 1: in * stride + t_k   */
  int64_t stride;       /* >= 1                                                      */
  int64_t in_shape[3];  /* input spatial shape (bounds of the neighbour lookup)      */
  int64_t out_shape[3]; /* output spatial shape (range filter of the candidates)     */
  int64_t chunk;        /* offsets per chunk of the candidate order (the reference's
                           chunk_size, kmap.py:270-278); <= 0 or >= K: one chunk   */
} st_outgeom;

/*
 * Dedup-table capacity and per-block counter length the output-coordinate
 * build needs for n input rows.  Fills *dedup_capacity (twice the candidates
 * that can pass the filters, at most 2^31 - 64; a smaller table works when
 * it holds the distinct outputs, and an overflow is reported in status) and
 * *num_blocks (input blocks of 256 rows x offset chunks).
 */
int st_outcoords_sizes(int64_t n, const st_outgeom* g, int64_t kernel_size, int64_t dilation,
                       int64_t* dedup_capacity, int64_t* num_blocks);

/*
 * Replaces the candidate expansion, stride / range filter and dedup of
 * _build_out_coords_normal / _transposed (kmap.py:213-444, expand_coords_kernel
 * :11-54, filter_unique_kernel :56-97, mask_spatial_range utils/spatial/tile.py).
 * Pass 1 of 2.  Candidates are enumerated chunk by chunk of g->chunk
 * offsets, input-major and offset-minor inside a chunk (the reference's
 * order, kmap.py:270-278; one chunk by default); every valid candidate is
 * inserted into the dedup table (dkeys/dvals, cleared to all-ones by the
 * caller) keeping the lowest candidate rank per coordinate.
 * block_counts (num_blocks + 1 int32) receives, after an exclusive scan, the
 * output-row offset of each block; block_counts[num_blocks] = N_out.
 */
int st_outcoords_plan(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                      const st_outgeom* g, uint64_t* dkeys, uint32_t* dvals, int64_t dcap, int32_t* block_counts,
                      int64_t num_blocks, int32_t* status, st_stream_t stream);

/*
 * Pass 2 of 2, after the caller read N_out = block_counts[num_blocks].
 * Writes out_coords (N_out, 4) in the input's coordinate dtype, ordered by
 * first occurrence in the candidate order; slot_out (dcap u32) maps dedup
 * slots to output rows (so dkeys + slot_out form the output-coordinate
 * table); and the kernel map in both directions, offset-major:
 *   nbr    (K, N_out): input row feeding output o through offset k, or -1
 *   invnbr (K, n)    : output row fed by input i through offset k, or -1
 * plus row masks out_masks (N_out, W) and in_masks (n, W), W = ceil(K/32).
 * nbr/invnbr must be pre-filled with -1 and the masks with 0 by the caller.
 * With nbr == NULL only out_coords and slot_out are written (hash-fly mode).
 * in_keys/in_vals/in_cap (optional) is the input-coordinate table the
 * reference's neighbour query would use (coords * stride for transposed):
 * when given, only the row that table resolves a coordinate to enters the
 * map, so duplicate input coordinates behave as a lookup would.
 */
int st_outcoords_emit(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                      const st_outgeom* g, const uint64_t* dkeys, const uint32_t* dvals, uint32_t* slot_out,
                      int64_t dcap, const int32_t* block_counts, int64_t num_blocks, const uint64_t* in_keys,
                      const uint32_t* in_vals, int64_t in_cap, void* out_coords, int64_t n_out, int32_t* nbr,
                      int32_t* invnbr, uint32_t* out_masks, uint32_t* in_masks, st_stream_t stream);

/*
 * Brick-index form of st_outcoords_sizes / _plan / _emit: the same output
 * coordinates in the same order (_build_out_coords_normal / _transposed,
 * kmap.py:213-444), deduplicated without a hash table.  The candidates'
 * output coordinates are indexed in 4x4x4 bricks of the output box
 * [0, batches) x [0, g->out_shape) and each distinct one keeps its lowest
 * candidate rank; a candidate whose rank is that minimum is the first
 * occurrence.  kernel_size / dilation bound the candidates per input row (as
 * in st_outcoords_sizes).  st_outcoords_brick_sizes fills the workspace bytes
 * and the block-counter length (blocks of 256 candidate ranks), or returns
 * ST_ERR_UNSUPPORTED when the box cannot be indexed (far larger than the
 * candidates, or an output shape beyond 32768): the caller then uses the hash
 * build.
 */
int st_outcoords_brick_sizes(int64_t n, const st_outgeom* g, int64_t batches, int64_t kernel_size,
                             int64_t dilation, int64_t* workspace_bytes, int64_t* num_blocks);

/*
 * Pass 1 of 2: index, lowest ranks, per-block first-occurrence counts;
 * block_counts (num_blocks + 1 int32) receives their exclusive scan and
 * block_counts[num_blocks] = N_out.  status (ST_STATUS_WORDS int32, cleared by
 * the call): ST_STATUS_OUT_OF_BOX counts candidates whose batch index lies
 * outside [0, batches) -- the index cannot hold them, so a nonzero count means
 * the caller must use the hash build instead.  ST_STATUS_OVERFLOW is nonzero
 * when the offsets reach more output bricks or voxels than kernel_size and
 * dilation bound (offsets that are not that kernel's): the index is then
 * sized too small, no array past its bound is written, N_out reads 0, emit
 * writes nothing and st_outcoords_brick_inverse maps every candidate to -1;
 * the caller must use the hash build instead.
 */
int st_outcoords_brick_plan(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                            const st_outgeom* g, int64_t batches, int64_t kernel_size, int64_t dilation,
                            void* workspace, int64_t workspace_bytes, int32_t* block_counts, int64_t num_blocks,
                            int32_t* status, st_stream_t stream);

/*
 * Pass 2 of 2: out_coords (N_out, 4) in the input's coordinate dtype; also
 * records each output's row in the workspace for st_outcoords_brick_inverse.
 */
int st_outcoords_brick_emit(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                            const st_outgeom* g, int64_t batches, int64_t kernel_size, int64_t dilation,
                            void* workspace, int64_t workspace_bytes, const int32_t* block_counts,
                            int64_t num_blocks, void* out_coords, int64_t n_out, st_stream_t stream);

/*
 * Kernel map of a strided / transposed convolution by query, the
 * reference's compute_neighbor_indices over the output coordinates
 * (conv.py:12-75, 180-188): for output row o and offset k the input
 * coordinate (b, o * s - t_k), or transposed (b, (o - t_k) / s) when s
 * divides every component, looked up in the brick index of the n_in input
 * rows (st_subm_index over [0, batches) x g->in_shape; a repeated coordinate
 * resolves to its lowest row).  Writes nbr (K, n_out) and out_masks
 * (n_out, W) whole: the map st_outcoords_emit writes with the
 * input-coordinate table.
 */
int st_kmap_strided_query(const void* out_coords, int coord_dtype, int64_t n_out, const int32_t* offsets,
                          const st_outgeom* g, int64_t batches, const void* in_index, int64_t in_index_bytes,
                          int64_t n_in, int32_t* nbr, uint32_t* out_masks, st_stream_t stream);

/*
 * The transposed map of the same convolution after st_outcoords_brick_emit
 * (same arguments and workspace), input-major: invnbr (K, n) = output row of
 * candidate (input i, offset k), -1 when the filters drop it or row i is not
 * the row the query resolves its coordinate to (in_index as for
 * st_kmap_strided_query), and in_masks (n, W); both written whole -- the
 * invnbr / in_masks st_outcoords_emit writes.
 */
int st_outcoords_brick_inverse(const void* in_coords, int coord_dtype, int64_t n, const int32_t* offsets,
                               const st_outgeom* g, int64_t batches, int64_t kernel_size, int64_t dilation,
                               const void* workspace, int64_t workspace_bytes, const void* in_index,
                               int64_t in_index_bytes, int32_t* invnbr, uint32_t* in_masks, st_stream_t stream);

/*
 * Transposed kernel map of an arbitrary map nbr (k, o) -> i (strides as in
 * st_kmap_query): invnbr[k * n_in + i] = o (offset-major), in_masks (n_in, W) row masks of
 * invnbr, and, if out_masks is non-null, out_masks (n_out, W) row masks of
 * nbr.  invnbr must be pre-filled with -1 and in_masks with 0.  Used when a
 * caller hands ConvPrecomputedNeighborGEMM a plain (N_out, K) map
 * (implicit_precomputed_gemm.py:237-242) and for a submanifold map that is not
 * its own transpose, whose transposed map feeds the atomic-free input gradient.
 * conflicts (optional, one int32, caller-zeroed): entries (k, o) -> i whose
 * (k, i) another output already holds -- a map invnbr cannot represent (one
 * input feeding two outputs through one offset: repeated output coordinates).
 */
int st_kmap_invert(const int32_t* nbr, int64_t nbr_k_stride, int64_t nbr_r_stride, int64_t n_out, int K,
                   int64_t n_in, int32_t* invnbr, uint32_t* in_masks, uint32_t* out_masks, int32_t* conflicts,
                   st_stream_t stream);

/*
 * Destination-row order for the gather-GEMM (no reference counterpart; the
 * reference tiles rows in storage order).  Rows are stably radix-sorted by
 * their offset bitmask (masks (n, mask_words), folded to 32 bits when
 * K > 32) so that 128-row gather-GEMM tiles share their offsets.  For
 * K = 27 (3x3x3, x-major offsets) the key's bits are the mask's bits ordered
 * by how many axes the offset leaves the centre on (centre lowest, corners
 * highest), then by index.  perm (n) gets the sorted row ids.  keys_tmp holds 2n u32, rows_tmp n int32, workspace
 * st_kmap_sort_workspace(n) bytes.
 */
int st_kmap_sort_workspace(int64_t n, size_t* bytes);
int st_kmap_sort_rows(const uint32_t* masks, int mask_words, int K, int64_t n, uint32_t* keys_tmp, int32_t* rows_tmp,
                      int32_t* perm, void* workspace, size_t workspace_bytes, st_stream_t stream);

/* Destination rows per gather-GEMM tile (the workgroup tile of st_gather_gemm). */
#define ST_TILE_ROWS 128

/*
 * Tile plan of a gather-GEMM (no reference counterpart; built once per kernel
 * map and reused by every layer and by forward and input gradient): for each
 * tile t of ST_TILE_ROWS destination rows, taken in perm order,
 *   tile_nk[t]                      number of offsets any row of the tile has,
 *   tile_klist[t * K + j]           those offsets, ascending (int16),
 *   tile_map[(t * K + j) * 128 + r] source row of tile row r through offset
 *                                   tile_klist[t * K + j] (-1 = none, also for
 *                                   map entries >= n_src).
 * ntiles = ceil(n_dst / 128); tile_klist holds ntiles * K entries and
 * tile_map ntiles * K * 128 (only the first tile_nk[t] offsets of a tile are
 * written).  map / row_masks as in st_gather_gemm (masks optional: all K).
 */
int st_tile_plan(const int32_t* map, int64_t map_k_stride, int64_t map_r_stride, const uint32_t* row_masks,
                 int mask_words, int K, const int32_t* perm, int64_t n_dst, int64_t n_src, int32_t* tile_nk,
                 int16_t* tile_klist, int32_t* tile_map, st_stream_t stream);

/*
 * Pair list of a kernel map for the weight gradient (replaces the per-tile
 * map walk of precomputed_bwd_weight_kernel, implicit_precomputed_gemm.py:180-230):
 * pairs (2P int32) = (in, out) for every map(k, out) in [0, n_in), sorted by
 * (k, out); kstart (K + 1) = first pair of each offset (kstart[K] = P);
 * cstart (K + 1) = first chunk of each offset when each offset's pairs are
 * cut into chunks of `chunk` pairs.  block_counts holds K * num_blocks + 1
 * int32 (num_blocks from st_kmap_pairs_sizes); pair_capacity >= K * n_out.
 * chunk = ST_PAIR_CHUNK_AUTO: the list picks the size itself, on the GPU, from
 * its pair count P -- the least power of two >= 1024 with P <= 2048 * size, so
 * at most min(2048 + K, K * n_out / 1024 + K) chunks (ST_PAIR_CHUNKS_AUTO_MAX)
 * -- and stores it in cstart[K + 1] (cstart then holds K + 2 entries).  Pass
 * ST_PAIR_CHUNK_AUTO on to the calls below that take the list; they read the
 * size from there.
 */
#define ST_PAIR_CHUNK_AUTO (-1)
#define ST_PAIR_CHUNKS_AUTO_MAX(n_out, K) \
  ((int64_t)(K) * (n_out) / 1024 + (K) < 2048 + (K) ? (int64_t)(K) * (n_out) / 1024 + (K) : 2048 + (int64_t)(K))
int st_kmap_pairs_sizes(int64_t n_out, int K, int64_t* num_blocks);
int st_kmap_pairs(const int32_t* map, int64_t map_k_stride, int64_t map_r_stride, int64_t n_out, int K, int64_t n_in,
                  int32_t* block_counts, int64_t num_blocks, int chunk, int32_t* kstart, int32_t* cstart,
                  int32_t* pairs, int64_t pair_capacity, st_stream_t stream);

/*
 * keys[c] (max_chunks u32) = row * 512 / n_out for the output row of the first
 * pair of chunk c of a pair list from st_kmap_pairs (a 9-bit bucket), 511 for
 * c >= the chunk count.  Stably sorting chunk ids by these keys
 * (st_kmap_sort_rows with K = 9, one key word per row: one radix pass) gives
 * the chunk order st_wgrad_pairs walks: chunks of every offset that touch the
 * same output rows -- and hence nearby input rows -- run together.  No
 * counterpart in the reference, whose weight-gradient grid walks
 * (N_out / BN, K, channel tiles) directly (implicit_precomputed_gemm.py:180-230).
 */
int st_kmap_pairs_chunk_keys(const int32_t* pairs, const int32_t* kstart, const int32_t* cstart, int K, int chunk,
                             int64_t max_chunks, int64_t n_out, uint32_t* keys, st_stream_t stream);

/*
 * The same chunk order in one launch: the keys above are nondecreasing within
 * each offset's run of chunks, so a chunk's place in their stable order follows
 * from a per-(offset, bucket) count table and one binary search in its own run
 * (keys and table in one workgroup's LDS).
 * order: max_chunks int32.  ST_ERR_UNSUPPORTED above 16384 chunks or 28
 * offsets (use the keys and st_kmap_sort_rows there).
 */
int st_kmap_pairs_chunk_order(const int32_t* pairs, const int32_t* kstart, const int32_t* cstart, int K, int chunk,
                              int64_t max_chunks, int64_t n_out, int32_t* order, st_stream_t stream);

/*
 * Everything the gather-GEMMs and the weight gradient need from one map, in
 * one call: the mask-sorted row order and the tile plan (st_kmap_sort_rows +
 * st_tile_plan) on `stream` and, with chunk > 0 or ST_PAIR_CHUNK_AUTO, the pair list and its chunk
 * order (st_kmap_pairs + st_kmap_pairs_chunk_order) on a stream of the
 * library's that forks from `stream` at the call and joins it again before
 * the tile plan ends -- so work queued on `stream` after the call sees every
 * buffer complete, and nothing else has to be synchronised.  That stream and
 * its two events are created on the first call with a pair list on a device
 * (the one resource this library creates; none is allocated in device
 * memory).  Calls from several host threads are serialised per device.
 *
 * st_kmap_plans_layout fills layout[ST_PLAN_FIELDS]: byte offsets into the
 * caller's `plan` buffer of the outputs below (each on a 256-byte boundary),
 * the two buffer sizes, the tile count and max_chunks.  `scratch` is only
 * used during the call's work on the GPU (stream order).
 * Row order and tiles cover the n_dst destination rows; the pairs are
 * (map[k, o], o) over the same map, o < n_dst, map entries >= n_src skipped.
 * bucket_bits (0..8; used when K + bucket_bits <= 32): rows are first
 * grouped into 2^bucket_bits slabs of the caller's row order (slab =
 * row * 2^bits / n_dst) and sorted by mask within each slab, so the tiles
 * that run together gather from one slab of input rows (more L2 reuse when
 * the rows are in spatial order, at the cost of tiles mixing more masks).
 * No counterpart in the reference, whose GEMMs read the (N_out, K) map
 * directly (implicit_precomputed_gemm.py:64-126, 180-230).
 */
enum {
  ST_PLAN_PERM = 0,       /* int32 [n_dst]                                   */
  ST_PLAN_TILE_NK,        /* int32 [tiles]                                   */
  ST_PLAN_TILE_KLIST,     /* int16 [tiles * K]                               */
  ST_PLAN_TILE_MAP,       /* int32 [tiles * K * 128]                         */
  ST_PLAN_PAIRS,          /* int32 [2 * K * n_dst] (in, out); chunk != 0     */
  ST_PLAN_KSTART,         /* int32 [K + 1]                                   */
  ST_PLAN_CSTART,         /* int32 [K + 1] (K + 2 with ST_PAIR_CHUNK_AUTO)   */
  ST_PLAN_CORDER,         /* int32 [max_chunks]                              */
  ST_PLAN_BYTES,          /* size of `plan`                                  */
  ST_PLAN_SCRATCH_BYTES,  /* size of `scratch`                               */
  ST_PLAN_TILES,          /* ceil(n_dst / 128)                               */
  ST_PLAN_MAX_CHUNKS,     /* K * n_dst / chunk + K (0 without a pair list;   *
                           * ST_PAIR_CHUNKS_AUTO_MAX with ST_PAIR_CHUNK_AUTO) */
  ST_PLAN_FIELDS
};
int st_kmap_plans_layout(int64_t n_dst, int K, int chunk, int64_t* layout);
int st_kmap_plans(const int32_t* map, int64_t map_k_stride, int64_t map_r_stride, const uint32_t* row_masks, int K,
                  int64_t n_dst, int64_t n_src, int chunk, int bucket_bits, void* plan, void* scratch,
                  st_stream_t stream);

/* ------------------------------------------------------------- gather-GEMM */

/*
 * Re-lays W (K, C_in, C_out) for the gather-GEMM's B operand (see
 * st_weight_mode).  Replaces nothing in the reference, which reads W in
 * place with 2-D strides inside each Triton kernel.
 */
int st_weight_prep(const void* w, void* out, int K, int C_in, int C_out, int mode, int dtype, st_stream_t stream);

/*
 * out[c] = sum over rows of Y[:, c] (Y (n, C) of `dtype`, fp32 sums, out of
 * `out_dtype`): the bias gradient of a convolution, which the reference gets
 * from autograd through its `out_feats += bias` (conv.py:227-228).  Two
 * passes, each column's rows summed in a fixed order (deterministic).
 * partials holds 1024 * C floats.
 */
int st_column_sum(const void* Y, int64_t n, int C, int dtype, float* partials, void* out, int out_dtype,
                  st_stream_t stream);

/*
 * No counterpart in the reference.  st_column_sum for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same kernels and result, bit for bit,
 * with the 1024 * C fp32 partials in a library-owned device array instead of a
 * caller workspace.  The array holds C <= ST_COLUMN_SUM_NOALLOC_MAX_C columns
 * (8 MiB per GPU, allocated with the library's code object on each GPU it runs
 * on and held until the process ends); larger C returns ST_ERR_ARG.  Nothing
 * here allocates.  `stream` (or the null stream) must belong to the current
 * device.  All calls on one GPU share its array: calls that overlap on one GPU
 * (concurrent streams or threads) race and must be serialised by the caller.
 */
#define ST_COLUMN_SUM_NOALLOC_MAX_C 2048
int st_column_sum_noalloc(const void* Y, int64_t n, int C, int dtype, void* out, int out_dtype, st_stream_t stream);

/*
 * No counterpart in the reference: a measurement helper.  Runs `blocks`
 * workgroups of 4 waves, each wave `iters` x 8 independent dense bf16 MFMAs
 * (16 x 16 x 32) on register operands, and writes one float per thread to out
 * (blocks * 256 floats); *flops receives the launch's floating-point operation
 * count (set before the launch), so flops / duration is the chip's sustained
 * bf16 MFMA rate.  The bench reports it beside the spec-sheet peak.
 */
int st_mfma_peak(int iters, int blocks, float* out, int64_t* flops, st_stream_t stream);

/*
 * Output-stationary gather-GEMM, the forward of ConvPrecomputedNeighborGEMM
 * (precomputed_fwd_kernel, implicit_precomputed_gemm.py:64-126) and, with the
 * transposed map, its input-gradient (precomputed_bwd_feat_kernel :129-177,
 * here a gather with no atomics):
 *   out[r, :] = sum over k of A[map(k, r), :] @ Bt[k]^T (+ bias)  (map < 0 or >= n_src adds 0)
 * A (n_src, Kd), Bt (K, Nd, Kd), bias (Nd, optional: NULL adds nothing; the
 * reference's `out_feats += bias`, conv.py:227-228, fused into the store),
 * out (n_dst, Nd), all of `dtype`, fp32 accumulation on MFMA.  map(k, r) = map[k * map_k_stride + r * map_r_stride]
 * and row_masks (n_dst, mask_words, optional) are indexed by destination row.
 * perm (optional) is the order destination rows are tiled in -- tile row t is
 * row perm[t] -- normally the mask-sorted order from st_kmap_sort_rows, so
 * rows sharing their offsets share MFMA slabs.  Offsets no row of a 128-row
 * tile has are skipped by the workgroup, offsets no row of a 32-row slab has
 * by that wave.
 */
int st_gather_gemm(const void* A, int64_t n_src, const int32_t* map, int64_t map_k_stride, int64_t map_r_stride,
                   const uint32_t* row_masks, int mask_words, const int32_t* perm, const void* Bt, const void* bias,
                   void* out, int64_t n_dst, int K, int Kd, int Nd, int dtype, st_stream_t stream);

/*
 * st_gather_gemm over a tile plan (st_tile_plan built with the same perm) --
 * the same reference kernels (implicit_precomputed_gemm.py:64-177) --:
 * the workgroup reads its tile's offsets and source rows contiguously
 * instead of gathering map entries and masks row by row.  Same result as
 * st_gather_gemm with that map.  Reductions wider than 128 (16-bit and
 * ST_F32_BF16X3) or 64 (ST_F32) return ST_ERR_UNSUPPORTED.  flags:
 * ST_GATHER_REVERSE_K multiplies offset k's sources by Bt[K - 1 - k] -- the
 * input gradient of a submanifold map that is its own transpose, read over
 * the forward's plan with the weights as given (W (K, C_in, C_out) is then
 * the Bt operand), with no ST_W_REVERSE copy: the same result bit for bit.
 */
enum st_gather_flags { ST_GATHER_REVERSE_K = 1 };
int st_gather_gemm_tiled(const void* A, int64_t n_src, const int32_t* perm, const int32_t* tile_nk,
                         const int16_t* tile_klist, const int32_t* tile_map, const void* Bt, const void* bias,
                         void* out, int64_t n_dst, int K, int Kd, int Nd, int dtype, int flags, st_stream_t stream);

/*
 * st_gather_gemm_tiled with the store epilogue of an evaluation-mode conv +
 * batch norm (+ residual) + ReLU block (nn/modules/blocks.py:21-124,
 * norm.py:105-112 with the running statistics):
 *   out[r, c] = act((sum + bias[c]) * scale[c] + shift[c] + residual[r, c])
 * bias and residual (n_dst x Nd, output rows) of `dtype`; scale, shift fp32
 * (Nd); NULL drops a term (shift needs scale); relu 0 / 1.  With
 * scale = weight / sqrt(running_var + eps) and
 * shift = beta - running_mean * scale this is the block's output in one pass.
 */
int st_gather_gemm_tiled_epilogue(const void* A, int64_t n_src, const int32_t* perm, const int32_t* tile_nk,
                                  const int16_t* tile_klist, const int32_t* tile_map, const void* Bt,
                                  const void* bias, const float* scale, const float* shift, const void* residual,
                                  int relu, void* out, int64_t n_dst, int K, int Kd, int Nd, int dtype,
                                  st_stream_t stream);

/*
 * Weight gradient of ConvPrecomputedNeighborGEMM (precomputed_bwd_weight_kernel,
 * implicit_precomputed_gemm.py:180-230) over the map itself:
 *   dW[k] = sum over o with map(k, o) >= 0 of X[map(k, o)]^T @ dY[o]
 * The map's n_out columns are cut into `splits` windows per offset, each one
 * workgroup's partial (partials: K * splits * C_in * C_out fp32 workspace),
 * reduced in a fixed order, so dW is bit-identical run to run.  16-bit rows
 * with C_in and C_out multiples of 128 run the window kernel: a workgroup
 * takes two offsets of one window, its waves the offsets' 128 x 64 halves,
 * each step's dY rows staged once for all four, steps in which an offset has
 * no pair skipped.  `rows` (optional, window kernel only, else
 * ST_ERR_UNSUPPORTED): the dY row of each map column, so that the caller can
 * hand the columns over in another order -- map(k, p) pairs X row map(k, p)
 * with dY row rows[p]; columns sorted by offset mask within slabs of the
 * output order make most offset steps all pairs or none.  NULL: column p is
 * dY row p.  Columns whose rows entry lies outside [0, n_out) add nothing.
 * Other shapes compact each (k, window) slice of map column k in LDS.
 * X (n_in, C_in) and dY (n_out, C_out) are `dtype` (map entries outside
 * [0, n_in) add nothing); dW (K, C_in, C_out) is written in `dw_dtype` (e.g.
 * fp32 master weights under bf16 activations).
 */
int st_wgrad(const void* X, int64_t n_in, const void* dY, const int32_t* map, int64_t map_k_stride,
             int64_t map_r_stride, const int32_t* rows, int64_t n_out, int K, int C_in, int C_out, int dtype,
             float* partials, int64_t splits, void* dW, int dw_dtype, st_stream_t stream);

/*
 * Weight gradient (precomputed_bwd_weight_kernel,
 * implicit_precomputed_gemm.py:180-230) over a pair list from st_kmap_pairs: every chunk of
 * `chunk` pairs is one equal-sized task (the centre offset of a submanifold
 * map has N pairs, the others far fewer), its C_in x C_out partial goes to
 * partials[chunk] (max_chunks * C_in * C_out fp32; max_chunks >= P / chunk + K,
 * or ST_PAIR_CHUNKS_AUTO_MAX for a list cut at ST_PAIR_CHUNK_AUTO, which is
 * passed here too) and each offset's chunks are summed in order.  Deterministic; fp32
 * gathers feed MFMA operands straight from HBM, 16-bit ones go through LDS.
 * chunk_order (optional, max_chunks int32): the order chunks are taken in
 * (st_kmap_pairs_chunk_keys); each workgroup takes a contiguous run of it and
 * the workgroups one XCD runs (launched round-robin over the 8 XCDs) take
 * adjacent runs, so chunks sharing input and output rows meet in one L2.
 * n_in / n_out: rows of X / dY (every pair indexes inside them).
 */
int st_wgrad_pairs(const void* X, int64_t n_in, const void* dY, int64_t n_out, const int32_t* pairs,
                   const int32_t* kstart, const int32_t* cstart, int K, int chunk, int64_t max_chunks,
                   const int32_t* chunk_order, int C_in, int C_out, int dtype, float* partials, void* dW, int dw_dtype,
                   st_stream_t stream);

/* ----------------------------------------------------- implicit hash-fly */

/* Lookup rule of the hash-fly kernels: for row r with coordinate c and offset k
 *   q = (c.xyz * mul + sign * offsets[k]) / div    (only when divisible)
 * looked up in the table if 0 <= q < bounds on every axis whose bound is > 0.
 * The forward bounds the input coordinate (the reference's in-bounds test,
 * implicit_hashfly_gemm.py:127); the input-gradient direction bounds the row
 * (row_bounds = the input shape) and leaves the output unbounded, since the
 * forward gives output rows outside the shape their in-bounds neighbours. */
typedef struct st_lookup {
  int32_t K;
  int32_t sign;          /* -1 forward (q = c*s - t_k), +1 input-gradient direction   */
  int64_t mul;
  int64_t div;
  int64_t bounds[3];     /* if > 0: q must satisfy 0 <= q < bounds on that axis       */
  int64_t row_bounds[3]; /* if > 0: rows with c outside [0, row_bounds) get no pairs  */
} st_lookup;

/*
 * Forward of ConvHashOnTheFlyImplicitGEMM (implicit_gemm_hash_on_fly_fwd_kernel,
 * implicit_hashfly_gemm.py:45-148) for a submanifold convolution (out = in
 * coordinates, stride 1, bounds = the index box), with the neighbours found
 * inside the GEMM in the coordinates' brick index (st_subm_index, same
 * geometry) instead of a hash table: no kernel map is stored.  Per 128-row
 * tile (rows 128t .. 128t + 127 of `rows`, a permutation of 0 .. n-1, or of
 * 0 .. n-1 itself when rows is NULL) each row looks up its K neighbours
 * (coords[r].xyz - offsets[k]; the lowest row of a repeated coordinate, as
 * the table holds), the tile's offset list is the union of its rows', and
 * out[r] = sum_k A[nbr(k, r)] Bt[k]^T (+ bias), Bt as st_gather_gemm's.
 * With rows = the st_kmap_sort_rows order of the offset masks
 * (st_kmap_subm_query with nbr = NULL) a tile's rows share their offsets, so
 * it loads fewer weight slices and runs fewer MFMAs; the sums do not change.
 * flags: 0 or ST_GATHER_REVERSE_K (offset k takes Bt[K - 1 - k]): the input
 * gradient of a submanifold map that is its own transpose (status DUPLICATE
 * and OUT_OF_BOX zero, offsets symmetric) takes the weights as given
 * (W (K, C_in, C_out) is then Bt) with no ST_W_REVERSE copy.  Bitwise
 * equal to st_hashfly_gemm and st_gather_gemm_tiled on the same rows.
 * st_subm_fly_ok(n, Kd, Nd, K, dtype) = 1 for the shapes built: Kd, Nd in
 * {64, 128} (split fp32 not at 128 x 128), K <= 27, dtype ST_BF16, ST_F16
 * or ST_F32_BF16X3, and n rows
 * of Kd elements under 2^31 - 64 bytes (the kernel addresses its operands
 * with 32-bit buffer offsets); others (and int64 coordinates) return
 * ST_ERR_UNSUPPORTED.  Host arithmetic only: it touches no device.
 */
int st_subm_fly_ok(int64_t n, int Kd, int Nd, int K, int dtype);
int st_subm_fly_gemm(const void* A, const void* coords, int coord_dtype, int64_t n, const int32_t* offsets, int K,
                     int64_t batches, int64_t sx, int64_t sy, int64_t sz, const void* index, int64_t index_bytes,
                     const int32_t* rows, const void* Bt, const void* bias, void* out, int Kd, int Nd, int dtype,
                     int flags, st_stream_t stream);

/*
 * Forward / input-gradient of ConvHashOnTheFlyImplicitGEMM
 * (implicit_gemm_hash_on_fly_fwd_kernel, implicit_hashfly_gemm.py:45-148, and
 * implicit_gemm_bwd_feat_kernel :151-237 recast as a gather): the same
 * gather-GEMM as st_gather_gemm with map(k, r) found by probing the table
 * inside the kernel, once per row tile rather than once per C_out tile.
 * dst_coords must be int16 or int32.
 */
int st_hashfly_gemm(const void* A, int64_t n_src, const void* dst_coords, int coord_dtype, int64_t n_dst,
                    const int32_t* offsets, const st_lookup* lk, const uint64_t* keys, const uint32_t* vals,
                    int64_t capacity, const void* Bt, const void* bias, void* out, int Kd, int Nd, int dtype,
                    st_stream_t stream);

/*
 * Weight gradient of ConvHashOnTheFlyImplicitGEMM (implicit_gemm_bwd_weight_kernel,
 * implicit_hashfly_gemm.py:239-328): st_wgrad with the pairs found by probing.
 * out_coords are the rows of dY; the table holds the rows of X.
 */
int st_hashfly_wgrad(const void* X, int64_t n_in, const void* dY, const void* out_coords, int coord_dtype,
                     int64_t n_out,
                     const int32_t* offsets, const st_lookup* lk, const uint64_t* keys, const uint32_t* vals,
                     int64_t capacity, int C_in, int C_out, int dtype, float* partials, int64_t splits, void* dW,
                     int dw_dtype, st_stream_t stream);

/* ------------------------------------------------------------ dense grids
 *
 * to_dense (utils/to_dense.py:30-282): out (batches, sx, sy, sz, C) of
 * `dtype`, channels last, is cleared and row r of feats (n, C) stored at the
 * cell of coords[r] = (b, x, y, z); coordinates outside the grid are skipped,
 * and a coordinate given twice keeps one of its rows.  st_from_dense is its
 * gradient (the reference's _to_dense_bwd_kernel): feats[r] = the cell of
 * coords[r], zeros outside the grid.
 */
int st_to_dense(const void* feats, int64_t n, int C, int dtype, const void* coords, int coord_dtype, int64_t batches,
                int64_t sx, int64_t sy, int64_t sz, void* out, st_stream_t stream);
int st_from_dense(const void* dense, int64_t batches, int64_t sx, int64_t sy, int64_t sz, int C, int dtype,
                  const void* coords, int coord_dtype, int64_t n, void* feats, st_stream_t stream);

/*
 * mask_spatial_range (utils/spatial/tile.py:16-85): mask[r] = 1 when row r's
 * (x, y, z) lies in [limits[0], limits[1]] x [limits[2], limits[3]] x
 * [limits[4], limits[5]] (inclusive; a host array of 6), else 0.
 */
int st_mask_spatial_range(const void* coords, int coord_dtype, int64_t n, const int64_t* limits, uint8_t* mask,
                          st_stream_t stream);

/* ------------------------------------------------------------ pooling, upsampling
 *
 * sparse_pooling (nn/functional/spatial.py:26-233): row r of coords goes to
 * the cell (b, floor((x + p - k/2) / s), ...) (spatial.py:104-107); the
 * outputs are the distinct cells in ascending (b, x, y, z) order.
 * st_pool_plan sorts the rows by cell (stable) into perm (n), writes the
 * first sorted position of each output into seg_start (n_out + 1, the last
 * entry = rows with a valid cell), each row's output into inv (n, -1 for a
 * cell outside the key range: b outside [0, 32767] or a spatial value outside
 * int16), the output coordinates into out_coords (rows 0 .. n_out-1 of an
 * n x 4 buffer of coord_dtype), and counts[0] = n_out, counts[1] = rows
 * without a valid cell.  workspace: st_pool_workspace(n) bytes.
 * st_pool_forward: out[o] = max (mode 0) or mean (mode 1) of its rows, fp32
 * arithmetic, rows in input order (deterministic).  st_pool_backward: each
 * row gets its output's gradient, whole where it equals the max (mode 0, the
 * reference's `in == out` rule) or divided by the row count (mode 1).
 */
int st_pool_workspace(int64_t n, size_t* bytes);
int st_pool_plan(const void* coords, int coord_dtype, int64_t n, int kernel_size, int stride, int padding,
                 void* workspace, size_t workspace_bytes, int32_t* perm, int32_t* seg_start, int32_t* inv,
                 void* out_coords, int32_t* counts, st_stream_t stream);
int st_pool_forward(const void* feats, int C, int dtype, const int32_t* perm, const int32_t* seg_start, int64_t n_out,
                    int mode, void* out, st_stream_t stream);
int st_pool_backward(const void* feats, const void* out, const void* dout, int64_t n, int C, int dtype,
                     const int32_t* inv, const int32_t* seg_start, int mode, void* dfeats, st_stream_t stream);

/*
 * sparse_upsample (spatial.py:236-436): row r becomes rows r * s^3 + q,
 * q = (dx * s + dy) * s + dz, at (b, x s + dx, y s + dy, z s + dz) with r's
 * features; the backward sums each row's s^3 output gradients (fp32).
 */
int st_upsample(const void* feats, const void* coords, int coord_dtype, int64_t n, int C, int dtype, int scale,
                void* out_feats, void* out_coords, st_stream_t stream);
int st_upsample_backward(const void* dout, int64_t n, int C, int dtype, int scale, void* dfeats, st_stream_t stream);

/* ------------------------------------------------------------ batch norm
 *
 * Per-sample batch normalisation of sparse features (sparse_batch_norm,
 * nn/functional/norm.py:20-112) with the residual add and ReLU of the
 * reference's blocks (nn/modules/blocks.py:21-124) fused into its output pass:
 *   out = act((Y - mean[b, c]) * invstd[b, c] * weight[c] + bias[c] + residual)
 * b = coords[r, 0] (rows with b outside [0, B) are written as zeros and left
 * out of the statistics).  Training: mean and biased variance of each sample's
 * rows (two passes, deterministic sums), running statistics (when given) move
 * by `momentum` towards their mean over the B samples (norm.py:86-90).
 * Evaluation: mean = running_mean, var = running_var, per channel.
 * Y, residual (optional), out: (n, C) of `dtype`; weight, bias (optional:
 * NULL means 1 and 0), running statistics: fp32 (C); mean, invstd: fp32
 * (B, C) in training, (C) in evaluation; counts: int32 (B), rows per sample.
 */
#define ST_BN_MAX_BATCH 4096
int st_bn_workspace(int64_t n, int C, int B, int64_t* floats);
int st_bn_forward(const void* Y, int64_t n, int C, int dtype, const void* coords, int coord_dtype, int B,
                  const float* weight, const float* bias, const void* residual, int relu, int training, float eps,
                  float momentum, float* running_mean, float* running_var, float* mean, float* invstd,
                  int32_t* counts, float* workspace, int64_t workspace_floats, void* out, st_stream_t stream);

/*
 * Gradients of st_bn_forward (the reference gets them from torch autograd
 * through its formula, including the paths through the sample mean and
 * variance): with g = dout masked by out > 0 under relu,
 *   dres = g (optional), dweight[c] = sum g * xhat, dbias[c] = sum g (fp32, optional),
 *   training:   dY = weight * invstd * (g - mean_b(g) - xhat * mean_b(g * xhat))
 *   evaluation: dY = weight * invstd * g
 * xhat = (Y - mean) * invstd.  Y and out are the forward's input and output
 * (out is read only under relu, and may be NULL otherwise); mean, invstd and
 * counts its saved statistics.  The workspace is
 * st_bn_workspace(n, C, training ? B : 1) floats.
 */
int st_bn_backward(const void* Y, const void* out, const void* dout, int64_t n, int C, int dtype, const void* coords,
                   int coord_dtype, int B, const float* weight, int relu, int training, const float* mean,
                   const float* invstd, const int32_t* counts, float* workspace, int64_t workspace_floats, void* dY,
                   void* dres, float* dweight, float* dbias, st_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SPARSETRITON_AMD_H */
