/*
 * riemann_hip.h — C ABI of the MI355X (gfx950) sparse-convolution hot path.
 *
 * The library is stateless: every buffer is owned by the caller (device
 * pointers unless stated otherwise), every call takes the HIP stream it runs
 * on, and nothing throws across the boundary. Each entry point returns an
 * rhip_status; on failure rhip_last_error() holds a thread-local message.
 * Calls whose output size is data-dependent (hash build, kernel-map count)
 * synchronise the stream once to read that size back to the host; all other
 * calls are asynchronous.
 *
 * Coordinates are int32 rows [N, ncol] with ncol = D + 1 and the batch index
 * first (reference: RiemannEngine/engine/tensor/sparse_tensor.cpp:70-77,
 * docs/concepts.md:41). Row indices are int32, as the reference's uint32
 * index_type (engine/foundation/types.hpp:30) restricted to < 2^31.
 * Weights are [K, Cin, Cout] row-major (engine/nn/conv.cpp:83-86).
 */
#ifndef RIEMANN_HIP_H
#define RIEMANN_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RHIP_ABI_VERSION 13
#define RHIP_MAX_COLS 8 /* batch column + up to 7 spatial axes */

typedef enum rhip_status {
  RHIP_OK = 0,
  RHIP_ERR_INVALID = 1,     /* bad argument: shape, size, null pointer */
  RHIP_ERR_HIP = 2,         /* a HIP runtime call failed */
  RHIP_ERR_UNSUPPORTED = 3, /* valid input this build cannot handle */
  RHIP_ERR_WORKSPACE = 4    /* workspace smaller than the queried size */
} rhip_status;

typedef enum rhip_dtype { RHIP_F32 = 0, RHIP_BF16 = 1 } rhip_dtype;

typedef enum rhip_key_mode {
  /* Rows packed into one 63-bit integer from the per-column [lo, hi]
   * range of the inserted set; probes compare integers only. */
  RHIP_KEY_PACKED64 = 0,
  /* Fallback when the ranges need more than 63 bits: slots hold a 32-bit
   * row hash plus a unique-row index and probes compare whole rows. */
  RHIP_KEY_ROWREF = 1
} rhip_key_mode;

/*
 * Descriptor of a built coordinate hash table (one coordinate map).
 * Filled by rhip_hash_build; passed by pointer to lookups and kernel maps.
 * Replaces CoordinateMapGPU + concurrent_unordered_map
 * (engine/grid/lattice_gpu.cuh:221-678, vendor/concurrent_unordered_map.cuh).
 */
typedef struct rhip_table {
  void *slots;            /* device, capacity * 16 bytes */
  int64_t capacity;       /* power of two, >= 2 * n */
  const int32_t *rows;    /* device [n_unique, ncol] unique coordinates */
  int64_t n_unique;
  int32_t ncol;
  int32_t mode;           /* rhip_key_mode */
  int32_t key_bits;       /* packed width (RHIP_KEY_PACKED64) */
  int32_t lo[RHIP_MAX_COLS];
  int32_t hi[RHIP_MAX_COLS];
  int32_t shift[RHIP_MAX_COLS];
  /* Trailing zero bits common to every (c - lo[c]) of a column (coordinates
   * at tensor stride 2^s have s); the locality key drops them. */
  int32_t tz[RHIP_MAX_COLS];
  /* Brick index, set by rhip_spatial_order when it is given brick storage
   * (else bricks is NULL): the unique rows in locality order, and a dense
   * grid over the bounding box of bricks of 2^(brick_levels * D) cells, each
   * entry a 64-bit occupancy mask of the brick's cells and the locality-order
   * position of its first row. A neighbour query reads one entry and a
   * popcount instead of probing the hash table. */
  const int32_t *order;
  void *bricks;
  int32_t morton_bits;  /* bits per spatial column of the locality key */
  int32_t brick_levels; /* Morton levels inside a brick */
  int32_t brick_dims[RHIP_MAX_COLS]; /* grid extent per column (0: batch) */
} rhip_table;

/* ---------------------------------------------------------------- misc */

const char *rhip_last_error(void);
int rhip_abi_version(void);

/* ---------------------------------------------------- coordinate hashing */

/* Bytes of slot storage for a table built over n rows (16 B per slot). */
size_t rhip_table_bytes(int64_t n);
int rhip_hash_workspace_bytes(int64_t n, int32_t ncol, size_t *bytes);

/*
 * Deduplicate n coordinate rows into a hash table. Unique rows are numbered
 * in first-occurrence order, exactly as the reference CPU map does:
 *   unique_coords = coords[mapping],  coords == unique_coords[inverse].
 * unique_coords needs room for n rows and mapping for n entries; only the
 * first table->n_unique are written. inverse (n entries) may be NULL.
 * Synchronises `stream` once to read n_unique. When some row repeats an
 * earlier one, the repeats' inverse entries are written by a launch queued
 * after that synchronisation: as with the asynchronous entry points, the
 * workspace and inverse stay in use until `stream` has passed the call.
 *
 * Replaces CoordinateMapGPU::insert_and_map (engine/grid/lattice_gpu.cu:157-243,
 * insert_and_map_kernel :26-51, remap_inverse_map :54-71), with the semantics
 * of CoordinateMapCPU::insert_and_map<true> (engine/grid/lattice_cpu.hpp:419-444).
 */
int rhip_hash_build(const int32_t *coords, int64_t n, int32_t ncol,
                    void *slots, size_t slots_bytes, void *workspace,
                    size_t workspace_bytes, int32_t *unique_coords,
                    int64_t *mapping, int64_t *inverse, rhip_table *table,
                    hipStream_t stream);

/*
 * result[i] = unique row index of queries[i] in the table, or -1.
 * Replaces CoordinateMapGPU::find (engine/grid/lattice_gpu.cu:265-301), which
 * returns only the hits; here misses are kept in place as -1.
 */
int rhip_hash_lookup(const rhip_table *table, const int32_t *queries,
                     int64_t n, int32_t *result, hipStream_t stream);

/*
 * Locality order of a table's unique rows: order[j] is the row processed at
 * position j, pos is its inverse. Rows are sorted by batch, then by the
 * Morton (bit-interleaved) code of their spatial columns, (c - lo) >> tz
 * each, when that fits in 63 bits, else by the packed key (x, then y, then
 * z); identity in RHIP_KEY_ROWREF mode. Used to order output rows so that
 * neighbouring positions have neighbouring rows; it does not renumber rows.
 *
 * With brick storage (rhip_brick_bytes(table) bytes, non-zero) and a Morton
 * order, also builds the table's brick index over `order` (which must then
 * outlive the table's use in kernel maps) and records it in *table; bricks
 * NULL or 0 bytes leave table->bricks NULL. rhip_brick_bytes is 0 when the
 * bounding box of bricks exceeds 16 entries per row or 2^23 entries.
 */
int rhip_order_workspace_bytes(int64_t n, size_t *bytes);
int rhip_brick_bytes(const rhip_table *table, size_t *bytes);
int rhip_spatial_order(rhip_table *table, int32_t *order, int32_t *pos, void *bricks,
                       size_t brick_bytes, void *workspace, size_t workspace_bytes,
                       hipStream_t stream);

/*
 * out = (b, floor(x_i / s_i) * s_i) for every row; s = out tensor stride
 * (host array of ncol-1 positive values). Feed `out` to rhip_hash_build to
 * get the strided coordinate map.
 * Replaces stride_copy (engine/grid/lattice_gpu.cu:305-336) with the
 * semantics of detail::stride_coordinate (engine/grid/stencil.hpp:35-52).
 */
int rhip_stride_coords(const int32_t *coords, int64_t n, int32_t ncol,
                       const int32_t *out_tensor_stride, int32_t *out,
                       hipStream_t stream);

/*
 * Generative expansion of a coordinate set through a kernel region:
 * out[i*K + k] = coords[i] + offsets[k] (batch column kept) for every input
 * row i and offset k. offsets is a DEVICE array [K, ncol-1] of scaled lattice
 * offsets: the region at the OUTPUT tensor stride. Feed out ([n*K, ncol]) to
 * rhip_hash_build; its unique rows (first occurrence in (i, k) order) are the
 * generated output map of a generative transposed convolution.
 * Replaces the transposed branch of CoordinateMapCPU::stride_region
 * (engine/grid/lattice_cpu.hpp:499-534) and kernel_region_insert
 * (engine/grid/lattice_gpu.cu:426-601); called through
 * CoordinateMapManager::stride_region (engine/grid/space_impl.hpp:352-381).
 */
int rhip_expand_coords(const int32_t *coords, int64_t n, int32_t ncol,
                       const int32_t *offsets, int32_t K, int32_t *out,
                       hipStream_t stream);

/* ------------------------------------------------------------ kernel map */

/* Workspace shared by the two phases of one kernel map (pass the same
 * buffer, unchanged, to rhip_kmap_count and rhip_kmap_fill). */
int rhip_kmap_workspace_bytes(int64_t n_in, int64_t n_out, int32_t K,
                              size_t *bytes);

/* Set by rhip_kmap_count for a map of a coordinate set onto itself (out_coords
 * are in_table's own rows, in order) whose stencil offsets are distinct and
 * closed under negation: one offset of each +/- pair is probed and the
 * transposed table is the forward table with each offset's negation. Pass
 * it to rhip_kmap_fill. */
#define RHIP_KMAP_SYMMETRIC 1
/* Reported by rhip_kmap_count when its probes read each output row's
 * neighbourhood bricks once (a symmetric 3^3 map in 3-D or 3^4 map in 4-D
 * whose in_table has a brick grid); the map is the same either way.
 * rhip_kmap_fill ignores it. */
#define RHIP_KMAP_BRICK_NBHD 2

/*
 * Phase 1 of kernel-map generation. For every output row and every offset
 * k, look up out_coords[row] + offsets[k] (batch column unchanged) in
 * in_table. offsets_host is a HOST array [K, ncol-1] of already scaled
 * lattice offsets (kernel_region::coordinate_at, engine/grid/stencil.hpp:
 * 223-278); the library copies it to the device. The rows are queried in
 * out_spatial_order (a locality order of the output map, e.g. from
 * rhip_spatial_order; NULL = row order) and then put in a processing order
 * that groups rows with equal neighbour masks (K <= 128; ties keep the
 * locality order). Outputs:
 *   out_order[p]   output row at processing position p (n_out entries);
 *   nbr[k*n_out+p] input row paired with out_order[p] under k, or -1;
 *   kmap_offsets   device int64 [K+1], CSR of the pairs per offset, copied
 *                  to kmap_offsets_host;
 *   *flags         RHIP_KMAP_SYMMETRIC and RHIP_KMAP_BRICK_NBHD bits, or 0
 *                  (flags may be NULL).
 * Synchronises `stream` once (to read the pair counts) when kmap_offsets_host
 * is given; with kmap_offsets_host NULL it is asynchronous, and the caller
 * sizes the pair lists of rhip_kmap_fill by the bound K * n_out (or reads
 * kmap_offsets itself first).
 * Replaces CoordinateMapGPU::kernel_map / direct_kernel_map / count_kernel
 * (engine/grid/lattice_gpu.cu:1140-1362, 1366-1549); the live reference
 * semantics are CoordinateMapCPU::kernel_map (engine/grid/lattice_cpu.hpp:606-673).
 */
int rhip_kmap_count(const rhip_table *in_table, const int32_t *out_coords,
                    const int32_t *out_spatial_order, int64_t n_out, int32_t K,
                    const int32_t *offsets_host, void *workspace,
                    size_t workspace_bytes, int32_t *nbr, int32_t *out_order,
                    int64_t *kmap_offsets, int64_t *kmap_offsets_host,
                    int32_t *flags, hipStream_t stream);

/*
 * Phase 2: emit the pairs of offset k at [kmap_offsets[k], kmap_offsets[k+1])
 * of in_rows / out_rows, ordered by offset, then by output processing
 * position (in_rows and out_rows both NULL: no pair lists; rhip_kmap_pairs
 * emits them later from the table). If nbr_t is not NULL, also fix a
 * processing order of the input rows (in_order, grouping equal transposed
 * masks; ties keep in_spatial_order, NULL = row order) and fill the
 * transposed table nbr_t[k*n_in+q] = output row paired with in_order[q]
 * under k, or -1. A symmetric map without pair lists and without nbr_t
 * launches nothing: its convolution runs from nbr alone (see
 * rhip_conv_backward_input). flags and the workspace must be what phase 1
 * produced. Asynchronous.
 * Replaces gpu_kernel_map::decompose (engine/grid/lattice_gpu.cuh:438-488);
 * the set of pairs equals the reference's cpu_kernel_map.
 */
int rhip_kmap_fill(const int32_t *nbr, const int32_t *out_order, int64_t n_out,
                   int32_t K, const int32_t *in_spatial_order, int64_t n_in,
                   int32_t flags, void *workspace, size_t workspace_bytes,
                   const int64_t *kmap_offsets, int32_t *in_rows,
                   int32_t *out_rows, int32_t *nbr_t, int32_t *in_order,
                   hipStream_t stream);

/* Workspace of rhip_kmap_pairs for a table of n_out positions and K offsets. */
int rhip_kmap_pairs_workspace_bytes(int64_t n_out, int32_t K, size_t *bytes);

/*
 * The pair lists of a finished map from its table: the same in_rows /
 * out_rows (order included) that rhip_kmap_fill emits, sized by
 * kmap_offsets[K] (the device CSR of rhip_kmap_count). For maps whose pair
 * lists are needed only sometimes (the pair-list weight gradient,
 * kernel_map_to_tensors): the build then writes no 8 P bytes it may never
 * read. Asynchronous.
 * Replaces the triplet output of gpu_kernel_map::decompose
 * (engine/grid/lattice_gpu.cuh:438-488) on demand.
 */
int rhip_kmap_pairs(const int32_t *nbr, const int32_t *out_order, int64_t n_out,
                    int32_t K, const int64_t *kmap_offsets, void *workspace,
                    size_t workspace_bytes, int32_t *in_rows, int32_t *out_rows,
                    hipStream_t stream);

/*
 * partner_host[a] = the offset b with offsets[b] = -offsets[a] (int32
 * wrap-around negation, the coordinate type's) for a stencil [K, D] (host)
 * closed under negation with distinct offsets; RHIP_ERR_UNSUPPORTED
 * otherwise. Host only. The partners of a symmetric map (RHIP_KMAP_SYMMETRIC)
 * are the weight permutation of its input gradient. Replaces the transposed
 * map a cached forward map yields by swap_in_out_map (engine/grid/
 * space_impl.hpp:649-697) for a map of a set onto itself.
 */
int rhip_stencil_partners(const int32_t *offsets_host, int32_t K, int32_t D,
                          int32_t *partner_host);

/* ----------------------------------------------------------- convolution */

/* Workspace of one layer's forward, input-gradient and weight-gradient calls
 * (the same buffer may serve all three, one call at a time) for a kernel map
 * with n_in input rows, n_out output rows and n_pairs pairs. */
int rhip_conv_workspace_bytes(int32_t K, int32_t cin, int32_t cout,
                              int32_t dtype, int64_t n_in, int64_t n_out,
                              int64_t n_pairs, size_t *bytes);

/* Workspace of one layer's forward, input-gradient and bias-gradient calls
 * alone (no weight gradient): the front part of the rhip_conv_workspace_bytes
 * layout. */
int rhip_conv_forward_workspace_bytes(int32_t K, int32_t cin, int32_t cout,
                                      int32_t dtype, int64_t n_in, int64_t n_out,
                                      size_t *bytes);

/*
 * Y[out_order[j]] = sum_k X[nbr[k*n_out+j]] @ W[k] (+ bias), fp32 accumulate.
 * x [n_in, cin], weight [K, cin, cout], y [n_out, cout], all in `dtype`;
 * bias is fp32 [cout] or NULL. Every output row is written.
 * Replaces the per-offset index_select -> matmul -> index_add_ loop of
 * evaluate_sparse_convolution (engine/nn/conv.cpp:47-64) and its bias add
 * (conv.cpp:135-136).
 */
int rhip_conv_forward(const void *x, int64_t n_in, int32_t cin,
                      const void *weight, int32_t K, int32_t cout,
                      const float *bias, const int32_t *nbr,
                      const int32_t *out_order, int64_t n_out, void *y,
                      int32_t dtype, void *workspace, size_t workspace_bytes,
                      hipStream_t stream);

/*
 * rhip_conv_forward without a workspace: no counterpart in the reference.
 * For callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): it calls no allocating
 * routine. The transposed weights go to an 8 MiB device array of the
 * library (one per GPU, held until the process ends), so K*cin*cout times
 * the dtype size must not exceed 8 MiB (RHIP_ERR_UNSUPPORTED otherwise),
 * and the offset axis is never split. Calls share that array: calls on one
 * stream run in order, and a call on another stream first waits (on the
 * device) for the previous call's kernels through an event the library
 * creates once per GPU, so eager calls from several streams take turns.
 * Under graph capture a call is refused (RHIP_ERR_INVALID) while another
 * stream's call may still be running; replays of a captured graph are not
 * ordered against other streams' calls by the library. Same arguments and
 * results as rhip_conv_forward.
 */
int rhip_conv_forward_noalloc(const void *x, int64_t n_in, int32_t cin,
                              const void *weight, int32_t K, int32_t cout,
                              const float *bias, const int32_t *nbr,
                              const int32_t *out_order, int64_t n_out, void *y,
                              int32_t dtype, hipStream_t stream);

/*
 * grad_bias[c] = sum over rows of grad_y[r][c] (grad_y [n_out, cout] in
 * dtype, grad_bias fp32 [cout], overwritten), fp32 accumulation in a fixed
 * order (deterministic). Workspace: either layer workspace above.
 * Replaces the bias half of the reference's autograd graph for
 * `output + bias_` (engine/nn/conv.cpp:135-136).
 */
int rhip_conv_bias_grad(const void *grad_y, int64_t n_out, int32_t cout,
                        int32_t dtype, float *grad_bias, void *workspace,
                        size_t workspace_bytes, hipStream_t stream);

/*
 * grad_x[in_order[j]] = sum_k grad_y[nbr_t[k*n_in+j]] @ W[p(k)]^T, where
 * p(k) = weight_perm[k] (device int32 [K]) or k when weight_perm is NULL.
 * A symmetric map (RHIP_KMAP_SYMMETRIC) needs no transposed table: pass its
 * nbr as nbr_t, its out_order as in_order and its stencil partners
 * (rhip_stencil_partners, uploaded) as weight_perm, since input row i pairs
 * with output row o under k exactly when o pairs with i under the partner
 * of k. With weight_perm, shapes the LDS-indexed kernel does not take copy
 * the reordered weights into the workspace first, so it is then required.
 * Replaces the autograd replay of IndexAddBackward/MmBackward/
 * IndexSelectBackward for dX (engine/nn/conv.cpp:62-63).
 */
int rhip_conv_backward_input(const void *grad_y, int64_t n_out, int32_t cout,
                             const void *weight, int32_t K, int32_t cin,
                             const int32_t *nbr_t, const int32_t *weight_perm,
                             const int32_t *in_order, int64_t n_in, void *grad_x,
                             int32_t dtype, void *workspace,
                             size_t workspace_bytes, hipStream_t stream);

/*
 * grad_w[k] = sum over pairs p of offset k of x[in_rows[p]]^T grad_y[out_rows[p]]
 * with fp32 accumulation; grad_w [K, cin, cout] in `dtype` is overwritten.
 * Deterministic: partial sums per pair range are added in a fixed order.
 * kmap_offsets is the device CSR from rhip_kmap_count.
 * Replaces the dW half of MmBackward in the reference's autograd graph
 * (engine/nn/conv.cpp:62) and sparse_convolution_backward_cpu_kernel's
 * kernel_grad (engine/ops/convolution_cpu.hpp:55-89).
 */
int rhip_conv_backward_weight(const void *x, int64_t n_in, int32_t cin,
                              const void *grad_y, int64_t n_out, int32_t cout,
                              int32_t K, const int64_t *kmap_offsets,
                              int64_t n_pairs, const int32_t *in_rows,
                              const int32_t *out_rows, void *grad_w,
                              int32_t dtype, void *workspace,
                              size_t workspace_bytes, hipStream_t stream);

/*
 * The same weight gradient from the dense neighbour table instead of the
 * pair list: grad_w[k] = sum over output positions j with
 * nbr[k*n_out+j] >= 0 of x[nbr[k*n_out+j]]^T grad_y[out_order[j]]
 * (out_order NULL = identity), fp32 accumulation, deterministic. Each dY
 * row is read once per group of offsets rather than once per pair, and the
 * X rows that neighbouring positions share are read once per position
 * range. Supported: bf16 with 16 or 32 input and output channels, and at
 * most 8 or at least 20 offsets with input channels a multiple of 16 and
 * output channels a multiple of 32 (each of x, grad_y and the table under
 * 2 GiB); other shapes return
 * RHIP_ERR_UNSUPPORTED, for which rhip_conv_backward_weight is the
 * fallback. Workspace as for rhip_conv_workspace_bytes.
 * Replaces the dW half of MmBackward (engine/nn/conv.cpp:62), like
 * rhip_conv_backward_weight.
 */
int rhip_conv_backward_weight_rows(const void *x, int64_t n_in, int32_t cin,
                                   const void *grad_y, int64_t n_out,
                                   int32_t cout, int32_t K, const int32_t *nbr,
                                   const int32_t *out_order, void *grad_w,
                                   int32_t dtype, void *workspace,
                                   size_t workspace_bytes, hipStream_t stream);

/* 1 if rhip_conv_backward_weight_rows takes this shape, else 0 (no status:
 * a pure query of its dispatch rules, for callers that decide ahead of time
 * whether the pair lists will be needed, e.g. RiemannConvolution's forward,
 * engine/nn/conv.cpp:104-138). */
int rhip_conv_backward_weight_rows_supported(int32_t dtype, int32_t cin, int32_t cout,
                                             int32_t K, int64_t n_in, int64_t n_out);

/* --------------------------------------------------------------- pooling */

/* Reductions of local and global pooling (engine/foundation/types.hpp:121-136:
 * LOCAL_{SUM,AVG,MAX}_POOLING and the GLOBAL_* modes, which reduce the same
 * three ways). */
typedef enum rhip_pool_mode {
  RHIP_POOL_SUM = 0,
  RHIP_POOL_AVG = 1, /* sum / number of pooled rows */
  RHIP_POOL_MAX = 2, /* NaN propagates; the gradient splits evenly between ties */
  /* Max as zeros.scatter_reduce("amax", include_self=False) computes it
   * (SparseTensor MAX_POOL quantization, engine/tensor/sparse_tensor.cpp:
   * 474-479): the forward equals RHIP_POOL_MAX; the backward also counts the
   * excluded zero as a tie when the maximum is 0 (t + 1 ways). Local pooling
   * only. */
  RHIP_POOL_MAX_SCATTER = 3
} rhip_pool_mode;

/* Workspace shared by the two phases of one stride map (pass the same
 * buffer, unchanged, to rhip_stride_map_count and rhip_stride_map_fill). */
int rhip_stride_map_workspace_bytes(int64_t n_in, int64_t n_out, size_t *bytes);

/*
 * Phase 1 of a pooling stride map (kernel size == stride): every input row
 * maps to the output row holding its floor-aligned coordinates
 * (b, floor(x_d / s_d) * s_d) in out_table; out_tensor_stride is a HOST array
 * [ncol-1]. The inputs are grouped by output (ascending input row within a
 * group) in the workspace and *k_max_host receives the largest group, the
 * height of the neighbour table of phase 2. Synchronises the stream once.
 * Fails with RHIP_ERR_INVALID when an input row has no output row, as the
 * reference's ASSERT does.
 * Replaces CoordinateMapCPU::stride_map (engine/grid/lattice_cpu.hpp:675-710)
 * behind stride_map_functor (engine/grid/space_impl.hpp:617-626, 660-669) and
 * CoordinateMapGPU::stride_map (engine/grid/lattice_gpu.cu:1553-1670).
 */
int rhip_stride_map_count(const rhip_table *out_table, const int32_t *in_coords,
                          int64_t n_in, const int32_t *out_tensor_stride,
                          void *workspace, size_t workspace_bytes,
                          int32_t *k_max_host, hipStream_t stream);

/*
 * Phase 1 of a group map, the same grouping for rows whose group is given:
 * row i belongs to group[i] in [0, n_groups) (e.g. the inverse map of
 * rhip_hash_build, each row's unique coordinate). Phase 2 is
 * rhip_stride_map_fill with n_in = n, n_out = n_groups; local pooling over
 * the result reduces each group (SparseTensor quantization). Workspace:
 * rhip_stride_map_workspace_bytes(n, n_groups). Synchronises once; fails
 * with RHIP_ERR_INVALID for a group outside [0, n_groups).
 * Replaces the index_add_ / scatter_reduce("amax") by row_to_unique of
 * SparseTensor::quantize_features (engine/tensor/sparse_tensor.cpp:447-481).
 */
int rhip_group_map_count(const int32_t *group, int64_t n, int64_t n_groups,
                         void *workspace, size_t workspace_bytes,
                         int32_t *k_max_host, hipStream_t stream);

/*
 * Phase 2: the stride map in the neighbour-table form of a kernel map
 * (columns by processing position, as rhip_kmap_count / rhip_kmap_fill):
 *   nbr [k_max, n_out]: nbr[k*n_out+p] = k-th input row (ascending) of the
 *                       output out_order[p], -1 past its group;
 *   nbr_t [1, n_in]:    nbr_t[q] = the output row of input in_order[q] (each
 *                       input has exactly one);
 *   in_rows/out_rows [n_in]: the reference's single pair list (one kernel
 *                       offset), grouped by output.
 * in_order / out_order are processing orders (permutations; NULL = row order),
 * e.g. the locality orders of the two maps.
 */
int rhip_stride_map_fill(int64_t n_in, int64_t n_out, int32_t k_max,
                         const int32_t *in_order, const int32_t *out_order,
                         void *workspace, size_t workspace_bytes, int32_t *nbr,
                         int32_t *nbr_t, int32_t *in_rows, int32_t *out_rows,
                         hipStream_t stream);

/*
 * Pooling form of a neighbour table [K, n] (a kernel map's nbr or nbr_t):
 * each column's entries >= 0 moved to its first rows in row order, -1 after
 * them, into out [K, n] (no aliasing); *k_used_host = the most entries of
 * one column, so that a pooling kernel reads only rows [0, k_used). Pooling
 * reduces a set of rows, so the offset a row came from does not matter
 * there (a convolution table must not be compacted). workspace: 4 bytes of
 * device memory. Synchronises once.
 */
int rhip_table_compact(const int32_t *table, int32_t K, int64_t n,
                       void *workspace, size_t workspace_bytes, int32_t *out,
                       int32_t *k_used_host, hipStream_t stream);

/* Workspace of rhip_pool_backward (max pooling keeps one fp32 per output
 * element; sum and average need none). */
int rhip_pool_workspace_bytes(int64_t n_out, int32_t C, int32_t mode,
                              size_t *bytes);

/*
 * Local pooling: y[out_order[p]] = reduce over k < K with i = nbr[k*n_out+p]
 * >= 0 of x[i] (channel-wise, fp32 accumulation, x and y in `dtype`); an
 * output with no input row is 0. counts [n_out] (optional) receives the
 * number of rows pooled into each output row, which average-pooling backward
 * needs. nbr and out_order are a kernel map's (rhip_kmap_count) or a stride
 * map's (rhip_stride_map_fill); out_order NULL = row order.
 * Replaces evaluate_pooling's per-output index_select + sum/mean/amax + stack
 * (engine/nn/pooling.cpp:80-150).
 */
int rhip_pool_forward(const void *x, int64_t n_in, int32_t C,
                      const int32_t *nbr, int32_t K, const int32_t *out_order,
                      int64_t n_out, int32_t mode, void *y, int32_t *counts,
                      int32_t dtype, hipStream_t stream);

/*
 * Local pooling backward: grad_x[i] for i = in_order[q] is the sum over k <
 * K_t with o = nbr_t[k*n_in+q] >= 0 of  sum: grad_y[o];  average: grad_y[o] /
 * counts[o];  max: grad_y[o] / t where x[i] == y[o] (t = number of pooled
 * rows equal to y[o], per channel), else 0. grad_x [n_in, C] is overwritten.
 * K and K_t are the row counts of nbr and nbr_t (equal for a kernel map; a
 * stride map's nbr_t has one row). Max pooling also needs x, y, nbr,
 * out_order and the workspace; average needs counts from rhip_pool_forward.
 * Replaces the autograd replay of StackBackward / SumBackward / MeanBackward /
 * AmaxBackward / IndexSelectBackward of evaluate_pooling
 * (engine/nn/pooling.cpp:120-140).
 */
int rhip_pool_backward(const void *grad_y, const void *y, const void *x,
                       int64_t n_out, int32_t C, const int32_t *nbr, int32_t K,
                       const int32_t *out_order, const int32_t *nbr_t,
                       int32_t K_t, const int32_t *in_order,
                       int64_t n_in, const int32_t *counts, int32_t mode,
                       void *grad_x, int32_t dtype, void *workspace,
                       size_t workspace_bytes, hipStream_t stream);

/* Workspace of the global-pooling calls over n rows, C channels and
 * n_batches batches (rhip_batch_count and rhip_batch_segments accept it with
 * any n_batches). */
int rhip_global_pool_workspace_bytes(int64_t n, int32_t C, int32_t n_batches,
                                     size_t *bytes);

/*
 * Number of batches of a coordinate set: max(batch column) + 1, 0 when every
 * batch index is negative or n == 0. Synchronises the stream once.
 * Replaces coordinates.select(1, 0).max() + 1
 * (engine/nn/pooling.cpp:207-212).
 */
int rhip_batch_count(const int32_t *coords, int64_t n, int32_t ncol,
                     void *workspace, size_t workspace_bytes,
                     int32_t *n_batches_host, hipStream_t stream);

/*
 * Rows grouped by batch: rows of batch b are members[seg[b] .. seg[b+1]) in
 * ascending row order (members [n], seg [n_batches+1]); rows whose batch is
 * outside [0, n_batches) follow seg[n_batches] and belong to no batch.
 * Replaces the per-batch at::nonzero(coordinates.select(1, 0) == batch)
 * (engine/nn/pooling.cpp:220-224).
 */
int rhip_batch_segments(const int32_t *coords, int64_t n, int32_t ncol,
                        int32_t n_batches, void *workspace, size_t workspace_bytes,
                        int32_t *members, int32_t *seg, hipStream_t stream);

/*
 * Global pooling: y[b] = reduce of x over the rows of batch b ([n_batches, C],
 * fp32 accumulation in a fixed order, 0 for an empty batch).
 * Replaces RiemannGlobalPoolingImpl::forward's per-batch reduction
 * (engine/nn/pooling.cpp:203-260).
 */
int rhip_global_pool_forward(const void *x, int64_t n, int32_t C,
                             const int32_t *members, const int32_t *seg,
                             int32_t n_batches, int32_t mode, void *y,
                             int32_t dtype, void *workspace,
                             size_t workspace_bytes, hipStream_t stream);

/*
 * Global pooling backward: grad_x[i] for a row of batch b = coords[i][0]:
 * sum: grad_y[b]; average: grad_y[b] / rows of b; max: grad_y[b] / t where
 * x[i] == y[b] (t tied rows per channel), else 0; 0 for rows outside every
 * batch. Max pooling also needs x, y, members and the workspace.
 * Replaces the autograd replay of the reference's global pooling graph
 * (engine/nn/pooling.cpp:225-259).
 */
int rhip_global_pool_backward(const void *grad_y, const void *y, const void *x,
                              const int32_t *coords, int32_t ncol, int64_t n,
                              int32_t C, const int32_t *members,
                              const int32_t *seg, int32_t n_batches,
                              int32_t mode, void *grad_x, int32_t dtype,
                              void *workspace, size_t workspace_bytes,
                              hipStream_t stream);

/* ------------------------------------------------------------ batch norm
 *
 * Batch normalisation of [n, C] features (fp32 or bf16) with fp32
 * statistics and parameters, as torch BatchNorm1d computes it for
 * RiemannBatchNorm (engine/nn/normalization.hpp:11-37): biased batch
 * variance for normalising, unbiased variance into running_var. The
 * forward optionally adds a residual and applies ReLU after the affine
 * transform, BasicBlock's `norm2 -> += residual -> relu` tail and the
 * `norm1 -> relu` of its first half (engine/nn/residual.cpp:44-51).
 */

/* Workspace bytes for rhip_bn_stats and rhip_bn_backward over n rows. */
int rhip_bn_workspace_bytes(int64_t n, int32_t C, size_t *bytes);

/*
 * Batch statistics: mean[c] and invstd[c] = 1 / sqrt(var_biased[c] + eps)
 * over n > 1 rows (fp64 sums in a fixed order: deterministic). When
 * running_mean / running_var are given they become
 * (1 - momentum) * old + momentum * (mean | var * n / (n - 1)).
 * Replaces BatchNorm1d's training-mode statistics (torch batch_norm).
 */
int rhip_bn_stats(const void *x, int64_t n, int32_t C, int32_t dtype, double eps,
                  double momentum, float *running_mean, float *running_var,
                  float *mean, float *invstd, void *workspace,
                  size_t workspace_bytes, hipStream_t stream);

/* invstd[c] = 1 / sqrt(var[c] + eps): evaluation with running statistics. */
int rhip_bn_invstd(const float *var, int32_t C, double eps, float *invstd,
                   hipStream_t stream);

/*
 * y = act((x - mean) * invstd * gamma + beta [+ residual]), act = ReLU when
 * relu != 0; gamma / beta may be null (affine = false), residual may be
 * null. y may alias x or residual.
 */
int rhip_bn_forward(const void *x, int64_t n, int32_t C, const float *mean,
                    const float *invstd, const float *gamma, const float *beta,
                    const void *residual, int32_t relu, void *y, int32_t dtype,
                    hipStream_t stream);

/*
 * Backward of rhip_bn_forward. g = grad_y, masked to y > 0 when relu != 0
 * (y = the forward's output); grad_residual = g; with batch statistics
 * (batch_stats != 0) grad_x = gamma * invstd * (g - mean(g) - xhat *
 * mean(g * xhat)), with running statistics grad_x = gamma * invstd * g;
 * grad_beta = sum g, grad_gamma = sum g * xhat, xhat = (x - mean) * invstd.
 * Any of grad_x, grad_residual, grad_gamma, grad_beta may be null.
 */
int rhip_bn_backward(const void *grad_y, const void *y, const void *x, int64_t n,
                     int32_t C, const float *mean, const float *invstd,
                     const float *gamma, int32_t relu, int32_t batch_stats,
                     void *grad_x, void *grad_residual, float *grad_gamma,
                     float *grad_beta, int32_t dtype, void *workspace,
                     size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RIEMANN_HIP_H */
