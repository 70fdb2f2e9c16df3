/*
 * oracle.c — CPU restatement of RiemannEngine's sparse-convolution hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the parity tests (and
 * bench.py's cpu_baseline leg) compare the HIP path against; nothing in the
 * shipped path links, loads or calls it.
 *
 * Every function cites the reference code it restates (paths relative to
 * the reference checkout, RiemannEngine/...). Pinning of each function
 * (see tests/test_oracle.py):
 *   oracle_insert_and_map   — pinned: brute force (numpy.unique first index)
 *                             and the inverse/mapping invariants.
 *   oracle_region_offsets   — pinned: closed forms for 3^D, 2^D cubes and
 *                             the 2D+1 cross; brute enumeration of CUSTOM.
 *   oracle_kernel_map       — pinned: brute-force sorted join of coordinate
 *                             sets and the dense active-site indicator.
 *   oracle_stride           — pinned: closed form floor(x/s)*s + np.unique.
 *   oracle_stride_region    — pinned: brute-force set of c + offset, the
 *                             closed count of 2^D children, and the
 *                             reference's own stride_region (oracle/_ref).
 *   oracle_conv_forward /
 *   oracle_conv_backward    — pinned: the three known-answer tests of
 *                             tests/convolution/test_cpu_convolution.cpp:15-61
 *                             and dense torch conv3d (a textbook routine) on
 *                             voxelised inputs, plus fp64 brute force.
 *   oracle_stride_map       — pinned: brute-force floor division per row and
 *                             the reference's own pooling (oracle/_ref).
 *   oracle_pool_forward /
 *   oracle_pool_backward    — pinned: the known answers of
 *                             tests/engine/test_layers.cpp:80-115, torch's
 *                             sum/mean/amax and their autograd (ties split
 *                             evenly) on the same groups, closed forms (sum of
 *                             ones = group sizes) and the reference (_ref).
 *   oracle_global_pool_*    — pinned: tests/engine/test_layers.cpp:58-78,
 *                             torch per-batch reductions + autograd, and the
 *                             reference (_ref).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ row hashing */

typedef struct {
  int64_t cap;    /* power of two */
  int64_t *slot;  /* unique id or -1 */
  const int32_t *rows; /* unique rows referenced by slot ids */
  int ncol;
} otab;

static uint64_t row_hash(const int32_t *r, int ncol) {
  /* FNV-1a over the row's 32-bit words (any hash works: the oracle only
   * needs set semantics, the reference uses murmur3, hashing.hpp:182-276). */
  uint64_t h = 1469598103934665603ull;
  for (int i = 0; i < ncol; ++i) {
    uint32_t v = (uint32_t)r[i];
    for (int b = 0; b < 4; ++b) {
      h ^= (v >> (8 * b)) & 0xffu;
      h *= 1099511628211ull;
    }
  }
  return h;
}

static int otab_init(otab *t, int64_t n, const int32_t *rows, int ncol) {
  t->cap = 16;
  while (t->cap < 2 * n + 1)
    t->cap <<= 1;
  t->slot = (int64_t *)malloc(sizeof(int64_t) * t->cap);
  if (!t->slot)
    return -1;
  for (int64_t i = 0; i < t->cap; ++i)
    t->slot[i] = -1;
  t->rows = rows;
  t->ncol = ncol;
  return 0;
}

static int64_t otab_find(const otab *t, const int32_t *r) {
  uint64_t h = row_hash(r, t->ncol) & (uint64_t)(t->cap - 1);
  for (;;) {
    int64_t u = t->slot[h];
    if (u < 0)
      return -1;
    if (memcmp(t->rows + u * t->ncol, r, sizeof(int32_t) * t->ncol) == 0)
      return u;
    h = (h + 1) & (uint64_t)(t->cap - 1);
  }
}

static void otab_put(otab *t, const int32_t *r, int64_t u) {
  uint64_t h = row_hash(r, t->ncol) & (uint64_t)(t->cap - 1);
  while (t->slot[h] >= 0)
    h = (h + 1) & (uint64_t)(t->cap - 1);
  t->slot[h] = u;
}

/*
 * Sequential dedup, first occurrence wins: CoordinateMapCPU::insert_and_map
 * <remap=true> (engine/grid/lattice_cpu.hpp:419-444) with the CPU functor
 * (engine/grid/space.cpp:17-58). unique_out gets the unique rows in
 * first-occurrence order, mapping[u] the first input row, inverse[r] the
 * unique id of row r. Returns n_unique (or -1 on allocation failure).
 */
int64_t oracle_insert_and_map(const int32_t *coords, int64_t n, int ncol,
                              int32_t *unique_out, int64_t *mapping,
                              int64_t *inverse) {
  otab t;
  if (otab_init(&t, n, unique_out, ncol))
    return -1;
  int64_t nu = 0;
  for (int64_t r = 0; r < n; ++r) {
    const int32_t *row = coords + r * ncol;
    int64_t u = otab_find(&t, row);
    if (u < 0) {
      memcpy(unique_out + nu * ncol, row, sizeof(int32_t) * ncol);
      otab_put(&t, row, nu);
      mapping[nu] = r;
      u = nu++;
    }
    if (inverse)
      inverse[r] = u;
  }
  free(t.slot);
  return nu;
}

/*
 * Stencil offsets, scaled by dilation * tensor_stride per axis:
 * kernel_region::coordinate_at (engine/grid/stencil.hpp:223-278) and
 * set_volume (:281-300). region: 0 HYPER_CUBE, 1 HYPER_CROSS, 2 CUSTOM
 * (custom [n_custom, D] lattice offsets). Writes out[K * D]; returns K.
 */
int oracle_region_offsets(int region, int D, const int32_t *kernel_size,
                          const int32_t *dilation, const int32_t *tensor_stride,
                          const int32_t *custom, int n_custom, int32_t *out) {
  int K = 0;
  if (region == 0) {
    K = 1;
    for (int i = 0; i < D; ++i)
      K *= kernel_size[i];
    for (int k = 0; k < K; ++k) {
      int idx = k;
      for (int i = 0; i < D; ++i) {
        int ks = kernel_size[i], c = idx % ks;
        idx /= ks;
        int step = dilation[i] * tensor_stride[i];
        out[k * D + i] = (ks % 2 == 0) ? c * step : (c - ks / 2) * step;
      }
    }
  } else if (region == 1) {
    K = 1;
    for (int i = 0; i < D; ++i)
      K += kernel_size[i] - 1;
    for (int k = 0; k < K; ++k) {
      for (int i = 0; i < D; ++i)
        out[k * D + i] = 0;
      if (k == 0)
        continue;
      int ind = k - 1, axis = 0;
      while (axis < D && ind >= kernel_size[axis] - 1) {
        ind -= kernel_size[axis] - 1;
        ++axis;
      }
      int r = (kernel_size[axis] - 1) / 2;
      int off = ind < r ? ind + 1 : ind - 2 * r;
      out[k * D + axis] = off * dilation[axis] * tensor_stride[axis];
    }
  } else {
    K = n_custom;
    for (int k = 0; k < K; ++k)
      for (int i = 0; i < D; ++i)
        out[k * D + i] = custom[k * D + i] * tensor_stride[i] * dilation[i];
  }
  return K;
}

/*
 * The live kernel map: CoordinateMapCPU::kernel_map
 * (engine/grid/lattice_cpu.hpp:606-673). For each output row o and offset k,
 * in = find(out[o] + offset_k) (batch column copied); hits are appended to
 * bucket k. The reference fills buckets from several threads, so only the
 * set of pairs is defined; here o runs in row order, so each bucket comes
 * out sorted by output row. counts[k] gets the bucket sizes; pairs are
 * written offset-major into in_rows/out_rows (capacity n_out * K).
 * Returns the total number of pairs.
 */
int64_t oracle_kernel_map(const int32_t *in_coords, int64_t n_in,
                          const int32_t *out_coords, int64_t n_out, int ncol,
                          const int32_t *offsets, int K, int32_t *in_rows,
                          int32_t *out_rows, int64_t *counts) {
  const int D = ncol - 1;
  otab t;
  if (otab_init(&t, n_in, in_coords, ncol))
    return -1;
  for (int64_t i = 0; i < n_in; ++i)
    otab_put(&t, in_coords + i * ncol, i);
  int32_t q[16];
  int64_t p = 0;
  for (int k = 0; k < K; ++k) {
    counts[k] = 0;
    for (int64_t o = 0; o < n_out; ++o) {
      const int32_t *src = out_coords + o * ncol;
      q[0] = src[0];
      for (int i = 0; i < D; ++i)
        q[i + 1] = src[i + 1] + offsets[k * D + i];
      int64_t u = otab_find(&t, q);
      if (u >= 0) {
        in_rows[p] = (int32_t)u;
        out_rows[p] = (int32_t)o;
        ++p;
        ++counts[k];
      }
    }
  }
  free(t.slot);
  return p;
}

/*
 * Strided output coordinates: CoordinateMapCPU::stride
 * (engine/grid/lattice_cpu.hpp:475-493) with detail::stride_coordinate
 * (engine/grid/stencil.hpp:35-44): (b, floor((float)x / s) * s) per row,
 * deduplicated. The reference walks its robin-hood table, so its row order
 * is implementation-defined; here rows follow first occurrence in input
 * order. out needs room for n rows; returns the unique count.
 */
int64_t oracle_stride(const int32_t *coords, int64_t n, int ncol,
                      const int32_t *stride, int32_t *out) {
  int32_t *tmp = (int32_t *)malloc(sizeof(int32_t) * (n > 0 ? n : 1) * ncol);
  int64_t *mapping = (int64_t *)malloc(sizeof(int64_t) * (n > 0 ? n : 1));
  for (int64_t r = 0; r < n; ++r) {
    tmp[r * ncol] = coords[r * ncol];
    for (int i = 1; i < ncol; ++i) {
      int s = stride[i - 1];
      tmp[r * ncol + i] = (int32_t)(floorf((float)coords[r * ncol + i] / (float)s) * (float)s);
    }
  }
  int64_t nu = oracle_insert_and_map(tmp, n, ncol, out, mapping, NULL);
  free(tmp);
  free(mapping);
  return nu;
}

/*
 * Generative expansion, the transposed branch of
 * CoordinateMapCPU::stride_region (engine/grid/lattice_cpu.hpp:499-534): every
 * input row c emits c + offsets[k] for each of the K offsets (the kernel
 * region at the output tensor stride, batch column kept); the generated map
 * is their unique set. The reference walks its robin-hood table, so its row
 * order is implementation-defined; here rows follow first occurrence over
 * (input row, offset). out needs room for n * K rows; returns the unique
 * count.
 */
int64_t oracle_stride_region(const int32_t *coords, int64_t n, int ncol,
                             const int32_t *offsets, int K, int32_t *out) {
  const int64_t m = n * K;
  int32_t *tmp = (int32_t *)malloc(sizeof(int32_t) * (m > 0 ? m : 1) * ncol);
  int64_t *mapping = (int64_t *)malloc(sizeof(int64_t) * (m > 0 ? m : 1));
  for (int64_t r = 0; r < n; ++r)
    for (int k = 0; k < K; ++k) {
      int32_t *o = tmp + (r * K + k) * ncol;
      o[0] = coords[r * ncol];
      for (int i = 1; i < ncol; ++i)
        o[i] = (int32_t)((uint32_t)coords[r * ncol + i] + (uint32_t)offsets[k * (ncol - 1) + i - 1]);
    }
  int64_t nu = oracle_insert_and_map(tmp, m, ncol, out, mapping, NULL);
  free(tmp);
  free(mapping);
  return nu;
}

/*
 * Forward: sparse_convolution_forward_cpu_kernel
 * (engine/ops/convolution_cpu.hpp:28-52) — the scalar form of
 * evaluate_sparse_convolution's index_select/matmul/index_add_ loop
 * (engine/nn/conv.cpp:47-64). Accumulates in double; y [n_out, cout] is
 * overwritten (zero-initialised as in conv.cpp:46). Pairs are given as a
 * CSR over offsets (kofs[K+1]); weight is [K, cin, cout].
 */
void oracle_conv_forward(const float *x, int64_t n_in, int cin,
                         const float *weight, int K, int cout,
                         const int64_t *kofs, const int32_t *in_rows,
                         const int32_t *out_rows, int64_t n_out, float *y) {
  double *acc = (double *)calloc((size_t)(n_out > 0 ? n_out : 1) * cout, sizeof(double));
  for (int k = 0; k < K; ++k) {
    const float *w = weight + (int64_t)k * cin * cout;
    for (int64_t p = kofs[k]; p < kofs[k + 1]; ++p) {
      int64_t i = in_rows[p], o = out_rows[p];
      if (i < 0 || i >= n_in || o < 0 || o >= n_out)
        continue; /* out-of-range rows are skipped, convolution_cpu.hpp:41-43 */
      const float *xr = x + i * cin;
      double *yr = acc + o * cout;
      for (int c = 0; c < cin; ++c) {
        double xv = xr[c];
        const float *wr = w + (int64_t)c * cout;
        for (int n = 0; n < cout; ++n)
          yr[n] += xv * wr[n];
      }
    }
  }
  for (int64_t e = 0; e < n_out * cout; ++e)
    y[e] = (float)acc[e];
  free(acc);
}

/*
 * Backward: sparse_convolution_backward_cpu_kernel
 * (engine/ops/convolution_cpu.hpp:55-89): dX[in] += dY[out] W_k^T and
 * dW_k += X[in]^T dY[out]; both outputs are overwritten. Double accumulation.
 */
void oracle_conv_backward(const float *x, int64_t n_in, int cin,
                          const float *grad_y, int64_t n_out, int cout,
                          const float *weight, int K, const int64_t *kofs,
                          const int32_t *in_rows, const int32_t *out_rows,
                          float *grad_x, float *grad_w) {
  double *gx = (double *)calloc((size_t)(n_in > 0 ? n_in : 1) * cin, sizeof(double));
  double *gw = (double *)calloc((size_t)K * cin * cout, sizeof(double));
  for (int k = 0; k < K; ++k) {
    const float *w = weight + (int64_t)k * cin * cout;
    double *gwk = gw + (int64_t)k * cin * cout;
    for (int64_t p = kofs[k]; p < kofs[k + 1]; ++p) {
      int64_t i = in_rows[p], o = out_rows[p];
      if (i < 0 || i >= n_in || o < 0 || o >= n_out)
        continue;
      const float *xr = x + i * cin;
      const float *gr = grad_y + o * cout;
      double *gxr = gx + i * cin;
      for (int c = 0; c < cin; ++c) {
        double s = 0.0;
        const float *wr = w + (int64_t)c * cout;
        double *gwr = gwk + (int64_t)c * cout;
        double xv = xr[c];
        for (int n = 0; n < cout; ++n) {
          s += (double)gr[n] * wr[n];
          gwr[n] += xv * gr[n];
        }
        gxr[c] += s;
      }
    }
  }
  for (int64_t e = 0; e < n_in * cin; ++e)
    grad_x[e] = (float)gx[e];
  for (int64_t e = 0; e < (int64_t)K * cin * cout; ++e)
    grad_w[e] = (float)gw[e];
  free(gx);
  free(gw);
}

/* ---------------------------------------------------------------- pooling */

/*
 * Stride map: CoordinateMapCPU::stride_map (engine/grid/lattice_cpu.hpp:675-710)
 * with detail::stride_coordinate (engine/grid/stencil.hpp:46-53): input row i
 * maps to the row of (b, floor((float)x / s) * s) in out_coords. in_to_out[i]
 * is that row or -1; returns the number of rows with none (the reference
 * ASSERTs there are none).
 */
int64_t oracle_stride_map(const int32_t *in_coords, int64_t n_in, int ncol,
                          const int32_t *out_coords, int64_t n_out,
                          const int32_t *stride, int32_t *in_to_out) {
  otab t;
  int32_t *tmp = (int32_t *)malloc(sizeof(int32_t) * ncol);
  int64_t miss = 0;
  otab_init(&t, n_out, out_coords, ncol);
  for (int64_t u = 0; u < n_out; ++u)
    if (otab_find(&t, out_coords + u * ncol) < 0)
      otab_put(&t, out_coords + u * ncol, u);
  for (int64_t r = 0; r < n_in; ++r) {
    tmp[0] = in_coords[r * ncol];
    for (int i = 1; i < ncol; ++i) {
      int s = stride[i - 1];
      tmp[i] = (int32_t)(floorf((float)in_coords[r * ncol + i] / (float)s) * (float)s);
    }
    int64_t o = otab_find(&t, tmp);
    in_to_out[r] = (int32_t)o;
    miss += o < 0;
  }
  free(tmp);
  free(t.slot);
  return miss;
}

/* mode: 0 sum, 1 average, 2 max (PoolingMode LOCAL_{SUM,AVG,MAX}_POOLING),
 * 3 max as zeros.scatter_reduce("amax", include_self=False): forward as 2,
 * backward counting the excluded zero as one more tie where the max is 0
 * (LibTorch's scatter_reduce backward; SparseTensor MAX_POOL quantization,
 * engine/tensor/sparse_tensor.cpp:474-479). */

/*
 * Local pooling: evaluate_pooling (engine/nn/pooling.cpp:80-150). The pairs
 * (in_rows[p], out_rows[p]) are gathered per output in pair order
 * (inputs_by_output), each group reduced by values.sum(0) / mean(0) /
 * amax({0}) (amax propagates NaN), an empty group gives zeros. Sums in double.
 * counts [n_out] (may be NULL) receives the group sizes.
 */
void oracle_pool_forward(const float *x, int64_t n_in, int C, const int32_t *in_rows,
                         const int32_t *out_rows, int64_t P, int64_t n_out, int mode,
                         float *y, int32_t *counts) {
  double *acc = (double *)malloc(sizeof(double) * (size_t)(n_out > 0 ? n_out : 1) * C);
  int64_t *cnt = (int64_t *)calloc((size_t)(n_out > 0 ? n_out : 1), sizeof(int64_t));
  for (int64_t e = 0; e < n_out * C; ++e)
    acc[e] = mode >= 2 ? -INFINITY : 0.0;
  for (int64_t p = 0; p < P; ++p) {
    int64_t i = in_rows[p], o = out_rows[p];
    if (i < 0 || i >= n_in || o < 0 || o >= n_out)
      continue;
    ++cnt[o];
    for (int c = 0; c < C; ++c) {
      double v = x[i * C + c];
      double *a = acc + o * C + c;
      if (mode >= 2)
        *a = (v > *a || isnan(v)) && !isnan(*a) ? v : *a;
      else
        *a += v;
    }
  }
  for (int64_t o = 0; o < n_out; ++o) {
    for (int c = 0; c < C; ++c) {
      double a = acc[o * C + c];
      y[o * C + c] = cnt[o] == 0 ? 0.f : (float)(mode == 1 ? a / (double)cnt[o] : a);
    }
    if (counts)
      counts[o] = (int32_t)cnt[o];
  }
  free(acc);
  free(cnt);
}

/*
 * Local pooling backward: the gradient LibTorch's autograd gives
 * evaluate_pooling's graph (pooling.cpp:120-140): sum passes grad_y[o] to
 * every pooled row, mean grad_y[o] / n, amax grad_y[o] / t to the t rows
 * equal to y[o] (per channel) and 0 to the rest. Accumulates in double over
 * the pairs; grad_x [n_in, C] is overwritten.
 */
void oracle_pool_backward(const float *x, const float *y, const float *grad_y, int64_t n_in,
                          int64_t n_out, int C, const int32_t *in_rows, const int32_t *out_rows,
                          int64_t P, int mode, float *grad_x) {
  double *gx = (double *)calloc((size_t)(n_in > 0 ? n_in : 1) * C, sizeof(double));
  int64_t *cnt = (int64_t *)calloc((size_t)(n_out > 0 ? n_out : 1), sizeof(int64_t));
  int64_t *ties = (int64_t *)calloc((size_t)(n_out > 0 ? n_out : 1) * C, sizeof(int64_t));
  for (int64_t p = 0; p < P; ++p) {
    int64_t i = in_rows[p], o = out_rows[p];
    if (i < 0 || i >= n_in || o < 0 || o >= n_out)
      continue;
    ++cnt[o];
    for (int c = 0; c < C; ++c)
      ties[o * C + c] += x[i * C + c] == y[o * C + c];
  }
  if (mode == 3)
    for (int64_t e = 0; e < n_out * C; ++e)
      ties[e] += y[e] == 0.0f;
  for (int64_t p = 0; p < P; ++p) {
    int64_t i = in_rows[p], o = out_rows[p];
    if (i < 0 || i >= n_in || o < 0 || o >= n_out)
      continue;
    for (int c = 0; c < C; ++c) {
      double g = grad_y[o * C + c];
      if (mode == 1)
        g /= (double)cnt[o];
      else if (mode >= 2)
        g = x[i * C + c] == y[o * C + c] ? g / (double)ties[o * C + c] : 0.0;
      gx[i * C + c] += g;
    }
  }
  for (int64_t e = 0; e < n_in * C; ++e)
    grad_x[e] = (float)gx[e];
  free(gx);
  free(cnt);
  free(ties);
}

/*
 * Global pooling: RiemannGlobalPoolingImpl::forward (engine/nn/pooling.cpp:
 * 203-260): B = max batch index + 1 (0 for no rows); output row b reduces the
 * rows whose batch index is b (sum / mean / amax; zeros for an empty batch).
 * y needs [min(B, max_b), C]; returns B.
 */
int64_t oracle_global_pool_forward(const float *x, const int32_t *coords, int64_t n, int ncol,
                                   int C, int mode, int64_t max_b, float *y) {
  int64_t B = 0;
  for (int64_t r = 0; r < n; ++r)
    if ((int64_t)coords[r * ncol] + 1 > B)
      B = (int64_t)coords[r * ncol] + 1;
  if (B > max_b)
    return B;
  int32_t *in_rows = (int32_t *)malloc(sizeof(int32_t) * (n > 0 ? n : 1));
  int32_t *out_rows = (int32_t *)malloc(sizeof(int32_t) * (n > 0 ? n : 1));
  int64_t P = 0;
  for (int64_t r = 0; r < n; ++r)
    if (coords[r * ncol] >= 0) {
      in_rows[P] = (int32_t)r;
      out_rows[P++] = coords[r * ncol];
    }
  oracle_pool_forward(x, n, C, in_rows, out_rows, P, B, mode, y, NULL);
  free(in_rows);
  free(out_rows);
  return B;
}

/* Backward of the above (autograd of the per-batch index_select + reduce). */
void oracle_global_pool_backward(const float *x, const float *y, const float *grad_y,
                                 const int32_t *coords, int64_t n, int ncol, int C, int64_t B,
                                 int mode, float *grad_x) {
  int32_t *in_rows = (int32_t *)malloc(sizeof(int32_t) * (n > 0 ? n : 1));
  int32_t *out_rows = (int32_t *)malloc(sizeof(int32_t) * (n > 0 ? n : 1));
  int64_t P = 0;
  for (int64_t r = 0; r < n; ++r)
    if (coords[r * ncol] >= 0 && coords[r * ncol] < B) {
      in_rows[P] = (int32_t)r;
      out_rows[P++] = coords[r * ncol];
    }
  oracle_pool_backward(x, y, grad_y, n, B, C, in_rows, out_rows, P, mode, grad_x);
  free(in_rows);
  free(out_rows);
}
