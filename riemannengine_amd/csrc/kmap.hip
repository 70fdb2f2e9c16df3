// Kernel-map generation for gfx950.
//
// Semantics: CoordinateMapCPU::kernel_map (RiemannEngine/engine/grid/
// lattice_cpu.hpp:606-673): for every output coordinate o and stencil offset
// k the input row holding o + offset_k (batch column unchanged) is paired
// with o under k. The reference CPU map fills per-offset buckets from many
// threads through fetch_add, so only the *set* of pairs is defined there; the
// dormant reference GPU map sorts triplets by offset with a radix sort
// (engine/grid/lattice_gpu.cuh:438-488).
//
// Here the map is produced in two passes without any sort:
//   1. query: one lane per (output position, offset) probes the input table
//      and writes a dense neighbour table nbr[k][j] (j = output position in
//      the output map's processing order); a wave ballot counts hits per
//      (offset, workgroup);
//   2. after an exclusive scan of those counts (offset-major), each
//      workgroup re-reads its slice of nbr and compacts the hits with a
//      ballot + mbcnt prefix, so pairs come out ordered by offset and then by
//      output position, deterministically.
// The dense tables (nbr and its transpose over the input map) drive the
// output-stationary convolution kernels; the pair lists drive dW.
#include <algorithm>

#include "rhip_internal.hpp"

namespace rhip {

constexpr int kMapBlock = 256;

__global__ __launch_bounds__(kMapBlock) void kmap_query_kernel(
    TableView t, const int32_t *__restrict__ out_coords,
    const int32_t *__restrict__ out_order, int64_t n_out,
    const int32_t *__restrict__ offsets, int32_t *__restrict__ nbr,
    int32_t *__restrict__ block_counts) {
  __shared__ int32_t wave_counts[kMapBlock / kWave];
  const int k = blockIdx.y;
  const int64_t j = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  const int D = t.ncol - 1;
  bool hit = false;
  if (j < n_out) {
    const int64_t o = out_order ? out_order[j] : j;
    int32_t c[RHIP_MAX_COLS];
#pragma unroll
    for (int i = 0; i < RHIP_MAX_COLS; ++i)
      c[i] = i < t.ncol ? out_coords[o * t.ncol + i] : 0;
#pragma unroll
    for (int i = 1; i < RHIP_MAX_COLS; ++i)
      if (i < t.ncol)
        c[i] += offsets[k * D + (i - 1)];
    const int32_t idx = table_find(t, c);
    nbr[k * n_out + j] = idx;
    hit = idx >= 0;
  }
  const uint64_t b = __ballot(hit);
  if (lane_id() == 0)
    wave_counts[threadIdx.x / kWave] = __popcll(b);
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t s = 0;
    for (int w = 0; w < kMapBlock / kWave; ++w)
      s += wave_counts[w];
    block_counts[static_cast<int64_t>(k) * gridDim.x + blockIdx.x] = s;
  }
}

__global__ void kmap_offsets_kernel(const int64_t *block_base,
                                    const int64_t *total, int K, int64_t nb,
                                    int64_t *kmap_offsets) {
  int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k < K)
    kmap_offsets[k] = block_base[static_cast<int64_t>(k) * nb];
  if (k == K)
    kmap_offsets[K] = *total;
}

__global__ __launch_bounds__(kMapBlock) void fill_i32_kernel(int32_t *p,
                                                             int64_t n,
                                                             int32_t v) {
  int64_t i = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (i < n)
    p[i] = v;
}

__global__ __launch_bounds__(kMapBlock) void kmap_emit_kernel(
    const int32_t *__restrict__ nbr, const int32_t *__restrict__ out_order,
    int64_t n_out, const int64_t *__restrict__ block_base,
    int32_t *__restrict__ in_rows, int32_t *__restrict__ out_rows,
    const int32_t *__restrict__ in_pos, int64_t n_in,
    int32_t *__restrict__ nbr_t) {
  __shared__ int32_t wave_counts[kMapBlock / kWave];
  const int k = blockIdx.y;
  const int64_t j = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  const int32_t v = j < n_out ? nbr[k * n_out + j] : -1;
  const bool hit = v >= 0;
  const uint64_t b = __ballot(hit);
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0)
    wave_counts[w] = __popcll(b);
  __syncthreads();
  int32_t before = 0;
  for (int i = 0; i < w; ++i)
    before += wave_counts[i];
  if (hit) {
    const int64_t p = block_base[static_cast<int64_t>(k) * gridDim.x + blockIdx.x] +
                      before + lanes_below(b);
    const int32_t o = out_order ? out_order[j] : static_cast<int32_t>(j);
    in_rows[p] = v;
    out_rows[p] = o;
    if (nbr_t) {
      const int64_t q = in_pos ? in_pos[v] : v;
      nbr_t[k * n_in + q] = o;
    }
  }
}

struct KmapWs {
  int32_t *block_counts;
  int64_t *block_base;
  int64_t *total;
};

static KmapWs carve_kmap(Carve &cv, int64_t n_out, int32_t K) {
  const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
  KmapWs w;
  w.block_counts = cv.take<int32_t>(nb * K);
  w.block_base = cv.take<int64_t>(nb * K);
  w.total = cv.take<int64_t>(1);
  return w;
}

} // namespace rhip

using namespace rhip;

extern "C" int rhip_kmap_workspace_bytes(int64_t n_out, int32_t K,
                                         size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n_out >= 0 && K >= 1, "need n_out >= 0 and K >= 1");
    Carve cv(nullptr, 0);
    carve_kmap(cv, n_out, K);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_kmap_count(const rhip_table *in_table,
                               const int32_t *out_coords,
                               const int32_t *out_order, int64_t n_out,
                               int32_t K, const int32_t *offsets, int32_t *nbr,
                               void *workspace, size_t workspace_bytes,
                               int64_t *kmap_offsets,
                               int64_t *kmap_offsets_host, hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(in_table != nullptr, "in_table is null");
    RHIP_CHECK_ARG(K >= 1 && K <= 65535, "K must be in [1, 65535]");
    RHIP_CHECK_ARG(n_out >= 0 && n_out < INT32_MAX, "bad n_out");
    RHIP_CHECK_ARG(kmap_offsets && kmap_offsets_host && workspace,
                   "kmap_offsets, kmap_offsets_host and workspace are required");
    Carve cv(workspace, workspace_bytes);
    KmapWs w = carve_kmap(cv, n_out, K);
    const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
    if (n_out == 0 || in_table->n_unique == 0) {
      // Empty map (space_impl.hpp:600-606 returns an empty map when either
      // side is empty); nbr is still well-defined: all -1.
      if (n_out > 0) {
        RHIP_CHECK_ARG(nbr != nullptr, "nbr is null");
        hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(n_out * K, kMapBlock)),
                           dim3(kMapBlock), 0, stream, nbr, n_out * K, -1);
        RHIP_LAUNCH_CHECK();
      }
      hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(nb * K, kMapBlock)),
                         dim3(kMapBlock), 0, stream, w.block_counts, nb * K, 0);
      RHIP_LAUNCH_CHECK();
      hipLaunchKernelGGL(scan_counts_kernel<0>, dim3(1), dim3(1024), 0, stream,
                         w.block_counts, nb * K, w.block_base, w.total);
      RHIP_LAUNCH_CHECK();
    } else {
      RHIP_CHECK_ARG(out_coords && offsets && nbr,
                     "out_coords, offsets and nbr are required");
      hipLaunchKernelGGL(kmap_query_kernel, dim3(nb, K), dim3(kMapBlock), 0,
                         stream, make_view(*in_table), out_coords, out_order,
                         n_out, offsets, nbr, w.block_counts);
      RHIP_LAUNCH_CHECK();
      hipLaunchKernelGGL(scan_counts_kernel<0>, dim3(1), dim3(1024), 0, stream,
                         w.block_counts, nb * K, w.block_base, w.total);
      RHIP_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(kmap_offsets_kernel, dim3(ceil_div(K + 1, 256)),
                       dim3(256), 0, stream, w.block_base, w.total, K, nb,
                       kmap_offsets);
    RHIP_LAUNCH_CHECK();
    RHIP_HIP(hipMemcpyAsync(kmap_offsets_host, kmap_offsets,
                            sizeof(int64_t) * (K + 1), hipMemcpyDeviceToHost,
                            stream));
    RHIP_HIP(hipStreamSynchronize(stream));
  });
}

extern "C" int rhip_kmap_fill(const int32_t *nbr, const int32_t *out_order,
                              int64_t n_out, int32_t K, const void *workspace,
                              size_t workspace_bytes,
                              const int64_t *kmap_offsets, int32_t *in_rows,
                              int32_t *out_rows, const int32_t *in_pos,
                              int64_t n_in, int32_t *nbr_t,
                              hipStream_t stream) {
  return guarded([&] {
    (void)kmap_offsets;
    RHIP_CHECK_ARG(K >= 1 && K <= 65535, "K must be in [1, 65535]");
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "bad sizes");
    Carve cv(const_cast<void *>(workspace), workspace_bytes);
    KmapWs w = carve_kmap(cv, n_out, K);
    const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
    if (nbr_t && n_in > 0) {
      hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(n_in * K, kMapBlock)),
                         dim3(kMapBlock), 0, stream, nbr_t, n_in * K, -1);
      RHIP_LAUNCH_CHECK();
    }
    if (n_out == 0)
      return;
    RHIP_CHECK_ARG(nbr != nullptr, "nbr is null");
    hipLaunchKernelGGL(kmap_emit_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream,
                       nbr, out_order, n_out, w.block_base, in_rows, out_rows,
                       in_pos, n_in, nbr_t);
    RHIP_LAUNCH_CHECK();
  });
}
