// Kernel-map generation for gfx950.
//
// Semantics: CoordinateMapCPU::kernel_map (RiemannEngine/engine/grid/
// lattice_cpu.hpp:606-673): for every output coordinate o and stencil offset
// k, the input row holding o + offset_k (batch column unchanged) is paired
// with o under k. The reference CPU map fills per-offset buckets from many
// threads through fetch_add, so only the *set* of pairs is defined there. The
// dormant reference GPU map sorts triplets by offset with a radix sort
// (engine/grid/lattice_gpu.cuh:438-488).
//
// The map built here serves the output-stationary convolution, so besides
// the pairs it fixes a *processing order* of the output rows (and of the
// input rows for the input gradient): rows are sorted by their neighbour
// mask (the set of offsets with a neighbour), ties kept in locality order.
// Consecutive rows then share their offset sets, so the convolution's
// 16-row MFMA groups rarely multiply a missing neighbour.
//
// Phase 1 (rhip_kmap_count):
//   query    one lane per (output, offset) probes the input table in the
//            output map's locality order -> nbr_sp[k][j];
//   masks    one lane per output row folds its K hits into a sort key;
//   sort     stable radix sort of rows by mask key (bits [0, min(K, 32)));
//   permute  nbr[k][p] = nbr_sp[k][j(p)], out_order[p] = row of p, and a
//            wave-ballot count of hits per (offset, workgroup);
//   scan     exclusive scan of the counts, offset-major -> CSR of pairs.
// Phase 2 (rhip_kmap_fill):
//   emit     ballot + mbcnt compaction of nbr into per-offset pair lists
//            (ordered by offset, then processing position), and the input
//            rows' transposed masks (atomicOr);
//   sort     input rows by transposed mask -> in_order / in_pos;
//   transpose nbr_t[k][in_pos[i]] = output row paired with i under k.
#include <algorithm>

#include "rhip_internal.hpp"

namespace rhip {

constexpr int kMapBlock = 256;
constexpr int kMaskedK = 128; // neighbour masks (and mask order) for K <= 128

__global__ __launch_bounds__(kMapBlock) void kmap_query_kernel(
    TableView t, const int32_t *__restrict__ out_coords,
    const int32_t *__restrict__ spatial, int64_t n_out,
    const int32_t *__restrict__ offsets, int32_t *__restrict__ nbr_sp) {
  const int k = blockIdx.y;
  const int64_t j = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (j >= n_out)
    return;
  const int D = t.ncol - 1;
  const int64_t o = spatial ? spatial[j] : j;
  int32_t c[RHIP_MAX_COLS];
#pragma unroll
  for (int i = 0; i < RHIP_MAX_COLS; ++i)
    c[i] = i < t.ncol ? out_coords[o * t.ncol + i] : 0;
#pragma unroll
  for (int i = 1; i < RHIP_MAX_COLS; ++i)
    if (i < t.ncol) // wrap-around add, as int32 coordinate arithmetic does
      c[i] = static_cast<int32_t>(static_cast<uint32_t>(c[i]) +
                                  static_cast<uint32_t>(offsets[k * D + (i - 1)]));
  nbr_sp[k * n_out + j] = table_find(t, c);
}

// 32-bit sort key of a neighbour mask: the mask itself for K <= 32, else a
// hash (equal masks get equal keys; unequal ones rarely collide, which only
// costs locality, never correctness).
__device__ __forceinline__ uint32_t mask_key32(uint64_t m0, uint64_t m1, int K) {
  if (K <= 32)
    return static_cast<uint32_t>(m0);
  return static_cast<uint32_t>(mix64(m0 ^ mix64(m1 ^ 0x9e3779b97f4a7c15ull)) >> 32);
}

__global__ __launch_bounds__(kMapBlock) void mask_key_kernel(
    const int32_t *__restrict__ nbr_sp, int64_t n, int K,
    uint32_t *__restrict__ keys, int32_t *__restrict__ vals) {
  const int64_t j = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (j >= n)
    return;
  uint64_t m0 = 0, m1 = 0;
  for (int k = 0; k < K; ++k) {
    const uint64_t h = nbr_sp[k * n + j] >= 0 ? 1ull : 0ull;
    if (k < 64)
      m0 |= h << k;
    else
      m1 |= h << (k - 64);
  }
  keys[j] = mask_key32(m0, m1, K);
  vals[j] = static_cast<int32_t>(j);
}

__device__ __forceinline__ int32_t block_hit_base(bool hit, int32_t *wave_counts,
                                                  uint64_t &ballot) {
  ballot = __ballot(hit);
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0)
    wave_counts[w] = __popcll(ballot);
  __syncthreads();
  int32_t before = 0;
  for (int i = 0; i < w; ++i)
    before += wave_counts[i];
  return before;
}

__global__ __launch_bounds__(kMapBlock) void kmap_permute_kernel(
    const int32_t *__restrict__ nbr_sp, const int32_t *__restrict__ jpos,
    const int32_t *__restrict__ spatial, int64_t n_out, int32_t *__restrict__ nbr,
    int32_t *__restrict__ out_order, int32_t *__restrict__ block_counts) {
  __shared__ int32_t wave_counts[kMapBlock / kWave];
  const int k = blockIdx.y;
  const int64_t p = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  bool hit = false;
  if (p < n_out) {
    const int64_t j = jpos ? jpos[p] : p;
    const int32_t v = nbr_sp[k * n_out + j];
    nbr[k * n_out + p] = v;
    hit = v >= 0;
    if (k == 0)
      out_order[p] = spatial ? spatial[j] : static_cast<int32_t>(j);
  }
  uint64_t b;
  block_hit_base(hit, wave_counts, b);
  if (threadIdx.x == kMapBlock - 1) {
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

__global__ __launch_bounds__(kMapBlock) void zero_u64_kernel(unsigned long long *p,
                                                             int64_t n) {
  int64_t i = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (i < n)
    p[i] = 0ull;
}

__global__ __launch_bounds__(kMapBlock) void kmap_emit_kernel(
    const int32_t *__restrict__ nbr, const int32_t *__restrict__ out_order,
    int64_t n_out, const int64_t *__restrict__ block_base,
    int32_t *__restrict__ in_rows, int32_t *__restrict__ out_rows,
    unsigned long long *__restrict__ mask_t) {
  __shared__ int32_t wave_counts[kMapBlock / kWave];
  const int k = blockIdx.y;
  const int64_t p = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  const int32_t v = p < n_out ? nbr[k * n_out + p] : -1;
  const bool hit = v >= 0;
  uint64_t b;
  const int32_t before = block_hit_base(hit, wave_counts, b);
  if (hit) {
    const int64_t q = block_base[static_cast<int64_t>(k) * gridDim.x + blockIdx.x] +
                      before + lanes_below(b);
    in_rows[q] = v;
    out_rows[q] = out_order[p];
    if (mask_t)
      atomicOr(&mask_t[2 * static_cast<int64_t>(v) + (k >> 6)], 1ull << (k & 63));
  }
}

__global__ __launch_bounds__(kMapBlock) void in_key_kernel(
    const unsigned long long *__restrict__ mask_t, const int32_t *__restrict__ spatial,
    int64_t n, int K, uint32_t *__restrict__ keys, int32_t *__restrict__ vals) {
  const int64_t q = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (q >= n)
    return;
  const int64_t i = spatial ? spatial[q] : q;
  keys[q] = mask_key32(mask_t[2 * i], mask_t[2 * i + 1], K);
  vals[q] = static_cast<int32_t>(q);
}

__global__ __launch_bounds__(kMapBlock) void in_order_kernel(
    const int32_t *__restrict__ qpos, const int32_t *__restrict__ spatial, int64_t n,
    int32_t *__restrict__ in_order, int32_t *__restrict__ in_pos) {
  const int64_t q = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (q >= n)
    return;
  const int64_t qs = qpos ? qpos[q] : q;
  const int32_t i = spatial ? spatial[qs] : static_cast<int32_t>(qs);
  in_order[q] = i;
  in_pos[i] = static_cast<int32_t>(q);
}

__global__ __launch_bounds__(kMapBlock) void kmap_transpose_kernel(
    const int32_t *__restrict__ nbr, const int32_t *__restrict__ out_order,
    int64_t n_out, const int32_t *__restrict__ in_pos, int64_t n_in,
    int32_t *__restrict__ nbr_t) {
  const int k = blockIdx.y;
  const int64_t p = blockIdx.x * (int64_t)kMapBlock + threadIdx.x;
  if (p >= n_out)
    return;
  const int32_t v = nbr[k * n_out + p];
  if (v >= 0)
    nbr_t[k * n_in + in_pos[v]] = out_order[p];
}

// Workspace: the per-block counts and their scan persist from phase 1 to
// phase 2; each phase's scratch reuses the same region after them.
struct KmapWs {
  int32_t *block_counts;
  int64_t *block_base;
  int64_t *total;
  // phase 1
  int32_t *nbr_sp;
  uint32_t *keys_a, *keys_b;
  int32_t *vals_a, *vals_b;
  void *sort_tmp;
  size_t sort_bytes;
  // phase 2
  unsigned long long *mask_t;
  uint32_t *tkeys_a, *tkeys_b;
  int32_t *tvals_a, *tvals_b, *in_pos;
  void *tsort_tmp;
  size_t tsort_bytes;
};

static KmapWs carve_kmap(Carve &cv, int64_t n_in, int64_t n_out, int32_t K) {
  const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
  const int64_t mo = std::max<int64_t>(n_out, 1), mi = std::max<int64_t>(n_in, 1);
  KmapWs w{};
  w.block_counts = cv.take<int32_t>(nb * K);
  w.block_base = cv.take<int64_t>(nb * K);
  w.total = cv.take<int64_t>(1);
  const size_t base = cv.used;
  w.nbr_sp = cv.take<int32_t>(mo * K);
  w.keys_a = cv.take<uint32_t>(mo);
  w.keys_b = cv.take<uint32_t>(mo);
  w.vals_a = cv.take<int32_t>(mo);
  w.vals_b = cv.take<int32_t>(mo);
  w.sort_bytes = sort_pairs_u32_bytes(mo);
  w.sort_tmp = cv.take<char>(w.sort_bytes);
  const size_t end1 = cv.used;
  cv.used = base;
  w.mask_t = cv.take<unsigned long long>(2 * mi);
  w.tkeys_a = cv.take<uint32_t>(mi);
  w.tkeys_b = cv.take<uint32_t>(mi);
  w.tvals_a = cv.take<int32_t>(mi);
  w.tvals_b = cv.take<int32_t>(mi);
  w.in_pos = cv.take<int32_t>(mi);
  w.tsort_bytes = sort_pairs_u32_bytes(mi);
  w.tsort_tmp = cv.take<char>(w.tsort_bytes);
  cv.used = std::max(cv.used, end1);
  return w;
}

} // namespace rhip

using namespace rhip;

extern "C" int rhip_kmap_workspace_bytes(int64_t n_in, int64_t n_out, int32_t K,
                                         size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0 && K >= 1, "need n_in, n_out >= 0 and K >= 1");
    Carve cv(nullptr, 0);
    carve_kmap(cv, n_in, n_out, K);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_kmap_count(const rhip_table *in_table, const int32_t *out_coords,
                               const int32_t *out_spatial_order, int64_t n_out,
                               int32_t K, const int32_t *offsets, void *workspace,
                               size_t workspace_bytes, int32_t *nbr, int32_t *out_order,
                               int64_t *kmap_offsets, int64_t *kmap_offsets_host,
                               hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(in_table != nullptr, "in_table is null");
    RHIP_CHECK_ARG(K >= 1 && K <= 65535, "K must be in [1, 65535]");
    RHIP_CHECK_ARG(n_out >= 0 && n_out < INT32_MAX, "bad n_out");
    RHIP_CHECK_ARG(kmap_offsets && kmap_offsets_host && workspace,
                   "kmap_offsets, kmap_offsets_host and workspace are required");
    Carve cv(workspace, workspace_bytes);
    KmapWs w = carve_kmap(cv, in_table->n_unique, n_out, K);
    const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
    if (n_out == 0) {
      hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(nb * K, kMapBlock)),
                         dim3(kMapBlock), 0, stream, w.block_counts, nb * K, 0);
      RHIP_LAUNCH_CHECK();
    } else {
      RHIP_CHECK_ARG(out_coords && offsets && nbr && out_order,
                     "out_coords, offsets, nbr and out_order are required");
      hipLaunchKernelGGL(kmap_query_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream,
                         make_view(*in_table), out_coords, out_spatial_order, n_out,
                         offsets, w.nbr_sp);
      RHIP_LAUNCH_CHECK();
      const int32_t *jpos = nullptr;
      if (K <= kMaskedK && n_out > 1 && in_table->n_unique > 0) {
        hipLaunchKernelGGL(mask_key_kernel, dim3(nb), dim3(kMapBlock), 0, stream,
                           w.nbr_sp, n_out, K, w.keys_a, w.vals_a);
        RHIP_LAUNCH_CHECK();
        sort_pairs_u32(w.sort_tmp, w.sort_bytes, w.keys_a, w.keys_b, w.vals_a, w.vals_b,
                       n_out, std::min<int>(K, 32), stream);
        jpos = w.vals_b;
      }
      hipLaunchKernelGGL(kmap_permute_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream,
                         w.nbr_sp, jpos, out_spatial_order, n_out, nbr, out_order,
                         w.block_counts);
      RHIP_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(scan_counts_kernel<0>, dim3(1), dim3(1024), 0, stream,
                       w.block_counts, nb * K, w.block_base, w.total);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(kmap_offsets_kernel, dim3(ceil_div(K + 1, 256)), dim3(256), 0,
                       stream, w.block_base, w.total, K, nb, kmap_offsets);
    RHIP_LAUNCH_CHECK();
    RHIP_HIP(hipMemcpyAsync(kmap_offsets_host, kmap_offsets, sizeof(int64_t) * (K + 1),
                            hipMemcpyDeviceToHost, stream));
    RHIP_HIP(hipStreamSynchronize(stream));
  });
}

extern "C" int rhip_kmap_fill(const int32_t *nbr, const int32_t *out_order, int64_t n_out,
                              int32_t K, const int32_t *in_spatial_order, int64_t n_in,
                              void *workspace, size_t workspace_bytes, int32_t *in_rows,
                              int32_t *out_rows, int32_t *nbr_t, int32_t *in_order,
                              hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(K >= 1 && K <= 65535, "K must be in [1, 65535]");
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    RHIP_CHECK_ARG(n_in >= 0 && n_in < INT32_MAX && n_out >= 0 && n_out < INT32_MAX,
                   "bad sizes");
    Carve cv(workspace, workspace_bytes);
    KmapWs w = carve_kmap(cv, n_in, n_out, K);
    const int64_t nb = std::max<int64_t>(1, ceil_div(n_out, kMapBlock));
    const bool want_t = nbr_t != nullptr && n_in > 0;
    RHIP_CHECK_ARG(!want_t || in_order != nullptr, "in_order is required with nbr_t");
    const bool masks = want_t && K <= kMaskedK && n_in > 1;
    if (masks) {
      hipLaunchKernelGGL(zero_u64_kernel, dim3(ceil_div(2 * n_in, kMapBlock)),
                         dim3(kMapBlock), 0, stream, w.mask_t, 2 * n_in);
      RHIP_LAUNCH_CHECK();
    }
    if (n_out > 0) {
      RHIP_CHECK_ARG(nbr && out_order, "nbr and out_order are required");
      hipLaunchKernelGGL(kmap_emit_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream, nbr,
                         out_order, n_out, w.block_base, in_rows, out_rows,
                         masks ? w.mask_t : nullptr);
      RHIP_LAUNCH_CHECK();
    }
    if (!want_t)
      return;
    const int64_t nbi = ceil_div(n_in, kMapBlock);
    const int32_t *qpos = nullptr;
    if (masks) {
      hipLaunchKernelGGL(in_key_kernel, dim3(nbi), dim3(kMapBlock), 0, stream, w.mask_t,
                         in_spatial_order, n_in, K, w.tkeys_a, w.tvals_a);
      RHIP_LAUNCH_CHECK();
      sort_pairs_u32(w.tsort_tmp, w.tsort_bytes, w.tkeys_a, w.tkeys_b, w.tvals_a, w.tvals_b,
                     n_in, std::min<int>(K, 32), stream);
      qpos = w.tvals_b;
    }
    hipLaunchKernelGGL(in_order_kernel, dim3(nbi), dim3(kMapBlock), 0, stream, qpos,
                       in_spatial_order, n_in, in_order, w.in_pos);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(n_in * K, kMapBlock)),
                       dim3(kMapBlock), 0, stream, nbr_t, n_in * K, -1);
    RHIP_LAUNCH_CHECK();
    if (n_out > 0) {
      hipLaunchKernelGGL(kmap_transpose_kernel, dim3(nb, K), dim3(kMapBlock), 0, stream,
                         nbr, out_order, n_out, w.in_pos, n_in, nbr_t);
      RHIP_LAUNCH_CHECK();
    }
  });
}
