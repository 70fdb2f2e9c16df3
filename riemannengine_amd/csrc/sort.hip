// Stable device radix sorts of (key, int32 value) pairs, used by the hash
// table (locality order), the kernel map (neighbour-mask order) and pooling
// (grouping rows by output). Least-significant-digit first with 8- or 9-bit
// digits: the fewest passes the key bits allow, then the narrowest digit for
// that many passes (26 bits: 3 passes of 9; 22 bits: 3 of 8). Wider digits
// cost more than they save: the tile scan runs one workgroup per digit, and
// on MI355X (410k keys) an 11-bit pass takes about 42 us against 21 for an
// 8-bit one. Three kernels per pass:
//
//   radix_hist_kernel     one wave per tile of 1024 keys: the tile's digit
//                         histogram, written tile-major [tiles][256];
//   radix_tile_scan_kernel one workgroup per digit: where the digit's run
//                         of each tile starts among the digit's keys, and
//                         the digit's total (the scatter adds the totals of
//                         the smaller digits);
//   radix_scatter_kernel  the same tiles again: each key's rank among the
//                         tile's keys with its digit, from wave ballots, in
//                         key order, so equal digits keep their order.
//
// A tile is processed in 16 rounds of 64 consecutive keys; within a round,
// 8 ballots find the lanes that share a digit (their rank is the count of
// such lanes below), and an LDS counter per digit carries the run across
// rounds. Every buffer the sort needs is carved from the caller's scratch;
// nothing is allocated or memset.
#include "rhip_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace rhip {
namespace {

constexpr int kMaxRadixBits = 9;
constexpr int kSortItems = 16;
constexpr int kSortTile = kWave * kSortItems;

// Active lanes whose R-bit digit equals this lane's.
template <int R> __device__ __forceinline__ uint64_t same_digit_lanes(uint32_t d) {
  uint64_t peers = __ballot(1);
#pragma unroll
  for (int b = 0; b < R; ++b) {
    const uint64_t bal = __ballot((d >> b) & 1u);
    peers &= ((d >> b) & 1u) ? bal : ~bal;
  }
  return peers;
}

// A pass's digit is (key >> shift) & dmask: dmask keeps the pass inside
// the caller's bit range.
template <typename K, int R>
__global__ __launch_bounds__(kWave) void radix_hist_kernel(const K *__restrict__ keys, int64_t n,
                                                           int shift, uint32_t dmask,
                                                           uint32_t *__restrict__ counts,
                                                           int64_t tiles) {
  constexpr int kDigits = 1 << R;
  __shared__ uint32_t hist[kDigits];
  const int lane = threadIdx.x;
  for (int d = lane; d < kDigits; d += kWave)
    hist[d] = 0;
  __syncthreads();
  const int64_t base = blockIdx.x * static_cast<int64_t>(kSortTile);
  K k[kSortItems];
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kWave + lane;
    k[r] = i < n ? keys[i] : K(0);
  }
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kWave + lane;
    if (i < n) {
      const uint32_t d = static_cast<uint32_t>(k[r] >> shift) & dmask;
      const uint64_t peers = same_digit_lanes<R>(d);
      if (lanes_below(peers) == 0) // one lane per digit adds the digit's count
        hist[d] += static_cast<uint32_t>(__popcll(peers));
    }
  }
  __syncthreads();
  for (int d = lane; d < kDigits; d += kWave)
    counts[blockIdx.x * static_cast<int64_t>(kDigits) + d] = hist[d];
}

// Workgroup d: starts[t][d] = sum of counts[t'][d] over t' < t (the run of
// digit d before tile t) and totals[d] = the digit's count. Thread i sums a
// contiguous block of tiles, an LDS scan orders the blocks.
constexpr int kScanThreads = 256;
__global__ __launch_bounds__(kScanThreads) void radix_tile_scan_kernel(
    const uint32_t *__restrict__ counts, int64_t tiles, int kDigits, int64_t *__restrict__ starts,
    int64_t *__restrict__ totals) {
  __shared__ int64_t part[2][kScanThreads];
  const int d = blockIdx.x, i = threadIdx.x;
  const int64_t per = (tiles + kScanThreads - 1) / kScanThreads;
  const int64_t t0 = i * per, t1 = t0 + per < tiles ? t0 + per : tiles;
  int64_t sum = 0;
  for (int64_t t = t0; t < t1; ++t)
    sum += counts[t * kDigits + d];
  part[0][i] = sum;
  __syncthreads();
  int cur = 0; // inclusive Hillis-Steele scan over the threads' sums
  for (int off = 1; off < kScanThreads; off <<= 1) {
    part[cur ^ 1][i] = part[cur][i] + (i >= off ? part[cur][i - off] : 0);
    cur ^= 1;
    __syncthreads();
  }
  int64_t run = part[cur][i] - sum;
  for (int64_t t = t0; t < t1; ++t) {
    starts[t * kDigits + d] = run;
    run += counts[t * kDigits + d];
  }
  if (i == kScanThreads - 1)
    totals[d] = part[cur][i];
}

// Output position of the tile's run of digit d: the counts of all smaller
// digits (an exclusive scan of totals, done by the wave: 4 digits a lane)
// plus the digit's runs in earlier tiles.
template <typename K, int R>
__global__ __launch_bounds__(kWave) void radix_scatter_kernel(
    const K *__restrict__ kin, const int32_t *__restrict__ vin, K *__restrict__ kout,
    int32_t *__restrict__ vout, int64_t n, int shift, uint32_t dmask,
    const int64_t *__restrict__ starts, const int64_t *__restrict__ totals) {
  constexpr int kDigits = 1 << R;
  __shared__ uint32_t run[kDigits];
  __shared__ int64_t start[kDigits];
  const int lane = threadIdx.x;
  constexpr int kPer = kDigits / kWave;
  int64_t tot[kPer], sum = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    tot[q] = totals[lane * kPer + q];
    sum += tot[q];
  }
  int64_t incl = sum; // inclusive scan of the lanes' sums
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int64_t o = __shfl_up(incl, off, kWave);
    if (lane >= off)
      incl += o;
  }
  int64_t below = incl - sum;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int d = lane * kPer + q;
    run[d] = 0;
    start[d] = below + starts[blockIdx.x * static_cast<int64_t>(kDigits) + d];
    below += tot[q];
  }
  __syncthreads();
  const int64_t base = blockIdx.x * static_cast<int64_t>(kSortTile);
  K k[kSortItems];
  int32_t v[kSortItems];
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kWave + lane;
    k[r] = i < n ? kin[i] : K(0);
    v[r] = i < n ? vin[i] : 0;
  }
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kWave + lane;
    if (i < n) {
      const uint32_t d = static_cast<uint32_t>(k[r] >> shift) & dmask;
      const uint64_t peers = same_digit_lanes<R>(d);
      const uint32_t rank = lanes_below(peers);
      // every lane reads the digit's run before its first lane advances it
      // (one wave: LDS operations complete in program order)
      const uint32_t before = run[d];
      const int64_t pos = start[d] + before + rank;
      kout[pos] = k[r];
      vout[pos] = v[r];
      if (rank == 0)
        run[d] = before + static_cast<uint32_t>(__popcll(peers));
    }
  }
}

struct SortWs {
  uint32_t *counts;
  int64_t *starts, *totals;
  void *keys;
  int32_t *vals;
};

template <typename K> SortWs carve_sort(Carve &cv, int64_t n) {
  const int64_t m = n < 1 ? 1 : n;
  const int64_t tiles = ceil_div(m, kSortTile);
  constexpr int kDigits = 1 << kMaxRadixBits;
  SortWs w{};
  w.counts = cv.take<uint32_t>(kDigits * tiles);
  w.starts = cv.take<int64_t>(kDigits * tiles);
  w.totals = cv.take<int64_t>(kDigits);
  w.keys = cv.take<K>(m);
  w.vals = cv.take<int32_t>(m);
  return w;
}

template <typename K> size_t sort_bytes(int64_t n) {
  Carve cv(nullptr, 0);
  carve_sort<K>(cv, n);
  return cv.used + 256;
}

template <typename K>
void sort_run(void *tmp, size_t tmp_bytes, const K *kin, K *kout, const int32_t *vin,
              int32_t *vout, int64_t n, int end_bit, hipStream_t s) {
  if (n <= 0)
    return;
  Carve cv(tmp, tmp_bytes);
  SortWs w = carve_sort<K>(cv, n);
  constexpr int kBits = 8 * static_cast<int>(sizeof(K));
  end_bit = end_bit < 1 ? 1 : (end_bit > kBits ? kBits : end_bit);
  const int passes = (end_bit + kMaxRadixBits - 1) / kMaxRadixBits;
  const int bits = std::max(8, (end_bit + passes - 1) / passes); // 8 or 9
  const int64_t tiles = ceil_div(n, kSortTile);
  // pass p writes the caller's output when (passes - 1 - p) is even, the
  // scratch pair otherwise, so the last pass lands in the output
  const K *src_k = kin;
  const int32_t *src_v = vin;
  for (int p = 0; p < passes; ++p) {
    const bool to_out = ((passes - 1 - p) % 2) == 0;
    K *dst_k = to_out ? kout : static_cast<K *>(w.keys);
    int32_t *dst_v = to_out ? vout : w.vals;
    const int shift = p * bits;
    const int width = std::min(bits, end_bit - shift);
    const uint32_t dmask = (1u << width) - 1u;
    auto pass = [&](auto r) {
      constexpr int R = decltype(r)::value;
      hipLaunchKernelGGL((radix_hist_kernel<K, R>), dim3(tiles), dim3(kWave), 0, s, src_k, n,
                         shift, dmask, w.counts, tiles);
      RHIP_LAUNCH_CHECK();
      hipLaunchKernelGGL(radix_tile_scan_kernel, dim3(1 << R), dim3(kScanThreads), 0, s,
                         w.counts, tiles, 1 << R, w.starts, w.totals);
      RHIP_LAUNCH_CHECK();
      hipLaunchKernelGGL((radix_scatter_kernel<K, R>), dim3(tiles), dim3(kWave), 0, s, src_k,
                         src_v, dst_k, dst_v, n, shift, dmask, w.starts, w.totals);
      RHIP_LAUNCH_CHECK();
    };
    if (bits == 8)
      pass(std::integral_constant<int, 8>{});
    else
      pass(std::integral_constant<int, 9>{});
    src_k = dst_k;
    src_v = dst_v;
  }
}

} // namespace

size_t sort_pairs_u32_bytes(int64_t n) { return sort_bytes<uint32_t>(n); }
size_t sort_pairs_u64_bytes(int64_t n) { return sort_bytes<uint64_t>(n); }

void sort_pairs_u32(void *tmp, size_t tmp_bytes, const uint32_t *kin, uint32_t *kout,
                    const int32_t *vin, int32_t *vout, int64_t n, int end_bit, hipStream_t s) {
  sort_run<uint32_t>(tmp, tmp_bytes, kin, kout, vin, vout, n, end_bit, s);
}

void sort_pairs_u64(void *tmp, size_t tmp_bytes, const uint64_t *kin, uint64_t *kout,
                    const int32_t *vin, int32_t *vout, int64_t n, int end_bit, hipStream_t s) {
  sort_run<uint64_t>(tmp, tmp_bytes, kin, kout, vin, vout, n, end_bit, s);
}

} // namespace rhip
