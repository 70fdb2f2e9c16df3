// Stable device radix sorts of (key, int32 value) pairs, used by the hash
// table (locality order), the kernel map (neighbour-mask order) and pooling
// (grouping rows by output). Least-significant-digit first with 8- or 9-bit
// digits: the fewest passes the key bits allow, then the narrowest digit for
// that many passes (26 bits: 3 passes of 9; 22 bits: 3 of 8; 16 bits: 2 of
// 8). Three kernels per pass over tiles of 2048 keys:
//
//   radix_hist_kernel     one workgroup per tile: the tile's digit counts
//                         (LDS atomics), stored digit-major, counts[d][tile];
//   radix_row_scan_kernel one wave per digit: exclusive scan of the digit's
//                         counts over the tiles (the digit's keys in earlier
//                         tiles) and the digit's total;
//   radix_scatter_kernel  one workgroup per tile: ranks its keys by digit
//                         (wave ballots in key order, so equal digits keep
//                         their order), scans the digit totals in LDS for
//                         where each digit starts, stages its keys in LDS by
//                         digit and writes each digit's run contiguously.
//
// Every buffer the sort needs is carved from the caller's scratch; nothing is
// allocated or memset.
#include "rhip_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace rhip {
namespace {

constexpr int kMaxRadixBits = 9;
constexpr int kMaxDigits = 1 << kMaxRadixBits;
constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
// 2048-key tiles: config 2's 409,553 keys make 200 workgroups per pass (100
// with 4096-key tiles left most CUs idle: mask sort 46 -> ~32 us)
constexpr int kSortItems = 8;
constexpr int kSortTile = kSortThreads * kSortItems;
constexpr int kWaveKeys = kSortTile / kSortWaves;

// Tiles of a sort of n keys, padded to a multiple of 4 so that each digit's
// row of the count table starts 16-byte aligned; the padding tiles hold no
// keys and count zero.
inline int64_t sort_tiles(int64_t n) { return ceil_div(ceil_div(n, kSortTile), 4) * 4; }

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

// Exclusive scan of one value per thread over the workgroup, in thread
// order; `wave_sum` is LDS scratch of kSortWaves entries. Contains a barrier.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *wave_sum) {
  const int lane = lane_id(), w = threadIdx.x / kWave;
  uint32_t incl = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint32_t o = __shfl_up(incl, off, kWave);
    if (lane >= off)
      incl += o;
  }
  if (lane == kWave - 1)
    wave_sum[w] = incl;
  __syncthreads();
  uint32_t before = 0;
  for (int i = 0; i < w; ++i)
    before += wave_sum[i];
  return before + incl - v;
}

// A pass's digit is (key >> shift) & dmask: dmask keeps the pass inside
// the caller's bit range. Launched over all (padded) tiles.
template <typename K>
__global__ __launch_bounds__(kSortThreads) void radix_hist_kernel(
    const K *__restrict__ keys, int64_t n, int shift, uint32_t dmask,
    uint32_t *__restrict__ counts, int64_t tiles) {
  __shared__ uint32_t hist[kMaxDigits];
  const int t = threadIdx.x;
  for (int d = t; d < kMaxDigits; d += kSortThreads)
    hist[d] = 0;
  __syncthreads();
  const int64_t base = blockIdx.x * static_cast<int64_t>(kSortTile);
  K k[kSortItems];
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int64_t i = base + r * kSortThreads + t;
    k[r] = i < n ? keys[i] : K(0);
  }
#pragma unroll
  for (int r = 0; r < kSortItems; ++r)
    if (base + r * kSortThreads + t < n)
      atomicAdd(&hist[static_cast<uint32_t>(k[r] >> shift) & dmask], 1u);
  __syncthreads();
  for (int d = t; d <= static_cast<int>(dmask); d += kSortThreads)
    counts[d * tiles + blockIdx.x] = hist[d];
}

// Per digit (one wave each, blockIdx.x = digit): exclusive scan of the
// digit's counts over the tiles, base[d][tile], and the digit's total.
__global__ __launch_bounds__(kWave) void radix_row_scan_kernel(const uint32_t *__restrict__ counts,
                                                              int64_t tiles,
                                                              uint32_t *__restrict__ base,
                                                              uint32_t *__restrict__ total) {
  const int lane = lane_id();
  const int64_t row = static_cast<int64_t>(blockIdx.x) * tiles;
  uint32_t carry = 0;
  for (int64_t t0 = 0; t0 < tiles; t0 += 4 * kWave) {
    // lane owns tiles t0 + 4 lane .. + 3 (tiles is a multiple of 4)
    const int64_t e = t0 + 4 * lane;
    const uint4 v = e < tiles ? *reinterpret_cast<const uint4 *>(counts + row + e)
                              : uint4{0u, 0u, 0u, 0u};
    const uint32_t sum = v.x + v.y + v.z + v.w;
    uint32_t incl = sum;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t o = __shfl_up(incl, off, kWave);
      if (lane >= off)
        incl += o;
    }
    uint4 o;
    o.x = carry + incl - sum;
    o.y = o.x + v.x;
    o.z = o.y + v.y;
    o.w = o.z + v.z;
    if (e < tiles)
      *reinterpret_cast<uint4 *>(base + row + e) = o;
    carry += __shfl(incl, kWave - 1, kWave);
  }
  if (lane == 0)
    total[blockIdx.x] = carry;
}

template <typename K, int R>
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const K *__restrict__ kin, const int32_t *__restrict__ vin, K *__restrict__ kout,
    int32_t *__restrict__ vout, int64_t n, int shift, uint32_t dmask,
    const uint32_t *__restrict__ base, const uint32_t *__restrict__ total, int64_t tiles) {
  constexpr int kDigits = 1 << R;
  constexpr int kPer = kDigits / kSortThreads; // digits per thread (1 or 2)
  __shared__ uint32_t wh[kSortWaves][kDigits]; // per-wave digit runs, then wave offsets
  __shared__ uint32_t loc[kDigits];            // the tile's digit runs start here in LDS
  __shared__ uint32_t gbase[kDigits];          // ... and here in the output
  __shared__ uint32_t wave_sum[2][kSortWaves];
  __shared__ K sk[kSortTile];
  __shared__ int32_t sv[kSortTile];
  const int t = threadIdx.x, lane = lane_id(), w = t / kWave;
  for (int i = t; i < kSortWaves * kDigits; i += kSortThreads)
    (&wh[0][0])[i] = 0;
  __syncthreads();
  const int64_t tile = blockIdx.x;
  const int64_t t0 = tile * kSortTile;
  const int tile_n = static_cast<int>(min<int64_t>(kSortTile, n - t0));

  // load (each wave a contiguous quarter) and rank within the wave, in key order
  K k[kSortItems];
  int32_t v[kSortItems];
  uint32_t dg[kSortItems], rk[kSortItems];
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int li = w * kWaveKeys + r * kWave + lane;
    const bool ok = li < tile_n;
    k[r] = ok ? kin[t0 + li] : K(0);
    v[r] = ok ? vin[t0 + li] : 0;
  }
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int li = w * kWaveKeys + r * kWave + lane;
    dg[r] = static_cast<uint32_t>(k[r] >> shift) & dmask;
    rk[r] = 0;
    if (li < tile_n) {
      const uint64_t peers = same_digit_lanes<R>(dg[r]);
      const uint32_t below = lanes_below(peers);
      // every lane reads the digit's run before its first lane advances it
      // (one wave: LDS operations complete in program order)
      const uint32_t run = wh[w][dg[r]];
      rk[r] = run + below;
      if (below == 0)
        wh[w][dg[r]] = run + static_cast<uint32_t>(__popcll(peers));
    }
  }
  __syncthreads();

  // this thread's digits: the tile's count (wave runs become wave offsets)
  // and the output position of the tile's run from the scanned count table
  uint32_t cnt_mine = 0;
  uint32_t cnt[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int d = t * kPer + q;
    uint32_t run = 0;
#pragma unroll
    for (int i = 0; i < kSortWaves; ++i) {
      const uint32_t c = wh[i][d];
      wh[i][d] = run;
      run += c;
    }
    cnt[q] = run;
    cnt_mine += run;
  }
  // where each digit's run starts in the output (keys of smaller digits, then
  // this digit's keys in earlier tiles) and in the tile
  uint32_t tot[kPer], tot_mine = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int d = t * kPer + q;
    tot[q] = d <= static_cast<int>(dmask) ? total[d] : 0u;
    tot_mine += tot[q];
  }
  uint32_t dstart = block_exclusive_scan(tot_mine, wave_sum[0]);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int d = t * kPer + q;
    gbase[d] = dstart + (d <= static_cast<int>(dmask) ? base[d * tiles + tile] : 0u);
    dstart += tot[q];
  }
  uint32_t lbase = block_exclusive_scan(cnt_mine, wave_sum[1]);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    loc[t * kPer + q] = lbase;
    lbase += cnt[q];
  }
  __syncthreads();

  // stage the tile in digit order, then write each digit's run
#pragma unroll
  for (int r = 0; r < kSortItems; ++r) {
    const int li = w * kWaveKeys + r * kWave + lane;
    if (li < tile_n) {
      const uint32_t p = loc[dg[r]] + wh[w][dg[r]] + rk[r];
      sk[p] = k[r];
      sv[p] = v[r];
    }
  }
  __syncthreads();
  for (int i = t; i < tile_n; i += kSortThreads) {
    const K key = sk[i];
    const uint32_t d = static_cast<uint32_t>(key >> shift) & dmask;
    const int64_t o = static_cast<int64_t>(gbase[d]) + (i - static_cast<int64_t>(loc[d]));
    kout[o] = key;
    vout[o] = sv[i];
  }
}

struct SortWs {
  uint32_t *counts;
  uint32_t *base;
  uint32_t *total;
  void *keys;
  int32_t *vals;
};

template <typename K> SortWs carve_sort(Carve &cv, int64_t n) {
  const int64_t m = n < 1 ? 1 : n;
  SortWs w{};
  w.counts = cv.take<uint32_t>(static_cast<size_t>(kMaxDigits) * sort_tiles(m));
  w.base = cv.take<uint32_t>(static_cast<size_t>(kMaxDigits) * sort_tiles(m));
  w.total = cv.take<uint32_t>(kMaxDigits);
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
  const int64_t grid = ceil_div(n, kSortTile);
  const int64_t tiles = sort_tiles(n); // the hist grid: padding tiles write zero counts
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
    hipLaunchKernelGGL((radix_hist_kernel<K>), dim3(tiles), dim3(kSortThreads), 0, s, src_k, n,
                       shift, dmask, w.counts, tiles);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(radix_row_scan_kernel, dim3(dmask + 1), dim3(kWave), 0, s, w.counts, tiles,
                       w.base, w.total);
    RHIP_LAUNCH_CHECK();
    auto pass = [&](auto r) {
      constexpr int R = decltype(r)::value;
      hipLaunchKernelGGL((radix_scatter_kernel<K, R>), dim3(grid), dim3(kSortThreads), 0, s,
                         src_k, src_v, dst_k, dst_v, n, shift, dmask, w.base, w.total, tiles);
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
