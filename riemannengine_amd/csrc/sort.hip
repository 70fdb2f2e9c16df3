// Stable device radix sorts of (key, int32 value) pairs, used by the hash
// table (locality order), the kernel map (neighbour-mask order) and pooling
// (grouping rows by output). Least-significant-digit first with 8- or 9-bit
// digits: the fewest passes the key bits allow, then the narrowest digit for
// that many passes (26 bits: 3 passes of 9; 22 bits: 3 of 8; 16 bits: 2 of
// 8). Two kernels per pass over tiles of 4096 keys:
//
//   radix_hist_kernel     one workgroup per tile: the tile's digit counts
//                         (LDS atomics), stored digit-major, counts[d][tile],
//                         so that one digit's counts over all tiles are
//                         contiguous;
//   radix_scatter_kernel  one workgroup per tile: ranks its keys by digit
//                         (wave ballots in key order, so equal digits keep
//                         their order), reads its digits' rows of the count
//                         table (16-byte loads) for the keys of each digit in
//                         all tiles and in the tiles before it, scans the
//                         digit totals for where each digit's run starts, and
//                         writes its keys staged in LDS by digit, so that each
//                         digit's run goes out contiguously.
//
// No tile waits on another: every count the scatter needs is final when it
// starts. Every buffer the sort needs is carved from the caller's scratch;
// nothing is allocated or memset.
#include "rhip_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace rhip {
namespace {

constexpr int kMaxRadixBits = 9;
constexpr int kMaxDigits = 1 << kMaxRadixBits;
constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / kWave;
constexpr int kSortItems = 16;
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

template <typename K, int R>
__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(
    const K *__restrict__ kin, const int32_t *__restrict__ vin, K *__restrict__ kout,
    int32_t *__restrict__ vout, int64_t n, int shift, uint32_t dmask,
    const uint32_t *__restrict__ counts, int64_t tiles) {
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

  // this thread's digits: the tile's count (wave runs become wave offsets),
  // and from the count table the keys in all tiles and in earlier tiles
  uint32_t cnt[kPer], before[kPer], total[kPer];
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
    before[q] = 0;
    total[q] = 0;
    if (d <= static_cast<int>(dmask)) {
      const uint4 *row = reinterpret_cast<const uint4 *>(counts + d * tiles);
      for (int64_t j = 0; j < tiles / 4; ++j) {
        const uint4 c = row[j];
        const int64_t tt = 4 * j;
        total[q] += c.x + c.y + c.z + c.w;
        before[q] += (tt < tile ? c.x : 0u) + (tt + 1 < tile ? c.y : 0u) +
                     (tt + 2 < tile ? c.z : 0u) + (tt + 3 < tile ? c.w : 0u);
      }
    }
  }
  // where each digit's run starts in the output, and in the tile
  uint32_t tot_mine = 0, cnt_mine = 0;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    tot_mine += total[q];
    cnt_mine += cnt[q];
  }
  uint32_t dbase = block_exclusive_scan(tot_mine, wave_sum[0]);
  uint32_t lbase = block_exclusive_scan(cnt_mine, wave_sum[1]);
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int d = t * kPer + q;
    gbase[d] = dbase + before[q];
    loc[d] = lbase;
    dbase += total[q];
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
  void *keys;
  int32_t *vals;
};

template <typename K> SortWs carve_sort(Carve &cv, int64_t n) {
  const int64_t m = n < 1 ? 1 : n;
  SortWs w{};
  w.counts = cv.take<uint32_t>(static_cast<size_t>(kMaxDigits) * sort_tiles(m));
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
    auto pass = [&](auto r) {
      constexpr int R = decltype(r)::value;
      hipLaunchKernelGGL((radix_scatter_kernel<K, R>), dim3(grid), dim3(kSortThreads), 0, s,
                         src_k, src_v, dst_k, dst_v, n, shift, dmask, w.counts, tiles);
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
