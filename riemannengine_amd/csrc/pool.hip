// Sparse pooling on gfx950: pooling stride maps, local sum/average/max
// pooling over a neighbour table, and global (per-batch) pooling.
//
// Local pooling is a gather-reduce: output row o reduces the input rows
// nbr[k*n_out + o] (k < K, -1 = none) channel-wise. Nothing is multiplied, so
// every kernel here is HBM/latency-bound integer-indexed streaming: one
// thread owns one output (or input) row's 16-byte channel slice (4 fp32 or
// 8 bf16), a wave covers 64 such slices, so the gathered rows are read as
// whole contiguous 16-byte-aligned segments. Accumulation is fp32.
//
// Reference semantics (engine/nn/pooling.cpp:80-150): empty outputs are
// zero, average divides the sum by the number of pooled rows, max
// propagates NaN (torch amax), and the max gradient is split evenly between
// tied inputs (torch amax backward). The stride map follows
// CoordinateMapCPU::stride_map (engine/grid/lattice_cpu.hpp:675-710).
#include "rhip_internal.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <initializer_list>
#include <type_traits>

namespace rhip {
namespace {

constexpr int kPoolThreads = 256;
// Rows one lane reduces per global-pooling chunk (per chunk: RPL rows times
// the row lanes of a block).
constexpr int kRowsPerLane = 16;

static int bit_width_u64(uint64_t v) { return v == 0 ? 0 : 64 - __builtin_clzll(v); }

// ------------------------------------------------------ vector row slices

// V consecutive channels of one row through one 16-byte access (V = 4 fp32,
// 8 bf16), or V = 1 for rows whose width is not a multiple of 16 bytes.
template <typename T, int V> struct Slice;

// Raw is the loaded 16 bytes (kept in registers until reduced): load_raw
// then widen = load.
template <> struct Slice<float, 4> {
  using Raw = float4;
  __device__ static __forceinline__ Raw load_raw(const float *p) {
    return *reinterpret_cast<const float4 *>(p);
  }
  __device__ static __forceinline__ void widen(const Raw &f, float *v) {
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  }
  __device__ static __forceinline__ void load(const float *p, float *v) { widen(load_raw(p), v); }
  __device__ static __forceinline__ void store(float *p, const float *v) {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};
template <> struct Slice<float, 8> {
  struct Raw {
    float4 a, b;
  };
  __device__ static __forceinline__ Raw load_raw(const float *p) {
    return {Slice<float, 4>::load_raw(p), Slice<float, 4>::load_raw(p + 4)};
  }
  __device__ static __forceinline__ void widen(const Raw &r, float *v) {
    Slice<float, 4>::widen(r.a, v);
    Slice<float, 4>::widen(r.b, v + 4);
  }
  __device__ static __forceinline__ void load(const float *p, float *v) {
    Slice<float, 4>::load(p, v);
    Slice<float, 4>::load(p + 4, v + 4);
  }
  __device__ static __forceinline__ void store(float *p, const float *v) {
    Slice<float, 4>::store(p, v);
    Slice<float, 4>::store(p + 4, v + 4);
  }
};
template <> struct Slice<float, 1> {
  using Raw = float;
  __device__ static __forceinline__ Raw load_raw(const float *p) { return *p; }
  __device__ static __forceinline__ void widen(const Raw &f, float *v) { v[0] = f; }
  __device__ static __forceinline__ void load(const float *p, float *v) { v[0] = *p; }
  __device__ static __forceinline__ void store(float *p, const float *v) { *p = v[0]; }
};
template <> struct Slice<__bf16, 8> {
  using Raw = uint4;
  __device__ static __forceinline__ Raw load_raw(const __bf16 *p) {
    return *reinterpret_cast<const uint4 *>(p);
  }
  // bf16 -> fp32 is exact: the 16 bits become the high half of the float.
  __device__ static __forceinline__ void widen(const Raw &u, float *v) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __uint_as_float(w[j] << 16);
      v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
  __device__ static __forceinline__ void load(const __bf16 *p, float *v) { widen(load_raw(p), v); }
  // fp32 -> bf16 rounds to nearest even
  __device__ static __forceinline__ void store(__bf16 *p, const float *v) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v[2 * j]));
      const uint32_t hi = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v[2 * j + 1]));
      w[j] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct Slice<__bf16, 1> {
  using Raw = __bf16;
  __device__ static __forceinline__ Raw load_raw(const __bf16 *p) { return *p; }
  __device__ static __forceinline__ void widen(const Raw &f, float *v) {
    v[0] = static_cast<float>(f);
  }
  __device__ static __forceinline__ void load(const __bf16 *p, float *v) {
    v[0] = static_cast<float>(*p);
  }
  __device__ static __forceinline__ void store(__bf16 *p, const float *v) {
    *p = static_cast<__bf16>(v[0]);
  }
};

// max as torch.amax: NaN wins, otherwise the larger value
__device__ __forceinline__ float max_nan(float acc, float v) {
  return (v > acc || v != v) ? v : acc;
}

template <int MODE> __device__ __forceinline__ float pool_init() {
  return MODE == RHIP_POOL_MAX ? -INFINITY : 0.f;
}

// -------------------------------------------------------- local pooling
//
// Thread t = tile * 256 + threadIdx.x owns processing position j = t / lpr
// and channels [(t % lpr) * V, +V); tiles come from xcd_tile, so runs of
// neighbouring positions (which gather the same rows) share an XCD's L2.
// The neighbour loop reads kChunk table entries first, then issues the
// chunk's gathers (each under its own lane mask), then reduces: up to kChunk
// row loads in flight per thread instead of one.
constexpr int kChunk = 8;

__device__ __forceinline__ int64_t pool_thread(int lane) {
  return xcd_tile(blockIdx.x) * static_cast<int64_t>(kPoolThreads) + lane;
}

// y[o] = reduce over k of x[nbr[k*n_out+j]] for the output o = order[j] at
// processing position j; counts[o] = number of rows pooled.
template <typename T, int MODE, int V>
__global__ __launch_bounds__(kPoolThreads) void pool_fwd_kernel(
    const T *__restrict__ x, int C, int lpr, const int32_t *__restrict__ nbr, int K,
    int64_t n_out, const int32_t *__restrict__ order, T *__restrict__ y,
    int32_t *__restrict__ counts) {
  const int64_t t = pool_thread(threadIdx.x);
  const int64_t j = t / lpr;
  if (j >= n_out)
    return;
  const int c0 = static_cast<int>(t - j * lpr) * V;
  const int64_t o = order ? order[j] : j;
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    acc[e] = pool_init<MODE>();
  int cnt = 0;
  for (int k0 = 0; k0 < K; k0 += kChunk) {
    int32_t idx[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      idx[u] = k0 + u < K ? nbr[(k0 + u) * n_out + j] : -1;
    typename Slice<T, V>::Raw raw[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      if (idx[u] >= 0)
        raw[u] = Slice<T, V>::load_raw(x + static_cast<int64_t>(idx[u]) * C + c0);
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      if (idx[u] < 0)
        continue;
      ++cnt;
      float v[V];
      Slice<T, V>::widen(raw[u], v);
#pragma unroll
      for (int e = 0; e < V; ++e)
        acc[e] = MODE == RHIP_POOL_MAX ? max_nan(acc[e], v[e]) : acc[e] + v[e];
    }
  }
  float out[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    out[e] = cnt == 0 ? 0.f
                      : (MODE == RHIP_POOL_AVG ? acc[e] / static_cast<float>(cnt) : acc[e]);
  Slice<T, V>::store(y + o * C + c0, out);
  if (counts != nullptr && c0 == 0)
    counts[o] = cnt;
}

// Max-pooling gradient share per output channel: gs[o][c] = gy[o][c] / (number
// of pooled rows whose value equals y[o][c]), 0 when none does.
// zero_tie: one more tie where y[o][c] == 0 (RHIP_POOL_MAX_SCATTER).
template <typename T, int V>
__global__ __launch_bounds__(kPoolThreads) void pool_maxshare_kernel(
    const T *__restrict__ gy, const T *__restrict__ x, const T *__restrict__ y, int C, int lpr,
    const int32_t *__restrict__ nbr, int K, int64_t n_out, const int32_t *__restrict__ order,
    int zero_tie, float *__restrict__ gs) {
  const int64_t t = pool_thread(threadIdx.x);
  const int64_t j = t / lpr;
  if (j >= n_out)
    return;
  const int c0 = static_cast<int>(t - j * lpr) * V;
  const int64_t o = order ? order[j] : j;
  float yv[V], cnt[V];
  Slice<T, V>::load(y + o * C + c0, yv);
#pragma unroll
  for (int e = 0; e < V; ++e)
    cnt[e] = (zero_tie && yv[e] == 0.f) ? 1.f : 0.f;
  for (int k0 = 0; k0 < K; k0 += kChunk) {
    int32_t idx[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      idx[u] = k0 + u < K ? nbr[(k0 + u) * n_out + j] : -1;
    typename Slice<T, V>::Raw raw[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      if (idx[u] >= 0)
        raw[u] = Slice<T, V>::load_raw(x + static_cast<int64_t>(idx[u]) * C + c0);
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      if (idx[u] < 0)
        continue;
      float v[V];
      Slice<T, V>::widen(raw[u], v);
#pragma unroll
      for (int e = 0; e < V; ++e)
        cnt[e] += v[e] == yv[e] ? 1.f : 0.f;
    }
  }
  float g[V], share[V];
  Slice<T, V>::load(gy + o * C + c0, g);
#pragma unroll
  for (int e = 0; e < V; ++e)
    share[e] = cnt[e] > 0.f ? g[e] / cnt[e] : 0.f;
  Slice<float, V>::store(gs + o * C + c0, share);
}

// gx[i] for the input i = order[j] at processing position j: the sum over k
// with o = nbr_t[k*n_in+j] >= 0 of
//   sum: gy[o];  average: gy[o] / counts[o];  max: gs[o] where x[i] == y[o].
template <typename T, int MODE, int V>
__global__ __launch_bounds__(kPoolThreads) void pool_bwd_kernel(
    const T *__restrict__ gy, const float *__restrict__ gs, const T *__restrict__ x,
    const T *__restrict__ y, int C, int lpr, const int32_t *__restrict__ nbr_t, int K,
    int64_t n_in, const int32_t *__restrict__ order, const int32_t *__restrict__ counts,
    T *__restrict__ gx) {
  const int64_t t = pool_thread(threadIdx.x);
  const int64_t j = t / lpr;
  if (j >= n_in)
    return;
  const int c0 = static_cast<int>(t - j * lpr) * V;
  const int64_t i = order ? order[j] : j;
  float acc[V], xv[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    acc[e] = 0.f;
  if (MODE == RHIP_POOL_MAX)
    Slice<T, V>::load(x + i * C + c0, xv);
  // max keeps two slices (y and the fp32 share) per entry: half the chunk
  constexpr int CH = MODE == RHIP_POOL_MAX ? kChunk / 2 : kChunk;
  for (int k0 = 0; k0 < K; k0 += CH) {
    int32_t idx[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u)
      idx[u] = k0 + u < K ? nbr_t[(k0 + u) * n_in + j] : -1;
    if (MODE == RHIP_POOL_MAX) {
      typename Slice<T, V>::Raw yraw[CH];
      typename Slice<float, V>::Raw sraw[CH];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        if (idx[u] >= 0) {
          yraw[u] = Slice<T, V>::load_raw(y + static_cast<int64_t>(idx[u]) * C + c0);
          sraw[u] = Slice<float, V>::load_raw(gs + static_cast<int64_t>(idx[u]) * C + c0);
        }
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        if (idx[u] < 0)
          continue;
        float yv[V], sv[V];
        Slice<T, V>::widen(yraw[u], yv);
        Slice<float, V>::widen(sraw[u], sv);
#pragma unroll
        for (int e = 0; e < V; ++e)
          acc[e] += xv[e] == yv[e] ? sv[e] : 0.f;
      }
    } else {
      typename Slice<T, V>::Raw raw[CH];
      float n[CH];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        if (idx[u] >= 0) {
          raw[u] = Slice<T, V>::load_raw(gy + static_cast<int64_t>(idx[u]) * C + c0);
          n[u] = MODE == RHIP_POOL_AVG ? static_cast<float>(counts[idx[u]]) : 1.f;
        }
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        if (idx[u] < 0)
          continue;
        float v[V];
        Slice<T, V>::widen(raw[u], v);
#pragma unroll
        for (int e = 0; e < V; ++e)
          acc[e] += MODE == RHIP_POOL_AVG ? v[e] / n[u] : v[e];
      }
    }
  }
  Slice<T, V>::store(gx + i * C + c0, acc);
}

// ------------------------------------------------------------ stride map

// keys[i] = row of (b, floor(x / s) * s) in the output table, vals[i] = i;
// a row with no output counts in miss[0] and its index goes to miss[1].
__global__ __launch_bounds__(kPoolThreads) void stride_lookup_kernel(
    TableView t, const int32_t *__restrict__ in, int64_t n, StrideArg st,
    uint32_t *__restrict__ keys, int32_t *__restrict__ vals,
    unsigned long long *__restrict__ miss) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  const bool valid = i < n; // every lane stays for the wave's shuffles
  int32_t c[RHIP_MAX_COLS];
  c[0] = valid ? in[i * t.ncol] : 0;
#pragma unroll
  for (int j = 1; j < RHIP_MAX_COLS; ++j)
    c[j] = valid && j < t.ncol ? floor_align(in[i * t.ncol + j], st.s[j - 1]) : 0;
  // input rows in one stride cell query the same output row: a row whose
  // cell repeats the previous lane's takes that run's answer
  const bool follow = repeats_prev_row(c, valid);
  const uint64_t heads = __ballot(!follow);
  int32_t o = -1;
  if (valid && !follow)
    o = table_find(t, c);
  o = __shfl(o, run_head(heads), kWave);
  if (!valid)
    return;
  if (o < 0) {
    atomicAdd(&miss[0], 1ull);
    atomicMin(&miss[1], static_cast<unsigned long long>(i));
  }
  keys[i] = o < 0 ? 0u : static_cast<uint32_t>(o);
  vals[i] = static_cast<int32_t>(i);
}

// keys[i] = group[i], vals[i] = i; a group outside [0, n_groups) counts in
// miss[0] and its row goes to miss[1].
__global__ __launch_bounds__(kPoolThreads) void group_keys_kernel(
    const int32_t *__restrict__ group, int64_t n, int64_t n_groups, uint32_t *__restrict__ keys,
    int32_t *__restrict__ vals, unsigned long long *__restrict__ miss) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  if (i >= n)
    return;
  const int32_t g = group[i];
  const bool ok = g >= 0 && g < n_groups;
  if (!ok) {
    atomicAdd(&miss[0], 1ull);
    atomicMin(&miss[1], static_cast<unsigned long long>(i));
  }
  keys[i] = ok ? static_cast<uint32_t>(g) : 0u;
  vals[i] = static_cast<int32_t>(i);
}

// start[o] = first sorted position of output o.
__global__ __launch_bounds__(kPoolThreads) void group_start_kernel(
    const uint32_t *__restrict__ skeys, int64_t n, int32_t *__restrict__ start) {
  const int64_t s = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  if (s >= n)
    return;
  const uint32_t o = skeys[s];
  if (s == 0 || skeys[s - 1] != o)
    start[o] = static_cast<int32_t>(s);
}

__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
    v = max(v, __shfl_xor(v, off, kWave));
  return v;
}

// Maximum over the workgroup (every thread gets it).
__device__ __forceinline__ int block_max(int v) {
  __shared__ int red[kPoolThreads / kWave];
  v = wave_max(v);
  if (lane_id() == 0)
    red[threadIdx.x / kWave] = v;
  __syncthreads();
  int m = red[0];
#pragma unroll
  for (int w = 1; w < kPoolThreads / kWave; ++w)
    m = max(m, red[w]);
  return m;
}

// Grid of the reductions below: grid-stride loops over at most this many
// workgroups, one atomic each (atomics on one address serialise).
constexpr int kReduceBlocks = 512;

// rank[s] = position of sorted entry s within its output's group; kmax =
// largest group size.
__global__ __launch_bounds__(kPoolThreads) void group_rank_kernel(
    const uint32_t *__restrict__ skeys, int64_t n, const int32_t *__restrict__ start,
    int32_t *__restrict__ rank, int32_t *__restrict__ kmax) {
  int m = 0;
  for (int64_t s = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x; s < n;
       s += static_cast<int64_t>(gridDim.x) * kPoolThreads) {
    const int r = static_cast<int>(s - start[skeys[s]]);
    rank[s] = r;
    m = max(m, r + 1);
  }
  m = block_max(m);
  if (threadIdx.x == 0 && m > 0)
    atomicMax(kmax, m);
}

// Count of unmatched rows = 0, smallest unmatched row = none.
__global__ void miss_init_kernel(unsigned long long *miss) {
  if (threadIdx.x == 0) {
    miss[0] = 0ull;
    miss[1] = ~0ull;
  }
}

// pos[order[p]] = p
__global__ __launch_bounds__(kPoolThreads) void invert_order_kernel(
    const int32_t *__restrict__ order, int64_t n, int32_t *__restrict__ pos) {
  const int64_t p = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  if (p < n)
    pos[order[p]] = static_cast<int32_t>(p);
}

__global__ __launch_bounds__(kPoolThreads) void fill_i32_kernel(int32_t *__restrict__ p,
                                                                int64_t n, int32_t v) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  if (i < n)
    p[i] = v;
}

// Tables by processing position: nbr column pos_out[o] (row = rank within
// the output's group), nbr_t column pos_in[i] (one row: each input has one
// output). Ranks past k_max (a k_max smaller than phase 1 found) are not
// written.
__global__ __launch_bounds__(kPoolThreads) void stride_scatter_kernel(
    const uint32_t *__restrict__ skeys, const int32_t *__restrict__ svals,
    const int32_t *__restrict__ rank, int64_t n_in, int64_t n_out, int32_t k_max,
    const int32_t *__restrict__ pos_in, const int32_t *__restrict__ pos_out,
    int32_t *__restrict__ nbr, int32_t *__restrict__ nbr_t, int32_t *__restrict__ in_rows,
    int32_t *__restrict__ out_rows) {
  const int64_t s = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  if (s >= n_in)
    return;
  const int32_t o = static_cast<int32_t>(skeys[s]);
  const int32_t i = svals[s];
  const int64_t r = rank[s];
  if (r >= k_max || o >= n_out)
    return;
  nbr[r * n_out + (pos_out ? pos_out[o] : o)] = i;
  nbr_t[pos_in ? pos_in[i] : i] = o;
  in_rows[s] = i;
  out_rows[s] = o;
}

// Column q of table [K, n]: its entries >= 0 moved to its first rows (row
// order kept), -1 after them; kmax = most such entries in one column.
__global__ __launch_bounds__(kPoolThreads) void table_compact_kernel(
    const int32_t *__restrict__ table, int K, int64_t n, int32_t *__restrict__ out,
    int32_t *__restrict__ kmax) {
  int m = 0;
  for (int64_t q = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x; q < n;
       q += static_cast<int64_t>(gridDim.x) * kPoolThreads) {
    int c = 0;
    for (int k = 0; k < K; ++k) {
      const int32_t v = table[k * n + q];
      if (v >= 0)
        out[static_cast<int64_t>(c++) * n + q] = v;
    }
    for (int k = c; k < K; ++k)
      out[k * n + q] = -1;
    m = max(m, c);
  }
  m = block_max(m);
  if (threadIdx.x == 0 && m > 0)
    atomicMax(kmax, m);
}

// --------------------------------------------------------- global pooling

__global__ __launch_bounds__(kPoolThreads) void batch_max_kernel(
    const int32_t *__restrict__ coords, int64_t n, int ncol, int32_t *__restrict__ bmax) {
  int m = INT_MIN;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kPoolThreads)
    m = max(m, coords[i * ncol]);
  m = block_max(m);
  if (threadIdx.x == 0 && m != INT_MIN)
    atomicMax(bmax, m);
}

// keys[i] = batch of row i, or B for a batch outside [0, B) (sorted last).
__global__ __launch_bounds__(kPoolThreads) void batch_keys_kernel(
    const int32_t *__restrict__ coords, int64_t n, int ncol, int32_t B,
    uint32_t *__restrict__ keys, int32_t *__restrict__ vals) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  if (i >= n)
    return;
  const int32_t b = coords[i * ncol];
  keys[i] = (b >= 0 && b < B) ? static_cast<uint32_t>(b) : static_cast<uint32_t>(B);
  vals[i] = static_cast<int32_t>(i);
}

// seg[b] = first sorted position whose key is >= b, for b in [0, B].
__global__ __launch_bounds__(kPoolThreads) void batch_bounds_kernel(
    const uint32_t *__restrict__ skeys, int64_t n, int32_t B, int32_t *__restrict__ seg) {
  const int64_t s = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  if (s > n)
    return;
  const int64_t prev = s == 0 ? -1 : static_cast<int64_t>(skeys[s - 1]);
  const int64_t cur = s == n ? static_cast<int64_t>(B) : static_cast<int64_t>(skeys[s]);
  for (int64_t b = prev + 1; b <= cur; ++b)
    seg[b] = static_cast<int32_t>(s);
}

// Chunks of rows per batch: nchunk[b] = ceil(rows of b / R).
__global__ __launch_bounds__(kPoolThreads) void chunk_count_kernel(
    const int32_t *__restrict__ seg, int32_t B, int R, int64_t *__restrict__ nchunk) {
  const int64_t b = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  if (b < B)
    nchunk[b] = (seg[b + 1] - seg[b] + R - 1) / R;
}

// The row lanes of a block reduce their own rows, then lane 0 of each
// channel slice combines the row lanes in order: a fixed summation order.
enum GlobalOp { kOpSum = 0, kOpMax = 1, kOpCountEq = 2 };

template <int OP> __device__ __forceinline__ float gop_init() {
  return OP == kOpMax ? -INFINITY : 0.f;
}
template <int OP> __device__ __forceinline__ float gop(float acc, float v) {
  return OP == kOpMax ? max_nan(acc, v) : acc + v;
}

// Stage 1: block g reduces chunk g (rows [seg[b] + (g - base[b]) * R, +R) of
// batch b, via members) into partial[g][c]. kOpCountEq counts rows equal to
// ref[b]. Channel tile blockIdx.y covers lanes [tile * lpt, +lpt).
template <typename T, int OP, int V>
__global__ __launch_bounds__(kPoolThreads) void gpool_partial_kernel(
    const T *__restrict__ x, const T *__restrict__ ref, int C, int lpr, int lpt,
    const int32_t *__restrict__ members, const int32_t *__restrict__ seg,
    const int64_t *__restrict__ base, int32_t B, int R, float *__restrict__ partial) {
  __shared__ float red[kPoolThreads * V];
  const int64_t g = blockIdx.x;
  if (g >= base[B])
    return;
  // batch b with base[b] <= g < base[b + 1]
  int lo = 0, hi = B; // invariant: base[lo] <= g < base[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (base[mid] <= g)
      lo = mid;
    else
      hi = mid;
  }
  const int b = lo;
  const int lane = threadIdx.x % lpt, rlane = threadIdx.x / lpt, rl = kPoolThreads / lpt;
  const int cc = blockIdx.y * lpt + lane;
  const bool active = cc < lpr && rlane < rl;
  const int c0 = cc * V;
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    acc[e] = gop_init<OP>();
  if (active) {
    float rv[V];
    if (OP == kOpCountEq)
      Slice<T, V>::load(ref + static_cast<int64_t>(b) * C + c0, rv);
    const int64_t s0 = seg[b] + (g - base[b]) * R;
    const int64_t s1 = min(s0 + R, static_cast<int64_t>(seg[b + 1]));
    for (int64_t s = s0 + rlane; s < s1; s += rl) {
      float v[V];
      Slice<T, V>::load(x + static_cast<int64_t>(members[s]) * C + c0, v);
#pragma unroll
      for (int e = 0; e < V; ++e)
        acc[e] = OP == kOpCountEq ? acc[e] + (v[e] == rv[e] ? 1.f : 0.f) : gop<OP>(acc[e], v[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < V; ++e)
    red[threadIdx.x * V + e] = acc[e];
  __syncthreads();
  if (active && rlane == 0) {
    for (int r = 1; r < rl; ++r)
#pragma unroll
      for (int e = 0; e < V; ++e)
        acc[e] = gop<OP == kOpMax ? kOpMax : kOpSum>(acc[e], red[(r * lpt + lane) * V + e]);
    Slice<float, V>::store(partial + g * C + c0, acc);
  }
}

// Stage 2: block (b, tile) combines the partials of batch b in order.
//   sum: y = total; average: y = total / rows (0 for an empty batch);
//   max: y = total (0 for an empty batch); count: gs = gy / total (0 if 0).
template <typename T, int OP, int V>
__global__ __launch_bounds__(kPoolThreads) void gpool_final_kernel(
    const float *__restrict__ partial, int C, int lpr, int lpt, const int32_t *__restrict__ seg,
    const int64_t *__restrict__ base, int mode, const T *__restrict__ gy, T *__restrict__ y,
    float *__restrict__ gs) {
  __shared__ float red[kPoolThreads * V];
  const int b = blockIdx.x;
  const int lane = threadIdx.x % lpt, rlane = threadIdx.x / lpt, rl = kPoolThreads / lpt;
  const int cc = blockIdx.y * lpt + lane;
  const bool active = cc < lpr && rlane < rl;
  const int c0 = cc * V;
  constexpr int COMB = OP == kOpMax ? kOpMax : kOpSum;
  float acc[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    acc[e] = gop_init<COMB>();
  if (active) {
    for (int64_t g = base[b] + rlane; g < base[b + 1]; g += rl) {
      float v[V];
      Slice<float, V>::load(partial + g * C + c0, v);
#pragma unroll
      for (int e = 0; e < V; ++e)
        acc[e] = gop<COMB>(acc[e], v[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < V; ++e)
    red[threadIdx.x * V + e] = acc[e];
  __syncthreads();
  if (!(active && rlane == 0))
    return;
  for (int r = 1; r < rl; ++r)
#pragma unroll
    for (int e = 0; e < V; ++e)
      acc[e] = gop<COMB>(acc[e], red[(r * lpt + lane) * V + e]);
  const int rows = seg[b + 1] - seg[b];
  float out[V];
  if (OP == kOpCountEq) {
    float g[V];
    Slice<T, V>::load(gy + static_cast<int64_t>(b) * C + c0, g);
#pragma unroll
    for (int e = 0; e < V; ++e)
      out[e] = acc[e] > 0.f ? g[e] / acc[e] : 0.f;
    Slice<float, V>::store(gs + static_cast<int64_t>(b) * C + c0, out);
    return;
  }
#pragma unroll
  for (int e = 0; e < V; ++e)
    out[e] = rows == 0 ? 0.f
                       : (mode == RHIP_POOL_AVG ? acc[e] / static_cast<float>(rows) : acc[e]);
  Slice<T, V>::store(y + static_cast<int64_t>(b) * C + c0, out);
}

// gx[i] for row i of batch b = coords[i][0]: sum gy[b]; average gy[b] / rows;
// max gs[b] where x[i] == y[b]; 0 for a batch outside [0, B).
template <typename T, int MODE, int V>
__global__ __launch_bounds__(kPoolThreads) void gpool_bwd_kernel(
    const T *__restrict__ gy, const float *__restrict__ gs, const T *__restrict__ x,
    const T *__restrict__ y, const int32_t *__restrict__ coords, int ncol, int64_t n, int C,
    int lpr, const int32_t *__restrict__ seg, int32_t B, T *__restrict__ gx) {
  const int64_t t = blockIdx.x * static_cast<int64_t>(kPoolThreads) + threadIdx.x;
  const int64_t i = t / lpr;
  if (i >= n)
    return;
  const int c0 = static_cast<int>(t - i * lpr) * V;
  const int32_t b = coords[i * ncol];
  float out[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    out[e] = 0.f;
  if (b >= 0 && b < B) {
    if (MODE == RHIP_POOL_MAX) {
      float xv[V], yv[V], s[V];
      Slice<T, V>::load(x + i * C + c0, xv);
      Slice<T, V>::load(y + static_cast<int64_t>(b) * C + c0, yv);
      Slice<float, V>::load(gs + static_cast<int64_t>(b) * C + c0, s);
#pragma unroll
      for (int e = 0; e < V; ++e)
        out[e] = xv[e] == yv[e] ? s[e] : 0.f;
    } else {
      Slice<T, V>::load(gy + static_cast<int64_t>(b) * C + c0, out);
      if (MODE == RHIP_POOL_AVG) {
        const float rows = static_cast<float>(seg[b + 1] - seg[b]);
#pragma unroll
        for (int e = 0; e < V; ++e)
          out[e] /= rows;
      }
    }
  }
  Slice<T, V>::store(gx + i * C + c0, out);
}

// ------------------------------------------------------------------ host

void check_dtype(int32_t dtype) {
  if (dtype != RHIP_F32 && dtype != RHIP_BF16)
    throw Error(RHIP_ERR_UNSUPPORTED, "dtype must be RHIP_F32 or RHIP_BF16");
}

void check_mode(int32_t mode, bool local = true) {
  if (mode != RHIP_POOL_SUM && mode != RHIP_POOL_AVG && mode != RHIP_POOL_MAX &&
      !(local && mode == RHIP_POOL_MAX_SCATTER))
    throw Error(RHIP_ERR_INVALID, local ? "mode must be RHIP_POOL_SUM, _AVG, _MAX or _MAX_SCATTER"
                                        : "mode must be RHIP_POOL_SUM, _AVG or _MAX");
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Elements per lane: one 16-byte slice when every row starts 16-byte aligned.
template <typename T> int slice_width(int C, std::initializer_list<const void *> ptrs) {
  constexpr int W = 16 / sizeof(T);
  if ((C % W) != 0)
    return 1;
  for (const void *p : ptrs)
    if (p != nullptr && !aligned16(p))
      return 1;
  return W;
}

unsigned grid_for(int64_t threads) {
  const int64_t blocks = ceil_div(threads, kPoolThreads);
  if (blocks > INT_MAX)
    throw Error(RHIP_ERR_UNSUPPORTED, "launch exceeds the grid limit");
  return static_cast<unsigned>(blocks < 1 ? 1 : blocks);
}

// Workgroups of the local-pooling kernels: whole XCD runs (pool_thread).
unsigned pool_grid(int64_t threads) {
  const int64_t blocks = xcd_grid(ceil_div(std::max<int64_t>(threads, 1), kPoolThreads));
  if (blocks > INT_MAX)
    throw Error(RHIP_ERR_UNSUPPORTED, "launch exceeds the grid limit");
  return static_cast<unsigned>(blocks);
}

// Dispatch f<V>() on the slice width.
template <typename T, typename F> void with_width(int V, F &&f) {
  if (V == 1)
    f(std::integral_constant<int, 1>{});
  else
    f(std::integral_constant<int, 16 / sizeof(T)>{});
}
// RHIP_POOL_MAX_SCATTER runs the max kernels (its zero tie is a flag).
template <typename F> void with_mode(int32_t mode, F &&f) {
  if (mode == RHIP_POOL_SUM)
    f(std::integral_constant<int, RHIP_POOL_SUM>{});
  else if (mode == RHIP_POOL_AVG)
    f(std::integral_constant<int, RHIP_POOL_AVG>{});
  else
    f(std::integral_constant<int, RHIP_POOL_MAX>{});
}

// --- stride map workspace
struct StrideWs {
  uint32_t *keys, *skeys;
  int32_t *vals, *svals, *rank, *start, *kmax, *pos_in, *pos_out;
  unsigned long long *miss;
  void *sort_tmp;
  size_t sort_bytes;
};

StrideWs carve_stride(Carve &cv, int64_t n_in, int64_t n_out) {
  StrideWs w{};
  const int64_t n = std::max<int64_t>(n_in, 1);
  w.keys = cv.take<uint32_t>(n);
  w.skeys = cv.take<uint32_t>(n);
  w.vals = cv.take<int32_t>(n);
  w.svals = cv.take<int32_t>(n);
  w.rank = cv.take<int32_t>(n);
  w.start = cv.take<int32_t>(std::max<int64_t>(n_out, 1));
  w.kmax = cv.take<int32_t>(1);
  w.pos_in = cv.take<int32_t>(n);
  w.pos_out = cv.take<int32_t>(std::max<int64_t>(n_out, 1));
  w.miss = cv.take<unsigned long long>(2);
  w.sort_bytes = sort_pairs_u32_bytes(n);
  w.sort_tmp = cv.take<char>(w.sort_bytes);
  return w;
}

// --- global pooling workspace
int lanes_per_row(int C, int V) { return (C + V - 1) / V; }
int lanes_per_tile(int lpr) { return std::min(lpr, kPoolThreads); }
int rows_per_chunk(int lpr) { return (kPoolThreads / lanes_per_tile(lpr)) * kRowsPerLane; }

struct GlobalWs {
  uint32_t *keys, *skeys;
  int32_t *vals, *bmax;
  void *sort_tmp;
  size_t sort_bytes;
  int64_t *nchunk, *base;
  float *partial, *gs;
};

// Chunks are sized for the narrowest lane layout (V = 1), which has the most.
GlobalWs carve_global(Carve &cv, int64_t n, int C, int32_t B) {
  GlobalWs w{};
  const int64_t m = std::max<int64_t>(n, 1);
  w.keys = cv.take<uint32_t>(m);
  w.skeys = cv.take<uint32_t>(m);
  w.vals = cv.take<int32_t>(m);
  w.bmax = cv.take<int32_t>(1);
  w.sort_bytes = sort_pairs_u32_bytes(m);
  w.sort_tmp = cv.take<char>(w.sort_bytes);
  const int64_t Bm = std::max<int32_t>(B, 1);
  w.nchunk = cv.take<int64_t>(Bm);
  w.base = cv.take<int64_t>(Bm + 1);
  const int R = rows_per_chunk(lanes_per_row(std::max(C, 1), 1));
  const int64_t chunks = ceil_div(m, R) + Bm;
  w.partial = cv.take<float>(chunks * std::max(C, 1));
  w.gs = cv.take<float>(Bm * std::max(C, 1));
  return w;
}

// Chunk table then both reduction stages; OP picks the reduction.
template <typename T, int OP, int V>
void global_reduce(const T *x, const T *ref, int C, const int32_t *members, const int32_t *seg,
                   int32_t B, int mode, const T *gy, T *y, GlobalWs &w, int64_t n,
                   hipStream_t s) {
  const int lpr = lanes_per_row(C, V), lpt = lanes_per_tile(lpr);
  const int R = rows_per_chunk(lpr);
  const unsigned tiles = static_cast<unsigned>(ceil_div(lpr, lpt));
  hipLaunchKernelGGL(chunk_count_kernel, dim3(grid_for(B)), dim3(kPoolThreads), 0, s, seg, B, R,
                     w.nchunk);
  RHIP_LAUNCH_CHECK();
  hipLaunchKernelGGL((scan_kernel<int64_t>), dim3(1), dim3(1024), 0, s, w.nchunk,
                     static_cast<int64_t>(B), w.base, w.base + B);
  RHIP_LAUNCH_CHECK();
  const int64_t max_chunks = ceil_div(std::max<int64_t>(n, 1), R) + B;
  if (max_chunks > INT_MAX)
    throw Error(RHIP_ERR_UNSUPPORTED, "too many rows for one global pooling launch");
  hipLaunchKernelGGL((gpool_partial_kernel<T, OP, V>), dim3(static_cast<unsigned>(max_chunks), tiles),
                     dim3(kPoolThreads), 0, s, x, ref, C, lpr, lpt, members, seg, w.base, B, R,
                     w.partial);
  RHIP_LAUNCH_CHECK();
  hipLaunchKernelGGL((gpool_final_kernel<T, OP, V>), dim3(static_cast<unsigned>(B), tiles),
                     dim3(kPoolThreads), 0, s, w.partial, C, lpr, lpt, seg, w.base, mode, gy, y,
                     w.gs);
  RHIP_LAUNCH_CHECK();
}

// Shared tail of the stride-map and group-map counts: sort (key, row) by key,
// rank rows within their key's group, read back the miss count and the
// largest group (one synchronisation). `message(row, count)` names a miss.
template <typename Msg>
int32_t group_rows(StrideWs &w, int64_t n, int64_t n_groups, hipStream_t stream, Msg message) {
  const unsigned grid = grid_for(n);
  sort_pairs_u32(w.sort_tmp, w.sort_bytes, w.keys, w.skeys, w.vals, w.svals, n,
                 bit_width_u64(static_cast<uint64_t>(n_groups - 1)), stream);
  hipLaunchKernelGGL(group_start_kernel, dim3(grid), dim3(kPoolThreads), 0, stream, w.skeys, n,
                     w.start);
  RHIP_LAUNCH_CHECK();
  hipLaunchKernelGGL(group_rank_kernel, dim3(std::min<unsigned>(grid, kReduceBlocks)),
                     dim3(kPoolThreads), 0, stream, w.skeys, n, w.start, w.rank, w.kmax);
  RHIP_LAUNCH_CHECK();
  unsigned long long miss[2];
  int32_t kmax = 0;
  RHIP_HIP(hipMemcpyAsync(miss, w.miss, sizeof(miss), hipMemcpyDeviceToHost, stream));
  RHIP_HIP(hipMemcpyAsync(&kmax, w.kmax, sizeof(kmax), hipMemcpyDeviceToHost, stream));
  RHIP_HIP(hipStreamSynchronize(stream));
  if (miss[0] != 0)
    throw Error(RHIP_ERR_INVALID, message(miss[1], miss[0]));
  const int64_t cells = static_cast<int64_t>(kmax) * std::max(n, n_groups);
  if (cells > (int64_t{1} << 31))
    throw Error(RHIP_ERR_UNSUPPORTED, std::to_string(kmax) +
                                          " rows in one group make the neighbour table too large");
  return kmax;
}

} // namespace
} // namespace rhip

using namespace rhip;

// ------------------------------------------------------------ stride map

extern "C" int rhip_stride_map_workspace_bytes(int64_t n_in, int64_t n_out, size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "counts must be >= 0");
    Carve cv(nullptr, 0);
    carve_stride(cv, n_in, n_out);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_stride_map_count(const rhip_table *out_table, const int32_t *in_coords,
                                     int64_t n_in, const int32_t *out_tensor_stride,
                                     void *workspace, size_t ws_bytes, int32_t *k_max_host,
                                     hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(out_table != nullptr && k_max_host != nullptr && out_tensor_stride != nullptr,
                   "out_table, out_tensor_stride and k_max_host are required");
    RHIP_CHECK_ARG(n_in >= 0 && n_in < INT_MAX, "n_in must be in [0, 2^31)");
    const int ncol = out_table->ncol;
    RHIP_CHECK_ARG(ncol >= 1 && ncol <= RHIP_MAX_COLS, "bad column count");
    StrideArg st{};
    for (int j = 0; j < ncol - 1; ++j) {
      RHIP_CHECK_ARG(out_tensor_stride[j] >= 1, "tensor stride must be positive");
      st.s[j] = out_tensor_stride[j];
    }
    *k_max_host = 0;
    if (n_in == 0)
      return;
    RHIP_CHECK_ARG(in_coords != nullptr && workspace != nullptr, "in_coords and workspace required");
    const int64_t n_out = out_table->n_unique;
    RHIP_CHECK_ARG(n_out >= 1, "output map is empty but inputs are not");
    Carve cv(workspace, ws_bytes);
    StrideWs w = carve_stride(cv, n_in, n_out);
    const unsigned grid = grid_for(n_in);
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(kPoolThreads), 0, stream, w.kmax, 1, 0);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(miss_init_kernel, dim3(1), dim3(kWave), 0, stream, w.miss);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(stride_lookup_kernel, dim3(grid), dim3(kPoolThreads), 0, stream,
                       make_view(*out_table), in_coords, n_in, st, w.keys, w.vals, w.miss);
    RHIP_LAUNCH_CHECK();
    *k_max_host = group_rows(w, n_in, n_out, stream, [](unsigned long long row,
                                                        unsigned long long count) {
      return "Invalid out_coordinate_map: input row " + std::to_string(row) +
             " has no floor-aligned output row (" + std::to_string(count) + " such rows)";
    });
  });
}

extern "C" int rhip_group_map_count(const int32_t *group, int64_t n, int64_t n_groups,
                                    void *workspace, size_t ws_bytes, int32_t *k_max_host,
                                    hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(k_max_host != nullptr, "k_max_host is null");
    RHIP_CHECK_ARG(n >= 0 && n < INT_MAX && n_groups >= 0 && n_groups < INT_MAX, "bad sizes");
    *k_max_host = 0;
    if (n == 0)
      return;
    RHIP_CHECK_ARG(n_groups >= 1, "rows but no groups");
    RHIP_CHECK_ARG(group != nullptr && workspace != nullptr, "group and workspace required");
    Carve cv(workspace, ws_bytes);
    StrideWs w = carve_stride(cv, n, n_groups);
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(kPoolThreads), 0, stream, w.kmax, 1, 0);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(miss_init_kernel, dim3(1), dim3(kWave), 0, stream, w.miss);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(group_keys_kernel, dim3(grid_for(n)), dim3(kPoolThreads), 0, stream, group,
                       n, n_groups, w.keys, w.vals, w.miss);
    RHIP_LAUNCH_CHECK();
    *k_max_host = group_rows(w, n, n_groups, stream, [](unsigned long long row,
                                                        unsigned long long count) {
      return "group of row " + std::to_string(row) + " is outside [0, n_groups) (" +
             std::to_string(count) + " such rows)";
    });
  });
}

extern "C" int rhip_stride_map_fill(int64_t n_in, int64_t n_out, int32_t k_max,
                                    const int32_t *in_order, const int32_t *out_order,
                                    void *workspace, size_t ws_bytes, int32_t *nbr,
                                    int32_t *nbr_t, int32_t *in_rows, int32_t *out_rows,
                                    hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0 && k_max >= 0, "counts must be >= 0");
    RHIP_CHECK_ARG(n_in == 0 || k_max >= 1, "k_max must come from rhip_stride_map_count");
    if (k_max == 0)
      return;
    RHIP_CHECK_ARG(nbr && nbr_t && in_rows && out_rows && workspace, "outputs are required");
    Carve cv(workspace, ws_bytes);
    StrideWs w = carve_stride(cv, n_in, n_out);
    const int64_t nn = static_cast<int64_t>(k_max) * n_out;
    hipLaunchKernelGGL(fill_i32_kernel, dim3(grid_for(nn)), dim3(kPoolThreads), 0, stream, nbr, nn,
                       -1);
    RHIP_LAUNCH_CHECK();
    if (in_order != nullptr) {
      hipLaunchKernelGGL(invert_order_kernel, dim3(grid_for(n_in)), dim3(kPoolThreads), 0,
                         stream, in_order, n_in, w.pos_in);
      RHIP_LAUNCH_CHECK();
    }
    if (out_order != nullptr) {
      hipLaunchKernelGGL(invert_order_kernel, dim3(grid_for(n_out)), dim3(kPoolThreads), 0,
                         stream, out_order, n_out, w.pos_out);
      RHIP_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(stride_scatter_kernel, dim3(grid_for(n_in)), dim3(kPoolThreads), 0, stream,
                       w.skeys, w.svals, w.rank, n_in, n_out, k_max,
                       in_order ? w.pos_in : nullptr, out_order ? w.pos_out : nullptr, nbr,
                       nbr_t, in_rows, out_rows);
    RHIP_LAUNCH_CHECK();
  });
}

// ---------------------------------------------------------- local pooling

extern "C" int rhip_pool_workspace_bytes(int64_t n_out, int32_t C, int32_t mode, size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n_out >= 0 && C >= 1, "bad sizes");
    check_mode(mode);
    *bytes = mode >= RHIP_POOL_MAX ? align_up(sizeof(float) * n_out * C, 256) + 256 : 256;
  });
}

extern "C" int rhip_pool_forward(const void *x, int64_t n_in, int32_t C, const int32_t *nbr,
                                 int32_t K, const int32_t *out_order, int64_t n_out, int32_t mode,
                                 void *y, int32_t *counts, int32_t dtype, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    check_mode(mode);
    RHIP_CHECK_ARG(C >= 1 && K >= 0 && n_in >= 0 && n_out >= 0, "bad sizes");
    if (n_out == 0)
      return;
    RHIP_CHECK_ARG(y != nullptr, "y is null");
    RHIP_CHECK_ARG(K == 0 || nbr != nullptr, "nbr is null");
    RHIP_CHECK_ARG(n_in == 0 || x != nullptr, "x is null");
    auto launch = [&](auto tag) {
      using T = decltype(tag);
      const int V = slice_width<T>(C, {x, y});
      with_mode(mode, [&](auto m) {
        with_width<T>(V, [&](auto v) {
          constexpr int M = decltype(m)::value, W = decltype(v)::value;
          const int lpr = C / W;
          hipLaunchKernelGGL((pool_fwd_kernel<T, M, W>), dim3(pool_grid(n_out * lpr)),
                             dim3(kPoolThreads), 0, stream, static_cast<const T *>(x), C, lpr,
                             nbr, K, n_out, out_order, static_cast<T *>(y), counts);
          RHIP_LAUNCH_CHECK();
        });
      });
    };
    if (dtype == RHIP_F32)
      launch(float{});
    else
      launch(__bf16{});
  });
}

extern "C" int rhip_pool_backward(const void *grad_y, const void *y, const void *x, int64_t n_out,
                                  int32_t C, const int32_t *nbr, int32_t K,
                                  const int32_t *out_order, const int32_t *nbr_t, int32_t K_t,
                                  const int32_t *in_order, int64_t n_in, const int32_t *counts,
                                  int32_t mode, void *grad_x, int32_t dtype, void *workspace,
                                  size_t ws_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    check_mode(mode);
    RHIP_CHECK_ARG(C >= 1 && K >= 0 && K_t >= 0 && n_in >= 0 && n_out >= 0, "bad sizes");
    if (n_in == 0)
      return;
    RHIP_CHECK_ARG(grad_x != nullptr, "grad_x is null");
    RHIP_CHECK_ARG(K_t == 0 || nbr_t != nullptr, "nbr_t is null");
    RHIP_CHECK_ARG(n_out == 0 || grad_y != nullptr, "grad_y is null");
    RHIP_CHECK_ARG(mode != RHIP_POOL_AVG || n_out == 0 || counts != nullptr,
                   "average pooling needs the forward counts");
    RHIP_CHECK_ARG(mode < RHIP_POOL_MAX || n_out == 0 ||
                       (x != nullptr && y != nullptr && nbr != nullptr && workspace != nullptr),
                   "max pooling needs x, y, nbr and the workspace");
    float *gs = nullptr;
    if (mode >= RHIP_POOL_MAX) {
      Carve cv(workspace, ws_bytes);
      gs = cv.take<float>(std::max<int64_t>(n_out, 1) * C);
    }
    auto launch = [&](auto tag) {
      using T = decltype(tag);
      const int V = slice_width<T>(C, {x, y, grad_y, grad_x});
      with_mode(mode, [&](auto m) {
        with_width<T>(V, [&](auto v) {
          constexpr int M = decltype(m)::value, W = decltype(v)::value;
          const int lpr = C / W;
          if (M == RHIP_POOL_MAX && n_out > 0) {
            hipLaunchKernelGGL((pool_maxshare_kernel<T, W>), dim3(pool_grid(n_out * lpr)),
                               dim3(kPoolThreads), 0, stream, static_cast<const T *>(grad_y),
                               static_cast<const T *>(x), static_cast<const T *>(y), C, lpr, nbr,
                               K, n_out, out_order, mode == RHIP_POOL_MAX_SCATTER ? 1 : 0, gs);
            RHIP_LAUNCH_CHECK();
          }
          hipLaunchKernelGGL((pool_bwd_kernel<T, M, W>), dim3(pool_grid(n_in * lpr)),
                             dim3(kPoolThreads), 0, stream, static_cast<const T *>(grad_y), gs,
                             static_cast<const T *>(x), static_cast<const T *>(y), C, lpr,
                             nbr_t, n_out == 0 ? 0 : K_t, n_in, in_order, counts,
                             static_cast<T *>(grad_x));
          RHIP_LAUNCH_CHECK();
        });
      });
    };
    if (dtype == RHIP_F32)
      launch(float{});
    else
      launch(__bf16{});
  });
}

extern "C" int rhip_table_compact(const int32_t *table, int32_t K, int64_t n, void *workspace,
                                  size_t ws_bytes, int32_t *out, int32_t *k_used_host,
                                  hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(k_used_host != nullptr, "k_used_host is null");
    RHIP_CHECK_ARG(K >= 1 && n >= 0, "bad sizes");
    *k_used_host = 0;
    if (n == 0)
      return;
    RHIP_CHECK_ARG(table && out && workspace, "table, out and workspace are required");
    RHIP_CHECK_ARG(table != out, "table and out must not alias");
    RHIP_CHECK_ARG(ws_bytes >= sizeof(int32_t), "workspace too small");
    int32_t *kmax = static_cast<int32_t *>(workspace);
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(kPoolThreads), 0, stream, kmax, 1, 0);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(table_compact_kernel, dim3(std::min<unsigned>(grid_for(n), kReduceBlocks)),
                       dim3(kPoolThreads), 0, stream, table, K, n, out, kmax);
    RHIP_LAUNCH_CHECK();
    int32_t used = 0;
    RHIP_HIP(hipMemcpyAsync(&used, kmax, sizeof(used), hipMemcpyDeviceToHost, stream));
    RHIP_HIP(hipStreamSynchronize(stream));
    *k_used_host = used;
  });
}

// --------------------------------------------------------- global pooling

extern "C" int rhip_global_pool_workspace_bytes(int64_t n, int32_t C, int32_t n_batches,
                                                size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n >= 0 && C >= 1 && n_batches >= 0, "bad sizes");
    Carve cv(nullptr, 0);
    carve_global(cv, n, C, n_batches);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_batch_count(const int32_t *coords, int64_t n, int32_t ncol, void *workspace,
                                size_t ws_bytes, int32_t *n_batches_host, hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(n_batches_host != nullptr, "n_batches_host is null");
    RHIP_CHECK_ARG(n >= 0 && n < INT_MAX && ncol >= 1 && ncol <= RHIP_MAX_COLS, "bad sizes");
    *n_batches_host = 0;
    if (n == 0)
      return;
    RHIP_CHECK_ARG(coords != nullptr && workspace != nullptr, "coords and workspace required");
    Carve cv(workspace, ws_bytes);
    GlobalWs w = carve_global(cv, n, 1, 0);
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(kPoolThreads), 0, stream, w.bmax, 1,
                       INT_MIN);
    RHIP_LAUNCH_CHECK();
    hipLaunchKernelGGL(batch_max_kernel, dim3(std::min<unsigned>(grid_for(n), kReduceBlocks)),
                       dim3(kPoolThreads), 0, stream, coords, n, ncol, w.bmax);
    RHIP_LAUNCH_CHECK();
    int32_t bmax = 0;
    RHIP_HIP(hipMemcpyAsync(&bmax, w.bmax, sizeof(bmax), hipMemcpyDeviceToHost, stream));
    RHIP_HIP(hipStreamSynchronize(stream));
    if (bmax >= (1 << 30))
      throw Error(RHIP_ERR_UNSUPPORTED, "batch index " + std::to_string(bmax) + " is too large");
    *n_batches_host = bmax < 0 ? 0 : bmax + 1;
  });
}

extern "C" int rhip_batch_segments(const int32_t *coords, int64_t n, int32_t ncol,
                                   int32_t n_batches, void *workspace, size_t ws_bytes,
                                   int32_t *members, int32_t *seg, hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(n >= 0 && n < INT_MAX && ncol >= 1 && ncol <= RHIP_MAX_COLS, "bad sizes");
    RHIP_CHECK_ARG(n_batches >= 0 && n_batches < (1 << 30), "bad batch count");
    RHIP_CHECK_ARG(seg != nullptr, "seg is null");
    if (n == 0) {
      hipLaunchKernelGGL(fill_i32_kernel, dim3(grid_for(n_batches + 1)), dim3(kPoolThreads), 0,
                         stream, seg, static_cast<int64_t>(n_batches) + 1, 0);
      RHIP_LAUNCH_CHECK();
      return;
    }
    RHIP_CHECK_ARG(coords && members && workspace, "coords, members and workspace required");
    Carve cv(workspace, ws_bytes);
    GlobalWs w = carve_global(cv, n, 1, 0);
    hipLaunchKernelGGL(batch_keys_kernel, dim3(grid_for(n)), dim3(kPoolThreads), 0, stream, coords,
                       n, ncol, n_batches, w.keys, w.vals);
    RHIP_LAUNCH_CHECK();
    sort_pairs_u32(w.sort_tmp, w.sort_bytes, w.keys, w.skeys, w.vals, members, n,
                   bit_width_u64(static_cast<uint64_t>(n_batches)), stream);
    hipLaunchKernelGGL(batch_bounds_kernel, dim3(grid_for(n + 1)), dim3(kPoolThreads), 0, stream,
                       w.skeys, n, n_batches, seg);
    RHIP_LAUNCH_CHECK();
  });
}

extern "C" int rhip_global_pool_forward(const void *x, int64_t n, int32_t C,
                                        const int32_t *members, const int32_t *seg,
                                        int32_t n_batches, int32_t mode, void *y, int32_t dtype,
                                        void *workspace, size_t ws_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    check_mode(mode, false);
    RHIP_CHECK_ARG(n >= 0 && C >= 1 && n_batches >= 0, "bad sizes");
    if (n_batches == 0)
      return;
    RHIP_CHECK_ARG(y && seg && workspace, "y, seg and workspace are required");
    RHIP_CHECK_ARG(n == 0 || (x != nullptr && members != nullptr), "x and members are required");
    Carve cv(workspace, ws_bytes);
    GlobalWs w = carve_global(cv, n, C, n_batches);
    auto launch = [&](auto tag) {
      using T = decltype(tag);
      const int V = slice_width<T>(C, {x, y});
      with_width<T>(V, [&](auto v) {
        constexpr int W = decltype(v)::value;
        const T *xt = static_cast<const T *>(x);
        T *yt = static_cast<T *>(y);
        if (mode == RHIP_POOL_MAX)
          global_reduce<T, kOpMax, W>(xt, nullptr, C, members, seg, n_batches, mode, nullptr, yt,
                                      w, n, stream);
        else
          global_reduce<T, kOpSum, W>(xt, nullptr, C, members, seg, n_batches, mode, nullptr, yt,
                                      w, n, stream);
      });
    };
    if (dtype == RHIP_F32)
      launch(float{});
    else
      launch(__bf16{});
  });
}

extern "C" int rhip_global_pool_backward(const void *grad_y, const void *y, const void *x,
                                         const int32_t *coords, int32_t ncol, int64_t n, int32_t C,
                                         const int32_t *members, const int32_t *seg,
                                         int32_t n_batches, int32_t mode, void *grad_x,
                                         int32_t dtype, void *workspace, size_t ws_bytes,
                                         hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    check_mode(mode, false);
    RHIP_CHECK_ARG(n >= 0 && C >= 1 && n_batches >= 0 && ncol >= 1 && ncol <= RHIP_MAX_COLS,
                   "bad sizes");
    if (n == 0)
      return;
    RHIP_CHECK_ARG(grad_x && coords && seg, "grad_x, coords and seg are required");
    RHIP_CHECK_ARG(n_batches == 0 || grad_y != nullptr, "grad_y is null");
    RHIP_CHECK_ARG(mode != RHIP_POOL_MAX || n_batches == 0 ||
                       (x && y && members && workspace),
                   "max pooling needs x, y, members and the workspace");
    GlobalWs w{};
    if (mode == RHIP_POOL_MAX && n_batches > 0) {
      Carve cv(workspace, ws_bytes);
      w = carve_global(cv, n, C, n_batches);
    }
    auto launch = [&](auto tag) {
      using T = decltype(tag);
      const int V = slice_width<T>(C, {x, y, grad_y, grad_x});
      with_mode(mode, [&](auto m) {
        with_width<T>(V, [&](auto v) {
          constexpr int M = decltype(m)::value, W = decltype(v)::value;
          const int lpr = C / W;
          if (M == RHIP_POOL_MAX && n_batches > 0)
            global_reduce<T, kOpCountEq, W>(static_cast<const T *>(x), static_cast<const T *>(y),
                                            C, members, seg, n_batches, mode,
                                            static_cast<const T *>(grad_y), nullptr, w, n, stream);
          hipLaunchKernelGGL((gpool_bwd_kernel<T, M, W>), dim3(grid_for(n * lpr)),
                             dim3(kPoolThreads), 0, stream, static_cast<const T *>(grad_y), w.gs,
                             static_cast<const T *>(x), static_cast<const T *>(y), coords, ncol, n,
                             C, lpr, seg, n_batches, static_cast<T *>(grad_x));
          RHIP_LAUNCH_CHECK();
        });
      });
    };
    if (dtype == RHIP_F32)
      launch(float{});
    else
      launch(__bf16{});
  });
}
