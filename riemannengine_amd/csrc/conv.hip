// Sparse convolution on gfx950 MFMA (fp32 and bf16 inputs, fp32 accumulate).
//
// Reference semantics (RiemannEngine/engine/nn/conv.cpp:47-64):
//   Y = 0; for k: Y.index_add_(0, out_k, X[in_k] @ W[k]);  Y += bias
// with the backward produced by LibTorch autograd:
//   dX = sum_k scatter_add(in_k, dY[out_k] @ W[k]^T),
//   dW[k] = X[in_k]^T @ dY[out_k].
//
// MI355X design:
//  * Forward and dX are one output-stationary implicit GEMM over the dense
//    neighbour table of the kernel map, whose rows come grouped by neighbour
//    mask (so a 16-row group rarely multiplies a missing neighbour). A
//    256-thread workgroup owns 128 output rows (4 waves x 2 groups of 16) and
//    up to 64 columns. It walks only the offsets with a neighbour in its rows;
//    for each it stages the weight slice in LDS with 16-byte copies from a
//    [K][ncols][cred] copy of the weights (reduction axis contiguous), gathers
//    each group's 16 neighbour rows straight into MFMA A-fragments (16-byte
//    loads, zero for a missing neighbour) and accumulates every offset in
//    registers. Each output row is written once: no atomics, no zero fill.
//  * dW is a split-pair reduction over the per-offset pair lists: a
//    workgroup stages 64 pairs of X and dY rows in LDS transposed (pair axis
//    contiguous), runs 16x16 MFMA tiles with pairs as the reduction axis and
//    adds each offset segment's tile to an fp32 accumulator with atomics.
//  * The reduction order inside an MFMA is a permutation of the reduced axis
//    chosen so that each lane reads 16 contiguous bytes; A and B use the same
//    permutation, so the sum is unchanged.
#include <algorithm>
#include <type_traits>

#include "rhip_internal.hpp"

namespace rhip {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaskWords = 4; // the MFMA paths handle K <= 128 offsets
constexpr int kXcds = 8;      // MI355X: 8 XCDs, workgroups dealt round-robin

template <typename T> struct Mfma;

// v_mfma_f32_16x16x4_f32: lane l supplies A[l%16][l/16], B[l/16][l%16];
// D[4*(l/16)+e][l%16] lands in element e. A 16-byte lane load covers four
// consecutive channels, consumed by four MFMAs.
template <> struct Mfma<float> {
  static constexpr int kCh = 16; // channels per wave-wide 16-byte load
  using Frag = v4f;
  __device__ static __forceinline__ Frag load(const float *p) {
    return *reinterpret_cast<const v4f *>(p);
  }
  __device__ static __forceinline__ Frag zero() { return v4f{0.f, 0.f, 0.f, 0.f}; }
  __device__ static __forceinline__ void mma(const Frag &a, const Frag &b, v4f &c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[3], b[3], c, 0, 0, 0);
  }
};

// v_mfma_f32_16x16x32_bf16 (gfx950): lane l supplies eight consecutive
// reduction elements of row l%16 (A) / column l%16 (B), group l/16.
template <> struct Mfma<__bf16> {
  static constexpr int kCh = 32;
  using Frag = v8bf;
  __device__ static __forceinline__ Frag load(const __bf16 *p) {
    return *reinterpret_cast<const v8bf *>(p);
  }
  __device__ static __forceinline__ Frag zero() {
    return __builtin_bit_cast(v8bf, uint4{0u, 0u, 0u, 0u});
  }
  __device__ static __forceinline__ void mma(const Frag &a, const Frag &b, v4f &c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(__bf16 v) { return static_cast<float>(v); }
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) {
  return static_cast<__bf16>(v);
}

// Workgroup id -> tile id. Workgroups are dealt to the 8 XCDs round-robin
// (id b runs on XCD b % 8); this mapping hands each XCD runs of kXcdRun
// consecutive tiles, so tiles that share neighbour rows share an L2, while
// the runs stay interleaved over the whole map to keep the XCDs balanced.
// The grid is padded to a multiple of 8 * kXcdRun (padding ids map past the
// last tile).
constexpr int kXcdRun = 16;
__device__ __forceinline__ int64_t xcd_tile(int64_t b) {
  const int64_t x = b % kXcds, m = b / kXcds;
  return ((m / kXcdRun) * kXcds + x) * kXcdRun + (m % kXcdRun);
}
inline int64_t xcd_grid(int64_t tiles) {
  return ceil_div(tiles, kXcds * kXcdRun) * kXcds * kXcdRun;
}

// ------------------------------------------------ output-stationary GEMM
//
// y[order[j]][col] = sum_k sum_c x[nbr[k][j]][c] * wt[k][col][c] (+ bias[col])
// wt is [K][ncols][cred] (reduction axis contiguous). A workgroup owns
// 4 * RG * 16 output rows and NT columns; RG: 16-row groups per wave; CSUB:
// 16-byte lane loads per staged channel chunk (chunk = CSUB * kCh channels).
template <typename T, int NT, int RG, int CSUB>
__global__ __launch_bounds__(kThreads) void conv_os_kernel(
    const T *__restrict__ x, int cred, const T *__restrict__ wt, int ncols,
    const float *__restrict__ bias, const int32_t *__restrict__ nbr,
    int64_t n_rows, int K, const int32_t *__restrict__ order,
    T *__restrict__ y) {
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  constexpr int CH = M::kCh;
  constexpr int EPL = CH / 4;            // elements per lane per load
  constexpr int VE = 16 / sizeof(T);     // elements per 16 bytes
  constexpr int CCH = CSUB * CH;         // channels per staged chunk
  constexpr int LDW = CCH + VE;          // LDS row stride (elements)
  constexpr int ROWS = kWaves * RG * 16; // output rows per workgroup
  constexpr int NB = NT / 16;
  constexpr int NV = NT * (CCH / VE);    // 16-byte pieces per staged chunk
  constexpr int NPT = (NV + kThreads - 1) / kThreads;

  __shared__ __align__(16) T sB[NT * LDW];
  __shared__ uint32_t smask[kWaves * RG][kMaskWords];
  __shared__ int32_t slist[32 * kMaskWords];
  __shared__ int32_t scount;

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int64_t tile = xcd_tile(blockIdx.x);
  const int64_t tile0 = tile * ROWS;
  if (tile0 >= n_rows)
    return; // padding workgroup (uniform)
  const int col0 = blockIdx.y * NT;

  // Offsets with any neighbour in each 16-row group: lanes of group g test
  // offset k0+g for the 16 rows; one ballot covers four offsets.
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const int64_t pos = tile0 + (wv * RG + r) * 16 + i16;
    uint32_t words[kMaskWords] = {0u, 0u, 0u, 0u};
    for (int k0 = 0; k0 < K; k0 += 4) {
      const int k = k0 + g;
      const int32_t v = (k < K && pos < n_rows) ? nbr[k * n_rows + pos] : -1;
      const uint64_t bal = __ballot(v >= 0);
#pragma unroll
      for (int gg = 0; gg < 4; ++gg) {
        if ((bal >> (16 * gg)) & 0xffffull) {
          const int kk = k0 + gg;
          words[kk >> 5] |= 1u << (kk & 31);
        }
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < kMaskWords; ++q)
        smask[wv * RG + r][q] = words[q];
    }
  }
  __syncthreads();
  // The workgroup's active offsets, in ascending order.
  if (threadIdx.x == 0) {
    int c = 0;
    for (int q = 0; q < kMaskWords; ++q) {
      uint32_t m = 0;
      for (int i = 0; i < kWaves * RG; ++i)
        m |= smask[i][q];
      while (m) {
        slist[c++] = q * 32 + __builtin_ctz(m);
        m &= m - 1;
      }
    }
    scount = c;
  }
  __syncthreads();
  const int nch = cred / CCH;
  const int S = scount * nch; // stages: (active offset, channel chunk)

  v4f acc[RG][NB];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      acc[r][nb] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < S; ++s) {
    const int k = slist[s / nch];
    const int cc0 = (s % nch) * CCH;
    // stage W[k][col0 : col0+NT][cc0 : cc0+CCH] (16-byte copies)
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int li = threadIdx.x + i * kThreads;
      if (li < NV) {
        const int n = li / (CCH / VE), cv = li % (CCH / VE);
        *reinterpret_cast<uint4 *>(&sB[n * LDW + cv * VE]) = *reinterpret_cast<const uint4 *>(
            wt + (static_cast<int64_t>(k) * ncols + col0 + n) * cred + cc0 + cv * VE);
      }
    }
    int32_t idx[RG];
    bool act[RG];
    bool wave_act = false;
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const int64_t pos = tile0 + (wv * RG + r) * 16 + i16;
      act[r] = (smask[wv * RG + r][k >> 5] >> (k & 31)) & 1u;
      idx[r] = (act[r] && pos < n_rows) ? nbr[k * n_rows + pos] : -1;
      wave_act |= act[r];
    }
    __syncthreads(); // chunk staged
    if (wave_act) {
      Frag a[RG][CSUB];
#pragma unroll
      for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int sub = 0; sub < CSUB; ++sub)
          a[r][sub] = idx[r] >= 0 ? M::load(x + static_cast<int64_t>(idx[r]) * cred + cc0 +
                                            sub * CH + g * EPL)
                                  : M::zero();
#pragma unroll
      for (int sub = 0; sub < CSUB; ++sub) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const Frag b =
              *reinterpret_cast<const Frag *>(&sB[(nb * 16 + i16) * LDW + sub * CH + g * EPL]);
#pragma unroll
          for (int r = 0; r < RG; ++r)
            if (act[r])
              M::mma(a[r][sub], b, acc[r][nb]);
        }
      }
    }
    __syncthreads(); // every wave is done reading the chunk
  }

#pragma unroll
  for (int r = 0; r < RG; ++r) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t pos = tile0 + (wv * RG + r) * 16 + 4 * g + e;
      if (pos < n_rows) {
        const int64_t o = order ? order[pos] : pos;
        T *dst = y + o * ncols + col0 + i16;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          float v = acc[r][nb][e];
          if (bias)
            v += bias[col0 + nb * 16 + i16];
          dst[nb * 16] = from_f32<T>(v);
        }
      }
    }
  }
}

// Any-shape fallback of conv_os_kernel: one lane per output element.
template <typename T>
__global__ __launch_bounds__(kThreads) void conv_os_generic_kernel(
    const T *__restrict__ x, int cred, const T *__restrict__ wt, int ncols,
    const float *__restrict__ bias, const int32_t *__restrict__ nbr,
    int64_t n_rows, int K, const int32_t *__restrict__ order,
    T *__restrict__ y) {
  const int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (t >= n_rows * ncols)
    return;
  const int64_t pos = t / ncols;
  const int col = static_cast<int>(t % ncols);
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const int32_t s = nbr[k * n_rows + pos];
    if (s < 0)
      continue;
    const T *xr = x + static_cast<int64_t>(s) * cred;
    const T *wr = wt + (static_cast<int64_t>(k) * ncols + col) * cred;
    for (int c = 0; c < cred; ++c)
      acc += to_f32(xr[c]) * to_f32(wr[c]);
  }
  if (bias)
    acc += bias[col];
  const int64_t o = order ? order[pos] : pos;
  y[o * ncols + col] = from_f32<T>(acc);
}

// wt[k][n][c] = w[k][c][n] (weights [K, cin, cout] -> [K, cout, cin]).
template <typename T>
__global__ __launch_bounds__(kThreads) void transpose_w_kernel(const T *__restrict__ w, int K,
                                                               int cin, int cout,
                                                               T *__restrict__ wt) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  const int64_t per = static_cast<int64_t>(cin) * cout;
  if (i >= K * per)
    return;
  const int64_t k = i / per, rem = i % per;
  const int c = static_cast<int>(rem / cout), n = static_cast<int>(rem % cout);
  wt[(k * cout + n) * cin + c] = w[i];
}

// ------------------------------------------------------------------- dW

constexpr int kPairChunk = 64;

// bf16: dw[k][ci][co] += sum_{p in k} x[in_rows[p]][ci] * gy[out_rows[p]][co]
// over the workgroup's pair range [blockIdx.x*ppb, +ppb), tile (MT x NTc).
// The pair axis is the MFMA reduction axis, so 64-pair chunks are staged in
// LDS transposed (pair axis contiguous).
template <typename T, int MT, int NTc>
__global__ __launch_bounds__(kThreads) void conv_dw_lds_kernel(
    const T *__restrict__ x, int cin, const T *__restrict__ gy, int cout,
    const int64_t *__restrict__ kofs, int K, const int32_t *__restrict__ in_rows,
    const int32_t *__restrict__ out_rows, int64_t n_pairs, int64_t ppb,
    float *__restrict__ dw) {
  using M = Mfma<T>;
  using Frag = typename M::Frag;
  constexpr int CH = M::kCh;
  constexpr int EPL = CH / 4;
  constexpr int VE = 16 / sizeof(T);
  constexpr int CP = kPairChunk;
  constexpr int LDP = CP + VE;
  constexpr int NBN = NTc / 16;
  constexpr int NBLK = (MT / 16) * NBN;
  constexpr int BPW = (NBLK + kWaves - 1) / kWaves;

  __shared__ __align__(16) T sX[MT * LDP];
  __shared__ __align__(16) T sG[NTc * LDP];

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = threadIdx.x / kWave;
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int tiles_n = cout / NTc;
  const int ci0 = (blockIdx.y / tiles_n) * MT;
  const int co0 = (blockIdx.y % tiles_n) * NTc;
  const int64_t pb = blockIdx.x * ppb;
  const int64_t pe = min(n_pairs, pb + ppb);
  if (pb >= pe)
    return; // uniform across the workgroup

  int k = 0;
  while (k < K - 1 && kofs[k + 1] <= pb)
    ++k;
  int64_t cur = pb;
  while (cur < pe) {
    const int64_t seg_end = min(pe, kofs[k + 1]);
    if (seg_end <= cur) { // offset k has no pairs
      ++k;
      continue;
    }
    v4f acc[BPW];
#pragma unroll
    for (int b = 0; b < BPW; ++b)
      acc[b] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int64_t c0 = cur; c0 < seg_end; c0 += CP) {
      __syncthreads();
      for (int li = threadIdx.x; li < CP * (MT / VE); li += kThreads) {
        const int p = li / (MT / VE), cv = li % (MT / VE);
        const int64_t pr = c0 + p;
        uint4 q = uint4{0u, 0u, 0u, 0u};
        if (pr < seg_end)
          q = *reinterpret_cast<const uint4 *>(
              x + static_cast<int64_t>(in_rows[pr]) * cin + ci0 + cv * VE);
        const T *e = reinterpret_cast<const T *>(&q);
#pragma unroll
        for (int j = 0; j < VE; ++j)
          sX[(cv * VE + j) * LDP + p] = e[j];
      }
      for (int li = threadIdx.x; li < CP * (NTc / VE); li += kThreads) {
        const int p = li / (NTc / VE), cv = li % (NTc / VE);
        const int64_t pr = c0 + p;
        uint4 q = uint4{0u, 0u, 0u, 0u};
        if (pr < seg_end)
          q = *reinterpret_cast<const uint4 *>(
              gy + static_cast<int64_t>(out_rows[pr]) * cout + co0 + cv * VE);
        const T *e = reinterpret_cast<const T *>(&q);
#pragma unroll
        for (int j = 0; j < VE; ++j)
          sG[(cv * VE + j) * LDP + p] = e[j];
      }
      __syncthreads();
#pragma unroll
      for (int s = 0; s < CP / CH; ++s) {
#pragma unroll
        for (int b = 0; b < BPW; ++b) {
          const int blk = wv + kWaves * b;
          if (blk < NBLK) {
            const int mi = blk / NBN, ni = blk % NBN;
            const Frag av = *reinterpret_cast<const Frag *>(
                &sX[(mi * 16 + i16) * LDP + s * CH + g * EPL]);
            const Frag bv = *reinterpret_cast<const Frag *>(
                &sG[(ni * 16 + i16) * LDP + s * CH + g * EPL]);
            M::mma(av, bv, acc[b]);
          }
        }
      }
    }
#pragma unroll
    for (int b = 0; b < BPW; ++b) {
      const int blk = wv + kWaves * b;
      if (blk < NBLK) {
        const int mi = blk / NBN, ni = blk % NBN;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ci = ci0 + mi * 16 + 4 * g + e;
          const int co = co0 + ni * 16 + i16;
          atomicAdd(&dw[(static_cast<int64_t>(k) * cin + ci) * cout + co], acc[b][e]);
        }
      }
    }
    cur = seg_end;
    ++k;
  }
}

// Any-shape fallback: one lane per dW element, looping over its pairs.
template <typename T>
__global__ __launch_bounds__(kThreads) void conv_dw_generic_kernel(
    const T *__restrict__ x, int cin, const T *__restrict__ gy, int cout,
    const int64_t *__restrict__ kofs, int K, const int32_t *__restrict__ in_rows,
    const int32_t *__restrict__ out_rows, float *__restrict__ dw) {
  const int64_t t = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (t >= static_cast<int64_t>(K) * cin * cout)
    return;
  const int k = static_cast<int>(t / (static_cast<int64_t>(cin) * cout));
  const int ci = static_cast<int>((t / cout) % cin);
  const int co = static_cast<int>(t % cout);
  float acc = 0.f;
  for (int64_t p = kofs[k]; p < kofs[k + 1]; ++p)
    acc += to_f32(x[static_cast<int64_t>(in_rows[p]) * cin + ci]) *
           to_f32(gy[static_cast<int64_t>(out_rows[p]) * cout + co]);
  dw[t] += acc;
}

__global__ __launch_bounds__(kThreads) void zero_f32_kernel(float *p, int64_t n) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (i < n)
    p[i] = 0.f;
}

template <typename T>
__global__ __launch_bounds__(kThreads) void cast_from_f32_kernel(const float *src,
                                                                 T *dst, int64_t n) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  if (i < n)
    dst[i] = from_f32<T>(src[i]);
}

// ------------------------------------------------------------------ host

static bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

template <typename T> constexpr int kChOf = Mfma<T>::kCh;

template <typename T, int NT, int RG, int CSUB>
static void launch_os(const T *x, int cred, const T *wt, int ncols,
                      const float *bias, const int32_t *nbr, int64_t n_rows,
                      int K, const int32_t *order, T *y, hipStream_t s) {
  constexpr int ROWS = kWaves * RG * 16;
  dim3 grid(static_cast<unsigned>(xcd_grid(ceil_div(n_rows, ROWS))), ncols / NT);
  hipLaunchKernelGGL((conv_os_kernel<T, NT, RG, CSUB>), grid, dim3(kThreads), 0, s, x,
                     cred, wt, ncols, bias, nbr, n_rows, K, order, y);
}

template <typename T, int NT>
static void pick_csub(const T *x, int cred, const T *wt, int ncols,
                      const float *bias, const int32_t *nbr, int64_t n_rows,
                      int K, const int32_t *order, T *y, hipStream_t s) {
  constexpr int CH = kChOf<T>;
  constexpr int RG = 2;
  if (cred % (2 * CH) == 0)
    launch_os<T, NT, RG, 2>(x, cred, wt, ncols, bias, nbr, n_rows, K, order, y, s);
  else
    launch_os<T, NT, RG, 1>(x, cred, wt, ncols, bias, nbr, n_rows, K, order, y, s);
}

// y[order[j]] = sum_k x[nbr[k][j]] @ W'[k] with W'[k][c][n] = wt[k][n][c].
template <typename T>
static void run_os(const T *x, int cred, const T *wt, int ncols,
                   const float *bias, const int32_t *nbr, int64_t n_rows, int K,
                   const int32_t *order, T *y, hipStream_t s) {
  if (n_rows == 0)
    return;
  constexpr int CH = kChOf<T>;
  const bool fast = cred % CH == 0 && ncols % 16 == 0 && K <= 32 * kMaskWords &&
                    aligned16(x) && aligned16(wt);
  if (!fast) {
    hipLaunchKernelGGL((conv_os_generic_kernel<T>), dim3(ceil_div(n_rows * ncols, kThreads)),
                       dim3(kThreads), 0, s, x, cred, wt, ncols, bias, nbr, n_rows, K,
                       order, y);
  } else if (ncols % 64 == 0) {
    pick_csub<T, 64>(x, cred, wt, ncols, bias, nbr, n_rows, K, order, y, s);
  } else if (ncols % 32 == 0) {
    pick_csub<T, 32>(x, cred, wt, ncols, bias, nbr, n_rows, K, order, y, s);
  } else {
    pick_csub<T, 16>(x, cred, wt, ncols, bias, nbr, n_rows, K, order, y, s);
  }
  RHIP_LAUNCH_CHECK();
}

template <typename T, int MT, int NTc>
static void launch_dw_lds(const T *x, int cin, const T *gy, int cout,
                          const int64_t *kofs, int K, const int32_t *in_rows,
                          const int32_t *out_rows, int64_t n_pairs, float *dw,
                          hipStream_t s) {
  const int tiles = (cin / MT) * (cout / NTc);
  // Aim for ~4 workgroups per CU over 256 CUs, at least 4 chunks each.
  const int64_t target = std::max<int64_t>(1, 1024 / tiles);
  int64_t ppb = ceil_div(n_pairs, target);
  ppb = std::max<int64_t>(4 * kPairChunk, ceil_div(ppb, kPairChunk) * kPairChunk);
  dim3 grid(static_cast<unsigned>(ceil_div(n_pairs, ppb)), tiles);
  hipLaunchKernelGGL((conv_dw_lds_kernel<T, MT, NTc>), grid, dim3(kThreads), 0, s, x, cin, gy,
                     cout, kofs, K, in_rows, out_rows, n_pairs, ppb, dw);
}

template <typename T, int MT>
static void pick_dw_lds_n(const T *x, int cin, const T *gy, int cout,
                          const int64_t *kofs, int K, const int32_t *in_rows,
                          const int32_t *out_rows, int64_t n_pairs, float *dw,
                          hipStream_t s) {
  if (cout % 64 == 0)
    launch_dw_lds<T, MT, 64>(x, cin, gy, cout, kofs, K, in_rows, out_rows, n_pairs, dw, s);
  else if (cout % 32 == 0)
    launch_dw_lds<T, MT, 32>(x, cin, gy, cout, kofs, K, in_rows, out_rows, n_pairs, dw, s);
  else
    launch_dw_lds<T, MT, 16>(x, cin, gy, cout, kofs, K, in_rows, out_rows, n_pairs, dw, s);
}

// fp32 result accumulated into dw (zeroed by the caller).
template <typename T>
static void run_dw(const T *x, int cin, const T *gy, int cout, const int64_t *kofs, int K,
                   const int32_t *in_rows, const int32_t *out_rows, int64_t n_pairs,
                   float *dw, hipStream_t s) {
  if (n_pairs == 0)
    return;
  constexpr int VE = 16 / sizeof(T);
  const bool fast = cin % 16 == 0 && cout % 16 == 0 && cin % VE == 0 && cout % VE == 0 &&
                    aligned16(x) && aligned16(gy);
  if (!fast) {
    hipLaunchKernelGGL((conv_dw_generic_kernel<T>),
                       dim3(ceil_div(static_cast<int64_t>(K) * cin * cout, kThreads)),
                       dim3(kThreads), 0, s, x, cin, gy, cout, kofs, K, in_rows, out_rows,
                       dw);
  } else if (cin % 64 == 0) {
    pick_dw_lds_n<T, 64>(x, cin, gy, cout, kofs, K, in_rows, out_rows, n_pairs, dw, s);
  } else if (cin % 32 == 0) {
    pick_dw_lds_n<T, 32>(x, cin, gy, cout, kofs, K, in_rows, out_rows, n_pairs, dw, s);
  } else {
    pick_dw_lds_n<T, 16>(x, cin, gy, cout, kofs, K, in_rows, out_rows, n_pairs, dw, s);
  }
  RHIP_LAUNCH_CHECK();
}

static void check_dtype(int32_t dtype) {
  if (dtype != RHIP_F32 && dtype != RHIP_BF16)
    throw Error(RHIP_ERR_UNSUPPORTED, "dtype must be RHIP_F32 or RHIP_BF16");
}

static size_t conv_ws_bytes(int32_t K, int32_t cin, int32_t cout) {
  // transposed weights (forward) or the fp32 dW accumulator (bf16 dW)
  return align_up(sizeof(float) * static_cast<size_t>(K) * cin * cout, 256) + 256;
}

} // namespace rhip

using namespace rhip;

extern "C" int rhip_conv_workspace_bytes(int32_t K, int32_t cin, int32_t cout,
                                         int32_t dtype, size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    check_dtype(dtype);
    *bytes = conv_ws_bytes(K, cin, cout);
  });
}

extern "C" int rhip_conv_forward(const void *x, int64_t n_in, int32_t cin,
                                 const void *weight, int32_t K, int32_t cout,
                                 const float *bias, const int32_t *nbr,
                                 const int32_t *out_order, int64_t n_out, void *y,
                                 int32_t dtype, void *workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "row counts must be >= 0");
    if (n_out == 0)
      return;
    RHIP_CHECK_ARG(y && weight && nbr, "y, weight and nbr are required");
    RHIP_CHECK_ARG(n_in == 0 || x != nullptr, "x is null");
    RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
    Carve cv(workspace, workspace_bytes);
    const int64_t nw = static_cast<int64_t>(K) * cin * cout;
    // the MFMA path reads W[k] column-wise: stage the [K, cout, cin] copy
    if (dtype == RHIP_F32) {
      float *wt = cv.take<float>(nw);
      hipLaunchKernelGGL((transpose_w_kernel<float>), dim3(ceil_div(nw, kThreads)),
                         dim3(kThreads), 0, stream, static_cast<const float *>(weight), K, cin,
                         cout, wt);
      RHIP_LAUNCH_CHECK();
      run_os<float>(static_cast<const float *>(x), cin, wt, cout, bias, nbr, n_out, K,
                    out_order, static_cast<float *>(y), stream);
    } else {
      __bf16 *wt = cv.take<__bf16>(nw);
      hipLaunchKernelGGL((transpose_w_kernel<__bf16>), dim3(ceil_div(nw, kThreads)),
                         dim3(kThreads), 0, stream, static_cast<const __bf16 *>(weight), K,
                         cin, cout, wt);
      RHIP_LAUNCH_CHECK();
      run_os<__bf16>(static_cast<const __bf16 *>(x), cin, wt, cout, bias, nbr, n_out, K,
                     out_order, static_cast<__bf16 *>(y), stream);
    }
  });
}

extern "C" int rhip_conv_backward_input(const void *grad_y, int64_t n_out,
                                        int32_t cout, const void *weight,
                                        int32_t K, int32_t cin,
                                        const int32_t *nbr_t,
                                        const int32_t *in_order, int64_t n_in,
                                        void *grad_x, int32_t dtype,
                                        void *workspace, size_t workspace_bytes,
                                        hipStream_t stream) {
  return guarded([&] {
    (void)workspace;
    (void)workspace_bytes;
    check_dtype(dtype);
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_in >= 0 && n_out >= 0, "row counts must be >= 0");
    if (n_in == 0)
      return;
    RHIP_CHECK_ARG(grad_x && weight && nbr_t, "grad_x, weight and nbr_t are required");
    RHIP_CHECK_ARG(n_out == 0 || grad_y != nullptr, "grad_y is null");
    // dX rows gather dY rows; W[k] [cin][cout] is already [n = cin][c = cout].
    if (dtype == RHIP_F32)
      run_os<float>(static_cast<const float *>(grad_y), cout,
                    static_cast<const float *>(weight), cin, nullptr, nbr_t, n_in, K,
                    in_order, static_cast<float *>(grad_x), stream);
    else
      run_os<__bf16>(static_cast<const __bf16 *>(grad_y), cout,
                     static_cast<const __bf16 *>(weight), cin, nullptr, nbr_t, n_in, K,
                     in_order, static_cast<__bf16 *>(grad_x), stream);
  });
}

extern "C" int rhip_conv_backward_weight(
    const void *x, int64_t n_in, int32_t cin, const void *grad_y, int64_t n_out,
    int32_t cout, int32_t K, const int64_t *kmap_offsets, int64_t n_pairs,
    const int32_t *in_rows, const int32_t *out_rows, void *grad_w, int32_t dtype,
    void *workspace, size_t workspace_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(K >= 1 && cin >= 1 && cout >= 1, "sizes must be positive");
    RHIP_CHECK_ARG(n_pairs >= 0 && n_in >= 0 && n_out >= 0, "bad sizes");
    RHIP_CHECK_ARG(grad_w != nullptr, "grad_w is null");
    RHIP_CHECK_ARG(n_pairs == 0 || (x && grad_y && kmap_offsets && in_rows && out_rows),
                   "x, grad_y, kmap_offsets, in_rows and out_rows are required");
    const int64_t nw = static_cast<int64_t>(K) * cin * cout;
    float *acc = nullptr;
    if (dtype == RHIP_F32) {
      acc = static_cast<float *>(grad_w);
    } else {
      RHIP_CHECK_ARG(workspace != nullptr, "workspace is null");
      Carve cv(workspace, workspace_bytes);
      acc = cv.take<float>(nw);
    }
    hipLaunchKernelGGL(zero_f32_kernel, dim3(ceil_div(nw, kThreads)), dim3(kThreads), 0,
                       stream, acc, nw);
    RHIP_LAUNCH_CHECK();
    if (dtype == RHIP_F32) {
      run_dw<float>(static_cast<const float *>(x), cin, static_cast<const float *>(grad_y),
                    cout, kmap_offsets, K, in_rows, out_rows, n_pairs, acc, stream);
    } else {
      run_dw<__bf16>(static_cast<const __bf16 *>(x), cin,
                     static_cast<const __bf16 *>(grad_y), cout, kmap_offsets, K, in_rows,
                     out_rows, n_pairs, acc, stream);
      hipLaunchKernelGGL((cast_from_f32_kernel<__bf16>), dim3(ceil_div(nw, kThreads)),
                         dim3(kThreads), 0, stream, acc, static_cast<__bf16 *>(grad_w), nw);
      RHIP_LAUNCH_CHECK();
    }
  });
}
