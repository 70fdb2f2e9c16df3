// Batch normalisation of sparse-tensor features on gfx950, for the residual
// encoder's BasicBlock (RiemannBatchNorm = torch BatchNorm1d over the feature
// matrix, engine/nn/normalization.hpp:11-37; BasicBlock, residual.cpp:44-52).
//
// Features are [n, C] row-major fp32 or bf16; statistics and parameters are
// fp32. One pass reads the features for the per-channel sums, one pass
// normalises them with the affine transform and, optionally, adds a
// residual and applies ReLU; the backward is one reduction pass and one
// apply pass. Per-channel sums run in fp64 with a fixed combination order,
// so results are deterministic and E[x^2] - E[x]^2 keeps fp32 accuracy.
//
// A thread owns one row's 16-byte channel slice (4 fp32 / 8 bf16 channels,
// or one channel for widths that are not a multiple of 16 bytes); the
// workgroup's row lanes stride over a chunk of rows and combine in LDS in
// lane order.
#include "rhip_internal.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <initializer_list>
#include <type_traits>

namespace rhip {
namespace {

constexpr int kNormThreads = 256;
constexpr int kMaxChunkRows = 1024; // rows per workgroup of a reduction pass, at most
constexpr int kReduceBlocks = 1024;  // reduction workgroups to aim for
constexpr int kUnroll = 4;       // rows loaded together by a reduction thread
constexpr int kApplyRows = 4;    // rows per thread of an elementwise pass

template <typename T, int V> struct Row;
template <> struct Row<float, 4> {
  __device__ static __forceinline__ void load(const float *p, float *v) {
    const float4 f = *reinterpret_cast<const float4 *>(p);
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  }
  __device__ static __forceinline__ void store(float *p, const float *v) {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
};
template <> struct Row<float, 1> {
  __device__ static __forceinline__ void load(const float *p, float *v) { v[0] = *p; }
  __device__ static __forceinline__ void store(float *p, const float *v) { *p = v[0]; }
};
template <> struct Row<__bf16, 8> {
  __device__ static __forceinline__ void load(const __bf16 *p, float *v) {
    const uint4 u = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __uint_as_float(w[j] << 16);
      v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
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
template <> struct Row<__bf16, 1> {
  __device__ static __forceinline__ void load(const __bf16 *p, float *v) {
    v[0] = static_cast<float>(*p);
  }
  __device__ static __forceinline__ void store(__bf16 *p, const float *v) {
    *p = static_cast<__bf16>(v[0]);
  }
};

// V consecutive fp32 per-channel values (16-byte loads when V > 1).
template <int V> __device__ __forceinline__ void load_coef(const float *p, float *v) {
  if constexpr (V == 1) {
    v[0] = *p;
  } else {
#pragma unroll
    for (int j = 0; j < V / 4; ++j) {
      const float4 f = reinterpret_cast<const float4 *>(p)[j];
      v[4 * j] = f.x, v[4 * j + 1] = f.y, v[4 * j + 2] = f.z, v[4 * j + 3] = f.w;
    }
  }
}
template <int V> __device__ __forceinline__ void load_coef_or(const float *p, float dflt, float *v) {
  if (p) {
    load_coef<V>(p, v);
  } else {
#pragma unroll
    for (int e = 0; e < V; ++e)
      v[e] = dflt;
  }
}

// Lane layout of a reduction workgroup: lpt lanes per row (channel slices of
// this channel tile), rl = 256 / lpt row lanes.
struct Lanes {
  int lane, rlane, rl, cc;
  bool active;
};
__device__ __forceinline__ Lanes lanes(int lpr, int lpt) {
  Lanes l;
  l.lane = threadIdx.x % lpt;
  l.rlane = threadIdx.x / lpt;
  l.rl = kNormThreads / lpt;
  l.cc = blockIdx.y * lpt + l.lane;
  l.active = l.cc < lpr && l.rlane < l.rl;
  return l;
}

// Combine the row lanes' two sums per channel in lane order; row lane 0
// writes part[blockIdx.x][0 / 1][c].
template <int V>
__device__ __forceinline__ void combine_rows(const Lanes &l, double (&a)[V], double (&b)[V],
                                             int C, double *__restrict__ part) {
  __shared__ double sa[kNormThreads * 8], sb[kNormThreads * 8];
#pragma unroll
  for (int e = 0; e < V; ++e) {
    sa[threadIdx.x * V + e] = a[e];
    sb[threadIdx.x * V + e] = b[e];
  }
  __syncthreads();
  if (!(l.active && l.rlane == 0))
    return;
  const int lpt = kNormThreads / l.rl;
  for (int r = 1; r < l.rl; ++r)
#pragma unroll
    for (int e = 0; e < V; ++e) {
      a[e] += sa[(r * lpt + l.lane) * V + e];
      b[e] += sb[(r * lpt + l.lane) * V + e];
    }
  double *dst = part + static_cast<int64_t>(blockIdx.x) * 2 * C;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    dst[l.cc * V + e] = a[e];
    dst[C + l.cc * V + e] = b[e];
  }
}

// part[b] = (sum x, sum x^2) over the rows of chunk b. A thread's rows are
// rl apart; kUnroll of them are loaded before any is summed.
template <typename T, int V>
__global__ __launch_bounds__(kNormThreads) void bn_sums_kernel(const T *__restrict__ x,
                                                               int64_t n, int C, int lpr, int lpt,
                                                               int64_t chunk,
                                                               double *__restrict__ part) {
  const Lanes l = lanes(lpr, lpt);
  double s[V], q[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    s[e] = q[e] = 0.0;
  if (l.active) {
    const int64_t r1 = min(n, (static_cast<int64_t>(blockIdx.x) + 1) * chunk);
    const T *p = x + l.cc * V;
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * chunk + l.rlane; r < r1;
         r += kUnroll * l.rl) {
      // rows past the chunk load the chunk's last row and count as zero: the
      // loads stay unconditional, so all kUnroll are in flight together
      float v[kUnroll][V];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        Row<T, V>::load(p + min(r + u * l.rl, r1 - 1) * C, v[u]);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const bool in = r + u * l.rl < r1;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float t = in ? v[u][e] : 0.f;
          s[e] += t;
          q[e] += static_cast<double>(t) * t;
        }
      }
    }
  }
  combine_rows<V>(l, s, q, C, part);
}

// part[b] = (sum g, sum g * xhat), g = dy masked by y > 0 when relu is set,
// xhat = (x - mean) * invstd.
template <typename T, int V>
__global__ __launch_bounds__(kNormThreads) void bn_grad_sums_kernel(
    const T *__restrict__ dy, const T *__restrict__ y, const T *__restrict__ x, int64_t n, int C,
    int lpr, int lpt, int64_t chunk, const float *__restrict__ mean,
    const float *__restrict__ invstd, int relu, double *__restrict__ part) {
  const Lanes l = lanes(lpr, lpt);
  double s[V], q[V];
#pragma unroll
  for (int e = 0; e < V; ++e)
    s[e] = q[e] = 0.0;
  if (l.active) {
    float mu[V], is[V];
    load_coef<V>(mean + l.cc * V, mu);
    load_coef<V>(invstd + l.cc * V, is);
    const int64_t r1 = min(n, (static_cast<int64_t>(blockIdx.x) + 1) * chunk);
    const int64_t c0 = l.cc * V;
    for (int64_t r = static_cast<int64_t>(blockIdx.x) * chunk + l.rlane; r < r1;
         r += kUnroll * l.rl) {
      float g[kUnroll][V], xv[kUnroll][V], yv[kUnroll][V];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) { // unconditional loads, as in bn_sums_kernel
        const int64_t o = min(r + u * l.rl, r1 - 1) * C + c0;
        Row<T, V>::load(dy + o, g[u]);
        Row<T, V>::load(x + o, xv[u]);
        Row<T, V>::load((relu ? y : dy) + o, yv[u]);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const bool in = r + u * l.rl < r1;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float ge = (!in || (relu && !(yv[u][e] > 0.f))) ? 0.f : g[u][e];
          s[e] += ge;
          q[e] += static_cast<double>(ge) * ((xv[u][e] - mu[e]) * is[e]);
        }
      }
    }
  }
  combine_rows<V>(l, s, q, C, part);
}

// Workgroup c: the chunks' sums of channel c added in a fixed order (a
// strided pass per thread, then a tree in LDS). mode 0 (statistics):
// mean, invstd and the running statistics; mode 1 (gradient): the two sums
// (dbeta, dgamma), also written to copy0 / copy1 when given.
__global__ __launch_bounds__(kNormThreads) void bn_final_kernel(
    const double *__restrict__ part, int64_t chunks, int64_t n, int C, int mode, double eps,
    double momentum, float *__restrict__ running_mean, float *__restrict__ running_var,
    float *__restrict__ out0, float *__restrict__ out1, float *__restrict__ copy0,
    float *__restrict__ copy1) {
  __shared__ double sa[kNormThreads], sb[kNormThreads];
  const int c = blockIdx.x;
  double a = 0.0, b = 0.0;
  for (int64_t k = threadIdx.x; k < chunks; k += kNormThreads) {
    a += part[k * 2 * C + c];
    b += part[k * 2 * C + C + c];
  }
  sa[threadIdx.x] = a;
  sb[threadIdx.x] = b;
  __syncthreads();
  for (int w = kNormThreads / 2; w > 0; w >>= 1) {
    if (static_cast<int>(threadIdx.x) < w) {
      sa[threadIdx.x] += sa[threadIdx.x + w];
      sb[threadIdx.x] += sb[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x != 0)
    return;
  if (mode == 1) { // out0 = sum g (dbeta), out1 = sum g * xhat (dgamma); copies optional
    const float g = static_cast<float>(sa[0]), gx = static_cast<float>(sb[0]);
    out0[c] = g;
    out1[c] = gx;
    if (copy0)
      copy0[c] = g;
    if (copy1)
      copy1[c] = gx;
    return;
  }
  const double mu = sa[0] / static_cast<double>(n);
  double var = sb[0] / static_cast<double>(n) - mu * mu; // biased
  var = var < 0.0 ? 0.0 : var;
  out0[c] = static_cast<float>(mu);
  out1[c] = static_cast<float>(1.0 / sqrt(var + eps));
  if (running_mean)
    running_mean[c] = static_cast<float>((1.0 - momentum) * running_mean[c] + momentum * mu);
  if (running_var)
    running_var[c] = static_cast<float>((1.0 - momentum) * running_var[c] +
                                        momentum * var * static_cast<double>(n) /
                                            static_cast<double>(n - 1));
}

// invstd = 1 / sqrt(running_var + eps) (evaluation with running statistics).
__global__ void bn_invstd_kernel(const float *__restrict__ var, int C, double eps,
                                 float *__restrict__ invstd) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c < C)
    invstd[c] = static_cast<float>(1.0 / sqrt(static_cast<double>(var[c]) + eps));
}

// y = act((x - mean) * invstd * gamma + beta [+ residual]) over rows
// blockIdx.x * rl * kApplyRows + rlane + j * rl, j < kApplyRows: a thread
// keeps its channel slice's coefficients and loads all its rows before the
// first store. y may alias x or residual: a thread writes only the slices it
// has read.
template <typename T, int V>
__global__ __launch_bounds__(kNormThreads) void bn_apply_kernel(
    const T *x, const T *residual, int64_t n, int C, int lpr, int lpt,
    const float *__restrict__ mean, const float *__restrict__ invstd,
    const float *__restrict__ gamma, const float *__restrict__ beta, int relu, T *y) {
  const Lanes l = lanes(lpr, lpt);
  if (!l.active)
    return;
  const int c0 = l.cc * V;
  float mu[V], k[V], b[V], is[V];
  load_coef<V>(mean + c0, mu);
  load_coef<V>(invstd + c0, is);
  load_coef_or<V>(gamma ? gamma + c0 : nullptr, 1.f, k);
  load_coef_or<V>(beta ? beta + c0 : nullptr, 0.f, b);
#pragma unroll
  for (int e = 0; e < V; ++e)
    k[e] *= is[e];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * l.rl * kApplyRows + l.rlane;
  if (r0 >= n)
    return;
  // rows past n load row n - 1 (unconditional loads stay in flight together)
  // and are not stored
  float v[kApplyRows][V], rv[kApplyRows][V];
#pragma unroll
  for (int u = 0; u < kApplyRows; ++u) {
    const int64_t o = min(r0 + u * l.rl, n - 1) * C + c0;
    Row<T, V>::load(x + o, v[u]);
    Row<T, V>::load((residual ? residual : x) + o, rv[u]);
  }
#pragma unroll
  for (int u = 0; u < kApplyRows; ++u) {
    const int64_t rr = r0 + u * l.rl;
    if (rr >= n)
      continue;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      float o = (v[u][e] - mu[e]) * k[e] + b[e];
      if (residual)
        o += rv[u][e];
      v[u][e] = relu ? fmaxf(o, 0.f) : o;
    }
    Row<T, V>::store(y + rr * C + c0, v[u]);
  }
}

// g = dy masked by y > 0 when relu is set; dresidual = g;
// batch statistics: dx = gamma * invstd * (g - sum_g / n - xhat * sum_gxhat / n);
// running statistics: dx = gamma * invstd * g. Rows as in bn_apply_kernel.
template <typename T, int V>
__global__ __launch_bounds__(kNormThreads) void bn_grad_apply_kernel(
    const T *__restrict__ dy, const T *__restrict__ y, const T *__restrict__ x, int64_t n, int C,
    int lpr, int lpt, const float *__restrict__ mean, const float *__restrict__ invstd,
    const float *__restrict__ gamma, const float *__restrict__ sum_g,
    const float *__restrict__ sum_gx, int relu, int batch_stats, T *__restrict__ dx,
    T *__restrict__ dres) {
  const Lanes l = lanes(lpr, lpt);
  if (!l.active)
    return;
  const int c0 = l.cc * V;
  const bool need_x = dx != nullptr && batch_stats;
  float mu[V], is[V], k[V], a[V], b[V];
  const float inv_n = 1.f / static_cast<float>(n);
  load_coef<V>(mean + c0, mu);
  load_coef<V>(invstd + c0, is);
  load_coef_or<V>(gamma ? gamma + c0 : nullptr, 1.f, k);
  load_coef_or<V>(batch_stats ? sum_g + c0 : nullptr, 0.f, a);
  load_coef_or<V>(batch_stats ? sum_gx + c0 : nullptr, 0.f, b);
#pragma unroll
  for (int e = 0; e < V; ++e) {
    k[e] *= is[e];
    a[e] *= inv_n;
    b[e] *= inv_n;
  }
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * l.rl * kApplyRows + l.rlane;
  if (r0 >= n)
    return;
  // rows past n load row n - 1 (as in bn_apply_kernel) and are not stored
  float g[kApplyRows][V], yv[kApplyRows][V], xv[kApplyRows][V];
#pragma unroll
  for (int u = 0; u < kApplyRows; ++u) {
    const int64_t o = min(r0 + u * l.rl, n - 1) * C + c0;
    Row<T, V>::load(dy + o, g[u]);
    Row<T, V>::load((relu ? y : dy) + o, yv[u]);
    Row<T, V>::load((need_x ? x : dy) + o, xv[u]);
  }
#pragma unroll
  for (int u = 0; u < kApplyRows; ++u) {
    const int64_t rr = r0 + u * l.rl;
    if (rr >= n)
      continue;
    const int64_t o = rr * C + c0;
    if (relu)
#pragma unroll
      for (int e = 0; e < V; ++e)
        g[u][e] = yv[u][e] > 0.f ? g[u][e] : 0.f;
    if (dres)
      Row<T, V>::store(dres + o, g[u]);
    if (dx == nullptr)
      continue;
    float out[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float xhat = need_x ? (xv[u][e] - mu[e]) * is[e] : 0.f;
      out[e] = k[e] * (g[u][e] - a[e] - xhat * b[e]);
    }
    Row<T, V>::store(dx + o, out);
  }
}

// ------------------------------------------------------------------ host

void check_dtype(int32_t dtype) {
  if (dtype != RHIP_F32 && dtype != RHIP_BF16)
    throw Error(RHIP_ERR_UNSUPPORTED, "dtype must be RHIP_F32 or RHIP_BF16");
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T> int width(int C, std::initializer_list<const void *> ptrs) {
  constexpr int W = 16 / sizeof(T);
  if (C % W != 0)
    return 1;
  for (const void *p : ptrs)
    if (p && !aligned16(p))
      return 1;
  return W;
}

template <typename T, typename F> void with_width(int V, F &&f) {
  if (V == 1)
    f(std::integral_constant<int, 1>{});
  else
    f(std::integral_constant<int, 16 / sizeof(T)>{});
}

template <typename F> void with_type(int32_t dtype, F &&f) {
  if (dtype == RHIP_F32)
    f(float{});
  else
    f(__bf16{});
}

// Rows per reduction workgroup: enough workgroups to fill the chip for small
// row counts (a multiple of 64 rows), at most kMaxChunkRows.
int64_t chunk_rows(int64_t n) {
  return std::min<int64_t>(kMaxChunkRows,
                           std::max<int64_t>(64, ceil_div(ceil_div(n, kReduceBlocks), 64) * 64));
}
int64_t chunks_of(int64_t n) { return std::max<int64_t>(1, ceil_div(n, chunk_rows(n))); }

struct NormWs {
  double *part;
  float *sum_g, *sum_gx;
};
NormWs carve_norm(Carve &cv, int64_t n, int C) {
  NormWs w{};
  w.part = cv.take<double>(chunks_of(n) * 2 * static_cast<int64_t>(C));
  w.sum_g = cv.take<float>(C);
  w.sum_gx = cv.take<float>(C);
  return w;
}

// Launch shape over [n, C] features: lpr slices per row, lpt of them per
// workgroup (grid.y over channel tiles), rl = 256 / lpt rows side by side.
// Reductions take chunk_rows(n) rows per workgroup, elementwise passes
// rl * kApplyRows.
template <typename T, int V, typename Launch>
void over_rows(int64_t n, int C, bool reduction, Launch &&launch) {
  const int lpr = C / V, lpt = std::min(lpr, kNormThreads), rl = kNormThreads / lpt;
  const int64_t gx = reduction ? chunks_of(n) : std::max<int64_t>(1, ceil_div(n, rl * kApplyRows));
  RHIP_CHECK_ARG(gx <= INT_MAX, "too many rows for one launch");
  launch(dim3(static_cast<unsigned>(gx), static_cast<unsigned>(ceil_div(lpr, lpt))), lpr, lpt);
}

} // namespace
} // namespace rhip

using namespace rhip;

extern "C" int rhip_bn_workspace_bytes(int64_t n, int32_t C, size_t *bytes) {
  return guarded([&] {
    RHIP_CHECK_ARG(bytes != nullptr, "bytes is null");
    RHIP_CHECK_ARG(n >= 0 && C >= 1, "bad sizes");
    Carve cv(nullptr, 0);
    carve_norm(cv, n, C);
    *bytes = cv.used + 256;
  });
}

extern "C" int rhip_bn_stats(const void *x, int64_t n, int32_t C, int32_t dtype, double eps,
                             double momentum, float *running_mean, float *running_var,
                             float *mean, float *invstd, void *workspace, size_t ws_bytes,
                             hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(C >= 1 && n >= 0, "bad sizes");
    RHIP_CHECK_ARG(n > 1, "Expected more than 1 value per channel when training");
    RHIP_CHECK_ARG(x && mean && invstd && workspace, "x, mean, invstd and workspace required");
    RHIP_CHECK_ARG(eps > 0, "eps must be positive");
    Carve cv(workspace, ws_bytes);
    NormWs w = carve_norm(cv, n, C);
    with_type(dtype, [&](auto tag) {
      using T = decltype(tag);
      with_width<T>(width<T>(C, {x}), [&](auto v) {
        constexpr int V = decltype(v)::value;
        over_rows<T, V>(n, C, true, [&](dim3 grid, int lpr, int lpt) {
          hipLaunchKernelGGL((bn_sums_kernel<T, V>), grid, dim3(kNormThreads), 0, stream,
                             static_cast<const T *>(x), n, C, lpr, lpt, chunk_rows(n), w.part);
          RHIP_LAUNCH_CHECK();
        });
      });
    });
    hipLaunchKernelGGL(bn_final_kernel, dim3(C), dim3(kNormThreads), 0, stream, w.part,
                       chunks_of(n), n, C, 0, eps, momentum, running_mean, running_var, mean,
                       invstd, nullptr, nullptr);
    RHIP_LAUNCH_CHECK();
  });
}

extern "C" int rhip_bn_invstd(const float *var, int32_t C, double eps, float *invstd,
                              hipStream_t stream) {
  return guarded([&] {
    RHIP_CHECK_ARG(C >= 1 && var && invstd, "bad arguments");
    hipLaunchKernelGGL(bn_invstd_kernel, dim3(ceil_div(C, 256)), dim3(256), 0, stream, var, C,
                       eps, invstd);
    RHIP_LAUNCH_CHECK();
  });
}

extern "C" int rhip_bn_forward(const void *x, int64_t n, int32_t C, const float *mean,
                               const float *invstd, const float *gamma, const float *beta,
                               const void *residual, int32_t relu, void *y, int32_t dtype,
                               hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(C >= 1 && n >= 0, "bad sizes");
    if (n == 0)
      return;
    RHIP_CHECK_ARG(x && y && mean && invstd, "x, y, mean and invstd are required");
    with_type(dtype, [&](auto tag) {
      using T = decltype(tag);
      with_width<T>(width<T>(C, {x, y, residual, mean, invstd, gamma, beta}), [&](auto v) {
        constexpr int V = decltype(v)::value;
        over_rows<T, V>(n, C, false, [&](dim3 grid, int lpr, int lpt) {
          hipLaunchKernelGGL((bn_apply_kernel<T, V>), grid, dim3(kNormThreads), 0, stream,
                             static_cast<const T *>(x), static_cast<const T *>(residual), n, C,
                             lpr, lpt, mean, invstd, gamma, beta, relu, static_cast<T *>(y));
          RHIP_LAUNCH_CHECK();
        });
      });
    });
  });
}

extern "C" int rhip_bn_backward(const void *grad_y, const void *y, const void *x, int64_t n,
                                int32_t C, const float *mean, const float *invstd,
                                const float *gamma, int32_t relu, int32_t batch_stats,
                                void *grad_x, void *grad_residual, float *grad_gamma,
                                float *grad_beta, int32_t dtype, void *workspace,
                                size_t ws_bytes, hipStream_t stream) {
  return guarded([&] {
    check_dtype(dtype);
    RHIP_CHECK_ARG(C >= 1 && n >= 0, "bad sizes");
    RHIP_CHECK_ARG(mean && invstd && workspace, "mean, invstd and workspace are required");
    RHIP_CHECK_ARG(n == 0 || (grad_y && x), "grad_y and x are required");
    RHIP_CHECK_ARG(n == 0 || !relu || y != nullptr, "relu needs y");
    Carve cv(workspace, ws_bytes);
    NormWs w = carve_norm(cv, n, C);
    const bool sums = (batch_stats && grad_x) || grad_gamma || grad_beta;
    with_type(dtype, [&](auto tag) {
      using T = decltype(tag);
      with_width<T>(width<T>(C, {grad_y, y, x, grad_x, grad_residual, mean, invstd, gamma}),
                    [&](auto v) {
        constexpr int V = decltype(v)::value;
        if (sums) { // n = 0: one empty chunk, zero sums
          over_rows<T, V>(n, C, true, [&](dim3 grid, int lpr, int lpt) {
            hipLaunchKernelGGL((bn_grad_sums_kernel<T, V>), grid, dim3(kNormThreads), 0, stream,
                               static_cast<const T *>(grad_y), static_cast<const T *>(y),
                               static_cast<const T *>(x), n, C, lpr, lpt, chunk_rows(n), mean,
                               invstd, relu, w.part);
            RHIP_LAUNCH_CHECK();
          });
          hipLaunchKernelGGL(bn_final_kernel, dim3(C), dim3(kNormThreads), 0, stream, w.part,
                             chunks_of(n), n, C, 1, 0.0, 0.0, nullptr, nullptr, w.sum_g,
                             w.sum_gx, grad_beta, grad_gamma);
          RHIP_LAUNCH_CHECK();
        }
        if (n > 0 && (grad_x || grad_residual)) {
          over_rows<T, V>(n, C, false, [&](dim3 grid, int lpr, int lpt) {
            hipLaunchKernelGGL((bn_grad_apply_kernel<T, V>), grid, dim3(kNormThreads), 0,
                               stream, static_cast<const T *>(grad_y), static_cast<const T *>(y),
                               static_cast<const T *>(x), n, C, lpr, lpt, mean, invstd, gamma,
                               w.sum_g, w.sum_gx, relu, batch_stats, static_cast<T *>(grad_x),
                               static_cast<T *>(grad_residual));
            RHIP_LAUNCH_CHECK();
          });
        }
      });
    });
  });
}
