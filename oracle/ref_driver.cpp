// Test infrastructure only: C entry points over the reference's own CPU path.
//
// oracle/ref.mk compiles the reference sources where they lie (space.cpp,
// stencil.cpp, conv.cpp, sparse_tensor.cpp under RiemannEngine/engine/) with
// CPU_ONLY, plus this file, into oracle/_ref/libriemann_ref.so. The functions
// below drive the reference's public C++ API (riemann::CoordinateManager on
// the CPU backend, riemann::RiemannConvolution) so that tests can check the
// oracle and the HIP path against the reference itself, and bench.py can time
// it as the CPU baseline. Nothing on the product path loads this library.
//
// Every function returns a count >= 0 or -1 with ref_last_error() set.
// Variable-size outputs are written only when they fit `cap`; call once with
// cap = 0 to learn the size.
#include "engine/grid/space.hpp"
#include "engine/nn/conv.hpp"
#include "engine/nn/pooling.hpp"
#include "engine/tensor/sparse_tensor.hpp"

#include <torch/torch.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <exception>
#include <memory>
#include <string>

namespace {

thread_local std::string g_error;

template <typename F> int64_t guarded(F &&body) {
  try {
    return body();
  } catch (const std::exception &e) {
    g_error = e.what();
    return -1;
  }
}

torch::Tensor int_rows(const int32_t *p, int64_t n, int ncol) {
  return torch::from_blob(const_cast<int32_t *>(p), {n, ncol}, torch::kInt32).clone();
}

torch::Tensor float_rows(const float *p, int64_t n, int64_t c) {
  return torch::from_blob(const_cast<float *>(p), {n, c}, torch::kFloat32).clone();
}

void copy_out(const torch::Tensor &t, void *dst) {
  auto c = t.contiguous();
  std::memcpy(dst, c.data_ptr(), c.numel() * c.element_size());
}

riemann::RegionType::Type region_of(int region) {
  return region == 1 ? riemann::RegionType::HYPER_CROSS : riemann::RegionType::HYPER_CUBE;
}

using CpuManager = riemann::cpu_manager_type<int32_t>;

} // namespace

extern "C" {

const char *ref_last_error() { return g_error.c_str(); }

// CoordinateManager::insert_and_map on the CPU backend (space.cpp:17-58):
// unique rows [n_u, ncol], mapping [n_u] and inverse [n]. Returns n_u.
int64_t ref_insert_and_map(const int32_t *coords, int64_t n, int ncol, int64_t cap,
                           int32_t *unique, int64_t *mapping, int64_t *inverse) {
  return guarded([&]() -> int64_t {
    riemann::CoordinateManager m(ncol - 1, riemann::CoordinateMapBackend::CPU);
    auto r = m.insert_and_map(int_rows(coords, n, ncol),
                              riemann::stride_type(static_cast<size_t>(ncol - 1), 1));
    auto u = m.get_coordinates(r.first).to(torch::kInt32);
    const int64_t nu = u.size(0);
    if (nu <= cap) {
      copy_out(u, unique);
      copy_out(r.second.first.to(torch::kInt64), mapping);
      copy_out(r.second.second.to(torch::kInt64), inverse);
    }
    return nu;
  });
}

// The kernel map a stride-`stride` convolution with a ks^D cube (region 0)
// or cross (region 1) builds over the unique rows `coords` (tensor stride 1),
// exactly as evaluate_sparse_convolution requests it (conv.cpp:38-42). The
// output map is the input map (stride 1) or CoordinateManager::stride's
// coarse map, whose rows go to out_coords. kofs [K+1]; pairs when P <= cap.
// Returns P; *n_out and *K are set.
int64_t ref_kernel_map(const int32_t *coords, int64_t n, int ncol, int ks, int stride, int dil,
                       int region, int64_t cap, int64_t *kofs, int32_t *in_rows,
                       int32_t *out_rows, int64_t out_cap, int32_t *out_coords, int64_t *n_out,
                       int32_t *K) {
  return guarded([&]() -> int64_t {
    const int D = ncol - 1;
    riemann::CoordinateManager m(D, riemann::CoordinateMapBackend::CPU);
    auto r = m.insert_and_map(int_rows(coords, n, ncol),
                              riemann::stride_type(static_cast<size_t>(D), 1));
    const auto in_key = r.first;
    const riemann::stride_type s(static_cast<size_t>(D), static_cast<uint32_t>(stride));
    const auto out_key = stride > 1 ? m.stride(in_key, s) : in_key;
    const auto &map = m.manager_ptr<CpuManager>()->kernel_map(
        &in_key, &out_key, riemann::stride_type(static_cast<size_t>(D), ks), s,
        riemann::stride_type(static_cast<size_t>(D), dil), region_of(region), at::Tensor(),
        false, false);
    auto oc = m.get_coordinates(out_key).to(torch::kInt32);
    *n_out = oc.size(0);
    if (oc.size(0) <= out_cap)
      copy_out(oc, out_coords);
    *K = static_cast<int32_t>(map.first.size());
    int64_t P = 0;
    kofs[0] = 0;
    for (size_t k = 0; k < map.first.size(); ++k) {
      P += static_cast<int64_t>(map.first[k].size());
      kofs[k + 1] = P;
    }
    if (P <= cap) {
      for (size_t k = 0; k < map.first.size(); ++k) {
        for (size_t i = 0; i < map.first[k].size(); ++i) {
          in_rows[kofs[k] + i] = static_cast<int32_t>(map.first[k][i]);
          out_rows[kofs[k] + i] = static_cast<int32_t>(map.second[k][i]);
        }
      }
    }
    return P;
  });
}

// RiemannConvolution(cin, cout, ks, stride, dil, bias=false, D) forward and
// backward on the CPU, in fp32 (dtype 0) or bf16 (dtype 1) exactly as the
// reference computes them (per-offset index_select -> matmul -> index_add_ in
// the feature dtype, LibTorch autograd for the gradients). x [n, cin] over
// the unique rows `coords`, w [K, cin, cout], gy [n_out, cout] in the
// reference's output row order (may be NULL: forward only). Outputs are fp32:
// y [n_out, cout], out_coords [n_out, ncol], gx [n, cin], gw [K, cin, cout];
// y/out_coords/gx/gw are written when n_out <= out_cap. Returns n_out.
int64_t ref_conv(const int32_t *coords, int64_t n, int ncol, const float *x, int cin,
                 const float *w, int K, int cout, int ks, int stride, int dil, int dtype,
                 const float *gy, int64_t out_cap, float *y, int32_t *out_coords, float *gx,
                 float *gw) {
  return guarded([&]() -> int64_t {
    const int D = ncol - 1;
    const auto dt = dtype == 1 ? torch::kBFloat16 : torch::kFloat32;
    auto mgr = std::make_shared<riemann::CoordinateManager>(D, riemann::CoordinateMapBackend::CPU);
    auto X = float_rows(x, n, cin).to(dt).detach().requires_grad_(true);
    riemann::SparseTensor input(X, int_rows(coords, n, ncol), mgr);
    riemann::RiemannConvolution conv(cin, cout, ks, stride, dil, false, false,
                                     riemann::ConvolutionMode::DEFAULT, D);
    auto &kernel = conv->base()->kernel_;
    TORCH_CHECK(kernel.size(0) == K, "kernel volume ", kernel.size(0), " != ", K);
    kernel.set_data(torch::from_blob(const_cast<float *>(w), {K, cin, cout}, torch::kFloat32)
                        .to(dt)
                        .clone());
    auto out = conv->forward(input);
    const int64_t n_out = out.F().size(0);
    if (n_out > out_cap)
      return n_out;
    copy_out(out.F().detach().to(torch::kFloat32), y);
    copy_out(mgr->get_coordinates(out.coordinate_map_key()).to(torch::kInt32), out_coords);
    if (gy != nullptr) {
      out.F().backward(float_rows(gy, n_out, cout).to(dt));
      copy_out(X.grad().to(torch::kFloat32), gx);
      copy_out(kernel.grad().to(torch::kFloat32), gw);
    }
    return n_out;
  });
}

// The generated map of a generative transposed convolution, from the
// reference's CoordinateMapManager::stride_region (space_impl.hpp:352-381,
// lattice_cpu.hpp:499-534), driven as its transposed pooling does
// (pooling.cpp:46-62): the input rows `coords` form the map at tensor stride
// in_stride, the region (ks^D cube or cross, dilation dil) sits at the output
// tensor stride in_stride / stride. Rows go to out when they fit cap.
// Returns the generated row count.
int64_t ref_stride_region(const int32_t *coords, int64_t n, int ncol, int in_stride, int stride,
                          int ks, int dil, int region, int64_t cap, int32_t *out) {
  return guarded([&]() -> int64_t {
    const int D = ncol - 1;
    TORCH_CHECK(stride > 0 && in_stride % stride == 0, "stride must divide in_stride");
    riemann::CoordinateManager m(D, riemann::CoordinateMapBackend::CPU);
    auto r = m.insert_and_map(int_rows(coords, n, ncol),
                              riemann::stride_type(static_cast<size_t>(D), in_stride));
    riemann::stride_type out_stride(static_cast<size_t>(D), in_stride / stride);
    riemann::stride_type kernel_size(static_cast<size_t>(D), ks);
    riemann::stride_type dilation(static_cast<size_t>(D), dil);
    riemann::cpu_kernel_region<int32_t> kregion(region_of(region), ncol, out_stride.data(),
                                                kernel_size.data(), dilation.data(), 0, nullptr,
                                                0, true);
    const auto generated = m.manager_ptr<CpuManager>()->stride_region(
        r.first.get_key(), kregion, out_stride, true);
    auto oc = m.get_coordinates(riemann::CoordinateMapKey(ncol, generated.first))
                  .to(torch::kInt32);
    if (oc.size(0) <= cap)
      copy_out(oc, out);
    return oc.size(0);
  });
}

// Times the reference's CPU kernel-map build alone, the work the GPU's
// hash build + kernel map replace: CoordinateManager::insert_and_map over the
// rows (the coordinate hash), then CpuManager::kernel_map for a ks^D stride-1
// cube over that map (lattice_cpu.hpp's neighbour search). Each of `reps`
// runs starts from a fresh manager; the means go to *hash_ms and *map_ms.
// Returns the pair count.
int64_t ref_map_time(const int32_t *coords, int64_t n, int ncol, int ks, int reps,
                     double *hash_ms, double *map_ms) {
  return guarded([&]() -> int64_t {
    const int D = ncol - 1;
    const auto rows = int_rows(coords, n, ncol);
    const riemann::stride_type one(static_cast<size_t>(D), 1);
    using clock = std::chrono::steady_clock;
    double th = 0.0, tm = 0.0;
    int64_t P = 0;
    for (int r = 0; r < std::max(reps, 1); ++r) {
      riemann::CoordinateManager m(D, riemann::CoordinateMapBackend::CPU);
      auto t0 = clock::now();
      auto key = m.insert_and_map(rows, one).first;
      auto t1 = clock::now();
      const auto &map = m.manager_ptr<CpuManager>()->kernel_map(
          &key, &key, riemann::stride_type(static_cast<size_t>(D), ks), one, one,
          riemann::RegionType::HYPER_CUBE, at::Tensor(), false, false);
      auto t2 = clock::now();
      th += std::chrono::duration<double, std::milli>(t1 - t0).count();
      tm += std::chrono::duration<double, std::milli>(t2 - t1).count();
      P = 0;
      for (const auto &v : map.first)
        P += static_cast<int64_t>(v.size());
    }
    *hash_ms = th / std::max(reps, 1);
    *map_ms = tm / std::max(reps, 1);
    return P;
  });
}

// Times the reference on the CPU: one RiemannConvolution forward (which
// builds and caches the kernel map) into *map_ms, then `reps` forward +
// backward steps reusing the cached map, their mean into *step_ms. Random
// operands from `seed`. Returns the pair count of the map.
int64_t ref_conv_time(const int32_t *coords, int64_t n, int ncol, int cin, int cout, int ks,
                      int dtype, int reps, int seed, double *map_ms, double *step_ms) {
  return guarded([&]() -> int64_t {
    const int D = ncol - 1;
    const auto dt = dtype == 1 ? torch::kBFloat16 : torch::kFloat32;
    torch::manual_seed(seed);
    auto mgr = std::make_shared<riemann::CoordinateManager>(D, riemann::CoordinateMapBackend::CPU);
    auto X = torch::randn({n, cin}).to(dt).detach().requires_grad_(true);
    riemann::SparseTensor input(X, int_rows(coords, n, ncol), mgr);
    riemann::RiemannConvolution conv(cin, cout, ks, 1, 1, false, false,
                                     riemann::ConvolutionMode::DEFAULT, D);
    auto &kernel = conv->base()->kernel_;
    kernel.set_data(kernel.detach().to(dt).clone());
    using clock = std::chrono::steady_clock;
    auto t0 = clock::now();
    auto out = conv->forward(input);
    *map_ms = std::chrono::duration<double, std::milli>(clock::now() - t0).count();
    auto gy = torch::randn_like(out.F());
    double total = 0.0;
    for (int r = 0; r < reps; ++r) {
      X.mutable_grad() = torch::Tensor();
      kernel.mutable_grad() = torch::Tensor();
      auto t1 = clock::now();
      auto o = conv->forward(input);
      o.F().backward(gy);
      total += std::chrono::duration<double, std::milli>(clock::now() - t1).count();
    }
    *step_ms = total / std::max(reps, 1);
    int64_t P = 0;
    const auto key = input.coordinate_map_key();
    const auto &map = mgr->manager_ptr<CpuManager>()->kernel_map(
        &key, &key, riemann::stride_type(static_cast<size_t>(D), ks),
        riemann::stride_type(static_cast<size_t>(D), 1),
        riemann::stride_type(static_cast<size_t>(D), 1), riemann::RegionType::HYPER_CUBE,
        at::Tensor(), false, false);
    for (const auto &v : map.first)
      P += static_cast<int64_t>(v.size());
    return P;
  });
}

// The reference's local pooling layers on the CPU (pooling.cpp:80-200):
// RiemannSumPooling / RiemannAvgPooling / RiemannMaxPooling (mode 0 / 1 / 2)
// with (ks, stride, dil), or, with transpose set, RiemannPoolingTranspose
// through its KernelGenerator constructor with that mode and
// expand_coordinates = expand. The input is the map of the unique rows
// `coords` at tensor stride in_stride with features x [n, C] (row order of
// `coords`), in fp32 (dtype 0) or bf16 (dtype 1). gy [n_out, C] in the
// output's row order (may be NULL: forward only). Outputs are fp32: y
// [n_out, C], out_coords [n_out, ncol], gx [n, C]; written when n_out <=
// out_cap. Returns n_out.
int64_t ref_pool(const int32_t *coords, int64_t n, int ncol, int in_stride, const float *x,
                 int C, int ks, int stride, int dil, int mode, int transpose, int expand,
                 int dtype, const float *gy, int64_t out_cap, float *y, int32_t *out_coords,
                 float *gx) {
  return guarded([&]() -> int64_t {
    const int D = ncol - 1;
    const auto dt = dtype == 1 ? torch::kBFloat16 : torch::kFloat32;
    auto mgr = std::make_shared<riemann::CoordinateManager>(D, riemann::CoordinateMapBackend::CPU);
    auto r = mgr->insert_and_map(int_rows(coords, n, ncol),
                                 riemann::stride_type(static_cast<size_t>(D), in_stride));
    TORCH_CHECK(r.second.first.numel() == n, "coordinates must be unique");
    auto X = float_rows(x, n, C).to(dt).detach().requires_grad_(true);
    riemann::SparseTensor input(X.index_select(0, r.second.first.to(torch::kLong)), r.first, mgr);
    const riemann::PoolingMode::Type pm =
        mode == 0 ? riemann::PoolingMode::LOCAL_SUM_POOLING
                  : (mode == 1 ? riemann::PoolingMode::LOCAL_AVG_POOLING
                               : riemann::PoolingMode::LOCAL_MAX_POOLING);
    riemann::SparseTensor out = [&] {
      if (transpose) {
        riemann::KernelGenerator gen({ks}, {stride}, {dil}, true, riemann::RegionType::HYPER_CUBE,
                                     {}, expand != 0, {}, D);
        riemann::RiemannPoolingTranspose layer(gen, D, pm);
        return layer->forward(input);
      }
      if (mode == 0)
        return riemann::RiemannSumPooling(ks, stride, dil, D)->forward(input);
      if (mode == 1)
        return riemann::RiemannAvgPooling(ks, stride, dil, D)->forward(input);
      return riemann::RiemannMaxPooling(ks, stride, dil, D)->forward(input);
    }();
    const int64_t n_out = out.F().size(0);
    if (n_out > out_cap)
      return n_out;
    copy_out(out.F().detach().to(torch::kFloat32), y);
    copy_out(mgr->get_coordinates(out.coordinate_map_key()).to(torch::kInt32), out_coords);
    if (gy != nullptr) {
      out.F().backward(float_rows(gy, n_out, C).to(dt));
      copy_out(X.grad().to(torch::kFloat32), gx);
    }
    return n_out;
  });
}

// RiemannGlobalPooling (pooling.cpp:203-260) with the GLOBAL_{SUM,AVG,MAX}_
// POOLING_PYTORCH_INDEX mode (mode 0 / 1 / 2) over the rows `coords` with
// features x [n, C]. Same conventions as ref_pool. Returns the batch count.
int64_t ref_global_pool(const int32_t *coords, int64_t n, int ncol, const float *x, int C,
                        int mode, int dtype, const float *gy, int64_t out_cap, float *y,
                        int32_t *out_coords, float *gx) {
  return guarded([&]() -> int64_t {
    const int D = ncol - 1;
    const auto dt = dtype == 1 ? torch::kBFloat16 : torch::kFloat32;
    auto mgr = std::make_shared<riemann::CoordinateManager>(D, riemann::CoordinateMapBackend::CPU);
    auto X = float_rows(x, n, C).to(dt).detach().requires_grad_(true);
    riemann::SparseTensor input(X, int_rows(coords, n, ncol), mgr);
    const riemann::PoolingMode::Type pm =
        mode == 0 ? riemann::PoolingMode::GLOBAL_SUM_POOLING_PYTORCH_INDEX
                  : (mode == 1 ? riemann::PoolingMode::GLOBAL_AVG_POOLING_PYTORCH_INDEX
                               : riemann::PoolingMode::GLOBAL_MAX_POOLING_PYTORCH_INDEX);
    riemann::RiemannGlobalPooling layer(pm);
    auto out = layer->forward(input);
    const int64_t B = out.F().size(0);
    if (B > out_cap)
      return B;
    copy_out(out.F().detach().to(torch::kFloat32), y);
    copy_out(mgr->get_coordinates(out.coordinate_map_key()).to(torch::kInt32), out_coords);
    if (gy != nullptr) {
      out.F().backward(float_rows(gy, B, C).to(dt));
      copy_out(X.grad().to(torch::kFloat32), gx);
    }
    return B;
  });
}

// SparseTensor construction with a quantization mode (sparse_tensor.cpp:62-114,
// 447-481): qmode is SparseTensorQuantizationMode (0 random subsample, 1
// unweighted average, 2 unweighted sum, 3 max pool) over the rows `coords`
// (duplicates allowed) with features x [n, C]. Same conventions as ref_pool.
// Returns the unique row count.
int64_t ref_quantize(const int32_t *coords, int64_t n, int ncol, const float *x, int C, int qmode,
                     int dtype, const float *gy, int64_t out_cap, float *y, int32_t *out_coords,
                     float *gx) {
  return guarded([&]() -> int64_t {
    const int D = ncol - 1;
    const auto dt = dtype == 1 ? torch::kBFloat16 : torch::kFloat32;
    auto mgr = std::make_shared<riemann::CoordinateManager>(D, riemann::CoordinateMapBackend::CPU);
    auto X = float_rows(x, n, C).to(dt).detach().requires_grad_(true);
    riemann::SparseTensor t(X, int_rows(coords, n, ncol), mgr,
                            static_cast<riemann::SparseTensorQuantizationMode::Type>(qmode));
    const int64_t nu = t.F().size(0);
    if (nu > out_cap)
      return nu;
    copy_out(t.F().detach().to(torch::kFloat32), y);
    copy_out(mgr->get_coordinates(t.coordinate_map_key()).to(torch::kInt32), out_coords);
    if (gy != nullptr) {
      t.F().backward(float_rows(gy, nu, C).to(dt));
      copy_out(X.grad().to(torch::kFloat32), gx);
    }
    return nu;
  });
}

// Threads LibTorch's CPU kernels use (the cores a baseline timing uses).
int ref_num_threads() { return at::get_num_threads(); }

} // extern "C"
