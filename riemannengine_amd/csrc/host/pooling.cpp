// Pooling layers over the HIP kernels. The reference copies the coordinates
// into a fresh CPU coordinate manager and pools with per-output
// index_select + sum/mean/amax + stack (RiemannEngine/engine/nn/pooling.cpp:
// 17-150); here the maps stay on the device in the input's manager and each
// direction is one C-ABI call (rhip_pool_forward / rhip_pool_backward,
// rhip_global_pool_forward / rhip_global_pool_backward).
#include <ATen/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "riemann.hpp"

namespace riemann {

namespace {

int32_t pool_dtype(const at::Tensor &t) {
  if (t.scalar_type() == torch::kFloat)
    return RHIP_F32;
  if (t.scalar_type() == torch::kBFloat16)
    return RHIP_BF16;
  TORCH_CHECK(false, "the HIP pooling computes fp32 or bf16 features, got ", t.scalar_type());
}

// LOCAL_* and GLOBAL_* modes -> the reduction (pooling.cpp:150-170).
int32_t pool_reduction(PoolingMode::Type mode) {
  switch (mode) {
  case PoolingMode::LOCAL_SUM_POOLING:
  case PoolingMode::GLOBAL_SUM_POOLING_DEFAULT:
  case PoolingMode::GLOBAL_SUM_POOLING_KERNEL:
  case PoolingMode::GLOBAL_SUM_POOLING_PYTORCH_INDEX:
    return RHIP_POOL_SUM;
  case PoolingMode::LOCAL_AVG_POOLING:
  case PoolingMode::GLOBAL_AVG_POOLING_DEFAULT:
  case PoolingMode::GLOBAL_AVG_POOLING_KERNEL:
  case PoolingMode::GLOBAL_AVG_POOLING_PYTORCH_INDEX:
    return RHIP_POOL_AVG;
  default:
    return RHIP_POOL_MAX;
  }
}

bool is_local(PoolingMode::Type mode) {
  return mode == PoolingMode::LOCAL_SUM_POOLING || mode == PoolingMode::LOCAL_AVG_POOLING ||
         mode == PoolingMode::LOCAL_MAX_POOLING;
}

hipStream_t stream_of(const at::Device &dev) {
  return c10::hip::getCurrentHIPStream(dev.index()).stream();
}

at::Tensor byte_buffer(size_t bytes, const at::Device &dev) {
  return torch::empty({static_cast<int64_t>(bytes)},
                      torch::TensorOptions().dtype(torch::kUInt8).device(dev));
}

// Processing orders are optional (an empty tensor = row order).
const int32_t *ptr_or_null(const at::Tensor &t) {
  return t.defined() && t.numel() > 0 ? t.data_ptr<int32_t>() : nullptr;
}

using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

// Inputs after the features are the map's integer tables (no gradient).
struct HipPoolingFunction : public torch::autograd::Function<HipPoolingFunction> {
  static at::Tensor forward(AutogradContext *ctx, at::Tensor features, at::Tensor nbr,
                            at::Tensor out_order, at::Tensor nbr_t, at::Tensor in_order,
                            int64_t n_out, int64_t reduction) {
    TORCH_CHECK(features.is_cuda(), "features must be a device tensor");
    const auto dev = features.device();
    at::DeviceGuard guard(dev);
    auto x = features.contiguous();
    const int64_t n_in = x.size(0), C = x.size(1);
    const int32_t K = static_cast<int32_t>(nbr.size(0));
    TORCH_CHECK(C >= 1, "pooling needs at least one channel");
    auto y = torch::empty({n_out, C}, x.options());
    auto counts = torch::empty({std::max<int64_t>(n_out, 1)},
                               torch::TensorOptions().dtype(torch::kInt32).device(dev));
    check_rhip(rhip_pool_forward(x.data_ptr(), n_in, static_cast<int32_t>(C),
                                 nbr.data_ptr<int32_t>(), K, ptr_or_null(out_order), n_out,
                                 static_cast<int32_t>(reduction), y.data_ptr(),
                                 counts.data_ptr<int32_t>(), pool_dtype(x), stream_of(dev)),
               "rhip_pool_forward");
    ctx->save_for_backward({x, reduction >= RHIP_POOL_MAX ? y : at::Tensor(), nbr, out_order,
                            nbr_t, in_order, counts});
    ctx->saved_data["reduction"] = reduction;
    return y;
  }

  static tensor_list backward(AutogradContext *ctx, tensor_list grads) {
    auto saved = ctx->get_saved_variables();
    auto x = saved[0], y = saved[1], nbr = saved[2], out_order = saved[3], nbr_t = saved[4];
    auto in_order = saved[5], counts = saved[6];
    const int64_t reduction = ctx->saved_data["reduction"].toInt();
    const auto dev = x.device();
    at::DeviceGuard guard(dev);
    const int64_t n_in = x.size(0), C = x.size(1), n_out = nbr.size(1);
    const int32_t K = static_cast<int32_t>(nbr.size(0));
    const int32_t K_t = static_cast<int32_t>(nbr_t.size(0));
    auto gy = grads[0].to(x.scalar_type()).contiguous();
    size_t bytes = 0;
    check_rhip(rhip_pool_workspace_bytes(n_out, static_cast<int32_t>(C),
                                         static_cast<int32_t>(reduction), &bytes),
               "rhip_pool_workspace_bytes");
    auto ws = byte_buffer(bytes, dev);
    auto gx = torch::empty_like(x);
    check_rhip(rhip_pool_backward(gy.data_ptr(), y.defined() ? y.data_ptr() : nullptr,
                                  x.data_ptr(), n_out, static_cast<int32_t>(C),
                                  nbr.data_ptr<int32_t>(), K, ptr_or_null(out_order),
                                  nbr_t.data_ptr<int32_t>(), K_t, ptr_or_null(in_order), n_in,
                                  counts.data_ptr<int32_t>(),
                                  static_cast<int32_t>(reduction), gx.data_ptr(), pool_dtype(x),
                                  ws.data_ptr(), ws.numel(), stream_of(dev)),
               "rhip_pool_backward");
    return {gx, {}, {}, {}, {}, {}, {}};
  }
};

// The batch grouping is computed once in forward and reused by backward.
struct HipGlobalPoolingFunction : public torch::autograd::Function<HipGlobalPoolingFunction> {
  static at::Tensor forward(AutogradContext *ctx, at::Tensor features, at::Tensor coords,
                            at::Tensor members, at::Tensor seg, int64_t n_batches,
                            int64_t reduction) {
    const auto dev = features.device();
    at::DeviceGuard guard(dev);
    auto x = features.contiguous();
    const int64_t n = x.size(0), C = x.size(1);
    size_t bytes = 0;
    check_rhip(rhip_global_pool_workspace_bytes(n, static_cast<int32_t>(C),
                                                static_cast<int32_t>(n_batches), &bytes),
               "rhip_global_pool_workspace_bytes");
    auto ws = byte_buffer(bytes, dev);
    auto y = torch::empty({n_batches, C}, x.options());
    check_rhip(rhip_global_pool_forward(x.data_ptr(), n, static_cast<int32_t>(C),
                                        members.data_ptr<int32_t>(), seg.data_ptr<int32_t>(),
                                        static_cast<int32_t>(n_batches),
                                        static_cast<int32_t>(reduction), y.data_ptr(),
                                        pool_dtype(x), ws.data_ptr(), ws.numel(), stream_of(dev)),
               "rhip_global_pool_forward");
    ctx->save_for_backward({x, reduction == RHIP_POOL_MAX ? y : at::Tensor(), coords, members,
                            seg});
    ctx->saved_data["reduction"] = reduction;
    ctx->saved_data["n_batches"] = n_batches;
    return y;
  }

  static tensor_list backward(AutogradContext *ctx, tensor_list grads) {
    auto saved = ctx->get_saved_variables();
    auto x = saved[0], y = saved[1], coords = saved[2], members = saved[3], seg = saved[4];
    const int64_t reduction = ctx->saved_data["reduction"].toInt();
    const int64_t n_batches = ctx->saved_data["n_batches"].toInt();
    const auto dev = x.device();
    at::DeviceGuard guard(dev);
    const int64_t n = x.size(0), C = x.size(1);
    auto gy = grads[0].to(x.scalar_type()).contiguous();
    size_t bytes = 0;
    check_rhip(rhip_global_pool_workspace_bytes(n, static_cast<int32_t>(C),
                                                static_cast<int32_t>(n_batches), &bytes),
               "rhip_global_pool_workspace_bytes");
    auto ws = byte_buffer(bytes, dev);
    auto gx = torch::empty_like(x);
    check_rhip(rhip_global_pool_backward(
                   gy.data_ptr(), y.defined() ? y.data_ptr() : nullptr, x.data_ptr(),
                   coords.data_ptr<int32_t>(), static_cast<int32_t>(coords.size(1)), n,
                   static_cast<int32_t>(C), members.data_ptr<int32_t>(), seg.data_ptr<int32_t>(),
                   static_cast<int32_t>(n_batches), static_cast<int32_t>(reduction), gx.data_ptr(),
                   pool_dtype(x), ws.data_ptr(), ws.numel(), stream_of(dev)),
               "rhip_global_pool_backward");
    return {gx, {}, {}, {}, {}, {}};
  }
};

// Output stride of a transposed layer: tensor stride / kernel stride, exact
// (detail::stride_tensor_stride, engine/grid/stencil.hpp:55-75).
stride_type transposed_stride(const stride_type &tensor_stride, const stride_type &kernel_stride) {
  stride_type out = tensor_stride;
  for (size_t axis = 0; axis < out.size(); ++axis) {
    TORCH_CHECK(kernel_stride[axis] != 0 && out[axis] % kernel_stride[axis] == 0,
                "Transpose pooling stride must divide tensor stride");
    out[axis] /= kernel_stride[axis];
  }
  return out;
}

// evaluate_pooling (pooling.cpp:17-150) on the device.
SparseTensor evaluate_pooling(const SparseTensor &input,
                              const KernelGenerator::KernelParams &params, PoolingMode::Type mode,
                              bool transpose, bool expand_coordinates) {
  TORCH_CHECK(input.F().is_floating_point(), "Sparse pooling requires floating-point features");
  TORCH_CHECK(input.F().is_cuda(), "features must be device tensors (no CPU pooling path)");
  auto manager = input.coordinate_manager();
  const CoordinateMapKey &in_key = input.coordinate_map_key();
  CoordinateMapKey out_key = in_key;
  if (!transpose) {
    // the output is the strided input map (pooling.cpp:36-40)
    out_key = manager->stride(in_key, params.kernel_stride);
  } else {
    // The reference generates the output in a fresh manager that holds only
    // the input map (pooling.cpp:46-68): the region expansion always runs
    // there unless the output key is the input's own key and expansion is
    // off, in which case the output rows are the input rows. Either way the
    // result becomes a new map of the input's manager (a colliding key gets
    // a random string id).
    const auto ik = in_key.get_key();
    const stride_type out_stride = transposed_stride(ik.first, params.kernel_stride);
    if (out_stride == ik.first && ik.second.empty() && !expand_coordinates) {
      out_key = manager->insert_and_map(input.C(), out_stride, "").first;
    } else {
      const auto offsets = region_offsets(params.region_type, params.kernel_size,
                                          params.kernel_dilation, out_stride,
                                          params.region_offsets);
      out_key = manager->stride_region(in_key, offsets, out_stride, true).first;
    }
  }
  const HipKernelMap &map = manager->kernel_map(in_key, out_key, params.kernel_size,
                                                params.kernel_stride, params.kernel_dilation,
                                                params.region_type, params.region_offsets,
                                                transpose, true);
  auto output = hip_sparse_pooling(input.F(), map, mode);
  TORCH_CHECK(output.size(0) == manager->size(out_key),
              "Pooling feature/map row count mismatch: features=", output.size(0),
              " map=", manager->size(out_key));
  return SparseTensor(std::move(output), out_key, std::move(manager));
}

} // namespace

at::Tensor hip_sparse_pooling(const at::Tensor &features, const HipKernelMap &map,
                              PoolingMode::Type mode) {
  TORCH_CHECK(is_local(mode), "Local pooling requires a local pooling mode");
  TORCH_CHECK(features.dim() == 2 && features.size(0) == map.n_in, "feature rows ",
              features.size(0), " != input map size ", map.n_in);
  if (map.symmetric)
    map.ensure_transposed();
  return HipPoolingFunction::apply(features, map.nbr, map.out_order, map.nbr_t, map.in_order,
                                   map.n_out, pool_reduction(mode));
}

at::Tensor hip_group_reduce(const at::Tensor &features, const at::Tensor &group,
                            int64_t n_groups, int32_t reduction) {
  TORCH_CHECK(features.is_cuda() && group.is_cuda(), "features and groups must be device tensors");
  TORCH_CHECK(features.dim() == 2 && group.dim() == 1 && group.size(0) == features.size(0),
              "one group per feature row");
  const auto dev = features.device();
  at::DeviceGuard guard(dev);
  const hipStream_t st = stream_of(dev);
  const int64_t n = features.size(0);
  auto g = group.to(torch::kInt32).contiguous();
  size_t bytes = 0;
  check_rhip(rhip_stride_map_workspace_bytes(n, n_groups, &bytes),
             "rhip_stride_map_workspace_bytes");
  auto ws = byte_buffer(bytes, dev);
  int32_t kmax = 0;
  check_rhip(rhip_group_map_count(g.data_ptr<int32_t>(), n, n_groups, ws.data_ptr(), ws.numel(),
                                  &kmax, st),
             "rhip_group_map_count");
  auto iopt = torch::TensorOptions().dtype(torch::kInt32).device(dev);
  const int64_t K = std::max<int32_t>(kmax, 1);
  auto nbr = kmax > 0 ? torch::empty({K, std::max<int64_t>(n_groups, 1)}, iopt)
                      : torch::full({K, std::max<int64_t>(n_groups, 1)}, -1, iopt);
  auto nbr_t = kmax > 0 ? torch::empty({1, std::max<int64_t>(n, 1)}, iopt)
                        : torch::full({1, std::max<int64_t>(n, 1)}, -1, iopt);
  auto pairs = torch::empty({2, std::max<int64_t>(n, 1)}, iopt);
  check_rhip(rhip_stride_map_fill(n, n_groups, kmax, nullptr, nullptr, ws.data_ptr(), ws.numel(),
                                  nbr.data_ptr<int32_t>(), nbr_t.data_ptr<int32_t>(),
                                  pairs[0].data_ptr<int32_t>(), pairs[1].data_ptr<int32_t>(), st),
             "rhip_stride_map_fill");
  auto row_order = torch::empty({0}, iopt); // row order on both sides
  return HipPoolingFunction::apply(features, nbr.slice(1, 0, n_groups), row_order,
                                   nbr_t.slice(1, 0, n), row_order, n_groups, reduction);
}

// ------------------------------------------------------------ layers

RiemannPoolingBaseImpl::RiemannPoolingBaseImpl(int kernel_size, int stride, int dilation,
                                               PoolingMode::Type mode, int dimension)
    : kernel_generator_({kernel_size}, {stride}, {dilation}, false, RegionType::HYPER_CUBE, {},
                        false, dimension),
      mode_(mode), dimension_(dimension) {
  TORCH_CHECK(is_local(mode), "Local pooling requires a local pooling mode");
}

RiemannPoolingBaseImpl::RiemannPoolingBaseImpl(KernelGenerator kernel_generator,
                                               PoolingMode::Type mode, int dimension)
    : kernel_generator_(std::move(kernel_generator)), mode_(mode), dimension_(dimension) {
  TORCH_CHECK(is_local(mode), "Local pooling requires a local pooling mode");
}

SparseTensor RiemannPoolingBaseImpl::forward(const SparseTensor &input) {
  TORCH_CHECK(input.dimension() == dimension_, "Input dimension mismatch");
  const auto params = kernel_generator_.get_kernel(input.tensor_stride(), false);
  return evaluate_pooling(input, params, mode_, false, false);
}

RiemannPoolingTransposeImpl::RiemannPoolingTransposeImpl(int kernel_size, int stride,
                                                         int dilation, bool expand_coordinates,
                                                         int dimension)
    : kernel_generator_({kernel_size}, {stride}, {dilation}, true, RegionType::HYPER_CUBE, {},
                        expand_coordinates, dimension),
      dimension_(dimension) {}

RiemannPoolingTransposeImpl::RiemannPoolingTransposeImpl(KernelGenerator kernel_generator,
                                                         int dimension, PoolingMode::Type mode)
    : kernel_generator_(std::move(kernel_generator)), dimension_(dimension), mode_(mode) {
  TORCH_CHECK(is_local(mode_), "Transpose pooling requires a local pooling mode");
}

SparseTensor RiemannPoolingTransposeImpl::forward(const SparseTensor &input) {
  TORCH_CHECK(input.dimension() == dimension_, "Input dimension mismatch");
  const auto params = kernel_generator_.get_kernel(input.tensor_stride(), true);
  return evaluate_pooling(input, params, mode_, true, kernel_generator_.expand_coordinates());
}

RiemannGlobalPoolingImpl::RiemannGlobalPoolingImpl(PoolingMode::Type mode) : mode_(mode) {
  TORCH_CHECK(!is_local(mode), "Global pooling requires a global PoolingMode");
}

SparseTensor RiemannGlobalPoolingImpl::forward(const SparseTensor &input) {
  const auto &features = input.F();
  TORCH_CHECK(features.is_cuda(), "features must be device tensors (no CPU pooling path)");
  const auto dev = features.device();
  at::DeviceGuard guard(dev);
  const hipStream_t st = stream_of(dev);
  const auto coords = input.C().contiguous();
  const int64_t n = coords.size(0);
  const int32_t ncol = static_cast<int32_t>(coords.size(1));
  size_t bytes = 0;
  check_rhip(rhip_global_pool_workspace_bytes(n, 1, 0, &bytes),
             "rhip_global_pool_workspace_bytes");
  auto ws = byte_buffer(bytes, dev);
  int32_t n_batches = 0;
  check_rhip(rhip_batch_count(coords.data_ptr<int32_t>(), n, ncol, ws.data_ptr(), ws.numel(),
                              &n_batches, st),
             "rhip_batch_count");
  auto iopt = torch::TensorOptions().dtype(torch::kInt32).device(dev);
  auto members = torch::empty({std::max<int64_t>(n, 1)}, iopt);
  auto seg = torch::empty({n_batches + 1}, iopt);
  check_rhip(rhip_batch_segments(coords.data_ptr<int32_t>(), n, ncol, n_batches, ws.data_ptr(),
                                 ws.numel(), members.data_ptr<int32_t>(),
                                 seg.data_ptr<int32_t>(), st),
             "rhip_batch_segments");
  auto pooled = HipGlobalPoolingFunction::apply(features, coords, members, seg, n_batches,
                                                pool_reduction(mode_));
  // output rows (b, 0, ..., 0), b = 0 .. n_batches - 1, inserted at the
  // input's tensor stride (pooling.cpp:213-219, 250-258)
  auto out_coords = torch::zeros({n_batches, ncol}, iopt);
  if (n_batches > 0)
    out_coords.select(1, 0).copy_(torch::arange(n_batches, iopt));
  auto inserted = input.coordinate_manager()->insert_and_map(out_coords, input.tensor_stride());
  if (n_batches > 0) {
    TORCH_CHECK(inserted.second.first.numel() == n_batches,
                "Global pooled coordinate map unexpectedly collapsed batches");
    pooled = pooled.index_select(0, inserted.second.first.to(torch::kLong));
  }
  return SparseTensor(std::move(pooled), std::move(inserted.first), input.coordinate_manager());
}

} // namespace riemann
