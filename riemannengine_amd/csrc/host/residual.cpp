// RiemannBatchNorm, RiemannReLU and BasicBlock: the config-5 callers of the
// convolution (RiemannEngine/engine/nn/normalization.hpp:11-37,
// residual.cpp:16-52). Batch normalisation of fp32 / bf16 device features
// runs through the HIP kernels (rhip_bn_*) with torch BatchNorm1d's
// semantics; BasicBlock folds its ReLUs and the residual addition into the
// normalisation passes. The coordinate key and manager pass through
// unchanged.
#include <ATen/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "riemann.hpp"

namespace riemann {

namespace {

hipStream_t stream_of(const at::Device &dev) {
  return c10::hip::getCurrentHIPStream(dev.index()).stream();
}

at::Tensor byte_buffer(size_t bytes, const at::Device &dev) {
  return torch::empty({static_cast<int64_t>(bytes)},
                      torch::TensorOptions().dtype(torch::kUInt8).device(dev));
}

int32_t norm_dtype(const at::Tensor &t) {
  return t.scalar_type() == torch::kBFloat16 ? RHIP_BF16 : RHIP_F32;
}

// Optional tensors travel through autograd as empty tensors.
bool present(const at::Tensor &t) { return t.defined() && t.numel() > 0; }
const float *fptr(const at::Tensor &t) { return present(t) ? t.data_ptr<float>() : nullptr; }
float *fptr_mut(at::Tensor &t) { return present(t) ? t.data_ptr<float>() : nullptr; }

using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

// act(batch_norm(features) [+ residual]), act = ReLU when `relu`. With
// batch_stats the statistics are the batch's (running ones updated when
// given), otherwise running_mean / running_var normalise.
struct HipBatchNormFunction : public torch::autograd::Function<HipBatchNormFunction> {
  static at::Tensor forward(AutogradContext *ctx, at::Tensor features, at::Tensor residual,
                            at::Tensor weight, at::Tensor bias, at::Tensor running_mean,
                            at::Tensor running_var, bool batch_stats, bool update, double eps,
                            double momentum, bool relu) {
    const auto dev = features.device();
    at::DeviceGuard guard(dev);
    auto x = features.contiguous();
    const int64_t n = x.size(0), C = x.size(1);
    const auto f32 = torch::TensorOptions().dtype(torch::kFloat).device(dev);
    auto res = present(residual) ? residual.to(x.scalar_type()).contiguous() : at::Tensor();
    TORCH_CHECK(!res.defined() || res.sizes() == x.sizes(),
                "residual features do not match the normalised features");
    at::Tensor mean, invstd;
    const hipStream_t stream = stream_of(dev);
    if (batch_stats) {
      mean = torch::empty({C}, f32);
      invstd = torch::empty({C}, f32);
      if (n > 0) {
        size_t bytes = 0;
        check_rhip(rhip_bn_workspace_bytes(n, static_cast<int32_t>(C), &bytes),
                   "rhip_bn_workspace_bytes");
        auto ws = byte_buffer(bytes, dev);
        check_rhip(rhip_bn_stats(x.data_ptr(), n, static_cast<int32_t>(C), norm_dtype(x), eps,
                                 momentum, update ? fptr_mut(running_mean) : nullptr,
                                 update ? fptr_mut(running_var) : nullptr,
                                 mean.data_ptr<float>(), invstd.data_ptr<float>(),
                                 ws.data_ptr(), ws.numel(), stream),
                   "rhip_bn_stats");
      }
    } else {
      mean = running_mean.clone(); // later training steps update the buffer in place
      invstd = torch::empty({C}, f32);
      check_rhip(rhip_bn_invstd(running_var.data_ptr<float>(), static_cast<int32_t>(C), eps,
                                invstd.data_ptr<float>(), stream),
                 "rhip_bn_invstd");
    }
    auto y = torch::empty_like(x);
    check_rhip(rhip_bn_forward(x.data_ptr(), n, static_cast<int32_t>(C), mean.data_ptr<float>(),
                               invstd.data_ptr<float>(), fptr(weight), fptr(bias),
                               res.defined() ? res.data_ptr() : nullptr, relu ? 1 : 0,
                               y.data_ptr(), norm_dtype(x), stream),
               "rhip_bn_forward");
    ctx->save_for_backward({x, relu ? y : at::Tensor(), mean, invstd, weight});
    ctx->saved_data["batch_stats"] = batch_stats;
    ctx->saved_data["relu"] = relu;
    ctx->saved_data["residual"] = res.defined();
    return y;
  }

  static tensor_list backward(AutogradContext *ctx, tensor_list grads) {
    auto saved = ctx->get_saved_variables();
    auto x = saved[0], y = saved[1], mean = saved[2], invstd = saved[3], weight = saved[4];
    const bool batch_stats = ctx->saved_data["batch_stats"].toBool();
    const bool relu = ctx->saved_data["relu"].toBool();
    const bool has_residual = ctx->saved_data["residual"].toBool();
    const auto dev = x.device();
    at::DeviceGuard guard(dev);
    const int64_t n = x.size(0), C = x.size(1);
    const auto f32 = torch::TensorOptions().dtype(torch::kFloat).device(dev);
    auto gy = grads[0].to(x.scalar_type()).contiguous();
    at::Tensor gx, gres, gw, gb;
    if (ctx->needs_input_grad(0))
      gx = torch::empty_like(x);
    if (has_residual && ctx->needs_input_grad(1))
      gres = torch::empty_like(x);
    // the kernels write every parameter gradient; zeros only for no rows
    auto param_grad = [&] { return n > 0 ? torch::empty({C}, f32) : torch::zeros({C}, f32); };
    if (present(weight) && ctx->needs_input_grad(2))
      gw = param_grad();
    if (present(weight) && ctx->needs_input_grad(3))
      gb = param_grad();
    if (n > 0 && (gx.defined() || gres.defined() || gw.defined() || gb.defined())) {
      size_t bytes = 0;
      check_rhip(rhip_bn_workspace_bytes(n, static_cast<int32_t>(C), &bytes),
                 "rhip_bn_workspace_bytes");
      auto ws = byte_buffer(bytes, dev);
      check_rhip(rhip_bn_backward(gy.data_ptr(), relu ? y.data_ptr() : nullptr, x.data_ptr(), n,
                                  static_cast<int32_t>(C), mean.data_ptr<float>(),
                                  invstd.data_ptr<float>(), fptr(weight), relu ? 1 : 0,
                                  batch_stats ? 1 : 0, gx.defined() ? gx.data_ptr() : nullptr,
                                  gres.defined() ? gres.data_ptr() : nullptr, fptr_mut(gw),
                                  fptr_mut(gb), norm_dtype(x), ws.data_ptr(), ws.numel(),
                                  stream_of(dev)),
                 "rhip_bn_backward");
    }
    return {gx, gres, gw, gb, {}, {}, {}, {}, {}, {}, {}};
  }
};

} // namespace

RiemannBatchNormImpl::RiemannBatchNormImpl(int64_t num_features, double eps, double momentum,
                                           bool affine, bool track_running_stats)
    : num_features_(num_features), eps_(eps), momentum_(momentum), affine_(affine),
      track_(track_running_stats) {
  normalization_ = register_module(
      "normalization",
      torch::nn::BatchNorm1d(torch::nn::BatchNorm1dOptions(num_features)
                                 .eps(eps)
                                 .momentum(momentum)
                                 .affine(affine)
                                 .track_running_stats(track_running_stats)));
}

void RiemannBatchNormImpl::reset() { normalization_->reset(); }

void RiemannBatchNormImpl::to(torch::Dtype, bool) {}

void RiemannBatchNormImpl::to(torch::Device device, torch::Dtype, bool non_blocking) {
  torch::nn::Module::to(device, non_blocking);
}

SparseTensor RiemannBatchNormImpl::forward(const SparseTensor &input) {
  return forward_fused(input, nullptr, false);
}

SparseTensor RiemannBatchNormImpl::forward_fused(const SparseTensor &input,
                                                 const SparseTensor *residual, bool relu) {
  const auto &x = input.F();
  TORCH_CHECK(x.dim() == 2 && x.size(1) == num_features_, "RiemannBatchNorm expects [N, ",
              num_features_, "] features, got ", x.sizes());
  if (residual) {
    // SparseTensor::operator+= (RiemannEngine/engine/tensor/sparse_tensor.cpp:381-387)
    TORCH_CHECK(input.coordinate_manager() == residual->coordinate_manager(),
                "Cannot add tensors from different managers");
    TORCH_CHECK(input.coordinate_map_key() == residual->coordinate_map_key(),
                "In-place addition requires same key");
  }
  const bool hip = x.is_cuda() && (x.scalar_type() == torch::kFloat ||
                                   x.scalar_type() == torch::kBFloat16);
  if (!hip) {
    // other dtypes: torch's own BatchNorm1d, as the reference runs it
    auto values = normalization_->forward(x);
    if (residual)
      values = values + residual->F();
    if (relu)
      values = torch::relu(values);
    return SparseTensor(std::move(values), input.coordinate_map_key(),
                        input.coordinate_manager());
  }
  auto &bn = *normalization_;
  const bool training = bn.is_training();
  const bool update = training && track_;
  if (update) {
    torch::NoGradGuard no_grad;
    bn.num_batches_tracked += 1;
  }
  auto empty = torch::empty({0}, x.options().dtype(torch::kFloat));
  auto values = HipBatchNormFunction::apply(
      x, residual ? residual->F() : empty, affine_ ? bn.weight : empty,
      affine_ ? bn.bias : empty, track_ ? bn.running_mean : empty,
      track_ ? bn.running_var : empty, training || !track_, update, eps_, momentum_, relu);
  return SparseTensor(std::move(values), input.coordinate_map_key(), input.coordinate_manager());
}

SparseTensor RiemannReLUImpl::forward(const SparseTensor &input) {
  // out of place: the features may be saved for a backward pass
  auto values = torch::relu(input.F());
  return SparseTensor(std::move(values), input.coordinate_map_key(), input.coordinate_manager());
}

BasicBlockImpl::BasicBlockImpl(int inplanes, int planes, int stride, int dilation,
                               torch::nn::AnyModule downsample, double bn_momentum, int dimension)
    : downsample_(std::move(downsample)), inplanes_(inplanes), planes_(planes), stride_(stride),
      dilation_(dilation), dimension_(dimension), bn_momentum_(bn_momentum),
      has_downsample_(!downsample_.is_empty()) {
  TORCH_CHECK(inplanes > 0 && planes > 0, "Block channels must be positive");
  TORCH_CHECK(stride > 0 && dilation > 0, "Block stride and dilation must be positive");
  TORCH_CHECK(dimension > 0, "Dimension must be positive");
  conv1_ = register_module("conv1", RiemannConvolution(inplanes_, planes_, 3, stride_, dilation_,
                                                       false, false, ConvolutionMode::DEFAULT,
                                                       dimension_));
  norm1_ = register_module("norm1", RiemannBatchNorm(planes_, 1e-5, bn_momentum_));
  conv2_ = register_module("conv2", RiemannConvolution(planes_, planes_, 3, 1, dilation_, false,
                                                       false, ConvolutionMode::DEFAULT,
                                                       dimension_));
  norm2_ = register_module("norm2", RiemannBatchNorm(planes_, 1e-5, bn_momentum_));
  relu_ = register_module("relu", RiemannReLU(true));
  if (has_downsample_)
    register_module("downsample", downsample_.ptr());
}

void BasicBlockImpl::reset() {
  conv1_->reset();
  conv2_->reset();
  norm1_->reset();
  norm2_->reset();
}

// relu(norm1(conv1)) and relu(norm2(conv2) + residual) are one batch-norm
// call each: the activation and the addition ride on the normalisation pass.
SparseTensor BasicBlockImpl::forward(const SparseTensor &input) {
  auto output = norm1_->forward_fused(conv1_->forward(input), nullptr, true);
  output = conv2_->forward(output);
  auto residual = has_downsample_ ? downsample_.forward<SparseTensor>(input) : input;
  return norm2_->forward_fused(output, &residual, true);
}

} // namespace riemann
