// RiemannBatchNorm, RiemannReLU and BasicBlock: the config-5 callers of the
// convolution (RiemannEngine/engine/nn/normalization.hpp:11-37,
// residual.cpp:16-52). Normalisation and activation are LibTorch ops on the
// feature matrix; the coordinate key and manager pass through unchanged.
#include "riemann.hpp"

namespace riemann {

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
  const auto &x = input.F();
  // batch statistics in fp32 for bf16 features, result in the feature dtype
  auto values = x.scalar_type() == torch::kBFloat16
                    ? normalization_->forward(x.to(torch::kFloat)).to(x.scalar_type())
                    : normalization_->forward(x);
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

SparseTensor BasicBlockImpl::forward(const SparseTensor &input) {
  auto residual = input;
  auto output = relu_->forward(norm1_->forward(conv1_->forward(input)));
  output = norm2_->forward(conv2_->forward(output));
  if (has_downsample_)
    residual = downsample_.forward<SparseTensor>(input);
  output += residual;
  return relu_->forward(output);
}

} // namespace riemann
