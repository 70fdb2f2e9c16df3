// Convolution layers over the HIP kernels: the gather-GEMM-scatter of
// evaluate_sparse_convolution (RiemannEngine/engine/nn/conv.cpp:9-66) and its
// autograd backward become three C-ABI calls, forward / dX / dW.
#include <ATen/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cmath>

#include "riemann.hpp"

namespace riemann {

namespace {

int32_t rhip_dtype(const at::Tensor &t) {
  if (t.scalar_type() == torch::kFloat)
    return RHIP_F32;
  if (t.scalar_type() == torch::kBFloat16)
    return RHIP_BF16;
  TORCH_CHECK(false, "the HIP convolution computes fp32 or bf16 features, got ",
              t.scalar_type());
}

// Workspace of a layer's calls; with_dw false: the forward, input-gradient
// and bias-gradient calls only (the front of the full layout).
at::Tensor conv_workspace(int32_t K, int64_t cin, int64_t cout, int32_t dt, int64_t n_in,
                          int64_t n_out, int64_t n_pairs, bool with_dw, const at::Device &dev) {
  size_t bytes = 0;
  if (with_dw)
    check_rhip(rhip_conv_workspace_bytes(K, static_cast<int32_t>(cin), static_cast<int32_t>(cout),
                                         dt, n_in, n_out, n_pairs, &bytes),
               "rhip_conv_workspace_bytes");
  else
    check_rhip(rhip_conv_forward_workspace_bytes(K, static_cast<int32_t>(cin),
                                                 static_cast<int32_t>(cout), dt, n_in, n_out,
                                                 &bytes),
               "rhip_conv_forward_workspace_bytes");
  return torch::empty({static_cast<int64_t>(bytes)},
                      torch::TensorOptions().dtype(torch::kUInt8).device(dev));
}

using torch::autograd::AutogradContext;
using torch::autograd::tensor_list;

// Inputs after (features, kernel, bias) are the kernel map's index tensors;
// they are integer tensors, so autograd gives them no gradient. bias is fp32
// [cout], or empty for none (autograd needs a defined tensor for every
// input); the forward adds it to the fp32 sums before rounding. The input
// gradient runs on (dx_table, dx_order) with weight slice wperm[k] for table
// row k (wperm empty: k): the transposed table, or for a symmetric map nbr
// itself with the stencil partners. pairs_dw: the weight gradient takes the
// pair lists (in_rows, out_rows), else the neighbour table.
struct HipConvolutionFunction : public torch::autograd::Function<HipConvolutionFunction> {
  static at::Tensor forward(AutogradContext *ctx, at::Tensor features, at::Tensor kernel,
                            at::Tensor bias, at::Tensor nbr, at::Tensor out_order,
                            at::Tensor dx_table, at::Tensor dx_order, at::Tensor wperm,
                            at::Tensor offsets, at::Tensor in_rows, at::Tensor out_rows,
                            int64_t n_out, int64_t n_pairs, bool pairs_dw) {
    TORCH_CHECK(features.is_cuda() && kernel.is_cuda(),
                "features and kernel must be device tensors");
    TORCH_CHECK(features.scalar_type() == kernel.scalar_type(),
                "features and kernel must share a dtype");
    const auto dev = features.device();
    at::DeviceGuard guard(dev);
    auto x = features.contiguous();
    auto w = kernel.contiguous();
    const int32_t K = static_cast<int32_t>(w.size(0));
    const int64_t cin = w.size(1), cout = w.size(2), n_in = x.size(0);
    TORCH_CHECK(x.size(1) == cin, "feature channels ", x.size(1), " != kernel in-channels ", cin);
    const int32_t dt = rhip_dtype(x);
    auto y = torch::empty({n_out, cout}, x.options());
    auto ws = conv_workspace(K, cin, cout, dt, n_in, n_out, n_pairs, false, dev);
    const bool has_bias = bias.numel() > 0;
    if (has_bias)
      TORCH_CHECK(bias.is_cuda() && bias.scalar_type() == torch::kFloat &&
                      bias.numel() == cout && bias.is_contiguous(),
                  "bias must be a contiguous fp32 device tensor of ", cout, " values");
    check_rhip(rhip_conv_forward(x.data_ptr(), n_in, static_cast<int32_t>(cin), w.data_ptr(), K,
                                 static_cast<int32_t>(cout),
                                 has_bias ? bias.data_ptr<float>() : nullptr,
                                 nbr.data_ptr<int32_t>(),
                                 out_order.data_ptr<int32_t>(), n_out, y.data_ptr(), dt,
                                 ws.data_ptr(), ws.numel(),
                                 c10::hip::getCurrentHIPStream(dev.index()).stream()),
               "rhip_conv_forward");
    ctx->save_for_backward({x, w, dx_table, dx_order, offsets, in_rows, out_rows, nbr, out_order,
                            wperm});
    ctx->saved_data["n_pairs"] = n_pairs;
    ctx->saved_data["pairs_dw"] = pairs_dw;
    ctx->saved_data["n_out"] = n_out;
    ctx->saved_data["has_bias"] = has_bias;
    return y;
  }

  static tensor_list backward(AutogradContext *ctx, tensor_list grads) {
    auto saved = ctx->get_saved_variables();
    auto x = saved[0], w = saved[1], dx_table = saved[2], dx_order = saved[3];
    auto offsets = saved[4], in_rows = saved[5], out_rows = saved[6];
    auto nbr = saved[7], out_order = saved[8], wperm = saved[9];
    const bool pairs_dw = ctx->saved_data["pairs_dw"].toBool();
    const int64_t n_pairs = ctx->saved_data["n_pairs"].toInt();
    const int64_t n_out = ctx->saved_data["n_out"].toInt();
    const auto dev = x.device();
    at::DeviceGuard guard(dev);
    const hipStream_t st = c10::hip::getCurrentHIPStream(dev.index()).stream();
    auto gy = grads[0].to(x.scalar_type()).contiguous();
    const int32_t K = static_cast<int32_t>(w.size(0));
    const int64_t cin = w.size(1), cout = w.size(2), n_in = x.size(0);
    const int32_t dt = rhip_dtype(x);
    const bool need_dw = ctx->needs_input_grad(1);
    auto ws = conv_workspace(K, cin, cout, dt, n_in, n_out, n_pairs, need_dw, dev);
    at::Tensor gx, gw, gb;
    if (ctx->saved_data["has_bias"].toBool() && ctx->needs_input_grad(2)) {
      gb = torch::empty({cout}, x.options().dtype(torch::kFloat));
      check_rhip(rhip_conv_bias_grad(gy.data_ptr(), n_out, static_cast<int32_t>(cout), dt,
                                     gb.data_ptr<float>(), ws.data_ptr(), ws.numel(), st),
                 "rhip_conv_bias_grad");
    }
    if (ctx->needs_input_grad(0)) {
      gx = torch::empty_like(x);
      check_rhip(rhip_conv_backward_input(gy.data_ptr(), n_out, static_cast<int32_t>(cout),
                                          w.data_ptr(), K, static_cast<int32_t>(cin),
                                          dx_table.data_ptr<int32_t>(),
                                          wperm.numel() > 0 ? wperm.data_ptr<int32_t>() : nullptr,
                                          dx_order.data_ptr<int32_t>(), n_in, gx.data_ptr(), dt,
                                          ws.data_ptr(), ws.numel(), st),
                 "rhip_conv_backward_input");
    }
    if (need_dw) {
      gw = torch::empty_like(w);
      int rc;
      if (!pairs_dw) {
        rc = rhip_conv_backward_weight_rows(
            x.data_ptr(), n_in, static_cast<int32_t>(cin), gy.data_ptr(), n_out,
            static_cast<int32_t>(cout), K, nbr.data_ptr<int32_t>(),
            out_order.numel() > 0 ? out_order.data_ptr<int32_t>() : nullptr, gw.data_ptr(), dt,
            ws.data_ptr(), ws.numel(), st);
      } else {
        TORCH_CHECK(in_rows.numel() == n_pairs, "the kernel map's pair lists were not built");
        rc = rhip_conv_backward_weight(x.data_ptr(), n_in, static_cast<int32_t>(cin),
                                       gy.data_ptr(), n_out, static_cast<int32_t>(cout), K,
                                       offsets.data_ptr<int64_t>(), n_pairs,
                                       in_rows.data_ptr<int32_t>(), out_rows.data_ptr<int32_t>(),
                                       gw.data_ptr(), dt, ws.data_ptr(), ws.numel(), st);
      }
      check_rhip(rc, "rhip_conv_backward_weight(_rows)");
    }
    return {gx, gw, gb, {}, {}, {}, {}, {}, {}, {}, {}, {}, {}, {}};
  }
};

} // namespace

at::Tensor hip_sparse_convolution(const at::Tensor &features, const at::Tensor &kernel,
                                  const HipKernelMap &map, const at::Tensor &bias) {
  TORCH_CHECK(kernel.dim() == 3 && kernel.size(0) == map.K, "kernel volume ", kernel.size(0),
              " does not match the kernel map's ", map.K, " offsets");
  TORCH_CHECK(features.size(0) == map.n_in, "feature rows ", features.size(0),
              " != input map size ", map.n_in);
  const at::Tensor b =
      bias.defined() ? bias
                     : torch::empty({0}, features.options().dtype(torch::kFloat));
  // dW from the neighbour table where the library has a kernel for the
  // shape, else from the pair lists (built now, once per map, when a weight
  // gradient may follow). bf16 maps of at most 8 offsets take the pair lists
  // when they hold fewer than 2 pairs per output row (a transposed stride-2
  // map), or pair each input row at most once (a stride-2 map) with channel
  // counts that are multiples of 64 (the per-wave pair kernel). Measured per
  // call: config 3's maps 19 us each against 27 and 46 for the table kernel;
  // config 5's C64->128, 128->256 and 256->256 downs 30, 30 and 27 us
  // against 46, 38 and 33.
  const int32_t dt = rhip_dtype(features);
  const int64_t kin = kernel.size(1), kout = kernel.size(2);
  const bool sparse_small =
      dt == RHIP_BF16 && map.K <= 8 &&
      (map.size() < 2 * map.n_out || (map.size() <= map.n_in && kin % 64 == 0 && kout % 64 == 0));
  const bool pairs_dw =
      sparse_small || rhip_conv_backward_weight_rows_supported(
                          dt, static_cast<int32_t>(kernel.size(1)),
                          static_cast<int32_t>(kernel.size(2)), map.K, map.n_in, map.n_out) == 0;
  const auto iempty = torch::empty({0}, map.nbr.options());
  at::Tensor in_rows = iempty, out_rows = iempty;
  if (pairs_dw && kernel.requires_grad() && torch::autograd::GradMode::is_enabled()) {
    map.ensure_pairs();
    in_rows = map.in_rows;
    out_rows = map.out_rows;
  }
  if (!map.symmetric)
    return HipConvolutionFunction::apply(features, kernel, b, map.nbr, map.out_order, map.nbr_t,
                                         map.in_order, iempty, map.offsets, in_rows, out_rows,
                                         map.n_out, map.size(), pairs_dw);
  return HipConvolutionFunction::apply(features, kernel, b, map.nbr, map.out_order, map.nbr,
                                       map.out_order, map.partner, map.offsets, in_rows, out_rows,
                                       map.n_out, map.size(), pairs_dw);
}

// ------------------------------------------------------------ layers

RiemannConvolutionBaseImpl::RiemannConvolutionBaseImpl(
    int in_channels, int out_channels, int kernel_size, int stride, int dilation, bool bias,
    bool is_transpose, bool expand_coordinates, ConvolutionMode::Type convolution_mode,
    int dimension, RegionType::Type region_type)
    : in_channels_(in_channels), out_channels_(out_channels), is_transpose_(is_transpose),
      use_mm_(false), dimension_(dimension), convolution_mode_(convolution_mode),
      kernel_generator_({kernel_size}, {stride}, {dilation}, is_transpose, region_type, {},
                        expand_coordinates, dimension),
      has_bias_(bias) {
  TORCH_CHECK(in_channels > 0 && out_channels > 0, "Convolution channel counts must be positive");
  const auto volume = kernel_generator_.kernel_volume();
  kernel_ = register_parameter("kernel", torch::empty({volume, in_channels_, out_channels_}));
  if (has_bias_)
    bias_ = register_parameter("bias", torch::empty({1, out_channels_}));
  reset_parameters(is_transpose_);
}

void RiemannConvolutionBaseImpl::reset() { reset_parameters(is_transpose_); }

void RiemannConvolutionBaseImpl::reset_parameters(bool is_transpose) {
  // U(-1/sqrt(fan), 1/sqrt(fan)), fan = channels * kernel volume
  // (engine/nn/conv.cpp:94-102)
  torch::NoGradGuard guard;
  const auto fan = (is_transpose ? out_channels_ : in_channels_) * kernel_generator_.kernel_volume();
  const auto bound = 1.0 / std::sqrt(static_cast<double>(fan));
  kernel_.uniform_(-bound, bound);
  if (bias_.defined())
    bias_.uniform_(-bound, bound);
}

SparseTensor RiemannConvolutionBaseImpl::forward(const SparseTensor &input) {
  TORCH_CHECK(input.dimension() == dimension_, "Input dimension mismatch");
  TORCH_CHECK(input.F().size(1) == in_channels_, "Input channel count does not match convolution");
  const auto params = kernel_generator_.get_kernel(input.tensor_stride(), is_transpose_);
  const auto input_key = input.coordinate_map_key().get_key();
  auto output_stride = input_key.first;
  for (size_t axis = 0; axis < output_stride.size(); ++axis) {
    const auto step = params.kernel_stride[axis];
    if (is_transpose_) {
      TORCH_CHECK(step != 0 && output_stride[axis] % step == 0,
                  "Transpose convolution stride must divide tensor stride");
      output_stride[axis] /= step;
    } else {
      output_stride[axis] *= step;
    }
  }
  CoordinateMapKey output_key(input.coordinate_map_key().get_coordinate_size(),
                              {output_stride, input_key.second});
  auto manager = input.coordinate_manager();
  if (!is_transpose_ && params.kernel_stride != stride_type(dimension_, 1))
    output_key = manager->stride(input.coordinate_map_key(), params.kernel_stride);
  if (is_transpose_ && params.expand_coordinates) {
    // Generative transposed convolution: the output map is generated from
    // the input through the kernel region at the output stride
    // (CoordinateMapManager::stride_region, engine/grid/space_impl.hpp:
    // 352-381), as the reference's transposed pooling builds it
    // (engine/nn/pooling.cpp:46-62); the reference's convolution stores the
    // flag but does not generate (engine/nn/conv.cpp:104-138).
    const auto offsets = region_offsets(params.region_type, params.kernel_size,
                                        params.kernel_dilation, output_stride,
                                        params.region_offsets);
    output_key = manager->stride_region(input.coordinate_map_key(), offsets, output_stride, true)
                     .first;
  }
  const HipKernelMap &map = manager->kernel_map(
      input.coordinate_map_key(), output_key, params.kernel_size, params.kernel_stride,
      params.kernel_dilation, params.region_type, params.region_offsets, is_transpose_, false);
  const auto &x = input.F();
  // the bias is added in the kernel, to the fp32 sums (conv.cpp:135-136 adds
  // it to the output afterwards)
  auto result = hip_sparse_convolution(
      x, kernel_.to(x.scalar_type()), map,
      bias_.defined() ? bias_.to(torch::kFloat).reshape({-1}) : at::Tensor());
  return SparseTensor(std::move(result), output_key, std::move(manager));
}

RiemannConvolutionImpl::RiemannConvolutionImpl(int in_channels, int out_channels, int kernel_size,
                                               int stride, int dilation, bool bias,
                                               bool expand_coordinates,
                                               ConvolutionMode::Type convolution_mode,
                                               int dimension)
    : in_channels_(in_channels), out_channels_(out_channels), kernel_size_(kernel_size),
      stride_(stride), dilation_(dilation), bias_(bias), expand_(expand_coordinates),
      mode_(convolution_mode), dimension_(dimension) {
  base_ = register_module(
      "base", std::make_shared<RiemannConvolutionBaseImpl>(
                  in_channels_, out_channels_, kernel_size_, stride_, dilation_, bias_, false,
                  expand_, mode_, dimension_));
}

void RiemannConvolutionImpl::reset() { base_->reset(); }

SparseTensor RiemannConvolutionImpl::forward(const SparseTensor &input) {
  return base_->forward(input);
}

RiemannConvolutionTransposeImpl::RiemannConvolutionTransposeImpl(
    int in_channels, int out_channels, int kernel_size, int stride, int dilation, bool bias,
    bool expand_coordinates, ConvolutionMode::Type convolution_mode, int dimension)
    : in_channels_(in_channels), out_channels_(out_channels), kernel_size_(kernel_size),
      stride_(stride), dilation_(dilation), bias_(bias), expand_(expand_coordinates),
      mode_(convolution_mode), dimension_(dimension) {
  base_ = register_module(
      "base", std::make_shared<RiemannConvolutionBaseImpl>(
                  in_channels_, out_channels_, kernel_size_, stride_, dilation_, bias_, true,
                  expand_, mode_, dimension_));
}

void RiemannConvolutionTransposeImpl::reset() { base_->reset(); }

SparseTensor RiemannConvolutionTransposeImpl::forward(const SparseTensor &input) {
  return base_->forward(input);
}

RiemannGenerativeConvolutionTransposeImpl::RiemannGenerativeConvolutionTransposeImpl(
    int in_channels, int out_channels, int kernel_size, int stride, int dilation, bool bias,
    ConvolutionMode::Type convolution_mode, int dimension)
    : in_channels_(in_channels), out_channels_(out_channels), kernel_size_(kernel_size),
      stride_(stride), dilation_(dilation), bias_(bias), mode_(convolution_mode),
      dimension_(dimension) {
  base_ = register_module(
      "base", std::make_shared<RiemannConvolutionBaseImpl>(
                  in_channels_, out_channels_, kernel_size_, stride_, dilation_, bias_, true,
                  true, mode_, dimension_));
}

void RiemannGenerativeConvolutionTransposeImpl::reset() { base_->reset(); }

SparseTensor RiemannGenerativeConvolutionTransposeImpl::forward(const SparseTensor &input) {
  return base_->forward(input);
}

} // namespace riemann
