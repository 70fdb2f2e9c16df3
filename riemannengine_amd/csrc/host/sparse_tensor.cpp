// SparseTensor over the HIP coordinate manager. Interface and error messages
// follow the reference (RiemannEngine/engine/tensor/sparse_tensor.hpp:18-60,
// sparse_tensor.cpp:62-114, 381-481), so its callers and tests see the same
// behaviour; coordinates live on the device only.
#include "riemann.hpp"

namespace riemann {

namespace {

// The constructor's argument contract (sparse_tensor.cpp:68-74).
void check_feature_coordinate_pair(const at::Tensor &features, const at::Tensor &coordinates) {
  TORCH_CHECK(features.dim() == 2, "Features must be a 2D tensor");
  TORCH_CHECK(coordinates.dim() == 2, "Coordinates must be a 2D tensor");
  TORCH_CHECK(features.size(0) == coordinates.size(0),
              "Features and coordinates must have same number of rows");
  TORCH_CHECK(coordinates.size(1) >= 2,
              "Coordinates must contain a batch column and spatial columns");
  TORCH_CHECK(coordinates.is_cuda(),
              "Coordinates must be a device tensor (the HIP path has no CPU fallback)");
}

// The pooling reduction that merges duplicate coordinates under `mode`, or
// -1 for the modes that pick rows instead of reducing them.
int reduction_of(SparseTensorQuantizationMode::Type mode) {
  switch (mode) {
  case SparseTensorQuantizationMode::UNWEIGHTED_SUM:
    return RHIP_POOL_SUM;
  case SparseTensorQuantizationMode::UNWEIGHTED_AVERAGE:
    return RHIP_POOL_AVG;
  case SparseTensorQuantizationMode::MAX_POOL:
    // scatter_reduce("amax", include_self=False) semantics, gradient included
    return RHIP_POOL_MAX_SCATTER;
  default:
    return -1;
  }
}

} // namespace

SparseTensor::SparseTensor(at::Tensor features, at::Tensor coordinates,
                           std::shared_ptr<CoordinateManager> manager,
                           SparseTensorQuantizationMode::Type quantization_mode,
                           GPUMemoryAllocatorBackend::Type alloc_type,
                           RiemannAlgorithm::Mode algo)
    : features_(std::move(features)), key_(static_cast<size_type>(coordinates.size(1))),
      dimension_(static_cast<int>(coordinates.size(1)) - 1) {
  check_feature_coordinate_pair(features_, coordinates);
  manager_ = manager ? std::move(manager)
                     : std::make_shared<CoordinateManager>(dimension_, CoordinateMapBackend::CUDA,
                                                           alloc_type, algo);
  TORCH_CHECK(manager_->D() == dimension_,
              "Coordinate manager dimension does not match coordinates");
  auto inserted = manager_->insert_and_map(coordinates.to(torch::kInt32).contiguous(),
                                           stride_type(static_cast<size_t>(dimension_), 1));
  key_ = std::move(inserted.first);
  features_ = quantize_features(features_, inserted.second.first, inserted.second.second,
                                manager_->size(key_), quantization_mode);
}

SparseTensor::SparseTensor(at::Tensor features, CoordinateMapKey coordinate_map_key,
                           std::shared_ptr<CoordinateManager> manager)
    : features_(std::move(features)), key_(std::move(coordinate_map_key)),
      manager_(std::move(manager)), dimension_(static_cast<int>(key_.get_coordinate_size()) - 1) {
  // the argument contract of sparse_tensor.cpp:104-113
  TORCH_CHECK(manager_, "Manager must not be null");
  TORCH_CHECK(features_.dim() == 2, "Features must be 2D");
  TORCH_CHECK(key_.is_key_set(), "Coordinate map key must be set");
  TORCH_CHECK(manager_->D() == dimension_,
              "Coordinate manager dimension does not match coordinate key");
  TORCH_CHECK(features_.size(0) == manager_->size(key_),
              "Feature row count must match coordinate map size");
}

at::Tensor SparseTensor::C() const {
  if (!coordinates_.has_value())
    coordinates_ = manager_->get_coordinates(key_);
  return coordinates_.value();
}

SparseTensor SparseTensor::with_features(at::Tensor features) const {
  return SparseTensor(std::move(features), key_, manager_);
}

SparseTensor &SparseTensor::operator+=(const SparseTensor &other) {
  TORCH_CHECK(manager_ == other.manager_, "Cannot add tensors from different managers");
  TORCH_CHECK(key_ == other.key_, "In-place addition requires same key");
  // out of place, so that autograd keeps both operands' history
  features_ = at::add(features_, other.features_);
  return *this;
}

SparseTensor SparseTensor::union_op(const SparseTensor &other, char op) const {
  const char *what = op == '+' ? "add" : op == '-' ? "subtract" : op == '*' ? "multiply"
                                                                            : "divide";
  // the argument contract of sparse_tensor.cpp:331-343
  TORCH_CHECK(dimension_ == other.dimension_, "Cannot ", what,
              " tensors with different dimensions");
  TORCH_CHECK(features_.size(1) == other.features_.size(1), "Cannot ", what,
              " tensors with different feature channel counts");
  TORCH_CHECK(features_.device() == other.features_.device(), "Cannot ", what,
              " tensors on different devices");
  stride_type stride = tensor_stride();
  const stride_type other_stride = other.tensor_stride();
  for (size_t i = 0; i < stride.size() && i < other_stride.size(); ++i)
    stride[i] = std::min(stride[i], other_stride[i]);
  at::DeviceGuard guard(features_.device());
  auto manager = std::make_shared<CoordinateManager>(dimension_, CoordinateMapBackend::CUDA);
  const int64_t n_self = features_.size(0);
  auto inserted = manager->insert_and_map(
      torch::cat({C(), other.C().to(C().device())}, 0).contiguous(), stride);
  const int64_t n = manager->size(inserted.first);
  const at::Tensor &row = inserted.second.second; // union row of every input row
  // each operand's rows are unique, so no two of them share a union row
  auto place = [&](const at::Tensor &f, const at::Tensor &rows) {
    return torch::zeros({n, f.size(1)}, f.options()).index_copy(0, rows, f);
  };
  const at::Tensor a = place(features_, row.slice(0, 0, n_self));
  const at::Tensor b = place(other.features_, row.slice(0, n_self));
  at::Tensor out = op == '+' ? a + b : op == '-' ? a - b : op == '*' ? a * b : a / b;
  return SparseTensor(std::move(out), std::move(inserted.first), std::move(manager));
}

SparseTensor SparseTensor::operator+(const SparseTensor &other) const {
  return union_op(other, '+');
}
SparseTensor SparseTensor::operator-(const SparseTensor &other) const {
  return union_op(other, '-');
}
SparseTensor SparseTensor::operator*(const SparseTensor &other) const {
  return union_op(other, '*');
}
SparseTensor SparseTensor::operator/(const SparseTensor &other) const {
  return union_op(other, '/');
}

SparseTensor SparseTensor::operator+(at::Scalar scalar) const {
  return with_features(at::add(features_, scalar));
}

SparseTensor SparseTensor::operator*(at::Scalar scalar) const {
  return with_features(at::mul(features_, scalar));
}

SparseTensor SparseTensor::to(c10::ScalarType dtype) const {
  return dtype == features_.scalar_type() ? *this : with_features(features_.to(dtype));
}

SparseTensor SparseTensor::float_() const { return to(at::kFloat); }

SparseTensor SparseTensor::double_() const { return to(at::kDouble); }

SparseTensor SparseTensor::to(torch::Device device) const {
  TORCH_CHECK(device.is_cuda(),
              "this build keeps sparse tensors on the device (HIP) coordinate manager; "
              "there is no CPU manager to move to");
  at::DeviceGuard guard(device);
  // The map's rows are unique and in first-occurrence order, so hashing them
  // into a fresh manager numbers them identically: the features move as
  // they are, row for row, with no gather.
  auto fresh = std::make_shared<CoordinateManager>(dimension_, CoordinateMapBackend::CUDA);
  const auto &name = key_.get_key();
  auto inserted = fresh->insert_and_map(C().to(device).contiguous(), name.first, name.second);
  TORCH_CHECK(fresh->size(inserted.first) == features_.size(0),
              "Coordinate map representative rows do not match map size");
  return SparseTensor(features_.to(device), std::move(inserted.first), std::move(fresh));
}

SparseTensor SparseTensor::detach() const { return with_features(features_.detach()); }

at::Tensor SparseTensor::quantize_features(const at::Tensor &features,
                                           const at::Tensor &first_rows,
                                           const at::Tensor &row_to_unique,
                                           int64_t unique_count,
                                           SparseTensorQuantizationMode::Type mode) {
  if (mode == SparseTensorQuantizationMode::NO_QUANTIZATION)
    return features;
  const int reduction = reduction_of(mode);
  if (reduction < 0) {
    TORCH_CHECK(mode == SparseTensorQuantizationMode::RANDOM_SUBSAMPLE,
                "Unknown quantization mode");
    // Unique rows are numbered in first-occurrence order: without
    // duplicates every row is its own first occurrence and nothing moves.
    if (unique_count == features.size(0))
      return features;
    return features.index_select(0, first_rows.to(features.device(), torch::kLong));
  }
  TORCH_CHECK(features.is_cuda(), "quantization runs on the device; got features on ",
              features.device());
  if (features.scalar_type() == torch::kFloat || features.scalar_type() == torch::kBFloat16)
    return hip_group_reduce(features, row_to_unique.to(features.device()), unique_count,
                            reduction);
  // other dtypes (fp64, fp16): torch's own scatter reductions, the operations
  // the reference applies to every dtype (sparse_tensor.cpp:461-477)
  const auto idx = row_to_unique.to(features.device(), torch::kLong);
  auto shape = features.sizes().vec();
  shape[0] = unique_count;
  auto out = torch::zeros(shape, features.options());
  if (reduction == RHIP_POOL_MAX_SCATTER) {
    auto index = idx.view({-1, 1}).expand_as(features);
    return out.scatter_reduce(0, index, features, "amax", /*include_self=*/false);
  }
  out = out.index_add(0, idx, features);
  if (reduction == RHIP_POOL_AVG) {
    auto counts = torch::zeros({unique_count}, features.options())
                      .index_add(0, idx, torch::ones({features.size(0)}, features.options()));
    out = out / counts.view({-1, 1});
  }
  return out;
}

} // namespace riemann
