// SparseTensor over the HIP coordinate manager
// (RiemannEngine/engine/tensor/sparse_tensor.cpp:62-114, 381-387, 447-481).
#include "riemann.hpp"

namespace riemann {

SparseTensor::SparseTensor(at::Tensor features, at::Tensor coordinates,
                           std::shared_ptr<CoordinateManager> manager,
                           SparseTensorQuantizationMode::Type quantization_mode,
                           GPUMemoryAllocatorBackend::Type alloc_type,
                           RiemannAlgorithm::Mode algo)
    : features_(std::move(features)), key_(static_cast<size_type>(coordinates.size(1))),
      dimension_(0) {
  TORCH_CHECK(features_.dim() == 2, "Features must be a 2D tensor");
  TORCH_CHECK(coordinates.dim() == 2, "Coordinates must be a 2D tensor");
  TORCH_CHECK(features_.size(0) == coordinates.size(0),
              "Features and coordinates must have same number of rows");
  TORCH_CHECK(coordinates.size(1) >= 2,
              "Coordinates must contain a batch column and spatial columns");
  TORCH_CHECK(coordinates.is_cuda(),
              "Coordinates must be a device tensor (the HIP path has no CPU fallback)");
  dimension_ = static_cast<int>(coordinates.size(1) - 1);
  if (!manager)
    manager = std::make_shared<CoordinateManager>(dimension_, CoordinateMapBackend::CUDA,
                                                  alloc_type, algo);
  TORCH_CHECK(manager->D() == dimension_,
              "Coordinate manager dimension does not match coordinates");
  manager_ = std::move(manager);
  stride_type unit_stride(static_cast<size_t>(dimension_), 1);
  auto inserted =
      manager_->insert_and_map(coordinates.to(torch::kInt32).contiguous(), unit_stride);
  key_ = std::move(inserted.first);
  features_ = quantize_features(features_, inserted.second.first, inserted.second.second,
                                manager_->size(key_), quantization_mode);
}

SparseTensor::SparseTensor(at::Tensor features, CoordinateMapKey coordinate_map_key,
                           std::shared_ptr<CoordinateManager> manager)
    : features_(std::move(features)), key_(std::move(coordinate_map_key)),
      manager_(std::move(manager)), dimension_(static_cast<int>(key_.get_coordinate_size()) - 1) {
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

SparseTensor &SparseTensor::operator+=(const SparseTensor &other) {
  TORCH_CHECK(manager_ == other.manager_, "Cannot add tensors from different managers");
  TORCH_CHECK(key_ == other.key_, "In-place addition requires same key");
  features_ = features_ + other.features_;
  return *this;
}

SparseTensor SparseTensor::operator+(at::Scalar scalar) const {
  return SparseTensor(features_ + scalar, key_, manager_);
}

SparseTensor SparseTensor::operator*(at::Scalar scalar) const {
  return SparseTensor(features_ * scalar, key_, manager_);
}

SparseTensor SparseTensor::to(c10::ScalarType dtype) const {
  return SparseTensor(features_.to(dtype), key_, manager_);
}

SparseTensor SparseTensor::to(torch::Device device) const {
  TORCH_CHECK(device.is_cuda(),
              "this build keeps sparse tensors on the device (HIP) coordinate manager; "
              "there is no CPU manager to move to");
  at::DeviceGuard guard(device);
  auto coordinates = C().to(device).contiguous();
  auto moved = features_.to(device);
  auto manager = std::make_shared<CoordinateManager>(dimension_, CoordinateMapBackend::CUDA);
  const auto key = key_.get_key();
  auto inserted = manager->insert_and_map(coordinates, key.first, key.second);
  const auto &first_rows = inserted.second.first;
  TORCH_CHECK(first_rows.numel() == manager->size(inserted.first),
              "Coordinate map representative rows do not match map size");
  return SparseTensor(moved.index_select(0, first_rows.to(device, torch::kLong)),
                      std::move(inserted.first), std::move(manager));
}

SparseTensor SparseTensor::detach() const {
  return SparseTensor(features_.detach(), key_, manager_);
}

at::Tensor SparseTensor::quantize_features(const at::Tensor &features,
                                           const at::Tensor &first_rows,
                                           const at::Tensor &row_to_unique,
                                           int64_t unique_count,
                                           SparseTensorQuantizationMode::Type mode) {
  const auto rows = first_rows.to(features.device());
  const auto inv = row_to_unique.to(features.device());
  switch (mode) {
  case SparseTensorQuantizationMode::RANDOM_SUBSAMPLE:
    // the first occurrence of each coordinate keeps its features
    if (features.size(0) == unique_count &&
        at::equal(rows, torch::arange(features.size(0), rows.options())))
      return features;
    return features.index_select(0, rows);
  case SparseTensorQuantizationMode::NO_QUANTIZATION:
    return features;
  default:
    break;
  }
  switch (mode) {
  case SparseTensorQuantizationMode::UNWEIGHTED_SUM:
  case SparseTensorQuantizationMode::UNWEIGHTED_AVERAGE:
  case SparseTensorQuantizationMode::MAX_POOL:
    // fp32 / bf16 device features: the group map and the pooling kernels
    // (deterministic; the max gradient is shared as scatter_reduce's, the
    // zero it starts from counting as a tie); other dtypes use torch's
    // index_add_ / scatter_reduce on the device, as the reference does
    if (features.is_cuda() && (features.scalar_type() == torch::kFloat ||
                               features.scalar_type() == torch::kBFloat16))
      return hip_group_reduce(features, inv, unique_count,
                              mode == SparseTensorQuantizationMode::UNWEIGHTED_SUM
                                  ? RHIP_POOL_SUM
                                  : (mode == SparseTensorQuantizationMode::UNWEIGHTED_AVERAGE
                                         ? RHIP_POOL_AVG
                                         : RHIP_POOL_MAX_SCATTER));
    break;
  default:
    break;
  }
  switch (mode) {
  case SparseTensorQuantizationMode::UNWEIGHTED_SUM:
  case SparseTensorQuantizationMode::UNWEIGHTED_AVERAGE: {
    auto result = torch::zeros({unique_count, features.size(1)}, features.options());
    result.index_add_(0, inv, features);
    if (mode == SparseTensorQuantizationMode::UNWEIGHTED_SUM)
      return result;
    auto counts = torch::zeros({unique_count}, features.options());
    counts.index_add_(0, inv, torch::ones({features.size(0)}, features.options()));
    return result / counts.clamp_min(1).unsqueeze(1);
  }
  case SparseTensorQuantizationMode::MAX_POOL: {
    auto result = torch::zeros({unique_count, features.size(1)}, features.options());
    return at::scatter_reduce(result, 0, inv.unsqueeze(1).expand_as(features), features, "amax",
                              false);
  }
  default:
    break;
  }
  TORCH_CHECK(false, "Unknown quantization mode");
}

} // namespace riemann
