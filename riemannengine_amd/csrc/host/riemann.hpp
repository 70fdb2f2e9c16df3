// Host side of the MI355X sparse-convolution path: the RiemannEngine
// SparseTensor / CoordinateManager / RiemannConvolution interface over
// LibTorch, with every kernel behind the C ABI of riemann_hip.h.
//
// Names, argument meaning and error behaviour follow the reference:
//   CoordinateMapKey            RiemannEngine/engine/grid/key.hpp:18-99
//   enums, key tuple types      RiemannEngine/engine/foundation/types.hpp:51-165
//   KernelGenerator             RiemannEngine/engine/grid/stencil.hpp:533-598,
//                               stencil.cpp:81-229
//   CoordinateManager           RiemannEngine/engine/grid/space.hpp:817-906,
//                               space_impl.hpp:258-350, 515-706
//   SparseTensor                RiemannEngine/engine/tensor/sparse_tensor.hpp:16-80
//   RiemannConvolution{,Transpose,GenerativeTranspose}
//                               RiemannEngine/engine/nn/conv.hpp:13-90
//   RiemannBatchNorm, BasicBlock
//                               RiemannEngine/engine/nn/normalization.hpp:11-37,
//                               residual.hpp:12-29
//   Riemann{Sum,Avg,Max}Pooling, RiemannPoolingTranspose, RiemannGlobal*Pooling
//                               RiemannEngine/engine/nn/pooling.hpp:11-131
// Only the device (HIP) backend exists here: a CPU coordinate manager or CPU
// coordinates raise an error instead of falling back to another path.
#pragma once

#include <torch/torch.h>

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "riemann_hip.h"

namespace riemann {

// ------------------------------------------------------------------ types

using index_type = uint32_t;
using size_type = uint32_t;
using stride_type = std::vector<uint32_t>;
using coordinate_map_key_type = std::pair<stride_type, std::string>;

namespace SparseTensorQuantizationMode {
enum Type {
  RANDOM_SUBSAMPLE = 0,
  UNWEIGHTED_AVERAGE = 1,
  UNWEIGHTED_SUM = 2,
  MAX_POOL = 3,
  NO_QUANTIZATION = 4
};
}
namespace GPUMemoryAllocatorBackend {
enum Type { PYTORCH = 0, CUDA = 1 };
}
namespace RiemannAlgorithm {
enum Mode { DEFAULT = 0, MEMORY_EFFICIENT = 1, SPEED_OPTIMIZED = 2 };
}
namespace CoordinateMapBackend {
enum Type { CPU = 0, CUDA = 1 };
}
namespace RegionType {
enum Type { HYPER_CUBE, HYPER_CROSS, CUSTOM };
}
namespace ConvolutionMode {
enum Type { DEFAULT, DIRECT_GEMM, COPY_GEMM };
}
namespace PoolingMode {
enum Type {
  LOCAL_SUM_POOLING,
  LOCAL_AVG_POOLING,
  LOCAL_MAX_POOLING,
  GLOBAL_SUM_POOLING_DEFAULT,
  GLOBAL_AVG_POOLING_DEFAULT,
  GLOBAL_MAX_POOLING_DEFAULT,
  GLOBAL_SUM_POOLING_KERNEL,
  GLOBAL_AVG_POOLING_KERNEL,
  GLOBAL_MAX_POOLING_KERNEL,
  GLOBAL_SUM_POOLING_PYTORCH_INDEX,
  GLOBAL_AVG_POOLING_PYTORCH_INDEX,
  GLOBAL_MAX_POOLING_PYTORCH_INDEX
};
}

// (in key, out key, kernel size, kernel stride, dilation, region type,
//  transpose flag, pooling flag): identity of one cached kernel map.
using kernel_map_key_type =
    std::tuple<coordinate_map_key_type, coordinate_map_key_type, stride_type, stride_type,
               stride_type, RegionType::Type, bool, bool>;

// Raises c10::Error with the library's message when a C-ABI call fails.
void check_rhip(int status, const char *what);

// ---------------------------------------------------------------- map key

class CoordinateMapKey {
public:
  CoordinateMapKey() = delete;
  explicit CoordinateMapKey(size_type coordinate_size);
  CoordinateMapKey(size_type coordinate_size, const coordinate_map_key_type &key);
  CoordinateMapKey(stride_type tensor_stride, std::string string_id = "");

  size_type get_coordinate_size() const { return coordinate_size_; }
  void set_key(stride_type tensor_stride, std::string string_id);
  void set_key(const coordinate_map_key_type &key);
  coordinate_map_key_type get_key() const;
  bool is_key_set() const noexcept { return key_set_; }
  stride_type get_tensor_stride() const { return key_.first; }
  uint64_t hash() const;
  bool operator==(const CoordinateMapKey &other) const;
  std::string to_string() const;

private:
  bool key_set_;
  size_type coordinate_size_;
  coordinate_map_key_type key_;
};

// ------------------------------------------------------------ kernel region

// Scaled lattice offsets [K, D] (int32, host) of a region: kernel index k ->
// offset, as kernel_region::coordinate_at enumerates them
// (RiemannEngine/engine/grid/stencil.hpp:223-278). custom: [K, D] int32
// lattice offsets for RegionType::CUSTOM.
at::Tensor region_offsets(RegionType::Type region, const stride_type &kernel_size,
                          const stride_type &dilation, const stride_type &tensor_stride,
                          const at::Tensor &custom = {});
int region_volume(RegionType::Type region, const stride_type &kernel_size,
                  const at::Tensor &custom);

// CUSTOM offsets as a dense int32 [N, D] host tensor (the reference's
// detail::normalize_region_offsets, engine/grid/stencil.cpp:11-36).
at::Tensor normalize_region_offsets(const at::Tensor &offsets, int dimension);

class KernelGenerator {
public:
  struct KernelParams {
    stride_type kernel_size;
    stride_type kernel_stride;
    stride_type kernel_dilation;
    RegionType::Type region_type;
    at::Tensor region_offsets;
    bool expand_coordinates;
    int D;
  };

  KernelGenerator(torch::IntArrayRef kernel_size, torch::IntArrayRef stride = {1},
                  torch::IntArrayRef dilation = {1}, bool is_transpose = false,
                  RegionType::Type region_type = RegionType::HYPER_CUBE,
                  at::Tensor region_offsets = {}, bool expand_coordinates = false,
                  int dimension = -1);

  int kernel_volume() const { return kernel_volume_; }
  const stride_type &kernel_size() const { return kernel_size_; }
  const stride_type &kernel_stride() const { return kernel_stride_; }
  const stride_type &kernel_dilation() const { return kernel_dilation_; }
  RegionType::Type region_type() const { return region_type_; }
  at::Tensor region_offsets() const {
    return region_offsets_.defined() ? region_offsets_.clone() : at::Tensor{};
  }
  bool expand_coordinates() const { return expand_coordinates_; }
  int dimension() const { return D_; }
  KernelParams get_kernel(const stride_type &tensor_stride, bool is_transpose) const;

private:
  stride_type kernel_size_, kernel_stride_, kernel_dilation_;
  bool is_transpose_;
  RegionType::Type region_type_;
  at::Tensor region_offsets_;
  bool expand_coordinates_;
  int D_;
  int kernel_volume_;
};

// ------------------------------------------------------- coordinate maps

// One coordinate map on the device: unique rows, the hash table over them
// and a locality order of the rows.
struct CoordinateMapHIP {
  at::Tensor storage;   // [n_in_rows, D+1] int32 buffer the unique rows live in
  at::Tensor coords;    // [n, D+1] int32 view of the unique rows
  at::Tensor slots;     // hash slots (bytes)
  at::Tensor order;     // [n] int32 locality order (Morton, else packed key)
  at::Tensor bricks;    // brick index over `order` (bytes; table.bricks NULL if none)
  rhip_table table;
  stride_type tensor_stride;
  int64_t size() const { return table.n_unique; }
};

// A kernel map: the dense neighbour table and processing order the
// convolution kernels consume, the per-offset pair counts (CSR) and, built on
// first use, the per-offset pair lists and the transposed table. A pooling
// stride map (stride_map set) has the reference's single pair list (offsets
// = [0, P]), an nbr K rows high (K = most inputs on one output) and a one-row
// nbr_t (each input has one output); swapped() exchanges the two tables.
// A symmetric map (a set onto itself, stencil closed under negation) keeps
// no transposed table: its input gradient runs on nbr with the stencil
// partners as weight permutation (rhip_conv_backward_input).
struct HipKernelMap {
  int32_t K = 0;
  bool stride_map = false;
  bool symmetric = false;
  int64_t n_in = 0, n_out = 0;
  std::vector<int64_t> offsets_host; // [K+1]
  at::Tensor offsets;                // device int64 [K+1]
  at::Tensor nbr;                    // int32 [K, n_out], -1 = no neighbour
  at::Tensor out_order;              // int32 output processing order
  std::vector<int32_t> partner_host; // symmetric: the offset that negates each offset
  at::Tensor partner;                // the same on the device (int32 [K])
  // built on first use (a cached map is shared as const): ensure_pairs(),
  // ensure_transposed()
  mutable at::Tensor in_rows, out_rows; // int32 [P]
  mutable at::Tensor nbr_t;             // int32 [K, n_in]
  mutable at::Tensor in_order;          // int32 input processing order
  int64_t size() const { return offsets_host.empty() ? 0 : offsets_host.back(); }
  // the pair lists from the table (rhip_kmap_pairs), once
  void ensure_pairs() const;
  // the transposed table of a symmetric map (rows of nbr under the partner
  // offsets) and its input order (the output order), once
  void ensure_transposed() const;
  // in and out exchanged (transposed convolution), zero copy once both
  // sides are built
  HipKernelMap swapped() const;
  // the reference's cpu_kernel_map layout: (in rows per offset, out rows per
  // offset), as int64 device tensors
  std::pair<std::vector<at::Tensor>, std::vector<at::Tensor>> per_offset() const;
};

class CoordinateManager {
public:
  CoordinateManager(int D, CoordinateMapBackend::Type backend = CoordinateMapBackend::CUDA,
                    GPUMemoryAllocatorBackend::Type alloc_type = GPUMemoryAllocatorBackend::PYTORCH,
                    RiemannAlgorithm::Mode algo = RiemannAlgorithm::DEFAULT);

  // Deduplicate coordinates (first occurrence wins) into a new map keyed by
  // (tensor_stride, string_id); a key collision picks a random string id.
  // Returns (key, (mapping = first input row per unique row, inverse = unique
  // row per input row)), both int64 on the device.
  std::pair<CoordinateMapKey, std::pair<at::Tensor, at::Tensor>>
  insert_and_map(const at::Tensor &coordinates, stride_type tensor_stride,
                 std::string string_id = "");

  // Output map of a strided convolution: (b, floor(x / s) * s) deduplicated,
  // keyed by (in stride * kernel stride, same string id). Reuses the map if
  // the key exists.
  CoordinateMapKey stride(const CoordinateMapKey &in_key, const stride_type &kernel_stride,
                          std::string string_id = "");

  // Generated map of a generative transposed convolution
  // (CoordinateMapManager::stride_region, engine/grid/space_impl.hpp:352-381):
  // the unique rows of c + offsets[k] over the input map's rows c, offsets
  // the region [K, D] (int32, host) at out_tensor_stride. Keyed by
  // (out_tensor_stride, ""); built when that key is new or `expand` is set
  // (then under a random id if the key exists). Returns (key, built).
  std::pair<CoordinateMapKey, bool> stride_region(const CoordinateMapKey &in_key,
                                                  const at::Tensor &offsets,
                                                  const stride_type &out_tensor_stride,
                                                  bool expand);

  at::Tensor get_coordinates(const CoordinateMapKey &key) const;
  uint32_t size(const CoordinateMapKey &key) const;
  bool exists(const CoordinateMapKey &key) const;

  // Cached kernel map between two maps of this manager (reference semantics:
  // empty if either side is empty; a transposed map reuses the swapped
  // forward map when cached, else generates out -> in with the region on the
  // finer map's stride and swaps).
  const HipKernelMap &kernel_map(const CoordinateMapKey &in_key, const CoordinateMapKey &out_key,
                                 const stride_type &kernel_size,
                                 const stride_type &kernel_stride,
                                 const stride_type &kernel_dilation,
                                 RegionType::Type region_type, const at::Tensor &offsets,
                                 bool is_transpose, bool is_pool);

  const CoordinateMapHIP &coordinate_map(const CoordinateMapKey &key) const;
  size_t kernel_map_cache_size() const { return kernel_maps_.size() + custom_maps_.size(); }
  int D() const { return D_; }
  CoordinateMapBackend::Type backend() const { return backend_; }
  std::string to_string() const;

private:
  coordinate_map_key_type random_key(const stride_type &tensor_stride,
                                     const std::string &string_id) const;
  CoordinateMapHIP build_map(const at::Tensor &coordinates, const stride_type &tensor_stride,
                             at::Tensor *mapping, at::Tensor *inverse) const;
  HipKernelMap generate(const CoordinateMapHIP &in_map, const CoordinateMapHIP &out_map,
                        const at::Tensor &offsets_host) const;
  // Every in_map row onto the out_map row of its floor-aligned coordinates
  // (CoordinateMapCPU::stride_map, engine/grid/lattice_cpu.hpp:675-710).
  HipKernelMap generate_stride_map(const CoordinateMapHIP &in_map,
                                   const CoordinateMapHIP &out_map) const;

  int D_;
  CoordinateMapBackend::Type backend_;
  GPUMemoryAllocatorBackend::Type alloc_type_;
  RiemannAlgorithm::Mode algo_;
  std::map<coordinate_map_key_type, CoordinateMapHIP> maps_;
  std::map<kernel_map_key_type, HipKernelMap> kernel_maps_;
  std::map<std::pair<kernel_map_key_type, std::vector<int32_t>>, HipKernelMap> custom_maps_;
};

// ------------------------------------------------------------ sparse tensor

class SparseTensor {
public:
  SparseTensor(at::Tensor features, at::Tensor coordinates,
               std::shared_ptr<CoordinateManager> manager = nullptr,
               SparseTensorQuantizationMode::Type quantization_mode =
                   SparseTensorQuantizationMode::RANDOM_SUBSAMPLE,
               GPUMemoryAllocatorBackend::Type alloc_type = GPUMemoryAllocatorBackend::PYTORCH,
               RiemannAlgorithm::Mode algo = RiemannAlgorithm::DEFAULT);
  SparseTensor(at::Tensor features, CoordinateMapKey coordinate_map_key,
               std::shared_ptr<CoordinateManager> manager);

  const at::Tensor &F() const noexcept { return features_; }
  at::Tensor C() const;
  const CoordinateMapKey &coordinate_map_key() const noexcept { return key_; }
  std::shared_ptr<CoordinateManager> coordinate_manager() const noexcept { return manager_; }
  stride_type tensor_stride() const { return key_.get_tensor_stride(); }
  int dimension() const noexcept { return dimension_; }
  torch::Device device() const { return features_.device(); }
  c10::ScalarType dtype() const { return features_.scalar_type(); }
  bool requires_grad() const { return features_.requires_grad(); }

  SparseTensor &operator+=(const SparseTensor &other);
  // Elementwise over the union of both operands' coordinates
  // (sparse_tensor.cpp:32-57, 331-379): the rows of both go through one
  // dedup hash build on a fresh manager at the finer tensor stride, each
  // operand's features land on their union rows and the other rows hold 0.
  SparseTensor operator+(const SparseTensor &other) const;
  SparseTensor operator-(const SparseTensor &other) const;
  SparseTensor operator*(const SparseTensor &other) const;
  SparseTensor operator/(const SparseTensor &other) const;
  SparseTensor operator+(at::Scalar scalar) const;
  SparseTensor operator*(at::Scalar scalar) const;
  SparseTensor to(c10::ScalarType dtype) const;
  SparseTensor float_() const;
  SparseTensor double_() const;
  // Re-hash onto `device` (RiemannEngine/engine/tensor/sparse_tensor.cpp:
  // 397-429): a new manager holding this map's rows, features aligned to its
  // representative rows. Device targets only (there is no CPU manager).
  SparseTensor to(torch::Device device) const;
  SparseTensor detach() const;

private:
  // The same map and manager with other features.
  SparseTensor with_features(at::Tensor features) const;
  // The union operation behind operator+, -, * and / (op: '+', '-', '*', '/').
  SparseTensor union_op(const SparseTensor &other, char op) const;
  static at::Tensor quantize_features(const at::Tensor &features, const at::Tensor &first_rows,
                                      const at::Tensor &row_to_unique, int64_t unique_count,
                                      SparseTensorQuantizationMode::Type mode);

  at::Tensor features_;
  mutable c10::optional<at::Tensor> coordinates_;
  CoordinateMapKey key_;
  std::shared_ptr<CoordinateManager> manager_;
  int dimension_;
};

// ---------------------------------------------------------------- layers

// Y = sum_k X[in_k] @ W[k] (+ bias) over the map, with its input, weight and
// bias gradients, through the HIP kernels (autograd-aware). features and
// kernel must share the dtype (fp32 or bf16); bias is an fp32 [cout] tensor
// or undefined.
at::Tensor hip_sparse_convolution(const at::Tensor &features, const at::Tensor &kernel,
                                  const HipKernelMap &map, const at::Tensor &bias = at::Tensor());

class RiemannConvolutionBaseImpl : public torch::nn::Cloneable<RiemannConvolutionBaseImpl> {
public:
  RiemannConvolutionBaseImpl(int in_channels, int out_channels, int kernel_size = 3,
                             int stride = 1, int dilation = 1, bool bias = false,
                             bool is_transpose = false, bool expand_coordinates = false,
                             ConvolutionMode::Type convolution_mode = ConvolutionMode::DEFAULT,
                             int dimension = 3,
                             RegionType::Type region_type = RegionType::HYPER_CUBE);
  void reset() override;
  void reset_parameters(bool is_transpose = false);
  SparseTensor forward(const SparseTensor &input);

  int in_channels_;
  int out_channels_;
  bool is_transpose_;
  bool use_mm_;
  int dimension_;
  ConvolutionMode::Type convolution_mode_;
  KernelGenerator kernel_generator_;
  torch::Tensor kernel_{nullptr};
  torch::Tensor bias_{nullptr};
  bool has_bias_;
};

class RiemannConvolutionImpl : public torch::nn::Cloneable<RiemannConvolutionImpl> {
public:
  RiemannConvolutionImpl(int in_channels, int out_channels, int kernel_size = 3, int stride = 1,
                         int dilation = 1, bool bias = false, bool expand_coordinates = false,
                         ConvolutionMode::Type convolution_mode = ConvolutionMode::DEFAULT,
                         int dimension = 3);
  void reset() override;
  SparseTensor forward(const SparseTensor &input);
  std::shared_ptr<RiemannConvolutionBaseImpl> base() { return base_; }

private:
  int in_channels_, out_channels_, kernel_size_, stride_, dilation_;
  bool bias_, expand_;
  ConvolutionMode::Type mode_;
  int dimension_;
  std::shared_ptr<RiemannConvolutionBaseImpl> base_{nullptr};
};
TORCH_MODULE(RiemannConvolution);

class RiemannConvolutionTransposeImpl
    : public torch::nn::Cloneable<RiemannConvolutionTransposeImpl> {
public:
  RiemannConvolutionTransposeImpl(int in_channels, int out_channels, int kernel_size = 3,
                                  int stride = 1, int dilation = 1, bool bias = false,
                                  bool expand_coordinates = false,
                                  ConvolutionMode::Type convolution_mode = ConvolutionMode::DEFAULT,
                                  int dimension = 3);
  void reset() override;
  SparseTensor forward(const SparseTensor &input);
  std::shared_ptr<RiemannConvolutionBaseImpl> base() { return base_; }

private:
  int in_channels_, out_channels_, kernel_size_, stride_, dilation_;
  bool bias_, expand_;
  ConvolutionMode::Type mode_;
  int dimension_;
  std::shared_ptr<RiemannConvolutionBaseImpl> base_{nullptr};
};
TORCH_MODULE(RiemannConvolutionTranspose);

// Transposed convolution whose output map is generated from the input
// through the kernel region (CoordinateManager::stride_region).
class RiemannGenerativeConvolutionTransposeImpl
    : public torch::nn::Cloneable<RiemannGenerativeConvolutionTransposeImpl> {
public:
  RiemannGenerativeConvolutionTransposeImpl(
      int in_channels, int out_channels, int kernel_size = 3, int stride = 1, int dilation = 1,
      bool bias = false, ConvolutionMode::Type convolution_mode = ConvolutionMode::DEFAULT,
      int dimension = 3);
  void reset() override;
  SparseTensor forward(const SparseTensor &input);
  std::shared_ptr<RiemannConvolutionBaseImpl> base() { return base_; }

private:
  int in_channels_, out_channels_, kernel_size_, stride_, dilation_;
  bool bias_;
  ConvolutionMode::Type mode_;
  int dimension_;
  std::shared_ptr<RiemannConvolutionBaseImpl> base_{nullptr};
};
TORCH_MODULE(RiemannGenerativeConvolutionTranspose);

class RiemannBatchNormImpl : public torch::nn::Cloneable<RiemannBatchNormImpl> {
public:
  RiemannBatchNormImpl(int64_t num_features, double eps = 1e-5, double momentum = 0.1,
                       bool affine = true, bool track_running_stats = true);
  void reset() override;
  SparseTensor forward(const SparseTensor &input);
  // act(normalised input [+ residual]), act = ReLU when `relu`: the
  // BasicBlock tails in one pass. residual must share input's manager and
  // key (SparseTensor::operator+=).
  SparseTensor forward_fused(const SparseTensor &input, const SparseTensor *residual, bool relu);
  // The affine parameters and running statistics stay fp32 under a dtype
  // cast of the model: bf16 features are normalised in fp32 (the usual
  // mixed-precision rule for normalisation layers). Device moves apply.
  using torch::nn::Module::to;
  void to(torch::Dtype dtype, bool non_blocking = false) override;
  void to(torch::Device device, torch::Dtype dtype, bool non_blocking = false) override;

private:
  int64_t num_features_;
  double eps_, momentum_;
  bool affine_, track_;
  torch::nn::BatchNorm1d normalization_{nullptr};
};
TORCH_MODULE(RiemannBatchNorm);

class RiemannReLUImpl : public torch::nn::Cloneable<RiemannReLUImpl> {
public:
  explicit RiemannReLUImpl(bool inplace = false) : inplace_(inplace) {}
  void reset() override {}
  SparseTensor forward(const SparseTensor &input);

private:
  bool inplace_;
};
TORCH_MODULE(RiemannReLU);

// ---------------------------------------------------------------- pooling

// Local pooling of features over a kernel or stride map through the HIP
// kernels (autograd-aware): mode LOCAL_{SUM,AVG,MAX}_POOLING.
at::Tensor hip_sparse_pooling(const at::Tensor &features, const HipKernelMap &map,
                              PoolingMode::Type mode);

// Reduce feature rows by group (rows with equal group[i] in [0, n_groups)),
// reduction RHIP_POOL_SUM / AVG / MAX, through the group map and the pooling
// kernels (autograd-aware); features fp32 or bf16 on the device.
at::Tensor hip_group_reduce(const at::Tensor &features, const at::Tensor &group,
                            int64_t n_groups, int32_t reduction);

class RiemannPoolingBaseImpl : public torch::nn::Cloneable<RiemannPoolingBaseImpl> {
public:
  RiemannPoolingBaseImpl(int kernel_size, int stride = 1, int dilation = 1,
                         PoolingMode::Type mode = PoolingMode::LOCAL_AVG_POOLING,
                         int dimension = 3);
  RiemannPoolingBaseImpl(KernelGenerator kernel_generator, PoolingMode::Type mode, int dimension);
  void reset() override {}
  SparseTensor forward(const SparseTensor &input);

private:
  KernelGenerator kernel_generator_;
  PoolingMode::Type mode_;
  int dimension_;
};
TORCH_MODULE(RiemannPoolingBase);

// RiemannSumPooling / RiemannAvgPooling / RiemannMaxPooling: the base layer
// with its mode fixed (engine/nn/pooling.hpp:26-63).
template <PoolingMode::Type Mode>
class RiemannLocalPoolingImpl : public torch::nn::Cloneable<RiemannLocalPoolingImpl<Mode>> {
public:
  RiemannLocalPoolingImpl(int kernel_size, int stride = 1, int dilation = 1, int dimension = 3)
      : kernel_size_(kernel_size), stride_(stride), dilation_(dilation), dimension_(dimension) {
    reset();
  }
  void reset() override {
    pooling_ = this->register_module(
        "pooling", RiemannPoolingBase(kernel_size_, stride_, dilation_, Mode, dimension_));
  }
  SparseTensor forward(const SparseTensor &input) { return pooling_->forward(input); }

private:
  int kernel_size_, stride_, dilation_, dimension_;
  RiemannPoolingBase pooling_{nullptr};
};
using RiemannSumPoolingImpl = RiemannLocalPoolingImpl<PoolingMode::LOCAL_SUM_POOLING>;
using RiemannAvgPoolingImpl = RiemannLocalPoolingImpl<PoolingMode::LOCAL_AVG_POOLING>;
using RiemannMaxPoolingImpl = RiemannLocalPoolingImpl<PoolingMode::LOCAL_MAX_POOLING>;
TORCH_MODULE(RiemannSumPooling);
TORCH_MODULE(RiemannAvgPooling);
TORCH_MODULE(RiemannMaxPooling);

// Unpooling onto a generated finer map (engine/nn/pooling.hpp:65-81,
// pooling.cpp:188-201); the output map is built from the input through the
// kernel region at the output stride.
class RiemannPoolingTransposeImpl : public torch::nn::Cloneable<RiemannPoolingTransposeImpl> {
public:
  RiemannPoolingTransposeImpl(int kernel_size, int stride, int dilation = 1,
                              bool expand_coordinates = false, int dimension = 3);
  RiemannPoolingTransposeImpl(KernelGenerator kernel_generator, int dimension,
                              PoolingMode::Type mode = PoolingMode::LOCAL_SUM_POOLING);
  void reset() override {}
  SparseTensor forward(const SparseTensor &input);

private:
  KernelGenerator kernel_generator_;
  int dimension_;
  PoolingMode::Type mode_ = PoolingMode::LOCAL_SUM_POOLING;
};
TORCH_MODULE(RiemannPoolingTranspose);

// One output row per batch index 0 .. max batch (engine/nn/pooling.hpp:83-131,
// pooling.cpp:203-260).
class RiemannGlobalPoolingImpl : public torch::nn::Cloneable<RiemannGlobalPoolingImpl> {
public:
  explicit RiemannGlobalPoolingImpl(
      PoolingMode::Type mode = PoolingMode::GLOBAL_AVG_POOLING_PYTORCH_INDEX);
  void reset() override {}
  SparseTensor forward(const SparseTensor &input);

private:
  PoolingMode::Type mode_;
};
TORCH_MODULE(RiemannGlobalPooling);

template <PoolingMode::Type Mode>
class RiemannGlobalModePoolingImpl
    : public torch::nn::Cloneable<RiemannGlobalModePoolingImpl<Mode>> {
public:
  explicit RiemannGlobalModePoolingImpl(PoolingMode::Type mode = Mode) : mode_(mode) { reset(); }
  void reset() override { pooling_ = this->register_module("pooling", RiemannGlobalPooling(mode_)); }
  SparseTensor forward(const SparseTensor &input) { return pooling_->forward(input); }

private:
  PoolingMode::Type mode_;
  RiemannGlobalPooling pooling_{nullptr};
};
using RiemannGlobalSumPoolingImpl =
    RiemannGlobalModePoolingImpl<PoolingMode::GLOBAL_SUM_POOLING_PYTORCH_INDEX>;
using RiemannGlobalAvgPoolingImpl =
    RiemannGlobalModePoolingImpl<PoolingMode::GLOBAL_AVG_POOLING_PYTORCH_INDEX>;
using RiemannGlobalMaxPoolingImpl =
    RiemannGlobalModePoolingImpl<PoolingMode::GLOBAL_MAX_POOLING_PYTORCH_INDEX>;
TORCH_MODULE(RiemannGlobalSumPooling);
TORCH_MODULE(RiemannGlobalAvgPooling);
TORCH_MODULE(RiemannGlobalMaxPooling);

// conv3 -> BN -> ReLU -> conv3 -> BN -> (+ residual) -> ReLU
// (RiemannEngine/engine/nn/residual.cpp:16-52)
class BasicBlockImpl : public torch::nn::Cloneable<BasicBlockImpl> {
public:
  static constexpr int expansion = 1;
  BasicBlockImpl(int inplanes, int planes, int stride = 1, int dilation = 1,
                 torch::nn::AnyModule downsample = torch::nn::AnyModule(),
                 double bn_momentum = 0.1, int dimension = 3);
  void reset() override;
  SparseTensor forward(const SparseTensor &input);

  RiemannConvolution conv1_{nullptr}, conv2_{nullptr};
  RiemannBatchNorm norm1_{nullptr}, norm2_{nullptr};
  RiemannReLU relu_{nullptr};
  torch::nn::AnyModule downsample_;
  int inplanes_, planes_, stride_, dilation_, dimension_;
  double bn_momentum_;
  bool has_downsample_ = false;
};
TORCH_MODULE(BasicBlock);

} // namespace riemann
