// CoordinateMapKey, region offsets, KernelGenerator and the HIP-backed
// CoordinateManager (coordinate maps + kernel-map cache).
#include <ATen/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <limits>
#include <map>
#include <mutex>
#include <random>
#include <sstream>

#include "riemann.hpp"

namespace riemann {

void check_rhip(int status, const char *what) {
  TORCH_CHECK(status == RHIP_OK, what, " failed (status ", status, "): ", rhip_last_error());
}

namespace {

void check_hip(hipError_t e, const char *what) {
  TORCH_CHECK(e == hipSuccess, what, " failed: ", hipGetErrorString(e));
}

hipStream_t current_stream(const at::Device &device) {
  return c10::hip::getCurrentHIPStream(device.index()).stream();
}

// A stencil's partner permutation on a device (int32 [K]), uploaded once
// per device and permutation and shared, read-only, by every symmetric map
// with it: its input gradient's weight permutation. The first upload goes
// from pinned memory on the current stream, ahead of the map count's
// synchronisation, so it has landed before any later map or stream uses it.
// The cache is never destroyed (its tensors must not outlive the runtime at
// process exit).
at::Tensor device_partners(const std::vector<int32_t> &partner, const at::Device &dev) {
  static std::mutex mu;
  static auto *cache = new std::map<std::pair<int, std::vector<int32_t>>, at::Tensor>();
  std::lock_guard<std::mutex> lock(mu);
  auto key = std::make_pair(static_cast<int>(dev.index()), partner);
  auto it = cache->find(key);
  if (it != cache->end())
    return it->second;
  const int64_t K = static_cast<int64_t>(partner.size());
  auto pinned = torch::empty({K}, torch::TensorOptions().dtype(torch::kInt32).pinned_memory(true));
  std::memcpy(pinned.data_ptr<int32_t>(), partner.data(), sizeof(int32_t) * K);
  at::Tensor t = pinned.to(dev, /*non_blocking=*/true);
  cache->emplace(std::move(key), t);
  return t;
}

at::Tensor device_bytes(size_t bytes, const at::Device &device) {
  return torch::empty({static_cast<int64_t>(std::max<size_t>(bytes, 1))},
                      torch::TensorOptions().dtype(torch::kUInt8).device(device));
}

// Several buffers in one device allocation: add() reserves 256-aligned byte
// ranges, alloc() makes the block, and take() returns each range as a
// tensor view (int32 or uint8) that keeps the block alive. A map build's
// long-lived buffers share one block, its scratch another: each allocator
// call costs the host a few microseconds on the build's critical path.
struct Block {
  std::vector<std::pair<size_t, size_t>> parts; // (offset, bytes)
  size_t used = 0;
  at::Tensor base;
  int add(size_t bytes) {
    const size_t off = (used + 255) / 256 * 256;
    parts.emplace_back(off, std::max<size_t>(bytes, 1));
    used = off + std::max<size_t>(bytes, 1);
    return static_cast<int>(parts.size()) - 1;
  }
  void alloc(const at::Device &dev) { base = device_bytes(used, dev); }
  at::Tensor bytes(int i) const {
    return base.narrow(0, static_cast<int64_t>(parts[i].first),
                       static_cast<int64_t>(parts[i].second));
  }
  at::Tensor i32(int i, at::IntArrayRef shape) const {
    return bytes(i).view(torch::kInt32).view(shape);
  }
  at::Tensor i64(int i, at::IntArrayRef shape) const {
    return bytes(i).view(torch::kInt64).view(shape);
  }
};

std::string stride_string(const stride_type &s) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < s.size(); ++i)
    o << (i ? ", " : "") << s[i];
  o << "]";
  return o.str();
}

stride_type to_stride_vector(torch::IntArrayRef v) {
  stride_type out;
  for (auto x : v) {
    TORCH_CHECK(x > 0, "kernel parameters must be positive");
    out.push_back(static_cast<uint32_t>(x));
  }
  return out;
}

} // namespace

// ------------------------------------------------------------ key

CoordinateMapKey::CoordinateMapKey(size_type coordinate_size)
    : key_set_(false), coordinate_size_(coordinate_size) {}

CoordinateMapKey::CoordinateMapKey(size_type coordinate_size, const coordinate_map_key_type &key)
    : key_set_(true), coordinate_size_(coordinate_size), key_(key) {
  TORCH_CHECK(coordinate_size_ - 1 == key_.first.size(),
              "Invalid tensor_stride: ", stride_string(key_.first),
              " coordinate_size: ", coordinate_size_);
}

CoordinateMapKey::CoordinateMapKey(stride_type tensor_stride, std::string string_id)
    : key_set_(true), coordinate_size_(static_cast<size_type>(tensor_stride.size() + 1)),
      key_(std::move(tensor_stride), std::move(string_id)) {}

void CoordinateMapKey::set_key(stride_type tensor_stride, std::string string_id) {
  TORCH_CHECK(coordinate_size_ - 1 == tensor_stride.size(), "Invalid tensor_stride size: ",
              stride_string(tensor_stride), " coordinate_size: ", coordinate_size_);
  key_ = {std::move(tensor_stride), std::move(string_id)};
  key_set_ = true;
}

void CoordinateMapKey::set_key(const coordinate_map_key_type &key) {
  set_key(key.first, key.second);
}

coordinate_map_key_type CoordinateMapKey::get_key() const {
  TORCH_CHECK(key_set_, "Key not set");
  return key_;
}

uint64_t CoordinateMapKey::hash() const {
  uint64_t h = 1469598103934665603ull; // FNV-1a over the stride, then the id
  for (auto v : key_.first) {
    h ^= v;
    h *= 1099511628211ull;
  }
  return h ^ std::hash<std::string>{}(key_.second);
}

bool CoordinateMapKey::operator==(const CoordinateMapKey &other) const {
  if (!key_set_ || !other.key_set_)
    return false;
  return key_ == other.key_;
}

std::string CoordinateMapKey::to_string() const {
  std::ostringstream o;
  o << "coordinate map key:" << stride_string(key_.first);
  if (!key_.second.empty())
    o << ":" << key_.second;
  return o.str();
}

// ------------------------------------------------------------ regions

at::Tensor normalize_region_offsets(const at::Tensor &offsets, int dimension) {
  TORCH_CHECK(dimension > 0, "CUSTOM region dimension must be positive");
  TORCH_CHECK(offsets.defined(), "region_offsets must be defined for CUSTOM");
  TORCH_CHECK(offsets.layout() == at::kStrided && offsets.dim() == 2,
              "region_offsets must be a dense [N, D] tensor");
  TORCH_CHECK(offsets.size(0) > 0 && offsets.size(0) <= std::numeric_limits<int>::max(),
              "region_offsets must have a non-empty, representable volume");
  TORCH_CHECK(offsets.size(1) == dimension, "region_offsets dimension mismatch");
  TORCH_CHECK(offsets.scalar_type() == at::kInt || offsets.scalar_type() == at::kLong,
              "region_offsets must contain int32 or int64 spatial offsets");
  auto host = offsets.to(at::kCPU).contiguous();
  if (host.scalar_type() == at::kLong) {
    TORCH_CHECK(host.min().item<int64_t>() >= std::numeric_limits<int32_t>::min() &&
                    host.max().item<int64_t>() <= std::numeric_limits<int32_t>::max(),
                "region_offsets values must fit int32");
  }
  return host.to(at::kInt).clone();
}

int region_volume(RegionType::Type region, const stride_type &kernel_size,
                  const at::Tensor &custom) {
  switch (region) {
  case RegionType::HYPER_CUBE: {
    int v = 1;
    for (auto k : kernel_size)
      v *= static_cast<int>(k);
    return v;
  }
  case RegionType::HYPER_CROSS: {
    int v = 1;
    for (auto k : kernel_size)
      v += static_cast<int>(k) - 1;
    return v;
  }
  case RegionType::CUSTOM:
    return custom.defined() ? static_cast<int>(custom.size(0)) : 0;
  }
  TORCH_CHECK(false, "Unknown region type");
}

at::Tensor region_offsets(RegionType::Type region, const stride_type &kernel_size,
                          const stride_type &dilation, const stride_type &tensor_stride,
                          const at::Tensor &custom) {
  const int D = static_cast<int>(kernel_size.size());
  TORCH_CHECK(dilation.size() == kernel_size.size() && tensor_stride.size() == kernel_size.size(),
              "kernel size, dilation and tensor stride must have the same length");
  const int K = region_volume(region, kernel_size, custom);
  // computed in plain int64 arithmetic (a few torch CPU ops here cost more
  // than the map's first kernels)
  std::vector<int64_t> o(static_cast<size_t>(K) * D, 0);
  std::vector<int64_t> step(D);
  for (int i = 0; i < D; ++i)
    step[i] = static_cast<int64_t>(dilation[i]) * tensor_stride[i];
  if (region == RegionType::HYPER_CUBE) {
    // axis 0 varies fastest; odd sizes centre on zero, even sizes start at 0
    for (int k = 0; k < K; ++k) {
      int64_t rem = k;
      for (int i = 0; i < D; ++i) {
        const int64_t ks = kernel_size[i];
        const int64_t idx = rem % ks;
        rem /= ks;
        o[static_cast<size_t>(k) * D + i] = (ks % 2 == 0 ? idx : idx - ks / 2) * step[i];
      }
    }
  } else if (region == RegionType::HYPER_CROSS) {
    // the centre, then per axis: +1 .. +r, then -r .. -1
    int k = 1;
    for (int axis = 0; axis < D; ++axis) {
      const int64_t r = (static_cast<int64_t>(kernel_size[axis]) - 1) / 2;
      for (int64_t ind = 0; ind < static_cast<int64_t>(kernel_size[axis]) - 1; ++ind, ++k)
        o[static_cast<size_t>(k) * D + axis] = (ind < r ? ind + 1 : ind - 2 * r) * step[axis];
    }
  } else {
    auto c = normalize_region_offsets(custom, D);
    auto ca = c.accessor<int32_t, 2>();
    for (int k = 0; k < K; ++k)
      for (int i = 0; i < D; ++i)
        o[static_cast<size_t>(k) * D + i] = static_cast<int64_t>(ca[k][i]) * step[i];
  }
  auto out = torch::empty({K, D}, torch::kInt32);
  int32_t *po = out.data_ptr<int32_t>();
  for (size_t i = 0; i < o.size(); ++i) {
    TORCH_CHECK(o[i] >= -static_cast<int64_t>(std::numeric_limits<int32_t>::max()) &&
                    o[i] <= std::numeric_limits<int32_t>::max(),
                "Scaled offsets must fit the coordinate type");
    po[i] = static_cast<int32_t>(o[i]);
  }
  return out;
}

// ------------------------------------------------------ KernelGenerator

KernelGenerator::KernelGenerator(torch::IntArrayRef kernel_size, torch::IntArrayRef stride,
                                 torch::IntArrayRef dilation, bool is_transpose,
                                 RegionType::Type region_type, at::Tensor offsets,
                                 bool expand_coordinates, int dimension)
    : kernel_size_(to_stride_vector(kernel_size)), kernel_stride_(to_stride_vector(stride)),
      kernel_dilation_(to_stride_vector(dilation)), is_transpose_(is_transpose),
      region_type_(region_type), region_offsets_(std::move(offsets)),
      expand_coordinates_(expand_coordinates), D_(dimension), kernel_volume_(0) {
  if (D_ <= 0)
    D_ = static_cast<int>(kernel_size_.size());
  // scalars broadcast across every spatial axis (engine/grid/stencil.cpp:108-117)
  if (kernel_size_.size() == 1 && D_ > 1)
    kernel_size_.assign(D_, kernel_size_[0]);
  if (kernel_stride_.size() == 1 && D_ > 1)
    kernel_stride_.assign(D_, kernel_stride_[0]);
  if (kernel_dilation_.size() == 1 && D_ > 1)
    kernel_dilation_.assign(D_, kernel_dilation_[0]);
  TORCH_CHECK(kernel_size_.size() == static_cast<size_t>(D_), "kernel_size dimension mismatch");
  TORCH_CHECK(kernel_stride_.size() == static_cast<size_t>(D_), "kernel_stride dimension mismatch");
  TORCH_CHECK(kernel_dilation_.size() == static_cast<size_t>(D_),
              "kernel_dilation dimension mismatch");
  if (region_type_ == RegionType::CUSTOM) {
    region_offsets_ = normalize_region_offsets(region_offsets_, D_);
  } else if (region_offsets_.defined()) {
    TORCH_CHECK(region_offsets_.numel() == 0,
                "region_offsets must be empty for HYPER_CUBE/HYPER_CROSS");
  }
  kernel_volume_ = region_volume(region_type_, kernel_size_, region_offsets_);
}

KernelGenerator::KernelParams KernelGenerator::get_kernel(const stride_type &tensor_stride,
                                                          bool is_transpose) const {
  (void)is_transpose;
  TORCH_CHECK(tensor_stride.size() == static_cast<size_t>(D_), "tensor_stride dimension mismatch");
  for (auto s : tensor_stride)
    TORCH_CHECK(s > 0, "tensor_stride must be positive");
  KernelParams p;
  p.kernel_size = kernel_size_;
  p.kernel_stride = kernel_stride_;
  p.kernel_dilation = kernel_dilation_;
  p.region_type = region_type_;
  p.region_offsets = region_type_ == RegionType::CUSTOM
                         ? region_offsets_.clone()
                         : torch::empty({0, D_}, torch::kInt32);
  p.expand_coordinates = expand_coordinates_;
  p.D = D_;
  return p;
}

// --------------------------------------------------------- kernel maps

void HipKernelMap::ensure_pairs() const {
  if (in_rows.defined())
    return;
  const auto dev = nbr.device();
  at::DeviceGuard guard(dev);
  const int64_t P = size();
  auto iopt = torch::TensorOptions().device(dev).dtype(torch::kInt32);
  // exact size: the pair counts are known
  auto ir = torch::empty({std::max<int64_t>(P, 1)}, iopt);
  auto orr = torch::empty({std::max<int64_t>(P, 1)}, iopt);
  if (P > 0) {
    size_t bytes = 0;
    check_rhip(rhip_kmap_pairs_workspace_bytes(n_out, K, &bytes),
               "rhip_kmap_pairs_workspace_bytes");
    auto ws = device_bytes(bytes, dev);
    check_rhip(rhip_kmap_pairs(nbr.data_ptr<int32_t>(), out_order.data_ptr<int32_t>(), n_out, K,
                               offsets.data_ptr<int64_t>(), ws.data_ptr(), ws.numel(),
                               ir.data_ptr<int32_t>(), orr.data_ptr<int32_t>(),
                               current_stream(dev)),
               "rhip_kmap_pairs");
  }
  in_rows = ir.slice(0, 0, P);
  out_rows = orr.slice(0, 0, P);
}

void HipKernelMap::ensure_transposed() const {
  if (nbr_t.defined())
    return;
  TORCH_CHECK(symmetric && static_cast<int32_t>(partner_host.size()) == K,
              "this kernel map has no transposed table");
  const auto dev = nbr.device();
  at::DeviceGuard guard(dev);
  const hipStream_t st = current_stream(dev);
  // i pairs with o under k iff o pairs with i under partner[k]: row k of
  // the table is row partner[k] of the transposed one
  auto t = torch::empty({K, std::max<int64_t>(n_in, 1)}, nbr.options());
  const size_t row = static_cast<size_t>(n_out) * sizeof(int32_t);
  for (int32_t k = 0; k < K && n_out > 0; ++k)
    check_hip(hipMemcpyAsync(t.data_ptr<int32_t>() + static_cast<int64_t>(partner_host[k]) * n_in,
                             nbr.data_ptr<int32_t>() + static_cast<int64_t>(k) * n_out, row,
                             hipMemcpyDeviceToDevice, st),
              "hipMemcpyAsync");
  nbr_t = t.slice(1, 0, n_in);
  in_order = out_order;
}

HipKernelMap HipKernelMap::swapped() const {
  ensure_pairs();
  if (symmetric)
    ensure_transposed();
  HipKernelMap m;
  m.K = K;
  m.stride_map = stride_map;
  m.n_in = n_out;
  m.n_out = n_in;
  m.offsets_host = offsets_host;
  m.offsets = offsets;
  m.in_rows = out_rows;
  m.out_rows = in_rows;
  m.nbr = nbr_t;
  m.nbr_t = nbr;
  m.in_order = out_order;
  m.out_order = in_order;
  return m;
}

std::pair<std::vector<at::Tensor>, std::vector<at::Tensor>> HipKernelMap::per_offset() const {
  ensure_pairs();
  std::vector<at::Tensor> ins, outs;
  for (int k = 0; k < (stride_map ? 1 : K); ++k) {
    const int64_t a = offsets_host[k], b = offsets_host[k + 1];
    ins.push_back(in_rows.slice(0, a, b).to(torch::kLong));
    outs.push_back(out_rows.slice(0, a, b).to(torch::kLong));
  }
  return {ins, outs};
}

// ------------------------------------------------------ CoordinateManager

CoordinateManager::CoordinateManager(int D, CoordinateMapBackend::Type backend,
                                     GPUMemoryAllocatorBackend::Type alloc_type,
                                     RiemannAlgorithm::Mode algo)
    : D_(D), backend_(backend), alloc_type_(alloc_type), algo_(algo) {
  TORCH_CHECK(D > 0 && D + 1 <= RHIP_MAX_COLS, "dimension must be in [1, ", RHIP_MAX_COLS - 1,
              "]");
  TORCH_CHECK(backend == CoordinateMapBackend::CUDA,
              "this build implements the device (HIP) coordinate-map backend only; "
              "there is no CPU coordinate manager");
}

coordinate_map_key_type CoordinateManager::random_key(const stride_type &tensor_stride,
                                                      const std::string &string_id) const {
  static thread_local std::mt19937_64 rng{std::random_device{}()};
  static const char alphabet[] = "abcdefghijklmnopqrstuvwxyz0123456789";
  coordinate_map_key_type key;
  do {
    std::string id = string_id + "_";
    for (int i = 0; i < 8; ++i)
      id.push_back(alphabet[rng() % (sizeof(alphabet) - 1)]);
    key = {tensor_stride, id};
  } while (maps_.count(key));
  return key;
}

CoordinateMapHIP CoordinateManager::build_map(const at::Tensor &coords,
                                              const stride_type &tensor_stride,
                                              at::Tensor *mapping, at::Tensor *inverse) const {
  const auto dev = coords.device();
  at::DeviceGuard guard(dev);
  const hipStream_t st = current_stream(dev);
  const int64_t n = coords.size(0);
  const int32_t ncol = static_cast<int32_t>(coords.size(1));
  CoordinateMapHIP m;
  m.tensor_stride = tensor_stride;
  auto iopt = torch::TensorOptions().device(dev);
  // the map's slots, unique rows and locality order in one block, and one
  // scratch block that the hash build and then the order use (stream-ordered:
  // the order's kernels run after the build's); the order's buffers, sized
  // by the row count (an upper bound of the unique rows), are allocated
  // before the build, whose end waits for the device: after it only the
  // brick grid is allocated before the order's launches
  const int64_t rows = std::max<int64_t>(n, 1);
  size_t ws_bytes = 0, ob = 0;
  check_rhip(rhip_hash_workspace_bytes(n, ncol, &ws_bytes), "rhip_hash_workspace_bytes");
  check_rhip(rhip_order_workspace_bytes(n, &ob), "rhip_order_workspace_bytes");
  Block own;
  const int i_slots = own.add(rhip_table_bytes(n));
  const int i_rows = own.add(sizeof(int32_t) * rows * ncol);
  const int i_order = own.add(sizeof(int32_t) * rows);
  own.alloc(dev);
  m.slots = own.bytes(i_slots);
  m.storage = own.i32(i_rows, {rows, ncol});
  m.order = own.i32(i_order, {rows});
  auto ws = device_bytes(std::max(ws_bytes, ob), dev);
  auto &ows = ws;
  auto map_t = torch::empty({rows}, iopt.dtype(torch::kInt64));
  at::Tensor inv_t;
  if (inverse)
    inv_t = torch::empty({rows}, iopt.dtype(torch::kInt64));
  check_rhip(rhip_hash_build(coords.data_ptr<int32_t>(), n, ncol, m.slots.data_ptr(),
                             m.slots.numel(), ws.data_ptr(), ws.numel(),
                             m.storage.data_ptr<int32_t>(), map_t.data_ptr<int64_t>(),
                             inverse ? inv_t.data_ptr<int64_t>() : nullptr, &m.table, st),
             "rhip_hash_build");
  const int64_t nu = m.table.n_unique;
  m.coords = m.storage.slice(0, 0, nu);
  if (nu > 0) {
    size_t bb = 0;
    check_rhip(rhip_brick_bytes(&m.table, &bb), "rhip_brick_bytes");
    m.bricks = device_bytes(std::max<size_t>(bb, 1), dev);
    check_rhip(rhip_spatial_order(&m.table, m.order.data_ptr<int32_t>(), nullptr,
                                  m.bricks.data_ptr(), bb, ows.data_ptr(),
                                  static_cast<size_t>(ows.numel()), st),
               "rhip_spatial_order");
  }
  m.order = m.order.slice(0, 0, nu);
  if (mapping)
    *mapping = map_t.slice(0, 0, nu);
  if (inverse)
    *inverse = inv_t.slice(0, 0, n);
  return m;
}

std::pair<CoordinateMapKey, std::pair<at::Tensor, at::Tensor>>
CoordinateManager::insert_and_map(const at::Tensor &coordinates, stride_type tensor_stride,
                                  std::string string_id) {
  // Argument checks of CoordinateMapManager::insert_and_map_cpp
  // (engine/grid/space_impl.hpp:268-282), with the device backend required.
  TORCH_CHECK(coordinates.is_contiguous(), "coordinates must be contiguous");
  TORCH_CHECK(coordinates.scalar_type() == torch::kInt, "coordinates must be int32");
  TORCH_CHECK(coordinates.is_cuda(),
              "coordinates must be a device tensor (the HIP path has no CPU fallback)");
  TORCH_CHECK(coordinates.dim() == 2, "coordinates must be a 2-D tensor");
  const auto coordinate_size = static_cast<size_type>(coordinates.size(1));
  TORCH_CHECK(coordinate_size - 1 == tensor_stride.size(),
              "The coordinate dimension (coordinate_size - 1): ", coordinate_size - 1,
              " must match the size of tensor stride: ", stride_string(tensor_stride));
  TORCH_CHECK(static_cast<int>(coordinate_size) == D_ + 1,
              "coordinates have ", coordinate_size, " columns; this manager expects ", D_ + 1);
  coordinate_map_key_type key{tensor_stride, string_id};
  if (maps_.count(key))
    key = random_key(tensor_stride, string_id);
  at::Tensor mapping, inverse;
  maps_.emplace(key, build_map(coordinates, tensor_stride, &mapping, &inverse));
  return {CoordinateMapKey(coordinate_size, key), {mapping, inverse}};
}

CoordinateMapKey CoordinateManager::stride(const CoordinateMapKey &in_key,
                                           const stride_type &kernel_stride,
                                           std::string string_id) {
  const auto ik = in_key.get_key();
  auto it = maps_.find(ik);
  TORCH_CHECK(it != maps_.end(), "coordinate map not found: ", in_key.to_string());
  TORCH_CHECK(kernel_stride.size() == ik.first.size(), "stride size mismatch");
  stride_type out_stride(ik.first);
  for (size_t i = 0; i < out_stride.size(); ++i) {
    TORCH_CHECK(kernel_stride[i] > 0, "kernel stride must be positive");
    out_stride[i] *= kernel_stride[i];
  }
  coordinate_map_key_type out_key{out_stride, string_id.empty() ? ik.second : string_id};
  if (!maps_.count(out_key)) {
    const CoordinateMapHIP &in_map = it->second;
    const auto dev = in_map.coords.device();
    at::DeviceGuard guard(dev);
    auto strided = torch::empty_like(in_map.coords);
    std::vector<int32_t> s(out_stride.begin(), out_stride.end());
    if (in_map.size() > 0)
      check_rhip(rhip_stride_coords(in_map.coords.data_ptr<int32_t>(), in_map.size(),
                                    static_cast<int32_t>(in_map.coords.size(1)), s.data(),
                                    strided.data_ptr<int32_t>(), current_stream(dev)),
                 "rhip_stride_coords");
    maps_.emplace(out_key, build_map(strided, out_stride, nullptr, nullptr));
  }
  return CoordinateMapKey(static_cast<size_type>(ik.first.size() + 1), out_key);
}

std::pair<CoordinateMapKey, bool>
CoordinateManager::stride_region(const CoordinateMapKey &in_key, const at::Tensor &offsets,
                                 const stride_type &out_tensor_stride, bool expand) {
  const auto ik = in_key.get_key();
  auto it = maps_.find(ik);
  TORCH_CHECK(it != maps_.end(), "coordinate map not found: ", in_key.to_string());
  TORCH_CHECK(out_tensor_stride.size() == ik.first.size(), "tensor stride size mismatch");
  TORCH_CHECK(offsets.dim() == 2 && offsets.size(1) == static_cast<int64_t>(ik.first.size()),
              "region offsets must be [K, D]");
  coordinate_map_key_type out_key{out_tensor_stride, ""};
  const bool exists = maps_.count(out_key) > 0;
  if (exists && !expand)
    return {CoordinateMapKey(static_cast<size_type>(ik.first.size() + 1), out_key), false};
  const CoordinateMapHIP &in_map = it->second;
  const auto dev = in_map.coords.device();
  at::DeviceGuard guard(dev);
  const int64_t K = offsets.size(0), n = in_map.size();
  const int32_t ncol = static_cast<int32_t>(in_map.coords.size(1));
  auto off = offsets.to(torch::kInt32).contiguous().to(dev);
  auto expanded = torch::empty({n * K, ncol}, in_map.coords.options());
  if (n > 0)
    check_rhip(rhip_expand_coords(in_map.coords.data_ptr<int32_t>(), n, ncol,
                                  off.data_ptr<int32_t>(), static_cast<int32_t>(K),
                                  expanded.data_ptr<int32_t>(), current_stream(dev)),
               "rhip_expand_coords");
  if (exists)
    out_key = random_key(out_tensor_stride, "");
  maps_.emplace(out_key, build_map(expanded, out_tensor_stride, nullptr, nullptr));
  return {CoordinateMapKey(static_cast<size_type>(ik.first.size() + 1), out_key), true};
}

const CoordinateMapHIP &CoordinateManager::coordinate_map(const CoordinateMapKey &key) const {
  auto it = maps_.find(key.get_key());
  // the reference ASSERTs with ERROR_MAP_NOT_FOUND (engine/foundation/errors.hpp:13)
  TORCH_CHECK(it != maps_.end(), "CoordinateMap not found: ", key.to_string());
  return it->second;
}

at::Tensor CoordinateManager::get_coordinates(const CoordinateMapKey &key) const {
  return coordinate_map(key).coords;
}

uint32_t CoordinateManager::size(const CoordinateMapKey &key) const {
  return static_cast<uint32_t>(coordinate_map(key).size());
}

bool CoordinateManager::exists(const CoordinateMapKey &key) const {
  return key.is_key_set() && maps_.count(key.get_key()) > 0;
}

HipKernelMap CoordinateManager::generate(const CoordinateMapHIP &in_map,
                                         const CoordinateMapHIP &out_map,
                                         const at::Tensor &offsets_host) const {
  const auto dev = in_map.coords.device();
  at::DeviceGuard guard(dev);
  const hipStream_t st = current_stream(dev);
  const int32_t K = static_cast<int32_t>(offsets_host.size(0));
  const int64_t n_in = in_map.size(), n_out = out_map.size();
  auto iopt = torch::TensorOptions().device(dev).dtype(torch::kInt32);
  auto offsets = offsets_host.to(at::kCPU).to(torch::kInt32).contiguous();
  HipKernelMap m;
  m.K = K;
  m.n_in = n_in;
  m.n_out = n_out;
  size_t ws_bytes = 0;
  check_rhip(rhip_kmap_workspace_bytes(n_in, n_out, K, &ws_bytes), "rhip_kmap_workspace_bytes");
  auto ws = device_bytes(ws_bytes, dev);
  // the map's table, processing order and CSR offsets in one block
  const int64_t rows_out = std::max<int64_t>(n_out, 1);
  Block own;
  const int i_nbr = own.add(sizeof(int32_t) * K * rows_out);
  const int i_order = own.add(sizeof(int32_t) * rows_out);
  const int i_ofs = own.add(sizeof(int64_t) * (K + 1));
  own.alloc(dev);
  auto nbr = own.i32(i_nbr, {K, rows_out});
  auto out_order = own.i32(i_order, {rows_out});
  m.offsets = own.i64(i_ofs, {K + 1});
  int32_t flags = 0;
  // A map of a set onto itself whose stencil is closed under negation is
  // symmetric (the count confirms it): its partners (shared per device and
  // stencil) are on the device ahead of the count, whose synchronisation
  // covers a first upload.
  auto upload_partners = [&]() { m.partner = device_partners(m.partner_host, dev); };
  if (&in_map == &out_map) {
    m.partner_host.resize(K);
    if (rhip_stencil_partners(offsets.data_ptr<int32_t>(), K,
                              static_cast<int32_t>(offsets.size(1)),
                              m.partner_host.data()) == RHIP_OK)
      upload_partners();
    else
      m.partner_host.clear();
  }
  // the one synchronisation: the count reads the pair counts back into
  // m.offsets_host
  m.offsets_host.resize(K + 1);
  check_rhip(rhip_kmap_count(&in_map.table, out_map.coords.data_ptr<int32_t>(),
                             out_map.order.data_ptr<int32_t>(), n_out, K,
                             offsets.data_ptr<int32_t>(), ws.data_ptr(), ws.numel(),
                             nbr.data_ptr<int32_t>(), out_order.data_ptr<int32_t>(),
                             m.offsets.data_ptr<int64_t>(), m.offsets_host.data(), &flags, st),
             "rhip_kmap_count");
  // A symmetric map keeps no transposed table (its input gradient runs on
  // nbr with the stencil partners as weight permutation); any other map gets
  // its transposed table and input order now. Pair lists wait for a caller
  // that needs them (ensure_pairs), sized exactly then.
  m.symmetric = (flags & RHIP_KMAP_SYMMETRIC) != 0;
  at::Tensor nbr_t, in_order;
  if (m.symmetric) {
    if (!m.partner.defined()) {
      m.partner_host.resize(K);
      check_rhip(rhip_stencil_partners(offsets.data_ptr<int32_t>(), K,
                                       static_cast<int32_t>(offsets.size(1)),
                                       m.partner_host.data()),
                 "rhip_stencil_partners");
      upload_partners();
    }
  } else {
    m.partner = at::Tensor();
    m.partner_host.clear();
    nbr_t = torch::empty({K, std::max<int64_t>(n_in, 1)}, iopt);
    in_order = torch::empty({std::max<int64_t>(n_in, 1)}, iopt);
    check_rhip(rhip_kmap_fill(nbr.data_ptr<int32_t>(), out_order.data_ptr<int32_t>(), n_out, K,
                              in_map.order.data_ptr<int32_t>(), n_in, flags, ws.data_ptr(),
                              ws.numel(), m.offsets.data_ptr<int64_t>(), nullptr, nullptr,
                              nbr_t.data_ptr<int32_t>(), in_order.data_ptr<int32_t>(), st),
               "rhip_kmap_fill");
  }
  m.nbr = nbr.slice(1, 0, n_out);
  m.out_order = out_order.slice(0, 0, n_out);
  if (!m.symmetric) {
    m.nbr_t = nbr_t.slice(1, 0, n_in);
    m.in_order = in_order.slice(0, 0, n_in);
  }
  return m;
}

HipKernelMap CoordinateManager::generate_stride_map(const CoordinateMapHIP &in_map,
                                                    const CoordinateMapHIP &out_map) const {
  const auto dev = in_map.coords.device();
  at::DeviceGuard guard(dev);
  const hipStream_t st = current_stream(dev);
  const int64_t n_in = in_map.size(), n_out = out_map.size();
  auto iopt = torch::TensorOptions().device(dev).dtype(torch::kInt32);
  std::vector<int32_t> s(out_map.tensor_stride.begin(), out_map.tensor_stride.end());
  size_t ws_bytes = 0;
  check_rhip(rhip_stride_map_workspace_bytes(n_in, n_out, &ws_bytes),
             "rhip_stride_map_workspace_bytes");
  auto ws = device_bytes(ws_bytes, dev);
  int32_t kmax = 0;
  check_rhip(rhip_stride_map_count(&out_map.table, in_map.coords.data_ptr<int32_t>(), n_in,
                                   s.data(), ws.data_ptr(), ws.numel(), &kmax, st),
             "rhip_stride_map_count");
  HipKernelMap m;
  m.stride_map = true;
  m.K = std::max<int32_t>(kmax, 1);
  m.n_in = n_in;
  m.n_out = n_out;
  // phase 2 writes every entry of the tables (-1 where no input lies)
  auto table = [&](int64_t cols) {
    return kmax > 0 ? torch::empty({m.K, std::max<int64_t>(cols, 1)}, iopt)
                    : torch::full({m.K, std::max<int64_t>(cols, 1)}, -1, iopt);
  };
  auto nbr = table(n_out);
  auto nbr_t = kmax > 0 ? torch::empty({1, std::max<int64_t>(n_in, 1)}, iopt)
                        : torch::full({1, std::max<int64_t>(n_in, 1)}, -1, iopt);
  auto in_rows = torch::empty({std::max<int64_t>(n_in, 1)}, iopt);
  auto out_rows = torch::empty({std::max<int64_t>(n_in, 1)}, iopt);
  check_rhip(rhip_stride_map_fill(n_in, n_out, kmax, in_map.order.data_ptr<int32_t>(),
                                  out_map.order.data_ptr<int32_t>(), ws.data_ptr(), ws.numel(),
                                  nbr.data_ptr<int32_t>(), nbr_t.data_ptr<int32_t>(),
                                  in_rows.data_ptr<int32_t>(), out_rows.data_ptr<int32_t>(), st),
             "rhip_stride_map_fill");
  m.offsets_host = {0, n_in}; // the reference's single pair list
  m.offsets = torch::tensor(m.offsets_host, torch::kInt64).to(dev);
  m.in_rows = in_rows.slice(0, 0, n_in);
  m.out_rows = out_rows.slice(0, 0, n_in);
  m.nbr = nbr.slice(1, 0, n_out);
  m.nbr_t = nbr_t.slice(1, 0, n_in);
  m.in_order = in_map.order;
  m.out_order = out_map.order;
  return m;
}

const HipKernelMap &CoordinateManager::kernel_map(
    const CoordinateMapKey &in_key, const CoordinateMapKey &out_key,
    const stride_type &kernel_size, const stride_type &kernel_stride,
    const stride_type &kernel_dilation, RegionType::Type region_type,
    const at::Tensor &offsets, bool is_transpose, bool is_pool) {
  const size_t kdim = kernel_size.size();
  TORCH_CHECK(kdim == kernel_stride.size(), "kernel size mismatch");
  TORCH_CHECK(kdim == kernel_dilation.size(), "kernel size mismatch");
  // a pooling layer whose kernel tiles the stride uses the stride map
  // (space_impl.hpp:617-626, 660-669)
  const bool use_stride_map =
      is_pool && region_type != RegionType::CUSTOM && kernel_stride == kernel_size;
  at::Tensor custom;
  std::vector<int32_t> custom_values;
  if (region_type == RegionType::CUSTOM) {
    custom = normalize_region_offsets(offsets, static_cast<int>(kdim));
    custom_values.assign(custom.data_ptr<int32_t>(), custom.data_ptr<int32_t>() + custom.numel());
  }
  const kernel_map_key_type key = std::make_tuple(in_key.get_key(), out_key.get_key(),
                                                  kernel_size, kernel_stride, kernel_dilation,
                                                  region_type, is_transpose, is_pool);
  auto find = [&](const kernel_map_key_type &k) -> const HipKernelMap * {
    if (region_type == RegionType::CUSTOM) {
      auto it = custom_maps_.find({k, custom_values});
      return it == custom_maps_.end() ? nullptr : &it->second;
    }
    auto it = kernel_maps_.find(k);
    return it == kernel_maps_.end() ? nullptr : &it->second;
  };
  auto store = [&](const kernel_map_key_type &k, HipKernelMap m) -> const HipKernelMap & {
    if (region_type == RegionType::CUSTOM)
      return custom_maps_[{k, custom_values}] = std::move(m);
    return kernel_maps_[k] = std::move(m);
  };
  if (const HipKernelMap *hit = find(key))
    return *hit;
  // A pooling map through a kernel region keeps its transposed table
  // compacted (rhip_table_compact): pooling reduces sets of rows, and the
  // input side of a strided map uses few of the K offsets.
  auto store_pool = [&](HipKernelMap m) -> const HipKernelMap & {
    if (is_pool && !m.stride_map && m.n_in > 0 && m.K > 1) {
      if (m.symmetric) // pooling reduces through the transposed table itself
        m.ensure_transposed();
      const auto dev = m.nbr_t.device();
      at::DeviceGuard guard(dev);
      auto src = m.nbr_t.contiguous();
      auto out = torch::empty_like(src);
      auto ws = device_bytes(256, dev);
      int32_t used = 0;
      check_rhip(rhip_table_compact(src.data_ptr<int32_t>(), static_cast<int32_t>(src.size(0)),
                                    src.size(1), ws.data_ptr(), ws.numel(),
                                    out.data_ptr<int32_t>(), &used, current_stream(dev)),
                 "rhip_table_compact");
      m.nbr_t = out.slice(0, 0, std::max<int32_t>(used, 1));
    }
    return store(key, std::move(m));
  };

  const CoordinateMapHIP &in_map = coordinate_map(in_key);
  const CoordinateMapHIP &out_map = coordinate_map(out_key);
  TORCH_CHECK(static_cast<int64_t>(kdim) + 1 == in_map.coords.size(1), "kernel size mismatch");
  TORCH_CHECK(static_cast<int64_t>(kdim) + 1 == out_map.coords.size(1), "kernel size mismatch");

  if (!is_transpose) {
    if (use_stride_map)
      return store(key, generate_stride_map(in_map, out_map));
    // region on the input map's tensor stride (space_impl.hpp:626-636)
    auto off = region_offsets(region_type, kernel_size, kernel_dilation, in_map.tensor_stride,
                              custom);
    return store_pool(generate(in_map, out_map, off));
  }
  const kernel_map_key_type fwd_key =
      std::make_tuple(out_key.get_key(), in_key.get_key(), kernel_size, kernel_stride,
                      kernel_dilation, region_type, false, is_pool);
  if (const HipKernelMap *fwd = find(fwd_key))
    return store_pool(fwd->swapped());
  // the stride map runs out -> in, then swapped (space_impl.hpp:660-669)
  if (use_stride_map)
    return store(key, generate_stride_map(out_map, in_map).swapped());
  // generated out -> in with the region on the output (finer) map's stride,
  // then swapped (space_impl.hpp:649-697)
  auto off = region_offsets(region_type, kernel_size, kernel_dilation, out_map.tensor_stride,
                            custom);
  return store_pool(generate(out_map, in_map, off).swapped());
}

std::string CoordinateManager::to_string() const {
  std::ostringstream o;
  o << "CoordinateManager(D=" << D_ << ", maps=" << maps_.size()
    << ", kernel_maps=" << kernel_map_cache_size() << ")";
  return o.str();
}

} // namespace riemann
