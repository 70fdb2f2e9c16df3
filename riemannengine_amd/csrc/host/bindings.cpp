// pybind11 module riemannengine_amd._C: the host layer's SparseTensor,
// CoordinateManager and layers, with the names and arguments of the
// reference's Python bindings (python/src/sparse_bindings.cpp:80-219,
// python/src/nn_bindings.cpp:89-150).
#include <torch/extension.h>

#include "riemann.hpp"

namespace py = pybind11;
using namespace riemann;

namespace {

template <typename Impl> using ModuleClass = py::class_<Impl, std::shared_ptr<Impl>>;
template <typename T> struct type_tag { using type = T; };

// torch_python registers torch::nn::Module itself, so the layers expose the
// module surface they need directly.
template <typename Impl> ModuleClass<Impl> bind_module(py::module_ &m, const char *name) {
  ModuleClass<Impl> cls(m, name);
  cls.def(
      "parameters", [](Impl &self, bool recurse) { return self.parameters(recurse); },
      py::arg("recurse") = true);
  cls.def(
      "named_parameters",
      [](Impl &self, bool recurse) {
        py::dict result;
        for (const auto &pair : self.named_parameters(recurse))
          result[py::str(pair.key())] = pair.value();
        return result;
      },
      py::arg("recurse") = true);
  cls.def(
      "named_buffers",
      [](Impl &self, bool recurse) {
        py::dict result;
        for (const auto &pair : self.named_buffers(recurse))
          result[py::str(pair.key())] = pair.value();
        return result;
      },
      py::arg("recurse") = true);
  cls.def(
      "train", [](Impl &self, bool mode) { self.train(mode); }, py::arg("mode") = true);
  cls.def("eval", [](Impl &self) { self.eval(); });
  cls.def_property_readonly("training", [](const Impl &self) { return self.is_training(); });
  cls.def(
      "to", [](Impl &self, at::Device device) { self.to(device); }, py::arg("device"));
  cls.def(
      "to", [](Impl &self, at::ScalarType dtype) { self.to(dtype); }, py::arg("dtype"));
  cls.def(
      "to_dtype", [](Impl &self, at::ScalarType dtype) { self.to(dtype); }, py::arg("dtype"));
  cls.def("zero_grad", [](Impl &self) { self.zero_grad(); });
  cls.def("reset", [](Impl &self) { self.reset(); });
  cls.def("__repr__", [name](const Impl &) { return std::string("<riemannengine_amd.nn.") + name + ">"; });
  return cls;
}

template <typename Impl> ModuleClass<Impl> bind_unary(py::module_ &m, const char *name) {
  auto cls = bind_module<Impl>(m, name);
  cls.def(
      "forward", [](Impl &self, const SparseTensor &input) { return self.forward(input); },
      py::arg("input"));
  cls.def(
      "__call__", [](Impl &self, const SparseTensor &input) { return self.forward(input); },
      py::arg("input"));
  return cls;
}

// A kernel map's fields by name (the reference's Python callers read maps as
// dicts); the pair lists and a symmetric map's transposed table are built on
// first access.
py::object kernel_map_field(const HipKernelMap &m, const std::string &name) {
  if (name == "K")
    return py::int_(m.K);
  if (name == "n_in")
    return py::int_(m.n_in);
  if (name == "n_out")
    return py::int_(m.n_out);
  if (name == "offsets")
    return py::cast(m.offsets);
  if (name == "offsets_host")
    return py::cast(m.offsets_host);
  if (name == "nbr")
    return py::cast(m.nbr);
  if (name == "out_order")
    return py::cast(m.out_order);
  if (name == "stride_map")
    return py::bool_(m.stride_map);
  if (name == "symmetric")
    return py::bool_(m.symmetric);
  if (name == "partner")
    return m.partner.defined() ? py::cast(m.partner) : py::none();
  if (name == "in_rows" || name == "out_rows") {
    m.ensure_pairs();
    return py::cast(name == "in_rows" ? m.in_rows : m.out_rows);
  }
  if (name == "nbr_t" || name == "in_order") {
    if (m.symmetric)
      m.ensure_transposed();
    return py::cast(name == "nbr_t" ? m.nbr_t : m.in_order);
  }
  throw py::key_error(name);
}

stride_type as_stride(const std::vector<int64_t> &v) {
  stride_type s;
  for (auto x : v) {
    TORCH_CHECK(x > 0, "strides and kernel sizes must be positive");
    s.push_back(static_cast<uint32_t>(x));
  }
  return s;
}

} // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "RiemannEngine host API over the MI355X HIP sparse-convolution kernels";

  py::enum_<SparseTensorQuantizationMode::Type>(m, "QuantizationMode")
      .value("RANDOM_SUBSAMPLE", SparseTensorQuantizationMode::RANDOM_SUBSAMPLE)
      .value("UNWEIGHTED_AVERAGE", SparseTensorQuantizationMode::UNWEIGHTED_AVERAGE)
      .value("UNWEIGHTED_SUM", SparseTensorQuantizationMode::UNWEIGHTED_SUM)
      .value("MAX_POOL", SparseTensorQuantizationMode::MAX_POOL)
      .value("NO_QUANTIZATION", SparseTensorQuantizationMode::NO_QUANTIZATION);
  py::enum_<CoordinateMapBackend::Type>(m, "CoordinateMapBackend")
      .value("CPU", CoordinateMapBackend::CPU)
      .value("CUDA", CoordinateMapBackend::CUDA);
  py::enum_<RiemannAlgorithm::Mode>(m, "RiemannAlgorithm")
      .value("DEFAULT", RiemannAlgorithm::DEFAULT)
      .value("MEMORY_EFFICIENT", RiemannAlgorithm::MEMORY_EFFICIENT)
      .value("SPEED_OPTIMIZED", RiemannAlgorithm::SPEED_OPTIMIZED);
  py::enum_<RegionType::Type>(m, "RegionType")
      .value("HYPER_CUBE", RegionType::HYPER_CUBE)
      .value("HYPER_CROSS", RegionType::HYPER_CROSS)
      .value("CUSTOM", RegionType::CUSTOM);
  py::enum_<ConvolutionMode::Type>(m, "ConvolutionMode")
      .value("DEFAULT", ConvolutionMode::DEFAULT)
      .value("DIRECT_GEMM", ConvolutionMode::DIRECT_GEMM)
      .value("COPY_GEMM", ConvolutionMode::COPY_GEMM);
  py::enum_<PoolingMode::Type>(m, "PoolingMode")
      .value("LOCAL_SUM_POOLING", PoolingMode::LOCAL_SUM_POOLING)
      .value("LOCAL_AVG_POOLING", PoolingMode::LOCAL_AVG_POOLING)
      .value("LOCAL_MAX_POOLING", PoolingMode::LOCAL_MAX_POOLING)
      .value("GLOBAL_SUM_POOLING_DEFAULT", PoolingMode::GLOBAL_SUM_POOLING_DEFAULT)
      .value("GLOBAL_AVG_POOLING_DEFAULT", PoolingMode::GLOBAL_AVG_POOLING_DEFAULT)
      .value("GLOBAL_MAX_POOLING_DEFAULT", PoolingMode::GLOBAL_MAX_POOLING_DEFAULT)
      .value("GLOBAL_SUM_POOLING_KERNEL", PoolingMode::GLOBAL_SUM_POOLING_KERNEL)
      .value("GLOBAL_AVG_POOLING_KERNEL", PoolingMode::GLOBAL_AVG_POOLING_KERNEL)
      .value("GLOBAL_MAX_POOLING_KERNEL", PoolingMode::GLOBAL_MAX_POOLING_KERNEL)
      .value("GLOBAL_SUM_POOLING_PYTORCH_INDEX", PoolingMode::GLOBAL_SUM_POOLING_PYTORCH_INDEX)
      .value("GLOBAL_AVG_POOLING_PYTORCH_INDEX", PoolingMode::GLOBAL_AVG_POOLING_PYTORCH_INDEX)
      .value("GLOBAL_MAX_POOLING_PYTORCH_INDEX", PoolingMode::GLOBAL_MAX_POOLING_PYTORCH_INDEX);

  m.def(
      "region_offsets",
      [](RegionType::Type region, const std::vector<int64_t> &kernel_size,
         const std::vector<int64_t> &dilation, const std::vector<int64_t> &tensor_stride,
         c10::optional<at::Tensor> custom) {
        return region_offsets(region, as_stride(kernel_size), as_stride(dilation),
                              as_stride(tensor_stride), custom.value_or(at::Tensor()));
      },
      py::arg("region"), py::arg("kernel_size"), py::arg("dilation"), py::arg("tensor_stride"),
      py::arg("custom") = py::none());

  py::class_<CoordinateMapKey>(m, "CoordinateMapKey")
      .def(py::init([](const std::vector<int64_t> &tensor_stride, std::string string_id) {
             return CoordinateMapKey(as_stride(tensor_stride), std::move(string_id));
           }),
           py::arg("tensor_stride"), py::arg("string_id") = "")
      .def_property_readonly("tensor_stride", &CoordinateMapKey::get_tensor_stride)
      .def_property_readonly("coordinate_size", &CoordinateMapKey::get_coordinate_size)
      .def_property_readonly("string_id",
                             [](const CoordinateMapKey &k) { return k.get_key().second; })
      .def("is_key_set", &CoordinateMapKey::is_key_set)
      .def("__eq__", [](const CoordinateMapKey &a, const CoordinateMapKey &b) { return a == b; })
      .def("__hash__", &CoordinateMapKey::hash)
      .def("__repr__", &CoordinateMapKey::to_string);

  // a cached map of a manager (alive as long as the manager): fields as
  // attributes or by name, m["in_rows"]
  py::class_<HipKernelMap>(m, "KernelMap")
      .def("__getitem__", &kernel_map_field)
      .def("__getattr__", &kernel_map_field)
      .def("__len__", &HipKernelMap::size)
      .def("__repr__", [](const HipKernelMap &k) {
        return "KernelMap(K=" + std::to_string(k.K) + ", n_in=" + std::to_string(k.n_in) +
               ", n_out=" + std::to_string(k.n_out) + ", pairs=" + std::to_string(k.size()) +
               (k.symmetric ? ", symmetric" : "") + ")";
      });

  py::class_<CoordinateManager, std::shared_ptr<CoordinateManager>>(m, "CoordinateManager")
      .def(py::init([](int dimension, CoordinateMapBackend::Type backend,
                       RiemannAlgorithm::Mode algorithm) {
             return std::make_shared<CoordinateManager>(
                 dimension, backend, GPUMemoryAllocatorBackend::PYTORCH, algorithm);
           }),
           py::arg("dimension"), py::arg("backend") = CoordinateMapBackend::CUDA,
           py::arg("algorithm") = RiemannAlgorithm::DEFAULT)
      .def_property_readonly("dimension", &CoordinateManager::D)
      .def(
          "insert_and_map",
          [](CoordinateManager &self, const at::Tensor &coordinates,
             const std::vector<int64_t> &tensor_stride, std::string string_id) {
            return self.insert_and_map(coordinates, as_stride(tensor_stride),
                                       std::move(string_id));
          },
          py::arg("coordinates"), py::arg("tensor_stride"), py::arg("string_id") = "")
      .def(
          "stride",
          [](CoordinateManager &self, const CoordinateMapKey &key,
             const std::vector<int64_t> &kernel_stride, std::string string_id) {
            return self.stride(key, as_stride(kernel_stride), std::move(string_id));
          },
          py::arg("coordinate_map_key"), py::arg("kernel_stride"), py::arg("string_id") = "")
      .def(
          "stride_region",
          [](CoordinateManager &self, const CoordinateMapKey &key, const at::Tensor &offsets,
             const std::vector<int64_t> &out_tensor_stride, bool expand) {
            return self.stride_region(key, offsets.to(at::kCPU), as_stride(out_tensor_stride),
                                      expand);
          },
          py::arg("coordinate_map_key"), py::arg("region_offsets"),
          py::arg("out_tensor_stride"), py::arg("expand_coordinates") = true)
      .def("size", [](const CoordinateManager &self,
                      const CoordinateMapKey &key) { return self.size(key); })
      .def("exists", &CoordinateManager::exists)
      .def("get_coordinates", &CoordinateManager::get_coordinates,
           py::arg("coordinate_map_key"))
      .def(
          "kernel_map",
          [](CoordinateManager &self, const CoordinateMapKey &in_key,
             const CoordinateMapKey &out_key, const std::vector<int64_t> &kernel_size,
             const std::vector<int64_t> &kernel_stride, const std::vector<int64_t> &dilation,
             RegionType::Type region, c10::optional<at::Tensor> offsets, bool is_transpose,
             bool is_pool) {
            return &self.kernel_map(in_key, out_key, as_stride(kernel_size),
                                    as_stride(kernel_stride), as_stride(dilation), region,
                                    offsets.value_or(at::Tensor()), is_transpose, is_pool);
          },
          py::return_value_policy::reference_internal,
          py::arg("in_key"), py::arg("out_key"), py::arg("kernel_size"),
          py::arg("kernel_stride"), py::arg("kernel_dilation"),
          py::arg("region_type") = RegionType::HYPER_CUBE, py::arg("offsets") = py::none(),
          py::arg("is_transpose") = false, py::arg("is_pool") = false)
      .def_property_readonly("kernel_map_cache_size", &CoordinateManager::kernel_map_cache_size)
      .def("__repr__", &CoordinateManager::to_string);

  py::class_<SparseTensor>(m, "SparseTensor")
      .def(py::init([](at::Tensor features, at::Tensor coordinates,
                       std::shared_ptr<CoordinateManager> manager,
                       SparseTensorQuantizationMode::Type quantization_mode,
                       RiemannAlgorithm::Mode algorithm) {
             return SparseTensor(std::move(features), std::move(coordinates), std::move(manager),
                                 quantization_mode, GPUMemoryAllocatorBackend::PYTORCH,
                                 algorithm);
           }),
           py::arg("features"), py::arg("coordinates"),
           py::arg("coordinate_manager") = std::shared_ptr<CoordinateManager>(),
           py::arg("quantization_mode") = SparseTensorQuantizationMode::RANDOM_SUBSAMPLE,
           py::arg("algorithm") = RiemannAlgorithm::DEFAULT)
      .def(py::init<at::Tensor, CoordinateMapKey, std::shared_ptr<CoordinateManager>>(),
           py::arg("features"), py::arg("coordinate_map_key"), py::arg("coordinate_manager"))
      .def_property_readonly("F", &SparseTensor::F)
      .def_property_readonly("C", &SparseTensor::C)
      .def_property_readonly("features", &SparseTensor::F)
      .def_property_readonly("coordinates", &SparseTensor::C)
      .def_property_readonly("coordinate_map_key", &SparseTensor::coordinate_map_key)
      .def_property_readonly("coordinate_manager", &SparseTensor::coordinate_manager)
      .def_property_readonly("tensor_stride", &SparseTensor::tensor_stride)
      .def_property_readonly("dimension", &SparseTensor::dimension)
      .def_property_readonly("device", &SparseTensor::device)
      .def_property_readonly("dtype", &SparseTensor::dtype)
      .def_property_readonly("requires_grad", &SparseTensor::requires_grad)
      .def_property_readonly("shape",
                             [](const SparseTensor &s) {
                               return py::make_tuple(s.F().size(0), s.F().size(1));
                             })
      .def("__len__", [](const SparseTensor &s) { return s.F().size(0); })
      .def("__add__", [](const SparseTensor &a, const SparseTensor &b) { return a + b; })
      .def("__sub__", [](const SparseTensor &a, const SparseTensor &b) { return a - b; })
      .def("__mul__", [](const SparseTensor &a, const SparseTensor &b) { return a * b; })
      .def("__truediv__", [](const SparseTensor &a, const SparseTensor &b) { return a / b; })
      .def("__add__", [](const SparseTensor &s, double v) { return s + v; })
      .def("__radd__", [](const SparseTensor &s, double v) { return s + v; })
      .def("__mul__", [](const SparseTensor &s, double v) { return s * v; })
      .def("__rmul__", [](const SparseTensor &s, double v) { return s * v; })
      .def("__iadd__", [](SparseTensor &s, const SparseTensor &o) -> SparseTensor & {
        return s += o;
      })
      .def("detach", &SparseTensor::detach)
      .def("to", py::overload_cast<torch::Device>(&SparseTensor::to, py::const_),
           py::arg("device"))
      .def("to", py::overload_cast<c10::ScalarType>(&SparseTensor::to, py::const_),
           py::arg("dtype"))
      .def("float", &SparseTensor::float_)
      .def("double", &SparseTensor::double_)
      // earlier spelling of to(dtype), kept as an alias
      .def("to_dtype", py::overload_cast<c10::ScalarType>(&SparseTensor::to, py::const_))
      .def("__repr__", [](const SparseTensor &s) {
        return "SparseTensor(rows=" + std::to_string(s.F().size(0)) +
               ", channels=" + std::to_string(s.F().size(1)) + ", " +
               s.coordinate_map_key().to_string() + ")";
      });

  auto nn = m.def_submodule("nn", "layers over the HIP sparse convolution");
  auto conv = bind_unary<RiemannConvolutionImpl>(nn, "RiemannConvolution");
  conv.def(py::init([](int in_channels, int out_channels, int kernel_size, int stride,
                       int dilation, bool bias, bool expand_coordinates,
                       ConvolutionMode::Type convolution_mode, int dimension) {
             return std::make_shared<RiemannConvolutionImpl>(in_channels, out_channels,
                                                             kernel_size, stride, dilation, bias,
                                                             expand_coordinates,
                                                             convolution_mode, dimension);
           }),
           py::arg("in_channels"), py::arg("out_channels"), py::arg("kernel_size") = 3,
           py::arg("stride") = 1, py::arg("dilation") = 1, py::arg("bias") = false,
           py::arg("expand_coordinates") = false,
           py::arg("convolution_mode") = ConvolutionMode::DEFAULT, py::arg("dimension") = 3);
  conv.def_property_readonly("kernel",
                             [](RiemannConvolutionImpl &self) { return self.base()->kernel_; });
  conv.def_property_readonly("bias",
                             [](RiemannConvolutionImpl &self) { return self.base()->bias_; });

  auto convt = bind_unary<RiemannConvolutionTransposeImpl>(nn, "RiemannConvolutionTranspose");
  convt.def(py::init([](int in_channels, int out_channels, int kernel_size, int stride,
                        int dilation, bool bias, bool expand_coordinates,
                        ConvolutionMode::Type convolution_mode, int dimension) {
              return std::make_shared<RiemannConvolutionTransposeImpl>(
                  in_channels, out_channels, kernel_size, stride, dilation, bias,
                  expand_coordinates, convolution_mode, dimension);
            }),
            py::arg("in_channels"), py::arg("out_channels"), py::arg("kernel_size") = 3,
            py::arg("stride") = 1, py::arg("dilation") = 1, py::arg("bias") = false,
            py::arg("expand_coordinates") = false,
            py::arg("convolution_mode") = ConvolutionMode::DEFAULT, py::arg("dimension") = 3);
  convt.def_property_readonly(
      "kernel", [](RiemannConvolutionTransposeImpl &self) { return self.base()->kernel_; });
  convt.def_property_readonly(
      "bias", [](RiemannConvolutionTransposeImpl &self) { return self.base()->bias_; });

  auto gconvt = bind_unary<RiemannGenerativeConvolutionTransposeImpl>(
      nn, "RiemannGenerativeConvolutionTranspose");
  gconvt.def(py::init([](int in_channels, int out_channels, int kernel_size, int stride,
                         int dilation, bool bias, ConvolutionMode::Type convolution_mode,
                         int dimension) {
               return std::make_shared<RiemannGenerativeConvolutionTransposeImpl>(
                   in_channels, out_channels, kernel_size, stride, dilation, bias,
                   convolution_mode, dimension);
             }),
             py::arg("in_channels"), py::arg("out_channels"), py::arg("kernel_size") = 3,
             py::arg("stride") = 1, py::arg("dilation") = 1, py::arg("bias") = false,
             py::arg("convolution_mode") = ConvolutionMode::DEFAULT, py::arg("dimension") = 3);
  gconvt.def_property_readonly("kernel", [](RiemannGenerativeConvolutionTransposeImpl &self) {
    return self.base()->kernel_;
  });

  bind_unary<RiemannBatchNormImpl>(nn, "RiemannBatchNorm")
      .def(py::init([](int64_t num_features, double eps, double momentum, bool affine,
                       bool track_running_stats) {
             return std::make_shared<RiemannBatchNormImpl>(num_features, eps, momentum, affine,
                                                           track_running_stats);
           }),
           py::arg("num_features"), py::arg("eps") = 1e-5, py::arg("momentum") = 0.1,
           py::arg("affine") = true, py::arg("track_running_stats") = true);
  bind_unary<RiemannReLUImpl>(nn, "RiemannReLU")
      .def(py::init([](bool inplace) { return std::make_shared<RiemannReLUImpl>(inplace); }),
           py::arg("inplace") = false);
  // pooling (python/src/nn_bindings.cpp:344-403)
  auto local_pool = [&](auto tag, const char *name) {
    using Impl = typename decltype(tag)::type;
    bind_unary<Impl>(nn, name)
        .def(py::init([](int kernel_size, int stride, int dilation, int dimension) {
               return std::make_shared<Impl>(kernel_size, stride, dilation, dimension);
             }),
             py::arg("kernel_size"), py::arg("stride") = 1, py::arg("dilation") = 1,
             py::arg("dimension") = 3);
  };
  local_pool(type_tag<RiemannAvgPoolingImpl>{}, "RiemannAvgPooling");
  local_pool(type_tag<RiemannSumPoolingImpl>{}, "RiemannSumPooling");
  local_pool(type_tag<RiemannMaxPoolingImpl>{}, "RiemannMaxPooling");
  bind_unary<RiemannPoolingTransposeImpl>(nn, "RiemannPoolingTranspose")
      .def(py::init([](int kernel_size, int stride, int dilation, bool expand_coordinates,
                       int dimension) {
             return std::make_shared<RiemannPoolingTransposeImpl>(
                 kernel_size, stride, dilation, expand_coordinates, dimension);
           }),
           py::arg("kernel_size"), py::arg("stride"), py::arg("dilation") = 1,
           py::arg("expand_coordinates") = false, py::arg("dimension") = 3)
      .def(py::init([](int kernel_size, int stride, int dilation, bool expand_coordinates,
                       int dimension, PoolingMode::Type mode) {
             return std::make_shared<RiemannPoolingTransposeImpl>(
                 KernelGenerator({kernel_size}, {stride}, {dilation}, true,
                                 RegionType::HYPER_CUBE, {}, expand_coordinates, dimension),
                 dimension, mode);
           }),
           py::arg("kernel_size"), py::arg("stride"), py::arg("dilation"),
           py::arg("expand_coordinates"), py::arg("dimension"), py::arg("mode"));
  bind_unary<RiemannGlobalPoolingImpl>(nn, "RiemannGlobalPooling")
      .def(py::init([](PoolingMode::Type mode) {
             return std::make_shared<RiemannGlobalPoolingImpl>(mode);
           }),
           py::arg("mode") = PoolingMode::GLOBAL_AVG_POOLING_PYTORCH_INDEX);
  bind_unary<RiemannGlobalSumPoolingImpl>(nn, "RiemannGlobalSumPooling")
      .def(py::init([]() { return std::make_shared<RiemannGlobalSumPoolingImpl>(); }));
  bind_unary<RiemannGlobalAvgPoolingImpl>(nn, "RiemannGlobalAvgPooling")
      .def(py::init([]() { return std::make_shared<RiemannGlobalAvgPoolingImpl>(); }));
  bind_unary<RiemannGlobalMaxPoolingImpl>(nn, "RiemannGlobalMaxPooling")
      .def(py::init([]() { return std::make_shared<RiemannGlobalMaxPoolingImpl>(); }));

  // downsample: an optional projection of the block input (a convolution),
  // registered as the module's "downsample" (residual.hpp:12-29)
  bind_unary<BasicBlockImpl>(nn, "BasicBlock")
      .def(py::init([](int inplanes, int planes, int stride, int dilation,
                       std::shared_ptr<RiemannConvolutionImpl> downsample, double bn_momentum,
                       int dimension) {
             torch::nn::AnyModule ds;
             if (downsample)
               ds = torch::nn::AnyModule(RiemannConvolution(downsample));
             return std::make_shared<BasicBlockImpl>(inplanes, planes, stride, dilation,
                                                     std::move(ds), bn_momentum, dimension);
           }),
           py::arg("inplanes"), py::arg("planes"), py::arg("stride") = 1,
           py::arg("dilation") = 1, py::arg("downsample") = py::none(), py::arg("bn_momentum") = 0.1,
           py::arg("dimension") = 3);
}
