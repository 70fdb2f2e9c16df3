"""MI355X-native sparse-convolution hot path of RiemannEngine.

Coordinate hashing, kernel-map generation, gather-GEMM-scatter sparse
convolution (forward, dX, dW) and sparse pooling (stride maps, local and
global sum / average / max) as hand-written gfx950 HIP kernels behind the C
ABI in include/riemann_hip.h (libriemann_hip.so).

* ``SparseTensor``, ``CoordinateManager``, ``CoordinateMapKey``, ``nn`` and
  the enums come from the C++ host layer (``_C``), which mirrors the
  reference's riemann_cpp API over LibTorch and calls the kernels through the
  C ABI;
* ``abi`` binds the C ABI directly with ctypes;
* ``stencil`` enumerates convolution offsets; ``scenes`` generates the seeded
  benchmark point clouds.

The native libraries are built in-tree (``python -m riemannengine_amd.build``);
using the host API without them raises ImportError: there is no CPU path.
"""
__version__ = "0.1.0"

_HOST_NAMES = ("SparseTensor", "CoordinateManager", "CoordinateMapKey", "QuantizationMode",
               "CoordinateMapBackend", "RiemannAlgorithm", "RegionType", "ConvolutionMode",
               "PoolingMode", "region_offsets", "nn")


def __getattr__(name):
    if name in _HOST_NAMES:
        import torch  # noqa: F401  (loads the HIP runtime the extension links against)
        try:
            from . import _C
        except ImportError as e:
            raise ImportError(
                "riemannengine_amd._C is not built: run `python -m riemannengine_amd.build`") from e
        return getattr(_C, name)
    raise AttributeError(f"module 'riemannengine_amd' has no attribute {name!r}")
