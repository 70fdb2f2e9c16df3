"""The reference's Python module path, ``riemannengine``, over the MI355X
sparse-convolution hot path.

Callers of the reference write ``import riemannengine`` and ``import
riemannengine.nn`` (python/riemannengine/__init__.py:14-37 registers the
extension's ``nn`` submodule in ``sys.modules``). This package gives them the
same spellings for the names on the hot path, re-exported from the C++ host
layer ``riemannengine_amd._C``, whose convolution, pooling and batch-norm
layers call the gfx950 kernels through the C ABI:

    SparseTensor, CoordinateManager, CoordinateMapKey, CoordinateMapBackend,
    ConvolutionMode, PoolingMode, QuantizationMode, RegionType,
    RiemannAlgorithm, nn (RiemannConvolution, RiemannConvolutionTranspose,
    RiemannGenerativeConvolutionTranspose, the pooling layers,
    RiemannBatchNorm, RiemannReLU, BasicBlock)

The reference's names outside that path (``adaptive``, ``gaussian``,
``occupancy``, ``TensorField``, the collation helpers, ``RiemannLinear``, ...)
are not provided. Without the built host layer the import raises: there is no
CPU fallback.
"""
import sys as _sys

# the host layer links against torch's HIP libraries: load them first
import torch as _torch  # noqa: F401

try:
    from riemannengine_amd import _C
except ImportError as e:  # pragma: no cover - depends on the build
    raise ImportError("riemannengine needs the built HIP host layer: run "
                      "`python -m riemannengine_amd.build`") from e

from riemannengine_amd._C import (  # noqa: F401
    ConvolutionMode,
    CoordinateManager,
    CoordinateMapBackend,
    CoordinateMapKey,
    PoolingMode,
    QuantizationMode,
    RegionType,
    RiemannAlgorithm,
    SparseTensor,
    region_offsets,
)
from riemannengine_amd import __version__  # noqa: F401

nn = _C.nn
_sys.modules[__name__ + ".nn"] = nn

__all__ = [
    "ConvolutionMode",
    "CoordinateManager",
    "CoordinateMapBackend",
    "CoordinateMapKey",
    "PoolingMode",
    "QuantizationMode",
    "RegionType",
    "RiemannAlgorithm",
    "SparseTensor",
    "nn",
    "region_offsets",
]
