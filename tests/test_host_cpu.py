"""C++ host layer (riemannengine_amd._C) without a GPU: it loads, mirrors the
reference's argument checks and error behaviour, enumerates stencil offsets
like the reference, and initialises layer parameters as the reference does.
No kernel runs here."""
import numpy as np
import pytest
import torch

import oracle
import riemannengine_amd as re_
from riemannengine_amd import stencil


def test_host_module_exports():
    for name in ("SparseTensor", "CoordinateManager", "CoordinateMapKey", "QuantizationMode",
                 "RegionType", "nn"):
        assert getattr(re_, name) is not None
    for name in ("RiemannConvolution", "RiemannConvolutionTranspose",
                 "RiemannGenerativeConvolutionTranspose", "RiemannBatchNorm", "RiemannReLU",
                 "BasicBlock"):
        assert hasattr(re_.nn, name)


@pytest.mark.parametrize("region,ks,dil,ts,custom", [
    ("cube", [3, 3, 3], [1, 1, 1], [1, 1, 1], None),
    ("cube", [2, 2, 2], [1, 1, 1], [2, 2, 2], None),
    ("cube", [3, 3, 3, 3], [2, 2, 2, 2], [1, 2, 1, 4], None),
    ("cube", [5, 3, 1], [1, 2, 1], [1, 1, 1], None),
    ("cross", [3, 3, 3], [1, 1, 1], [1, 1, 1], None),
    ("cross", [5, 3], [1, 1], [2, 1], None),
    ("custom", [3, 3, 3], [2, 2, 2], [1, 1, 3], np.array([[1, 0, 0], [0, -2, 3], [0, 0, 0]])),
])
def test_region_offsets_match_oracle_and_python(region, ks, dil, ts, custom):
    """The C++ enumeration (used by the layers), the Python one (used by
    bench.py) and the oracle (pinned by closed forms) agree offset for offset."""
    rt = {"cube": re_.RegionType.HYPER_CUBE, "cross": re_.RegionType.HYPER_CROSS,
          "custom": re_.RegionType.CUSTOM}[region]
    got = re_.region_offsets(rt, ks, dil, ts,
                             None if custom is None else torch.from_numpy(custom)).numpy()
    D = len(ks)
    ref = oracle.region_offsets(D, ks, dil, ts, region, custom)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(stencil.region_offsets(D, ks, dil, ts, region, custom), ref)


def test_device_backend_only():
    with pytest.raises(RuntimeError, match="no CPU coordinate manager"):
        re_.CoordinateManager(3, re_.CoordinateMapBackend.CPU)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        re_.SparseTensor(torch.zeros(3, 2), torch.zeros(3, 4, dtype=torch.int32))


def test_coordinate_map_key():
    k = re_.CoordinateMapKey([2, 2, 2], "x")
    assert k.coordinate_size == 4 and k.tensor_stride == [2, 2, 2] and k.string_id == "x"
    assert k == re_.CoordinateMapKey([2, 2, 2], "x")
    assert not (k == re_.CoordinateMapKey([2, 2, 2], "y"))
    assert "coordinate map key:[2, 2, 2]:x" in repr(k)


@pytest.mark.parametrize("cin,cout,ks,D,transpose", [(4, 8, 3, 3, False), (16, 32, 3, 3, False),
                                                     (8, 4, 2, 3, True), (3, 5, 3, 4, False)])
def test_conv_parameters_like_reference(cin, cout, ks, D, transpose):
    """kernel [K, Cin, Cout], bias [1, Cout], U(+-1/sqrt(fan)) with fan =
    Cin*K (Cout*K transposed): engine/nn/conv.cpp:70-102."""
    torch.manual_seed(0)
    cls = re_.nn.RiemannConvolutionTranspose if transpose else re_.nn.RiemannConvolution
    conv = cls(cin, cout, kernel_size=ks, stride=1, bias=True, dimension=D)
    K = ks ** D
    assert tuple(conv.kernel.shape) == (K, cin, cout)
    assert tuple(conv.bias.shape) == (1, cout)
    bound = 1.0 / np.sqrt((cout if transpose else cin) * K)
    w = conv.kernel.detach()
    assert w.abs().max().item() <= bound
    assert w.abs().max().item() > 0.9 * bound  # uniform over the whole interval
    assert conv.bias.detach().abs().max().item() <= bound
    assert set(conv.named_parameters()) == {"base.kernel", "base.bias"}


def test_basic_block_structure():
    blk = re_.nn.BasicBlock(8, 8)
    names = set(blk.named_parameters())
    assert {"conv1.base.kernel", "conv2.base.kernel", "norm1.normalization.weight",
            "norm2.normalization.bias"} <= names
    assert {"norm1.normalization.running_mean", "norm2.normalization.running_var",
            "norm1.normalization.num_batches_tracked"} <= set(blk.named_buffers())
    blk.eval()
    assert not blk.training


def test_basic_block_registers_downsample():
    """A projection passed as `downsample` is one of the block's parameters
    (tests/engine/test_layers.cpp:303-318)."""
    proj = re_.nn.RiemannConvolution(8, 16, kernel_size=1, stride=2)
    blk = re_.nn.BasicBlock(8, 16, stride=2, downsample=proj)
    p = blk.named_parameters()
    assert "downsample.base.kernel" in p
    assert p["downsample.base.kernel"].data_ptr() == proj.kernel.data_ptr()
    assert "downsample.base.kernel" not in re_.nn.BasicBlock(8, 8).named_parameters()


def test_batch_norm_state_names_match_torch():
    """RiemannBatchNorm keeps torch BatchNorm1d's parameters and buffers
    under `normalization.` (engine/nn/normalization.hpp:14-23)."""
    bn = re_.nn.RiemannBatchNorm(6)
    ref = torch.nn.BatchNorm1d(6)
    assert set(bn.named_parameters()) == {"normalization." + k for k, _ in
                                          ref.named_parameters()}
    assert set(bn.named_buffers()) == {"normalization." + k for k, _ in ref.named_buffers()}
    assert set(re_.nn.RiemannBatchNorm(6, affine=False).named_parameters()) == set()


def test_invalid_layer_arguments():
    with pytest.raises(RuntimeError, match="channel counts must be positive"):
        re_.nn.RiemannConvolution(0, 4)
    with pytest.raises(RuntimeError, match="positive"):
        re_.nn.RiemannConvolution(4, 4, kernel_size=0)


def test_reference_module_path():
    """`import riemannengine` and `import riemannengine.nn`, the reference's
    module path (python/riemannengine/__init__.py:14-37), expose the host
    layer's classes themselves."""
    import riemannengine
    import riemannengine.nn as rnn
    assert riemannengine.SparseTensor is re_.SparseTensor
    assert riemannengine.CoordinateManager is re_.CoordinateManager
    assert rnn is re_.nn and rnn.RiemannConvolution is re_.nn.RiemannConvolution
    for name in riemannengine.__all__:
        assert getattr(riemannengine, name) is not None
