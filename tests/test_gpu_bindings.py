"""The reference's Python binding smoke tests (python/tests/test_bindings.py:
10-115, TestSparseTensor and TestNN) on device tensors, written against the
reference's module path `riemannengine`: construction, quantization, the
coordinate manager, convolution forward and backward, the strided
convolution, ReLU and batch norm, global pooling, the BasicBlock and an
optimizer step. The layers run the HIP kernels through the C ABI. The
reference's RiemannLinear test (:106-110) is left out: the linear layer is
not on the sparse-convolution path."""
import pytest
import torch

import riemannengine as re_
import riemannengine.nn  # noqa: F401  (the submodule import the reference supports)

from helpers import DEV

pytestmark = pytest.mark.gpu


def make_sparse_tensor(n=64, channels=4, dimension=3, batch=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    coords = torch.randint(0, 10, (n, dimension), generator=g, dtype=torch.int32)
    batch_idx = torch.randint(0, batch, (n, 1), generator=g, dtype=torch.int32)
    coords = torch.cat([batch_idx, coords], dim=1)
    feats = torch.randn(n, channels, generator=g)
    return re_.SparseTensor(feats.to(DEV), coords.to(DEV))


class TestSparseTensor:
    def test_construction(self):
        x = make_sparse_tensor()
        assert x.F.shape[1] == 4
        assert x.C.shape[1] == 4  # batch + 3 spatial
        assert x.F.shape[0] == x.C.shape[0]
        assert len(x) == x.F.shape[0]
        assert x.dimension == 3
        assert list(x.tensor_stride) == [1, 1, 1]
        assert "SparseTensor" in repr(x)
        assert x.F.is_cuda and x.C.is_cuda

    def test_quantization_modes(self):
        coords = torch.zeros(4, 4, dtype=torch.int32, device=DEV)  # all duplicates
        feats = torch.ones(4, 2, device=DEV)
        x = re_.SparseTensor(feats, coords,
                             quantization_mode=re_.QuantizationMode.UNWEIGHTED_SUM)
        assert len(x) == 1
        assert torch.allclose(x.F, torch.full((1, 2), 4.0, device=DEV))

    def test_arithmetic(self):
        x = make_sparse_tensor()
        y = (x + x) * 2.0
        assert torch.allclose(y.F, x.F * 4.0)

    def test_coordinate_manager_shared(self):
        x = make_sparse_tensor()
        manager = x.coordinate_manager
        assert manager is not None
        y = re_.SparseTensor(torch.randn(len(x), 2, device=DEV), x.C,
                             coordinate_manager=manager)
        assert y.coordinate_manager is not None


class TestNN:
    def test_convolution_forward_backward(self):
        x = make_sparse_tensor(channels=4)
        conv = re_.nn.RiemannConvolution(4, 8, kernel_size=3, dimension=3)
        conv.to(DEV)
        y = conv(x)
        assert y.F.shape[1] == 8
        y.F.sum().backward()
        grads = [p.grad for p in conv.parameters()]
        assert grads and all(g is not None for g in grads)

    def test_strided_convolution(self):
        x = make_sparse_tensor(channels=4)
        conv = re_.nn.RiemannConvolution(4, 8, kernel_size=2, stride=2)
        conv.to(DEV)
        y = conv(x)
        assert list(y.tensor_stride) == [2, 2, 2]

    def test_activation_and_norm(self):
        x = make_sparse_tensor(channels=4)
        relu = re_.nn.RiemannReLU()
        bn = re_.nn.RiemannBatchNorm(4)
        bn.to(DEV)
        y = relu(bn(x))
        assert (y.F >= 0).all()
        bn.eval()
        assert not bn.training

    def test_global_pooling(self):
        x = make_sparse_tensor(channels=4, batch=2)
        pool = re_.nn.RiemannGlobalAvgPooling()
        y = pool(x)
        assert tuple(y.F.shape) == (2, 4)

    def test_basic_block(self):
        x = make_sparse_tensor(channels=8)
        block = re_.nn.BasicBlock(8, 8)
        block.to(DEV)
        y = block(x)
        assert y.F.shape[1] == 8

    def test_optimizer_integration(self):
        x = make_sparse_tensor(channels=4)
        conv = re_.nn.RiemannConvolution(4, 4, bias=True)
        conv.to(DEV)
        optimizer = torch.optim.SGD(conv.parameters(), lr=0.1)
        before = conv.kernel.detach().clone()
        loss = conv(x).F.pow(2).sum()
        loss.backward()
        optimizer.step()
        assert not torch.allclose(before, conv.kernel.detach())


def test_union_binary_operations_match_numpy():
    """x + y, x - y, x * y over two different coordinate sets and tensor
    strides (sparse_tensor.cpp:32-57): the result holds the union of both
    sets in first-occurrence order (x's rows, then y's new ones) at the finer
    stride, each operand's features on its rows and 0 elsewhere."""
    import numpy as np
    g = torch.Generator().manual_seed(4)
    ca = torch.randint(0, 6, (300, 4), generator=g, dtype=torch.int32)
    cb = torch.randint(0, 6, (200, 4), generator=g, dtype=torch.int32)
    ca[:, 0] %= 2
    cb[:, 0] %= 2
    x = re_.SparseTensor(torch.randn(300, 3, generator=g).to(DEV), ca.to(DEV))
    y = re_.SparseTensor(torch.randn(200, 3, generator=g).to(DEV), cb.to(DEV))
    xc, yc = x.C.cpu().numpy(), y.C.cpu().numpy()
    xf, yf = x.F.cpu().numpy(), y.F.cpu().numpy()
    rows = {}
    for r in np.concatenate([xc, yc]).tolist():
        rows.setdefault(tuple(r), len(rows))
    ua, ub = np.zeros((len(rows), 3), np.float32), np.zeros((len(rows), 3), np.float32)
    ua[[rows[tuple(r)] for r in xc.tolist()]] = xf
    ub[[rows[tuple(r)] for r in yc.tolist()]] = yf
    for op, ref in (("+", ua + ub), ("-", ua - ub), ("*", ua * ub)):
        z = {"+": lambda: x + y, "-": lambda: x - y, "*": lambda: x * y}[op]()
        assert len(z) == len(rows)
        np.testing.assert_array_equal(z.C.cpu().numpy(), np.array(list(rows), np.int32))
        np.testing.assert_allclose(z.F.cpu().numpy(), ref, rtol=1e-6, atol=1e-6, err_msg=op)
        assert list(z.tensor_stride) == [1, 1, 1]
