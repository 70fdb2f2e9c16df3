"""The HIP path against the reference itself: the reference's CPU path is
compiled from source into oracle/_ref (oracle/ref.mk) and travels with the
tree, so the GPU box runs it next to the HIP kernels on the same inputs.

* kernel maps and strided output coordinates: bit-exact after ordering both
  sides' pairs by (offset, input coordinate, output coordinate);
* convolution forward, dX, dW: rel 1e-4 (fp32) and 2e-2 (bf16) of the
  reference's own result. The bf16 reference computes in bf16 (per-offset
  matmul and index_add_, conv.cpp:59-61), so this pins the bf16 path against
  the reference's arithmetic, not only against an fp32 restatement;
* the C++ host layer's RiemannConvolution against the reference's
  RiemannConvolution with the same weights.
Skipped where the reference library was not built."""
import numpy as np
import pytest
import torch

import oracle
from oracle import ref
from riemannengine_amd import abi
import riemannengine_amd as re_
from helpers import DEV, TOL, assert_rel, to_dev, random_coords

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not ref.available(),
                                 reason="oracle/_ref not built (no reference checkout)")]


def _canonical_by_coords(kofs, ir, orr, in_coords, out_coords):
    ks = np.repeat(np.arange(len(kofs) - 1), np.diff(kofs))
    t = np.concatenate([ks[:, None], in_coords[ir], out_coords[orr]], 1)
    return t[np.lexsort(t.T[::-1])]


def _align(rows_from, rows_to):
    """Permutation p with rows_from[p] == rows_to."""
    idx = {tuple(r): i for i, r in enumerate(rows_from.tolist())}
    return np.array([idx[tuple(r)] for r in rows_to.tolist()], np.int64)


def _gpu_map(c, ks, stride, dil, region):
    D = c.shape[1] - 1
    tin = abi.hash_build(to_dev(c))
    tout = tin if stride == 1 else abi.hash_build(abi.stride_coords(to_dev(c), [stride] * D))
    km = abi.kernel_map(tin, tout, oracle.region_offsets(D, ks, dil, 1, region))
    return tin, tout, km


@pytest.mark.parametrize("D,ks,stride,dil,region", [
    (3, 3, 1, 1, "cube"), (3, 3, 1, 2, "cube"), (3, 3, 1, 1, "cross"), (3, 2, 2, 1, "cube"),
    (3, 3, 2, 1, "cube"), (4, 3, 1, 1, "cube")])
def test_kernel_map_matches_reference(D, ks, stride, dil, region):
    rng = np.random.default_rng(D * 10 + ks + stride + dil)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, D, 16))
    print(f"ref kmap D={D} ks={ks} s={stride} dil={dil} {region} n={len(c)}", flush=True)
    kofs, ir, orr, oc = ref.kernel_map(c, ks, stride, dil, region)
    tin, tout, km = _gpu_map(c, ks, stride, dil, region)
    goc = tout.ucoords.cpu().numpy()
    assert sorted(map(tuple, goc.tolist())) == sorted(map(tuple, oc.tolist()))
    np.testing.assert_array_equal(km.offsets_host, kofs)
    np.testing.assert_array_equal(
        _canonical_by_coords(km.offsets_host, km.in_rows.cpu().numpy(), km.out_rows.cpu().numpy(),
                             c, goc),
        _canonical_by_coords(kofs, ir, orr, c, oc))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D,ks,stride,cin,cout", [
    (3, 3, 1, 64, 64), (3, 2, 2, 32, 64), (4, 3, 1, 32, 32)])
def test_conv_matches_reference(dtype, D, ks, stride, cin, cout):
    rng = np.random.default_rng(ks * 7 + stride + D + cin)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 8000, D, 12))
    K = ks ** D
    bf = (lambda a: torch.from_numpy(a).to(torch.bfloat16).float().numpy()) \
        if dtype == torch.bfloat16 else (lambda a: a)
    x = bf(rng.standard_normal((len(c), cin)).astype(np.float32))
    w = bf((rng.standard_normal((K, cin, cout)) * np.sqrt(2.0 / (cin * K))).astype(np.float32))
    gy_of = lambda oc: bf(np.random.default_rng(9).standard_normal((len(oc), cout))
                          .astype(np.float32))
    print(f"ref conv D={D} ks={ks} s={stride} {cin}->{cout} {dtype} n={len(c)}", flush=True)
    y_r, oc, gx_r, gw_r = ref.conv(c, x, w, gy=gy_of, ks=ks, stride=stride,
                                   bf16=dtype == torch.bfloat16)
    tin, tout, km = _gpu_map(c, ks, stride, 1, "cube")
    goc = tout.ucoords.cpu().numpy()
    p = _align(oc, goc)  # reference output row of each GPU output row
    gy = gy_of(oc)[p]
    y = abi.conv_forward(to_dev(x, dtype), to_dev(w, dtype), km)
    gx = abi.conv_backward_input(to_dev(gy, dtype), to_dev(w, dtype), km)
    gw = abi.conv_backward_weight(to_dev(x, dtype), to_dev(gy, dtype), km, K)
    tol = TOL[dtype]
    assert_rel(y.float().cpu().numpy(), y_r[p], tol, "Y vs reference")
    assert_rel(gx.float().cpu().numpy(), gx_r, tol, "dX vs reference")
    assert_rel(gw.float().cpu().numpy(), gw_r, tol, "dW vs reference")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_host_layer_matches_reference_layer(dtype):
    """riemannengine_amd.nn.RiemannConvolution on the GPU against the
    reference's RiemannConvolution on the CPU, same weights and inputs."""
    rng = np.random.default_rng(21)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 8000, 3, 12))
    cin, cout = 32, 64
    torch.manual_seed(4)
    conv = re_.nn.RiemannConvolution(cin, cout, kernel_size=3, dimension=3)
    conv.to(DEV)
    w = conv.kernel.detach().to(dtype).float().cpu().numpy()
    x = torch.from_numpy(rng.standard_normal((len(c), cin)).astype(np.float32)).to(dtype).float()
    gy = torch.from_numpy(rng.standard_normal((len(c), cout)).astype(np.float32)).to(dtype).float()
    y_r, oc, gx_r, gw_r = ref.conv(c, x.numpy(), w, gy=gy.numpy(), bf16=dtype == torch.bfloat16)
    np.testing.assert_array_equal(oc, c)
    feats = x.to(DEV, dtype).requires_grad_(True)
    st = re_.SparseTensor(feats, torch.from_numpy(c).to(DEV))
    y = conv(st)
    np.testing.assert_array_equal(y.C.cpu().numpy(), c)
    (y.F.float() * gy.to(DEV)).sum().backward()
    tol = TOL[dtype]
    assert_rel(y.F.detach().float().cpu().numpy(), y_r, tol, "layer Y vs reference")
    assert_rel(feats.grad.float().cpu().numpy(), gx_r, tol, "layer dX vs reference")
    assert_rel(conv.kernel.grad.float().cpu().numpy(), gw_r, tol, "layer dW vs reference")
