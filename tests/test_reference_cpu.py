"""The oracle against the reference itself (its CPU path compiled from source
into oracle/_ref by oracle/ref.mk): dedup, kernel maps, strided output
coordinates and convolution forward/backward, including the reference's own
bf16 arithmetic. Skipped where the reference library was not built."""
import numpy as np
import pytest

import oracle
from oracle import ref
from helpers import random_coords

pytestmark = pytest.mark.skipif(not ref.available(),
                                reason="oracle/_ref not built (no reference checkout)")


def _coord_index(rows):
    return {tuple(r): i for i, r in enumerate(rows.tolist())}


def _canonical_by_coords(kofs, ir, orr, in_coords, out_coords):
    """(k, input coordinate, output coordinate) triplets, sorted: independent
    of either side's row order."""
    ks = np.repeat(np.arange(len(kofs) - 1), np.diff(kofs))
    t = np.concatenate([ks[:, None], in_coords[ir], out_coords[orr]], 1)
    return t[np.lexsort(t.T[::-1])]


def test_insert_and_map_matches_reference():
    rng = np.random.default_rng(0)
    c = random_coords(rng, 4000, 3, 6)  # many duplicates
    u, m, inv = ref.insert_and_map(c)
    ou, om, oinv = oracle.insert_and_map(c)
    np.testing.assert_array_equal(u, ou)
    np.testing.assert_array_equal(m, om)
    np.testing.assert_array_equal(inv, oinv)


@pytest.mark.parametrize("D,ks,stride,dil,region", [
    (3, 3, 1, 1, "cube"), (3, 3, 1, 2, "cube"), (3, 3, 1, 1, "cross"), (3, 2, 2, 1, "cube"),
    (3, 3, 2, 1, "cube"), (4, 3, 1, 1, "cube"), (2, 5, 1, 1, "cube"), (3, 2, 1, 1, "cube")])
def test_kernel_map_matches_reference(D, ks, stride, dil, region):
    rng = np.random.default_rng(D * 10 + ks + stride)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 3000, D, 10))
    kofs, ir, orr, oc = ref.kernel_map(c, ks, stride, dil, region)
    # the strided output set is floor(x/s)*s; its row order in the reference
    # is an implementation detail of its hash map
    ocs = c if stride == 1 else oracle.stride(c, [stride] * D)
    assert sorted(map(tuple, oc.tolist())) == sorted(map(tuple, ocs.tolist()))
    off = oracle.region_offsets(D, ks, dil, 1, region)
    okofs, oir, oorr = oracle.kernel_map(c, ocs, off)
    np.testing.assert_array_equal(np.diff(kofs), np.diff(okofs))
    np.testing.assert_array_equal(_canonical_by_coords(kofs, ir, orr, c, oc),
                                  _canonical_by_coords(okofs, oir, oorr, c, ocs))


def _oracle_conv_on(c, oc, x, w, gy, D, ks, stride, dil=1):
    off = oracle.region_offsets(D, ks, dil, 1)
    kofs, ir, orr = oracle.kernel_map(c, oc, off)
    y = oracle.conv_forward(x, w, kofs, ir, orr, len(oc))
    gx, gw = oracle.conv_backward(x, gy, w, kofs, ir, orr)
    return y, gx, gw


@pytest.mark.parametrize("D,ks,stride,cin,cout", [
    (3, 3, 1, 16, 32), (3, 2, 2, 8, 16), (4, 3, 1, 8, 8), (3, 3, 2, 4, 12)])
def test_conv_fp32_matches_reference(D, ks, stride, cin, cout):
    rng = np.random.default_rng(ks * 7 + stride + D)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 2500, D, 9))
    K = ks ** D
    x = rng.standard_normal((len(c), cin)).astype(np.float32)
    w = (rng.standard_normal((K, cin, cout)) / np.sqrt(cin * K)).astype(np.float32)
    gy_of = lambda oc: np.random.default_rng(5).standard_normal((len(oc), cout)).astype(np.float32)
    y, oc, gx, gw = ref.conv(c, x, w, gy=gy_of, ks=ks, stride=stride)
    ry, rgx, rgw = _oracle_conv_on(c, oc, x, w, gy_of(oc), D, ks, stride)
    for got, exp in ((y, ry), (gx, rgx), (gw, rgw)):
        assert np.abs(got - exp).max() <= 1e-5 * np.abs(exp).max()


def test_reference_bf16_is_within_the_bf16_bar():
    """The reference computes bf16 convolutions in bf16 (matmul, then
    index_add_ per offset, conv.cpp:59-61). Its distance to the fp32 result
    on the same bf16 operands is what the 2e-2 bf16 bar has to cover."""
    import torch
    rng = np.random.default_rng(3)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 3000, 3, 9))
    cin = cout = 64
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    x = bf(rng.standard_normal((len(c), cin)).astype(np.float32))
    w = bf((rng.standard_normal((27, cin, cout)) / np.sqrt(cin * 27)).astype(np.float32))
    gy = bf(rng.standard_normal((len(c), cout)).astype(np.float32))
    y, oc, gx, gw = ref.conv(c, x, w, gy=gy, bf16=True)
    np.testing.assert_array_equal(oc, c)
    ry, rgx, rgw = _oracle_conv_on(c, c, x, w, gy, 3, 3, 1)
    errs = [np.abs(g - e).max() / np.abs(e).max() for g, e in ((y, ry), (gx, rgx), (gw, rgw))]
    assert max(errs) <= 2e-2, errs
    assert max(errs) > 1e-4  # it really is bf16 arithmetic


# ---------------------------------------------------------------- pooling

from helpers import oracle_pool_layer, coord_grad, align  # noqa: E402


@pytest.mark.parametrize("mode", ["sum", "avg", "max"])
@pytest.mark.parametrize("ks,stride,transpose,expand", [
    (2, 2, False, False), (3, 2, False, False), (3, 1, False, False),
    (2, 2, True, False), (3, 2, True, False), (2, 2, True, True)])
def test_pool_layer_matches_reference(mode, ks, stride, transpose, expand):
    """The reference's pooling layers (stride map when kernel == stride, else
    the kernel map; transposed: generated finer map, swapped map) against the
    oracle: same output coordinates, values and input gradients (fp32)."""
    rng = np.random.default_rng(ks * 7 + stride + 3 * transpose)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 1500, 3, 12))
    in_stride = 1
    if transpose:
        c, in_stride = oracle.stride(c, [2, 2, 2]), 2
    x = rng.integers(-4, 5, (len(c), 3)).astype(np.float32)  # ties for max
    gy = lambda oc: coord_grad(oc, 3)  # noqa: E731
    y, oc, gx = ref.pool(c, x, mode, ks, stride, in_stride=in_stride, transpose=transpose,
                         expand=expand, gy=gy)
    out, oy, ogx = oracle_pool_layer(c, x, mode, ks, stride, in_stride=in_stride,
                                     transpose=transpose, expand=expand, gy=gy)
    p = align(oc, out)
    np.testing.assert_allclose(y, oy[p], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(gx, ogx, rtol=1e-5, atol=1e-5)


def test_pool_layer_bf16_matches_reference_within_tolerance():
    """The reference computes bf16 pooling in bf16 tensors; the oracle in
    fp32 on the same (bf16-representable) inputs: within the bf16 bound."""
    rng = np.random.default_rng(9)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 1500, 3, 12))
    x = rng.standard_normal((len(c), 4)).astype(np.float32)
    x = np.asarray(torch_bf16_round(x), np.float32)
    for mode in ("sum", "avg", "max"):
        y, oc, _ = ref.pool(c, x, mode, 3, 2, bf16=True)
        out, oy, _ = oracle_pool_layer(c, x, mode, 3, 2)
        p = align(oc, out)
        scale = np.abs(oy).max()
        assert np.abs(y - oy[p]).max() <= 2e-2 * scale, mode


def torch_bf16_round(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).float().numpy()


def test_transposed_odd_stride_map_raises_like_reference():
    """Kernel 3 == stride 3 transposed: the generated rows c - 1 floor onto a
    coarse row that may not exist; the reference ASSERTs, the oracle counts
    the misses."""
    rng = np.random.default_rng(4)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 500, 3, 12))
    coarse = oracle.stride(c, [3, 3, 3])
    with pytest.raises(RuntimeError, match="Invalid out_coordinate_map"):
        ref.pool(coarse, np.ones((len(coarse), 1), np.float32), "sum", 3, 3, in_stride=3,
                 transpose=True)
    fine = oracle.stride_region(coarse, oracle.region_offsets(3, 3, 1, 1))
    _, miss = oracle.stride_map(fine, coarse, [3, 3, 3])
    assert miss > 0


@pytest.mark.parametrize("mode", ["sum", "avg", "max"])
def test_global_pool_matches_reference(mode):
    rng = np.random.default_rng(21)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 900, 3, 10, batch=4))
    c = c[c[:, 0] != 2]  # an empty batch
    x = rng.integers(-3, 4, (len(c), 5)).astype(np.float32)
    gy = rng.standard_normal((4, 5)).astype(np.float32)
    y, oc, gx = ref.global_pool(c, x, mode, gy=gy)
    assert oc.tolist() == [[b, 0, 0, 0] for b in range(4)]
    oy = oracle.global_pool_forward(x, c, mode)
    np.testing.assert_allclose(y, oy, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gx, oracle.global_pool_backward(x, oy, gy, c, mode),
                               rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("mode", ["avg", "sum", "max"])
def test_quantization_matches_reference(mode):
    """SparseTensor quantization (reduce feature rows by their unique
    coordinate) = local pooling over the group map rows -> inverse map:
    the oracle's pooling on (arange, inverse) against the reference's
    SparseTensor constructor, values and gradients."""
    rng = np.random.default_rng(50 + len(mode))
    c = random_coords(rng, 3000, 3, 6)  # many duplicates
    x = rng.integers(-3, 4, (len(c), 4)).astype(np.float32)
    gy = lambda oc: coord_grad(oc, 4)  # noqa: E731
    y, oc, gx = ref.quantize(c, x, mode, gy=gy)
    uq, _, inv = oracle.insert_and_map(c)
    p = align(oc, uq)
    rows = np.arange(len(c), dtype=np.int32)
    om = "max_scatter" if mode == "max" else mode  # scatter_reduce's gradient
    oy, _ = oracle.pool_forward(x, rows, inv.astype(np.int32), len(uq), om)
    np.testing.assert_allclose(y, oy[p], rtol=1e-5, atol=1e-5)
    ogx = oracle.pool_backward(x, oy, gy(uq), rows, inv.astype(np.int32), om)
    np.testing.assert_allclose(gx, ogx, rtol=1e-5, atol=1e-5)
