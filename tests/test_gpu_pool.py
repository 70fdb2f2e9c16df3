"""Pooling on the GPU through the C ABI and the host layer, against the CPU
oracle and (where oracle/_ref is built) the reference itself: stride maps
(bit-exact), local sum / average / max pooling over kernel and stride maps,
transposed pooling, global pooling, forward and backward, fp32 and bf16.
Values: rel 1e-4 (fp32) / 2e-2 (bf16), norm-wise (helpers.assert_rel); max
pooling values are compared exactly in fp32 (a max is one of its inputs)."""
import json
import os

import numpy as np
import pytest
import torch

import oracle
import riemannengine_amd as re_
from riemannengine_amd import abi
from helpers import (DEV, TOL, align, assert_rel, coord_grad, lookup, oracle_pool_layer,
                     random_coords, to_dev)

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _bf16_round(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).float().numpy()


def _check_table(km, in_to_out):
    """nbr / nbr_t of a stride map, columns by processing position (output
    out_order[p], input in_order[q]): every input in exactly one (k, out)
    slot, nbr_t (one row) each input's output, inputs ascending within an
    output."""
    nbr, nbr_t = km.nbr.cpu().numpy(), km.nbr_t.cpu().numpy()
    oo, io = km.out_order.cpu().numpy(), km.in_order.cpu().numpy()
    K, n_out = nbr.shape
    n_in = nbr_t.shape[1]
    ks, ps = np.nonzero(nbr >= 0)
    ins, os_ = nbr[ks, ps], oo[ps]
    assert len(ins) == n_in and np.array_equal(np.sort(ins), np.arange(n_in))
    np.testing.assert_array_equal(in_to_out[ins], os_)
    pos_in = np.empty(n_in, np.int64)
    pos_in[io] = np.arange(n_in)
    assert nbr_t.shape == (1, n_in)
    np.testing.assert_array_equal(nbr_t[0, pos_in[ins]], os_)
    assert (nbr_t >= 0).sum() == n_in
    counts = np.bincount(in_to_out, minlength=n_out)
    assert K == counts.max()
    for k in range(1, K):  # filled rows are a prefix of each column, ascending
        both = (nbr[k] >= 0)
        assert np.all(nbr[k - 1][both] >= 0) and np.all(nbr[k][both] > nbr[k - 1][both])


@pytest.mark.parametrize("stride", [[2, 2, 2], [4, 1, 2]])
def test_stride_map_matches_oracle(stride):
    rng = np.random.default_rng(sum(stride))
    c, _, _ = oracle.insert_and_map(random_coords(rng, 30000, 3, 40))
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(tin.ucoords, stride))
    km = abi.stride_map(tin, tout, stride)
    out = tout.ucoords.cpu().numpy()
    exp, miss = oracle.stride_map(c, out, stride)
    assert miss == 0
    _check_table(km, exp)
    ir, orr = km.in_rows.cpu().numpy(), km.out_rows.cpu().numpy()
    np.testing.assert_array_equal(exp[ir], orr)  # the single pair list
    assert km.n_pairs == len(c) and np.all(np.diff(orr) >= 0)


def test_stride_map_sorted_input_matches_oracle():
    """Input rows in coordinate order: neighbouring rows share a stride cell,
    so the lookups come in runs that one lane resolves for the whole run."""
    rng = np.random.default_rng(11)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 30000, 3, 12))
    c = c[np.lexsort(c[:, ::-1].T)]
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(tin.ucoords, [2, 2, 2]))
    km = abi.stride_map(tin, tout, [2, 2, 2])
    exp, miss = oracle.stride_map(c, tout.ucoords.cpu().numpy(), [2, 2, 2])
    assert miss == 0
    _check_table(km, exp)
    np.testing.assert_array_equal(exp[km.in_rows.cpu().numpy()], km.out_rows.cpu().numpy())


def test_stride_map_unmatched_run_counts_every_row():
    """The rows of a stride cell missing from the output map all count in
    the error, the run's followers included."""
    rng = np.random.default_rng(12)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 10))
    c = c[np.lexsort(c[:, ::-1].T)]
    sc = c.copy()
    sc[:, 1:] = np.floor_divide(c[:, 1:], 2) * 2  # each row's floor-aligned row
    cells, counts = np.unique(sc, axis=0, return_counts=True)
    drop = cells[np.argmax(counts)]
    keep = cells[np.any(cells != drop, axis=1)]
    missing = np.flatnonzero(np.all(sc == drop, axis=1))
    assert np.any(np.diff(missing) == 1)  # some missing row follows another
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(to_dev(keep))
    with pytest.raises(RuntimeError, match=f"input row {missing[0]} .*\\({len(missing)} such rows\\)"):
        abi.stride_map(tin, tout, [2, 2, 2])


def test_stride_map_unmatched_input_raises():
    """An input whose floor-aligned row is not in the output map: the host
    gets an error (the reference ASSERTs); every kernel still ends normally."""
    rng = np.random.default_rng(1)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 2000, 3, 20))
    out = oracle.stride(c, [2, 2, 2])
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(to_dev(out[1:]))
    with pytest.raises(RuntimeError, match="Invalid out_coordinate_map"):
        abi.stride_map(tin, tout, [2, 2, 2])


def _maps(kind, c):
    """GPU map + the oracle's pair list: kind 'stride' (kernel 2 == stride 2),
    'kernel' (kernel 3, stride 2) or 'compact' (the same, in pooling form)."""
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(tin.ucoords, [2, 2, 2]))
    out = tout.ucoords.cpu().numpy()
    if kind == "stride":
        km = abi.stride_map(tin, tout, [2, 2, 2])
        m, _ = oracle.stride_map(c, out, [2, 2, 2])
        return km, np.arange(len(c), dtype=np.int32), m, len(out)
    off = oracle.region_offsets(3, 3, 1, 1)
    km = abi.kernel_map(tin, tout, off)
    if kind == "compact":
        km = abi.pooling_map(km)
        assert km.nbr_t.shape[0] <= 8  # stride 2, kernel 3: at most 2 coarse rows per axis
    _, ir, orr = oracle.kernel_map(c, out, off)
    return km, ir, orr, len(out)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["sum", "avg", "max"])
@pytest.mark.parametrize("kind,C", [("stride", 32), ("kernel", 64), ("compact", 64),
                                    ("stride", 3), ("kernel", 5), ("compact", 5)])
def test_pool_matches_oracle(kind, C, mode, dtype):
    """C = 32/64: 16-byte channel slices; C = 3/5: one channel per lane."""
    rng = np.random.default_rng(C + len(mode))
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 30))
    km, ir, orr, n_out = _maps(kind, c)
    x = rng.integers(-4, 5, (len(c), C)).astype(np.float32) * 0.5  # ties for max
    xd = to_dev(x, dtype)
    y, counts = abi.pool_forward(xd, km, mode)
    oy, ocnt = oracle.pool_forward(x, ir, orr, n_out, mode)
    np.testing.assert_array_equal(counts.cpu().numpy(), ocnt)
    if mode == "max" or dtype == torch.float32 and mode == "sum":
        np.testing.assert_array_equal(_np(y), _bf16_round(oy) if dtype == torch.bfloat16 else oy)
    else:
        assert_rel(_np(y), oy, TOL[dtype], "y")
    gy = rng.standard_normal((n_out, C)).astype(np.float32)
    if dtype == torch.bfloat16:
        gy = _bf16_round(gy)
    gx = abi.pool_backward(to_dev(gy, dtype), y, xd, km, counts, mode)
    ogx = oracle.pool_backward(x, _np(y), gy, ir, orr, mode)
    assert_rel(_np(gx), ogx, TOL[dtype], "dX")


def test_table_compact():
    rng = np.random.default_rng(12)
    t = np.where(rng.random((27, 5000)) < 0.2, rng.integers(0, 900, (27, 5000)), -1)
    t[:, 7] = -1  # an empty column
    got = abi.table_compact(to_dev(t.astype(np.int32))).cpu().numpy()
    counts = (t >= 0).sum(0)
    assert got.shape == (counts.max(), 5000)
    for q in range(5000):
        col = t[:, q][t[:, q] >= 0]
        np.testing.assert_array_equal(got[:len(col), q], col)
        assert np.all(got[len(col):, q] == -1)


def test_pool_empty_outputs_and_nan():
    """Outputs with no input row are 0 in every mode; a NaN input makes its
    output's max NaN (torch amax)."""
    rng = np.random.default_rng(8)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 3000, 3, 20))
    tin = abi.hash_build(to_dev(c))
    extra = np.array([[0, 1000, 1000, 1000], [1, -999, 5, 5]], np.int32)
    out = np.concatenate([oracle.stride(c, [2, 2, 2]), extra])
    tout = abi.hash_build(to_dev(out))
    off = oracle.region_offsets(3, 3, 1, 1)
    km = abi.kernel_map(tin, tout, off)
    x = rng.standard_normal((len(c), 8)).astype(np.float32)
    x[5, 3] = np.nan
    for mode in ("sum", "avg", "max"):
        y, counts = abi.pool_forward(to_dev(x), km, mode)
        yn = _np(y)
        assert np.all(yn[-2:] == 0) and np.all(counts.cpu().numpy()[-2:] == 0)
        q = int(np.nonzero(km.in_order.cpu().numpy() == 5)[0][0])
        rows = km.nbr_t.cpu().numpy()[:, q]
        assert np.all(np.isnan(yn[rows[rows >= 0], 3]))


def test_pool_empty_input_map():
    tin = abi.hash_build(to_dev(np.zeros((0, 4), np.int32)))
    tout = abi.hash_build(to_dev(np.array([[0, 0, 0, 0]], np.int32)))
    km = abi.kernel_map(tin, tout, oracle.region_offsets(3, 3, 1, 1))
    y, _ = abi.pool_forward(torch.zeros((0, 4), device=DEV), km, "max")
    assert y.shape == (1, 4) and float(y.abs().sum()) == 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["sum", "avg", "max"])
@pytest.mark.parametrize("C", [64, 7])
def test_global_pool_matches_oracle(mode, dtype, C):
    rng = np.random.default_rng(C * 3 + len(mode))
    c = random_coords(rng, 50000, 3, 40, batch=6)
    c[c[:, 0] == 3, 0] = 4  # batch 3 is empty
    c[:7, 0] = -1           # rows of no batch
    x = rng.integers(-5, 6, (len(c), C)).astype(np.float32) * 0.25
    xd = to_dev(x, dtype)
    cd = to_dev(c)
    segs = abi.batch_segments(cd)
    assert segs.n_batches == 6
    seg = segs.seg.cpu().numpy()
    b = c[:, 0]
    np.testing.assert_array_equal(np.diff(seg), np.bincount(b[b >= 0], minlength=6))
    mem = segs.members.cpu().numpy()
    for k in range(6):
        np.testing.assert_array_equal(mem[seg[k]:seg[k + 1]], np.nonzero(b == k)[0])
    y = abi.global_pool_forward(xd, segs, mode)
    oy = oracle.global_pool_forward(x, c, mode)
    if mode == "max":
        np.testing.assert_array_equal(_np(y), oy)
    else:
        assert_rel(_np(y), oy, TOL[dtype] if dtype == torch.bfloat16 else 1e-5, "y")
    gy = _bf16_round(rng.standard_normal((6, C)).astype(np.float32))
    gx = abi.global_pool_backward(to_dev(gy, dtype), y, xd, cd, segs, mode)
    assert_rel(_np(gx), oracle.global_pool_backward(x, _np(y), gy, c, mode), TOL[dtype], "dX")


# ------------------------------------------------------------ host layer

def _golden():
    here = os.path.dirname(os.path.abspath(__file__))
    with open(os.path.join(here, "golden", "kat_layers_pooling.json")) as f:
        return json.load(f)


def test_layer_known_answers():
    """tests/engine/test_layers.cpp:58-115 through the host layers on the GPU."""
    d = _golden()
    s = d["strided"]["input"]
    x = re_.SparseTensor(torch.tensor(s["features"], device=DEV),
                         torch.tensor(s["coords"], dtype=torch.int32, device=DEV))
    layers = {"avg": re_.nn.RiemannAvgPooling(2, 2), "max": re_.nn.RiemannMaxPooling(2, 2),
              "sum": re_.nn.RiemannSumPooling(2, 2)}
    for kat in d["strided"]["kats"]:
        y = layers[kat["mode"]](x)
        assert len(y) == s["out_rows"] and y.tensor_stride == s["out_tensor_stride"]
        rows = {tuple(r[1:]): i for i, r in enumerate(y.C.cpu().tolist())}
        got = float(y.F[rows[tuple(kat["coordinate"])], 0])
        assert abs(got - kat["expected"]) <= d["tolerance_abs"], kat
    g = d["global"]["input"]
    x = re_.SparseTensor(torch.tensor(g["features"], device=DEV),
                         torch.tensor(g["coords"], dtype=torch.int32, device=DEV))
    glob = {"avg": re_.nn.RiemannGlobalAvgPooling(), "max": re_.nn.RiemannGlobalMaxPooling(),
            "sum": re_.nn.RiemannGlobalSumPooling()}
    for kat in d["global"]["kats"]:
        y = glob[kat["mode"]](x)
        rows = {r[0]: i for i, r in enumerate(y.C.cpu().tolist())}
        np.testing.assert_allclose(_np(y.F)[rows[kat["batch"]]], kat["expected"],
                                   atol=d["tolerance_abs"])


@pytest.mark.parametrize("mode", ["sum", "avg", "max"])
@pytest.mark.parametrize("ks,stride,transpose,expand", [
    (2, 2, False, False), (3, 2, False, False), (3, 1, False, False),
    (2, 2, True, False), (3, 2, True, False), (2, 2, True, True)])
def test_layer_matches_oracle_and_reference(mode, ks, stride, transpose, expand):
    """Layers on the GPU vs the oracle's restatement of the reference's layer
    and, where built, the reference layer itself (fp32)."""
    from oracle import ref
    rng = np.random.default_rng(ks * 7 + stride + 3 * transpose)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 6000, 3, 16))
    in_stride = 1
    mgr = re_.CoordinateManager(3)
    if transpose:
        c, in_stride = oracle.stride(c, [2, 2, 2]), 2
    key, _ = mgr.insert_and_map(to_dev(c), [in_stride] * 3)
    x = rng.integers(-4, 5, (len(c), 6)).astype(np.float32)
    xf = to_dev(x).requires_grad_(True)
    inp = re_.SparseTensor(xf, key, mgr)
    PM = re_.PoolingMode
    pm = {"sum": PM.LOCAL_SUM_POOLING, "avg": PM.LOCAL_AVG_POOLING, "max": PM.LOCAL_MAX_POOLING}
    if transpose:
        layer = re_.nn.RiemannPoolingTranspose(ks, stride, 1, expand, 3, pm[mode])
    else:
        layer = {"sum": re_.nn.RiemannSumPooling, "avg": re_.nn.RiemannAvgPooling,
                 "max": re_.nn.RiemannMaxPooling}[mode](ks, stride)
    y = layer(inp)
    oc = y.C.cpu().numpy()
    assert y.tensor_stride == [in_stride // stride if transpose else in_stride * stride] * 3
    (y.F * to_dev(coord_grad(oc, 6))).sum().backward()
    gy = lambda o: coord_grad(o, 6)  # noqa: E731
    out, oy, ogx = oracle_pool_layer(c, x, mode, ks, stride, in_stride=in_stride,
                                     transpose=transpose, expand=expand, gy=gy)
    p = align(oc, out)
    assert_rel(_np(y.F), oy[p], 1e-5, "y")
    assert_rel(_np(xf.grad), ogx, 1e-5, "dX")
    if ref.available():
        ry, roc, rgx = ref.pool(c, x, mode, ks, stride, in_stride=in_stride,
                                transpose=transpose, expand=expand, gy=gy)
        q = align(roc, oc)
        assert_rel(_np(y.F)[q], ry, 1e-5, "y vs reference")
        assert_rel(_np(xf.grad), rgx, 1e-5, "dX vs reference")


@pytest.mark.parametrize("mode", ["sum", "avg", "max"])
def test_global_layer_matches_reference(mode):
    from oracle import ref
    rng = np.random.default_rng(30 + len(mode))
    c, _, _ = oracle.insert_and_map(random_coords(rng, 8000, 3, 20, batch=3))
    x = rng.standard_normal((len(c), 16)).astype(np.float32)
    xf = to_dev(x).requires_grad_(True)
    PM = re_.PoolingMode
    pm = {"sum": PM.GLOBAL_SUM_POOLING_PYTORCH_INDEX, "avg": PM.GLOBAL_AVG_POOLING_PYTORCH_INDEX,
          "max": PM.GLOBAL_MAX_POOLING_PYTORCH_INDEX}[mode]
    y = re_.nn.RiemannGlobalPooling(pm)(re_.SparseTensor(xf, to_dev(c)))
    assert y.C.cpu().tolist() == [[b, 0, 0, 0] for b in range(3)]
    gy = rng.standard_normal((3, 16)).astype(np.float32)
    (y.F * to_dev(gy)).sum().backward()
    oy = oracle.global_pool_forward(x, c, mode)
    assert_rel(_np(y.F), oy, 1e-5, "y")
    assert_rel(_np(xf.grad), oracle.global_pool_backward(x, oy, gy, c, mode), 1e-5, "dX")
    if ref.available():
        ry, _, rgx = ref.global_pool(c, x, mode, gy=gy)
        assert_rel(_np(y.F), ry, 1e-5, "y vs reference")
        assert_rel(_np(xf.grad), rgx, 1e-5, "dX vs reference")


def test_layer_bf16_matches_reference():
    from oracle import ref
    rng = np.random.default_rng(40)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 6000, 3, 16))
    x = _bf16_round(rng.standard_normal((len(c), 16)).astype(np.float32))
    for mode, layer in (("avg", re_.nn.RiemannAvgPooling(3, 2)),
                        ("max", re_.nn.RiemannMaxPooling(2, 2))):
        y = layer(re_.SparseTensor(to_dev(x, torch.bfloat16), to_dev(c)))
        assert y.F.dtype == torch.bfloat16
        oc = y.C.cpu().numpy()
        ks, st = (3, 2) if mode == "avg" else (2, 2)
        out, oy, _ = oracle_pool_layer(c, x, mode, ks, st)
        assert_rel(_np(y.F), oy[align(oc, out)], 2e-2, mode)
        if ref.available():
            ry, roc, _ = ref.pool(c, x, mode, ks, st, bf16=True)
            assert_rel(_np(y.F)[align(roc, oc)], ry, 2e-2, mode + " vs reference")


def test_pool_down_up_full_size_properties():
    """BASELINE config-2-sized cloud (C = 64): stride-map sum pooling
    conserves the channel sums; average x counts = sum; max dominates every
    member; transposed sum pooling of the pooled tensor returns each input's
    group total (a pooling -> unpooling round trip)."""
    rng = np.random.default_rng(77)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 250000, 3, 120, batch=2))
    x = torch.randn(len(c), 64, device=DEV)
    inp = re_.SparseTensor(x, to_dev(c))
    s = re_.nn.RiemannSumPooling(2, 2)(inp)
    torch.testing.assert_close(s.F.sum(0), x.sum(0), rtol=1e-4, atol=1e-2)
    a = re_.nn.RiemannAvgPooling(2, 2)(inp)
    cnt = re_.nn.RiemannSumPooling(2, 2)(re_.SparseTensor(torch.ones(len(c), 1, device=DEV),
                                                          to_dev(c)))
    torch.testing.assert_close(a.F * cnt.F, s.F, rtol=1e-5, atol=1e-4)
    m = re_.nn.RiemannMaxPooling(2, 2)(inp)
    up = re_.nn.RiemannPoolingTranspose(2, 2)(re_.SparseTensor(m.F, m.coordinate_map_key,
                                                               m.coordinate_manager))
    # every input row sits in a 2^3 cell whose generated children include it
    fine = up.C.cpu().numpy()
    assert len(fine) == 8 * len(m)
    pos = lookup(fine, c)
    assert bool((up.F[to_dev(pos)] >= x).all())
    us = re_.nn.RiemannPoolingTranspose(2, 2)(re_.SparseTensor(s.F, s.coordinate_map_key,
                                                               s.coordinate_manager))
    # unpooling the sums back onto the input rows: each row gets its cell total
    np.testing.assert_array_equal(us.C.cpu().numpy(), fine)
    parent = np.concatenate([c[:, :1], np.floor_divide(c[:, 1:], 2) * 2], 1)
    sc = _np(s.F)[lookup(s.C.cpu().numpy(), parent)]
    np.testing.assert_allclose(_np(us.F)[pos], sc, rtol=1e-6, atol=1e-6)


# ------------------------------------------------------ quantization

def test_group_map_matches_oracle():
    rng = np.random.default_rng(60)
    c = random_coords(rng, 40000, 3, 10)  # heavy duplication
    uq, _, inv = oracle.insert_and_map(c)
    km = abi.group_map(to_dev(inv.astype(np.int32)), len(uq))
    _check_table(km, inv.astype(np.int64))
    with pytest.raises(RuntimeError, match="outside"):
        abi.group_map(to_dev(np.array([0, 3, 1], np.int32)), 2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["avg", "sum", "max"])
def test_quantization_matches_oracle_and_reference(mode, dtype):
    """SparseTensor(features, coords, quantization_mode) reduces duplicate
    rows through the group map + pooling kernels: values and gradients vs
    the oracle (pooling over rows -> inverse; max with scatter_reduce's zero
    tie) and the reference's own constructor; deterministic."""
    from oracle import ref
    rng = np.random.default_rng(70 + len(mode))
    c = random_coords(rng, 30000, 3, 12)
    x = rng.integers(-3, 3, (len(c), 8)).astype(np.float32)  # maxima at 0 and ties
    Q = re_.QuantizationMode
    q = {"avg": Q.UNWEIGHTED_AVERAGE, "sum": Q.UNWEIGHTED_SUM, "max": Q.MAX_POOL}[mode]
    xf = to_dev(x, dtype).requires_grad_(True)
    t = re_.SparseTensor(xf, to_dev(c), quantization_mode=q)
    uq, _, inv = oracle.insert_and_map(c)
    np.testing.assert_array_equal(t.C.cpu().numpy(), uq)
    gy = coord_grad(uq, 8)
    if dtype == torch.bfloat16:
        gy = _bf16_round(gy)
    (t.F * to_dev(gy, dtype)).sum().backward()
    om = "max_scatter" if mode == "max" else mode
    rows = np.arange(len(c), dtype=np.int32)
    oy, _ = oracle.pool_forward(x, rows, inv.astype(np.int32), len(uq), om)
    assert_rel(_np(t.F), oy, TOL[dtype], "y")
    assert_rel(_np(xf.grad), oracle.pool_backward(x, oy, gy, rows, inv.astype(np.int32), om),
               TOL[dtype], "dX")
    again = re_.SparseTensor(xf.detach(), to_dev(c), quantization_mode=q)
    assert torch.equal(again.F, t.F.detach())
    if ref.available() and dtype == torch.float32:
        ry, roc, rgx = ref.quantize(c, x, mode, gy=lambda o: coord_grad(o, 8))
        p = align(roc, uq)
        assert_rel(_np(t.F)[p], ry, 1e-5, "y vs reference")
        assert_rel(_np(xf.grad), rgx, 1e-5, "dX vs reference")


def test_sparse_tensor_to_device_rehashes():
    rng = np.random.default_rng(80)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 5000, 3, 15))
    x = torch.randn(len(c), 4, device=DEV)
    t = re_.SparseTensor(x, to_dev(c))
    m = t.to(DEV)
    assert m.coordinate_manager is not t.coordinate_manager
    np.testing.assert_array_equal(m.C.cpu().numpy(), t.C.cpu().numpy())
    assert torch.equal(m.F, t.F)
    with pytest.raises(RuntimeError, match="no CPU manager"):
        t.to(torch.device("cpu"))
