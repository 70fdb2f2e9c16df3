"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something that does not restate it:
the reference's own known-answer tests (golden fixture), brute force, closed
forms, or a textbook routine (dense torch conv3d on a voxelised grid).
Runs on the CPU only.
"""
import json
import os
from itertools import product

import numpy as np
import pytest
import torch

import oracle

TOL_F32 = 1e-5  # the reference KATs use CHECK_NEAR(..., 1e-5)


def _kats(golden_dir):
    with open(os.path.join(golden_dir, "kat_cpu_convolution.json")) as f:
        return json.load(f)["kats"]


def _csr(maps_in, maps_out):
    kofs = np.concatenate([[0], np.cumsum([len(m) for m in maps_in])]).astype(np.int64)
    return kofs, np.concatenate(maps_in).astype(np.int32), np.concatenate(maps_out).astype(np.int32)


def test_kats_from_reference(golden_dir):
    """tests/convolution/test_cpu_convolution.cpp:15-61 through the oracle."""
    for kat in _kats(golden_dir):
        kofs, ir, orr = _csr(kat["in_maps"], kat["out_maps"])
        x = np.array(kat["x"], np.float32).reshape(kat["n_in"], kat["cin"])
        w = np.array(kat["weight"], np.float32).reshape(len(kat["in_maps"]), kat["cin"], kat["cout"])
        if kat["kind"] == "forward":
            y = oracle.conv_forward(x, w, kofs, ir, orr, kat["n_out"])
            np.testing.assert_allclose(y.ravel(), kat["expected_y"], atol=TOL_F32, rtol=0)
        else:
            gy = np.array(kat["grad_y"], np.float32).reshape(kat["n_out"], kat["cout"])
            gx, gw = oracle.conv_backward(x, gy, w, kofs, ir, orr)
            np.testing.assert_allclose(gx.ravel(), kat["expected_grad_x"], atol=TOL_F32, rtol=0)
            np.testing.assert_allclose(gw.ravel(), kat["expected_grad_w"], atol=TOL_F32, rtol=0)


def test_kat_out_of_range_rows_are_skipped():
    """convolution_cpu.hpp:41-43: pairs with rows outside the tensors are ignored."""
    x = np.ones((2, 1), np.float32)
    w = np.ones((1, 1, 1), np.float32)
    y = oracle.conv_forward(x, w, np.array([0, 2]), np.array([0, 5]), np.array([1, 1]), 2)
    np.testing.assert_array_equal(y.ravel(), [0, 1])


def _first_occurrence_unique(c):
    _, idx, inv = np.unique(c, axis=0, return_index=True, return_inverse=True)
    order = np.argsort(idx, kind="stable")
    rank = np.empty_like(order)
    rank[order] = np.arange(order.size)
    return c[idx[order]], idx[order], rank[inv.ravel()]


@pytest.mark.parametrize("ncol,span,n", [(4, 6, 2000), (5, 4, 3000), (4, 1000, 500), (2, 3, 50)])
def test_insert_and_map_brute_force(ncol, span, n):
    rng = np.random.default_rng(ncol * 1000 + n)
    c = rng.integers(-span, span, (n, ncol)).astype(np.int32)
    uq, mp, inv = oracle.insert_and_map(c)
    buq, bmp, binv = _first_occurrence_unique(c)
    np.testing.assert_array_equal(uq, buq)
    np.testing.assert_array_equal(mp, bmp)
    np.testing.assert_array_equal(inv, binv)
    np.testing.assert_array_equal(uq[inv], c)  # lattice_cpu.hpp:413-417 invariant
    np.testing.assert_array_equal(c[mp], uq)


def test_insert_and_map_empty():
    uq, mp, inv = oracle.insert_and_map(np.zeros((0, 4), np.int32))
    assert uq.shape == (0, 4) and mp.size == 0 and inv.size == 0


def test_region_offsets_closed_forms():
    # 3^3: k = (dx+1) + 3(dy+1) + 9(dz+1), axis 0 (x) fastest (stencil.hpp:232-247)
    off = oracle.region_offsets(3, 3)
    exp = np.array([(dx, dy, dz) for dz in (-1, 0, 1) for dy in (-1, 0, 1) for dx in (-1, 0, 1)])
    np.testing.assert_array_equal(off, exp)
    # even size: non-negative offsets, k = dx + 2dy + 4dz
    off = oracle.region_offsets(3, 2)
    exp = np.array([(dx, dy, dz) for dz in (0, 1) for dy in (0, 1) for dx in (0, 1)])
    np.testing.assert_array_equal(off, exp)
    # 3^4 with t slowest; scaled by dilation * tensor stride
    off = oracle.region_offsets(4, 3, dilation=2, tensor_stride=[1, 2, 1, 4])
    exp = np.array([(2 * dx, 4 * dy, 2 * dz, 8 * dt) for dt in (-1, 0, 1) for dz in (-1, 0, 1)
                    for dy in (-1, 0, 1) for dx in (-1, 0, 1)])
    np.testing.assert_array_equal(off, exp)
    # cross: centre, then +a, -a per axis (stencil.hpp:250-268)
    off = oracle.region_offsets(3, 3, region="cross")
    exp = np.array([(0, 0, 0), (1, 0, 0), (-1, 0, 0), (0, 1, 0), (0, -1, 0), (0, 0, 1), (0, 0, -1)])
    np.testing.assert_array_equal(off, exp)
    off = oracle.region_offsets(2, [5, 3], region="cross")
    exp = np.array([(0, 0), (1, 0), (2, 0), (-2, 0), (-1, 0), (0, 1), (0, -1)])
    np.testing.assert_array_equal(off, exp)
    cust = np.array([[1, 0, 0], [0, -2, 3]])
    off = oracle.region_offsets(3, 3, dilation=2, tensor_stride=[1, 1, 3], region="custom", custom=cust)
    np.testing.assert_array_equal(off, cust * np.array([2, 2, 6]))


def _brute_kernel_map(cin, cout, off):
    """Dictionary join, independent of the oracle's hashing."""
    where = {tuple(r): i for i, r in enumerate(cin.tolist())}
    trip = []
    for k, o in product(range(off.shape[0]), range(cout.shape[0])):
        q = cout[o].copy()
        q[1:] += off[k]
        i = where.get(tuple(q.tolist()))
        if i is not None:
            trip.append((k, o, i))
    return np.array(sorted(trip), np.int64).reshape(-1, 3)


@pytest.mark.parametrize("D,ks,dil,ts,region", [
    (3, 3, 1, 1, "cube"), (3, 2, 1, 1, "cube"), (3, 3, 2, 1, "cube"),
    (3, 3, 1, 2, "cube"), (4, 3, 1, 1, "cube"), (3, 3, 1, 1, "cross"), (2, 5, 1, 1, "cube")])
def test_kernel_map_brute_force(D, ks, dil, ts, region):
    rng = np.random.default_rng(7 + D * 10 + ks)
    n = 400
    c = np.concatenate([rng.integers(0, 2, (n, 1)), rng.integers(-4, 5, (n, D)) * ts], 1).astype(np.int32)
    c, _, _ = oracle.insert_and_map(c)
    off = oracle.region_offsets(D, ks, dil, ts, region)
    kofs, ir, orr = oracle.kernel_map(c, c, off)
    got = oracle.canonical_pairs(kofs, ir, orr)
    np.testing.assert_array_equal(got, _brute_kernel_map(c, c, off))
    # buckets come out ordered by output row
    for k in range(off.shape[0]):
        assert np.all(np.diff(orr[kofs[k]:kofs[k + 1]]) > 0)


def test_kernel_map_against_dense_indicator():
    """Pair count per offset = sum over the grid of active(x) * active(x + off)."""
    rng = np.random.default_rng(3)
    g = rng.random((12, 12, 12)) < 0.3
    pts = np.argwhere(g)
    c = np.concatenate([np.zeros((len(pts), 1), int), pts], 1).astype(np.int32)
    off = oracle.region_offsets(3, 3)
    kofs, _, _ = oracle.kernel_map(c, c, off)
    pad = np.pad(g, 1)
    for k, (dx, dy, dz) in enumerate(off):
        shifted = pad[1 + dx:13 + dx, 1 + dy:13 + dy, 1 + dz:13 + dz]
        assert kofs[k + 1] - kofs[k] == int((g & shifted).sum())


def test_kernel_map_empty_sides():
    off = oracle.region_offsets(3, 3)
    e = np.zeros((0, 4), np.int32)
    c = np.array([[0, 1, 2, 3]], np.int32)
    for a, b in ((e, c), (c, e), (e, e)):
        kofs, ir, orr = oracle.kernel_map(a, b, off)
        assert kofs[-1] == 0 and ir.size == 0


@pytest.mark.parametrize("s", [[2, 2, 2], [4, 4, 4], [2, 3, 1]])
def test_stride_closed_form(s):
    rng = np.random.default_rng(sum(s))
    c = np.concatenate([rng.integers(0, 3, (1000, 1)), rng.integers(-50, 50, (1000, 3))], 1).astype(np.int32)
    got = oracle.stride(c, s)
    exp = c.copy()
    exp[:, 1:] = np.floor_divide(c[:, 1:], s) * np.array(s)
    exp, _, _ = _first_occurrence_unique(exp)
    np.testing.assert_array_equal(got, exp)


def _dense_conv3d_check(ks, stride, dil, seed):
    """Sparse conv (oracle) == dense conv3d evaluated at active sites, for the
    forward and both gradients (torch autograd on the dense conv, fp64)."""
    rng = np.random.default_rng(seed)
    S = 10
    g = rng.random((S, S, S)) < 0.25
    pts = np.argwhere(g)  # (x, y, z)
    c = np.concatenate([np.zeros((len(pts), 1), int), pts], 1).astype(np.int32)
    n, cin, cout = len(pts), 3, 4
    x = rng.standard_normal((n, cin)).astype(np.float32)
    D = 3
    K = ks ** 3
    w = rng.standard_normal((K, cin, cout)).astype(np.float32)
    if stride == 1:
        cout_coords = c
        off = oracle.region_offsets(D, ks, dil, 1)
    else:
        cout_coords = oracle.stride(c, [stride] * 3)
        off = oracle.region_offsets(D, ks, dil, 1)
    kofs, ir, orr = oracle.kernel_map(c, cout_coords, off)
    y = oracle.conv_forward(x, w, kofs, ir, orr, len(cout_coords))
    gy = rng.standard_normal(y.shape).astype(np.float32)
    gx, gw = oracle.conv_backward(x, gy, w, kofs, ir, orr)

    # dense: layout [1, C, X, Y, Z]; torch cross-correlation
    xd = torch.zeros((1, cin, S, S, S), dtype=torch.float64)
    xd[0, :, pts[:, 0], pts[:, 1], pts[:, 2]] = torch.from_numpy(x.T.astype(np.float64))
    xd.requires_grad_(True)
    wd = torch.zeros((cout, cin, ks, ks, ks), dtype=torch.float64)
    for k, (dx, dy, dz) in enumerate(off // dil if dil > 1 else off):
        a, b, cc = (dx + ks // 2, dy + ks // 2, dz + ks // 2) if ks % 2 else (dx, dy, dz)
        wd[:, :, a, b, cc] = torch.from_numpy(w[k].T.astype(np.float64))
    wd.requires_grad_(True)
    pad = (ks // 2) * dil if ks % 2 else 0
    yd = torch.nn.functional.conv3d(xd, wd, stride=stride, padding=pad, dilation=dil)
    oc = cout_coords[:, 1:] // stride
    ysel = yd[0, :, oc[:, 0], oc[:, 1], oc[:, 2]].T
    np.testing.assert_allclose(y, ysel.detach().numpy(), rtol=1e-5, atol=1e-5)
    (ysel * torch.from_numpy(gy.astype(np.float64))).sum().backward()
    gxd = xd.grad[0, :, pts[:, 0], pts[:, 1], pts[:, 2]].T.numpy()
    np.testing.assert_allclose(gx, gxd, rtol=1e-5, atol=1e-5)
    gwd = np.zeros_like(w)
    for k, (dx, dy, dz) in enumerate(off // dil if dil > 1 else off):
        a, b, cc = (dx + ks // 2, dy + ks // 2, dz + ks // 2) if ks % 2 else (dx, dy, dz)
        gwd[k] = wd.grad[:, :, a, b, cc].T.numpy()
    np.testing.assert_allclose(gw, gwd, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("ks,stride,dil,seed", [(3, 1, 1, 0), (3, 1, 2, 1), (2, 2, 1, 2), (5, 1, 1, 3)])
def test_conv_matches_dense_conv3d(ks, stride, dil, seed):
    _dense_conv3d_check(ks, stride, dil, seed)


def test_conv_4d_brute_force():
    """D=4, K=81: fp64 brute force straight from coordinates."""
    rng = np.random.default_rng(11)
    pts = np.unique(rng.integers(0, 4, (60, 4)), axis=0)
    c = np.concatenate([np.zeros((len(pts), 1), int), pts], 1).astype(np.int32)
    off = oracle.region_offsets(4, 3)
    kofs, ir, orr = oracle.kernel_map(c, c, off)
    x = rng.standard_normal((len(c), 2)).astype(np.float32)
    w = rng.standard_normal((81, 2, 3)).astype(np.float32)
    y = oracle.conv_forward(x, w, kofs, ir, orr, len(c))
    where = {tuple(r): i for i, r in enumerate(c.tolist())}
    exp = np.zeros((len(c), 3))
    for o in range(len(c)):
        for k in range(81):
            q = c[o].copy()
            q[1:] += off[k]
            i = where.get(tuple(q.tolist()))
            if i is not None:
                exp[o] += x[i].astype(np.float64) @ w[k].astype(np.float64)
    np.testing.assert_allclose(y, exp, rtol=1e-5, atol=1e-5)


def test_checks_catch_planted_mistakes():
    """A check that cannot fail pins nothing: plant the mistakes a kernel is
    likely to make (sign of the offset, swapped in/out operands, mirrored
    weight index, a dropped pair) into the oracle's inputs on the CPU and
    confirm the brute-force references reject every one."""
    rng = np.random.default_rng(5)
    c = np.concatenate([np.zeros((200, 1)), rng.integers(-3, 4, (200, 3))], 1).astype(np.int32)
    c, _, _ = oracle.insert_and_map(c)
    off = oracle.region_offsets(3, 3)
    ref = _brute_kernel_map(c, c, off)
    kofs, ir, orr = oracle.kernel_map(c, c, off)
    assert np.array_equal(oracle.canonical_pairs(kofs, ir, orr), ref)
    # wrong sign of the offset
    kofs_n, ir_n, orr_n = oracle.kernel_map(c, c, -off)
    assert not np.array_equal(oracle.canonical_pairs(kofs_n, ir_n, orr_n), ref)
    # swapped operands
    assert not np.array_equal(oracle.canonical_pairs(kofs, orr, ir), ref)
    # a dropped pair
    kofs_d = np.minimum(kofs, kofs[-1] - 1)
    assert not np.array_equal(oracle.canonical_pairs(kofs_d, ir[:-1], orr[:-1]), ref)
    # mirrored weight index against the dense textbook convolution
    x = rng.standard_normal((len(c), 2)).astype(np.float32)
    w = rng.standard_normal((27, 2, 2)).astype(np.float32)
    y = oracle.conv_forward(x, w, kofs, ir, orr, len(c))
    y_bad = oracle.conv_forward(x, w[::-1].copy(), kofs, ir, orr, len(c))
    assert not np.allclose(y, y_bad, rtol=1e-4, atol=1e-4)
