"""Pins the pooling functions of the CPU oracle: the reference's own known
answers (tests/engine/test_layers.cpp:58-115, as fixtures), brute force for
the stride map, torch's sum/mean/amax and their autograd (ties split evenly)
on the same groups, and closed forms."""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from helpers import random_coords


def _kats(golden_dir):
    with open(os.path.join(golden_dir, "kat_layers_pooling.json")) as f:
        return json.load(f)


def test_strided_pooling_known_answers(golden_dir):
    d = _kats(golden_dir)
    inp = d["strided"]["input"]
    c = np.array(inp["coords"], np.int32)
    x = np.array(inp["features"], np.float32)
    out = oracle.stride(c, inp["out_tensor_stride"])
    assert len(out) == inp["out_rows"]
    in_to_out, miss = oracle.stride_map(c, out, inp["out_tensor_stride"])
    assert miss == 0
    rows = {tuple(r[1:]): i for i, r in enumerate(out.tolist())}
    for kat in d["strided"]["kats"]:
        y, _ = oracle.pool_forward(x, np.arange(len(c)), in_to_out, len(out), kat["mode"])
        got = y[rows[tuple(kat["coordinate"])], 0]
        assert abs(got - kat["expected"]) <= d["tolerance_abs"], kat


def test_global_pooling_known_answers(golden_dir):
    d = _kats(golden_dir)
    inp = d["global"]["input"]
    c = np.array(inp["coords"], np.int32)
    x = np.array(inp["features"], np.float32)
    for kat in d["global"]["kats"]:
        y = oracle.global_pool_forward(x, c, kat["mode"])
        assert y.shape == (2, 2)
        np.testing.assert_allclose(y[kat["batch"]], kat["expected"], atol=d["tolerance_abs"])


def test_stride_map_brute_force():
    rng = np.random.default_rng(3)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 3000, 3, 40))
    for s in ([2, 2, 2], [3, 1, 4]):
        out = oracle.stride(c, s)
        in_to_out, miss = oracle.stride_map(c, out, s)
        assert miss == 0
        expect = np.concatenate([c[:, :1], np.floor_divide(c[:, 1:], s) * np.array(s)], 1)
        np.testing.assert_array_equal(out[in_to_out], expect)
    # a row whose strided coordinates are absent counts as a miss
    in_to_out, miss = oracle.stride_map(c, out[1:], [3, 1, 4])
    assert miss == np.sum(in_to_out < 0) and miss > 0


def _torch_pool(x, in_rows, out_rows, n_out, mode, gy):
    """evaluate_pooling's graph written with torch ops: per output, index_select
    of its rows, then sum / mean / amax; zeros for an empty output."""
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    ys = []
    for o in range(n_out):
        rows = torch.tensor(in_rows[out_rows == o], dtype=torch.long)
        if len(rows) == 0:
            ys.append(torch.zeros(x.shape[1], dtype=torch.float64))
            continue
        v = xt.index_select(0, rows)
        ys.append(v.sum(0) if mode == "sum" else v.mean(0) if mode == "avg" else v.amax(0))
    y = torch.stack(ys)
    (y * torch.tensor(gy, dtype=torch.float64)).sum().backward()
    return y.detach().numpy(), xt.grad.numpy()


@pytest.mark.parametrize("mode", ["sum", "avg", "max"])
def test_pool_matches_torch_graph(mode):
    rng = np.random.default_rng(11)
    n_in, n_out, C = 60, 25, 5
    P = 150
    in_rows = rng.integers(0, n_in, P).astype(np.int32)
    out_rows = rng.integers(0, n_out - 3, P).astype(np.int32)  # 3 empty outputs
    keep = np.unique(np.stack([in_rows, out_rows], 1), axis=0)  # one pair per (in, out)
    in_rows, out_rows = keep[:, 0].copy(), keep[:, 1].copy()
    x = rng.integers(-3, 4, (n_in, C)).astype(np.float32)  # small integers: many ties
    gy = rng.standard_normal((n_out, C)).astype(np.float32)
    y, counts = oracle.pool_forward(x, in_rows, out_rows, n_out, mode)
    ty, tgx = _torch_pool(x, in_rows, out_rows, n_out, mode, gy)
    np.testing.assert_allclose(y, ty, rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(counts, np.bincount(out_rows, minlength=n_out))
    gx = oracle.pool_backward(x, y, gy, in_rows, out_rows, mode)
    np.testing.assert_allclose(gx, tgx, rtol=1e-5, atol=1e-6)


def test_pool_closed_forms():
    rng = np.random.default_rng(5)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 2000, 3, 25))
    out = oracle.stride(c, [2, 2, 2])
    m, _ = oracle.stride_map(c, out, [2, 2, 2])
    ones = np.ones((len(c), 3), np.float32)
    y, counts = oracle.pool_forward(ones, np.arange(len(c)), m, len(out), "sum")
    np.testing.assert_array_equal(y[:, 0], np.bincount(m))  # sum of ones = group size
    y, _ = oracle.pool_forward(ones * 7.5, np.arange(len(c)), m, len(out), "avg")
    np.testing.assert_array_equal(y, 7.5)
    # one-hot: the max of a group is 1 exactly where the group holds the hot row
    hot = np.zeros((len(c), 1), np.float32)
    hot[17] = 1
    y, _ = oracle.pool_forward(hot, np.arange(len(c)), m, len(out), "max")
    assert y.sum() == 1 and y[m[17], 0] == 1
    # max gradient: all-equal group splits evenly
    g = oracle.pool_backward(ones, np.ones((len(out), 3), np.float32),
                             np.ones((len(out), 3), np.float32), np.arange(len(c)), m, "max")
    np.testing.assert_allclose(g[:, 0], 1.0 / np.bincount(m)[m])


@pytest.mark.parametrize("mode", ["sum", "avg", "max"])
def test_global_pool_matches_torch(mode):
    rng = np.random.default_rng(13)
    n, C = 80, 4
    c = random_coords(rng, n, 3, 10, batch=4)
    c[c[:, 0] == 2, 0] = 3  # batch 2 empty: zero row
    x = rng.integers(-2, 3, (n, C)).astype(np.float32)
    y = oracle.global_pool_forward(x, c, mode)
    assert y.shape == (4, C) and np.all(y[2] == 0)
    gy = rng.standard_normal((4, C)).astype(np.float32)
    ty, tgx = _torch_pool(x, np.arange(n, dtype=np.int32), c[:, 0], 4, mode, gy)
    np.testing.assert_allclose(y, ty, rtol=1e-6, atol=1e-6)
    gx = oracle.global_pool_backward(x, y, gy, c, mode)
    np.testing.assert_allclose(gx, tgx, rtol=1e-5, atol=1e-6)


def test_planted_mistake_fails_the_torch_check():
    """A plausible slip (average divided by the number of kernel offsets
    instead of the pooled rows) is caught by the torch comparison above."""
    rng = np.random.default_rng(2)
    in_rows = np.array([0, 1, 2, 3], np.int32)
    out_rows = np.array([0, 0, 0, 1], np.int32)
    x = rng.standard_normal((4, 2)).astype(np.float32)
    y, _ = oracle.pool_forward(x, in_rows, out_rows, 2, "sum")
    wrong = y / 8.0  # "K = 8" instead of the group sizes 3 and 1
    ty, _ = _torch_pool(x, in_rows, out_rows, 2, "avg", np.zeros((2, 2), np.float32))
    assert not np.allclose(wrong, ty, rtol=1e-5)
    good, _ = oracle.pool_forward(x, in_rows, out_rows, 2, "avg")
    np.testing.assert_allclose(good, ty, rtol=1e-6)


def test_scatter_max_gradient_matches_torch():
    """Mode max_scatter = zeros.scatter_reduce("amax", include_self=False) as
    the reference's MAX_POOL quantization computes it: torch's backward
    counts the excluded zero as a tie where the maximum is 0."""
    rng = np.random.default_rng(17)
    n, G, C = 200, 40, 3
    group = rng.integers(0, G, n).astype(np.int32)
    group[:G] = np.arange(G)  # every group non-empty
    x = rng.integers(-3, 2, (n, C)).astype(np.float32)  # many maxima at 0
    gy = rng.standard_normal((G, C)).astype(np.float32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    idx = torch.tensor(group, dtype=torch.long)[:, None].expand(n, C)
    r = torch.zeros(G, C, dtype=torch.float64).scatter_reduce(0, idx, xt, "amax",
                                                              include_self=False)
    (r * torch.tensor(gy, dtype=torch.float64)).sum().backward()
    rows = np.arange(n, dtype=np.int32)
    y, _ = oracle.pool_forward(x, rows, group, G, "max_scatter")
    np.testing.assert_array_equal(y, r.detach().numpy())
    np.testing.assert_allclose(oracle.pool_backward(x, y, gy, rows, group, "max_scatter"),
                               xt.grad.numpy(), rtol=1e-6, atol=1e-7)
    assert (y == 0).any()  # the case that differs from plain max is exercised
    plain = oracle.pool_backward(x, y, gy, rows, group, "max")
    assert not np.allclose(plain, xt.grad.numpy())
