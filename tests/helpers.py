"""Shared helpers of the GPU parity tests (HIP path through the C ABI vs the
CPU oracle)."""
import numpy as np
import torch

import oracle
from riemannengine_amd import abi

DEV = torch.device("cuda:0")

# Tolerances stated by the task: outputs and gradients within rel 1e-4 (fp32)
# and 2e-2 (bf16) of the reference CPU path. "rel" is norm-wise here:
# max|got - ref| <= tol * max|ref| over the whole tensor.
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def assert_rel(got, ref, tol, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    scale = max(np.abs(ref).max(initial=0.0), 1e-30)
    err = np.abs(got - ref).max(initial=0.0)
    assert err <= tol * scale, f"{what}: max err {err:.3e} > {tol:.1e} * {scale:.3e}"


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t if dtype is None else t.to(dtype)


def gpu_tables_and_map(in_coords, out_coords, offsets, same=False):
    tin = abi.hash_build(to_dev(in_coords))
    tout = tin if same else abi.hash_build(to_dev(out_coords))
    km = abi.kernel_map(tin, tout, to_dev(offsets))
    return tin, tout, km


def gpu_canonical(km):
    return oracle.canonical_pairs(km.offsets_host, km.in_rows.cpu().numpy(),
                                  km.out_rows.cpu().numpy())


def random_coords(rng, n, D=3, span=20, batch=2):
    c = np.concatenate([rng.integers(0, batch, (n, 1)), rng.integers(-span, span, (n, D))], 1)
    return c.astype(np.int32)


def oracle_pool_layer(c, x, mode, ks, stride, dil=1, in_stride=1, transpose=False,
                      expand=False, gy=None):
    """What the reference's pooling layer computes on the map of unique rows c
    at tensor stride in_stride (engine/nn/pooling.cpp:17-201), from the
    oracle: (out_coords, y, grad_x or None). gy is a callable(out_coords)."""
    D = c.shape[1] - 1
    if not transpose:
        out_stride = in_stride * stride
        out = oracle.stride(c, [out_stride] * D)
        if ks == stride:  # stride map
            in_rows, miss = np.arange(len(c), dtype=np.int32), 0
            out_rows, miss = oracle.stride_map(c, out, [out_stride] * D)
            assert miss == 0
        else:
            _, in_rows, out_rows = oracle.kernel_map(
                c, out, oracle.region_offsets(D, ks, dil, in_stride))
    else:
        out_stride = in_stride // stride
        off = oracle.region_offsets(D, ks, dil, out_stride)
        out = c if (out_stride == in_stride and not expand) else oracle.stride_region(c, off)
        if ks == stride:  # stride map fine -> coarse, swapped
            in_rows, miss = oracle.stride_map(out, c, [in_stride] * D)
            assert miss == 0
            out_rows = np.arange(len(out), dtype=np.int32)
        else:  # fine -> coarse map with the region at the fine stride, swapped
            _, out_rows, in_rows = oracle.kernel_map(out, c, off)
    y, _ = oracle.pool_forward(x, in_rows, out_rows, len(out), mode)
    gx = None
    if gy is not None:
        gx = oracle.pool_backward(x, y, gy(out), in_rows, out_rows, mode)
    return out, y, gx


def coord_grad(oc, C, seed=0):
    """A gradient that is a fixed function of the output coordinates, so that
    two implementations with different output row orders get the same one."""
    oc = np.asarray(oc, np.float64)
    w = np.array([1.3, 2.1, 0.7, 3.3, 0.4, 1.9, 2.7, 0.9][:oc.shape[1]])
    base = oc @ w + seed
    return np.sin(base[:, None] * 0.37 + np.arange(C)[None, :] * 0.5).astype(np.float32)


def align(ref_coords, coords):
    """Permutation p with coords[p] == ref_coords (row sets must be equal)."""
    idx = {tuple(r): i for i, r in enumerate(np.asarray(coords).tolist())}
    assert len(idx) == len(coords) == len(ref_coords)
    return np.array([idx[tuple(r)] for r in np.asarray(ref_coords).tolist()], np.int64)


def lookup(table, rows):
    """Row index in `table` of every row of `rows` (all must be present)."""
    idx = {tuple(r): i for i, r in enumerate(np.asarray(table).tolist())}
    return np.array([idx[tuple(r)] for r in np.asarray(rows).tolist()], np.int64)
