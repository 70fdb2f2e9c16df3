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
