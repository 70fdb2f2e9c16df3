"""Stencil offsets of a convolution region (product side, host only).

Enumerates the lattice offsets of kernel index k exactly as
kernel_region::coordinate_at does (RiemannEngine/engine/grid/stencil.hpp:
223-278) and sizes the region as set_volume does (:281-300):

* HYPER_CUBE: axis 0 (x) varies fastest, idx_i = (k / prod_{j<i} ks_j) % ks_i;
  odd sizes centre on zero, (idx_i - ks_i // 2) * dil_i * ts_i; even sizes
  enumerate non-negative offsets idx_i * dil_i * ts_i. K = prod ks_i.
* HYPER_CROSS: the centre first, then one axis at a time, offsets
  1..r then -r..-1 with r = (ks_i - 1) // 2. K = 1 + sum (ks_i - 1).
* CUSTOM: given lattice offsets, scaled by ts_i * dil_i.

The offsets are computed once per (kernel, tensor stride) on the host with
numpy and handed to the kernel-map generator as a device [K, D] array.
"""
from __future__ import annotations

from typing import Optional, Sequence, Union

import numpy as np

HYPER_CUBE, HYPER_CROSS, CUSTOM = "cube", "cross", "custom"

IntOrSeq = Union[int, Sequence[int]]


def _per_axis(v: IntOrSeq, D: int, name: str) -> np.ndarray:
    """Scalar broadcast of kernel parameters (KernelGenerator's ctor,
    engine/grid/stencil.cpp:81-150 expands a single value to every axis)."""
    a = np.asarray(v, dtype=np.int64).reshape(-1)
    if a.size == 1:
        a = np.repeat(a, D)
    if a.size != D:
        raise ValueError(f"{name} needs 1 or {D} values, got {a.size}")
    if np.any(a <= 0):
        raise ValueError(f"{name} must be positive")
    return a


def kernel_volume(D: int, kernel_size: IntOrSeq = 3, region: str = HYPER_CUBE,
                  custom: Optional[np.ndarray] = None) -> int:
    ks = _per_axis(kernel_size, D, "kernel_size")
    if region == HYPER_CUBE:
        return int(np.prod(ks))
    if region == HYPER_CROSS:
        return int(1 + np.sum(ks - 1))
    if region == CUSTOM:
        return 0 if custom is None else int(np.asarray(custom).shape[0])
    raise ValueError(f"unknown region {region!r}")


def region_offsets(D: int, kernel_size: IntOrSeq = 3, dilation: IntOrSeq = 1,
                   tensor_stride: IntOrSeq = 1, region: str = HYPER_CUBE,
                   custom: Optional[np.ndarray] = None) -> np.ndarray:
    """Scaled offsets [K, D] (int32), row k = offset of kernel index k."""
    ks = _per_axis(kernel_size, D, "kernel_size")
    dil = _per_axis(dilation, D, "dilation")
    ts = _per_axis(tensor_stride, D, "tensor_stride")
    step = dil * ts
    if region == HYPER_CUBE:
        K = int(np.prod(ks))
        k = np.arange(K, dtype=np.int64)
        out = np.empty((K, D), np.int64)
        div = 1
        for i in range(D):
            idx = (k // div) % ks[i]
            div *= ks[i]
            centre = 0 if ks[i] % 2 == 0 else ks[i] // 2
            out[:, i] = (idx - centre) * step[i]
    elif region == HYPER_CROSS:
        rows = [np.zeros(D, np.int64)]
        for axis in range(D):
            r = (ks[axis] - 1) // 2
            for ind in range(ks[axis] - 1):
                v = np.zeros(D, np.int64)
                v[axis] = (ind + 1 if ind < r else ind - 2 * r) * step[axis]
                rows.append(v)
        out = np.stack(rows)
    elif region == CUSTOM:
        if custom is None:
            raise ValueError("CUSTOM region needs offsets")
        c = np.asarray(custom, np.int64)
        if c.ndim != 2 or c.shape[1] != D:
            raise ValueError(f"custom offsets must be [K, {D}]")
        out = c * step
    else:
        raise ValueError(f"unknown region {region!r}")
    if np.any(np.abs(out) >= 2**31):
        raise ValueError("scaled offsets overflow int32")
    return out.astype(np.int32)
