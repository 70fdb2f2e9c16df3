"""CPU oracle for the sparse-convolution hot path — TEST INFRASTRUCTURE ONLY.

numpy wrappers over ``oracle/oracle.c`` (a restatement of RiemannEngine's CPU
semantics, each C function cites the reference file:line it follows). Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this package, and only as the checker; the shipped path never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")

_lib = None
_i64p = ctypes.POINTER(ctypes.c_int64)


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_insert_and_map.restype = i64
        L.oracle_insert_and_map.argtypes = [vp, i64, i32, vp, vp, vp]
        L.oracle_region_offsets.restype = i32
        L.oracle_region_offsets.argtypes = [i32, i32, vp, vp, vp, vp, i32, vp]
        L.oracle_kernel_map.restype = i64
        L.oracle_kernel_map.argtypes = [vp, i64, vp, i64, i32, vp, i32, vp, vp, vp]
        L.oracle_stride.restype = i64
        L.oracle_stride.argtypes = [vp, i64, i32, vp, vp]
        L.oracle_stride_region.restype = i64
        L.oracle_stride_region.argtypes = [vp, i64, i32, vp, i32, vp]
        L.oracle_conv_forward.restype = None
        L.oracle_conv_forward.argtypes = [vp, i64, i32, vp, i32, i32, vp, vp, vp, i64, vp]
        L.oracle_conv_backward.restype = None
        L.oracle_conv_backward.argtypes = [vp, i64, i32, vp, i64, i32, vp, i32, vp, vp, vp,
                                           vp, vp]
        L.oracle_stride_map.restype = i64
        L.oracle_stride_map.argtypes = [vp, i64, i32, vp, i64, vp, vp]
        L.oracle_pool_forward.restype = None
        L.oracle_pool_forward.argtypes = [vp, i64, i32, vp, vp, i64, i64, i32, vp, vp]
        L.oracle_pool_backward.restype = None
        L.oracle_pool_backward.argtypes = [vp, vp, vp, i64, i64, i32, vp, vp, i64, i32, vp]
        L.oracle_global_pool_forward.restype = i64
        L.oracle_global_pool_forward.argtypes = [vp, vp, i64, i32, i32, i32, i64, vp]
        L.oracle_global_pool_backward.restype = None
        L.oracle_global_pool_backward.argtypes = [vp, vp, vp, vp, i64, i32, i32, i64, i32, vp]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


REGION = {"cube": 0, "cross": 1, "custom": 2}


def insert_and_map(coords):
    """(unique_rows, mapping, inverse), first occurrence wins."""
    coords = _c(coords, np.int32)
    n, ncol = coords.shape
    uq = np.empty((max(n, 1), ncol), np.int32)
    mp = np.empty(max(n, 1), np.int64)
    inv = np.empty(max(n, 1), np.int64)
    nu = lib().oracle_insert_and_map(_p(coords), n, ncol, _p(uq), _p(mp), _p(inv))
    return uq[:nu], mp[:nu], inv[:n]


def region_offsets(D, kernel_size=3, dilation=1, tensor_stride=1, region="cube", custom=None):
    """Scaled stencil offsets [K, D] in the reference's enumeration order."""
    def vec(v):
        return _c(np.broadcast_to(np.asarray(v), (D,)), np.int32)
    ks, dil, ts = vec(kernel_size), vec(dilation), vec(tensor_stride)
    cust = _c(custom if custom is not None else np.zeros((1, D)), np.int32)
    ncust = cust.shape[0] if custom is not None else 0
    kmax = int(np.prod(ks)) + int(np.sum(ks)) + ncust + 1
    out = np.empty((kmax, D), np.int32)
    K = lib().oracle_region_offsets(REGION[region], D, _p(ks), _p(dil), _p(ts), _p(cust),
                                    ncust, _p(out))
    return out[:K].copy()


def kernel_map(in_coords, out_coords, offsets):
    """(kofs[K+1], in_rows[P], out_rows[P]); bucket k sorted by output row."""
    a, b = _c(in_coords, np.int32), _c(out_coords, np.int32)
    off = _c(offsets, np.int32)
    K = off.shape[0]
    ncol = a.shape[1] if a.size else b.shape[1]
    cap = max(b.shape[0] * K, 1)
    ir, orr = np.empty(cap, np.int32), np.empty(cap, np.int32)
    counts = np.empty(K, np.int64)
    P = lib().oracle_kernel_map(_p(a), a.shape[0], _p(b), b.shape[0], ncol, _p(off), K,
                                _p(ir), _p(orr), _p(counts))
    kofs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    return kofs, ir[:P].copy(), orr[:P].copy()


def stride(coords, out_tensor_stride):
    coords = _c(coords, np.int32)
    n, ncol = coords.shape
    s = _c(out_tensor_stride, np.int32)
    out = np.empty((max(n, 1), ncol), np.int32)
    nu = lib().oracle_stride(_p(coords), n, ncol, _p(s), _p(out))
    return out[:nu].copy()


def stride_region(coords, offsets):
    """Generated map of a generative transposed convolution: the unique rows
    of c + offsets[k] over input rows c and offsets k (first occurrence)."""
    coords = _c(coords, np.int32)
    n, ncol = coords.shape
    off = _c(offsets, np.int32)
    K = off.shape[0]
    out = np.empty((max(n * K, 1), ncol), np.int32)
    nu = lib().oracle_stride_region(_p(coords), n, ncol, _p(off), K, _p(out))
    return out[:nu].copy()


def conv_forward(x, weight, kofs, in_rows, out_rows, n_out):
    x, w = _c(x, np.float32), _c(weight, np.float32)
    K, cin, cout = w.shape
    y = np.empty((max(n_out, 1), cout), np.float32)
    lib().oracle_conv_forward(_p(x), x.shape[0], cin, _p(w), K, cout, _p(_c(kofs, np.int64)),
                              _p(_c(in_rows, np.int32)), _p(_c(out_rows, np.int32)), n_out,
                              _p(y))
    return y[:n_out]


def conv_backward(x, grad_y, weight, kofs, in_rows, out_rows):
    x, gy, w = _c(x, np.float32), _c(grad_y, np.float32), _c(weight, np.float32)
    K, cin, cout = w.shape
    gx = np.empty((max(x.shape[0], 1), cin), np.float32)
    gw = np.empty((K, cin, cout), np.float32)
    lib().oracle_conv_backward(_p(x), x.shape[0], cin, _p(gy), gy.shape[0], cout, _p(w), K,
                               _p(_c(kofs, np.int64)), _p(_c(in_rows, np.int32)),
                               _p(_c(out_rows, np.int32)), _p(gx), _p(gw))
    return gx[:x.shape[0]], gw


def canonical_pairs(kofs, in_rows, out_rows, in_coords=None, out_coords=None):
    """Sorted (k, out, in) triplets; with coordinates given, rows are replaced
    by their coordinates so that maps over differently ordered row sets
    compare equal. Returns an int64 array [P, 3] or [P, 1 + 2*ncol]."""
    kofs = np.asarray(kofs)
    ks = np.repeat(np.arange(len(kofs) - 1), np.diff(kofs))
    ir, orr = np.asarray(in_rows, np.int64), np.asarray(out_rows, np.int64)
    if in_coords is None:
        t = np.stack([ks, orr, ir], axis=1)
    else:
        t = np.concatenate([ks[:, None], np.asarray(out_coords)[orr],
                            np.asarray(in_coords)[ir]], axis=1).astype(np.int64)
    if t.shape[0] == 0:
        return t
    idx = np.lexsort(t.T[::-1])
    return t[idx]


POOL_MODE = {"sum": 0, "avg": 1, "max": 2, "max_scatter": 3}


def stride_map(in_coords, out_coords, out_tensor_stride):
    """in_to_out [n_in]: the output row of each input's floor-aligned
    coordinates (-1 where there is none) and the number of such misses."""
    a, b = _c(in_coords, np.int32), _c(out_coords, np.int32)
    ncol = a.shape[1]
    s = _c(out_tensor_stride, np.int32)
    r = np.empty(max(a.shape[0], 1), np.int32)
    miss = lib().oracle_stride_map(_p(a), a.shape[0], ncol, _p(b), b.shape[0], _p(s), _p(r))
    return r[:a.shape[0]], int(miss)


def pool_forward(x, in_rows, out_rows, n_out, mode):
    """(y [n_out, C], counts [n_out]) of local pooling over the pair list."""
    x = _c(x, np.float32)
    C = x.shape[1]
    ir, orr = _c(in_rows, np.int32), _c(out_rows, np.int32)
    y = np.empty((max(n_out, 1), C), np.float32)
    cnt = np.empty(max(n_out, 1), np.int32)
    lib().oracle_pool_forward(_p(x), x.shape[0], C, _p(ir), _p(orr), ir.shape[0], n_out,
                              POOL_MODE[mode], _p(y), _p(cnt))
    return y[:n_out], cnt[:n_out]


def pool_backward(x, y, grad_y, in_rows, out_rows, mode):
    x, y, gy = _c(x, np.float32), _c(y, np.float32), _c(grad_y, np.float32)
    C = x.shape[1]
    ir, orr = _c(in_rows, np.int32), _c(out_rows, np.int32)
    gx = np.empty((max(x.shape[0], 1), C), np.float32)
    lib().oracle_pool_backward(_p(x), _p(y), _p(gy), x.shape[0], y.shape[0], C, _p(ir),
                               _p(orr), ir.shape[0], POOL_MODE[mode], _p(gx))
    return gx[:x.shape[0]]


def global_pool_forward(x, coords, mode):
    """y [B, C] with B = max batch index + 1."""
    x, c = _c(x, np.float32), _c(coords, np.int32)
    n, ncol = c.shape
    C = x.shape[1]
    B = lib().oracle_global_pool_forward(_p(x), _p(c), n, ncol, C, POOL_MODE[mode], 0, None)
    y = np.empty((max(B, 1), C), np.float32)
    lib().oracle_global_pool_forward(_p(x), _p(c), n, ncol, C, POOL_MODE[mode], B, _p(y))
    return y[:B]


def global_pool_backward(x, y, grad_y, coords, mode):
    x, y, gy, c = (_c(x, np.float32), _c(y, np.float32), _c(grad_y, np.float32),
                   _c(coords, np.int32))
    n, ncol = c.shape
    gx = np.empty((max(n, 1), x.shape[1]), np.float32)
    lib().oracle_global_pool_backward(_p(x), _p(y), _p(gy), _p(c), n, ncol, x.shape[1],
                                      y.shape[0], POOL_MODE[mode], _p(gx))
    return gx[:n]
