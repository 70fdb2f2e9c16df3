"""Test infrastructure only: ctypes access to the reference's own CPU path.

oracle/ref.mk compiles the reference sources (RiemannEngine/engine/grid/
space.cpp, stencil.cpp, nn/conv.cpp, nn/pooling.cpp, tensor/sparse_tensor.cpp)
with CPU_ONLY
plus oracle/ref_driver.cpp into oracle/_ref/libriemann_ref.so. Tests use it to
check the oracle and the HIP path against the reference itself; bench.py
times it as the CPU baseline. ``available()`` is False where the library was
not built (the reference checkout is absent), and callers skip.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libriemann_ref.so")
_LIB = None

_vp, _i64, _i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32


def available() -> bool:
    return os.path.exists(LIB_PATH)


def lib():
    global _LIB
    if _LIB is None:
        import torch  # noqa: F401  (loads the LibTorch the library links against)
        L = ctypes.CDLL(LIB_PATH)
        L.ref_last_error.restype = ctypes.c_char_p
        L.ref_insert_and_map.restype = _i64
        L.ref_insert_and_map.argtypes = [_vp, _i64, ctypes.c_int, _i64, _vp, _vp, _vp]
        L.ref_kernel_map.restype = _i64
        L.ref_kernel_map.argtypes = [_vp, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, _i64, _vp, _vp, _vp, _i64, _vp,
                                     ctypes.POINTER(_i64), ctypes.POINTER(_i32)]
        L.ref_conv.restype = _i64
        L.ref_conv.argtypes = [_vp, _i64, ctypes.c_int, _vp, ctypes.c_int, _vp, ctypes.c_int,
                               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int, _vp, _i64, _vp, _vp, _vp, _vp]
        L.ref_conv_time.restype = _i64
        L.ref_conv_time.argtypes = [_vp, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double)]
        L.ref_map_time.restype = _i64
        L.ref_map_time.argtypes = [_vp, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(ctypes.c_double)]
        L.ref_stride_region.restype = _i64
        L.ref_stride_region.argtypes = [_vp, _i64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int, _i64, _vp]
        L.ref_pool.restype = _i64
        L.ref_pool.argtypes = [_vp, _i64, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_int,
                               ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                               ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _i64, _vp, _vp,
                               _vp]
        L.ref_global_pool.restype = _i64
        L.ref_global_pool.argtypes = [_vp, _i64, ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, _vp, _i64, _vp, _vp, _vp]
        L.ref_quantize.restype = _i64
        L.ref_quantize.argtypes = [_vp, _i64, ctypes.c_int, _vp, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, _vp, _i64, _vp, _vp, _vp]
        L.ref_num_threads.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _check(v):
    if v < 0:
        raise RuntimeError("reference: " + lib().ref_last_error().decode(errors="replace"))
    return v


def insert_and_map(coords):
    """(unique rows, mapping, inverse) from CoordinateManager::insert_and_map."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    u = np.empty((n, ncol), np.int32)
    m = np.empty(n, np.int64)
    inv = np.empty(n, np.int64)
    nu = _check(lib().ref_insert_and_map(_p(c), n, ncol, n, _p(u), _p(m), _p(inv)))
    return u[:nu], m[:nu], inv


def kernel_map(coords, ks=3, stride=1, dilation=1, region="cube"):
    """The kernel map a conv with these parameters builds over the unique rows
    `coords`: (kofs [K+1], in_rows, out_rows, out_coords)."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    reg = {"cube": 0, "cross": 1}[region]
    kofs = np.zeros(4097, np.int64)
    n_out, K = _i64(0), _i32(0)
    args = (_p(c), n, ncol, ks, stride, dilation, reg)
    P = _check(lib().ref_kernel_map(*args, 0, _p(kofs), None, None, 0, None,
                                    ctypes.byref(n_out), ctypes.byref(K)))
    ir = np.empty(max(P, 1), np.int32)
    orr = np.empty(max(P, 1), np.int32)
    oc = np.empty((max(n_out.value, 1), ncol), np.int32)
    _check(lib().ref_kernel_map(*args, P, _p(kofs), _p(ir), _p(orr), n_out.value, _p(oc),
                                ctypes.byref(n_out), ctypes.byref(K)))
    return kofs[:K.value + 1].copy(), ir[:P], orr[:P], oc[:n_out.value]


def conv(coords, x, w, gy=None, ks=3, stride=1, dilation=1, bf16=False):
    """RiemannConvolution forward (+ backward when gy is given) on the CPU.
    Returns (y, out_coords, gx, gw), fp32 arrays; with gy=None, gx/gw are None.
    gy must follow the reference's output row order (out_coords): pass
    gy=callable(out_coords) to build it from the output coordinates."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    K, cin, cout = w.shape
    args = (_p(c), n, ncol, _p(x), cin, _p(w), K, cout, ks, stride, dilation, 1 if bf16 else 0)
    n_out = _check(lib().ref_conv(*args, None, 0, None, None, None, None))
    y = np.empty((n_out, cout), np.float32)
    oc = np.empty((n_out, ncol), np.int32)
    if callable(gy):
        _check(lib().ref_conv(*args, None, n_out, _p(y), _p(oc), None, None))
        gy = gy(oc)
    g = None if gy is None else np.ascontiguousarray(gy, np.float32)
    gx = np.empty((n, cin), np.float32) if g is not None else None
    gw = np.empty((K, cin, cout), np.float32) if g is not None else None
    _check(lib().ref_conv(*args, _p(g), n_out, _p(y), _p(oc), _p(gx), _p(gw)))
    return y, oc, gx, gw


def conv_time(coords, cin, cout, ks=3, bf16=False, reps=3, seed=0):
    """(pairs, map ms, mean fwd+bwd step ms) of the reference on the CPU: the
    first forward builds the kernel map, the timed steps reuse it."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    map_ms, step_ms = ctypes.c_double(0), ctypes.c_double(0)
    P = _check(lib().ref_conv_time(_p(c), n, ncol, cin, cout, ks, 1 if bf16 else 0, reps, seed,
                                   ctypes.byref(map_ms), ctypes.byref(step_ms)))
    return P, map_ms.value, step_ms.value


def map_time(coords, ks=3, reps=3):
    """(pairs, hash ms, kernel-map ms) of the reference's CPU map build over
    the rows `coords`: insert_and_map, then the ks^D cube kernel map, each the
    mean of `reps` runs from a fresh manager."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    h, m = ctypes.c_double(0), ctypes.c_double(0)
    P = _check(lib().ref_map_time(_p(c), n, ncol, ks, reps, ctypes.byref(h), ctypes.byref(m)))
    return P, h.value, m.value


def stride_region(coords, in_stride, stride, ks, dilation=1, region="cube"):
    """Generated rows of CoordinateMapManager::stride_region for a generative
    transposed conv from tensor stride in_stride to in_stride / stride."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    reg = {"cube": 0, "cross": 1}[region]
    args = (_p(c), n, ncol, in_stride, stride, ks, dilation, reg)
    m = _check(lib().ref_stride_region(*args, 0, None))
    out = np.empty((max(m, 1), ncol), np.int32)
    _check(lib().ref_stride_region(*args, m, _p(out)))
    return out[:m]


POOL_MODE = {"sum": 0, "avg": 1, "max": 2}


def pool(coords, x, mode="avg", ks=2, stride=2, dilation=1, gy=None, in_stride=1,
         transpose=False, expand=False, bf16=False):
    """The reference's local pooling layer (RiemannSumPooling / AvgPooling /
    MaxPooling, or RiemannPoolingTranspose with that mode) on the unique rows
    `coords` at tensor stride in_stride with features x (row order of coords).
    Returns (y, out_coords, gx); gy follows out_coords' row order, or is a
    callable(out_coords) that builds it; gx is None without gy."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    x = np.ascontiguousarray(x, np.float32)
    C = x.shape[1]
    args = (_p(c), n, ncol, in_stride, _p(x), C, ks, stride, dilation, POOL_MODE[mode],
            int(transpose), int(expand), 1 if bf16 else 0)
    n_out = _check(lib().ref_pool(*args, None, 0, None, None, None))
    y = np.empty((max(n_out, 1), C), np.float32)
    oc = np.empty((max(n_out, 1), ncol), np.int32)
    if callable(gy):
        _check(lib().ref_pool(*args, None, n_out, _p(y), _p(oc), None))
        gy = gy(oc[:n_out])
    g = None if gy is None else np.ascontiguousarray(gy, np.float32)
    gx = np.empty((n, C), np.float32) if g is not None else None
    _check(lib().ref_pool(*args, _p(g), n_out, _p(y), _p(oc), _p(gx)))
    return y[:n_out], oc[:n_out], gx


def global_pool(coords, x, mode="avg", gy=None, bf16=False):
    """RiemannGlobalPooling (GLOBAL_*_POOLING_PYTORCH_INDEX) on the CPU.
    Returns (y [B, C], out_coords [B, ncol], gx)."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    x = np.ascontiguousarray(x, np.float32)
    C = x.shape[1]
    args = (_p(c), n, ncol, _p(x), C, POOL_MODE[mode], 1 if bf16 else 0)
    B = _check(lib().ref_global_pool(*args, None, 0, None, None, None))
    g = None if gy is None else np.ascontiguousarray(gy, np.float32)
    y = np.empty((max(B, 1), C), np.float32)
    oc = np.empty((max(B, 1), ncol), np.int32)
    gx = np.empty((n, C), np.float32) if g is not None else None
    _check(lib().ref_global_pool(*args, _p(g), B, _p(y), _p(oc), _p(gx)))
    return y[:B], oc[:B], gx


QUANT_MODE = {"subsample": 0, "avg": 1, "sum": 2, "max": 3}


def quantize(coords, x, mode="avg", gy=None, bf16=False):
    """SparseTensor(x, coords, quantization_mode) on the CPU: (features [n_u, C],
    unique coordinates [n_u, ncol], gx); gy in the unique rows' order, or a
    callable(unique coords) that builds it."""
    c = np.ascontiguousarray(coords, np.int32)
    n, ncol = c.shape
    x = np.ascontiguousarray(x, np.float32)
    C = x.shape[1]
    args = (_p(c), n, ncol, _p(x), C, QUANT_MODE[mode], 1 if bf16 else 0)
    nu = _check(lib().ref_quantize(*args, None, 0, None, None, None))
    y = np.empty((max(nu, 1), C), np.float32)
    oc = np.empty((max(nu, 1), ncol), np.int32)
    if callable(gy):
        _check(lib().ref_quantize(*args, None, nu, _p(y), _p(oc), None))
        gy = gy(oc[:nu])
    g = None if gy is None else np.ascontiguousarray(gy, np.float32)
    gx = np.empty((n, C), np.float32) if g is not None else None
    _check(lib().ref_quantize(*args, _p(g), nu, _p(y), _p(oc), _p(gx)))
    return y[:nu], oc[:nu], gx


def num_threads() -> int:
    return int(lib().ref_num_threads())
