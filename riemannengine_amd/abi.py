"""ctypes binding of the C ABI in ``include/riemann_hip.h``.

This is the thinnest possible host layer over ``libriemann_hip.so``: torch
tensors provide device memory and the current HIP stream, every kernel runs
through the C entry points. It is what the parity tests call, and it fails
loudly (``RuntimeError``) when the library is missing; there is no CPU path.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libriemann_hip.so")
MAX_COLS = 8

F32, BF16 = 0, 1
KEY_PACKED64, KEY_ROWREF = 0, 1
KMAP_SYMMETRIC = 1
KMAP_BRICK_NBHD = 2  # rhip_kmap_count's probes read each row's neighbourhood bricks once
POOL_SUM, POOL_AVG, POOL_MAX, POOL_MAX_SCATTER = 0, 1, 2, 3
POOL_MODES = {"sum": POOL_SUM, "avg": POOL_AVG, "max": POOL_MAX, "max_scatter": POOL_MAX_SCATTER}

# Every function the header declares (checked by the CPU test suite).
EXPORTS = (
    "rhip_last_error", "rhip_abi_version", "rhip_table_bytes",
    "rhip_hash_workspace_bytes", "rhip_hash_build", "rhip_hash_lookup",
    "rhip_order_workspace_bytes", "rhip_brick_bytes", "rhip_spatial_order",
    "rhip_stride_coords",
    "rhip_expand_coords", "rhip_kmap_workspace_bytes", "rhip_kmap_count", "rhip_kmap_fill",
    "rhip_kmap_pairs_workspace_bytes", "rhip_kmap_pairs", "rhip_stencil_partners",
    "rhip_conv_backward_weight_rows_supported",
    "rhip_conv_workspace_bytes", "rhip_conv_forward_workspace_bytes", "rhip_conv_forward",
    "rhip_conv_forward_noalloc", "rhip_conv_bias_grad",
    "rhip_conv_backward_input", "rhip_conv_backward_weight", "rhip_conv_backward_weight_rows",
    "rhip_stride_map_workspace_bytes", "rhip_stride_map_count", "rhip_group_map_count",
    "rhip_stride_map_fill",
    "rhip_table_compact", "rhip_pool_workspace_bytes", "rhip_pool_forward",
    "rhip_pool_backward",
    "rhip_global_pool_workspace_bytes", "rhip_batch_count", "rhip_batch_segments",
    "rhip_global_pool_forward", "rhip_global_pool_backward",
    "rhip_bn_workspace_bytes", "rhip_bn_stats", "rhip_bn_invstd", "rhip_bn_forward",
    "rhip_bn_backward",
)


class RhipTable(ctypes.Structure):
    _fields_ = [
        ("slots", ctypes.c_void_p), ("capacity", ctypes.c_int64),
        ("rows", ctypes.c_void_p), ("n_unique", ctypes.c_int64),
        ("ncol", ctypes.c_int32), ("mode", ctypes.c_int32),
        ("key_bits", ctypes.c_int32),
        ("lo", ctypes.c_int32 * MAX_COLS), ("hi", ctypes.c_int32 * MAX_COLS),
        ("shift", ctypes.c_int32 * MAX_COLS), ("tz", ctypes.c_int32 * MAX_COLS),
        ("order", ctypes.c_void_p), ("bricks", ctypes.c_void_p),
        ("morton_bits", ctypes.c_int32), ("brick_levels", ctypes.c_int32),
        ("brick_dims", ctypes.c_int32 * MAX_COLS),
    ]


_vp, _i64, _i32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t
_P = ctypes.POINTER


def _declare(lib):
    sig = {
        "rhip_last_error": (ctypes.c_char_p, []),
        "rhip_abi_version": (ctypes.c_int, []),
        "rhip_table_bytes": (_sz, [_i64]),
        "rhip_hash_workspace_bytes": (ctypes.c_int, [_i64, _i32, _P(_sz)]),
        "rhip_hash_build": (ctypes.c_int, [_vp, _i64, _i32, _vp, _sz, _vp, _sz, _vp,
                                           _vp, _vp, _P(RhipTable), _vp]),
        "rhip_hash_lookup": (ctypes.c_int, [_P(RhipTable), _vp, _i64, _vp, _vp]),
        "rhip_order_workspace_bytes": (ctypes.c_int, [_i64, _P(_sz)]),
        "rhip_brick_bytes": (ctypes.c_int, [_P(RhipTable), _P(_sz)]),
        "rhip_spatial_order": (ctypes.c_int, [_P(RhipTable), _vp, _vp, _vp, _sz, _vp, _sz, _vp]),
        "rhip_stride_coords": (ctypes.c_int, [_vp, _i64, _i32, _P(_i32), _vp, _vp]),
        "rhip_expand_coords": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i32, _vp, _vp]),
        "rhip_kmap_workspace_bytes": (ctypes.c_int, [_i64, _i64, _i32, _P(_sz)]),
        "rhip_kmap_count": (ctypes.c_int, [_P(RhipTable), _vp, _vp, _i64, _i32, _P(_i32),
                                           _vp, _sz, _vp, _vp, _vp, _P(_i64), _P(_i32),
                                           _vp]),
        "rhip_kmap_fill": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp, _i64, _i32, _vp, _sz,
                                          _vp, _vp, _vp, _vp, _vp, _vp]),
        "rhip_conv_workspace_bytes": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i64, _i64, _i64,
                                                     _P(_sz)]),
        "rhip_conv_forward": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i32, _i32, _vp, _vp,
                                             _vp, _i64, _vp, _i32, _vp, _sz, _vp]),
        "rhip_conv_forward_workspace_bytes": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i64, _i64,
                                                             _P(_sz)]),
        "rhip_conv_bias_grad": (ctypes.c_int, [_vp, _i64, _i32, _i32, _vp, _vp, _sz, _vp]),
        "rhip_conv_forward_noalloc": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i32, _i32, _vp,
                                                     _vp, _vp, _i64, _vp, _i32, _vp]),
        "rhip_conv_backward_input": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i32, _i32,
                                                    _vp, _vp, _vp, _i64, _vp, _i32, _vp,
                                                    _sz, _vp]),
        "rhip_conv_backward_weight_rows_supported": (ctypes.c_int, [_i32, _i32, _i32, _i32,
                                                                    _i64, _i64]),
        "rhip_kmap_pairs_workspace_bytes": (ctypes.c_int, [_i64, _i32, _P(_sz)]),
        "rhip_kmap_pairs": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp, _vp, _sz, _vp, _vp, _vp]),
        "rhip_stencil_partners": (ctypes.c_int, [_P(_i32), _i32, _i32, _P(_i32)]),
        "rhip_conv_backward_weight": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i64, _i32,
                                                     _i32, _vp, _i64, _vp, _vp, _vp,
                                                     _i32, _vp, _sz, _vp]),
        "rhip_conv_backward_weight_rows": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i64, _i32, _i32,
                                                          _vp, _vp, _vp, _i32, _vp, _sz, _vp]),
        "rhip_stride_map_workspace_bytes": (ctypes.c_int, [_i64, _i64, _P(_sz)]),
        "rhip_stride_map_count": (ctypes.c_int, [_P(RhipTable), _vp, _i64, _P(_i32), _vp, _sz,
                                                 _P(_i32), _vp]),
        "rhip_group_map_count": (ctypes.c_int, [_vp, _i64, _i64, _vp, _sz, _P(_i32), _vp]),
        "rhip_stride_map_fill": (ctypes.c_int, [_i64, _i64, _i32, _vp, _vp, _vp, _sz, _vp, _vp,
                                                _vp, _vp, _vp]),
        "rhip_table_compact": (ctypes.c_int, [_vp, _i32, _i64, _vp, _sz, _vp, _P(_i32), _vp]),
        "rhip_pool_workspace_bytes": (ctypes.c_int, [_i64, _i32, _i32, _P(_sz)]),
        "rhip_pool_forward": (ctypes.c_int, [_vp, _i64, _i32, _vp, _i32, _vp, _i64, _i32, _vp,
                                             _vp, _i32, _vp]),
        "rhip_pool_backward": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _vp, _i32, _vp, _vp,
                                              _i32, _vp, _i64, _vp, _i32, _vp, _i32, _vp, _sz,
                                              _vp]),
        "rhip_global_pool_workspace_bytes": (ctypes.c_int, [_i64, _i32, _i32, _P(_sz)]),
        "rhip_batch_count": (ctypes.c_int, [_vp, _i64, _i32, _vp, _sz, _P(_i32), _vp]),
        "rhip_batch_segments": (ctypes.c_int, [_vp, _i64, _i32, _i32, _vp, _sz, _vp, _vp,
                                               _vp]),
        "rhip_global_pool_forward": (ctypes.c_int, [_vp, _i64, _i32, _vp, _vp, _i32, _i32,
                                                    _vp, _i32, _vp, _sz, _vp]),
        "rhip_global_pool_backward": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i32, _i64, _i32,
                                                     _vp, _vp, _i32, _i32, _vp, _i32, _vp,
                                                     _sz, _vp]),
        "rhip_bn_workspace_bytes": (ctypes.c_int, [_i64, _i32, _P(_sz)]),
        "rhip_bn_stats": (ctypes.c_int, [_vp, _i64, _i32, _i32, ctypes.c_double,
                                         ctypes.c_double, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
        "rhip_bn_invstd": (ctypes.c_int, [_vp, _i32, ctypes.c_double, _vp, _vp]),
        "rhip_bn_forward": (ctypes.c_int, [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp,
                                           _i32, _vp]),
        "rhip_bn_backward": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _i32,
                                            _i32, _vp, _vp, _vp, _vp, _i32, _vp, _sz, _vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIB = None


def lib():
    """Load libriemann_hip.so (torch is imported first so both share one HIP
    runtime: both libraries ask for the soname libamdhip64.so.7)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m riemannengine_amd.build hip`")
        _LIB = _declare(ctypes.CDLL(LIB_PATH))
    return _LIB


def _check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().rhip_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a device tensor (the HIP path has no CPU fallback)")


def _sizeq(fn, *args) -> int:
    out = _sz(0)
    _check(fn(*args, ctypes.byref(out)), fn.__name__)
    return int(out.value)


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise RuntimeError(f"unsupported feature dtype {dt}; the HIP path computes fp32 or bf16")


# ------------------------------------------------------------------ tables

@dataclass
class CoordTable:
    """A built coordinate map: hash slots + unique rows + locality order."""
    struct: RhipTable
    slots: torch.Tensor
    ucoords: torch.Tensor          # [n_unique, ncol] int32
    mapping: torch.Tensor          # [n_unique] int64 first input row
    inverse: Optional[torch.Tensor]  # [n] int64
    order: torch.Tensor            # [n_unique] int32 processing order
    pos: torch.Tensor              # [n_unique] int32 inverse of order
    keep: list = field(default_factory=list)

    @property
    def n(self) -> int:
        return int(self.struct.n_unique)

    @property
    def ncol(self) -> int:
        return int(self.struct.ncol)

    def lookup(self, queries: torch.Tensor) -> torch.Tensor:
        queries = queries.to(torch.int32).contiguous()
        _require_cuda(queries, "queries")
        out = torch.empty(queries.shape[0], dtype=torch.int32, device=queries.device)
        _check(lib().rhip_hash_lookup(ctypes.byref(self.struct), _ptr(queries),
                                      queries.shape[0], _ptr(out), _stream(queries.device)),
               "rhip_hash_lookup")
        return out


def hash_build(coords: torch.Tensor, with_inverse: bool = True,
               with_order: bool = True) -> CoordTable:
    """Deduplicate int32 rows [n, ncol] on the GPU (first occurrence wins)."""
    _require_cuda(coords, "coords")
    if coords.dtype != torch.int32 or coords.dim() != 2:
        raise RuntimeError("coords must be a 2-D int32 tensor")
    coords = coords.contiguous()
    L, dev = lib(), coords.device
    n, ncol = coords.shape
    slots = torch.empty(int(L.rhip_table_bytes(n)), dtype=torch.uint8, device=dev)
    ws = torch.empty(_sizeq(L.rhip_hash_workspace_bytes, n, ncol), dtype=torch.uint8, device=dev)
    ucoords = torch.empty((max(n, 1), ncol), dtype=torch.int32, device=dev)
    mapping = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
    inverse = torch.empty(max(n, 1), dtype=torch.int64, device=dev) if with_inverse else None
    st = RhipTable()
    _check(L.rhip_hash_build(_ptr(coords), n, ncol, _ptr(slots), slots.numel(), _ptr(ws),
                             ws.numel(), _ptr(ucoords), _ptr(mapping), _ptr(inverse),
                             ctypes.byref(st), _stream(dev)), "rhip_hash_build")
    nu = int(st.n_unique)
    order = torch.empty(max(nu, 1), dtype=torch.int32, device=dev)
    pos = torch.empty(max(nu, 1), dtype=torch.int32, device=dev)
    keep = []
    if with_order and nu > 0:
        ows = torch.empty(_sizeq(L.rhip_order_workspace_bytes, nu), dtype=torch.uint8, device=dev)
        bb = ctypes.c_size_t(0)
        _check(L.rhip_brick_bytes(ctypes.byref(st), ctypes.byref(bb)), "rhip_brick_bytes")
        bricks = torch.empty(max(int(bb.value), 1), dtype=torch.uint8, device=dev)
        keep.append(bricks)
        _check(L.rhip_spatial_order(ctypes.byref(st), _ptr(order), _ptr(pos), _ptr(bricks),
                                    int(bb.value), _ptr(ows), ows.numel(), _stream(dev)),
               "rhip_spatial_order")
    elif nu > 0:
        torch.arange(nu, out=order[:nu])
        pos[:nu].copy_(order[:nu])
    return CoordTable(st, slots, ucoords[:nu], mapping[:nu],
                      inverse[:n] if inverse is not None else None, order[:nu], pos[:nu],
                      keep)


def stride_coords(coords: torch.Tensor, out_tensor_stride) -> torch.Tensor:
    """(b, floor(x/s)*s) per row on the GPU."""
    _require_cuda(coords, "coords")
    coords = coords.to(torch.int32).contiguous()
    n, ncol = coords.shape
    s = (ctypes.c_int32 * (ncol - 1))(*[int(v) for v in out_tensor_stride])
    out = torch.empty_like(coords)
    _check(lib().rhip_stride_coords(_ptr(coords), n, ncol, s, _ptr(out), _stream(coords.device)),
           "rhip_stride_coords")
    return out


def expand_coords(coords: torch.Tensor, offsets) -> torch.Tensor:
    """Generative expansion: row i*K + k = coords[i] + offsets[k] (batch
    kept); offsets [K, D] are the region at the output tensor stride. Hash
    the result (hash_build) for the generated output map."""
    _require_cuda(coords, "coords")
    coords = coords.to(torch.int32).contiguous()
    n, ncol = coords.shape
    off = torch.as_tensor(np.asarray(offsets.cpu() if torch.is_tensor(offsets) else offsets),
                          dtype=torch.int32).to(coords.device).contiguous()
    K = off.shape[0]
    if off.dim() != 2 or off.shape[1] != ncol - 1:
        raise RuntimeError("offsets must be [K, D]")
    out = torch.empty((n * K, ncol), dtype=torch.int32, device=coords.device)
    _check(lib().rhip_expand_coords(_ptr(coords), n, ncol, _ptr(off), K, _ptr(out),
                                    _stream(coords.device)), "rhip_expand_coords")
    return out


# ------------------------------------------------------------- kernel maps

class KernelMap:
    """Per-offset (in, out) pairs plus the dense neighbour tables.

    nbr[k, j]   : input row of output position j (output order) or -1
    nbr_t[k, i] : output row of input position i (input order) or -1
    offsets     : CSR over pairs, pairs of offset k at [offsets[k], offsets[k+1])

    The pair lists (in_rows, out_rows) are emitted from nbr on first access
    (rhip_kmap_pairs), at their exact size. A symmetric map (a set onto
    itself, stencil closed under negation) has `partner` (device int32 [K],
    the offset that negates each offset) and no transposed table: its input
    gradient runs on nbr with partner as weight permutation; nbr_t and
    in_order, if read, are built then from nbr's rows.
    """

    def __init__(self, K, n_in, n_out, offsets, offsets_host, in_rows, out_rows, nbr, nbr_t,
                 in_order, out_order, symmetric=False, partner=None, flags=0):
        self.K, self.n_in, self.n_out = K, n_in, n_out
        self.flags = flags  # RHIP_KMAP_* bits reported by rhip_kmap_count
        self.offsets, self.offsets_host = offsets, offsets_host
        self._in_rows, self._out_rows = in_rows, out_rows
        self.nbr, self._nbr_t = nbr, nbr_t
        self._in_order, self.out_order = in_order, out_order
        self.symmetric, self.partner = symmetric, partner

    @property
    def n_pairs(self) -> int:
        return int(self.offsets_host[-1])

    def _build_pairs(self):
        L = lib()
        dev = self.nbr.device
        P = self.n_pairs
        ir = torch.empty(max(P, 1), dtype=torch.int32, device=dev)
        orr = torch.empty(max(P, 1), dtype=torch.int32, device=dev)
        if P > 0:
            ws = torch.empty(_sizeq(L.rhip_kmap_pairs_workspace_bytes, self.n_out, self.K),
                             dtype=torch.uint8, device=dev)
            _check(L.rhip_kmap_pairs(_ptr(self.nbr), _ptr(self.out_order), self.n_out, self.K,
                                     _ptr(self.offsets), _ptr(ws), ws.numel(), _ptr(ir),
                                     _ptr(orr), _stream(dev)), "rhip_kmap_pairs")
        self._in_rows, self._out_rows = ir[:P], orr[:P]

    @property
    def in_rows(self) -> torch.Tensor:
        if self._in_rows is None:
            self._build_pairs()
        return self._in_rows

    @property
    def out_rows(self) -> torch.Tensor:
        if self._out_rows is None:
            self._build_pairs()
        return self._out_rows

    def _build_transposed(self):
        # i pairs with o under k iff o pairs with i under partner[k]
        inv = torch.empty(self.K, dtype=torch.long, device=self.nbr.device)
        inv[self.partner.long()] = torch.arange(self.K, device=self.nbr.device)
        self._nbr_t = self.nbr.index_select(0, inv)
        self._in_order = self.out_order

    @property
    def nbr_t(self) -> torch.Tensor:
        if self._nbr_t is None:
            self._build_transposed()
        return self._nbr_t

    @property
    def in_order(self) -> torch.Tensor:
        if self._in_order is None:
            self._build_transposed()
        return self._in_order

    def swapped(self) -> "KernelMap":
        """Transposed map: in and out exchanged (zero copy once built)."""
        return KernelMap(self.K, self.n_out, self.n_in, self.offsets, self.offsets_host,
                         self.out_rows, self.in_rows, self.nbr_t, self.nbr,
                         self.out_order, self.in_order)

    def pairs(self, k: int):
        a, b = int(self.offsets_host[k]), int(self.offsets_host[k + 1])
        return self.in_rows[a:b], self.out_rows[a:b]


def stencil_partners(offsets) -> Optional[np.ndarray]:
    """The offset that negates each offset of a stencil [K, D] (host), or None
    where the stencil is not closed under negation (rhip_stencil_partners)."""
    off = np.ascontiguousarray(np.asarray(offsets, dtype=np.int32))
    K, D = off.shape
    out = np.empty(K, np.int32)
    st = lib().rhip_stencil_partners(off.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), K, D,
                                     out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
    return out if st == 0 else None


_PARTNERS = {}


def _device_partners(ph: np.ndarray, dev) -> torch.Tensor:
    """A stencil's partner permutation on a device, uploaded once per device
    and permutation and shared (read-only) by the symmetric maps with it. The
    first upload goes from pinned memory on the current stream, ahead of the
    map count's synchronisation."""
    key = (torch.device(dev).index, ph.tobytes())
    t = _PARTNERS.get(key)
    if t is None:
        t = torch.from_numpy(ph).pin_memory().to(dev, non_blocking=True)
        _PARTNERS[key] = t
    return t


def kernel_map(in_table: CoordTable, out_table: CoordTable, offsets) -> KernelMap:
    """Pairs (in, out) with coord(in) = coord(out) + offsets[k] (batch kept),
    the dense neighbour tables and the processing orders of both sides.
    offsets: [K, D] int32 (numpy or tensor; read on the host). The pair
    lists are built when first read; a symmetric map builds no transposed
    table (see KernelMap)."""
    L = lib()
    dev = in_table.ucoords.device
    offsets = torch.as_tensor(np.asarray(offsets.cpu() if torch.is_tensor(offsets) else offsets),
                              dtype=torch.int32).contiguous()
    K = offsets.shape[0]
    if offsets.dim() != 2 or offsets.shape[1] != in_table.ncol - 1:
        raise RuntimeError("offsets must be [K, D]")
    if out_table.ncol != in_table.ncol:
        raise RuntimeError("input and output maps have different coordinate widths")
    n_out, n_in = out_table.n, in_table.n
    st = _stream(dev)
    nbr = torch.empty((K, max(n_out, 1)), dtype=torch.int32, device=dev)
    out_order = torch.empty(max(n_out, 1), dtype=torch.int32, device=dev)
    ws = torch.empty(_sizeq(L.rhip_kmap_workspace_bytes, n_in, n_out, K), dtype=torch.uint8,
                     device=dev)
    kofs = torch.empty(K + 1, dtype=torch.int64, device=dev)
    flags = ctypes.c_int32(0)
    off_host = offsets.numpy()
    # a map of a table onto itself whose stencil is closed under negation is
    # symmetric (the count confirms it): its partners go to the device ahead
    # of the count, which then waits for that copy with its own kernels
    nbr_t = in_order = partner = None
    if out_table is in_table:
        ph = stencil_partners(off_host)
        if ph is not None:
            partner = _device_partners(ph, dev)
    # the one read-back: the count synchronises and fills kofs_host
    kofs_host = np.empty(K + 1, np.int64)
    _check(L.rhip_kmap_count(ctypes.byref(in_table.struct), _ptr(out_table.ucoords),
                             _ptr(out_table.order), n_out, K,
                             off_host.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), _ptr(ws),
                             ws.numel(), _ptr(nbr), _ptr(out_order), _ptr(kofs),
                             kofs_host.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                             ctypes.byref(flags), st), "rhip_kmap_count")
    symmetric = bool(flags.value & KMAP_SYMMETRIC)
    if symmetric and partner is None:
        partner = _device_partners(stencil_partners(off_host), dev)
    if not symmetric:
        partner = None
        nbr_t = torch.empty((K, max(n_in, 1)), dtype=torch.int32, device=dev)
        in_order = torch.empty(max(n_in, 1), dtype=torch.int32, device=dev)
        _check(L.rhip_kmap_fill(_ptr(nbr), _ptr(out_order), n_out, K, _ptr(in_table.order),
                                n_in, flags.value, _ptr(ws), ws.numel(), _ptr(kofs), None, None,
                                _ptr(nbr_t), _ptr(in_order), st), "rhip_kmap_fill")
        nbr_t, in_order = nbr_t[:, :n_in], in_order[:n_in]
    return KernelMap(K, n_in, n_out, kofs, kofs_host, None, None, nbr[:, :n_out], nbr_t,
                     in_order, out_order[:n_out], symmetric=symmetric, partner=partner,
                     flags=flags.value)


# ------------------------------------------------------------ convolution

def _conv_ws(K, cin, cout, dtype, dev, kmap: "KernelMap") -> torch.Tensor:
    return torch.empty(_sizeq(lib().rhip_conv_workspace_bytes, K, cin, cout, dtype, kmap.n_in,
                              kmap.n_out, kmap.n_pairs), dtype=torch.uint8, device=dev)


def _conv_fwd_ws(K, cin, cout, dtype, dev, kmap: "KernelMap") -> torch.Tensor:
    """Workspace of the forward, input-gradient and bias-gradient calls."""
    return torch.empty(_sizeq(lib().rhip_conv_forward_workspace_bytes, K, cin, cout, dtype,
                              kmap.n_in, kmap.n_out), dtype=torch.uint8, device=dev)


def conv_bias_grad(grad_y: torch.Tensor) -> torch.Tensor:
    """Column sums of grad_y in fp32 (the bias gradient) via rhip_conv_bias_grad."""
    _require_cuda(grad_y, "grad_y")
    grad_y = grad_y.contiguous()
    n, C = grad_y.shape
    gb = torch.empty(C, dtype=torch.float32, device=grad_y.device)
    ws = torch.empty(_sizeq(lib().rhip_conv_forward_workspace_bytes, 1, 1, C,
                            _dtype_code(grad_y.dtype), 0, n), dtype=torch.uint8,
                     device=grad_y.device)
    _check(lib().rhip_conv_bias_grad(_ptr(grad_y), n, C, _dtype_code(grad_y.dtype), _ptr(gb),
                                     _ptr(ws), ws.numel(), _stream(grad_y.device)),
           "rhip_conv_bias_grad")
    return gb


def conv_forward(x: torch.Tensor, weight: torch.Tensor, kmap: KernelMap,
                 bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Y[out] = sum_k X[in_k] @ W[k] (+ bias) through rhip_conv_forward."""
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x = x.contiguous()
    weight = weight.to(x.dtype).contiguous()
    K, cin, cout = weight.shape
    if K != kmap.K or x.shape[1] != cin or x.shape[0] != kmap.n_in:
        raise RuntimeError("shape mismatch between features, weight and kernel map")
    b = None if bias is None else bias.reshape(-1).to(torch.float32).contiguous()
    y = torch.empty((kmap.n_out, cout), dtype=x.dtype, device=x.device)
    ws = _conv_fwd_ws(K, cin, cout, dt, x.device, kmap)
    _check(lib().rhip_conv_forward(_ptr(x), kmap.n_in, cin, _ptr(weight), K, cout, _ptr(b),
                                   _ptr(kmap.nbr), _ptr(kmap.out_order), kmap.n_out, _ptr(y),
                                   dt, _ptr(ws), ws.numel(), _stream(x.device)),
           "rhip_conv_forward")
    return y


def conv_forward_noalloc(x: torch.Tensor, weight: torch.Tensor, kmap: KernelMap,
                         bias: Optional[torch.Tensor] = None,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The forward through rhip_conv_forward_noalloc (the library's own
    device scratch instead of a workspace). `out` may be given so that the
    call itself allocates nothing.

    Nothing is converted here (a conversion would allocate): x and weight
    must be contiguous and of one dtype, bias (if any) a contiguous fp32
    vector of cout values and out a contiguous [n_out, cout] tensor of x's
    dtype, all on x's device; anything else raises ValueError before the
    library is called."""
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    if weight.dim() != 3:
        raise ValueError("weight must be [K, cin, cout]")
    K, cin, cout = weight.shape
    if K != kmap.K or x.dim() != 2 or x.shape[1] != cin or x.shape[0] != kmap.n_in:
        raise RuntimeError("shape mismatch between features, weight and kernel map")
    if weight.dtype != x.dtype:
        raise ValueError(f"weight dtype {weight.dtype} differs from x dtype {x.dtype}")
    for name, t in (("x", x), ("weight", weight)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if t.device != x.device:
            raise ValueError(f"{name} must be on {x.device}")
    if bias is not None:
        if (bias.dtype != torch.float32 or not bias.is_contiguous() or bias.numel() != cout
                or bias.device != x.device):
            raise ValueError(f"bias must be a contiguous fp32 tensor of {cout} values on "
                             f"{x.device}")
    if out is None:
        out = torch.empty((kmap.n_out, cout), dtype=x.dtype, device=x.device)
    elif (out.dtype != x.dtype or tuple(out.shape) != (kmap.n_out, cout)
          or not out.is_contiguous() or out.device != x.device):
        raise ValueError(f"out must be a contiguous [{kmap.n_out}, {cout}] {x.dtype} tensor "
                         f"on {x.device}")
    _check(lib().rhip_conv_forward_noalloc(_ptr(x), kmap.n_in, cin, _ptr(weight), K, cout,
                                           _ptr(bias), _ptr(kmap.nbr), _ptr(kmap.out_order),
                                           kmap.n_out, _ptr(out), dt, _stream(x.device)),
           "rhip_conv_forward_noalloc")
    return out


def conv_backward_input(grad_y: torch.Tensor, weight: torch.Tensor, kmap: KernelMap) -> torch.Tensor:
    _require_cuda(grad_y, "grad_y")
    dt = _dtype_code(grad_y.dtype)
    grad_y = grad_y.contiguous()
    weight = weight.to(grad_y.dtype).contiguous()
    K, cin, cout = weight.shape
    gx = torch.empty((kmap.n_in, cin), dtype=grad_y.dtype, device=grad_y.device)
    ws = _conv_fwd_ws(K, cin, cout, dt, grad_y.device, kmap)
    if kmap.symmetric:  # nbr with the stencil partners as weight permutation
        table, perm, order = kmap.nbr, kmap.partner, kmap.out_order
    else:
        table, perm, order = kmap.nbr_t, None, kmap.in_order
    _check(lib().rhip_conv_backward_input(_ptr(grad_y), kmap.n_out, cout, _ptr(weight), K, cin,
                                          _ptr(table), _ptr(perm), _ptr(order), kmap.n_in,
                                          _ptr(gx), dt, _ptr(ws), ws.numel(),
                                          _stream(grad_y.device)), "rhip_conv_backward_input")
    return gx


def conv_backward_weight(x: torch.Tensor, grad_y: torch.Tensor, kmap: KernelMap,
                         K: int, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x, grad_y = x.contiguous(), grad_y.to(x.dtype).contiguous()
    cin, cout = x.shape[1], grad_y.shape[1]
    gw = torch.empty((K, cin, cout), dtype=x.dtype, device=x.device)
    ws = _conv_ws(K, cin, cout, dt, x.device, kmap)
    _check(lib().rhip_conv_backward_weight(_ptr(x), kmap.n_in, cin, _ptr(grad_y), kmap.n_out,
                                           cout, K, _ptr(kmap.offsets), kmap.n_pairs,
                                           _ptr(kmap.in_rows), _ptr(kmap.out_rows), _ptr(gw),
                                           dt, _ptr(ws), ws.numel(), _stream(x.device)),
           "rhip_conv_backward_weight")
    return gw if out_dtype is None else gw.to(out_dtype)


RHIP_ERR_UNSUPPORTED = 3


def conv_weight_grad(x: torch.Tensor, grad_y: torch.Tensor, kmap: KernelMap,
                     K: int) -> torch.Tensor:
    """dW as the convolution layer computes it: from the neighbour table where
    the library has a kernel for the shape, else from the pair list. bf16
    maps of at most 8 offsets also take the pair list, which is faster there,
    when they hold fewer than 2 pairs per output row (a transposed stride-2
    map: one neighbour per row) or pair each input row at most once (a
    stride-2 map) with channel counts that are multiples of 64."""
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x, grad_y = x.contiguous(), grad_y.to(x.dtype).contiguous()
    cin, cout = x.shape[1], grad_y.shape[1]
    gw = torch.empty((K, cin, cout), dtype=x.dtype, device=x.device)
    ws = _conv_ws(K, cin, cout, dt, x.device, kmap)
    st = RHIP_ERR_UNSUPPORTED
    pair_list = x.dtype == torch.bfloat16 and K <= 8 and (
        kmap.n_pairs < 2 * kmap.n_out
        or (kmap.n_pairs <= kmap.n_in and cin % 64 == 0 and cout % 64 == 0))
    if not pair_list:
        st = lib().rhip_conv_backward_weight_rows(_ptr(x), kmap.n_in, cin, _ptr(grad_y),
                                                  kmap.n_out, cout, K, _ptr(kmap.nbr),
                                                  _ptr(kmap.out_order), _ptr(gw), dt, _ptr(ws),
                                                  ws.numel(), _stream(x.device))
    if st == RHIP_ERR_UNSUPPORTED:
        st = lib().rhip_conv_backward_weight(_ptr(x), kmap.n_in, cin, _ptr(grad_y), kmap.n_out,
                                             cout, K, _ptr(kmap.offsets), kmap.n_pairs,
                                             _ptr(kmap.in_rows), _ptr(kmap.out_rows), _ptr(gw),
                                             dt, _ptr(ws), ws.numel(), _stream(x.device))
    _check(st, "rhip_conv_backward_weight(_rows)")
    return gw


def conv_backward_weight_rows(x: torch.Tensor, grad_y: torch.Tensor, kmap: KernelMap,
                              K: int) -> torch.Tensor:
    """dW from the kernel map's neighbour table (bf16 with 16 or 32 channels;
    K <= 8 or K >= 20 with cin % 16 == 0 and cout % 32 == 0; other shapes
    raise)."""
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x, grad_y = x.contiguous(), grad_y.to(x.dtype).contiguous()
    cin, cout = x.shape[1], grad_y.shape[1]
    gw = torch.empty((K, cin, cout), dtype=x.dtype, device=x.device)
    ws = _conv_ws(K, cin, cout, dt, x.device, kmap)
    _check(lib().rhip_conv_backward_weight_rows(_ptr(x), kmap.n_in, cin, _ptr(grad_y),
                                                kmap.n_out, cout, K, _ptr(kmap.nbr),
                                                _ptr(kmap.out_order), _ptr(gw), dt, _ptr(ws),
                                                ws.numel(), _stream(x.device)),
           "rhip_conv_backward_weight_rows")
    return gw


# ---------------------------------------------------------------- pooling

def stride_map(in_table: CoordTable, out_table: CoordTable, out_tensor_stride) -> KernelMap:
    """Pooling stride map (kernel size == stride): every input row onto the
    output row of its floor-aligned coordinates, in the neighbour-table form
    (nbr: K = largest number of inputs on one output rows; nbr_t: one row).
    The pair list is the reference's single offset: offsets = [0, P]."""
    L = lib()
    dev = in_table.ucoords.device
    n_in, n_out = in_table.n, out_table.n
    s = (ctypes.c_int32 * MAX_COLS)(*[int(v) for v in out_tensor_stride])
    st = _stream(dev)
    ws = torch.empty(_sizeq(L.rhip_stride_map_workspace_bytes, n_in, n_out), dtype=torch.uint8,
                     device=dev)
    kmax = ctypes.c_int32(0)
    _check(L.rhip_stride_map_count(ctypes.byref(out_table.struct), _ptr(in_table.ucoords), n_in,
                                   s, _ptr(ws), ws.numel(), ctypes.byref(kmax), st),
           "rhip_stride_map_count")
    K = max(int(kmax.value), 1)
    # phase 2 writes every entry of the tables (-1 where no input lies)
    table = torch.empty if kmax.value > 0 else (lambda *a, **k: torch.full(*a, -1, **k))
    nbr = table((K, max(n_out, 1)), dtype=torch.int32, device=dev)
    nbr_t = table((1, max(n_in, 1)), dtype=torch.int32, device=dev)
    in_rows = torch.empty(max(n_in, 1), dtype=torch.int32, device=dev)
    out_rows = torch.empty(max(n_in, 1), dtype=torch.int32, device=dev)
    _check(L.rhip_stride_map_fill(n_in, n_out, int(kmax.value), _ptr(in_table.order),
                                  _ptr(out_table.order), _ptr(ws), ws.numel(), _ptr(nbr),
                                  _ptr(nbr_t), _ptr(in_rows), _ptr(out_rows), st),
           "rhip_stride_map_fill")
    kofs_host = np.array([0, n_in], dtype=np.int64)
    return KernelMap(K, n_in, n_out, torch.as_tensor(kofs_host).to(dev), kofs_host,
                     in_rows[:n_in], out_rows[:n_in], nbr[:, :n_out], nbr_t[:, :n_in],
                     in_table.order, out_table.order)


def group_map(group: torch.Tensor, n_groups: int) -> KernelMap:
    """Rows grouped by a given group id (e.g. a hash build's inverse map), in
    the stride map's form: nbr [K, n_groups] (rows of each group ascending,
    K = largest group), nbr_t [1, n] (each row's group), row order."""
    _require_cuda(group, "group")
    L = lib()
    dev = group.device
    group = group.to(torch.int32).contiguous()
    n = group.shape[0]
    st = _stream(dev)
    ws = torch.empty(_sizeq(L.rhip_stride_map_workspace_bytes, n, n_groups), dtype=torch.uint8,
                     device=dev)
    kmax = ctypes.c_int32(0)
    _check(L.rhip_group_map_count(_ptr(group), n, n_groups, _ptr(ws), ws.numel(),
                                  ctypes.byref(kmax), st), "rhip_group_map_count")
    K = max(int(kmax.value), 1)
    table = torch.empty if kmax.value > 0 else (lambda *a, **k: torch.full(*a, -1, **k))
    nbr = table((K, max(n_groups, 1)), dtype=torch.int32, device=dev)
    nbr_t = table((1, max(n, 1)), dtype=torch.int32, device=dev)
    in_rows = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    out_rows = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    _check(L.rhip_stride_map_fill(n, n_groups, int(kmax.value), None, None, _ptr(ws), ws.numel(),
                                  _ptr(nbr), _ptr(nbr_t), _ptr(in_rows), _ptr(out_rows), st),
           "rhip_stride_map_fill")
    kofs_host = np.array([0, n], dtype=np.int64)
    iota = lambda m: torch.arange(m, dtype=torch.int32, device=dev)  # noqa: E731
    return KernelMap(K, n, n_groups, torch.as_tensor(kofs_host).to(dev), kofs_host, in_rows[:n],
                     out_rows[:n], nbr[:, :n_groups], nbr_t[:, :n], iota(n), iota(n_groups))


def table_compact(table: torch.Tensor) -> torch.Tensor:
    """Pooling form of a neighbour table [K, n]: each column's entries moved
    to its first rows; returns the rows in use [k_used, n] (at least one)."""
    _require_cuda(table, "table")
    table = table.contiguous()
    K, n = table.shape
    out = torch.empty_like(table)
    ws = torch.empty(256, dtype=torch.uint8, device=table.device)
    used = ctypes.c_int32(0)
    _check(lib().rhip_table_compact(_ptr(table), K, n, _ptr(ws), ws.numel(), _ptr(out),
                                    ctypes.byref(used), _stream(table.device)),
           "rhip_table_compact")
    return out[:max(int(used.value), 1)]


def pooling_map(kmap: KernelMap) -> KernelMap:
    """A kernel map for pooling: its transposed table compacted (the input
    side of a strided pooling map has few of the K offsets)."""
    return KernelMap(kmap.K, kmap.n_in, kmap.n_out, kmap.offsets, kmap.offsets_host,
                     kmap._in_rows, kmap._out_rows, kmap.nbr, table_compact(kmap.nbr_t),
                     kmap.in_order, kmap.out_order)


def _pool_mode(mode) -> int:
    if isinstance(mode, str):
        return POOL_MODES[mode]
    return int(mode)


def pool_forward(x: torch.Tensor, kmap: KernelMap, mode="avg"):
    """(y [n_out, C], counts [n_out]) of local pooling over kmap.nbr."""
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x = x.contiguous()
    if x.shape[0] != kmap.n_in:
        raise RuntimeError("features do not match the map's input rows")
    C = x.shape[1]
    y = torch.empty((kmap.n_out, C), dtype=x.dtype, device=x.device)
    counts = torch.empty(max(kmap.n_out, 1), dtype=torch.int32, device=x.device)
    _check(lib().rhip_pool_forward(_ptr(x), kmap.n_in, C, _ptr(kmap.nbr), kmap.nbr.shape[0],
                                   _ptr(kmap.out_order), kmap.n_out, _pool_mode(mode), _ptr(y),
                                   _ptr(counts), dt, _stream(x.device)), "rhip_pool_forward")
    return y, counts[:kmap.n_out]


def pool_backward(grad_y: torch.Tensor, y: torch.Tensor, x: torch.Tensor, kmap: KernelMap,
                  counts: torch.Tensor, mode="avg") -> torch.Tensor:
    _require_cuda(grad_y, "grad_y")
    dt = _dtype_code(x.dtype)
    m = _pool_mode(mode)
    grad_y, y, x = grad_y.to(x.dtype).contiguous(), y.contiguous(), x.contiguous()
    C = x.shape[1]
    gx = torch.empty((kmap.n_in, C), dtype=x.dtype, device=x.device)
    ws = torch.empty(_sizeq(lib().rhip_pool_workspace_bytes, kmap.n_out, C, m),
                     dtype=torch.uint8, device=x.device)
    _check(lib().rhip_pool_backward(_ptr(grad_y), _ptr(y), _ptr(x), kmap.n_out, C,
                                    _ptr(kmap.nbr), kmap.nbr.shape[0], _ptr(kmap.out_order),
                                    _ptr(kmap.nbr_t), kmap.nbr_t.shape[0],
                                    _ptr(kmap.in_order), kmap.n_in, _ptr(counts), m, _ptr(gx),
                                    dt, _ptr(ws), ws.numel(), _stream(x.device)),
           "rhip_pool_backward")
    return gx


@dataclass
class BatchSegments:
    """Rows grouped by batch: rows of batch b are members[seg[b]:seg[b+1]]."""
    n_batches: int
    members: torch.Tensor
    seg: torch.Tensor


def batch_segments(coords: torch.Tensor) -> BatchSegments:
    _require_cuda(coords, "coords")
    L = lib()
    coords = coords.to(torch.int32).contiguous()
    n, ncol = coords.shape
    dev = coords.device
    ws = torch.empty(_sizeq(L.rhip_global_pool_workspace_bytes, n, 1, 0), dtype=torch.uint8,
                     device=dev)
    B = ctypes.c_int32(0)
    _check(L.rhip_batch_count(_ptr(coords), n, ncol, _ptr(ws), ws.numel(), ctypes.byref(B),
                              _stream(dev)), "rhip_batch_count")
    members = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    seg = torch.empty(B.value + 1, dtype=torch.int32, device=dev)
    _check(L.rhip_batch_segments(_ptr(coords), n, ncol, B.value, _ptr(ws), ws.numel(),
                                 _ptr(members), _ptr(seg), _stream(dev)), "rhip_batch_segments")
    return BatchSegments(int(B.value), members[:n], seg)


def global_pool_forward(x: torch.Tensor, segs: BatchSegments, mode="avg") -> torch.Tensor:
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x = x.contiguous()
    n, C = x.shape
    y = torch.empty((segs.n_batches, C), dtype=x.dtype, device=x.device)
    ws = torch.empty(_sizeq(lib().rhip_global_pool_workspace_bytes, n, C, segs.n_batches),
                     dtype=torch.uint8, device=x.device)
    _check(lib().rhip_global_pool_forward(_ptr(x), n, C, _ptr(segs.members), _ptr(segs.seg),
                                          segs.n_batches, _pool_mode(mode), _ptr(y), dt,
                                          _ptr(ws), ws.numel(), _stream(x.device)),
           "rhip_global_pool_forward")
    return y


def global_pool_backward(grad_y: torch.Tensor, y: torch.Tensor, x: torch.Tensor,
                         coords: torch.Tensor, segs: BatchSegments, mode="avg") -> torch.Tensor:
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    grad_y, y, x = grad_y.to(x.dtype).contiguous(), y.contiguous(), x.contiguous()
    coords = coords.to(torch.int32).contiguous()
    n, C = x.shape
    gx = torch.empty((n, C), dtype=x.dtype, device=x.device)
    ws = torch.empty(_sizeq(lib().rhip_global_pool_workspace_bytes, n, C, segs.n_batches),
                     dtype=torch.uint8, device=x.device)
    _check(lib().rhip_global_pool_backward(_ptr(grad_y), _ptr(y), _ptr(x), _ptr(coords),
                                           coords.shape[1], n, C, _ptr(segs.members),
                                           _ptr(segs.seg), segs.n_batches, _pool_mode(mode),
                                           _ptr(gx), dt, _ptr(ws), ws.numel(),
                                           _stream(x.device)), "rhip_global_pool_backward")
    return gx


def bn_stats(x: torch.Tensor, eps: float = 1e-5, momentum: float = 0.1,
             running_mean: Optional[torch.Tensor] = None,
             running_var: Optional[torch.Tensor] = None):
    """(mean, invstd) fp32 [C] of x's batch statistics; the running
    statistics, when given (fp32 [C], contiguous), are updated in place."""
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x = x.contiguous()
    n, C = x.shape
    f32 = dict(dtype=torch.float32, device=x.device)
    mean, invstd = torch.empty(C, **f32), torch.empty(C, **f32)
    ws = torch.empty(_sizeq(lib().rhip_bn_workspace_bytes, n, C), dtype=torch.uint8,
                     device=x.device)
    _check(lib().rhip_bn_stats(_ptr(x), n, C, dt, eps, momentum, _ptr(running_mean),
                               _ptr(running_var), _ptr(mean), _ptr(invstd), _ptr(ws),
                               ws.numel(), _stream(x.device)), "rhip_bn_stats")
    return mean, invstd


def bn_invstd(var: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    _require_cuda(var, "var")
    var = var.float().contiguous()
    out = torch.empty_like(var)
    _check(lib().rhip_bn_invstd(_ptr(var), var.numel(), eps, _ptr(out), _stream(var.device)),
           "rhip_bn_invstd")
    return out


def bn_forward(x: torch.Tensor, mean: torch.Tensor, invstd: torch.Tensor,
               gamma: Optional[torch.Tensor] = None, beta: Optional[torch.Tensor] = None,
               residual: Optional[torch.Tensor] = None, relu: bool = False) -> torch.Tensor:
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x = x.contiguous()
    n, C = x.shape
    if residual is not None:
        residual = residual.to(x.dtype).contiguous()
        if residual.shape != x.shape:
            raise RuntimeError("residual does not match the features")
    y = torch.empty_like(x)
    _check(lib().rhip_bn_forward(_ptr(x), n, C, _ptr(mean), _ptr(invstd), _ptr(gamma),
                                 _ptr(beta), _ptr(residual), int(relu), _ptr(y), dt,
                                 _stream(x.device)), "rhip_bn_forward")
    return y


def bn_backward(grad_y: torch.Tensor, y: Optional[torch.Tensor], x: torch.Tensor,
                mean: torch.Tensor, invstd: torch.Tensor, gamma: Optional[torch.Tensor] = None,
                relu: bool = False, batch_stats: bool = True, want_residual: bool = False):
    """(grad_x, grad_residual or None, grad_gamma, grad_beta)."""
    _require_cuda(x, "x")
    dt = _dtype_code(x.dtype)
    x = x.contiguous()
    grad_y = grad_y.to(x.dtype).contiguous()
    y = None if y is None else y.contiguous()
    n, C = x.shape
    gx = torch.empty_like(x)
    gr = torch.empty_like(x) if want_residual else None
    f32 = dict(dtype=torch.float32, device=x.device)
    gg, gb = torch.empty(C, **f32), torch.empty(C, **f32)
    ws = torch.empty(_sizeq(lib().rhip_bn_workspace_bytes, n, C), dtype=torch.uint8,
                     device=x.device)
    _check(lib().rhip_bn_backward(_ptr(grad_y), _ptr(y), _ptr(x), n, C, _ptr(mean),
                                  _ptr(invstd), _ptr(gamma), int(relu), int(batch_stats),
                                  _ptr(gx), _ptr(gr), _ptr(gg), _ptr(gb), dt, _ptr(ws),
                                  ws.numel(), _stream(x.device)), "rhip_bn_backward")
    return gx, gr, gg, gb
