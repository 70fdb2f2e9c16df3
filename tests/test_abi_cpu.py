"""The C-ABI library loads and exports exactly what include/riemann_hip.h
declares; argument validation works without a GPU. No kernels run here."""
import ctypes
import os
import re
import subprocess

import pytest

from riemannengine_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "riemann_hip.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return set(re.findall(r"\b(rhip_[a-z0-9_]+)\s*\(", txt))


def test_library_exports_every_declared_symbol():
    L = abi.lib()
    declared = _declared()
    assert declared == set(abi.EXPORTS)
    for name in declared:
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", abi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (rhip_[a-z0-9_]+)", out))
    assert exported == declared


def test_abi_version_and_struct_layout():
    assert abi.lib().rhip_abi_version() == 13
    # void*, int64, void*, int64, 3 x int32, 4 x int32[8] (172 bytes, padded to 176),
    # 2 x void*, 2 x int32, int32[8] -> 232 bytes
    assert ctypes.sizeof(abi.RhipTable) == 232


def test_workspace_queries():
    L = abi.lib()
    assert abi._sizeq(L.rhip_hash_workspace_bytes, 1000, 4) > 1000 * 8
    # per-wave hit counts and their scans for each offset, the mask sort's keys
    # and values (two pairs)
    assert abi._sizeq(L.rhip_kmap_workspace_bytes, 1000, 1000, 27) > 27 * 16 * 12 + 4 * 1000 * 4
    # transposed weights + fp32 accumulator, plus the dW partial tiles
    base = 27 * 64 * 64 * (2 + 4)
    assert abi._sizeq(L.rhip_conv_workspace_bytes, 27, 64, 64, abi.BF16, 1000, 1000, 0) >= base
    assert abi._sizeq(L.rhip_conv_workspace_bytes, 27, 64, 64, abi.BF16, 10**5, 10**5,
                      10**6) > base
    # few rows, wide channels: fp32 partial sums of the split offset axis
    wide = abi._sizeq(L.rhip_conv_workspace_bytes, 27, 256, 256, abi.BF16, 1000, 1000, 0)
    assert wide >= 27 * 256 * 256 * (2 + 4) + 2 * 1000 * 256 * 4
    assert L.rhip_table_bytes(100) == 256 * 16  # next power of two >= 2n, 16 B slots
    # forward / dX / dbias alone: transposed weights and the bias chunk sums,
    # without the dW partial tiles and accumulator behind them
    fwd = abi._sizeq(L.rhip_conv_forward_workspace_bytes, 27, 64, 64, abi.BF16, 10**5, 10**5)
    full = abi._sizeq(L.rhip_conv_workspace_bytes, 27, 64, 64, abi.BF16, 10**5, 10**5, 10**6)
    assert 27 * 64 * 64 * 2 + 256 * 64 * 4 <= fwd < full - 27 * 64 * 64 * 4


@pytest.mark.parametrize("call,msg", [
    (lambda L, t: L.rhip_hash_build(None, 10, 1, None, 0, None, 0, None, None, None,
                                    ctypes.byref(t), None), "ncol"),
    (lambda L, t: L.rhip_hash_build(None, -1, 4, None, 0, None, 0, None, None, None,
                                    ctypes.byref(t), None), "row count"),
    (lambda L, t: L.rhip_kmap_count(ctypes.byref(t), None, None, 10, 0, None, None, 0, None,
                                    None, None, None, None, None), "K must"),
    (lambda L, t: L.rhip_conv_forward(None, 1, 4, None, 27, 8, None, None, None, 1, None, 7,
                                      None, 0, None), "dtype"),
])
def test_invalid_arguments_are_reported(call, msg):
    L = abi.lib()
    t = abi.RhipTable()
    status = call(L, t)
    assert status != 0
    assert msg in L.rhip_last_error().decode()


def test_cpu_tensors_are_rejected():
    import torch
    with pytest.raises(RuntimeError, match="device tensor"):
        abi.hash_build(torch.zeros((4, 4), dtype=torch.int32))


def test_stencil_partners_and_rows_query_without_a_gpu():
    """rhip_stencil_partners (host only): the 3^3 cube's offsets negate in
    reverse enumeration order (k -> 26 - k), the cross stencil pairs +r with
    -r, the even 2^3 cube has no partners; rhip_conv_backward_weight_rows_
    supported answers without a GPU."""
    import numpy as np
    import oracle
    p = abi.stencil_partners(oracle.region_offsets(3, 3))
    assert p is not None and list(p) == list(range(26, -1, -1))
    off = oracle.region_offsets(3, 5, region="cross")
    p = abi.stencil_partners(off)
    assert p is not None and np.array_equal(off[p], -off)
    assert abi.stencil_partners(oracle.region_offsets(3, 2)) is None
    assert abi.stencil_partners(np.array([[1, 0], [-1, 0], [1, 0]], np.int32)) is None
    L = abi.lib()
    assert L.rhip_conv_backward_weight_rows_supported(abi.F32, 64, 64, 27, 1000, 1000) == 1
    assert L.rhip_conv_backward_weight_rows_supported(abi.F32, 64, 64, 13, 1000, 1000) == 0
    assert L.rhip_conv_backward_weight_rows_supported(abi.BF16, 16, 32, 13, 1000, 1000) == 1
    assert L.rhip_conv_backward_weight_rows_supported(7, 64, 64, 27, 1000, 1000) == 0
