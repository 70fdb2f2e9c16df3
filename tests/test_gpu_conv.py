"""GPU sparse convolution (forward, dX, dW) through the C ABI vs the oracle
(restating engine/ops/convolution_cpu.hpp and engine/nn/conv.cpp:47-64).
Tolerance: norm-wise rel 1e-4 for fp32 and 2e-2 for bf16 (helpers.TOL)."""
import json
import os

import numpy as np
import pytest
import torch

import oracle
from riemannengine_amd import abi, scenes
from helpers import DEV, TOL, assert_rel, to_dev, random_coords, gpu_tables_and_map

pytestmark = pytest.mark.gpu


def _oracle_conv(km, x, w, gy):
    """Oracle forward/backward on the GPU map's own pairs."""
    kofs = km.offsets_host
    ir, orr = km.in_rows.cpu().numpy(), km.out_rows.cpu().numpy()
    y = oracle.conv_forward(x, w, kofs, ir, orr, km.n_out)
    gx, gw = oracle.conv_backward(x, gy, w, kofs, ir, orr)
    return y, gx, gw


def _run_and_check(km, cin, cout, dtype, seed, bias=False, tag=""):
    rng = np.random.default_rng(seed)
    K = km.K
    x = rng.standard_normal((km.n_in, cin)).astype(np.float32)
    w = (rng.standard_normal((K, cin, cout)) / np.sqrt(cin * K)).astype(np.float32)
    gy = rng.standard_normal((km.n_out, cout)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32) if bias else None
    xt, wt, gyt = to_dev(x, dtype), to_dev(w, dtype), to_dev(gy, dtype)
    # the oracle sees exactly the (possibly bf16-rounded) operands
    x64, w64, gy64 = (t.float().cpu().numpy() for t in (xt, wt, gyt))
    print(f"conv {tag} K={K} cin={cin} cout={cout} {dtype} n_in={km.n_in} "
          f"n_out={km.n_out} P={km.n_pairs}", flush=True)
    y = abi.conv_forward(xt, wt, km, bias=None if b is None else to_dev(b))
    gx = abi.conv_backward_input(gyt, wt, km)
    gw = abi.conv_backward_weight(xt, gyt, km, K)
    torch.cuda.synchronize()
    ry, rgx, rgw = _oracle_conv(km, x64, w64, gy64)
    if b is not None:
        ry = ry + b
    tol = TOL[dtype]
    assert_rel(y.float().cpu().numpy(), ry, tol, "forward")
    assert_rel(gx.float().cpu().numpy(), rgx, tol, "dX")
    assert_rel(gw.float().cpu().numpy(), rgw, tol, "dW")


@pytest.mark.parametrize("cin,cout,dtype", [
    (16, 32, torch.float32), (64, 64, torch.float32), (32, 48, torch.float32),
    (128, 64, torch.float32), (64, 256, torch.float32), (3, 5, torch.float32),
    (64, 64, torch.bfloat16), (32, 64, torch.bfloat16), (128, 128, torch.bfloat16),
    (256, 32, torch.bfloat16), (16, 16, torch.bfloat16), (8, 24, torch.bfloat16),
    # bf16 reductions of 16 / 48 channels: padded to the 32-channel MFMA
    (16, 32, torch.bfloat16), (48, 16, torch.bfloat16), (16, 48, torch.bfloat16)])
def test_conv_3x3x3_matches_oracle(cin, cout, dtype):
    rng = np.random.default_rng(cin + cout)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 6000, 3, 12))
    off = oracle.region_offsets(3, 3)
    _, _, km = gpu_tables_and_map(c, c, off, same=True)
    _run_and_check(km, cin, cout, dtype, seed=cin * 7 + cout, tag="3^3")


@pytest.mark.parametrize("extra", [6, 70])
@pytest.mark.parametrize("cin,cout,dtype", [
    (64, 64, torch.float32), (32, 32, torch.float32), (64, 64, torch.bfloat16),
    (128, 128, torch.bfloat16), (32, 64, torch.bfloat16)])
def test_fast_forward_kernel_equals_general_kernel(cin, cout, dtype, extra):
    """Stencils of at most 32 offsets run on the LDS-indexed forward/dX
    kernel with one mask word, those of 33 to 96 on it with three, larger
    ones on the general kernel; all add a row's active offsets in ascending
    order. The 3^3 map and the same map with 6 (K = 33) or 70 (K = 97) more
    offsets that pair nothing must give bit-identical forward and dX (the
    extra weights are never read). The cloud is large enough that no kernel
    splits its offset axis over workgroups (a split changes the order of the
    sums)."""
    rng = np.random.default_rng(cin * 3 + cout)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 60000, 3, 30))
    off = oracle.region_offsets(3, 3)
    far = np.array([[200 + i, 200, 200] for i in range(extra)], np.int32)  # beyond the span
    tin = abi.hash_build(to_dev(c))
    km27 = abi.kernel_map(tin, tin, to_dev(off))
    kmx = abi.kernel_map(tin, tin, to_dev(np.concatenate([off, far])))
    assert kmx.K == 27 + extra and kmx.n_pairs == km27.n_pairs
    x = to_dev(rng.standard_normal((km27.n_in, cin)).astype(np.float32), dtype)
    gy = to_dev(rng.standard_normal((km27.n_out, cout)).astype(np.float32), dtype)
    w = rng.standard_normal((27 + extra, cin, cout)).astype(np.float32) / np.sqrt(cin * 27)
    w27, wx = to_dev(w[:27], dtype), to_dev(w, dtype)
    print(f"fast vs K={27 + extra} kernel cin={cin} cout={cout} {dtype}", flush=True)
    assert torch.equal(abi.conv_forward(x, w27, km27), abi.conv_forward(x, wx, kmx))
    # the 3^3 map is symmetric: its usual input gradient runs on nbr with
    # partner weights (offsets summed in another order); over its transposed
    # table it adds them in ascending order like the K = 33 / 97 map
    assert not kmx.symmetric and km27.symmetric
    assert torch.equal(_dx_over_transposed_table(gy, w27, km27),
                       abi.conv_backward_input(gy, wx, kmx))


def _dx_over_transposed_table(gy, w, km):
    """The input gradient over the map's transposed table (built from nbr's
    rows for a symmetric map) without a weight permutation."""
    K, cin, cout = w.shape
    gx = torch.empty((km.n_in, cin), dtype=gy.dtype, device=gy.device)
    ws = abi._conv_fwd_ws(K, cin, cout, abi._dtype_code(gy.dtype), gy.device, km)
    abi._check(abi.lib().rhip_conv_backward_input(
        abi._ptr(gy), km.n_out, cout, abi._ptr(w), K, cin, abi._ptr(km.nbr_t), None,
        abi._ptr(km.in_order), km.n_in, abi._ptr(gx), abi._dtype_code(gy.dtype), abi._ptr(ws),
        ws.numel(), abi._stream(gy.device)), "rhip_conv_backward_input")
    return gx


def test_conv_bias_fp32():
    rng = np.random.default_rng(1)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 3000, 3, 10))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    _run_and_check(km, 32, 32, torch.float32, seed=3, bias=True, tag="bias")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_offset_split_matches_unsplit_and_oracle(dtype):
    """Few rows with wide channels split the offset axis over workgroups
    (fp32 partial sums reduced in a fixed order, bias added once): forward
    with bias and dX vs the oracle, and dX vs the unsplit kernel (no
    workspace)."""
    rng = np.random.default_rng(21)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 2500, 3, 9))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    _run_and_check(km, 256, 256, dtype, seed=5, bias=True, tag="split")
    g = torch.Generator().manual_seed(3)
    gy = torch.randn(km.n_out, 256, generator=g).to(dtype).to(DEV)
    w = (torch.randn(27, 256, 256, generator=g) / 80).to(dtype).to(DEV)
    split = abi.conv_backward_input(gy, w, km)
    plain = torch.empty_like(split)
    abi._check(abi.lib().rhip_conv_backward_input(
        abi._ptr(gy), km.n_out, 256, abi._ptr(w), 27, 256, abi._ptr(km.nbr_t), None,
        abi._ptr(km.in_order), km.n_in, abi._ptr(plain), abi._dtype_code(dtype), None, 0,
        abi._stream(gy.device)), "rhip_conv_backward_input")
    assert_rel(split.float().cpu().numpy(), plain.float().cpu().numpy(),
               1e-5 if dtype == torch.float32 else 1e-2, "split vs unsplit dX")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv_4d_81_offsets(dtype):
    rng = np.random.default_rng(81)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 8000, 4, 7, batch=1))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(4, 3), same=True)
    _run_and_check(km, 32, 32, dtype, seed=4, tag="3^4")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_strided_and_transposed(dtype):
    """2^3 s2 down (C64->128) then the transposed 2^3 s2 up (C128->64) over the
    swapped map, as config 3 runs them."""
    rng = np.random.default_rng(23)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 30))
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    km = abi.kernel_map(tin, tout, to_dev(oracle.region_offsets(3, 2)))
    _run_and_check(km, 64, 128, dtype, seed=5, tag="down")
    _run_and_check(km.swapped(), 128, 64, dtype, seed=6, tag="up")


def test_stride2_dw_dispatch_bf16():
    """bf16 2^3 stride-2 maps pair each input row once: with channel counts
    that are multiples of 64 the dispatch (abi.conv_weight_grad, as the host
    layer) takes the per-wave pair-list kernel, else the neighbour table;
    both against the oracle."""
    rng = np.random.default_rng(31)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 12))  # about half the cells
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    km = abi.kernel_map(tin, tout, to_dev(oracle.region_offsets(3, 2)))
    assert km.n_pairs == km.n_in and km.n_pairs >= 2 * km.n_out
    g = torch.Generator().manual_seed(3)
    for cin, cout, path in ((64, 128, "pairs"), (128, 64, "pairs"), (32, 64, "rows")):
        x = torch.randn(km.n_in, cin, generator=g).to(torch.bfloat16).to(DEV)
        gy = torch.randn(km.n_out, cout, generator=g).to(torch.bfloat16).to(DEV)
        print(f"stride-2 dW dispatch {cin}->{cout}", flush=True)
        got = abi.conv_weight_grad(x, gy, km, 8)
        want = (abi.conv_backward_weight(x, gy, km, 8) if path == "pairs"
                else abi.conv_backward_weight_rows(x, gy, km, 8))
        assert torch.equal(got, want), path
        _, _, rgw = _oracle_conv(km, x.float().cpu().numpy(),
                                 np.zeros((8, cin, cout), np.float32), gy.float().cpu().numpy())
        assert_rel(got.float().cpu().numpy(), rgw, TOL[torch.bfloat16], f"{cin}->{cout} dW")


@pytest.mark.parametrize("npts,cin,cout", [(1, 64, 64), (33, 64, 128), (65, 128, 64),
                                           (700, 192, 64), (3000, 64, 192)])
def test_pair_list_dw_bf16_tiles_small_maps(npts, cin, cout):
    """The per-wave pair-list dW (bf16, 64-channel tiles) where offsets hold
    no pairs, fewer than one 32-pair step or a few steps, and with 3 tiles
    per axis, against the oracle on the map's own pairs; repeat calls are
    bitwise equal."""
    rng = np.random.default_rng(npts + cin)
    c, _, _ = oracle.insert_and_map(random_coords(rng, npts, 3, 4 if npts < 100 else 9))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    g = torch.Generator().manual_seed(npts)
    x = torch.randn(km.n_in, cin, generator=g).to(torch.bfloat16).to(DEV)
    gy = torch.randn(km.n_out, cout, generator=g).to(torch.bfloat16).to(DEV)
    print(f"pair-list dW bf16 {cin}->{cout} n={km.n_in} P={km.n_pairs}", flush=True)
    gw = abi.conv_backward_weight(x, gy, km, km.K)
    assert torch.equal(gw, abi.conv_backward_weight(x, gy, km, km.K))
    _, _, rgw = _oracle_conv(km, x.float().cpu().numpy(),
                             np.zeros((km.K, cin, cout), np.float32), gy.float().cpu().numpy())
    assert_rel(gw.float().cpu().numpy(), rgw, TOL[torch.bfloat16], f"{npts} {cin}->{cout} dW")


def _rows_check(km, cin, cout, seed, tag, dtype=torch.bfloat16):
    """dW from the neighbour table vs the oracle on the map's own pairs (the
    oracle sees the operands rounded to dtype) and vs the pair-list kernel."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(km.n_in, cin, generator=g).to(dtype).to(DEV)
    gy = torch.randn(km.n_out, cout, generator=g).to(dtype).to(DEV)
    print(f"dW rows {tag} {dtype} cin={cin} cout={cout} n_in={km.n_in} n_out={km.n_out}",
          flush=True)
    rows = abi.conv_backward_weight_rows(x, gy, km, km.K)
    pairs = abi.conv_backward_weight(x, gy, km, km.K)
    _, _, rgw = _oracle_conv(km, x.float().cpu().numpy(),
                             np.zeros((km.K, cin, cout), np.float32), gy.float().cpu().numpy())
    assert_rel(rows.float().cpu().numpy(), rgw, TOL[dtype], f"{tag} rows dW")
    assert_rel(rows.float().cpu().numpy(), pairs.float().cpu().numpy(),
               1e-5 if dtype == torch.float32 else 1e-2, f"{tag} rows vs pairs dW")
    return x, gy, rows


@pytest.mark.parametrize("cin,cout", [(16, 16), (16, 32), (32, 16), (32, 32)])
def test_weight_gradient_from_neighbour_table(cin, cout):
    rng = np.random.default_rng(cin * 3 + cout)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 9000, 3, 14))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    _rows_check(km, cin, cout, seed=cin + cout, tag="3^3")


def test_weight_gradient_from_neighbour_table_strided_and_4d():
    """A 2^3 stride-2 map (n_in != n_out), its swapped (transposed) map, and
    an 81-offset 4D map (offset groups not dividing K)."""
    rng = np.random.default_rng(29)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 30))
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    km = abi.kernel_map(tin, tout, to_dev(oracle.region_offsets(3, 2)))
    _rows_check(km, 32, 32, seed=1, tag="down")
    _rows_check(km.swapped(), 32, 16, seed=2, tag="up")
    c4, _, _ = oracle.insert_and_map(random_coords(rng, 6000, 4, 7, batch=1))
    _, _, km4 = gpu_tables_and_map(c4, c4, oracle.region_offsets(4, 3), same=True)
    _rows_check(km4, 32, 32, seed=3, tag="3^4")


@pytest.mark.parametrize("cin,cout", [(16, 64), (64, 64), (48, 128), (16, 32), (32, 96),
                                      (128, 64), (64, 192)])
def test_weight_gradient_from_neighbour_table_f32(cin, cout):
    """fp32: the position-stationary kernels (16-channel input slices with 64
    or 32 output channels per tile and all 27 offsets in one workgroup; 64 x
    64 tiles with 4 offsets per workgroup where both channel counts are
    multiples of 64)."""
    rng = np.random.default_rng(cin + 7 * cout)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 9000, 3, 14))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    _rows_check(km, cin, cout, seed=cin + cout, tag="3^3", dtype=torch.float32)


def test_weight_gradient_from_neighbour_table_f32_strided_4d_and_tiny():
    """fp32 over a 3^3 stride-2 map and its transpose (n_in != n_out), an
    81-offset 4D map (three offset groups), maps smaller than one
    64-position segment, and 2^3 stride-2 maps (8 offsets: 2 per wave) in
    fp32 and bf16."""
    rng = np.random.default_rng(31)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 30))
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    km = abi.kernel_map(tin, tout, to_dev(oracle.region_offsets(3, 3)))
    _rows_check(km, 64, 128, seed=1, tag="down", dtype=torch.float32)
    _rows_check(km.swapped(), 128, 64, seed=2, tag="up", dtype=torch.float32)
    km8 = abi.kernel_map(tin, tout, to_dev(oracle.region_offsets(3, 2)))
    _rows_check(km8, 64, 128, seed=6, tag="2^3 down", dtype=torch.float32)
    _rows_check(km8.swapped(), 128, 64, seed=7, tag="2^3 up", dtype=torch.float32)
    _rows_check(km8, 64, 128, seed=8, tag="2^3 down bf16")
    xb, gyb, _ = _rows_check(km8.swapped(), 128, 32, seed=9, tag="2^3 up bf16")
    # the layer dispatch keeps a bf16 map of at most 8 offsets with fewer than
    # 2 pairs per output row (the transposed map: one each) on the pair list
    up8 = km8.swapped()
    assert up8.n_pairs < 2 * up8.n_out
    assert torch.equal(abi.conv_weight_grad(xb, gyb, up8, up8.K),
                       abi.conv_backward_weight(xb, gyb, up8, up8.K))
    # 13 offsets (5^3 cross) stay on the pair list: the table entry rejects
    # them and the layer dispatch falls back
    c13 = oracle.region_offsets(3, 5, region="cross")
    assert c13.shape[0] == 13
    km13 = abi.kernel_map(tin, tin, to_dev(c13))
    x13 = torch.randn(km13.n_in, 64, device=DEV)
    gy13 = torch.randn(km13.n_out, 64, device=DEV)
    with pytest.raises(RuntimeError, match="at most 8 or at least 20 offsets"):
        abi.conv_backward_weight_rows(x13, gy13, km13, km13.K)
    assert torch.equal(abi.conv_weight_grad(x13, gy13, km13, km13.K),
                       abi.conv_backward_weight(x13, gy13, km13, km13.K))
    c4, _, _ = oracle.insert_and_map(random_coords(rng, 6000, 4, 7, batch=1))
    _, _, km4 = gpu_tables_and_map(c4, c4, oracle.region_offsets(4, 3), same=True)
    _rows_check(km4, 16, 64, seed=3, tag="3^4", dtype=torch.float32)
    _rows_check(km4, 32, 32, seed=5, tag="3^4 C32", dtype=torch.float32)
    _rows_check(km4, 64, 64, seed=7, tag="3^4 C64", dtype=torch.float32)
    for npts in (1, 5, 63, 65):
        ct, _, _ = oracle.insert_and_map(random_coords(rng, npts, 3, 3))
        _, _, kmt = gpu_tables_and_map(ct, ct, oracle.region_offsets(3, 3), same=True)
        _rows_check(kmt, 16, 64, seed=npts, tag=f"tiny{npts}", dtype=torch.float32)
        _rows_check(kmt, 64, 64, seed=npts, tag=f"tiny{npts} C64", dtype=torch.float32)


@pytest.mark.parametrize("cin", [32, 64])
def test_weight_gradient_from_neighbour_table_f32_row_order_and_empty(cin):
    """out_order NULL (the table indexed by output row) gives the same dW as
    the processing-order table; no output rows gives zeros."""
    import types
    rng = np.random.default_rng(37)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 5000, 3, 12))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    x, gy, rows = _rows_check(km, cin, 64, seed=4, tag="order", dtype=torch.float32)
    nbr = km.nbr.view(km.K, km.n_out)
    by_row = torch.empty_like(nbr)
    by_row[:, km.out_order.long()] = nbr
    km_rows = types.SimpleNamespace(n_in=km.n_in, n_out=km.n_out, n_pairs=km.n_pairs, K=km.K,
                                    nbr=by_row.contiguous().view(-1), out_order=None)
    rows2 = abi.conv_backward_weight_rows(x, gy, km_rows, km.K)
    # the positions are summed in another order: equal to rounding
    assert_rel(rows2.cpu().numpy(), rows.cpu().numpy(), 1e-5, "row-indexed table dW")
    km0 = types.SimpleNamespace(n_in=km.n_in, n_out=0, n_pairs=0, K=km.K,
                                nbr=km.nbr, out_order=km.out_order)
    z = abi.conv_backward_weight_rows(x, gy[:0], km0, km.K)
    assert z.shape == (km.K, cin, 64) and not z.any()


def test_weight_gradient_from_neighbour_table_f32_full_size():
    """Config-2 size (4 indoor scenes, about 410k rows, C64): the table kernel
    against the pair-list kernel, which sums the same products in another
    order (fp32, rel 1e-5)."""
    c = scenes.indoor_batch(4, 2)
    t = abi.hash_build(to_dev(c))
    km = abi.kernel_map(t, t, to_dev(oracle.region_offsets(3, 3)))
    g = torch.Generator().manual_seed(9)
    x = torch.randn(km.n_in, 64, generator=g).to(DEV)
    gy = torch.randn(km.n_out, 64, generator=g).to(DEV)
    print(f"dW rows full size n={km.n_out} P={km.n_pairs}", flush=True)
    rows = abi.conv_backward_weight_rows(x, gy, km, km.K)
    pairs = abi.conv_backward_weight(x, gy, km, km.K)
    assert_rel(rows.cpu().numpy(), pairs.cpu().numpy(), 1e-5, "full-size rows vs pairs dW")
    auto = abi.conv_weight_grad(x, gy, km, km.K)
    assert torch.equal(auto, rows), "the layer dispatch takes the table kernel for fp32 C64"
    again = abi.conv_backward_weight_rows(x, gy, km, km.K)
    assert torch.equal(again, rows), "dW is deterministic"


@pytest.mark.parametrize("cin,cout", [(64, 64), (16, 128), (48, 64)])
def test_weight_gradient_from_neighbour_table_bf16_wide(cin, cout):
    """bf16 with 64-channel output tiles: the position-stationary kernel with
    the step's rows transposed through each wave's LDS rows."""
    rng = np.random.default_rng(cin + 11 * cout)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 9000, 3, 14))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    _rows_check(km, cin, cout, seed=cin + cout, tag="3^3")


def test_weight_gradient_from_neighbour_table_bf16_wide_strided_4d_tiny_full():
    """bf16 64-channel tiles over a 3^3 stride-2 map and its transpose, an
    81-offset 4D map, maps smaller than one segment, and config 2's full
    size against the pair-list kernel."""
    rng = np.random.default_rng(41)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 30))
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    km = abi.kernel_map(tin, tout, to_dev(oracle.region_offsets(3, 3)))
    _rows_check(km, 64, 128, seed=1, tag="down")
    _rows_check(km.swapped(), 128, 64, seed=2, tag="up")
    c4, _, _ = oracle.insert_and_map(random_coords(rng, 6000, 4, 7, batch=1))
    _, _, km4 = gpu_tables_and_map(c4, c4, oracle.region_offsets(4, 3), same=True)
    _rows_check(km4, 32, 64, seed=3, tag="3^4")
    for npts in (1, 33, 65):
        ct, _, _ = oracle.insert_and_map(random_coords(rng, npts, 3, 3))
        _, _, kmt = gpu_tables_and_map(ct, ct, oracle.region_offsets(3, 3), same=True)
        _rows_check(kmt, 16, 64, seed=npts, tag=f"tiny{npts}")
    cf = scenes.indoor_batch(4, 2)
    t = abi.hash_build(to_dev(cf))
    kmf = abi.kernel_map(t, t, to_dev(oracle.region_offsets(3, 3)))
    g = torch.Generator().manual_seed(9)
    x = torch.randn(kmf.n_in, 64, generator=g).to(torch.bfloat16).to(DEV)
    gy = torch.randn(kmf.n_out, 64, generator=g).to(torch.bfloat16).to(DEV)
    print(f"dW rows bf16 full size n={kmf.n_out}", flush=True)
    rows = abi.conv_backward_weight_rows(x, gy, kmf, kmf.K)
    pairs = abi.conv_backward_weight(x, gy, kmf, kmf.K)
    assert_rel(rows.float().cpu().numpy(), pairs.float().cpu().numpy(), 1e-2,
               "bf16 full-size rows vs pairs dW")
    assert torch.equal(abi.conv_weight_grad(x, gy, kmf, kmf.K), rows)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cin,cout", [(256, 256), (128, 64), (96, 192)])
def test_weight_gradient_from_neighbour_table_wide_channels(dtype, cin, cout):
    """Many channel slices and output tiles per range (the grid's unit
    decomposition, few ranges): the table kernels against the pair-list
    kernel, which sums the same products in another order."""
    rng = np.random.default_rng(cin + cout)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 12000, 3, 16))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    g = torch.Generator().manual_seed(cin)
    x = torch.randn(km.n_in, cin, generator=g).to(dtype).to(DEV)
    gy = torch.randn(km.n_out, cout, generator=g).to(dtype).to(DEV)
    print(f"dW rows wide {dtype} {cin}->{cout} n={km.n_out}", flush=True)
    rows = abi.conv_backward_weight_rows(x, gy, km, km.K)
    pairs = abi.conv_backward_weight(x, gy, km, km.K)
    assert_rel(rows.float().cpu().numpy(), pairs.float().cpu().numpy(),
               1e-5 if dtype == torch.float32 else 1e-2, f"wide {cin}->{cout} rows vs pairs dW")


def test_weight_gradient_from_neighbour_table_rejects_other_shapes():
    rng = np.random.default_rng(2)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 500, 3, 8))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    x = torch.zeros(km.n_in, 64, dtype=torch.bfloat16, device=DEV)
    gy = torch.zeros(km.n_out, 48, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="16 or 32"):
        abi.conv_backward_weight_rows(x, gy, km, km.K)
    gy48 = torch.zeros(km.n_out, 48, dtype=torch.float32, device=DEV)
    with pytest.raises(RuntimeError, match="16 or 32"):
        abi.conv_backward_weight_rows(x[:, :32].float().contiguous(), gy48, km, km.K)


def test_kats_through_the_gpu(golden_dir):
    """The reference KATs (identity and permuted K=1 maps) run through the
    C-ABI kernels with hand-built maps."""
    with open(os.path.join(golden_dir, "kat_cpu_convolution.json")) as f:
        kats = json.load(f)["kats"]
    for kat in kats:
        ir = np.array(kat["in_maps"][0], np.int32)
        orr = np.array(kat["out_maps"][0], np.int32)
        nbr = np.full((1, kat["n_out"]), -1, np.int32)
        nbr[0, orr] = ir
        nbr_t = np.full((1, kat["n_in"]), -1, np.int32)
        nbr_t[0, ir] = orr
        km = abi.KernelMap(1, kat["n_in"], kat["n_out"], to_dev(np.array([0, len(ir)], np.int64)),
                           np.array([0, len(ir)], np.int64), to_dev(ir), to_dev(orr),
                           to_dev(nbr), to_dev(nbr_t), to_dev(np.arange(kat["n_in"], dtype=np.int32)),
                           to_dev(np.arange(kat["n_out"], dtype=np.int32)))
        x = to_dev(np.array(kat["x"], np.float32).reshape(kat["n_in"], kat["cin"]))
        w = to_dev(np.array(kat["weight"], np.float32).reshape(1, kat["cin"], kat["cout"]))
        if kat["kind"] == "forward":
            y = abi.conv_forward(x, w, km).cpu().numpy().ravel()
            np.testing.assert_allclose(y, kat["expected_y"], atol=1e-5, rtol=0)
        else:
            gy = to_dev(np.array(kat["grad_y"], np.float32).reshape(kat["n_out"], kat["cout"]))
            gx = abi.conv_backward_input(gy, w, km).cpu().numpy().ravel()
            gw = abi.conv_backward_weight(x, gy, km, 1).cpu().numpy().ravel()
            np.testing.assert_allclose(gx, kat["expected_grad_x"], atol=1e-5, rtol=0)
            np.testing.assert_allclose(gw, kat["expected_grad_w"], atol=1e-5, rtol=0)


def test_config1_sphere_shell_full():
    """Config 1 end to end: 51,554 voxels, 3^3, C16->32 fp32, U(-1,1)
    features, Kaiming-normal weights; map, Y, dX, dW vs the oracle."""
    c = scenes.sphere_shell()
    off = oracle.region_offsets(3, 3)
    _, _, km = gpu_tables_and_map(c, c, off, same=True)
    assert km.n_pairs == 544970
    x = scenes.features(len(c), 16, seed=1, dist="uniform")
    w = scenes.kaiming_weight(27, 16, 32, seed=2)
    gy = scenes.features(len(c), 32, seed=3)
    y = abi.conv_forward(to_dev(x), to_dev(w), km)
    gx = abi.conv_backward_input(to_dev(gy), to_dev(w), km)
    gw = abi.conv_backward_weight(to_dev(x), to_dev(gy), km, 27)
    # the dW dispatch the layer and the bench time (neighbour-table kernels)
    gw_timed = abi.conv_weight_grad(to_dev(x), to_dev(gy), km, 27)
    ry, rgx, rgw = _oracle_conv(km, x, w, gy)
    assert_rel(y.cpu().numpy(), ry, 1e-4, "Y")
    assert_rel(gx.cpu().numpy(), rgx, 1e-4, "dX")
    assert_rel(gw.cpu().numpy(), rgw, 1e-4, "dW (pair list)")
    assert_rel(gw_timed.cpu().numpy(), rgw, 1e-4, "dW (timed dispatch)")


def test_config1_sphere_shell_bf16_vs_torch():
    """Config 1 in bf16 (C16->32: the forward's 16-channel reduction runs on
    the MFMA kernel padded to 32 channels) against the PyTorch fp32
    gather-matmul-scatter on the same bf16 operands, norm-wise 2e-2."""
    c = scenes.sphere_shell()
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    x = to_dev(scenes.features(len(c), 16, seed=1, dist="uniform"), torch.bfloat16)
    w = to_dev(scenes.kaiming_weight(27, 16, 32, seed=2), torch.bfloat16)
    gy = to_dev(scenes.features(len(c), 32, seed=3), torch.bfloat16)
    print(f"config 1 bf16 n={km.n_out} P={km.n_pairs}", flush=True)
    y = abi.conv_forward(x, w, km)
    gx = abi.conv_backward_input(gy, w, km)
    gw = abi.conv_weight_grad(x, gy, km, 27)
    ry, rgx, rgw = _torch_gather_gemm_scatter(km, x, w, gy)
    tol = TOL[torch.bfloat16]
    assert_rel(y.float().cpu().numpy(), ry.cpu().numpy(), tol, "Y")
    assert_rel(gx.float().cpu().numpy(), rgx.cpu().numpy(), tol, "dX")
    assert_rel(gw.float().cpu().numpy(), rgw.cpu().numpy(), tol, "dW")


def _torch_gather_gemm_scatter(km, x, w, gy):
    """Plain PyTorch fp32 version of the reference loop (conv.cpp:47-64) on
    the GPU, with autograd for dX and dW."""
    x = x.detach().float().requires_grad_(True)
    w = w.detach().float().requires_grad_(True)
    y = torch.zeros((km.n_out, w.shape[2]), device=x.device)
    for k in range(km.K):
        ir, orr = km.pairs(k)
        if ir.numel():
            y = y.index_add(0, orr.long(), x.index_select(0, ir.long()) @ w[k])
    y.backward(gy.float())
    return y.detach(), x.grad, w.grad


@pytest.mark.parametrize("cin", [64, 128, 256])
def test_bf16_forward_untransposed_weights(cin):
    """bf16 128-column tiles without an offset-axis split read W itself (two
    transposed LDS reads per B operand) instead of a transposed copy: a 3^3
    map with enough rows that the forward does not split (> 55k output rows
    at C_out = 128), against the plain PyTorch fp32 gather-matmul-scatter."""
    c = scenes.indoor_batch(1, 4)
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    assert km.n_out > 60000
    g = torch.Generator(device="cpu").manual_seed(cin)
    x = torch.randn((km.n_in, cin), generator=g).to(DEV, torch.bfloat16)
    w = (torch.randn((27, cin, 128), generator=g) * (2.0 / (cin * 27)) ** 0.5).to(DEV, torch.bfloat16)
    gy = torch.zeros((km.n_out, 128), device=DEV)
    print(f"untransposed-weight forward C{cin}->128 n={km.n_out}", flush=True)
    y = abi.conv_forward(x, w, km)
    ry, _, _ = _torch_gather_gemm_scatter(km, x, w, gy)
    assert_rel(y.float().cpu().numpy(), ry.cpu().numpy(), TOL[torch.bfloat16], "Y")
    assert torch.equal(y, abi.conv_forward(x, w, km))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config2_full_size_vs_torch(dtype):
    """Config 2 at full size (4 x ~100k voxels, C64, 3^3) against the plain
    PyTorch fp32 gather-matmul-scatter on the same bf16/fp32 operands."""
    c = scenes.indoor_batch(4, 2)
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    g = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn((km.n_in, 64), generator=g).to(DEV, dtype)
    w = (torch.randn((27, 64, 64), generator=g) * (2.0 / (64 * 27)) ** 0.5).to(DEV, dtype)
    gy = torch.randn((km.n_out, 64), generator=g).to(DEV, dtype)
    y = abi.conv_forward(x, w, km)
    gx = abi.conv_backward_input(gy, w, km)
    gw = abi.conv_backward_weight(x, gy, km, 27)
    # the dW dispatch the layer and the bench time (neighbour-table kernels)
    gw_timed = abi.conv_weight_grad(x, gy, km, 27)
    ry, rgx, rgw = _torch_gather_gemm_scatter(km, x, w, gy)
    tol = TOL[dtype]
    assert_rel(y.float().cpu().numpy(), ry.cpu().numpy(), tol, "Y")
    assert_rel(gx.float().cpu().numpy(), rgx.cpu().numpy(), tol, "dX")
    assert_rel(gw.float().cpu().numpy(), rgw.cpu().numpy(), tol, "dW (pair list)")
    assert_rel(gw_timed.float().cpu().numpy(), rgw.cpu().numpy(), tol, "dW (timed dispatch)")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bias_gradient_column_sums(dtype):
    """rhip_conv_bias_grad: fp32 column sums in a fixed order, for row counts
    below and above one row per chunk and channel counts below, at and above
    one workgroup's 256 threads; bitwise repeatable."""
    g = torch.Generator(device="cpu").manual_seed(9)
    for n, C in ((1, 3), (100, 64), (5000, 5), (300000, 64), (2000, 300)):
        gy = torch.randn((n, C), generator=g).to(DEV, dtype)
        got = abi.conv_bias_grad(gy)
        ref = gy.double().sum(0).float()
        assert_rel(got.cpu().numpy(), ref.cpu().numpy(), 1e-5, f"dbias n={n} C={C}")
        assert torch.equal(got, abi.conv_bias_grad(gy))


def test_resident_weight_kernel_on_large_maps():
    """bf16 maps of at least 131072 output rows whose weights for all output
    columns fit in LDS take the resident-weight kernel: a 3^3 same-set map
    with 32 channels and the transposed 2^3 map (8 offsets, C64->32), forward
    and input gradient, against the plain PyTorch fp32 gather-matmul-scatter
    on the same bf16 operands."""
    c = scenes.indoor_batch(4, 3)
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    assert km.n_out >= 131072
    g = torch.Generator(device="cpu").manual_seed(5)
    dt = torch.bfloat16
    x = torch.randn((km.n_in, 32), generator=g).to(DEV, dt)
    w = (torch.randn((27, 32, 32), generator=g) * 0.05).to(DEV, dt)
    gy = torch.randn((km.n_out, 32), generator=g).to(DEV, dt)
    ry, rgx, _ = _torch_gather_gemm_scatter(km, x, w, gy)
    assert_rel(abi.conv_forward(x, w, km).float().cpu().numpy(), ry.cpu().numpy(), TOL[dt],
               "3^3 Y")
    assert_rel(abi.conv_backward_input(gy, w, km).float().cpu().numpy(), rgx.cpu().numpy(),
               TOL[dt], "3^3 dX")
    tf = abi.hash_build(to_dev(c))
    tc = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    up = abi.kernel_map(tf, tc, oracle.region_offsets(3, 2)).swapped()
    assert up.n_out >= 131072
    xc = torch.randn((up.n_in, 64), generator=g).to(DEV, dt)
    wu = (torch.randn((8, 64, 32), generator=g) * 0.1).to(DEV, dt)
    gyf = torch.randn((up.n_out, 32), generator=g).to(DEV, dt)
    ry, rgx, _ = _torch_gather_gemm_scatter(up, xc, wu, gyf)
    assert_rel(abi.conv_forward(xc, wu, up).float().cpu().numpy(), ry.cpu().numpy(), TOL[dt],
               "2^3 transposed Y")
    assert_rel(abi.conv_backward_input(gyf, wu, up).float().cpu().numpy(), rgx.cpu().numpy(),
               TOL[dt], "2^3 transposed dX")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_repeat_calls_are_bitwise_deterministic(dtype):
    """Forward and dX accumulate in registers in a fixed order; dW writes one
    partial tile per workgroup and sums them in a fixed order: all three are
    bitwise repeatable."""
    rng = np.random.default_rng(12)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 10000, 3, 15))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    x = to_dev(rng.standard_normal((km.n_in, 64)).astype(np.float32), dtype)
    w = to_dev(rng.standard_normal((27, 64, 64)).astype(np.float32), dtype)
    gy = to_dev(rng.standard_normal((km.n_out, 64)).astype(np.float32), dtype)
    assert torch.equal(abi.conv_forward(x, w, km), abi.conv_forward(x, w, km))
    assert torch.equal(abi.conv_backward_input(gy, w, km), abi.conv_backward_input(gy, w, km))
    assert torch.equal(abi.conv_backward_weight(x, gy, km, 27),
                       abi.conv_backward_weight(x, gy, km, 27))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_config3_lidar_down_up_full_size(dtype):
    """Config 3 at its stated size (the batch of two sweeps, 151,273 voxels,
    ~150k quoted): 2^3 stride-2 conv C64->128 over the LiDAR batch, then the
    2^3 transposed conv C128->64 back onto the input coordinates (the
    swapped map), forward and backward, against the plain PyTorch fp32
    gather-matmul-scatter on the same operands. bf16 is the configuration's
    dtype; fp32 takes the other dW kernels. Both dW entry points are checked:
    the pair-list kernel and the dispatch the bench and the layer time."""
    c = scenes.lidar_batch(2, 3)
    assert len(c) >= 140000
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    down = abi.kernel_map(tin, tout, oracle.region_offsets(3, 2))
    up = down.swapped()
    assert down.n_pairs == down.n_in  # every fine voxel has exactly one parent
    g = torch.Generator(device="cpu").manual_seed(3)
    dt = dtype
    x = torch.randn((down.n_in, 64), generator=g).to(DEV, dt)
    wd = (torch.randn((8, 64, 128), generator=g) * (2.0 / 512) ** 0.5).to(DEV, dt)
    wu = (torch.randn((8, 128, 64), generator=g) * (2.0 / 1024) ** 0.5).to(DEV, dt)
    gz = torch.randn((down.n_in, 64), generator=g).to(DEV, dt)
    print(f"config 3 {dt}: fine {down.n_in} coarse {down.n_out}", flush=True)
    y = abi.conv_forward(x, wd, down)
    z = abi.conv_forward(y, wu, up)
    gy = abi.conv_backward_input(gz, wu, up)
    gwu = abi.conv_backward_weight(y, gz, up, 8)
    gwu_t = abi.conv_weight_grad(y, gz, up, 8)
    gx = abi.conv_backward_input(gy, wd, down)
    gwd = abi.conv_backward_weight(x, gy, down, 8)
    gwd_t = abi.conv_weight_grad(x, gy, down, 8)
    tol = TOL[dt]
    ry, _, _ = _torch_gather_gemm_scatter(down, x, wd, torch.zeros_like(y))
    assert_rel(y.float().cpu().numpy(), ry.cpu().numpy(), tol, "down Y")
    rz, rgy, rgwu = _torch_gather_gemm_scatter(up, y, wu, gz)
    assert_rel(z.float().cpu().numpy(), rz.cpu().numpy(), tol, "up Y")
    assert_rel(gy.float().cpu().numpy(), rgy.cpu().numpy(), tol, "up dX")
    assert_rel(gwu.float().cpu().numpy(), rgwu.cpu().numpy(), tol, "up dW (pair list)")
    assert_rel(gwu_t.float().cpu().numpy(), rgwu.cpu().numpy(), tol, "up dW (timed dispatch)")
    _, rgx, rgwd = _torch_gather_gemm_scatter(down, x, wd, gy)
    assert_rel(gx.float().cpu().numpy(), rgx.cpu().numpy(), tol, "down dX")
    assert_rel(gwd.float().cpu().numpy(), rgwd.cpu().numpy(), tol, "down dW (pair list)")
    assert_rel(gwd_t.float().cpu().numpy(), rgwd.cpu().numpy(), tol, "down dW (timed dispatch)")


def test_config4_4d_full_size():
    """Config 4 at full size: the 8-frame 4-D shell (232,528 voxels), 3^4
    (81 offsets) C32->32 fp32, forward and backward, against the plain
    PyTorch fp32 gather-matmul-scatter."""
    c = scenes.moving_shell_4d()
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(4, 3), same=True)
    assert km.n_in == 232528 and km.symmetric
    g = torch.Generator(device="cpu").manual_seed(4)
    x = torch.randn((km.n_in, 32), generator=g).to(DEV)
    w = (torch.randn((81, 32, 32), generator=g) * (2.0 / (32 * 81)) ** 0.5).to(DEV)
    gy = torch.randn((km.n_out, 32), generator=g).to(DEV)
    y = abi.conv_forward(x, w, km)
    gx = abi.conv_backward_input(gy, w, km)
    gw = abi.conv_backward_weight(x, gy, km, 81)
    # the dW dispatch the layer and the bench time (neighbour-table kernels)
    gw_timed = abi.conv_weight_grad(x, gy, km, 81)
    ry, rgx, rgw = _torch_gather_gemm_scatter(km, x, w, gy)
    assert_rel(y.cpu().numpy(), ry.cpu().numpy(), 1e-4, "Y")
    assert_rel(gx.cpu().numpy(), rgx.cpu().numpy(), 1e-4, "dX")
    assert_rel(gw.cpu().numpy(), rgw.cpu().numpy(), 1e-4, "dW (pair list)")
    assert_rel(gw_timed.cpu().numpy(), rgw.cpu().numpy(), 1e-4, "dW (timed dispatch)")


@pytest.mark.parametrize("cin,cout,dtype", [
    (64, 64, torch.float32), (64, 64, torch.bfloat16), (32, 128, torch.bfloat16),
    (3, 5, torch.float32), (16, 48, torch.bfloat16)])
def test_symmetric_input_gradient_runs_on_nbr_with_partner_weights(cin, cout, dtype):
    """A symmetric map's input gradient runs on its forward table nbr with
    the stencil partners as weight permutation (the LDS-indexed kernel reads
    slice partner[k] itself; the generic kernel (3->5) and the padded bf16
    reduction (48 output channels) copy the reordered weights first). It
    equals the input gradient over the materialised transposed table
    without a permutation (the sums run in another offset order: within the
    dtype's rounding) and the oracle's."""
    rng = np.random.default_rng(cin * 5 + cout)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 12000, 3, 15))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    assert km.symmetric
    w = to_dev((rng.standard_normal((27, cin, cout)) / np.sqrt(27 * cout)).astype(np.float32),
               dtype)
    gy = to_dev(rng.standard_normal((km.n_out, cout)).astype(np.float32), dtype)
    print(f"symmetric dX cin={cin} cout={cout} {dtype}", flush=True)
    got = abi.conv_backward_input(gy, w, km)  # nbr + partner permutation
    ref = torch.empty_like(got)
    ws = abi._conv_fwd_ws(27, cin, cout, abi._dtype_code(dtype), DEV, km)
    abi._check(abi.lib().rhip_conv_backward_input(
        abi._ptr(gy), km.n_out, cout, abi._ptr(w), 27, cin, abi._ptr(km.nbr_t), None,
        abi._ptr(km.in_order), km.n_in, abi._ptr(ref), abi._dtype_code(dtype), abi._ptr(ws),
        ws.numel(), abi._stream(DEV)), "rhip_conv_backward_input")
    torch.cuda.synchronize()
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert_rel(got.float().cpu().numpy(), ref.float().cpu().numpy(), tol, "perm vs nbr_t")
    _, rgx, _ = _oracle_conv(km, np.zeros((km.n_in, cin), np.float32),
                             w.float().cpu().numpy(), gy.float().cpu().numpy())
    assert_rel(got.float().cpu().numpy(), rgx, TOL[dtype], "dX vs oracle")


def test_weight_permutation_outside_the_lds_kernel_needs_the_workspace():
    """Without a workspace a weight permutation is refused (RHIP_ERR_INVALID)
    for a shape the LDS-indexed kernel does not take, before any launch."""
    rng = np.random.default_rng(2)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 2000, 3, 10))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    gy = to_dev(rng.standard_normal((km.n_out, 5)).astype(np.float32))
    w = to_dev(rng.standard_normal((27, 3, 5)).astype(np.float32))
    gx = torch.empty((km.n_in, 3), device=DEV)
    st = abi.lib().rhip_conv_backward_input(abi._ptr(gy), km.n_out, 5, abi._ptr(w), 27, 3,
                                            abi._ptr(km.nbr), abi._ptr(km.partner),
                                            abi._ptr(km.out_order), km.n_in, abi._ptr(gx),
                                            abi.F32, None, 0, abi._stream(DEV))
    assert st == 1 and "workspace" in abi.lib().rhip_last_error().decode()
