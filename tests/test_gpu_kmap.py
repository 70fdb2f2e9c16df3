"""GPU kernel maps and strided output coordinates vs the oracle: bit-exact
after canonical ordering, plus the dense neighbour tables."""
import numpy as np
import pytest
import torch

import oracle
from riemannengine_amd import abi, scenes
from helpers import DEV, to_dev, random_coords, gpu_tables_and_map, gpu_canonical

pytestmark = pytest.mark.gpu


def _ref_map(cin, cout, off):
    kofs, ir, orr = oracle.kernel_map(cin, cout, off)
    return kofs, oracle.canonical_pairs(kofs, ir, orr)


def _inverse_perm(order, n):
    order = np.asarray(order, np.int64)
    np.testing.assert_array_equal(np.sort(order), np.arange(n))  # a permutation
    pos = np.empty(n, np.int64)
    pos[order] = np.arange(n)
    return pos


def _mask_groups(table):
    """Number of runs of equal neighbour masks along the processing order."""
    m = (table >= 0).T
    if m.shape[0] < 2:
        return m.shape[0]
    return int(1 + np.any(m[1:] != m[:-1], axis=1).sum())


_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _mix64(k):
    """MurmurHash3's 64-bit finalizer on uint64 arrays (wrapping products)."""
    k = k ^ (k >> np.uint64(33))
    k = k * np.uint64(0xff51afd7ed558ccd)
    k = k ^ (k >> np.uint64(33))
    k = k * np.uint64(0xc4ceb9fe1a85ec53)
    return k ^ (k >> np.uint64(33))


def _mask_keys(table):
    """Sort key of each column's neighbour mask: the mask for K <= 16, else
    the neighbour count, largest first, above a hash of the mask's two 64-bit
    words: (31 - count) above 11 hash bits for K <= 31, (127 - min(count, 127))
    above 15 hash bits otherwise."""
    K = table.shape[0]
    hit = (table >= 0).astype(np.uint64)
    m = np.zeros((2, table.shape[1]), np.uint64)
    for k in range(K):
        m[k // 64] |= hit[k] << np.uint64(k % 64)
    if K <= 16:
        return m[0]
    count = (np.bitwise_count(m[0]) + np.bitwise_count(m[1])).astype(np.uint64)
    with np.errstate(over="ignore"):
        h = _mix64(m[0] ^ _mix64(m[1] ^ np.uint64(0x9e3779b97f4a7c15)))
    if K <= 31:
        return ((np.uint64(31) - count) << np.uint64(11)) | (h >> np.uint64(53))
    count = np.minimum(count, np.uint64(127))
    return ((np.uint64(127) - count) << np.uint64(15)) | (h >> np.uint64(49))


def _check_tables(km, tin, tout):
    """nbr/nbr_t hold exactly the pairs at the map's processing positions;
    the orders are permutations that group equal neighbour masks."""
    nbr = km.nbr.cpu().numpy()
    nbr_t = km.nbr_t.cpu().numpy()
    pos_out = _inverse_perm(km.out_order.cpu().numpy(), km.n_out)
    pos_in = _inverse_perm(km.in_order.cpu().numpy(), km.n_in)
    ks = np.repeat(np.arange(km.K), np.diff(km.offsets_host))
    ir, orr = km.in_rows.cpu().numpy(), km.out_rows.cpu().numpy()
    dense = np.full((km.K, km.n_out), -1, np.int64)
    dense[ks, pos_out[orr]] = ir
    np.testing.assert_array_equal(nbr, dense)
    dense_t = np.full((km.K, km.n_in), -1, np.int64)
    dense_t[ks, pos_in[ir]] = orr
    np.testing.assert_array_equal(nbr_t, dense_t)
    # pairs of one offset come out in processing order of the output rows
    for k in range(km.K):
        a, b = km.offsets_host[k], km.offsets_host[k + 1]
        assert np.all(np.diff(pos_out[orr[a:b]]) > 0)
    if km.K <= 128:
        # rows are in mask-key order (a symmetric map orders its input side
        # like its output side); with K <= 16 the key is the mask and equal
        # masks are contiguous
        tabs = (nbr,) if km.symmetric else (nbr, nbr_t)
        if km.symmetric:
            np.testing.assert_array_equal(km.in_order.cpu().numpy(), km.out_order.cpu().numpy())
        for tab in tabs:
            assert np.all(np.diff(_mask_keys(tab).astype(np.int64)) >= 0)
            if km.K <= 16:
                distinct = len(np.unique((tab >= 0).T, axis=0)) if tab.shape[1] else 0
                assert _mask_groups(tab) == distinct


@pytest.mark.parametrize("D,ks,dil,ts,region", [
    (3, 3, 1, 1, "cube"), (3, 3, 2, 1, "cube"), (3, 3, 1, 2, "cube"), (3, 5, 1, 1, "cube"),
    (4, 3, 1, 1, "cube"), (3, 3, 1, 1, "cross"), (2, 3, 1, 1, "cube"), (3, 1, 1, 1, "cube"),
    (3, 2, 1, 1, "cube")])
def test_same_set_map_matches_oracle(D, ks, dil, ts, region):
    rng = np.random.default_rng(D * 100 + ks * 10 + dil)
    c = random_coords(rng, 20000, D, 14) * np.array([1] + [ts] * D, np.int32)
    c, _, _ = oracle.insert_and_map(c)
    off = oracle.region_offsets(D, ks, dil, ts, region)
    print(f"kmap D={D} ks={ks} dil={dil} ts={ts} {region} K={len(off)}", flush=True)
    tin, tout, km = gpu_tables_and_map(c, c, off, same=True)
    kofs, ref = _ref_map(c, c, off)
    np.testing.assert_array_equal(km.offsets_host, kofs)
    np.testing.assert_array_equal(gpu_canonical(km), ref)
    _check_tables(km, tin, tout)
    # odd cubes and crosses are closed under negation: half the offsets are probed
    assert km.symmetric == (ks % 2 == 1)
    # the 3^3 cube in 3-D and the 3^4 cube in 4-D, in cell units (tensor
    # stride 1 or 2, no dilation), read each row's neighbourhood bricks once;
    # the general path below must agree
    nbhd = D in (3, 4) and ks == 3 and dil == 1 and region == "cube"
    assert bool(km.flags & abi.KMAP_BRICK_NBHD) == nbhd
    # the same coordinates in a second table take the general path; it must
    # agree with the mirrored one row for row
    _, tout2, km2 = gpu_tables_and_map(c, c, off, same=False)
    assert not km2.symmetric and not km2.flags & abi.KMAP_BRICK_NBHD
    np.testing.assert_array_equal(km2.offsets_host, kofs)
    np.testing.assert_array_equal(km2.out_order.cpu().numpy(), km.out_order.cpu().numpy())
    np.testing.assert_array_equal(km2.nbr.cpu().numpy(), km.nbr.cpu().numpy())
    np.testing.assert_array_equal(km2.in_rows.cpu().numpy(), km.in_rows.cpu().numpy())
    np.testing.assert_array_equal(km2.out_rows.cpu().numpy(), km.out_rows.cpu().numpy())
    _check_tables(km2, tin, tout2)


def test_custom_region():
    rng = np.random.default_rng(5)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 5000, 3, 8))
    cust = np.array([[0, 0, 0], [2, -1, 0], [-3, 0, 1], [1, 1, 1]])
    off = oracle.region_offsets(3, 3, region="custom", custom=cust)
    tin, tout, km = gpu_tables_and_map(c, c, off, same=True)
    assert not km.symmetric
    np.testing.assert_array_equal(gpu_canonical(km), _ref_map(c, c, off)[1])
    _check_tables(km, tin, tout)
    # a custom set that is point symmetric takes the mirrored path
    sym = np.array([[1, 0, -2], [0, 3, 0], [0, 0, 0], [0, -3, 0], [-1, 0, 2]])
    off = oracle.region_offsets(3, 3, region="custom", custom=sym)
    tin, tout, km = gpu_tables_and_map(c, c, off, same=True)
    assert km.symmetric
    np.testing.assert_array_equal(gpu_canonical(km), _ref_map(c, c, off)[1])
    _check_tables(km, tin, tout)


@pytest.mark.parametrize("s", [2, 4])
def test_strided_output_coords_and_map(s):
    """2^3 stride-s conv: output coords (b, floor(x/s)*s) in first-occurrence
    order (row order bit-exact with the oracle), map = children per parent."""
    rng = np.random.default_rng(s)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 30000, 3, 40))
    coarse_gpu = abi.stride_coords(to_dev(c), [s] * 3)
    tout = abi.hash_build(coarse_gpu)
    ref_coarse = oracle.stride(c, [s] * 3)
    np.testing.assert_array_equal(tout.ucoords.cpu().numpy(), ref_coarse)
    tin = abi.hash_build(to_dev(c))
    off = oracle.region_offsets(3, 2, 1, 1)  # kernel region on the input stride
    km = abi.kernel_map(tin, tout, to_dev(off))
    kofs, ref = _ref_map(c, ref_coarse, off)
    np.testing.assert_array_equal(gpu_canonical(km), ref)
    if s == 2:
        assert km.n_pairs == len(c)  # every fine voxel has exactly one parent
    _check_tables(km, tin, tout)


def test_stride_negative_and_mixed():
    c = np.array([[0, -1, -2, -3], [0, -4, 5, 0], [1, 3, -3, 7], [0, -1, -1, -4]], np.int32)
    got = abi.stride_coords(to_dev(c), [2, 3, 4]).cpu().numpy()
    exp = c.copy()
    exp[:, 1:] = np.floor_divide(c[:, 1:], [2, 3, 4]) * np.array([2, 3, 4])
    np.testing.assert_array_equal(got, exp)


def test_transposed_map_is_swapped_forward_map():
    """space_impl.hpp:649-697: the transposed map (coarse -> fine) equals the
    forward map (fine -> coarse) with in/out exchanged; generating it from
    the fine side with the region on the fine stride gives the same set."""
    rng = np.random.default_rng(8)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 30))
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    off = oracle.region_offsets(3, 2, 1, 1)
    fwd = abi.kernel_map(tin, tout, to_dev(off))
    tr = fwd.swapped()
    ref_kofs, ir, orr = oracle.kernel_map(c, tout.ucoords.cpu().numpy(), off)
    np.testing.assert_array_equal(gpu_canonical(tr), oracle.canonical_pairs(ref_kofs, orr, ir))
    assert tr.n_in == fwd.n_out and tr.n_out == fwd.n_in


def test_empty_sides():
    off = oracle.region_offsets(3, 3)
    c = np.array([[0, 1, 2, 3], [0, 1, 2, 4]], np.int32)
    e = abi.hash_build(torch.zeros((0, 4), dtype=torch.int32, device=DEV))
    t = abi.hash_build(to_dev(c))
    for tin, tout in ((e, t), (t, e), (e, e)):
        km = abi.kernel_map(tin, tout, to_dev(off))
        assert km.n_pairs == 0
        assert (km.nbr == -1).all() and (km.nbr_t == -1).all()


@pytest.mark.parametrize("cfg", ["sphere", "indoor", "shell4d"])
def test_config_maps_match_oracle(cfg):
    c = {"sphere": scenes.sphere_shell, "indoor": lambda: scenes.indoor_batch(4, 2),
         "shell4d": scenes.moving_shell_4d}[cfg]()
    D = c.shape[1] - 1
    off = oracle.region_offsets(D, 3)
    print(f"config map {cfg} n={len(c)} K={len(off)}", flush=True)
    tin, tout, km = gpu_tables_and_map(c, c, off, same=True)
    kofs, ref = _ref_map(c, c, off)
    np.testing.assert_array_equal(km.offsets_host, kofs)
    np.testing.assert_array_equal(gpu_canonical(km), ref)
    # same-set stride-1 maps are symmetric: P_k == P_{K-1-k}
    cnt = np.diff(km.offsets_host)
    np.testing.assert_array_equal(cnt, cnt[::-1])
    if cfg == "sphere":
        assert len(c) == 51554 and km.n_pairs == 544970
    # every configuration's map (3^3 in 3-D, 3^4 in 4-D) takes the
    # neighbourhood-brick probes
    assert km.flags & abi.KMAP_BRICK_NBHD


def test_lidar_down_up_maps():
    c = scenes.lidar_batch(2, 3)
    tin = abi.hash_build(to_dev(c))
    tout = abi.hash_build(abi.stride_coords(to_dev(c), [2, 2, 2]))
    off = oracle.region_offsets(3, 2)
    km = abi.kernel_map(tin, tout, to_dev(off))
    assert km.n_pairs == len(c)  # P_down = N_fine
    np.testing.assert_array_equal(gpu_canonical(km),
                                  _ref_map(c, tout.ucoords.cpu().numpy(), off)[1])


@pytest.mark.parametrize("ks,region", [(2, "cube"), (3, "cube"), (3, "cross")])
def test_generative_expansion_matches_oracle_and_reference(ks, region):
    """Generated map of a generative transposed conv (stride 2 -> 1): the
    unique rows of c + offset over the coarse rows c, offsets at the output
    stride. Bit-exact with the oracle in first-occurrence order over (row,
    offset); the same set as the reference's own stride_region."""
    from oracle import ref
    rng = np.random.default_rng(ks + 7)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 20000, 3, 30))
    coarse = oracle.stride(c, [2, 2, 2])
    off = oracle.region_offsets(3, ks, 1, 1, region)
    gen = abi.hash_build(abi.expand_coords(to_dev(coarse), off))
    got = gen.ucoords.cpu().numpy()
    np.testing.assert_array_equal(got, oracle.stride_region(coarse, off))
    if ks == 2:  # the 2^3 children of every coarse voxel, all distinct
        assert len(got) == 8 * len(coarse)
    if ref.available():
        exp = ref.stride_region(coarse, 2, 2, ks, 1, region)
        assert sorted(map(tuple, got.tolist())) == sorted(map(tuple, exp.tolist()))


@pytest.mark.parametrize("same", [True, False])
def test_row_reference_kernel_map(same):
    """A coordinate set whose column ranges need more than 63 bits builds a
    row-reference table (whole-row compares); its kernel map comes from
    kmap_query_kernel. Dense clusters scattered over the full int32 range,
    so that neighbours exist: the map is bit-exact with the oracle after
    canonical ordering, same-set (symmetric path) and onto another set."""
    rng = np.random.default_rng(21)
    centres = rng.integers(-2**31 + 64, 2**31 - 64, (40, 4), dtype=np.int64)
    pts = []
    for cen in centres:
        pts.append(cen + np.concatenate([rng.integers(0, 2, (300, 1)),
                                         rng.integers(-6, 7, (300, 3))], 1))
    c = np.unique(np.concatenate(pts).astype(np.int32), axis=0)
    c = c[rng.permutation(len(c))]
    if same:
        cout = c
    else:  # half the rows, and shifted copies of a third of them
        shifted = c[1::3] + np.array([0, 1, 0, 0], np.int32)
        cout = np.unique(np.concatenate([c[::2], shifted]), axis=0)
    off = oracle.region_offsets(3, 3)
    tin, tout, km = gpu_tables_and_map(c, cout, off, same=same)
    assert tin.struct.mode == abi.KEY_ROWREF
    _, ref = _ref_map(c, cout, off)
    np.testing.assert_array_equal(gpu_canonical(km), ref)
    assert km.n_pairs > len(cout)  # neighbours were found


def test_kmap_count_with_host_readback_matches_async():
    """rhip_kmap_count with a host array for the pair counts (the call reads
    them back and synchronises) gives the same CSR, neighbour table and order
    as the asynchronous form that abi.kernel_map uses (no host array, CSR
    read after the fill)."""
    import ctypes
    rng = np.random.default_rng(21)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 5000, 3, 11))
    off = oracle.region_offsets(3, 3)
    t, _, km = gpu_tables_and_map(c, c, off, same=True)
    L = abi.lib()
    K, n = off.shape[0], t.n
    nbr = torch.empty((K, n), dtype=torch.int32, device=DEV)
    order = torch.empty(n, dtype=torch.int32, device=DEV)
    ws = torch.empty(abi._sizeq(L.rhip_kmap_workspace_bytes, n, n, K), dtype=torch.uint8,
                     device=DEV)
    kofs = torch.empty(K + 1, dtype=torch.int64, device=DEV)
    kofs_host = np.full(K + 1, -7, dtype=np.int64)
    flags = ctypes.c_int32(0)
    off32 = np.ascontiguousarray(off, dtype=np.int32)
    rc = L.rhip_kmap_count(ctypes.byref(t.struct), abi._ptr(t.ucoords), abi._ptr(t.order), n, K,
                           off32.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), abi._ptr(ws),
                           ws.numel(), abi._ptr(nbr), abi._ptr(order), abi._ptr(kofs),
                           kofs_host.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                           ctypes.byref(flags), abi._stream(torch.device(DEV)))
    assert rc == 0, abi.lib().rhip_last_error()
    # the host array is filled before the call returns
    np.testing.assert_array_equal(kofs_host, km.offsets_host)
    np.testing.assert_array_equal(kofs.cpu().numpy(), km.offsets_host)
    assert torch.equal(nbr, km.nbr) and torch.equal(order, km.out_order)
    assert bool(flags.value & abi.KMAP_SYMMETRIC) == km.symmetric


@pytest.mark.parametrize("same", [True, False])
def test_lazy_pair_lists_equal_the_fill_emission(same):
    """rhip_kmap_pairs (the pair lists built from a finished table, as the
    maps now do on first use) writes exactly what rhip_kmap_fill emits when
    given pair buffers: same pairs, same order. same=True is a symmetric map
    (its fill then writes the transposed table too), False the general path."""
    rng = np.random.default_rng(31)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 30000, 3, 16))
    off = oracle.region_offsets(3, 3)
    tin = abi.hash_build(to_dev(c))
    tout = tin if same else abi.hash_build(to_dev(c))
    km = abi.kernel_map(tin, tout, off)
    assert km.symmetric == same
    L = abi.lib()
    K, n_in, n_out, P = km.K, km.n_in, km.n_out, km.n_pairs
    ws = torch.empty(abi._sizeq(L.rhip_kmap_workspace_bytes, n_in, n_out, K), dtype=torch.uint8,
                     device=DEV)
    nbr = torch.empty((K, n_out), dtype=torch.int32, device=DEV)
    order = torch.empty(n_out, dtype=torch.int32, device=DEV)
    kofs = torch.empty(K + 1, dtype=torch.int64, device=DEV)
    flags = abi.ctypes.c_int32(0)
    o = np.ascontiguousarray(off, np.int32)
    abi._check(L.rhip_kmap_count(abi.ctypes.byref(tin.struct), abi._ptr(tout.ucoords),
                                 abi._ptr(tout.order), n_out, K,
                                 o.ctypes.data_as(abi.ctypes.POINTER(abi.ctypes.c_int32)),
                                 abi._ptr(ws), ws.numel(), abi._ptr(nbr), abi._ptr(order),
                                 abi._ptr(kofs), None, abi.ctypes.byref(flags), abi._stream(DEV)),
               "rhip_kmap_count")
    ir = torch.empty(K * n_out, dtype=torch.int32, device=DEV)
    orr = torch.empty(K * n_out, dtype=torch.int32, device=DEV)
    nbr_t = torch.empty((K, n_in), dtype=torch.int32, device=DEV)
    in_order = torch.empty(n_in, dtype=torch.int32, device=DEV)
    abi._check(L.rhip_kmap_fill(abi._ptr(nbr), abi._ptr(order), n_out, K, abi._ptr(tin.order),
                                n_in, flags.value, abi._ptr(ws), ws.numel(), abi._ptr(kofs),
                                abi._ptr(ir), abi._ptr(orr), abi._ptr(nbr_t),
                                abi._ptr(in_order), abi._stream(DEV)), "rhip_kmap_fill")
    torch.cuda.synchronize()
    assert torch.equal(nbr, km.nbr) and torch.equal(order, km.out_order)
    assert torch.equal(ir[:P], km.in_rows) and torch.equal(orr[:P], km.out_rows)
    # the transposed table of a symmetric map built from nbr's rows equals
    # the one the fill writes
    assert torch.equal(nbr_t, km.nbr_t) and torch.equal(in_order, km.in_order)


def test_symmetric_map_partners_are_the_negated_offsets():
    """A symmetric map's partner offsets negate its stencil, and its pair
    lists are the swapped pair lists under the partner offset."""
    rng = np.random.default_rng(8)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 8000, 3, 12))
    off = oracle.region_offsets(3, 3, 2)
    _, _, km = gpu_tables_and_map(c, c, off, same=True)
    assert km.symmetric
    p = km.partner.cpu().numpy()
    np.testing.assert_array_equal(off[p], -off)
    for k in range(km.K):
        a, b = km.pairs(k)
        ta, tb = km.pairs(int(p[k]))
        got = sorted(zip(a.cpu().tolist(), b.cpu().tolist()))
        assert got == sorted(zip(tb.cpu().tolist(), ta.cpu().tolist()))
