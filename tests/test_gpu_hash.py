"""GPU coordinate hashing vs the oracle: bit-exact unique rows, mapping and
inverse (first-occurrence order), lookups, locality order."""
import numpy as np
import pytest
import torch

import oracle
from riemannengine_amd import abi, scenes
from helpers import DEV, to_dev, random_coords

pytestmark = pytest.mark.gpu


def _check_build(c):
    print(f"hash build n={c.shape[0]} ncol={c.shape[1]}", flush=True)
    t = abi.hash_build(to_dev(c))
    uq, mp, inv = oracle.insert_and_map(c)
    assert t.n == uq.shape[0]
    np.testing.assert_array_equal(t.ucoords.cpu().numpy(), uq)
    np.testing.assert_array_equal(t.mapping.cpu().numpy(), mp)
    np.testing.assert_array_equal(t.inverse.cpu().numpy(), inv)
    return t


@pytest.mark.parametrize("n,D,span", [(1, 3, 5), (1000, 3, 4), (50000, 3, 20), (30000, 4, 6),
                                      (200000, 3, 60), (5000, 1, 100), (4000, 6, 3)])
def test_build_matches_oracle(n, D, span):
    rng = np.random.default_rng(n + D)
    _check_build(random_coords(rng, n, D, span))


def test_scan_order_points_match_oracle():
    """Raw quantised LiDAR points in scan order, the input a coordinate map
    deduplicates: most repeats follow the same point, in runs that one lane
    inserts for the whole run (the car-height recipe, whose near ground
    puts many beams into each voxel), and the configuration's own sweeps."""
    c = scenes.lidar_batch(2, 3, unique=False, recipe="literal")
    assert np.all(c[1:] == c[:-1], axis=1).sum() > len(c) // 3
    t = _check_build(c)
    assert t.n == len(scenes.lidar_batch(2, 3, recipe="literal"))
    c = scenes.lidar_batch(2, 3, unique=False)
    t = _check_build(c)
    assert t.n == len(scenes.lidar_batch(2, 3)) == 151273


@pytest.mark.parametrize("span", [20, 30000])
def test_runs_of_repeats_match_oracle(span):
    """Runs of one row of random lengths (some longer than a wave), and rows
    that come back later after other rows; span 30000 leaves no room for
    the row in the key word (the first row is kept beside the key)."""
    rng = np.random.default_rng(span)
    base = random_coords(rng, 6000, 3, span)
    reps = rng.integers(1, 12, len(base))
    reps[rng.integers(0, len(base), 20)] = rng.integers(60, 200, 20)
    c = np.repeat(base, reps, axis=0)
    c = np.concatenate([c, base[rng.integers(0, len(base), 3000)], c[:5000]])
    print(f"runs: {len(c)} rows", flush=True)
    _check_build(c)


def test_lookup_repeated_queries():
    """Queries in runs (present, absent and out-of-range rows) take their
    run's answer."""
    rng = np.random.default_rng(5)
    c = random_coords(rng, 20000, 3, 30)
    t = abi.hash_build(to_dev(c))
    rows = np.concatenate([c[:3000], random_coords(rng, 1000, 3, 40),
                           np.array([[0, 2**31 - 1, 0, 0], [1, -2**31, 7, 7]], np.int32)])
    q = np.repeat(rows, rng.integers(1, 90, len(rows)), axis=0)
    got = t.lookup(to_dev(q)).cpu().numpy()
    uq, _, _ = oracle.insert_and_map(c)
    where = {tuple(r): i for i, r in enumerate(uq.tolist())}
    np.testing.assert_array_equal(got, [where.get(tuple(r), -1) for r in q.tolist()])


def test_build_empty():
    t = abi.hash_build(torch.zeros((0, 4), dtype=torch.int32, device=DEV))
    assert t.n == 0
    assert (t.lookup(torch.tensor([[0, 0, 0, 0]], dtype=torch.int32, device=DEV)) == -1).all()


def test_row_reference_mode_for_wide_ranges():
    """Columns spanning the full int32 range cannot pack into 63 bits; the
    table falls back to comparing whole rows."""
    rng = np.random.default_rng(9)
    base = rng.integers(-2**31, 2**31 - 1, (3000, 4), dtype=np.int64).astype(np.int32)
    c = np.concatenate([base, base[rng.integers(0, 3000, 2000)]])[rng.permutation(5000)]
    t = _check_build(c)
    assert t.struct.mode == abi.KEY_ROWREF
    q = np.concatenate([c[:100], c[:100] + 1])
    got = t.lookup(to_dev(q)).cpu().numpy()
    uq, _, inv = oracle.insert_and_map(c)
    where = {tuple(r): i for i, r in enumerate(uq.tolist())}
    exp = [where.get(tuple(r), -1) for r in q.tolist()]
    np.testing.assert_array_equal(got, exp)


def test_lookup_present_absent_and_out_of_range():
    rng = np.random.default_rng(4)
    c = random_coords(rng, 20000, 3, 30)
    t = abi.hash_build(to_dev(c))
    assert t.struct.mode == abi.KEY_PACKED64
    q = np.concatenate([c[:5000], random_coords(rng, 5000, 3, 40),
                        np.array([[0, 2**31 - 1, 0, 0], [-5, 0, 0, 0], [1, -2**31, 7, 7]], np.int32)])
    got = t.lookup(to_dev(q)).cpu().numpy()
    uq, _, _ = oracle.insert_and_map(c)
    where = {tuple(r): i for i, r in enumerate(uq.tolist())}
    exp = np.array([where.get(tuple(r), -1) for r in q.tolist()])
    np.testing.assert_array_equal(got, exp)


def _morton_order(rows):
    """Batch first, then the Morton code of the spatial offsets from the
    column minima, each shifted right by the trailing zero bits all offsets
    of its column share (bit b of column j at b * D + (D - j)), stable."""
    rows = rows.astype(np.int64)
    D = rows.shape[1] - 1
    rel = rows - rows.min(axis=0)
    tz = []
    for j in range(D + 1):
        o = int(np.bitwise_or.reduce(rel[:, j]))
        tz.append((o & -o).bit_length() - 1 if o else 0)
    sh = np.stack([rel[:, j] >> tz[j] for j in range(D + 1)], 1)
    wide = int(max(int(sh[:, j].max()).bit_length() for j in range(1, D + 1)))
    key = rel[:, 0] << (wide * D)
    for b in range(wide):
        for j in range(1, D + 1):
            key |= ((sh[:, j] >> b) & 1) << (b * D + (D - j))
    return np.argsort(key, kind="stable")


@pytest.mark.parametrize("stride", [1, 2, 4])
def test_spatial_order_is_morton_permutation(stride):
    rng = np.random.default_rng(2)
    c = random_coords(rng, 40000, 3, 50, batch=3)
    c[:, 1:] *= stride
    t = abi.hash_build(to_dev(c))
    order = t.order.cpu().numpy()
    pos = t.pos.cpu().numpy()
    np.testing.assert_array_equal(np.sort(order), np.arange(t.n))
    np.testing.assert_array_equal(pos[order], np.arange(t.n))
    np.testing.assert_array_equal(order, _morton_order(t.ucoords.cpu().numpy()))
    # a compact set gets a brick index over this order
    assert t.struct.bricks is not None and t.struct.morton_bits > 0


def _brick_walk(rows):
    """(grid entries, Morton indices of the grid walk, entry limit) of a set
    of unique rows: bricks of 2^(6 // D) cells per column over the shifted
    offsets, each column's brick extent rounded up to a power of two in the
    walk, batches on top."""
    rows = rows.astype(np.int64)
    D = rows.shape[1] - 1
    rel = rows - rows.min(axis=0)
    L, entries, walk = 6 // D, int(rel[:, 0].max()) + 1, int(rel[:, 0].max()) + 1
    for j in range(1, D + 1):
        o = int(np.bitwise_or.reduce(rel[:, j]))
        tz = (o & -o).bit_length() - 1 if o else 0
        dim = (int(rel[:, j].max()) >> tz >> L) + 1
        entries *= dim
        walk *= 1 << (dim - 1).bit_length()
    return entries, walk, min(1 << 23, max(4096, 16 * len(rows)))


def _spatial_order(t, with_bricks, ws_bytes=None):
    """rhip_spatial_order once more on a built table (a copy of its struct),
    with or without brick storage, in a workspace of ws_bytes (default: the
    size rhip_order_workspace_bytes gives): (struct, order, pos)."""
    import ctypes
    L = abi.lib()
    st = abi.RhipTable.from_buffer_copy(t.struct)
    n = t.n
    order = torch.empty(n, dtype=torch.int32, device=DEV)
    pos = torch.empty(n, dtype=torch.int32, device=DEV)
    if ws_bytes is None:
        ws_bytes = abi._sizeq(L.rhip_order_workspace_bytes, n)
    ows = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    bb = ctypes.c_size_t(0)
    if with_bricks:
        assert L.rhip_brick_bytes(ctypes.byref(st), ctypes.byref(bb)) == 0
    bricks = torch.empty(max(int(bb.value), 1), dtype=torch.uint8, device=DEV)
    rc = L.rhip_spatial_order(ctypes.byref(st), abi._ptr(order), abi._ptr(pos),
                              abi._ptr(bricks) if with_bricks else None, int(bb.value),
                              abi._ptr(ows), ows.numel(), abi._stream(torch.device(DEV)))
    assert rc == 0, L.rhip_last_error()
    torch.cuda.synchronize()
    return st, order.cpu().numpy(), pos.cpu().numpy()


# (D, rows, span, stride, which): which = the path the brick storage takes,
# "walk" (counting sort through the grid in brick Morton order) or "sort"
# (radix sort of the keys, then the grid filled from the sorted keys)
_ORDER_SETS = [(1, 3000, 2000, 1, "walk"), (2, 20000, 200, 1, "walk"), (3, 40000, 50, 2, "walk"),
               (3, 30000, 37, 1, "walk"), (4, 30000, 12, 1, "walk"), (5, 20000, 5, 2, "walk"),
               (6, 4000, 3, 1, "walk"), (6, 80000, 9, 1, "sort")]


@pytest.mark.parametrize("D,n,span,stride,which", _ORDER_SETS)
def test_spatial_order_paths_agree_with_morton(D, n, span, stride, which):
    """The locality order with a brick grid (walked, or filled after a sort
    when the power-of-two padding makes the walk too long) and without one
    (sort only) is the Morton order of the rows; the brick path is the one
    the set's shape selects. A walk marks the cells with a byte each where
    the workspace holds them (always, at the size rhip_order_workspace_bytes
    gives, for these sets) and with atomic ORs into the grid otherwise: a
    workspace of only the walk's chunk totals and bases takes the atomic
    marks, and both give the same order."""
    rng = np.random.default_rng(D * 1000 + span)
    c = random_coords(rng, n, D, span, batch=2)
    c[:, 1:] *= stride
    print(f"spatial order D={D} n={n} span={span} stride={stride} path={which}", flush=True)
    t = abi.hash_build(to_dev(c))
    rows = t.ucoords.cpu().numpy()
    entries, walk, limit = _brick_walk(rows)
    assert entries <= limit
    walks = walk <= max(8 * entries, 1 << 22)
    assert walks == (which == "walk")
    exp = _morton_order(rows)
    runs = [(True, None), (False, None)]
    if walks:  # chunks of 1024 walk indices: int32 totals, int64 bases, one int64, 256-aligned
        chunks = -(-walk // 1024)
        a256 = lambda b: -(-b // 256) * 256
        runs.append((True, a256(4 * chunks) + a256(8 * chunks) + 8))
    for with_bricks, ws in runs:
        st, order, pos = _spatial_order(t, with_bricks, ws)
        np.testing.assert_array_equal(order, exp)
        np.testing.assert_array_equal(pos[order], np.arange(t.n))
        assert (st.bricks is not None) == with_bricks


@pytest.mark.parametrize("n,span", [(4000, 3), (80000, 9)])
def test_six_dim_cross_map_through_bricks(n, span):
    """A 6-D kernel map (cross stencil) whose neighbour probes go through the
    brick grid, walked (small set) or filled after the sort (large set)."""
    rng = np.random.default_rng(n)
    c, _, _ = oracle.insert_and_map(random_coords(rng, n, 6, span))
    off = oracle.region_offsets(6, 3, region="cross")
    print(f"6-D cross map n={len(c)} K={len(off)}", flush=True)
    t = abi.hash_build(to_dev(c))
    assert t.struct.bricks is not None
    km = abi.kernel_map(t, t, to_dev(off))
    kofs, in_rows, out_rows = oracle.kernel_map(c, c, off)
    np.testing.assert_array_equal(km.offsets_host, kofs)
    np.testing.assert_array_equal(
        oracle.canonical_pairs(km.offsets_host, km.in_rows.cpu().numpy(), km.out_rows.cpu().numpy()),
        oracle.canonical_pairs(kofs, in_rows, out_rows))


@pytest.mark.parametrize("cfg", ["sphere", "indoor", "lidar", "shell4d"])
def test_config_coordinate_sets(cfg):
    c = {"sphere": scenes.sphere_shell, "indoor": lambda: scenes.indoor_batch(4, 2),
         "lidar": lambda: scenes.lidar_batch(2, 3), "shell4d": scenes.moving_shell_4d}[cfg]()
    rng = np.random.default_rng(1)
    dup = np.concatenate([c, c[rng.integers(0, len(c), len(c) // 3)]])[rng.permutation(len(c) * 4 // 3)]
    _check_build(dup)
