"""The C++ host layer (SparseTensor / CoordinateManager / RiemannConvolution
over the C ABI) on the GPU, against the CPU oracle. Mirrors the reference's
behavioural tests (tests/engine/test_layers.cpp:132-148, 289-317;
python/tests/test_bindings.py:74-88) with values pinned to the oracle.
Tolerances: rel 1e-4 (fp32), 2e-2 (bf16), norm-wise as in helpers.assert_rel."""
import numpy as np
import pytest
import torch

import oracle
import riemannengine_amd as re_
from helpers import DEV, TOL, assert_rel, random_coords

pytestmark = pytest.mark.gpu


def _cloud(seed=0, n=3000, D=3, span=12, batch=2, dup=0.2):
    rng = np.random.default_rng(seed)
    c = random_coords(rng, n, D, span, batch)
    if dup:
        c = np.concatenate([c, c[rng.integers(0, n, int(n * dup))]])[rng.permutation(int(n * (1 + dup)))]
    return c.astype(np.int32)


def _np(t):
    return t.detach().float().cpu().numpy()


def test_sparse_tensor_quantization_modes():
    c = _cloud(1)
    rng = np.random.default_rng(2)
    f = rng.standard_normal((len(c), 3)).astype(np.float32)
    uq, mp, inv = oracle.insert_and_map(c)
    cd, fd = torch.from_numpy(c).to(DEV), torch.from_numpy(f).to(DEV)
    Q = re_.QuantizationMode
    x = re_.SparseTensor(fd, cd)
    assert len(x) == len(uq) and x.dimension == 3 and x.tensor_stride == [1, 1, 1]
    np.testing.assert_array_equal(x.C.cpu().numpy(), uq)
    np.testing.assert_array_equal(_np(x.F), f[mp])  # first occurrence keeps its row
    s = re_.SparseTensor(fd, cd, quantization_mode=Q.UNWEIGHTED_SUM)
    exp = np.zeros((len(uq), 3)); np.add.at(exp, inv, f)
    np.testing.assert_allclose(_np(s.F), exp, rtol=1e-5, atol=1e-5)
    a = re_.SparseTensor(fd, cd, quantization_mode=Q.UNWEIGHTED_AVERAGE)
    cnt = np.bincount(inv, minlength=len(uq))[:, None]
    np.testing.assert_allclose(_np(a.F), exp / cnt, rtol=1e-5, atol=1e-5)
    m = re_.SparseTensor(fd, cd, quantization_mode=Q.MAX_POOL)
    mx = np.full((len(uq), 3), -np.inf); np.maximum.at(mx, inv, f)
    np.testing.assert_array_equal(_np(m.F), mx)


def test_manager_insert_stride_and_cache():
    c = _cloud(3, dup=0)
    uq, mp, inv = oracle.insert_and_map(c)
    mgr = re_.CoordinateManager(3)
    key, (mapping, inverse) = mgr.insert_and_map(torch.from_numpy(c).to(DEV), [1, 1, 1])
    np.testing.assert_array_equal(mapping.cpu().numpy(), mp)
    np.testing.assert_array_equal(inverse.cpu().numpy(), inv)
    # a second insert under the same key gets a fresh random id
    key2, _ = mgr.insert_and_map(torch.from_numpy(c).to(DEV), [1, 1, 1])
    assert not (key2 == key) and key2.tensor_stride == [1, 1, 1]
    skey = mgr.stride(key, [2, 2, 2])
    assert skey.tensor_stride == [2, 2, 2] and mgr.exists(skey)
    np.testing.assert_array_equal(mgr.get_coordinates(skey).cpu().numpy(), oracle.stride(uq, [2, 2, 2]))
    assert mgr.stride(key, [2, 2, 2]) == skey  # reused
    off = oracle.region_offsets(3, 3)
    km = mgr.kernel_map(key, key, [3, 3, 3], [1, 1, 1], [1, 1, 1])
    kofs, ir, orr = oracle.kernel_map(uq, uq, off)
    got = oracle.canonical_pairs(km["offsets_host"], km["in_rows"].cpu().numpy(), km["out_rows"].cpu().numpy())
    np.testing.assert_array_equal(got, oracle.canonical_pairs(kofs, ir, orr))
    n = mgr.kernel_map_cache_size
    mgr.kernel_map(key, key, [3, 3, 3], [1, 1, 1], [1, 1, 1])
    assert mgr.kernel_map_cache_size == n  # cached
    # transposed map from the cached forward strided map = swapped pairs
    fwd = mgr.kernel_map(key, skey, [2, 2, 2], [2, 2, 2], [1, 1, 1])
    tr = mgr.kernel_map(skey, key, [2, 2, 2], [2, 2, 2], [1, 1, 1], is_transpose=True)
    np.testing.assert_array_equal(
        oracle.canonical_pairs(tr["offsets_host"], tr["in_rows"].cpu().numpy(), tr["out_rows"].cpu().numpy()),
        oracle.canonical_pairs(fwd["offsets_host"], fwd["out_rows"].cpu().numpy(), fwd["in_rows"].cpu().numpy()))
    # a pooling map whose kernel tiles the stride is the stride map: one pair
    # list, each input on its floor-aligned output (the same pairs here)
    sm = mgr.kernel_map(key, skey, [2, 2, 2], [2, 2, 2], [1, 1, 1], is_pool=True)
    assert sm["stride_map"] and sm["offsets_host"][1] == len(uq) == sm["offsets_host"][-1]
    np.testing.assert_array_equal(
        np.sort(sm["in_rows"].cpu().numpy()), np.arange(len(uq)))
    pairs = lambda m: sorted(zip(m["in_rows"].cpu().tolist(), m["out_rows"].cpu().tolist()))  # noqa: E731
    assert pairs(sm) == pairs(fwd)


def _conv_check(x_np, c, conv, dtype, out_coords_ref=None, in_coords=None, offsets=None, seed=5):
    """Run conv through the host layer with autograd and compare Y, dX, dW
    (and bias gradient) with the oracle on the same map."""
    feats = torch.from_numpy(x_np).to(DEV, dtype).requires_grad_(True)
    x = re_.SparseTensor(feats, torch.from_numpy(c).to(DEV))
    y = conv(x)
    rng = np.random.default_rng(seed)
    gy = torch.from_numpy(rng.standard_normal(tuple(y.F.shape)).astype(np.float32)).to(DEV, dtype)
    (y.F.float() * gy.float()).sum().backward()
    cin_coords = x.C.cpu().numpy() if in_coords is None else in_coords
    cout_coords = y.C.cpu().numpy()
    if out_coords_ref is not None:
        np.testing.assert_array_equal(cout_coords, out_coords_ref)
    kofs, ir, orr = oracle.kernel_map(cin_coords, cout_coords, offsets)
    w = _np(conv.kernel.to(dtype))
    xin = _np(feats)
    ry = oracle.conv_forward(xin, w, kofs, ir, orr, len(cout_coords))
    if conv.bias is not None:
        ry = ry + _np(conv.bias.to(dtype))
    rgx, rgw = oracle.conv_backward(xin, _np(gy), w, kofs, ir, orr)
    tol = TOL[dtype]
    assert_rel(_np(y.F), ry, tol, "Y")
    assert_rel(_np(feats.grad), rgx, tol, "dX")
    assert_rel(_np(conv.kernel.grad), rgw, tol, "dW")
    if conv.bias is not None:
        assert_rel(_np(conv.bias.grad).ravel(), _np(gy).sum(0), tol, "dbias")
    return x, y


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cin,cout", [(16, 32), (64, 64)])
def test_convolution_layer_matches_oracle(dtype, cin, cout):
    c, _, _ = oracle.insert_and_map(_cloud(7, dup=0))
    torch.manual_seed(0)
    conv = re_.nn.RiemannConvolution(cin, cout, kernel_size=3, bias=True, dimension=3)
    conv.to(DEV)
    x_np = np.random.default_rng(1).standard_normal((len(c), cin)).astype(np.float32)
    x, y = _conv_check(x_np, c, conv, dtype, offsets=oracle.region_offsets(3, 3))
    assert y.coordinate_map_key == x.coordinate_map_key  # stride 1 keeps the map


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_strided_then_transposed(dtype):
    """2x2x2 stride-2 down, then the transposed conv back onto the input
    coordinates (tests/engine/test_layers.cpp:132-148), values vs oracle."""
    c, _, _ = oracle.insert_and_map(_cloud(9, n=4000, span=20, dup=0))
    torch.manual_seed(1)
    down = re_.nn.RiemannConvolution(32, 64, kernel_size=2, stride=2, dimension=3)
    up = re_.nn.RiemannConvolutionTranspose(64, 32, kernel_size=2, stride=2, dimension=3)
    down.to(DEV)
    up.to(DEV)
    x_np = np.random.default_rng(2).standard_normal((len(c), 32)).astype(np.float32)
    off2 = oracle.region_offsets(3, 2)
    x, y = _conv_check(x_np, c, down, dtype, out_coords_ref=oracle.stride(c, [2, 2, 2]), offsets=off2)
    assert y.tensor_stride == [2, 2, 2] and len(y) < len(x)
    # transposed: coarse -> fine over the swapped map
    yf = y.F.detach().clone().requires_grad_(True)
    ys = re_.SparseTensor(yf, y.coordinate_map_key, y.coordinate_manager)
    z = up(ys)
    assert z.tensor_stride == [1, 1, 1] and z.coordinate_map_key == x.coordinate_map_key
    gz = torch.randn(tuple(z.F.shape), generator=torch.Generator().manual_seed(3)).to(DEV, dtype)
    (z.F.float() * gz.float()).sum().backward()
    coarse = y.C.cpu().numpy()
    kofs, ir, orr = oracle.kernel_map(c, coarse, off2)  # fine <- coarse forward map
    w = _np(up.kernel.to(dtype))
    ry = oracle.conv_forward(_np(yf), w, kofs, orr, ir, len(c))  # swapped
    rgx, rgw = oracle.conv_backward(_np(yf), _np(gz), w, kofs, orr, ir)
    tol = TOL[dtype]
    assert_rel(_np(z.F), ry, tol, "up Y")
    assert_rel(_np(yf.grad), rgx, tol, "up dX")
    assert_rel(_np(up.kernel.grad), rgw, tol, "up dW")


def test_transposed_stride_must_divide_tensor_stride():
    c, _, _ = oracle.insert_and_map(_cloud(4, dup=0))
    x = re_.SparseTensor(torch.randn(len(c), 4, device=DEV), torch.from_numpy(c).to(DEV))
    up = re_.nn.RiemannConvolutionTranspose(4, 4, kernel_size=2, stride=2)
    up.to(DEV)
    with pytest.raises(RuntimeError, match="stride must divide"):
        up(x)


def test_transposed_without_finer_map_fails():
    """A transposed convolution maps onto the finer map {tensor_stride / s,
    same id}; when the manager holds no such map the reference ASSERTs with
    ERROR_MAP_NOT_FOUND (space_impl.hpp:576-578)."""
    c, _, _ = oracle.insert_and_map(_cloud(4, dup=0))
    c[:, 1:] *= 2  # coordinates of a tensor-stride-2 map
    mgr = re_.CoordinateManager(3)
    key, _ = mgr.insert_and_map(torch.from_numpy(c).to(DEV), [2, 2, 2])
    x = re_.SparseTensor(torch.randn(len(c), 4, device=DEV), key, mgr)
    assert x.tensor_stride == [2, 2, 2]
    up = re_.nn.RiemannConvolutionTranspose(4, 4, kernel_size=2, stride=2)
    up.to(DEV)
    with pytest.raises(RuntimeError, match="CoordinateMap not found"):
        up(x)


def test_sparse_tensor_reference_spellings():
    """The reference's Python surface (python/src/sparse_bindings.cpp:
    149-191): shape, requires_grad, to(dtype) beside to(device), float(),
    double(), scalar arithmetic from either side; module.to(dtype)."""
    c, _, _ = oracle.insert_and_map(_cloud(6, dup=0))
    f = torch.randn(len(c), 8, device=DEV)
    x = re_.SparseTensor(f, torch.from_numpy(c).to(DEV))
    assert x.shape == (len(c), 8) and x.requires_grad is False
    assert re_.SparseTensor(f.clone().requires_grad_(True), torch.from_numpy(c).to(DEV)).requires_grad
    b = x.to(torch.bfloat16)
    assert b.dtype == torch.bfloat16 and b.coordinate_map_key == x.coordinate_map_key
    assert b.float().dtype == torch.float32 and x.double().dtype == torch.float64
    assert torch.equal(x.to(torch.device("cuda:0")).F, x.F)
    assert torch.equal((2.0 * x).F, 2.0 * x.F) and torch.equal((1.0 + x).F, x.F + 1.0)
    conv = re_.nn.RiemannConvolution(8, 4, kernel_size=3)
    conv.to(DEV)
    conv.to(torch.bfloat16)
    assert conv.kernel.dtype == torch.bfloat16
    assert conv(b).F.dtype == torch.bfloat16


def test_quantization_reductions_other_dtypes():
    """Sum / average / max quantization of fp32 and bf16 features runs on the
    HIP pooling kernels; other dtypes (fp64 here) take torch's scatter
    reductions, as the reference does for every dtype
    (sparse_tensor.cpp:461-477). The row-picking modes take any dtype."""
    c = _cloud(7, n=500)
    cd = torch.from_numpy(c).to(DEV)
    f = torch.randn(len(c), 3, device=DEV, dtype=torch.float64)
    fn = f.cpu().numpy()
    Q = re_.QuantizationMode
    uq, mp, inv = oracle.insert_and_map(c)
    assert len(uq) < len(c)  # the cloud repeats rows
    nu = len(uq)
    want_sum = np.zeros((nu, 3))
    np.add.at(want_sum, inv, fn)
    counts = np.bincount(inv, minlength=nu)[:, None]
    want_max = np.full((nu, 3), -np.inf)
    np.maximum.at(want_max, inv, fn)
    for mode, want in ((Q.UNWEIGHTED_SUM, want_sum), (Q.UNWEIGHTED_AVERAGE, want_sum / counts),
                       (Q.MAX_POOL, want_max)):
        x = re_.SparseTensor(f, cd, quantization_mode=mode)
        assert x.F.dtype == torch.float64
        np.testing.assert_allclose(x.F.cpu().numpy(), want, rtol=1e-12, atol=1e-12)
    x = re_.SparseTensor(f, cd, quantization_mode=Q.RANDOM_SUBSAMPLE)
    np.testing.assert_array_equal(x.F.cpu().numpy(), fn[mp])


def test_convolution_4d():
    c, _, _ = oracle.insert_and_map(_cloud(11, n=3000, D=4, span=6, batch=1, dup=0))
    torch.manual_seed(2)
    conv = re_.nn.RiemannConvolution(8, 16, kernel_size=3, dimension=4)
    conv.to(DEV)
    x_np = np.random.default_rng(4).standard_normal((len(c), 8)).astype(np.float32)
    _conv_check(x_np, c, conv, torch.float32, offsets=oracle.region_offsets(4, 3))


def test_basic_block_forward_backward_matches_composition():
    """BasicBlock = conv3 -> BN -> ReLU -> conv3 -> BN -> +x -> ReLU
    (engine/nn/residual.cpp:44-52), checked against the oracle convolutions
    composed with torch's batch norm (training mode, batch statistics); the
    gradient reaches conv1's kernel (tests/engine/test_layers.cpp:289-301)."""
    c, _, _ = oracle.insert_and_map(_cloud(13, dup=0))
    torch.manual_seed(3)
    blk = re_.nn.BasicBlock(16, 16)
    blk.to(DEV)
    x_np = np.random.default_rng(5).standard_normal((len(c), 16)).astype(np.float32)
    feats = torch.from_numpy(x_np).to(DEV).requires_grad_(True)
    x = re_.SparseTensor(feats, torch.from_numpy(c).to(DEV))
    out = blk(x)
    out.F.sum().backward()
    p = blk.named_parameters()
    assert p["conv1.base.kernel"].grad is not None and p["conv1.base.kernel"].grad.abs().sum() > 0
    assert feats.grad is not None and torch.isfinite(feats.grad).all()
    off = oracle.region_offsets(3, 3)
    kofs, ir, orr = oracle.kernel_map(c, c, off)
    conv = lambda v, w: torch.from_numpy(oracle.conv_forward(v.numpy(), _np(w), kofs, ir, orr, len(c)))
    bn = lambda v: torch.nn.functional.batch_norm(v, None, None, training=True, eps=1e-5)
    xr = torch.from_numpy(x_np)
    h = torch.relu(bn(conv(xr, p["conv1.base.kernel"])))
    ref = torch.relu(bn(conv(h, p["conv2.base.kernel"])) + xr)
    assert_rel(_np(out.F), ref.numpy(), 1e-4, "block")


def _encoder(dtype, seed=7):
    """Config 5's encoder: 4 stages of 2 BasicBlocks and a 2^3 stride-2 conv,
    channels 32 -> 64 -> 128 -> 256."""
    torch.manual_seed(seed)
    chans = [32, 64, 128, 256]
    mods = []
    for i, c in enumerate(chans):
        mods += [re_.nn.BasicBlock(c, c), re_.nn.BasicBlock(c, c),
                 re_.nn.RiemannConvolution(c, chans[min(i + 1, 3)], kernel_size=2, stride=2,
                                           dimension=3)]
    for m in mods:
        m.to(DEV)
        m.to_dtype(dtype)
    return mods


def test_config5_encoder_full_size():
    """Config 5 at full size: 8 indoor scenes through the encoder in bf16,
    forward and backward in the host layer. Every stage's maps are built on
    the first pass and reused from the manager's cache on the second; the
    bf16 run agrees with the same encoder in fp32 (same initial weights)."""
    from riemannengine_amd import scenes
    c = scenes.indoor_batch(8, 2)
    coords = torch.from_numpy(c).to(DEV)
    feats = torch.randn((len(c), 32), generator=torch.Generator().manual_seed(1)).to(DEV)
    outs = {}
    for dtype in (torch.bfloat16, torch.float32):
        mods = _encoder(dtype)
        x = re_.SparseTensor(feats.to(dtype).requires_grad_(True), coords)
        print(f"config 5 {dtype}: {len(x)} voxels", flush=True)
        mgr = x.coordinate_manager
        for rep in range(2):
            h = x
            for m in mods:
                h = m(h)
            if rep == 0:
                n_maps = mgr.kernel_map_cache_size
            else:
                assert mgr.kernel_map_cache_size == n_maps  # maps reused
        assert h.tensor_stride == [16, 16, 16] and h.F.shape[1] == 256
        h.F.float().sum().backward()
        k0 = mods[0].named_parameters()["conv1.base.kernel"]
        assert k0.grad is not None and torch.isfinite(k0.grad.float()).all()
        outs[dtype] = h.F.detach().float().cpu().numpy()
    assert_rel(outs[torch.bfloat16], outs[torch.float32], 5e-2, "bf16 vs fp32 encoder output")


@pytest.mark.parametrize("ks", [2, 3])
def test_generative_transposed_convolution(ks):
    """RiemannGenerativeConvolutionTranspose generates its output map from
    the coarse input (stride_region, the region at the output stride) instead
    of requiring the finer map: output rows = the oracle's generated set;
    since a stride-1 map already exists, the generated one gets its own key.
    Values and gradients vs the oracle over the swapped forward map."""
    c, _, _ = oracle.insert_and_map(_cloud(17, n=4000, span=20, dup=0))
    torch.manual_seed(5)
    down = re_.nn.RiemannConvolution(8, 16, kernel_size=2, stride=2, dimension=3)
    gen = re_.nn.RiemannGenerativeConvolutionTranspose(16, 8, kernel_size=ks, stride=2,
                                                        dimension=3)
    down.to(DEV)
    gen.to(DEV)
    x = re_.SparseTensor(torch.randn(len(c), 8, device=DEV), torch.from_numpy(c).to(DEV))
    y = down(x)
    yf = y.F.detach().clone().requires_grad_(True)
    ys = re_.SparseTensor(yf, y.coordinate_map_key, y.coordinate_manager)
    z = gen(ys)
    coarse = y.C.cpu().numpy()
    off = oracle.region_offsets(3, ks, 1, 1)
    fine = oracle.stride_region(coarse, off)
    np.testing.assert_array_equal(z.C.cpu().numpy(), fine)
    assert z.tensor_stride == [1, 1, 1] and not (z.coordinate_map_key == x.coordinate_map_key)
    gz = torch.randn(tuple(z.F.shape), generator=torch.Generator().manual_seed(6)).to(DEV)
    (z.F * gz).sum().backward()
    kofs, ir, orr = oracle.kernel_map(fine, coarse, off)  # fine <- coarse, then swapped
    w = _np(gen.kernel)
    assert_rel(_np(z.F), oracle.conv_forward(_np(yf), w, kofs, orr, ir, len(fine)), 1e-4, "Y")
    rgx, rgw = oracle.conv_backward(_np(yf), _np(gz), w, kofs, orr, ir)
    assert_rel(_np(yf.grad), rgx, 1e-4, "dX")
    assert_rel(_np(gen.kernel.grad), rgw, 1e-4, "dW")
    # the manager's own entry point: an existing (stride, "") key is kept
    # unless expansion is asked for
    mgr = y.coordinate_manager
    k1, built = mgr.stride_region(y.coordinate_map_key, torch.from_numpy(off), [1, 1, 1], False)
    assert not built and k1.tensor_stride == [1, 1, 1]
