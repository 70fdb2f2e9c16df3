"""Batch normalisation through the HIP kernels (rhip_bn_*), against torch's
batch norm in float64 on the CPU: RiemannBatchNorm is torch BatchNorm1d over
the feature matrix (engine/nn/normalization.hpp:11-37), and BasicBlock folds
its ReLUs and residual addition into the normalisation
(engine/nn/residual.cpp:44-51). Tolerances: rel 1e-4 (fp32) and 2e-2 (bf16),
norm-wise as in helpers.assert_rel; batch statistics rel 1e-5."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
import riemannengine_amd as re_
from riemannengine_amd import abi
from helpers import DEV, TOL, assert_rel, random_coords

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _inputs(n, C, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, C, generator=g) * 3 + 5).to(dtype)  # offset mean: cancellation
    r = torch.randn(n, C, generator=g).to(dtype)
    gy = torch.randn(n, C, generator=g).to(dtype)
    gamma = torch.rand(C, generator=g) + 0.5
    beta = torch.randn(C, generator=g)
    return x, r, gy, gamma, beta


def _reference(x, r, gy, gamma, beta, relu, training=True, rm=None, rv=None, momentum=0.1,
               eps=1e-5):
    """torch batch_norm (+ residual) (+ relu) in float64 with its autograd."""
    xd = x.double().requires_grad_(True)
    rd = None if r is None else r.double().requires_grad_(True)
    gd = None if gamma is None else gamma.double().requires_grad_(True)
    bd = None if beta is None else beta.double().requires_grad_(True)
    y = F.batch_norm(xd, rm, rv, gd, bd, training, momentum, eps)
    if rd is not None:
        y = y + rd
    if relu:
        y = torch.relu(y)
    (y * gy.double()).sum().backward()
    grad = lambda t: None if t is None else t.grad
    return y.detach(), xd.grad, grad(rd), grad(gd), grad(bd)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("C", [1, 3, 5, 32, 64, 256])
def test_batch_statistics_and_running_update(dtype, C):
    n = 4099
    x, *_ = _inputs(n, C, dtype, seed=C)
    rm = torch.randn(C).to(DEV)
    rv = (torch.rand(C) + 0.5).to(DEV)
    rm0, rv0 = rm.cpu().double(), rv.cpu().double()
    mean, invstd = abi.bn_stats(x.to(DEV), 1e-5, 0.1, rm, rv)
    xd = x.double()
    mu, var = xd.mean(0), xd.var(0, unbiased=False)
    np.testing.assert_allclose(_np(mean), mu.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(_np(invstd), (1 / torch.sqrt(var + 1e-5)).numpy(), rtol=1e-5)
    # torch BatchNorm1d: exponential average with the unbiased variance
    np.testing.assert_allclose(_np(rm), (0.9 * rm0 + 0.1 * mu).numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(rv), (0.9 * rv0 + 0.1 * xd.var(0, unbiased=True)).numpy(),
                               rtol=1e-5)


def test_statistics_are_deterministic_and_exact_on_constants():
    x = torch.full((100003, 8), 2.5, device=DEV)
    mean, invstd = abi.bn_stats(x, 1e-5)
    assert torch.all(mean == 2.5)
    np.testing.assert_allclose(_np(invstd), 1 / np.sqrt(1e-5), rtol=1e-6)
    y = torch.randn(300001, 64, device=DEV)
    a = abi.bn_stats(y, 1e-5)
    b = abi.bn_stats(y, 1e-5)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_single_row_raises_like_torch():
    with pytest.raises(RuntimeError, match="Expected more than 1 value per channel"):
        abi.bn_stats(torch.randn(1, 4, device=DEV))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("C,residual,relu", [(32, False, False), (32, False, True),
                                             (64, True, True), (5, True, True),
                                             (3, False, True), (256, True, False)])
def test_forward_backward_match_torch(dtype, C, residual, relu):
    n = 3001
    x, r, gy, gamma, beta = _inputs(n, C, dtype, seed=7 * C + residual)
    r = r if residual else None
    ref = _reference(x, r, gy, gamma, beta, relu)
    xg, gg, bg = x.to(DEV), gamma.to(DEV), beta.to(DEV)
    mean, invstd = abi.bn_stats(xg)
    y = abi.bn_forward(xg, mean, invstd, gg, bg, None if r is None else r.to(DEV), relu)
    assert y.dtype == dtype
    tol = TOL[dtype]
    assert_rel(_np(y), ref[0].numpy(), tol, "y")
    gx, gr, ggam, gbet = abi.bn_backward(gy.to(DEV), y, xg, mean, invstd, gg, relu=relu,
                                         want_residual=residual)
    assert_rel(_np(gx), ref[1].numpy(), tol, "grad x")
    if residual:
        assert_rel(_np(gr), ref[2].numpy(), tol, "grad residual")
    assert_rel(_np(ggam), ref[3].numpy(), tol, "grad gamma")
    assert_rel(_np(gbet), ref[4].numpy(), tol, "grad beta")


def test_forward_without_affine_and_in_place():
    x, _, _, _, _ = _inputs(1000, 16, torch.float32, seed=3)
    xg = x.to(DEV)
    mean, invstd = abi.bn_stats(xg)
    y = abi.bn_forward(xg, mean, invstd)
    ref = F.batch_norm(x.double(), None, None, training=True, eps=1e-5)
    assert_rel(_np(y), ref.numpy(), 1e-4, "no affine")
    # y aliasing x (documented as allowed)
    z = xg.clone()
    assert abi.lib().rhip_bn_forward(
        abi._ptr(z), 1000, 16, abi._ptr(mean), abi._ptr(invstd), None, None, None, 1,
        abi._ptr(z), abi.F32, abi._stream(z.device)) == 0
    torch.testing.assert_close(z, torch.relu(y))


def test_running_statistics_backward_matches_torch_eval():
    """Evaluation mode: normalised by running statistics, gradient without
    the batch-statistics terms."""
    x, r, gy, gamma, beta = _inputs(2000, 32, torch.float32, seed=9)
    rm, rv = torch.randn(32) * 4, torch.rand(32) * 9 + 1
    ref = _reference(x, r, gy, gamma, beta, relu=True, training=False, rm=rm.double(),
                     rv=rv.double())
    invstd = abi.bn_invstd(rv.to(DEV), 1e-5)
    xg = x.to(DEV)
    y = abi.bn_forward(xg, rm.to(DEV), invstd, gamma.to(DEV), beta.to(DEV), r.to(DEV), True)
    assert_rel(_np(y), ref[0].numpy(), 1e-4, "eval y")
    gx, gr, gg, gb = abi.bn_backward(gy.to(DEV), y, xg, rm.to(DEV), invstd, gamma.to(DEV),
                                     relu=True, batch_stats=False, want_residual=True)
    for got, want, what in ((gx, ref[1], "x"), (gr, ref[2], "residual"), (gg, ref[3], "gamma"),
                            (gb, ref[4], "beta")):
        assert_rel(_np(got), want.numpy(), 1e-4, "eval grad " + what)


def test_empty_rows_backward_gives_zero_parameter_gradients():
    x = torch.empty(0, 8, device=DEV)
    mean = torch.zeros(8, device=DEV)
    invstd = torch.ones(8, device=DEV)
    gx, _, gg, gb = abi.bn_backward(torch.empty(0, 8, device=DEV), None, x, mean, invstd,
                                    torch.ones(8, device=DEV))
    assert gx.shape == (0, 8) and torch.all(gg == 0) and torch.all(gb == 0)


def test_full_size_bf16_statistics():
    """A config-5 stage's shape (about 1M rows, 32 channels, bf16)."""
    from riemannengine_amd import scenes
    n = len(scenes.indoor_batch(8, 2))
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(n, 32, generator=g) * 2 - 1).to(torch.bfloat16)
    mean, invstd = abi.bn_stats(x.to(DEV))
    xd = x.double()
    np.testing.assert_allclose(_np(mean), xd.mean(0).numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(invstd), (1 / torch.sqrt(xd.var(0, unbiased=False) + 1e-5))
                               .numpy(), rtol=1e-5)


# ------------------------------------------------------------------ layers


def _layer_input(n_pts, C, dtype, seed):
    rng = np.random.default_rng(seed)
    c, _, _ = oracle.insert_and_map(random_coords(rng, n_pts, 3, 14))
    f = (torch.from_numpy(rng.standard_normal((len(c), C)).astype(np.float32)) * 2 + 1)
    feats = f.to(dtype).to(DEV).requires_grad_(True)
    return re_.SparseTensor(feats, torch.from_numpy(c).to(DEV)), feats


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_batch_norm_layer_matches_torch_module(dtype):
    """Two training steps then evaluation: outputs, gradients, running
    statistics and num_batches_tracked as torch.nn.BatchNorm1d's."""
    C = 32
    layer = re_.nn.RiemannBatchNorm(C, momentum=0.2)
    layer.to(DEV)
    layer.to_dtype(dtype)  # parameters and statistics stay fp32
    p = layer.named_parameters()
    with torch.no_grad():
        p["normalization.weight"].copy_(torch.rand(C) + 0.5)
        p["normalization.bias"].copy_(torch.randn(C))
    ref = torch.nn.BatchNorm1d(C, momentum=0.2).double()
    with torch.no_grad():
        ref.weight.copy_(p["normalization.weight"].cpu().double())
        ref.bias.copy_(p["normalization.bias"].cpu().double())
    tol = TOL[dtype]
    for step in range(3):
        if step == 2:
            layer.eval()
            ref.eval()
        x, feats = _layer_input(2500, C, dtype, seed=20 + step)
        out = layer(x)
        assert out.F.dtype == dtype and out.coordinate_map_key == x.coordinate_map_key
        xr = feats.detach().cpu().double().requires_grad_(True)
        yr = ref(xr)
        gy = torch.randn(yr.shape, generator=torch.Generator().manual_seed(step))
        for q in list(p.values()) + list(ref.parameters()):
            q.grad = None
        (out.F.float() * gy.to(DEV)).sum().backward()
        (yr * gy.double()).sum().backward()
        assert_rel(_np(out.F), yr.detach().numpy(), tol, f"step {step} y")
        assert_rel(_np(feats.grad), xr.grad.numpy(), tol, f"step {step} grad x")
        assert_rel(_np(p["normalization.weight"].grad), ref.weight.grad.numpy(), tol,
                   f"step {step} grad weight")
        assert_rel(_np(p["normalization.bias"].grad), ref.bias.grad.numpy(), tol,
                   f"step {step} grad bias")
        b = layer.named_buffers()
        np.testing.assert_allclose(_np(b["normalization.running_mean"]),
                                   ref.running_mean.numpy(), rtol=1e-4, atol=1e-5)
        np.testing.assert_allclose(_np(b["normalization.running_var"]),
                                   ref.running_var.numpy(), rtol=1e-4)
        assert int(b["normalization.num_batches_tracked"]) == int(ref.num_batches_tracked)


@pytest.mark.parametrize("affine,track", [(False, True), (True, False), (False, False)])
def test_batch_norm_layer_options(affine, track):
    C = 8
    layer = re_.nn.RiemannBatchNorm(C, affine=affine, track_running_stats=track)
    layer.to(DEV)
    ref = torch.nn.BatchNorm1d(C, affine=affine, track_running_stats=track).double()
    for mode in ("train", "eval"):
        getattr(layer, mode)()
        getattr(ref, mode)()
        x, feats = _layer_input(800, C, torch.float32, seed=31)
        out = layer(x)
        xr = feats.detach().cpu().double().requires_grad_(True)
        yr = ref(xr)
        # a random weighting: the gradient of a plain sum is 0 under batch statistics
        gy = torch.randn(yr.shape, generator=torch.Generator().manual_seed(8))
        (out.F * gy.to(DEV)).sum().backward()
        (yr * gy.double()).sum().backward()
        assert_rel(_np(out.F), yr.detach().numpy(), 1e-4, f"{mode} y")
        assert_rel(_np(feats.grad), xr.grad.numpy(), 1e-4, f"{mode} grad x")
    assert set(layer.named_buffers()) == (
        {"normalization.running_mean", "normalization.running_var",
         "normalization.num_batches_tracked"} if track else set())


def _torch_conv(x, w, kofs, ir, orr, n_out):
    """Gather-GEMM-scatter over the oracle's kernel map in torch (autograd);
    kofs[k]:kofs[k+1] is offset k's bucket of (in_rows, out_rows) pairs."""
    k_of_pair = torch.from_numpy(np.repeat(np.arange(len(kofs) - 1), np.diff(kofs)))
    ir, orr = torch.from_numpy(ir.astype(np.int64)), torch.from_numpy(orr.astype(np.int64))
    prod = torch.bmm(x[ir].unsqueeze(1), w[k_of_pair]).squeeze(1)
    return torch.zeros(n_out, w.shape[2], dtype=x.dtype).index_add(0, orr, prod)


def test_basic_block_backward_matches_torch_composition():
    """BasicBlock's fused BN + ReLU / BN + residual + ReLU against the
    reference's composition (conv3 -> BN -> ReLU -> conv3 -> BN -> += ->
    ReLU) in float64 torch autograd: output and every gradient."""
    rng = np.random.default_rng(41)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 3000, 3, 12))
    torch.manual_seed(5)
    blk = re_.nn.BasicBlock(16, 16)
    blk.to(DEV)
    x_np = rng.standard_normal((len(c), 16)).astype(np.float32)
    feats = torch.from_numpy(x_np).to(DEV).requires_grad_(True)
    out = blk(re_.SparseTensor(feats, torch.from_numpy(c).to(DEV)))
    gy = torch.randn(out.F.shape, generator=torch.Generator().manual_seed(6))
    (out.F * gy.to(DEV)).sum().backward()
    p = blk.named_parameters()
    kofs, ir, orr = oracle.kernel_map(c, c, oracle.region_offsets(3, 3))
    leaf = {k: v.detach().cpu().double().requires_grad_(True) for k, v in p.items()}
    xr = torch.from_numpy(x_np).double().requires_grad_(True)
    bn = lambda v, i: F.batch_norm(v, None, None, leaf[f"norm{i}.normalization.weight"],
                                   leaf[f"norm{i}.normalization.bias"], True, 0.1, 1e-5)
    h = torch.relu(bn(_torch_conv(xr, leaf["conv1.base.kernel"], kofs, ir, orr, len(c)), 1))
    ref = torch.relu(bn(_torch_conv(h, leaf["conv2.base.kernel"], kofs, ir, orr, len(c)), 2) + xr)
    (ref * gy.double()).sum().backward()
    assert_rel(_np(out.F), ref.detach().numpy(), 1e-4, "block y")
    assert_rel(_np(feats.grad), xr.grad.numpy(), 1e-4, "block grad x")
    for k, v in p.items():
        assert_rel(_np(v.grad), leaf[k].grad.numpy(), 1e-4, "block grad " + k)


def test_basic_block_with_downsample_matches_torch_composition():
    """BasicBlock(8, 16, stride=2) with a 1x1 stride-2 projection
    (tests/engine/test_layers.cpp:303-318): output channels and tensor
    stride as the reference checks, values and gradients against
    relu(bn2(conv2(relu(bn1(conv1 x)))) + proj x) in float64 torch autograd
    over the oracle's maps."""
    rng = np.random.default_rng(43)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 3000, 3, 14))
    torch.manual_seed(6)
    proj = re_.nn.RiemannConvolution(8, 16, kernel_size=1, stride=2)
    blk = re_.nn.BasicBlock(8, 16, stride=2, downsample=proj)
    blk.to(DEV)
    x_np = rng.standard_normal((len(c), 8)).astype(np.float32)
    feats = torch.from_numpy(x_np).to(DEV).requires_grad_(True)
    out = blk(re_.SparseTensor(feats, torch.from_numpy(c).to(DEV)))
    assert out.F.shape[1] == 16 and out.tensor_stride == [2, 2, 2]
    gy = torch.randn(out.F.shape, generator=torch.Generator().manual_seed(7))
    (out.F * gy.to(DEV)).sum().backward()
    p = blk.named_parameters()
    c2 = out.C.cpu().numpy()
    np.testing.assert_array_equal(np.unique(c2, axis=0), np.unique(oracle.stride(c, [2, 2, 2]), axis=0))
    m1 = oracle.kernel_map(c, c2, oracle.region_offsets(3, 3))
    m2 = oracle.kernel_map(c2, c2, oracle.region_offsets(3, 3) * 2)
    mp = oracle.kernel_map(c, c2, oracle.region_offsets(3, 1))
    leaf = {k: v.detach().cpu().double().requires_grad_(True) for k, v in p.items()}
    xr = torch.from_numpy(x_np).double().requires_grad_(True)
    bn = lambda v, i: F.batch_norm(v, None, None, leaf[f"norm{i}.normalization.weight"],
                                   leaf[f"norm{i}.normalization.bias"], True, 0.1, 1e-5)
    n2 = len(c2)
    h = torch.relu(bn(_torch_conv(xr, leaf["conv1.base.kernel"], *m1, n2), 1))
    res = _torch_conv(xr, leaf["downsample.base.kernel"], *mp, n2)
    ref = torch.relu(bn(_torch_conv(h, leaf["conv2.base.kernel"], *m2, n2), 2) + res)
    (ref * gy.double()).sum().backward()
    assert_rel(_np(out.F), ref.detach().numpy(), 1e-4, "block y")
    assert_rel(_np(feats.grad), xr.grad.numpy(), 1e-4, "block grad x")
    for k, v in p.items():
        assert_rel(_np(v.grad), leaf[k].grad.numpy(), 1e-4, "block grad " + k)


def _torch_conv_gpu(x, w, km):
    """fp32 gather-GEMM-scatter over a GPU kernel map's per-offset pairs, on
    the GPU (autograd)."""
    y = torch.zeros((km.n_out, w.shape[2]), device=x.device, dtype=x.dtype)
    for k in range(km.K):
        ir, orr = km.pairs(k)
        if ir.numel():
            y = y.index_add(0, orr.long(), x.index_select(0, ir.long()) @ w[k])
    return y


class _RoundBF16(torch.autograd.Function):
    """Rounds to bf16 in the forward and the gradient to bf16 in the backward:
    where the bf16 path stores a tensor (or its gradient) in bf16."""

    @staticmethod
    def forward(ctx, v):
        return v.to(torch.bfloat16).float()

    @staticmethod
    def backward(ctx, g):
        return g.to(torch.bfloat16).float()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_basic_block_config5_stage1_full_size(dtype):
    """Config 5's first stage at full size: 8 indoor scenes (808,219 voxels),
    one BasicBlock(32, 32), forward and backward, against the reference's
    composition (conv3 -> BN -> ReLU -> conv3 -> BN -> += -> ReLU,
    residual.cpp:44-52) in fp32 torch on the GPU over the same map's pairs,
    with the block's own parameters and input.

    fp32: rel 1e-4. bf16: rel 2e-2, against the same composition with its
    tensors rounded to bf16 where the bf16 path stores them (each conv and
    batch-norm output and the gradients between the layers): the parameter
    gradients are sums over 800k rows that cancel to a few per mille of their
    terms, so bf16 storage alone moves them several percent from fp32.

    Over 26M activations some pre-activations lie within rounding of zero,
    where the reference's ReLU would decide differently and its gradient
    element differ by its whole value; the reference therefore takes the
    HIP path's ReLU decisions: the block output's sign for the last ReLU, and
    for the inner one the same kernels' conv -> BN -> ReLU recomputed through
    the C ABI (deterministic kernels on the same operands, same values)."""
    from riemannengine_amd import scenes
    c = scenes.indoor_batch(8, 2)
    torch.manual_seed(8)
    blk = re_.nn.BasicBlock(32, 32)
    blk.to(DEV)
    blk.to(dtype)
    g = torch.Generator().manual_seed(9)
    feats = torch.randn(len(c), 32, generator=g).to(DEV, dtype).requires_grad_(True)
    x = re_.SparseTensor(feats, torch.from_numpy(c).to(DEV))
    n = len(x)
    print(f"config-5 stage-1 block n={n} {dtype}", flush=True)
    assert n == 808219
    out = blk(x)
    gy = torch.randn(out.F.shape, generator=g).to(DEV, dtype)
    (out.F.float() * gy.float()).sum().backward()
    t = abi.hash_build(x.C.contiguous())
    km = abi.kernel_map(t, t, oracle.region_offsets(3, 3))
    p = blk.named_parameters()
    w1 = p["conv1.base.kernel"].detach()
    g1, b1 = p["norm1.normalization.weight"].detach(), p["norm1.normalization.bias"].detach()
    # the inner ReLU's decisions of the HIP path
    y1 = abi.conv_forward(feats.detach(), w1, km)
    m1, s1 = abi.bn_stats(y1)
    mask1 = abi.bn_forward(y1, m1, s1, g1.float(), b1.float(), relu=True) > 0
    mask2 = out.F.detach() > 0
    R = _RoundBF16.apply if dtype == torch.bfloat16 else (lambda v: v)
    leaf = {k: v.detach().float().requires_grad_(True) for k, v in p.items()}
    xr = feats.detach().float().requires_grad_(True)
    bn = lambda v, i: F.batch_norm(v, None, None, leaf[f"norm{i}.normalization.weight"],
                                   leaf[f"norm{i}.normalization.bias"], True, 0.1, 1e-5)
    z1 = bn(R(_torch_conv_gpu(xr, leaf["conv1.base.kernel"], km)), 1)
    h = R(z1 * mask1)
    ref = R((bn(R(_torch_conv_gpu(h, leaf["conv2.base.kernel"], km)), 2) + xr) * mask2)
    (ref * gy.float()).sum().backward()
    flips = int(((z1 > 0) != mask1).sum())
    print(f"inner ReLU decisions that differ from the reference's own: {flips} of "
          f"{mask1.numel()}", flush=True)
    assert flips < mask1.numel() // 1000
    tol = TOL[dtype]
    assert_rel(_np(out.F), _np(ref), tol, "block y")
    assert_rel(_np(feats.grad), _np(xr.grad), tol, "block grad x")
    for k, v in p.items():
        assert_rel(_np(v.grad), _np(leaf[k].grad), tol, "block grad " + k)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config5_stage3_full_size(dtype):
    """Config 5's third stage at full size: the 2^3 stride-2 conv C64->128
    that takes stage 2 (tensor stride 2, 8 indoor scenes) down to stage 3
    (tensor stride 4), then one BasicBlock(128, 128) on the stage-3 maps
    (3^3 offsets scaled by the tensor stride), forward and backward through
    the host layer, against the reference's composition (conv.cpp:47-64,
    residual.cpp:44-52) in fp32 torch on the GPU over the same maps' pairs,
    with the layers' own parameters and input. Tolerances, bf16 rounding and
    ReLU decisions are handled as in the stage-1 test above."""
    from riemannengine_amd import scenes
    c = scenes.indoor_batch(8, 2)
    mgr = re_.CoordinateManager(3)
    k1, _ = mgr.insert_and_map(torch.from_numpy(c).to(DEV), [1, 1, 1])
    k2 = mgr.stride(k1, [2, 2, 2])
    c2 = mgr.get_coordinates(k2)
    torch.manual_seed(10)
    down = re_.nn.RiemannConvolution(64, 128, kernel_size=2, stride=2, dimension=3)
    blk = re_.nn.BasicBlock(128, 128)
    for m in (down, blk):
        m.to(DEV)
        m.to_dtype(dtype)
    g = torch.Generator().manual_seed(11)
    feats = torch.randn(len(c2), 64, generator=g).to(DEV, dtype).requires_grad_(True)
    x2 = re_.SparseTensor(feats, k2, mgr)
    h = down(x2)
    out = blk(h)
    n3 = len(out)
    print(f"config-5 stage-3: stage-2 rows {len(c2)}, stage-3 rows {n3} {dtype}", flush=True)
    assert list(h.tensor_stride) == [4, 4, 4] and n3 > 30000
    gy = torch.randn(out.F.shape, generator=g).to(DEV, dtype)
    (out.F.float() * gy.float()).sum().backward()

    c3 = h.C.contiguous()
    t2 = abi.hash_build(c2.contiguous())
    t3 = abi.hash_build(c3)
    kmd = abi.kernel_map(t2, t3, oracle.region_offsets(3, 2, 1, 2))
    km3 = abi.kernel_map(t3, t3, oracle.region_offsets(3, 3, 1, 4))
    assert kmd.n_pairs == len(c2)  # every stage-2 voxel has exactly one parent
    pd = dict(down.named_parameters())
    pb = blk.named_parameters()
    w1 = pb["conv1.base.kernel"].detach()
    g1, b1 = pb["norm1.normalization.weight"].detach(), pb["norm1.normalization.bias"].detach()
    y1 = abi.conv_forward(h.F.detach(), w1, km3)
    m1, s1 = abi.bn_stats(y1)
    mask1 = abi.bn_forward(y1, m1, s1, g1.float(), b1.float(), relu=True) > 0
    mask2 = out.F.detach() > 0
    R = _RoundBF16.apply if dtype == torch.bfloat16 else (lambda v: v)
    leaf_d = {k: v.detach().float().requires_grad_(True) for k, v in pd.items()}
    leaf = {k: v.detach().float().requires_grad_(True) for k, v in pb.items()}
    xr = feats.detach().float().requires_grad_(True)
    bn = lambda v, i: F.batch_norm(v, None, None, leaf[f"norm{i}.normalization.weight"],
                                   leaf[f"norm{i}.normalization.bias"], True, 0.1, 1e-5)
    hr = R(_torch_conv_gpu(xr, leaf_d["base.kernel"], kmd))
    assert_rel(_np(h.F), _np(hr), TOL[dtype], "downsample y")
    z1 = bn(R(_torch_conv_gpu(hr, leaf["conv1.base.kernel"], km3)), 1)
    hh = R(z1 * mask1)
    ref = R((bn(R(_torch_conv_gpu(hh, leaf["conv2.base.kernel"], km3)), 2) + hr) * mask2)
    (ref * gy.float()).sum().backward()
    flips = int(((z1 > 0) != mask1).sum())
    assert flips < mask1.numel() // 1000
    tol = TOL[dtype]
    assert_rel(_np(out.F), _np(ref), tol, "block y")
    assert_rel(_np(feats.grad), _np(xr.grad), tol, "stage-2 grad x")
    for k, v in pb.items():
        assert_rel(_np(v.grad), _np(leaf[k].grad), tol, "block grad " + k)
    for k, v in pd.items():
        assert_rel(_np(v.grad), _np(leaf_d[k].grad), tol, "downsample grad " + k)
