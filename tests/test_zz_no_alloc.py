"""rhip_conv_forward_noalloc (the forward without a workspace, with the
transposed weights in the library's own device scratch) against
rhip_conv_forward: two calls in a row, the second on a smaller map with other
weights, fp32 and bf16, within the path's tolerance (rel 1e-4 fp32, 2e-2
bf16; the workspace call may split the offset axis of a small map and add
the splits' partial sums, which rounds differently). The size limit is
rejected without a GPU call."""
import numpy as np
import pytest
import torch

import oracle
from riemannengine_amd import abi
from helpers import DEV, TOL, assert_rel, random_coords, gpu_tables_and_map, to_dev


def test_noalloc_rejects_weights_beyond_the_scratch():
    L = abi.lib()
    # 27 x 256 x 512 fp32 weights = 13.5 MiB > 8 MiB
    st = L.rhip_conv_forward_noalloc(None, 1, 256, None, 27, 512, None, None, None, 1, None,
                                     abi.F32, None)
    assert st == 3  # RHIP_ERR_UNSUPPORTED
    assert "scratch" in L.rhip_last_error().decode()


def test_noalloc_wrapper_raises_instead_of_converting(monkeypatch):
    """conv_forward_noalloc converts nothing (a conversion would allocate):
    each operand that the library would misread raises ValueError before
    the library is called. Host tensors stand in for device ones here (the
    device check is switched off and the library is never reached)."""
    from types import SimpleNamespace
    monkeypatch.setattr(abi, "_require_cuda", lambda t, name: None)
    monkeypatch.setattr(abi, "lib", lambda: pytest.fail("the library was called"))
    km = SimpleNamespace(K=27, n_in=10, n_out=7)
    f32, bf = torch.float32, torch.bfloat16
    x = torch.zeros(10, 16)
    w = torch.zeros(27, 16, 32)
    ok_out = torch.empty(7, 32)
    cases = {
        "weight dtype": dict(weight=w.to(bf)),
        "x not contiguous": dict(x=torch.zeros(16, 10).t()),
        "weight not contiguous": dict(weight=torch.zeros(27, 32, 16).transpose(1, 2)),
        "bias bf16": dict(bias=torch.zeros(32, dtype=bf)),
        "bias size": dict(bias=torch.zeros(31)),
        "bias not contiguous": dict(bias=torch.zeros(64)[::2]),
        "out dtype": dict(out=torch.empty(7, 32, dtype=bf)),
        "out shape": dict(out=torch.empty(7, 31)),
        "out not contiguous": dict(out=torch.empty(32, 7).t()),
    }
    for what, kw in cases.items():
        args = dict(x=x, weight=w, bias=torch.zeros(32, dtype=f32), out=ok_out)
        args.update(kw)
        with pytest.raises(ValueError):
            abi.conv_forward_noalloc(args["x"], args["weight"], km, bias=args["bias"],
                                     out=args["out"])
            pytest.fail(what)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_forward_matches_workspace_forward(dtype):
    rng = np.random.default_rng(3)
    for n, cin, cout, bias in ((12000, 64, 64, True), (3000, 32, 16, False)):
        c, _, _ = oracle.insert_and_map(random_coords(rng, n, 3, 18))
        _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
        print(f"noalloc {dtype} n={km.n_in} cin={cin} cout={cout} bias={bias}", flush=True)
        x = to_dev(rng.standard_normal((km.n_in, cin)).astype(np.float32), dtype)
        w = to_dev((rng.standard_normal((27, cin, cout)) / 20).astype(np.float32), dtype)
        b = to_dev(rng.standard_normal(cout).astype(np.float32)) if bias else None
        ref = abi.conv_forward(x, w, km, bias=b)
        out = torch.empty_like(ref)
        got = abi.conv_forward_noalloc(x, w, km, bias=b, out=out)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert_rel(got.float().cpu().numpy(), ref.float().cpu().numpy(), TOL[dtype],
                   f"noalloc vs workspace forward, n={km.n_in}")


@pytest.mark.gpu
def test_noalloc_calls_from_two_streams_take_turns():
    """Two calls on two streams back to back, with other weights each: the
    second waits for the first's kernels before it rewrites the shared
    scratch, so both outputs equal the workspace forward's."""
    rng = np.random.default_rng(7)
    c, _, _ = oracle.insert_and_map(random_coords(rng, 40000, 3, 30))
    _, _, km = gpu_tables_and_map(c, c, oracle.region_offsets(3, 3), same=True)
    x = to_dev(rng.standard_normal((km.n_in, 64)).astype(np.float32))
    w1 = to_dev((rng.standard_normal((27, 64, 64)) / 40).astype(np.float32))
    w2 = to_dev((rng.standard_normal((27, 64, 64)) / 40).astype(np.float32))
    ref1, ref2 = abi.conv_forward(x, w1, km), abi.conv_forward(x, w2, km)
    out1, out2 = torch.empty_like(ref1), torch.empty_like(ref2)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(3):
        with torch.cuda.stream(s1):
            abi.conv_forward_noalloc(x, w1, km, out=out1)
        with torch.cuda.stream(s2):
            abi.conv_forward_noalloc(x, w2, km, out=out2)
        torch.cuda.synchronize()
        assert_rel(out1.cpu().numpy(), ref1.cpu().numpy(), TOL[torch.float32], "stream 1")
        assert_rel(out2.cpu().numpy(), ref2.cpu().numpy(), TOL[torch.float32], "stream 2")
