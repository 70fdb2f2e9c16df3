#!/usr/bin/env python3
"""Sparse-convolution hot-path benchmark on one MI355X.

Workload (config 2 of the benchmark set): batch 4 synthetic indoor scenes,
~100k unique voxels each on a 5 cm grid, 3x3x3 stride-1 convolution
C_in = C_out = 64, features N(0,1), Kaiming-normal weights. One "step" is
the convolution forward, the input gradient and the weight gradient over the
whole batch with the kernel map prebuilt (as in training, where maps are
cached by the coordinate manager). Inputs are resident in HBM before the
timed region starts.

Printed as ONE JSON line:
  value        whole-job Mvoxels/s = N_in / (host-clock time per timed step,
               forward + dX + dW) / 1e6
  kernel_map_ms  hash build + locality order + kernel map, from device coords,
               through the C++ CoordinateManager (insert_and_map + kernel_map)
  kernel_map_roofline  the map build's algorithmic bytes (hash: rows read, slot
               and row-index writes; map: both sides' rows, one 8-byte probe
               per query, the pairs and offsets) / kernel_map_ms vs 8 TB/s
  bf16         the same step in bf16 (fp32 accumulate): its own ms_per_step,
               breakdown and HBM roofline with measured traffic
  roofline     the dominant kernel's algorithmic FLOP/s (fp32, MFMA-bound) or
               bytes/s (bf16, HBM-bound), from HIP events recorded on the
               stream the kernels run on around the dW pass of every tenth
               timed step (an event record idles the device ~6 us), against
               MI355X's published peak
  breakdown_ms per-pass event times from untimed steps after the timed ones
               (events between every pass would cost the timed steps a few
               microseconds each)
  cpu_baseline the reference's own CPU path (compiled from its sources into
               oracle/_ref) timed on one scene of the same workload, or the
               scalar C oracle where that library was not built
  cpu_kernel_map_baseline  the reference's CPU map build alone (same sample)

--gpus N > 1 is refused: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import contextlib
import gc
import json
import os
import platform
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# MI355X published peaks (dense): HBM3E bandwidth and MFMA throughput.
PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {"f32": 157.3, "bf16": 2500.0}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--dtype", choices=["f32", "bf16"], default=None,
                    help="feature/weight dtype (fp32 accumulate); default: the config's own "
                         "(f32 for configs 1, 2, 4; bf16 for 3, 5)")
    ap.add_argument("--config", type=int, choices=[1, 2, 3, 4, 5], default=2,
                    help="benchmark configuration; 2 (the default) is the headline line, the "
                         "others print a line of their own for the record")
    ap.add_argument("--op", choices=["conv", "pool"], default="conv",
                    help="conv (default): the headline convolution line; pool: a line of its "
                         "own for the pooling path on the config-2 coordinates")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU oracle timing (profiling runs)")
    ap.add_argument("--map-reps", type=int, default=20)
    ap.add_argument("--no-other-configs", action="store_true",
                    help="the headline run without the compact records of configs 1, 3, 4, 5")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="calibration mode: time a plain device copy of this many MiB "
                         "(the kernel of known traffic the HBM byte counters are checked "
                         "against) and exit")
    return ap.parse_args()


def copy_calibration(mib: int) -> None:
    """Copy an int32 buffer of `mib` MiB five times on the device: a kernel of
    known traffic (mib MiB read + mib MiB written per launch) against which
    the HBM byte counters are scaled."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.arange(n, dtype=torch.int32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(5):
        dst.copy_(src)
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / 5
    print(json.dumps({"copy_mib": mib, "ms": round(ms, 4),
                      "GBps": round(2 * mib * (1 << 20) / (ms * 1e-3) / 1e9, 1)}), flush=True)


def conv_traffic(n_in, n_out, P, K, cin, cout, s):
    """Algorithmic FLOPs and compulsory HBM bytes per launch of each pass.

    F = 2 P Cin Cout per pass. Bytes: read the gathered operand rows once,
    the weights once, write the result rows once, read the (in, out) int32
    pair list once (8 P); dW keeps an fp32 accumulator (K Cin Cout 4 B).
    """
    F = 2.0 * P * cin * cout
    w = K * cin * cout * s
    return {
        "forward": (F, n_in * cin * s + w + n_out * cout * s + 8.0 * P),
        "backward_input": (F, n_out * cout * s + w + n_in * cin * s + 8.0 * P),
        "backward_weight": (F, n_in * cin * s + n_out * cout * s + K * cin * cout * 4 + 8.0 * P),
    }


def measured_traffic(dtype: str, pass_name, record: str = "traffic_config2.json"):
    """(HBM bytes per launch of a pass's kernels, source) from the committed
    rocprofv3 passes, profiles/traffic_config2.json for the convolution and
    traffic_pool.json for pooling: read bytes from the
    TCC_EA0_RDREQ_{32B,64B,128B} request counts, write bytes from WRITE_SIZE,
    both exact on a device copy of known size; pass_name None reads a record
    of its own, such as the kernel-map build's ("kernel_map"). The source
    names the record and the commit of the kernels it was taken on; (None,
    None) if absent."""
    path = os.path.join(ROOT, "profiles", record)
    try:
        with open(path) as f:
            doc = json.load(f)
        rec = doc[dtype] if pass_name is None else doc[dtype][pass_name]
    except (OSError, KeyError, ValueError):
        return None, None
    src = f"profiles/{record}"
    if doc.get("kernels_commit"):
        src += f" (kernels at commit {doc['kernels_commit']})"
    return round(float(rec["traffic_bytes"])), src


def measured_mfma(dtype: str, pass_name: str, flop: float):
    """Counter-backed MFMA record of a config-2 pass from the committed
    rocprofv3 passes (profiles/traffic_config2.json): the share of the
    kernel's time the matrix pipes were busy, the MFMA FLOP issued per
    algorithmic FLOP (work on masked rows of the 16-row groups and empty
    positions shows as > 1) and the clock the box ran at; None if absent."""
    path = os.path.join(ROOT, "profiles", "traffic_config2.json")
    try:
        with open(path) as f:
            doc = json.load(f)
        rec = doc[dtype][pass_name]
        return {"util": round(rec["mfma_util"], 4),
                "flop_ratio": round(rec["mfma_flop"] / flop, 4),
                "clock_ghz": round(rec["clock_ghz"], 3),
                "source": "profiles/traffic_config2.json (SQ_VALU_MFMA_BUSY_CYCLES, "
                          "SQ_INSTS_VALU_MFMA_MOPS_*, GRBM_GUI_ACTIVE; kernels at commit %s)"
                          % doc.get("kernels_commit")}
    except (OSError, KeyError, ValueError, ZeroDivisionError):
        return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(coords, offsets, cin, cout, seed, dtype):
    """The CPU baseline on scene 0 of the workload (a bounded sample, ~1-3 s).

    Where oracle/_ref was built, it is the reference itself: its CPU path
    (CoordinateManager + RiemannConvolution over LibTorch, compiled from the
    reference sources) with LibTorch's intra-op threads. The first forward
    builds the kernel map; the timed fwd+dX+dW steps reuse it. Otherwise the
    scalar C oracle on one thread. Returns the cpu_baseline record."""
    import oracle  # checker and CPU baseline only; never on the GPU path
    from oracle import ref

    c1 = coords[coords[:, 0] == 0]
    K = offsets.shape[0]
    if ref.available():
        reps = 3
        P, first_ms, step_ms = ref.conv_time(c1, cin, cout, ks=3, bf16=dtype == "bf16",
                                             reps=reps, seed=seed)
        return {
            "value": round(len(c1) / (step_ms * 1e-3) / 1e6, 6),
            "unit": "Mvoxels/s",
            "cores": ref.num_threads(),
            "kind": "reference",
            "sample": (f"scene 0 of the workload: {len(c1)} voxels, P={P}, 3^3 C{cin}->{cout} "
                       f"{dtype} fwd+dX+dW, mean of {reps} steps ({step_ms:.1f} ms each) with "
                       f"the map cached; first forward incl. kernel map {first_ms:.1f} ms"),
            "first_forward_ms": round(first_ms, 2),
            "cpu_model": cpu_model(),
            "nproc": os.cpu_count(),
        }
    rng = np.random.default_rng(seed + 100)
    x = rng.standard_normal((len(c1), cin)).astype(np.float32)
    w = (rng.standard_normal((K, cin, cout)) * np.sqrt(2.0 / (cin * K))).astype(np.float32)
    gy = rng.standard_normal((len(c1), cout)).astype(np.float32)
    t0 = time.perf_counter()
    kofs, ir, orr = oracle.kernel_map(c1, c1, offsets)
    t_map = time.perf_counter() - t0
    t0 = time.perf_counter()
    oracle.conv_forward(x, w, kofs, ir, orr, len(c1))
    oracle.conv_backward(x, gy, w, kofs, ir, orr)
    t_conv = time.perf_counter() - t0
    return {
        "value": round(len(c1) / t_conv / 1e6, 6),
        "unit": "Mvoxels/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"scene 0 of the workload: {len(c1)} voxels, P={int(kofs[-1])}, "
                   f"3^3 C{cin}->{cout} fp32 fwd+dX+dW with the map prebuilt "
                   f"({t_conv:.2f} s); kernel map alone {t_map * 1e3:.1f} ms"),
        "kernel_map_ms": round(t_map * 1e3, 2),
        "cpu_model": cpu_model(),
        "nproc": os.cpu_count(),
    }



# ------------------------------------------------------- other configs

def cpu_map_baseline(coords):
    """The reference's CPU kernel-map build (insert_and_map, then the 3^3 cube
    kernel map) on scene 0 of the workload, timed apart from the convolution;
    None where oracle/_ref was not built (the scalar C oracle's map time is in
    the cpu_baseline record then)."""
    from oracle import ref  # CPU baseline only
    if not ref.available():
        return None
    c1 = coords[coords[:, 0] == 0]
    reps = 3
    P, hash_ms, map_ms = ref.map_time(c1, ks=3, reps=reps)
    return {
        "value": round(len(c1) / ((hash_ms + map_ms) * 1e-3) / 1e6, 4),
        "unit": "Mvoxels/s",
        "ms": round(hash_ms + map_ms, 2),
        "hash_ms": round(hash_ms, 2),
        "kernel_map_ms": round(map_ms, 2),
        "cores": ref.num_threads(),
        "kind": "reference",
        "sample": (f"scene 0 of the workload: {len(c1)} voxels, P={P}; "
                   f"CoordinateManager::insert_and_map then the 3^3 kernel map, "
                   f"mean of {reps} runs from a fresh manager"),
    }


@contextlib.contextmanager
def _no_gc():
    """Timed regions run with Python's cyclic collector off (collected just
    before): a full collection stalls the launching thread for tens of ms,
    which the GPU sees as idle time inside whichever pass it lands in."""
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


def _timed_passes(passes, steps, warmup):
    """Run the named passes in order `warmup` times, then `steps` timed times
    (host clock around a synchronize), then up to 10 untimed times with HIP
    events between passes (torch's current stream, where the C ABI and the
    host layer launch): event records cost a step a few microseconds, so
    they stay out of the timed steps. Returns (mean ms per pass, wall ms per
    step)."""
    import torch
    for _ in range(warmup):
        for _, fn in passes:
            fn()
    torch.cuda.synchronize()
    with _no_gc():
        t0 = time.perf_counter()
        for _ in range(steps):
            for _, fn in passes:
                fn()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
    nb = max(3, min(steps, 10))
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(passes) + 1)]
          for _ in range(nb)]
    for i in range(nb):
        ev[i][0].record()
        for j, (_, fn) in enumerate(passes):
            fn()
            ev[i][j + 1].record()
    torch.cuda.synchronize()
    per = {name: statistics.mean(e[j].elapsed_time(e[j + 1]) for e in ev)
           for j, (name, _) in enumerate(passes)}
    return per, wall


def _map_time(build, reps, warmup=5):
    """Host-clock median of `build()` over `reps` builds after `warmup`
    untimed ones (hash + map calls read sizes back), the way the steps get
    their warm-up."""
    import torch
    out, ms = None, []
    with _no_gc():
        for i in range(warmup + reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = build()
            torch.cuda.synchronize()
            if i >= warmup:
                ms.append((time.perf_counter() - t0) * 1e3)
    return out, statistics.median(ms)


def _roof(F, B, ms, dtype):
    """(bound, achieved, peak, unit, frac, t_roof_ms) of one pass: bound by
    whichever of the MFMA peak (the dtype's) and the HBM peak would take
    longer on its algorithmic work."""
    t_f = F / (PEAK_TFLOPS[dtype] * 1e12)
    t_b = B / (PEAK_HBM_GBS * 1e9)
    dur = ms * 1e-3
    if t_f >= t_b:
        rec = {"bound": "mfma", "achieved": round(F / dur / 1e12, 3), "peak": PEAK_TFLOPS[dtype],
               "unit": "TFLOP/s"}
    else:
        rec = {"bound": "hbm", "achieved": round(B / dur / 1e9, 1), "peak": PEAK_HBM_GBS,
               "unit": "GB/s"}
    rec["frac"] = round(max(t_f, t_b) / dur, 4)
    rec["ms"] = round(ms, 4)
    return rec


def _event_time(fn, reps=10, warm=3):
    """Mean duration (ms) of fn() from HIP events on torch's current stream
    (where the C ABI launches)."""
    import torch
    for _ in range(warm):
        fn()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record()
    for i in range(reps):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    return statistics.mean(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))


def config5_per_kernel(stage_in, stage_out, chans, dt, s, reps=10):
    """Config 5's kernels one by one, at each stage's real shapes, through
    the C ABI on maps built from the encoder's own coordinates: per stage,
    the 3^3 conv (C->C; 4 per step: two BasicBlocks of two convs) forward,
    dX and dW, the 2^3 stride-2 conv (C->C') forward, dX and dW (1 per
    step), and batch norm forward (statistics + apply with ReLU) and
    backward (4 each per step). Each entry: HIP-event mean over `reps`
    launches and its roofline fraction (bytes of the section-3 table for
    batch norm: statistics N C s, apply 2 N C s, backward sums 3 N C s and
    apply 5 N C s with the residual)."""
    import torch
    from riemannengine_amd import abi, stencil
    out = []
    g = torch.Generator(device="cpu").manual_seed(5)
    dev = stage_in[0].device
    rnd = lambda *shape: torch.randn(shape, generator=g).to(dev, dt)
    dname = "f32" if dt == torch.float32 else "bf16"
    for i, (ci, co_) in enumerate(zip(stage_in, stage_out)):
        C, Cn = chans[i], chans[min(i + 1, 3)]
        ts = 2 ** i
        ti = abi.hash_build(ci.contiguous())
        tn = abi.hash_build(co_.contiguous())
        k3 = abi.kernel_map(ti, ti, stencil.region_offsets(3, 3, 1, ts))
        kd = abi.kernel_map(ti, tn, stencil.region_offsets(3, 2, 1, ts))
        n, nn_ = k3.n_in, kd.n_out
        for op, km, cin, cout, count in (("conv 3^3", k3, C, C, 4), ("conv 2^3 s2", kd, C, Cn, 1)):
            x, gy = rnd(km.n_in, cin), rnd(km.n_out, cout)
            w = rnd(km.K, cin, cout) * 0.05
            work = conv_traffic(km.n_in, km.n_out, km.n_pairs, km.K, cin, cout, s)
            for pname, fn in (("forward", lambda: abi.conv_forward(x, w, km)),
                              ("backward_input", lambda: abi.conv_backward_input(gy, w, km)),
                              ("backward_weight", lambda: abi.conv_weight_grad(x, gy, km, km.K))):
                ms = _event_time(fn, reps)
                F, B = work[pname]
                rec = {"stage": i + 1, "op": f"{op} C{cin}->{cout}", "pass": pname,
                       "rows_in": km.n_in, "rows_out": km.n_out, "pairs": km.n_pairs,
                       "per_step": count}
                rec.update(_roof(F, B, ms, dname))
                out.append(rec)
            del x, gy, w
        x, r, gy = rnd(n, C), rnd(n, C), rnd(n, C)
        gamma = torch.ones(C, device=dev)
        beta = torch.zeros(C, device=dev)
        st = {}

        def bn_fwd():
            st["m"], st["v"] = abi.bn_stats(x)
            st["y"] = abi.bn_forward(x, st["m"], st["v"], gamma, beta, residual=r, relu=True)

        bn_fwd()
        for pname, fn, B in (
                ("batch norm forward", bn_fwd, n * C * s * 4),
                ("batch norm backward",
                 lambda: abi.bn_backward(gy, st["y"], x, st["m"], st["v"], gamma, relu=True,
                                         want_residual=True), n * C * s * 8)):
            ms = _event_time(fn, reps)
            rec = {"stage": i + 1, "op": f"batch norm C{C}", "pass": pname, "rows_in": n,
                   "per_step": 4}
            rec.update(_roof(0.0, float(B), ms, dname))
            out.append(rec)
        del x, r, gy, k3, kd, ti, tn
    return out


def run_other_config(args):
    """Configs 1, 3, 4 and 5 of the benchmark set, one JSON record each:
      1  sphere shell (N = 51,554), 3^3 C16->32, fwd+dX+dW (C ABI)
      3  LiDAR batch 2 (151,273 voxels): 2^3 stride-2 conv C64->128, then the
         2^3 transposed conv C128->64 back onto the input coordinates,
         fwd+bwd (C ABI)
      4  4-D moving shell (N = 232,528), 3^4 (81 offsets) C32->32 (C ABI)
      5  residual encoder on 8 indoor scenes: 4 stages of 2 BasicBlocks and a
         2^3 stride-2 conv, channels 32->64->128->256, fwd+bwd through the
         C++ host layer (autograd, batch norm, maps cached by the manager)
    value = N_in / ms_per_step (Mvoxels/s) with the maps prebuilt; the step
    roofline fraction divides the step's roofline time by the timed
    ms_per_step; `passes` gives each pass's own roofline fraction from
    event times (config 5: `per_kernel`, each kernel at each stage)."""
    import torch
    from riemannengine_amd import abi, scenes, stencil

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (the HIP path has no CPU fallback)", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dt = torch.float32 if args.dtype == "f32" else torch.bfloat16
    s = 4 if args.dtype == "f32" else 2
    g = torch.Generator(device="cpu").manual_seed(args.seed)
    rnd = lambda *shape: torch.randn(shape, generator=g).to(dev, dt)
    kaiming = lambda K, ci, co: rnd(K, ci, co) * (2.0 / (ci * K)) ** 0.5
    cfg = args.config
    extra = {}
    work = {}  # pass name -> (F, B)

    if cfg in (1, 4):
        if cfg == 1:
            c_np, D, cin, cout = scenes.sphere_shell(), 3, 16, 32
            desc = "config 1: sphere shell r=64, 3^3 stride-1 conv C16->32, fwd+dX+dW"
        else:
            c_np, D, cin, cout = scenes.moving_shell_4d(), 4, 32, 32
            desc = "config 4: 4-D shell, 8 frames, 3^4 (81 offsets) stride-1 conv C32->32, fwd+dX+dW"
        coords = torch.from_numpy(c_np).to(dev)
        off = stencil.region_offsets(D, 3)
        K = off.shape[0]
        (table, km), map_ms = _map_time(
            lambda: (lambda t: (t, abi.kernel_map(t, t, off)))(abi.hash_build(coords)),
            args.map_reps)
        n_in = km.n_in
        x, w, gy = rnd(n_in, cin), kaiming(K, cin, cout), rnd(n_in, cout)
        passes = [("forward", lambda: abi.conv_forward(x, w, km)),
                  ("backward_input", lambda: abi.conv_backward_input(gy, w, km)),
                  ("backward_weight", lambda: abi.conv_weight_grad(x, gy, km, K))]
        work = conv_traffic(n_in, n_in, km.n_pairs, K, cin, cout, s)
        extra = {"n_voxels": n_in, "pairs": km.n_pairs, "offsets": K, "c_in": cin, "c_out": cout}
    elif cfg == 3:
        c_np = scenes.lidar_batch(2, 3)
        coords = torch.from_numpy(c_np).to(dev)
        off = stencil.region_offsets(3, 2)

        def build():
            tf = abi.hash_build(coords)
            tc = abi.hash_build(abi.stride_coords(coords, [2, 2, 2]))
            return tf, tc, abi.kernel_map(tf, tc, off)
        (tf, tc, down), map_ms = _map_time(build, args.map_reps)
        up = down.swapped()
        n_f, n_c, P = down.n_in, down.n_out, down.n_pairs
        x, wd, wu = rnd(n_f, 64), kaiming(8, 64, 128), kaiming(8, 128, 64)
        y = abi.conv_forward(x, wd, down)
        gz = rnd(n_f, 64)
        gy = abi.conv_backward_input(gz, wu, up)
        passes = [("down_forward", lambda: abi.conv_forward(x, wd, down)),
                  ("up_forward", lambda: abi.conv_forward(y, wu, up)),
                  ("up_backward_input", lambda: abi.conv_backward_input(gz, wu, up)),
                  ("up_backward_weight", lambda: abi.conv_weight_grad(y, gz, up, 8)),
                  ("down_backward_input", lambda: abi.conv_backward_input(gy, wd, down)),
                  ("down_backward_weight", lambda: abi.conv_weight_grad(x, gy, down, 8))]
        for pre, (ni, no, ci, co) in (("down_", (n_f, n_c, 64, 128)), ("up_", (n_c, n_f, 128, 64))):
            for name, fb in conv_traffic(ni, no, P, 8, ci, co, s).items():
                work[pre + name] = fb
        n_in = n_f
        desc = ("config 3: LiDAR batch 2, 2^3 stride-2 conv C64->128 then 2^3 transposed conv "
                "C128->64 onto the input coordinates, fwd+bwd")
        extra = {"n_voxels": n_f, "n_coarse": n_c, "pairs": P, "c": [64, 128, 64]}
    else:  # config 5
        import riemannengine_amd as re_
        c_np = scenes.indoor_batch(8, args.seed)
        coords = torch.from_numpy(c_np).to(dev)
        chans = [32, 64, 128, 256]
        mods = []
        for i, c in enumerate(chans):
            mods += [re_.nn.BasicBlock(c, c), re_.nn.BasicBlock(c, c),
                     re_.nn.RiemannConvolution(c, chans[min(i + 1, 3)], kernel_size=2, stride=2,
                                               dimension=3)]
        for m in mods:
            m.to(dev)
            m.to_dtype(dt)
        feats = rnd(len(c_np), 32)
        x0 = re_.SparseTensor(feats, coords)
        n_in = len(x0)
        state = {}
        stage_in, stage_out = [], []

        def forward(record=False):
            h = x0
            for j, m in enumerate(mods):
                if record and j % 3 == 0:
                    stage_in.append(h.C)
                h = m(h)
                if record and j % 3 == 2:
                    stage_out.append(h.C)
            state["out"] = h

        def backward():
            state["out"].F.float().sum().backward()
            for m in mods:
                m.zero_grad()

        torch.cuda.synchronize()
        t0 = time.perf_counter()
        forward(record=True)  # builds every stage's maps; the manager caches them
        torch.cuda.synchronize()
        first_ms = (time.perf_counter() - t0) * 1e3
        backward()
        passes = [("forward", forward), ("backward", backward)]
        map_ms = None
        desc = ("config 5: residual encoder on 8 indoor scenes, 4 stages x (2 BasicBlocks + "
                "2^3 stride-2 conv), C 32->64->128->256, fwd+bwd through the host layer")
        extra = {"n_voxels": n_in, "out_voxels": len(state["out"]), "stages": 4,
                 "channels": chans, "first_forward_ms_incl_maps": round(first_ms, 2)}

    per, wall = _timed_passes(passes, args.steps, args.warmup)
    line = {
        "metric": f"sparse conv fwd+bwd Mvoxels/s (config {cfg})",
        "value": round(n_in / (wall * 1e-3) / 1e6, 3),
        "unit": "Mvoxels/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": args.dtype,
        "data": "synthetic (seeded scenes; random N(0,1) features, Kaiming-normal weights)",
        "config": dict({"workload": desc, "seed": args.seed, "accumulate": "f32"}, **extra),
        "kernel_map_ms": None if map_ms is None else round(map_ms, 3),
        "breakdown_ms": {k: round(v, 4) for k, v in per.items()},
        "breakdown_source": "events around each pass in untimed steps after the timed ones",
    }
    if work:
        flop = sum(v[0] for v in work.values())
        byts = sum(v[1] for v in work.values())
        t_roof = max(flop / (PEAK_TFLOPS[args.dtype] * 1e12), byts / (PEAK_HBM_GBS * 1e9))
        line["step_roofline"] = {"t_roof_ms": round(t_roof * 1e3, 4),
                                 "frac": round(t_roof * 1e3 / wall, 4),
                                 "frac_source": "t_roof / timed ms_per_step",
                                 "flop": flop, "bytes": byts}
        line["passes"] = {name: _roof(*work[name], per[name], args.dtype) for name in per}
        dom = max(per, key=per.get)
        line["roofline"] = dict(line["passes"][dom], **{"pass": dom})
    else:  # config 5: each kernel at each stage
        pk = config5_per_kernel(stage_in, stage_out, chans, dt, s)
        t_roof = sum(r["frac"] * r["ms"] * r["per_step"] for r in pk)
        t_sum = sum(r["ms"] * r["per_step"] for r in pk)
        line["per_kernel"] = pk
        line["step_roofline"] = {
            "t_roof_ms": round(t_roof, 4), "frac": round(t_roof / wall, 4),
            "frac_source": "sum over the per-kernel entries of (roofline time x launches per "
                           "step) / timed ms_per_step",
            "kernels_ms": round(t_sum, 4)}
        dom = max(pk, key=lambda r: r["ms"] * r["per_step"])
        line["roofline"] = dict(dom)
    return line


def compact(line):
    """The fields of a config's line that the headline line carries."""
    keep = ("value", "unit", "dtype", "ms_per_step", "kernel_map_ms", "breakdown_ms",
            "step_roofline", "roofline", "passes", "per_kernel")
    out = {k: line[k] for k in keep if k in line}
    out["config"] = line["config"]
    return out


def pool_traffic(kind, n_in, n_out, K, C, s, ncol=4, K_t=None):
    """Algorithmic HBM bytes of one pooling kernel pass: every feature row it
    must touch read (or written) once, plus its index tables (nbr K rows,
    nbr_t K_t rows, default K); no re-reads."""
    K_t = K if K_t is None else K_t
    if kind == "forward":      # x rows, nbr [K, n_out], order; y, counts
        return n_in * C * s + K * n_out * 4 + n_out * 4 + n_out * C * s + n_out * 4
    if kind == "backward":     # gy rows, counts, nbr_t [K_t, n_in], order; gx
        return n_out * C * s + n_out * 4 + K_t * n_in * 4 + n_in * 4 + n_in * C * s
    if kind == "max_backward":  # share pass (y, gy, x, nbr; gs fp32) + gather pass
        share = 2 * n_out * C * s + n_in * C * s + K * n_out * 4 + n_out * 4 + n_out * C * 4
        gather = n_in * C * s + n_out * C * s + n_out * C * 4 + K_t * n_in * 4 + n_in * 4 \
            + n_in * C * s
        return share + gather
    if kind == "global_forward":   # x rows + members; y (n_out = batches) negligible
        return n_in * C * s + n_in * 4 + n_out * C * s
    if kind == "global_backward":  # coordinate rows (batch column) + gx
        return n_in * ncol * 4 + n_in * C * s + n_out * C * s
    raise ValueError(kind)


def pool_cpu_baseline(coords_np, C, seed, rows=20000):
    """The reference's pooling layers on the CPU (oracle/_ref) over a bounded
    sample of the workload: the first `rows` voxels of scene 0 in (x, y, z)
    order (a slab of the scene), RiemannMaxPooling(2, 2), RiemannAvgPooling
    (3, 2) and RiemannGlobalAvgPooling, forward + backward each, fp32. The
    reference builds its pooling maps on every call (pooling.cpp:17-75), so
    they are part of its time; it pools output by output, which is why the
    sample is a slab (the whole 100k-voxel scene takes minutes)."""
    from oracle import ref
    if not ref.available():
        return None
    scene = coords_np[coords_np[:, 0] == 0]
    scene = scene[np.lexsort(scene[:, ::-1].T)][:rows]
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((len(scene), C)).astype(np.float32)
    total = 0.0
    for mode, ks in (("max", 2), ("avg", 3)):
        y, _, _ = ref.pool(scene, x, mode, ks, 2)
        gy = np.ones_like(y)
        t0 = time.perf_counter()
        ref.pool(scene, x, mode, ks, 2, gy=gy)
        total += time.perf_counter() - t0
    gy = np.ones((1, C), np.float32)
    t0 = time.perf_counter()
    ref.global_pool(scene, x, "avg", gy=gy)
    total += time.perf_counter() - t0
    return {"value": round(len(scene) / total / 1e6, 5), "unit": "Mvoxels/s",
            "cores": ref.num_threads(), "kind": "reference",
            "sample": f"first {len(scene)} voxels of scene 0 in (x, y, z) order, C={C} fp32, "
                      "one max 2^3/2 + avg 3^3/2 + global avg forward+backward, maps included",
            "ms": round(total * 1e3, 1), "cpu": cpu_model()}


def run_pool(args):
    """Pooling line: on the config-2 coordinates (4 indoor scenes), C = 64,
    one step = RiemannMaxPooling(2, 2) over the stride map, RiemannAvgPooling
    (3, 2) over the 3^3 kernel map and global average pooling, forward and
    backward each, through the C ABI with the maps prebuilt."""
    import torch
    from riemannengine_amd import abi, scenes, stencil

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (the HIP path has no CPU fallback)", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dt = torch.float32 if args.dtype == "f32" else torch.bfloat16
    s = 4 if args.dtype == "f32" else 2
    C = 64
    coords_np = scenes.indoor_batch(4, args.seed)
    coords = torch.from_numpy(coords_np).to(dev)
    off3 = stencil.region_offsets(3, 3)

    def build():
        tf = abi.hash_build(coords)
        tc = abi.hash_build(abi.stride_coords(coords, [2, 2, 2]))
        return tf, tc, abi.stride_map(tf, tc, [2, 2, 2]), \
            abi.pooling_map(abi.kernel_map(tf, tc, off3)), abi.batch_segments(coords)
    (tf, tc, sm, km, segs), map_ms = _map_time(build, args.map_reps)
    n_in, n_out = tf.n, tc.n
    g = torch.Generator(device="cpu").manual_seed(args.seed)
    x = torch.randn((n_in, C), generator=g).to(dev, dt)
    gy = torch.randn((n_out, C), generator=g).to(dev, dt)
    gyb = torch.randn((segs.n_batches, C), generator=g).to(dev, dt)
    ym, cm = abi.pool_forward(x, sm, "max")
    ya, ca = abi.pool_forward(x, km, "avg")
    yg = abi.global_pool_forward(x, segs, "avg")
    passes = [("max2_forward", lambda: abi.pool_forward(x, sm, "max")),
              ("max2_backward", lambda: abi.pool_backward(gy, ym, x, sm, cm, "max")),
              ("avg3_forward", lambda: abi.pool_forward(x, km, "avg")),
              ("avg3_backward", lambda: abi.pool_backward(gy, ya, x, km, ca, "avg")),
              ("global_forward", lambda: abi.global_pool_forward(x, segs, "avg")),
              ("global_backward", lambda: abi.global_pool_backward(gyb, yg, x, coords, segs,
                                                                   "avg"))]
    per, wall = _timed_passes(passes, args.steps, args.warmup)
    B = {"max2_forward": pool_traffic("forward", n_in, n_out, sm.K, C, s),
         "max2_backward": pool_traffic("max_backward", n_in, n_out, sm.K, C, s,
                                       K_t=sm.nbr_t.shape[0]),
         "avg3_forward": pool_traffic("forward", n_in, n_out, km.K, C, s),
         "avg3_backward": pool_traffic("backward", n_in, n_out, km.K, C, s,
                                       K_t=km.nbr_t.shape[0]),
         "global_forward": pool_traffic("global_forward", n_in, segs.n_batches, 0, C, s),
         "global_backward": pool_traffic("global_backward", n_in, segs.n_batches, 0, C, s)}
    dom = max(per, key=per.get)
    achieved = B[dom] / (per[dom] * 1e-3) / 1e9
    kernels = {"max2_forward": "pool_fwd_kernel (max, stride map)",
               "max2_backward": "pool_maxshare_kernel + pool_bwd_kernel (max, stride map)",
               "avg3_forward": "pool_fwd_kernel (avg, 3^3 kernel map)",
               "avg3_backward": "pool_bwd_kernel (avg, 3^3 kernel map)",
               "global_forward": "gpool_partial_kernel + gpool_final_kernel (avg)",
               "global_backward": "gpool_bwd_kernel (avg)"}
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic(args.dtype, dom, "traffic_pool.json")[0],
            "traffic_source": measured_traffic(args.dtype, dom, "traffic_pool.json")[1],
            "kernel": kernels[dom],
            "kernel_ms": round(per[dom], 4), "algorithmic": {"bytes": B[dom]}}
    t_roof = sum(B.values()) / (PEAK_HBM_GBS * 1e9)
    line = {
        "metric": "sparse pooling fwd+bwd Mvoxels/s (max 2^3/2 + avg 3^3/2 + global avg, C64)",
        "value": round(n_in / (wall * 1e-3) / 1e6, 3), "unit": "Mvoxels/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(wall, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": args.dtype,
        "data": "synthetic (seeded indoor scenes; random N(0,1) features and gradients)",
        "config": {"workload": "pooling on the config-2 coordinates (indoor scenes batch 4): "
                               "max 2^3 stride 2 (stride map), avg 3^3 stride 2 (kernel map), "
                               "global avg; forward+backward, maps prebuilt",
                   "n_voxels": n_in, "n_coarse": n_out, "stride_map_rows": sm.K,
                   "kernel_map_pairs": km.n_pairs, "batches": segs.n_batches, "channels": C,
                   "seed": args.seed, "accumulate": "f32"},
        "kernel_map_ms": round(map_ms, 3),
        "breakdown_ms": {k: round(v, 4) for k, v in per.items()},
        "step_roofline": {"t_roof_ms": round(t_roof * 1e3, 4),
                          "frac": round(t_roof * 1e3 / wall, 4),
                          "frac_source": "t_roof / timed ms_per_step", "bytes": sum(B.values())},
        "roofline": roof,
        "cpu_baseline": None if args.no_cpu_baseline else pool_cpu_baseline(coords_np, C,
                                                                            args.seed),
    }
    return line


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py: --gpus {max(args.gpus, world)} refused: this build runs and is measured "
              "on one GPU only (the path shards by scene; see the sharding notes)",
              file=sys.stderr)
        sys.exit(2)

    if args.copy_mib > 0:
        copy_calibration(args.copy_mib)
        return
    args.dtype_given = args.dtype is not None
    if args.dtype is None:
        args.dtype = "bf16" if args.config in (3, 5) else "f32"
    if args.op == "pool":
        print(json.dumps(run_pool(args)), flush=True)
        return
    if args.config != 2:
        print(json.dumps(run_other_config(args)), flush=True)
        return

    import torch
    from riemannengine_amd import abi, scenes, stencil

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (the HIP path has no CPU fallback)", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cin = cout = 64

    # ---------------------------------------------------------- workload
    coords_np = scenes.indoor_batch(4, args.seed)
    offsets_np = stencil.region_offsets(3, 3)
    K = offsets_np.shape[0]
    coords = torch.from_numpy(coords_np).to(dev)
    torch.cuda.synchronize()

    # kernel map: hash build + locality order + map (count, fill), from
    # coordinates already on the device; these calls read sizes back to the
    # host, so they are timed on the host clock around a synchronize. The
    # headline time goes through the C++ CoordinateManager (insert_and_map,
    # then kernel_map: the drop-in API, as the reference's CPU time below);
    # the C ABI driven from Python (abi.hash_build + abi.kernel_map, whose
    # result the steps use) is timed beside it.
    import riemannengine_amd as rea

    def manager_build():
        mgr = rea.CoordinateManager(3)
        key, _ = mgr.insert_and_map(coords, [1, 1, 1])
        return mgr.kernel_map(key, key, [3, 3, 3], [1, 1, 1], [1, 1, 1])

    def abi_build():
        table = abi.hash_build(coords)
        return abi.kernel_map(table, table, offsets_np)

    mgr_map, kmap_ms = _map_time(manager_build, args.map_reps)
    km, abi_map_ms = _map_time(abi_build, args.map_reps)
    assert int(mgr_map["offsets_host"][-1]) == km.n_pairs
    n_in = n_out = km.n_in
    P = km.n_pairs
    D = coords_np.shape[1] - 1
    # algorithmic bytes of the map build: hash build (read the rows, one slot
    # write, one row index) and map (read both sides' rows, one 8-byte probe
    # per query, write the pairs and the offsets)
    b_hash = len(coords_np) * (D + 1) * 4 + len(coords_np) * 8 + len(coords_np) * 4
    b_map = (n_in + n_out) * (D + 1) * 4 + K * n_out * 8 + 8 * P + 4 * (K + 1)
    map_gbs = (b_hash + b_map) / (kmap_ms * 1e-3) / 1e9
    map_traffic = measured_traffic("kernel_map", None)
    kmap_roof = {"bound": "hbm", "achieved": round(map_gbs, 1), "peak": PEAK_HBM_GBS,
                 "unit": "GB/s", "frac": round(map_gbs / PEAK_HBM_GBS, 4),
                 "algorithmic": {"hash_bytes": b_hash, "map_bytes": b_map},
                 "ms": round(kmap_ms, 3),
                 "path": "C++ CoordinateManager.insert_and_map + kernel_map",
                 "c_abi_from_python_ms": round(abi_map_ms, 3),
                 "traffic": map_traffic[0], "traffic_source": map_traffic[1],
                 "note": "host clock around the build calls, which read sizes back to the host"}

    dtypes = [args.dtype] if args.dtype_given else ["f32", "bf16"]
    records = {dt_name: conv_step_record(args, dt_name, km, n_in, n_out, P, K, cin, cout)
               for dt_name in dtypes}
    head = records[dtypes[0]]
    line = {
        "metric": "sparse conv fwd+bwd Mvoxels/s @3^3 C64",
        "value": head["value"],
        "unit": "Mvoxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtypes[0],
        "data": "synthetic (seeded indoor scenes; random N(0,1) features, Kaiming-normal weights)",
        "config": {"workload": "config 2: indoor scenes batch 4, 3^3 stride-1 conv C64->64, "
                               "fwd+dX+dW, kernel map prebuilt",
                   "n_voxels": n_in, "pairs": P, "offsets": K, "c_in": cin, "c_out": cout,
                   "seed": args.seed, "accumulate": "f32"},
        "kernel_map_ms": round(kmap_ms, 3),
        "kernel_map_roofline": kmap_roof,
        "breakdown_ms": head["breakdown_ms"],
        "step_roofline": head["step_roofline"],
        "roofline": head["roofline"],
    }
    for dt_name in dtypes[1:]:
        line[dt_name] = records[dt_name]
    if not args.dtype_given and not args.no_other_configs:
        # the other configurations, each in its own dtype, as compact records
        import copy
        import torch
        line["configs"] = {}
        for cfg in (1, 3, 4, 5):
            sub = copy.copy(args)
            sub.config = cfg
            sub.dtype = "bf16" if cfg in (3, 5) else "f32"
            line["configs"][str(cfg)] = compact(run_other_config(sub))
            gc.collect()
            torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(coords_np, offsets_np, cin, cout, args.seed,
                                            dtypes[0])
        line["cpu_kernel_map_baseline"] = cpu_map_baseline(coords_np)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


def conv_step_record(args, dtype, km, n_in, n_out, P, K, cin, cout):
    """Config 2 in one dtype: Mvoxels/s over the timed steps (forward, dX and
    dW through the C ABI, the map prebuilt), the per-pass event times, the
    whole-step roofline and the dominant pass's roofline with its measured
    HBM traffic."""
    import torch
    from riemannengine_amd import abi
    dev = torch.device("cuda:0")
    dt = torch.float32 if dtype == "f32" else torch.bfloat16
    s = 4 if dtype == "f32" else 2
    g = torch.Generator(device="cpu").manual_seed(args.seed)
    x = torch.randn((n_in, cin), generator=g).to(dev, dt)
    w = (torch.randn((K, cin, cout), generator=g) * (2.0 / (cin * K)) ** 0.5).to(dev, dt)
    gy = torch.randn((n_out, cout), generator=g).to(dev, dt)

    def step(ev=None):
        """One step; ev: None, two events around dW, or four around each pass."""
        if ev is not None and len(ev) == 4:
            ev[0].record()
        abi.conv_forward(x, w, km)
        if ev is not None and len(ev) == 4:
            ev[1].record()
        abi.conv_backward_input(gy, w, km)
        if ev is not None:
            ev[-2].record()
        abi.conv_weight_grad(x, gy, km, K)
        if ev is not None:
            ev[-1].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # every tenth timed step (at least one) records events around the dW
    # pass, the dominant pass of this workload in both dtypes: an event record
    # leaves the device idle for ~6 us (kernel trace: a gap at each one), so
    # events in every step would add ~12 us to each
    every = 10
    sampled = set(range(0, args.steps, every))
    events = {i: [torch.cuda.Event(enable_timing=True) for _ in range(2)] for i in sampled}
    torch.cuda.synchronize()
    with _no_gc():
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(events.get(i))
        torch.cuda.synchronize()
        total_s = time.perf_counter() - t0
    ms_per_step = total_s * 1e3 / args.steps
    dw_timed = statistics.mean(e[0].elapsed_time(e[1]) for e in events.values())

    # per-pass breakdown from untimed steps after the timed region
    names = ["forward", "backward_input", "backward_weight"]
    nb = max(3, min(args.steps, 10))
    bev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(nb)]
    for i in range(nb):
        step(bev[i])
    torch.cuda.synchronize()
    per = {n: statistics.mean(e[j].elapsed_time(e[j + 1]) for e in bev)
           for j, n in enumerate(names)}
    work = conv_traffic(n_in, n_out, P, K, cin, cout, s)
    dom = max(names, key=lambda n: per[n])
    F, B = work[dom]
    # the dominant pass's duration from the timed steps where that is dW
    kernel_ms = dw_timed if dom == "backward_weight" else per[dom]
    dur_s = kernel_ms * 1e-3
    if dtype == "f32":
        roof = {"bound": "mfma", "achieved": round(F / dur_s / 1e12, 3),
                "peak": PEAK_TFLOPS["f32"], "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": round(B / dur_s / 1e9, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"], roof["traffic_source"] = measured_traffic(dtype, dom)
    roof["mfma"] = measured_mfma(dtype, dom, F)
    roof["kernel"] = {"forward": "conv_os_lds_kernel (forward)",
                      "backward_input": "conv_os_lds_kernel (dX)",
                      "backward_weight": (
                          "conv_dw_pos64_kernel + conv_dw_rows_reduce_kernel (dW pass)"
                          if dtype == "f32" else
                          "conv_dw_shx_bf16_kernel + conv_dw_rows_reduce_kernel (dW pass)")}[dom]
    roof["kernel_ms"] = round(kernel_ms, 4)
    roof["kernel_ms_source"] = ("events around dW in every %dth timed step" % every
                                if dom == "backward_weight"
                                else "events in %d untimed steps after the timed ones" % nb)
    roof["algorithmic"] = {"flop": F, "bytes": B}

    # whole-step roofline: max(compute, memory) time at peak / measured
    Ft = sum(v[0] for v in work.values())
    Bt = sum(v[1] for v in work.values())
    t_roof = max(Ft / (PEAK_TFLOPS[dtype] * 1e12), Bt / (PEAK_HBM_GBS * 1e9))
    return {
        "value": round(n_in / (ms_per_step * 1e-3) / 1e6, 3),
        "unit": "Mvoxels/s",
        "dtype": dtype,
        "ms_per_step": round(ms_per_step, 4),
        "breakdown_ms": {n: round(per[n], 4) for n in names},
        "breakdown_source": "events around each pass in %d untimed steps after the timed ones" % nb,
        "step_roofline": {"t_roof_ms": round(t_roof * 1e3, 4),
                          "frac": round(t_roof * 1e3 / ms_per_step, 4),
                          "frac_source": "t_roof / timed ms_per_step",
                          "flop": Ft, "bytes": Bt},
        "roofline": roof,
    }


if __name__ == "__main__":
    main()
