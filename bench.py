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
  value        whole-job Mvoxels/s = N_in / (t_fwd + t_dX + t_dW) / 1e6
  kernel_map_ms  hash build + locality order + kernel map, from device coords
  roofline     the dominant kernel's algorithmic FLOP/s (fp32, MFMA-bound) or
               bytes/s (bf16, HBM-bound), from HIP events recorded on the
               stream the kernels run on, against MI355X's published peak
  cpu_baseline the reference's own CPU path (compiled from its sources into
               oracle/_ref) timed on one scene of the same workload, or the
               scalar C oracle where that library was not built

--gpus N > 1 is refused: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
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
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--dtype", choices=["f32", "bf16"], default="f32",
                    help="feature/weight dtype of the headline line (fp32 accumulate)")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the CPU oracle timing (profiling runs)")
    ap.add_argument("--map-reps", type=int, default=5)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="calibration mode: time a plain device copy of this many MiB "
                         "(the reference kernel for scaling FETCH_SIZE/WRITE_SIZE) and exit")
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


def measured_traffic(dtype: str, pass_name: str):
    """HBM bytes per launch of a pass's kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes (profiles/traffic_config2.json, scaled by
    the counters' reading for a device copy of known size); None if absent."""
    path = os.path.join(ROOT, "profiles", "traffic_config2.json")
    try:
        with open(path) as f:
            rec = json.load(f)[dtype][pass_name]
    except (OSError, KeyError, ValueError):
        return None
    return round(float(rec["traffic_bytes"]))


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

    import torch
    from riemannengine_amd import abi, scenes, stencil

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (the HIP path has no CPU fallback)", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dt = torch.float32 if args.dtype == "f32" else torch.bfloat16
    s = 4 if args.dtype == "f32" else 2
    cin = cout = 64

    # ---------------------------------------------------------- workload
    coords_np = scenes.indoor_batch(4, args.seed)
    offsets_np = stencil.region_offsets(3, 3)
    K = offsets_np.shape[0]
    coords = torch.from_numpy(coords_np).to(dev)
    offsets = torch.from_numpy(offsets_np).to(dev)
    torch.cuda.synchronize()

    # kernel map: hash build + locality order + map (count, fill), from
    # coordinates already on the device; these calls read sizes back to the
    # host, so they are timed on the host clock around a synchronize.
    map_ms = []
    for _ in range(args.map_reps + 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        table = abi.hash_build(coords)
        km = abi.kernel_map(table, table, offsets)
        torch.cuda.synchronize()
        map_ms.append((time.perf_counter() - t0) * 1e3)
    kmap_ms = statistics.median(map_ms[1:])
    n_in = n_out = km.n_in
    P = km.n_pairs

    g = torch.Generator(device="cpu").manual_seed(args.seed)
    x = torch.randn((n_in, cin), generator=g).to(dev, dt)
    w = (torch.randn((K, cin, cout), generator=g) * (2.0 / (cin * K)) ** 0.5).to(dev, dt)
    gy = torch.randn((n_out, cout), generator=g).to(dev, dt)

    def step(ev=None):
        if ev is not None:
            ev[0].record()
        abi.conv_forward(x, w, km)
        if ev is not None:
            ev[1].record()
        abi.conv_backward_input(gy, w, km)
        if ev is not None:
            ev[2].record()
        abi.conv_backward_weight(x, gy, km, K)
        if ev is not None:
            ev[3].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    total_s = time.perf_counter() - t0
    ms_per_step = total_s * 1e3 / args.steps

    names = ["forward", "backward_input", "backward_weight"]
    per = {n: statistics.mean(e[j].elapsed_time(e[j + 1]) for e in events)
           for j, n in enumerate(names)}
    work = conv_traffic(n_in, n_out, P, K, cin, cout, s)
    dom = max(names, key=lambda n: per[n])
    F, B = work[dom]
    dur_s = per[dom] * 1e-3
    if args.dtype == "f32":
        roof = {"bound": "mfma", "achieved": round(F / dur_s / 1e12, 3),
                "peak": PEAK_TFLOPS["f32"], "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": round(B / dur_s / 1e9, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = measured_traffic(args.dtype, dom)
    roof["kernel"] = {"forward": "conv_os_kernel (forward)",
                      "backward_input": "conv_os_kernel (dX)",
                      "backward_weight": "conv_dw_kernel + conv_dw_reduce_kernel (dW pass)"}[dom]
    roof["kernel_ms"] = round(per[dom], 4)
    roof["algorithmic"] = {"flop": F, "bytes": B}

    # whole-step roofline: max(compute, memory) time at peak / measured
    Ft = sum(v[0] for v in work.values())
    Bt = sum(v[1] for v in work.values())
    t_roof = max(Ft / (PEAK_TFLOPS[args.dtype] * 1e12), Bt / (PEAK_HBM_GBS * 1e9))
    step_ms_events = sum(per.values())

    value = n_in / (ms_per_step * 1e-3) / 1e6
    line = {
        "metric": "sparse conv fwd+bwd Mvoxels/s @3^3 C64",
        "value": round(value, 3),
        "unit": "Mvoxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded indoor scenes; random N(0,1) features, Kaiming-normal weights)",
        "config": {"workload": "config 2: indoor scenes batch 4, 3^3 stride-1 conv C64->64, "
                               "fwd+dX+dW, kernel map prebuilt",
                   "n_voxels": n_in, "pairs": P, "offsets": K, "c_in": cin, "c_out": cout,
                   "seed": args.seed, "accumulate": "f32"},
        "kernel_map_ms": round(kmap_ms, 3),
        "breakdown_ms": {n: round(per[n], 4) for n in names},
        "step_roofline": {"t_roof_ms": round(t_roof * 1e3, 4),
                          "frac": round(t_roof * 1e3 / step_ms_events, 4),
                          "flop": Ft, "bytes": Bt},
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(coords_np, offsets_np, cin, cout, args.seed,
                                            args.dtype)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
