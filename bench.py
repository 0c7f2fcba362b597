"""Benchmark: the 128->128 fp16 SubMConv3d layer over 500k surface voxels.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--encoder]

One step is one forward of the layer over the whole batch, with its indice
pairs cached under its ``indice_key`` (as a network reuses them), inputs
already resident in HBM.  The pair build, the execution-order plan and the
fused conv kernel are also timed on their own with HIP events on the stream
they run on.  Prints ONE JSON line:
  value         voxels/s of the layer (N_in / step time)
  roofline      the conv kernel against MI355X's dense fp16 MFMA peak
  cpu_baseline  the CPU oracle (a numpy port of the reference's CPU path)
                timed on this host on the same workload
Other workloads (``--workload``) are for exploration; the default is the one
the headline metric is quoted on.  ``--encoder`` times a multi-layer
workload's whole network instead of its first layer: the VoxelNet-style
encoder as a SparseSequential with an eval-mode BatchNorm1d + ReLU after every
layer but the last (fused into the conv stores, and unfused for comparison),
or the strided + inverse pair.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK = {  # MI355X published dense peaks
    "float16": (2500.0, "TFLOP/s"), "bfloat16": (2500.0, "TFLOP/s"),
    "float32": (157.3, "TFLOP/s"),
}
HBM_PEAK_GBS = 8000.0
DTYPE_TAG = {"float32": "f32", "float16": "f16", "bfloat16": "bf16"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the GPU needs some tens of milliseconds of load to reach its steady clock:
    # 100 warm-up steps of this layer take ~40 ms
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="subm128_surface500k")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run one elementwise negation over this many MiB (a copy-like "
                         "kernel of known size to scale FETCH_SIZE / WRITE_SIZE counters by)")
    ap.add_argument("--encoder", action="store_true",
                    help="time the workload's whole network (all layers) instead of layer 0")
    ap.add_argument("--verbose", action="store_true")
    return ap.parse_args()


def log(args, *a):
    if args.verbose:
        print(*a, file=sys.stderr, flush=True)


def cpu_baseline(w, feats, weight, bias, layer):
    """Oracle (numpy port of the reference CPU path) on the whole workload, once."""
    from oracle import conv as OC
    from oracle import pairs as OP
    try:
        from threadpoolctl import threadpool_limits, threadpool_info
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    cores = min(len(os.sched_getaffinity(0)), 16)
    ctx = threadpool_limits(cores) if threadpool_limits else None
    try:
        t0 = time.perf_counter()
        pr = OP.subm_pairs(w.indices, w.spatial_shape, w.batch_size, layer["kernel_size"],
                           layer["dilation"])
        t1 = time.perf_counter()
        Wk = OC.normalize_weight(weight, layer["kernel_size"], layer["c_in"], layer["c_out"])
        OC.conv_forward(feats, Wk, bias, pr.pairs_in, pr.pairs_out, len(w.indices), np.float32)
        t2 = time.perf_counter()
    finally:
        if ctx is not None:
            ctx.unpack() if hasattr(ctx, "unpack") else None
    n = len(w.indices)
    return {
        "value": n / (t2 - t1), "unit": "voxels/s", "cores": cores, "kind": "port",
        "sample": (f"whole workload once ({n} voxels, fp32 accumulate; numpy restatement of "
                   "indices.py dense-table pair build + functional.py slot loop)"),
        "pair_build_ms": (t1 - t0) * 1e3, "conv_ms": (t2 - t1) * 1e3,
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the sparse-conv path here runs on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    import torch

    import trispconv.pytorch as spconv
    from trispconv.pytorch.indices import generate_subm_indice_pairs, generate_strided_indice_pairs
    from trispconv_amd import workloads

    dev = torch.device("cuda:0")
    if args.copy_probe_mib:
        # an elementwise kernel with a recognisable name (neg) that reads and
        # writes exactly copy_probe_mib MiB: the scale for FETCH_SIZE / WRITE_SIZE
        src = torch.ones(args.copy_probe_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    w = workloads.make_workload(args.workload)
    # The ~170k objects that the imports leave behind would make every full
    # garbage collection a ~40 ms pause inside the timed loops; freeze them
    # (the collector then only walks objects made from here on).
    import gc
    gc.collect()
    gc.freeze()
    if args.encoder:
        encoder_bench(args, w, dev)
        return
    layer = w.layers[0]
    dt = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[w.dtype]
    rng = np.random.default_rng(w.seed)
    feats_np = workloads.features(rng, len(w.indices), layer["c_in"])
    w_np, b_np = workloads.layer_params(rng, layer)
    n_in = len(w.indices)

    idx = torch.from_numpy(w.indices).to(dev)
    feats = torch.from_numpy(feats_np).to(dev).to(dt)
    key = "bench"
    if layer["kind"] == "subm":
        mod = spconv.SubMConv3d(layer["c_in"], layer["c_out"], layer["kernel_size"],
                                dilation=layer["dilation"], indice_key=key)
    else:
        mod = spconv.SparseConv3d(layer["c_in"], layer["c_out"], layer["kernel_size"],
                                  stride=layer["stride"], padding=layer["padding"],
                                  dilation=layer["dilation"], indice_key=key)
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(w_np))
        mod.bias.copy_(torch.from_numpy(b_np))
    mod = mod.to(dev).to(dt)
    stream = torch.cuda.current_stream(dev)

    def build_pairs():
        if layer["kind"] == "subm":
            return generate_subm_indice_pairs(idx, w.spatial_shape, w.batch_size,
                                              layer["kernel_size"], layer["dilation"])
        return generate_strided_indice_pairs(idx, w.spatial_shape, w.batch_size,
                                             layer["kernel_size"], layer["stride"],
                                             layer["padding"], layer["dilation"])

    def event_ms(fn, reps):
        """Median over reps of the stream time between events around fn()."""
        times = []
        for _ in range(reps):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            b.synchronize()
            times.append(a.elapsed_time(b))
        return float(np.median(times))

    # ---- pair build (includes its one count read-back) and plan.  The build
    # makes what the convolution consumes (the neighbour map and pair_num);
    # the reference-format padded pair tables are made on first access and
    # timed separately.
    for _ in range(2):
        build_pairs()
    pair_ms = event_ms(build_pairs, 10)

    def build_with_tables():
        build_pairs()._ensure_tables()
    tables_ms = event_ms(build_with_tables, 10)
    data = build_pairs()
    n_out = len(data.out_indices)

    def plan():
        data._order = None
        data.execution_order(n_out, dev, layer["c_in"] * (4 if w.dtype == "float32" else 2))
    plan()
    plan_ms = event_ms(plan, 10)
    P = int(data.pair_num.sum())
    log(args, f"pairs P={P} n_out={n_out} pair_ms={pair_ms:.3f} plan_ms={plan_ms:.3f}")

    # ---- the timed step: the layer with cached pairs
    x = spconv.SparseConvTensor(feats, idx, list(w.spatial_shape), w.batch_size)
    x.indice_dict[key] = data
    # Each step launches exactly one kernel (the fused conv) on ``stream``, so
    # the HIP events around the timed loop give that kernel's average launch
    # duration; back-to-back launches keep the GPU busy between them.
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.no_grad():
        for _ in range(args.warmup):
            y = mod(x)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(args.steps):
            y = mod(x)
        ev1.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    step_ms = (t1 - t0) * 1e3 / args.steps
    kern_ms = ev0.elapsed_time(ev1) / args.steps
    flops = 2.0 * P * layer["c_in"] * layer["c_out"]
    tflops = flops / (kern_ms * 1e-3) / 1e12
    peak, unit = PEAK[w.dtype]
    elem = 4 if w.dtype == "float32" else 2
    # algorithmic bytes of one launch: input rows read once, output written
    # once, the neighbour map and the order read once, the packed weight once
    k_vol = int(np.prod(layer["kernel_size"]))
    pb_bytes = 16 * n_in + 8 * n_in + 8 * k_vol * n_in + 8 * P
    alg_bytes = (n_in * layer["c_in"] * elem + n_out * layer["c_out"] * elem
                 + n_out * k_vol * 4 + n_out * 4 + k_vol * layer["c_in"] * layer["c_out"] * elem)

    result = {
        "metric": "voxels/sec + effective TFLOP/s per SubMConv3d layer; indice-pair build ms",
        "value": n_in / (step_ms * 1e-3),
        "unit": "voxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_TAG[w.dtype],
        "data": "synthetic (seeded surface voxels, N(0,1) features, kaiming-uniform KRSC weights)",
        "config": {"workload": w.name, "layer": f"{layer['kind']} {layer['kernel_size']} "
                   f"{layer['c_in']}->{layer['c_out']}", "voxels": n_in,
                   "spatial_shape": list(w.spatial_shape), "batch": w.batch_size, "pairs": P},
        "tflops_effective": flops / (step_ms * 1e-3) / 1e12,
        "pair_build_ms": pair_ms,
        "pair_build_with_tables_ms": tables_ms,
        # 16N coords + 8N insert + 8KN probes + 8P pair tables (the build's
        # algorithmic bytes, as a hash build of this layer would move them)
        "pair_build_hbm": {"algorithmic_bytes": pb_bytes, "gbs": pb_bytes / (pair_ms * 1e6),
                           "frac": pb_bytes / (pair_ms * 1e6) / HBM_PEAK_GBS},
        "plan_ms": plan_ms,
        "conv_kernel_ms": kern_ms,
        "roofline": roofline(layer, k_vol, tflops, peak, unit, alg_bytes, kern_ms),
    }
    traffic = measured_traffic(w.name, kern_ms)
    if traffic is not None:
        result["roofline"]["traffic"] = traffic["bytes"]
        result["roofline"]["traffic_source"] = traffic["source"]
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, rounded(feats_np, dt), rounded(w_np, dt),
                                              rounded(b_np, dt), layer)
    print(json.dumps(result), flush=True)


def build_network(w, dt, dev, rng):
    """The workload's layers as one SparseSequential.  Each layer but the last
    is followed by an eval-mode BatchNorm1d (random affine and running
    statistics) and a ReLU when the workload is the VoxelNet-style encoder."""
    import torch
    import torch.nn as nn

    import trispconv.pytorch as spconv
    from trispconv_amd import workloads

    mods = []
    bn_relu = w.name.startswith("voxelnet")
    for i, lay in enumerate(w.layers):
        if lay["kind"] == "subm":
            m = spconv.SubMConv3d(lay["c_in"], lay["c_out"], lay["kernel_size"],
                                  dilation=lay["dilation"], indice_key=lay["indice_key"])
        elif lay["kind"] == "strided":
            m = spconv.SparseConv3d(lay["c_in"], lay["c_out"], lay["kernel_size"],
                                    stride=lay["stride"], padding=lay["padding"],
                                    dilation=lay["dilation"], indice_key=lay["indice_key"])
        else:
            m = spconv.SparseInverseConv3d(lay["c_in"], lay["c_out"], lay["kernel_size"],
                                           indice_key=lay["indice_key"])
        wk, bk = workloads.layer_params(rng, lay)
        with torch.no_grad():
            m.weight.copy_(torch.from_numpy(wk))
            m.bias.copy_(torch.from_numpy(bk))
        mods.append(m)
        if bn_relu and i + 1 < len(w.layers):
            bn = nn.BatchNorm1d(lay["c_out"])
            with torch.no_grad():
                bn.weight.copy_(torch.from_numpy(rng.uniform(0.5, 1.5, lay["c_out"])))
                bn.bias.copy_(torch.from_numpy(rng.uniform(-0.2, 0.2, lay["c_out"])))
                bn.running_mean.copy_(torch.from_numpy(rng.uniform(-0.1, 0.1, lay["c_out"])))
                bn.running_var.copy_(torch.from_numpy(rng.uniform(0.5, 1.5, lay["c_out"])))
            mods += [bn, nn.ReLU()]
    return spconv.SparseSequential(*mods).to(dev).to(dt).eval()


def encoder_bench(args, w, dev):
    """The whole network of a multi-layer workload, three ways: pairs cached
    with the BatchNorm/ReLU epilogues fused (value), pairs cached unfused, and
    cold (a fresh tensor, so every layer builds its pairs and plan)."""
    import torch

    import trispconv.pytorch as spconv
    from trispconv_amd import workloads

    dt = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[w.dtype]
    rng = np.random.default_rng(w.seed)
    feats = torch.from_numpy(workloads.features(rng, len(w.indices), w.layers[0]["c_in"]))
    feats = feats.to(dev).to(dt)
    idx = torch.from_numpy(w.indices).to(dev)
    net = build_network(w, dt, dev, rng)
    n_in = len(w.indices)
    stream = torch.cuda.current_stream(dev)

    def fresh():
        return spconv.SparseConvTensor(feats, idx, list(w.spatial_shape), w.batch_size)

    warm = fresh()

    def timed(fn, steps, warmup):
        with torch.no_grad():
            for _ in range(warmup):
                y = fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                y = fn()
            torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps, y

    net.fuse_epilogues = True
    fused_ms, y = timed(lambda: net(warm), args.steps, args.warmup)
    net.fuse_epilogues = False
    unfused_ms, y_plain = timed(lambda: net(warm), args.steps, max(args.warmup // 4, 3))
    net.fuse_epilogues = True
    cold_steps = max(args.steps // 10, 5)
    cold_ms, _ = timed(lambda: net(fresh()), cold_steps, 3)
    # the fused forward captured once in a HIP graph and replayed: the GPU's
    # own time per pass, without the host's launch time
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        y_graph = net(warm)
    graph_ms, _ = timed(graph.replay, args.steps, args.warmup)
    graph_equal = bool(torch.equal(y_graph.features, y.features))
    rel = float((y.features.float() - y_plain.features.float()).abs().max()
                / y_plain.features.float().abs().max().clamp_min(1e-30))

    # per-layer conv time (pairs cached, fused epilogue), events on the stream
    per_layer = []
    flops_total = 0.0
    with torch.no_grad():
        x = warm
        mods = list(net.children())
        i = 0
        while i < len(mods):
            m = mods[i]
            i += 1
            if not isinstance(m, spconv.SparseConvolution):
                continue
            from trispconv_amd.pytorch.modules import _fusable
            ep, used = _fusable(mods, i, m, x)
            out = m.forward_with_epilogue(x, ep)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(20):  # back to back: the layer's GPU time, launches overlapped
                out = m.forward_with_epilogue(x, ep)
            b.record(stream)
            b.synchronize()
            if m.inverse:
                P = int(x.indice_dict[m.indice_key].pair_num.sum())
            else:
                P = int(out.indice_dict[m.indice_key].pair_num.sum()) if m.indice_key else 0
            f = 2.0 * P * m.in_channels * m.out_channels
            flops_total += f
            ms = a.elapsed_time(b) / 20
            per_layer.append({"layer": f"{'inverse' if m.inverse else 'subm' if m.subm else 'strided'}"
                              f" {tuple(m.kernel_size)} {m.in_channels}->{m.out_channels}",
                              "rows_out": int(out.features.shape[0]), "pairs": P, "ms": ms,
                              "tflops": f / (ms * 1e-3) / 1e12,
                              "epilogue": None if ep is None else
                              ("bn+relu" if ep.mean is not None and ep.relu else
                               "bn" if ep.mean is not None else "relu")})
            x = out
            i += used
    # the BEV handoff: the last tensor to a dense (B, C, D, H, W) volume, here
    # and with the reference's three torch passes (tensor.py:72-99)
    def dense_ref():
        D, H, W = x.spatial_shape
        grid = torch.zeros((x.batch_size, D, H, W, x.features.shape[1]), dtype=x.features.dtype,
                           device=dev)
        i = x.indices.long()
        grid[i[:, 0], i[:, 1], i[:, 2], i[:, 3]] = x.features
        return grid.permute(0, 4, 1, 2, 3).contiguous()

    def ms_of(fn, reps=20):
        fn()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        b.synchronize()
        return a.elapsed_time(b) / reps

    dense_ms = ms_of(lambda: x.dense())
    dense_torch_ms = ms_of(dense_ref)
    dense_ok = bool(torch.equal(x.dense(), dense_ref()))
    result = {
        "metric": "voxels/sec + effective TFLOP/s per SubMConv3d layer; indice-pair build ms",
        "value": n_in / (fused_ms * 1e-3),
        "unit": "voxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": fused_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_TAG[w.dtype],
        "data": "synthetic (seeded voxels, N(0,1) features, kaiming-uniform KRSC weights, "
                "random BatchNorm affine and running statistics)",
        "config": {"workload": f"{w.name} (whole network, {len(w.layers)} conv layers)",
                   "voxels": n_in, "spatial_shape": list(w.spatial_shape), "batch": w.batch_size},
        "network_ms_fused": fused_ms,
        "network_ms_unfused": unfused_ms,
        "network_ms_cold": cold_ms,
        "network_ms_graph": graph_ms,
        "graph_equal": graph_equal,
        "fused_vs_unfused_rel_err": rel,
        "tflops_effective": flops_total / (fused_ms * 1e-3) / 1e12,
        "layers": per_layer,
        "dense": {"shape": [x.batch_size, int(x.features.shape[1])] + list(x.spatial_shape),
                  "ms": dense_ms, "torch_three_pass_ms": dense_torch_ms, "equal": dense_ok},
    }
    print(json.dumps(result), flush=True)


def roofline(layer, k_vol, tflops, peak, unit, alg_bytes, kern_ms):
    """The conv kernel against its bound: MFMA peak on the 32x32-tile path
    (C_in a multiple of 16, C_out of 32, K <= 64), else HBM bandwidth (the
    narrow-MFMA and VALU paths serve narrow layers whose arithmetic is
    small)."""
    if layer["c_in"] % 16 == 0 and layer["c_out"] % 32 == 0 and k_vol <= 64:
        return {"bound": "mfma", "achieved": tflops, "peak": peak, "unit": unit,
                "frac": tflops / peak, "traffic": None, "algorithmic_bytes": alg_bytes,
                "kernel": "conv_mfma_kernel"}
    gbs = alg_bytes / (kern_ms * 1e6)
    return {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gbs / HBM_PEAK_GBS, "traffic": None, "algorithmic_bytes": alg_bytes,
            "kernel": "conv_narrow_kernel" if layer["c_in"] % 4 == 0
            and layer["c_out"] % 16 == 0 else "conv_valu_kernel"}


def measured_traffic(workload: str, kern_ms: float):
    """HBM bytes per launch of the conv kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of this workload, or None.

    Counters cannot be read inside a timed run, so the figure comes from the
    profile summary; it is used only while the kernel's average duration in
    that profile is within 15% of the live measurement (a stale profile of an
    older kernel is not reported).
    """
    path = ROOT / "profiles" / f"conv_mfma_{workload}_traffic.txt"
    if not path.exists():
        return None
    vals = {}
    for line in path.read_text().splitlines():
        if ":" in line and not line.startswith("#"):
            k, _, v = line.partition(":")
            vals[k.strip()] = v.strip()
    try:
        prof_us = float(vals["kernel_avg_us"])
        nbytes = float(vals["traffic_bytes_per_launch"])
    except (KeyError, ValueError):
        return None
    if abs(prof_us - kern_ms * 1e3) > 0.15 * prof_us:
        return None
    return {"bytes": nbytes, "source": f"profiles/{path.name}"}


def rounded(a, dt):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dt).float().numpy()


if __name__ == "__main__":
    main()
