"""Benchmark: the five sparse-convolution workloads on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload all|NAME]
                    [--no-cpu-baseline]

One step is one forward of a workload's network over the whole batch with
its indice pairs cached under their ``indice_key`` (as a network reuses
them), inputs already resident in HBM:

  subm16_uniform20k      SubM 3^3 16->16 fp32, 20k uniform voxels in 128^3
  strided64_lidar2x200k  SparseConv3d k3 s2 p1 64->64 fp32, 2 x 200k LiDAR-like
  subm128_surface500k    SubM 3^3 128->128 fp16, 500k surface voxels in 256^3
                         (the headline layer: top-level value and roofline)
  inverse_blob4x150k     SparseConv3d 32->64 s2 + SparseInverseConv3d 64->32,
                         bf16, 4 x 150k blob voxels
  voxelnet_encoder4x60k  SparseSequential encoder, 11 conv layers with eval
                         BatchNorm1d + ReLU (fused into the conv stores), fp16

Prints one short JSON line per workload, the headline layer's last (its
``value`` = voxels/s = N_in / step time); the full results, per layer, go to
``--detail`` (default: trispconv_bench_detail.json in the temp directory).
Each workload gets:
voxels/s, effective TFLOP/s, per-layer conv times (HIP events on the stream
the kernels run on, between the layers of the network run in order; each
includes the few microseconds its event adds, so a network's layer times sum
to more than its step), pair-build times with their fraction of HBM
bandwidth, the dominant conv kernel against its roofline (fp16/bf16/fp32 MFMA
peak or HBM, whichever its arithmetic intensity makes the bound), and the
reference's CPU path timed on this host (``cpu_baseline``).
"""
from __future__ import annotations

import argparse
import copy
import gc
import json
import os
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_TFLOPS = {"float16": 2500.0, "bfloat16": 2500.0, "float32": 157.3}  # MI355X dense MFMA
HBM_PEAK_GBS = 8000.0
DTYPE_TAG = {"float32": "f32", "float16": "f16", "bfloat16": "bf16"}
HEADLINE = "subm128_surface500k"
SETTLE_MS = 80.0  # untimed back-to-back steps before the warm-up steps
METRIC = "voxels/sec + effective TFLOP/s per SubMConv3d layer; indice-pair build ms"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the GPU needs some tens of milliseconds of load to reach its steady clock:
    # 100 warm-up steps of the headline layer take ~40 ms
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="all",
                    help="'all' (default: every workload, headline on top) or one workload name")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run one elementwise negation over this many MiB (a copy-like "
                         "kernel of known size to scale FETCH_SIZE / WRITE_SIZE counters by)")
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--detail",
                    default=str(Path(tempfile.gettempdir()) / "trispconv_bench_detail.json"),
                    help="file for every workload's full results (per layer); stdout gets one "
                         "short line per workload, the headline last")
    return ap.parse_args()


def log(args, *a):
    if args.verbose:
        print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ network
def layer_modules(w, rng):
    """The workload's layers as (conv module, batch-norm module or None) with
    seeded weights; every layer gets an indice_key so that a step reuses its
    pairs.  The VoxelNet-style encoder has an eval-mode BatchNorm1d (random
    affine and running statistics) and a ReLU after every layer but the last."""
    import torch
    import torch.nn as nn

    import trispconv.pytorch as spconv
    from trispconv_amd import workloads

    out = []
    bn_relu = w.name.startswith("voxelnet")
    for i, lay in enumerate(w.layers):
        key = lay["indice_key"] or f"layer{i}"
        if lay["kind"] == "subm":
            m = spconv.SubMConv3d(lay["c_in"], lay["c_out"], lay["kernel_size"],
                                  dilation=lay["dilation"], indice_key=key)
        elif lay["kind"] == "strided":
            m = spconv.SparseConv3d(lay["c_in"], lay["c_out"], lay["kernel_size"],
                                    stride=lay["stride"], padding=lay["padding"],
                                    dilation=lay["dilation"], indice_key=key)
        else:
            m = spconv.SparseInverseConv3d(lay["c_in"], lay["c_out"], lay["kernel_size"],
                                           indice_key=key)
        wk, bk = workloads.layer_params(rng, lay)
        with torch.no_grad():
            m.weight.copy_(torch.from_numpy(wk))
            m.bias.copy_(torch.from_numpy(bk))
        bn = None
        if bn_relu and i + 1 < len(w.layers):
            bn = nn.BatchNorm1d(lay["c_out"])
            with torch.no_grad():
                bn.weight.copy_(torch.from_numpy(rng.uniform(0.5, 1.5, lay["c_out"])))
                bn.bias.copy_(torch.from_numpy(rng.uniform(-0.2, 0.2, lay["c_out"])))
                bn.running_mean.copy_(torch.from_numpy(rng.uniform(-0.1, 0.1, lay["c_out"])))
                bn.running_var.copy_(torch.from_numpy(rng.uniform(0.5, 1.5, lay["c_out"])))
        out.append((m, bn))
    return out


def sequential(mods, dt, dev):
    import torch.nn as nn

    import trispconv.pytorch as spconv
    seq = []
    for m, bn in mods:
        seq.append(m)
        if bn is not None:
            seq += [bn, nn.ReLU()]
    return spconv.SparseSequential(*seq).to(dev).to(dt).eval()


# ------------------------------------------------------------------ rooflines
def conv_alg_bytes(n_in, n_out, c_in, c_out, k_vol, elem, planned):
    """Algorithmic bytes of one conv launch: input rows read once, output
    rows written once, the neighbour map and (when planned) the order read
    once, the packed weight once."""
    return (n_in * c_in * elem + n_out * c_out * elem + n_out * k_vol * 4
            + (n_out * 4 if planned else 0) + k_vol * c_in * c_out * elem)


def roofline(flops, alg_bytes, kern_ms, dtype, kernel, workload, layer, rows_out):
    """The conv kernel of one layer against its bound: MFMA peak when its
    arithmetic intensity (flops per algorithmic byte) reaches the ridge point
    of the dtype's peak over 8 TB/s, else HBM bandwidth; both fractions are
    given."""
    peak = PEAK_TFLOPS[dtype]
    ridge = peak * 1e12 / (HBM_PEAK_GBS * 1e9)
    tflops = flops / (kern_ms * 1e-3) / 1e12
    gbs = alg_bytes / (kern_ms * 1e6)
    mfma = flops / max(alg_bytes, 1) >= ridge
    r = {"bound": "mfma" if mfma else "hbm",
         "achieved": tflops if mfma else gbs,
         "peak": peak if mfma else HBM_PEAK_GBS,
         "unit": "TFLOP/s" if mfma else "GB/s",
         "frac": (tflops / peak) if mfma else (gbs / HBM_PEAK_GBS),
         "traffic": None,
         "algorithmic_bytes": int(alg_bytes), "flops": flops,
         "mfma_frac": tflops / peak, "hbm_frac": gbs / HBM_PEAK_GBS,
         "kernel": kernel, "kernel_ms": kern_ms, "layer": layer, "rows_out": rows_out}
    t = measured_traffic(kernel, workload, kern_ms, f"{layer}, {rows_out} output rows")
    if t is not None:
        r["traffic"] = t["bytes"]
        r["traffic_source"] = t["source"]
    return r


def measured_traffic(kernel: str, workload: str, kern_ms: float, layer_tag: str):
    """HBM bytes per launch of a conv kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of this workload, or None.

    Counters cannot be read inside a timed run, so the figure comes from the
    profile summary.  It is used only for the layer the summary names (layer
    and output rows, in its first line) and only while the kernel's duration
    in that profile is within 15% (or 5 us, for kernels of a few
    microseconds whose timing here includes launch gaps) of the live
    measurement, so a stale profile of an older kernel is not reported.
    """
    path = ROOT / "profiles" / f"{kernel.replace('_kernel', '')}_{workload}_traffic.txt"
    if not path.exists():
        return None
    text = path.read_text().splitlines()
    if not text or not text[0].endswith(f"layer {layer_tag}"):
        return None
    vals = {}
    for line in text:
        if ":" in line and not line.startswith("#"):
            k, _, v = line.partition(":")
            vals[k.strip()] = v.strip()
    try:
        prof_us = float(vals["kernel_avg_us"].split()[0])
        nbytes = float(vals["traffic_bytes_per_launch"].split()[0])
    except (KeyError, ValueError):
        return None
    if abs(prof_us - kern_ms * 1e3) > max(0.15 * prof_us, 5.0):
        return None
    return {"bytes": nbytes, "source": f"profiles/{path.name}"}


def pair_build_bytes(kind, n_in, n_out, k_vol, pairs):
    """Algorithmic bytes of a pair build.
    SubM: 16N coordinates + 8N table insert + 8KN probes + 8P pair tables.
    Strided: 16N coordinates + 8KN candidate keys + 16 N_out (output set and
    its ranks) + 16 N_out output coordinates + 8P pair tables.
    Inverse: 8P forward tables read + 4P remapped ids + 4 K N_out map +
    32 N_out coordinates gathered."""
    if kind == "subm":
        return 16 * n_in + 8 * n_in + 8 * k_vol * n_in + 8 * pairs
    if kind == "strided":
        return 16 * n_in + 8 * k_vol * n_in + 16 * n_out + 16 * n_out + 8 * pairs
    return 8 * pairs + 4 * pairs + 4 * k_vol * n_out + 32 * n_out


# ------------------------------------------------------------------ GPU side
def bench_gpu(w, args, dev, mods, feats, idx):
    """Pair builds, plans, per-layer conv kernels and the whole cached step."""
    import torch

    import trispconv.pytorch as spconv
    from trispconv.pytorch.indices import (generate_inverse_indice_pairs,
                                           generate_strided_indice_pairs,
                                           generate_subm_indice_pairs)
    from trispconv_amd import _lib as L
    from trispconv_amd.pytorch.modules import _fusable

    stream = torch.cuda.current_stream(dev)
    n_in = len(w.indices)

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

    def back_to_back_ms(fn, reps):
        """Stream time per call of reps back-to-back calls (launches overlap
        the previous kernel, so this is the GPU time of one call)."""
        fn()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        b.synchronize()
        return a.elapsed_time(b) / reps

    net = sequential(mods, feats.dtype, dev)
    convs = [m for m in net.children() if isinstance(m, spconv.SparseConvolution)]

    def fresh():
        return spconv.SparseConvTensor(feats, idx, list(w.spatial_shape), w.batch_size)

    # ---- cold pass: every pair build and plan, then the convolutions
    with torch.no_grad():
        for _ in range(2):
            net(fresh())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        cold_reps = 5
        for _ in range(cold_reps):
            net(fresh())
        torch.cuda.synchronize()
        cold_ms = (time.perf_counter() - t0) * 1e3 / cold_reps
    warm = fresh()

    # ---- per layer: pair build, plan, conv kernel (pairs cached, epilogue fused)
    layers = []
    seq = []  # (module, fused epilogue) of each layer, in order
    mods_list = list(net.children())
    with torch.no_grad():
        x = warm
        net(x)  # caches every key in warm.indice_dict
        i = 0
        while i < len(mods_list):
            m = mods_list[i]
            i += 1
            if not isinstance(m, spconv.SparseConvolution):
                continue
            ep, used = _fusable(mods_list, i, m, x)
            kind = "inverse" if m.inverse else "subm" if m.subm else "strided"
            k_vol = int(np.prod(m.kernel_size))
            elem = x.features.element_size()
            # the pair build of this layer on its own input
            if kind == "subm":
                build = lambda x=x, m=m: generate_subm_indice_pairs(  # noqa: E731
                    x.indices, tuple(x.spatial_shape), x.batch_size, m.kernel_size, m.dilation)
            elif kind == "strided":
                build = lambda x=x, m=m: generate_strided_indice_pairs(  # noqa: E731
                    x.indices, tuple(x.spatial_shape), x.batch_size, m.kernel_size, m.stride,
                    m.padding, m.dilation)
            else:
                fwd = x.indice_dict[m.indice_key]
                build = lambda fwd=fwd: generate_inverse_indice_pairs(fwd)  # noqa: E731
            pair_ms = event_ms(build, 10)
            # the same build with pair_num read on the host (a submanifold
            # build returns once its coordinates are checked and leaves the
            # counts on the device until they are read)
            counts_ms = event_ms(lambda build=build: build().pair_num, 10)
            data = build()
            n_out = len(data.out_indices)
            P = int(data.pair_num.sum())

            def plan(data=data, n_out=n_out, c_in=m.in_channels, elem=elem):
                data._order = None
                return data.execution_order(n_out, dev, c_in * elem, eager=True)
            planned = plan() is not None
            plan_ms = event_ms(plan, 10) if planned else 0.0
            out = m.forward_with_epilogue(x, ep)
            seq.append((m, ep))
            flops = 2.0 * P * m.in_channels * m.out_channels
            kname = L.lib().tsc_conv_kernel_name(L.dtype_code(x.features.dtype), m.in_channels,
                                                 m.out_channels, k_vol, n_out).decode()
            cached = x.indice_dict[m.indice_key] if kind != "inverse" else \
                x.indice_dict[m.indice_key]._inverse_cache
            was_planned = cached is not None and cached._order is not None
            alg = conv_alg_bytes(len(x.indices), n_out, m.in_channels, m.out_channels, k_vol, elem,
                                 was_planned)
            pb = pair_build_bytes(kind, len(x.indices), n_out, k_vol, P)
            layers.append({
                "layer": f"{kind} {tuple(m.kernel_size)} {m.in_channels}->{m.out_channels}",
                "rows_in": len(x.indices), "rows_out": n_out, "pairs": P,
                "conv_ms": None, "tflops": None,  # set below, from the layer sequence
                "pair_build_ms": pair_ms,
                "pair_build_with_counts_ms": counts_ms,
                "pair_build_hbm": {"algorithmic_bytes": int(pb), "gbs": pb / (pair_ms * 1e6),
                                   "frac": pb / (pair_ms * 1e6) / HBM_PEAK_GBS},
                "plan_ms": plan_ms,
                "epilogue": None if ep is None else
                ("bn+relu" if ep.mean is not None and ep.relu else
                 "bn" if ep.mean is not None else "relu"),
                "roofline": {"flops": flops, "algorithmic_bytes": alg, "kernel": kname},
            })
            x = out
            i += used

    # ---- per-layer conv times as the step runs them: the layers in order,
    # each on the previous one's output, with events between them (median
    # over 20 passes).  Timing a layer alone, back to back on one input,
    # gives other cache states than the network and can differ by a third.
    reps = 20
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(seq) + 1)] for _ in range(reps)]
    with torch.no_grad():
        for r in range(reps):
            y = warm
            evs[r][0].record(stream)
            for j, (m, ep) in enumerate(seq):
                y = m.forward_with_epilogue(y, ep)
                evs[r][j + 1].record(stream)
        torch.cuda.synchronize()
    for j, lay in enumerate(layers):
        conv_ms = float(np.median([evs[r][j].elapsed_time(evs[r][j + 1]) for r in range(reps)]))
        rf = lay["roofline"]
        lay["conv_ms"] = conv_ms
        lay["tflops"] = rf["flops"] / (conv_ms * 1e-3) / 1e12
        lay["roofline"] = roofline(rf["flops"], rf["algorithmic_bytes"], conv_ms, w.dtype,
                                   rf["kernel"], w.name, lay["layer"], lay["rows_out"])

    # ---- the timed step: the whole network with cached pairs.  For a
    # one-layer workload the step is one kernel launch, so the events around
    # the loop give that kernel's average duration.  Before the W warm-up
    # steps, untimed steps run back to back for SETTLE_MS: the GPU needs some
    # tens of milliseconds of continuous load to reach its steady clock (the
    # per-layer timing above syncs after every pass), and a handful of
    # warm-up steps of a 0.3 ms layer is not that.
    with torch.no_grad():
        t_settle = time.perf_counter()
        while (time.perf_counter() - t_settle) * 1e3 < SETTLE_MS:
            for _ in range(16):
                y = net(warm)
            torch.cuda.synchronize()
        for _ in range(args.warmup):
            y = net(warm)
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(args.steps):
            y = net(warm)
        ev1.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    step_ms = (t1 - t0) * 1e3 / args.steps
    gpu_step_ms = ev0.elapsed_time(ev1) / args.steps
    if len(layers) == 1:
        # the timed loop's own kernel duration is the layer's
        lay = layers[0]
        lay["conv_ms"] = gpu_step_ms
        lay["tflops"] = 2.0 * lay["pairs"] * convs[0].in_channels * convs[0].out_channels \
            / (gpu_step_ms * 1e-3) / 1e12
        lay["roofline"] = roofline(lay["roofline"]["flops"], lay["roofline"]["algorithmic_bytes"],
                                   gpu_step_ms, w.dtype, lay["roofline"]["kernel"], w.name,
                                   lay["layer"], lay["rows_out"])
    res = {"step_ms": step_ms, "gpu_step_ms": gpu_step_ms, "network_ms_cold": cold_ms,
           "layers": layers, "y": y}
    if len(layers) > 1:
        # the fused forward captured once in a HIP graph and replayed
        graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(graph):
            y_graph = net(warm)
        res["network_ms_graph"] = back_to_back_ms(graph.replay, args.steps)
        res["graph_equal"] = bool(torch.equal(y_graph.features, y.features))
    return res


# ------------------------------------------------------------------ CPU side
def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# CPU time of one timed convolution pass: runs estimated longer are timed on a
# fixed fraction of every slot's pairs and scaled up (the op sequence is the
# same; its cost is linear in the pairs)
CPU_CONV_RUN_S = 3.0


def cpu_baseline(w, feats_np, params, mods_np):
    """The reference's CPU path (oracle.torch_path: its torch op sequence) on
    this host, with every affinity core: the pair builds of the whole
    workload (one warm-up, median of 3), then the convolutions with their
    batch norm and ReLU on those pairs in the workload's dtype and in fp32
    (one warm-up, median of 3 each; a pass estimated over CPU_CONV_RUN_S runs
    on a fixed fraction of every slot's pairs and is scaled up)."""
    import torch
    import torch.nn as nn

    from oracle import torch_path as TP

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    native = {"float32": torch.float32, "float16": torch.float16,
              "bfloat16": torch.bfloat16}[w.dtype]
    layers = [dict(lay, indice_key=lay["indice_key"] or f"layer{i}")
              for i, lay in enumerate(w.layers)]

    def pair_pass():
        """All pair builds of one forward; returns (seconds, per-layer
        (pairs, rows in))."""
        cache, out = {}, []
        idx = torch.from_numpy(w.indices)
        shape = tuple(w.spatial_shape)
        t = 0.0
        for lay in layers:
            t0 = time.perf_counter()
            pr = TP.build_pairs(lay, idx, shape, w.batch_size, cache)
            t += time.perf_counter() - t0
            out.append((pr, len(idx)))
            if lay["kind"] == "inverse" and tuple(pr.kernel_size) == (1, 1, 1):
                continue  # modules.py:162-173 keeps the input's coordinates
            idx, shape = pr.out_indices, pr.output_spatial_shape
        return t, out

    pair_pass()
    runs = [pair_pass() for _ in range(3)]
    pair_s = float(np.median([r[0] for r in runs]))
    per_layer = runs[-1][1]

    def conv_pass(dt, frac):
        """Every layer's convolution (+ batch norm and ReLU) on frac of each
        slot's pairs; returns seconds."""
        g = torch.Generator().manual_seed(0)
        t = 0.0
        for (pr, n_in), (wk, bk), bnd, lay in zip(per_layer, params, bn_of[dt], layers):
            x = torch.randn(n_in, wk.shape[4], generator=g).to(dt)
            W = TP.normalize_weight(torch.from_numpy(wk).to(dt), lay["kernel_size"],
                                    wk.shape[4], wk.shape[0])
            pin = [p[: int(np.ceil(frac * p.numel()))] for p in pr.pairs_in]
            pout = [p[: int(np.ceil(frac * p.numel()))] for p in pr.pairs_out]
            t0 = time.perf_counter()
            y = TP.conv_forward(x, W, torch.from_numpy(bk).to(dt), pin, pout,
                                len(pr.out_indices))
            if bnd is not None:
                y = nn.functional.relu(bnd(y))
            t += time.perf_counter() - t0
        return t

    bn_of = {dt: [None if bn is None else copy.deepcopy(bn).to(dt) for bn in mods_np]
             for dt in {native, torch.float32}}

    def conv_timed(dt):
        probe = 1.0 / 32
        est = conv_pass(dt, probe) / probe  # also the warm-up
        frac = 1.0 if est <= CPU_CONV_RUN_S else CPU_CONV_RUN_S / est
        conv_pass(dt, frac)
        t = float(np.median([conv_pass(dt, frac) for _ in range(3)]))
        return t / frac, frac

    with torch.no_grad():
        conv_s, frac = conv_timed(native)
        n = len(w.indices)
        res = {"cores": cores, "kind": "port", "cpu_model": cpu_model(),
               "dtype": DTYPE_TAG[w.dtype],
               "sample": (f"whole workload ({n} voxels, {len(layers)} layer(s)): the reference's "
                          "torch op sequence on CPU tensors; pair builds (indices.py dense table / "
                          "unique, modules.py inverse remap) in full, median of 3 after a "
                          "warm-up; convolutions (functional.py per-slot gather, matmul, "
                          "index_add_ in the features' dtype"
                          + (", then BatchNorm1d + ReLU" if any(b is not None for b in mods_np)
                             else "")
                          + f") on {frac:.3g} of every slot's pairs, scaled by its inverse, "
                          "median of 3 after a warm-up"),
               "pair_build_ms": pair_s * 1e3, "conv_ms": conv_s * 1e3, "conv_pairs_frac": frac,
               "value": n / conv_s, "unit": "voxels/s",
               "value_with_pairs": n / (pair_s + conv_s)}
        if native != torch.float32:
            conv32, frac32 = conv_timed(torch.float32)
            res["conv_ms_fp32"] = conv32 * 1e3
            res["conv_pairs_frac_fp32"] = frac32
            res["value_fp32"] = n / conv32
    return res


# ------------------------------------------------------------------ one workload
def bench_workload(name, args, dev):
    import torch

    from trispconv_amd import workloads

    w = workloads.make_workload(name)
    dt = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}[w.dtype]
    rng = np.random.default_rng(w.seed)
    n_in = len(w.indices)
    feats_np = workloads.features(rng, n_in, w.layers[0]["c_in"])
    mods = layer_modules(w, rng)
    feats = torch.from_numpy(feats_np).to(dev).to(dt)
    idx = torch.from_numpy(w.indices).to(dev)
    log(args, f"{name}: {n_in} voxels")
    g = bench_gpu(w, args, dev, mods, feats, idx)
    layers = g["layers"]
    flops = sum(lay["roofline"]["flops"] for lay in layers)
    # the dominant kernel: the layer whose conv takes longest (for the
    # strided + inverse pair, the inverse layer the workload is named for)
    if name.startswith("inverse"):
        dom = layers[-1]
    else:
        dom = max(layers, key=lambda lay: lay["conv_ms"])
    res = {
        "workload": name,
        "layers_desc": [lay["layer"] for lay in layers],
        "voxels": n_in, "batch": w.batch_size, "spatial_shape": list(w.spatial_shape),
        "dtype": DTYPE_TAG[w.dtype],
        "pairs": sum(lay["pairs"] for lay in layers),
        "ms_per_step": g["step_ms"],
        "gpu_ms_per_step": g["gpu_step_ms"],
        "voxels_per_s": n_in / (g["step_ms"] * 1e-3),
        "tflops_effective": flops / (g["step_ms"] * 1e-3) / 1e12,
        "pair_build_ms": sum(lay["pair_build_ms"] for lay in layers),
        "pair_build_with_counts_ms": sum(lay["pair_build_with_counts_ms"] for lay in layers),
        "plan_ms": sum(lay["plan_ms"] for lay in layers),
        "network_ms_cold": g["network_ms_cold"],
        "voxels_per_s_cold": n_in / (g["network_ms_cold"] * 1e-3),
        "roofline": dict(dom["roofline"], layer=dom["layer"]),
    }
    if len(layers) == 1:
        res["pair_build_hbm"] = layers[0]["pair_build_hbm"]
    else:
        res["layers"] = layers
    for k in ("network_ms_graph", "graph_equal"):
        if k in g:
            res[k] = g[k]
    del g
    torch.cuda.synchronize()
    if not args.no_cpu_baseline:
        params = [(m.weight.detach().float().cpu().numpy(), m.bias.detach().float().cpu().numpy())
                  for m, _ in mods]
        bns = [None if bn is None else bn.float().cpu().eval() for _, bn in mods]
        cb = cpu_baseline(w, feats_np, params, bns)
        res["cpu_baseline"] = cb
        res["gpu_over_cpu"] = res["voxels_per_s"] / cb["value"]
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the sparse-conv path here runs on a single MI355X and shards by batch "
              "without exchange, so the per-GPU figure is the figure)", file=sys.stderr)
        sys.exit(2)
    import torch

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
    names = workloads.WORKLOAD_NAMES if args.workload == "all" else [args.workload]
    # the headline first, so that its timed loop runs on a fresh process
    names = sorted(names, key=lambda n: n != HEADLINE)
    # The ~170k objects that the imports leave behind would make every full
    # garbage collection a ~40 ms pause inside the timed loops; freeze them
    # (the collector then only walks objects made from here on).
    gc.collect()
    gc.freeze()
    results = {}
    for name in names:
        results[name] = bench_workload(name, args, dev)
        gc.collect()
        torch.cuda.empty_cache()
        log(args, json.dumps(results[name]))
    head = results[names[0]]
    # every field of every workload, per layer, goes to a file; stdout gets
    # one short line per workload, the headline line last
    detail = Path(args.detail)
    detail.parent.mkdir(parents=True, exist_ok=True)
    detail.write_text(json.dumps({"configs": results}, indent=1))
    for name in names[1:]:
        print(json.dumps(config_line(results[name])), flush=True)
    print(json.dumps(headline_line(head, args, detail)), flush=True)


def _sig(x, digits=4):
    """Floats rounded to a few significant digits, recursively (short lines)."""
    if isinstance(x, float):
        return float(f"{x:.{digits}g}")
    if isinstance(x, dict):
        return {k: _sig(v, digits) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return [_sig(v, digits) for v in x]
    return x


_ROOF_KEYS = ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel", "kernel_ms",
              "layer", "rows_out", "mfma_frac", "hbm_frac")


def _short_roofline(r):
    out = {k: r.get(k) for k in _ROOF_KEYS}
    if r.get("traffic"):
        out["traffic_over_algorithmic"] = r["traffic"] / r["algorithmic_bytes"]
    out["algorithmic_bytes"] = r["algorithmic_bytes"]
    return out


def _short_cpu(cb):
    if cb is None:
        return None
    keys = ("value", "unit", "cores", "kind", "dtype", "conv_pairs_frac", "pair_build_ms",
            "conv_ms", "value_fp32", "conv_pairs_frac_fp32", "conv_ms_fp32")
    out = {k: cb[k] for k in keys if k in cb}
    out["sample"] = (f"{cb['dtype']} conv on {cb['conv_pairs_frac']:.3g} of every slot's pairs "
                     "(scaled by its inverse), pair builds in full; reference torch op sequence "
                     "on CPU tensors, median of 3")
    return out


def config_line(res):
    """One workload as a short JSON line (~1 KB)."""
    line = {
        "config_result": res["workload"], "dtype": res["dtype"], "voxels": res["voxels"],
        "batch": res["batch"], "pairs": res["pairs"], "ms_per_step": res["ms_per_step"],
        "voxels_per_s": res["voxels_per_s"], "tflops_effective": res["tflops_effective"],
        "pair_build_ms": res["pair_build_ms"], "plan_ms": res["plan_ms"],
        "network_ms_cold": res["network_ms_cold"],
    }
    if "pair_build_hbm" in res:
        line["pair_build_hbm_frac"] = res["pair_build_hbm"]["frac"]
    if "layers" in res:
        line["layer_conv_ms"] = [lay["conv_ms"] for lay in res["layers"]]
        line["layer_pair_build_ms"] = [lay["pair_build_ms"] for lay in res["layers"]]
        line["layer_pair_build_hbm_frac"] = [lay["pair_build_hbm"]["frac"]
                                             for lay in res["layers"]]
    for k in ("network_ms_graph", "graph_equal"):
        if k in res:
            line[k] = res[k]
    line["roofline"] = _short_roofline(res["roofline"])
    line["cpu_baseline"] = _short_cpu(res.get("cpu_baseline"))
    return _sig(line)


def headline_line(head, args, detail):
    """The headline workload's line, the last one printed (under 2 KB)."""
    lay = head.get("layers_desc", [""])[0]
    line = {
        "metric": METRIC,
        "value": head["voxels_per_s"],
        "unit": "voxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded voxels, N(0,1) features, kaiming-uniform KRSC weights, "
                "U(-0.1,0.1) biases)",
        "config": {"workload": head["workload"], "layer": lay, "voxels": head["voxels"],
                   "spatial_shape": head["spatial_shape"], "batch": head["batch"],
                   "pairs": head["pairs"]},
        "tflops_effective": head["tflops_effective"],
        "conv_kernel_ms": head["roofline"]["kernel_ms"],
        "pair_build_ms": head["pair_build_ms"],
        "pair_build_with_counts_ms": head["pair_build_with_counts_ms"],
        "pair_build_hbm_frac": head.get("pair_build_hbm", {}).get("frac"),
        "plan_ms": head["plan_ms"],
        "network_ms_cold": head["network_ms_cold"],
        "roofline": _short_roofline(head["roofline"]),
        "cpu_baseline": _short_cpu(head.get("cpu_baseline")),
        "detail": str(detail),
    }
    return _sig(line, 5)


if __name__ == "__main__":
    main()
