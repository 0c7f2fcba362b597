"""Seeded synthetic sparse-voxel workloads.

Five workloads cover the path: a uniform SubM layer, a LiDAR-like strided
layer, the 500k-voxel surface SubM layer, a strided/inverse pair on Gaussian
blobs and a VoxelNet-style encoder.  Coordinates are unique and randomly
permuted (as the reference's own generators leave them,
trispconv/testing/sparse_data.py:40, tests/generate_spconv_goldens.py:49),
features are N(0,1), weights are KRSC kaiming-uniform over the
(C_out, K*C_in) view (trispconv/pytorch/modules.py:75) and biases U(-0.1, 0.1).

Everything here is numpy on the host; callers move tensors to the device.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

__all__ = [
    "Workload",
    "uniform_voxels",
    "surface_voxels",
    "blob_voxels",
    "make_workload",
    "WORKLOAD_NAMES",
    "kaiming_krsc",
]


@dataclass
class Workload:
    name: str
    indices: np.ndarray            # (N, 4) int32, (b, z, y, x)
    spatial_shape: Tuple[int, int, int]
    batch_size: int
    dtype: str                     # "float32" | "float16" | "bfloat16"
    layers: List[Dict] = field(default_factory=list)
    seed: int = 0


def _orthonormal(rng: np.random.Generator, n: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    n = n / np.linalg.norm(n)
    a = np.array([1.0, 0.0, 0.0]) if abs(n[0]) < 0.9 else np.array([0.0, 1.0, 0.0])
    u = np.cross(n, a)
    u /= np.linalg.norm(u)
    v = np.cross(n, u)
    return u, v


def _unique_in_order(keys: np.ndarray) -> np.ndarray:
    _, first = np.unique(keys, return_index=True)
    return keys[np.sort(first)]


def _pack(b: int, zyx: np.ndarray, shape) -> np.ndarray:
    D, H, W = shape
    z, y, x = zyx[:, 0], zyx[:, 1], zyx[:, 2]
    return ((b * D + z) * H + y) * W + x


def _unpack(keys: np.ndarray, shape) -> np.ndarray:
    D, H, W = shape
    x = keys % W
    r = keys // W
    y = r % H
    r = r // H
    z = r % D
    b = r // D
    return np.stack([b, z, y, x], axis=1).astype(np.int32)


def uniform_voxels(shape, n_per_sample: List[int], seed: int) -> np.ndarray:
    """Unique voxels drawn uniformly from the grid, per sample, then permuted."""
    rng = np.random.default_rng(seed)
    D, H, W = shape
    total = D * H * W
    parts = []
    for b, n in enumerate(n_per_sample):
        cells = rng.choice(total, size=n, replace=False)
        parts.append(b * total + cells)
    keys = np.concatenate(parts)
    keys = keys[rng.permutation(len(keys))]
    return _unpack(keys.astype(np.int64), shape)


def _surface_points(rng, shape, kind: str) -> np.ndarray:
    """Points on one random plane patch or cylinder, sampled at 0.45-voxel spacing."""
    D, H, W = shape
    ext = np.array([D, H, W], dtype=np.float64)
    c = rng.uniform(0, 1, 3) * ext
    step = 0.45
    if kind == "plane":
        n = rng.normal(size=3)
        if D < 0.2 * min(H, W):
            # thin-in-z (LiDAR-like) grids: mostly near-horizontal ground and walls
            n = np.array([rng.normal() * 4.0, rng.normal(), rng.normal()])
        u, v = _orthonormal(rng, n)
        L = rng.uniform(0.15, 0.5) * min(H, W)
        a = np.arange(-L / 2, L / 2, step)
        A, Bm = np.meshgrid(a, a, indexing="ij")
        pts = c + A.reshape(-1, 1) * u + Bm.reshape(-1, 1) * v
    else:
        d = rng.normal(size=3)
        if D < 0.2 * min(H, W):
            d = np.array([1.0, rng.normal() * 0.1, rng.normal() * 0.1])  # upright poles / trees
        d /= np.linalg.norm(d)
        e1, e2 = _orthonormal(rng, d)
        r = rng.uniform(3.0, 0.08 * min(H, W) + 3.0)
        L = rng.uniform(0.3, 1.0) * (D if D < 0.2 * min(H, W) else 0.5 * min(H, W))
        th = np.arange(0, 2 * math.pi, step / r)
        h = np.arange(-L / 2, L / 2, step)
        T, Hh = np.meshgrid(th, h, indexing="ij")
        T = T.reshape(-1, 1)
        Hh = Hh.reshape(-1, 1)
        pts = c + Hh * d + r * (np.cos(T) * e1 + np.sin(T) * e2)
    p = np.floor(pts).astype(np.int64)
    ok = (p >= 0).all(1) & (p[:, 0] < D) & (p[:, 1] < H) & (p[:, 2] < W)
    return p[ok]


def surface_voxels(shape, n_per_sample: List[int], seed: int) -> np.ndarray:
    """Thin-shell occupancy: voxelised random plane patches and cylinders.

    Shapes are added until each sample holds at least n voxels; the first n
    unique voxels in generation order are kept, then all rows are permuted.
    """
    rng = np.random.default_rng(seed)
    parts = []
    for b, n in enumerate(n_per_sample):
        acc = np.empty(0, dtype=np.int64)
        while len(acc) < n:
            kind = "plane" if rng.uniform() < 0.5 else "cylinder"
            pts = _surface_points(rng, shape, kind)
            if len(pts) == 0:
                continue
            acc = _unique_in_order(np.concatenate([acc, _pack(b, pts, shape)]))
        parts.append(acc[:n])
    keys = np.concatenate(parts)
    keys = keys[rng.permutation(len(keys))]
    return _unpack(keys, shape)


def blob_voxels(shape, n_per_sample: List[int], seed: int, sigma: float = 8.0) -> np.ndarray:
    """Clustered occupancy: rounded samples of isotropic Gaussian blobs."""
    rng = np.random.default_rng(seed)
    D, H, W = shape
    ext = np.array([D, H, W], dtype=np.float64)
    parts = []
    for b, n in enumerate(n_per_sample):
        acc = np.empty(0, dtype=np.int64)
        while len(acc) < n:
            c = rng.uniform(0, 1, 3) * ext
            pts = np.rint(c + rng.normal(size=(4096, 3)) * sigma).astype(np.int64)
            ok = (pts >= 0).all(1) & (pts[:, 0] < D) & (pts[:, 1] < H) & (pts[:, 2] < W)
            acc = _unique_in_order(np.concatenate([acc, _pack(b, pts[ok], shape)]))
        parts.append(acc[:n])
    keys = np.concatenate(parts)
    keys = keys[rng.permutation(len(keys))]
    return _unpack(keys, shape)


def kaiming_krsc(rng: np.random.Generator, c_out: int, ksize, c_in: int) -> np.ndarray:
    """KRSC weight, kaiming-uniform over the (C_out, K*C_in) view.

    torch's kaiming_uniform_ defaults (a=0, fan_in, leaky_relu) give the bound
    sqrt(2) * sqrt(3 / fan_in) with fan_in = K*C_in (modules.py:75).
    """
    kd, kh, kw = ksize
    fan_in = kd * kh * kw * c_in
    bound = math.sqrt(2.0) * math.sqrt(3.0 / fan_in)
    return rng.uniform(-bound, bound, size=(c_out, kd, kh, kw, c_in)).astype(np.float32)


def _layer(kind, c_in, c_out, k, s=1, p=0, d=1, key=None):
    to3 = lambda v: (v, v, v) if isinstance(v, int) else tuple(v)  # noqa: E731
    return {"kind": kind, "c_in": c_in, "c_out": c_out, "kernel_size": to3(k),
            "stride": to3(s), "padding": to3(p), "dilation": to3(d), "indice_key": key}


WORKLOAD_NAMES = ["subm16_uniform20k", "strided64_lidar2x200k", "subm128_surface500k",
                  "inverse_blob4x150k", "voxelnet_encoder4x60k"]


def make_workload(name: str, scale: float = 1.0) -> Workload:
    """Build one of the five named workloads; ``scale`` shrinks voxel counts for tests."""
    def n(v):
        return max(16, int(round(v * scale)))

    if name == "subm16_uniform20k":
        shape = (128, 128, 128)
        idx = uniform_voxels(shape, [n(20_000)], seed=1)
        return Workload(name, idx, shape, 1, "float32",
                        [_layer("subm", 16, 16, 3)], seed=1)
    if name == "strided64_lidar2x200k":
        shape = (41, 1600, 1408)
        idx = surface_voxels(shape, [n(200_000)] * 2, seed=2)
        return Workload(name, idx, shape, 2, "float32",
                        [_layer("strided", 64, 64, 3, 2, 1)], seed=2)
    if name == "subm128_surface500k":
        shape = (256, 256, 256)
        idx = surface_voxels(shape, [n(500_000)], seed=3)
        return Workload(name, idx, shape, 1, "float16",
                        [_layer("subm", 128, 128, 3)], seed=3)
    if name == "inverse_blob4x150k":
        shape = (512, 512, 64)
        idx = blob_voxels(shape, [n(150_000)] * 4, seed=4)
        return Workload(name, idx, shape, 4, "bfloat16",
                        [_layer("strided", 32, 64, 3, 2, 1, key="k"),
                         _layer("inverse", 64, 32, 3, key="k")], seed=4)
    if name == "voxelnet_encoder4x60k":
        shape = (41, 1600, 1408)
        idx = surface_voxels(shape, [n(60_000)] * 4, seed=5)
        layers = [_layer("subm", 4, 16, 3, key="subm1")]
        c_prev = 16
        for i, c in enumerate([32, 64, 64]):
            layers.append(_layer("strided", c_prev, c, 3, 2, 1, key=f"spconv{i + 2}"))
            layers.append(_layer("subm", c, c, 3, key=f"subm{i + 2}"))
            layers.append(_layer("subm", c, c, 3, key=f"subm{i + 2}"))
            c_prev = c
        layers.append(_layer("strided", 64, 128, (3, 1, 1), (2, 1, 1), 0, key="spconv_down2"))
        return Workload(name, idx, shape, 4, "float16", layers, seed=5)
    raise KeyError(f"unknown workload {name!r}; choose from {WORKLOAD_NAMES}")


def layer_params(rng: np.random.Generator, layer: Dict) -> Tuple[np.ndarray, np.ndarray]:
    """KRSC weight and U(-0.1, 0.1) bias for one layer description."""
    w = kaiming_krsc(rng, layer["c_out"], layer["kernel_size"], layer["c_in"])
    b = rng.uniform(-0.1, 0.1, size=(layer["c_out"],)).astype(np.float32)
    return w, b


def features(rng: np.random.Generator, n: int, c: int) -> np.ndarray:
    return rng.standard_normal(size=(n, c), dtype=np.float32)
