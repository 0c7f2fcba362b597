"""Oracle: indice-pair generation restated in numpy (test infrastructure only).

Follows the reference's algorithms step by step, including its data
structures (a dense lookup table over the whole grid for submanifold pairs,
``unique(sorted)`` for strided outputs), because the point is to reproduce
the exact pair order and output row order:

* ``subm_pairs``     — trispconv/pytorch/indices.py:67-140
* ``strided_pairs``  — trispconv/pytorch/indices.py:143-259
* ``inverse_pairs``  — trispconv/pytorch/modules.py:175-212

Pair lists are returned as lists of K int64 arrays, ``pair_num`` as an
int64 array of length K, coordinates as (N, 4) int32 arrays in (b, z, y, x).
"""
from __future__ import annotations

from dataclasses import dataclass
from itertools import product
from typing import List, Tuple

import numpy as np


@dataclass
class OraclePairs:
    out_indices: np.ndarray        # (N_out, 4) int32
    pairs_in: List[np.ndarray]     # K arrays of int64
    pairs_out: List[np.ndarray]    # K arrays of int64
    pair_num: np.ndarray           # (K,) int64
    input_indices: np.ndarray
    input_spatial_shape: Tuple[int, int, int]
    output_spatial_shape: Tuple[int, int, int]
    kernel_size: Tuple[int, int, int]
    stride: Tuple[int, int, int]
    padding: Tuple[int, int, int]
    dilation: Tuple[int, int, int]
    subm: bool


def to3(v) -> Tuple[int, int, int]:
    """indices.py:26-29."""
    if isinstance(v, (int, np.integer)):
        return (int(v),) * 3
    return tuple(int(e) for e in v)


def output_spatial_shape(shape, k, s, p, d) -> Tuple[int, int, int]:
    """(S + 2p - d(k-1) - 1) // s + 1 per axis — indices.py:32-42."""
    return tuple((S + 2 * pp - dd * (kk - 1) - 1) // ss + 1
                 for S, kk, ss, pp, dd in zip(shape, k, s, p, d))


def encode(idx: np.ndarray, D: int, H: int, W: int) -> np.ndarray:
    """b*DHW + z*HW + y*W + x in int64 — indices.py:45-51."""
    i = idx.astype(np.int64)
    return i[:, 0] * (D * H * W) + i[:, 1] * (H * W) + i[:, 2] * W + i[:, 3]


def dense_lookup(idx: np.ndarray, D: int, H: int, W: int, batch_size: int) -> np.ndarray:
    """Table over the whole grid: row id at each occupied cell, -1 elsewhere.

    indices.py:54-64.  With repeated coordinates the later row wins, which is
    what numpy's sequential fancy assignment does.
    """
    table = np.full(batch_size * D * H * W, -1, dtype=np.int64)
    table[encode(idx, D, H, W)] = np.arange(len(idx), dtype=np.int64)
    return table


def subm_pairs(indices: np.ndarray, spatial_shape, batch_size: int,
               kernel_size, dilation=1) -> OraclePairs:
    """Submanifold pairs — indices.py:67-140.

    Slot k runs over (kz, ky, kx) lexicographically (indices.py:92-94) with the
    offset measured from the kernel centre (:96-98).  For each slot the output
    rows r are scanned in ascending order; the pair (in=j, out=r) is emitted
    when the shifted coordinate is inside the grid (:104) and occupied (:114-115).
    """
    kD, kH, kW = to3(kernel_size)
    dz, dy, dx = to3(dilation)
    D, H, W = (int(v) for v in spatial_shape)
    table = dense_lookup(indices, D, H, W, batch_size)
    i = indices.astype(np.int64)
    b, z, y, x = i[:, 0], i[:, 1], i[:, 2], i[:, 3]
    pairs_in, pairs_out, pair_num = [], [], []
    for kz in range(kD):
        for ky in range(kH):
            for kx in range(kW):
                nz = z + (kz - kD // 2) * dz
                ny = y + (ky - kH // 2) * dy
                nx = x + (kx - kW // 2) * dx
                inside = (nz >= 0) & (nz < D) & (ny >= 0) & (ny < H) & (nx >= 0) & (nx < W)
                rows = np.nonzero(inside)[0]
                hit = table[b[rows] * (D * H * W) + nz[rows] * (H * W) + ny[rows] * W + nx[rows]]
                keep = hit >= 0
                pairs_in.append(hit[keep].astype(np.int64))
                pairs_out.append(rows[keep].astype(np.int64))
                pair_num.append(int(keep.sum()))
    return OraclePairs(indices, pairs_in, pairs_out, np.array(pair_num, dtype=np.int64),
                       indices, tuple(spatial_shape), tuple(spatial_shape),
                       (kD, kH, kW), (1, 1, 1), (0, 0, 0), (dz, dy, dx), True)


def strided_pairs(indices: np.ndarray, spatial_shape, batch_size: int, kernel_size,
                  stride=1, padding=0, dilation=1) -> OraclePairs:
    """Strided pairs and the new active set — indices.py:143-259.

    For slot k = (kz, ky, kx) in product order (:177) and each input i in
    ascending order, c = coord + p - k*d (:178-180) is a candidate when every
    axis has c mod s == 0 under floor-mod and 0 <= c // s < out (:182-187).
    The output set is the sorted unique set of candidate keys (:219-229); the
    pair's output id is the rank of its key in that set (:235-240).
    """
    kD, kH, kW = to3(kernel_size)
    st = to3(stride)
    pd = to3(padding)
    dl = to3(dilation)
    shape = tuple(int(v) for v in spatial_shape)
    oD, oH, oW = output_spatial_shape(shape, (kD, kH, kW), st, pd, dl)
    K = kD * kH * kW
    i = indices.astype(np.int64)
    b, z, y, x = i[:, 0], i[:, 1], i[:, 2], i[:, 3]
    cand_in, cand_key, cand_k = [], [], []
    for k, (kz, ky, kx) in enumerate(product(range(kD), range(kH), range(kW))):
        cz = z + pd[0] - kz * dl[0]
        cy = y + pd[1] - ky * dl[1]
        cx = x + pd[2] - kx * dl[2]
        ok = (np.mod(cz, st[0]) == 0) & (np.mod(cy, st[1]) == 0) & (np.mod(cx, st[2]) == 0)
        oz, oy, ox = np.floor_divide(cz, st[0]), np.floor_divide(cy, st[1]), np.floor_divide(cx, st[2])
        ok &= (oz >= 0) & (oz < oD) & (oy >= 0) & (oy < oH) & (ox >= 0) & (ox < oW)
        rows = np.nonzero(ok)[0]
        if len(rows) == 0:
            continue
        cand_in.append(rows)
        cand_key.append(b[rows] * (oD * oH * oW) + oz[rows] * (oH * oW) + oy[rows] * oW + ox[rows])
        cand_k.append(np.full(len(rows), k, dtype=np.int64))
    common = dict(input_indices=indices, input_spatial_shape=shape,
                  output_spatial_shape=(oD, oH, oW), kernel_size=(kD, kH, kW),
                  stride=st, padding=pd, dilation=dl, subm=False)
    if not cand_in:
        empty = np.empty(0, dtype=np.int64)
        return OraclePairs(np.empty((0, 4), dtype=np.int32), [empty] * K, [empty] * K,
                           np.zeros(K, dtype=np.int64), **common)
    all_in = np.concatenate(cand_in)
    all_key = np.concatenate(cand_key)
    all_k = np.concatenate(cand_k)
    uniq, rank = np.unique(all_key, return_inverse=True)
    ub = uniq // (oD * oH * oW)
    rem = uniq % (oD * oH * oW)
    out_indices = np.stack([ub, rem // (oH * oW), (rem % (oH * oW)) // oW, rem % oW],
                           axis=1).astype(np.int32)
    pairs_in, pairs_out, pair_num = [], [], []
    for k in range(K):
        sel = all_k == k
        pairs_in.append(all_in[sel].astype(np.int64))
        pairs_out.append(rank[sel].astype(np.int64))
        pair_num.append(int(sel.sum()))
    return OraclePairs(out_indices, pairs_in, pairs_out, np.array(pair_num, dtype=np.int64),
                       **common)


def inverse_pairs(fwd: OraclePairs) -> OraclePairs:
    """Pair swap for SparseInverseConv3d — modules.py:175-212.

    Output rows are the forward input rows that took part in at least one
    forward pair, kept in ascending input-row order (:178-182, :196).  Slot k
    reads forward outputs and writes the compact id of the forward input
    (:193-194); pair_num is the forward's (:202).
    """
    parts = [p for p in fwd.pairs_in if len(p) > 0]
    part = np.unique(np.concatenate(parts)) if parts else np.empty(0, dtype=np.int64)
    id_map = np.full(len(fwd.input_indices), -1, dtype=np.int64)
    id_map[part] = np.arange(len(part), dtype=np.int64)
    pairs_in = [p.copy() for p in fwd.pairs_out]
    pairs_out = [id_map[p] for p in fwd.pairs_in]
    out_indices = fwd.input_indices[part] if len(part) else np.empty((0, 4), dtype=np.int32)
    return OraclePairs(out_indices, pairs_in, pairs_out, fwd.pair_num.copy(),
                       fwd.out_indices, fwd.output_spatial_shape, fwd.input_spatial_shape,
                       fwd.kernel_size, fwd.stride, fwd.padding, fwd.dilation, False)
