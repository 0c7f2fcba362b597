"""Brute-force pair enumeration for tiny grids — an independent check of the oracle.

The oracle follows the reference's gather formulation (shift each voxel by
the slot offset, look it up; or c = x + p - k*d followed by a floor-mod test).
This module derives the same lists from the forward convolution relation
instead: input i feeds output o through slot k exactly when

    subm:     coord(i) == coord(o) + (k_idx - k//2) * d         (same batch)
    strided:  coord(i) == coord(o) * s - p + k_idx * d           (same batch)

by testing every (i, o, k) triple — multiplication only, no division, no
lookup table — and then orders each slot by the normative rule (subm: output
row ascending; strided: input row ascending; strided outputs sorted by key).
"""
from __future__ import annotations

from itertools import product

import numpy as np


def _offsets(ksize):
    return list(product(range(ksize[0]), range(ksize[1]), range(ksize[2])))


def subm(indices, spatial_shape, ksize, dilation):
    idx = [tuple(int(v) for v in r) for r in indices]
    where = {}
    for j, c in enumerate(idx):
        where[c] = j          # later rows win on repeated coordinates
    K = len(_offsets(ksize))
    pin = [[] for _ in range(K)]
    pout = [[] for _ in range(K)]
    for r, (b, z, y, x) in enumerate(idx):
        for k, (a, bb, c) in enumerate(_offsets(ksize)):
            q = (b, z + (a - ksize[0] // 2) * dilation[0], y + (bb - ksize[1] // 2) * dilation[1],
                 x + (c - ksize[2] // 2) * dilation[2])
            if not all(0 <= q[1 + t] < spatial_shape[t] for t in range(3)):
                continue
            # exhaustive scan, not a dict lookup, so that a wrong key formula
            # in the oracle cannot be mirrored here
            for j in range(len(idx)):
                if idx[j] == q and where[q] == j:
                    pin[k].append(j)
                    pout[k].append(r)
    return pin, pout


def strided(indices, spatial_shape, batch_size, ksize, stride, padding, dilation):
    out_shape = tuple((spatial_shape[t] + 2 * padding[t] - dilation[t] * (ksize[t] - 1) - 1)
                      // stride[t] + 1 for t in range(3))
    idx = [tuple(int(v) for v in r) for r in indices]
    triples = []   # (k, i, out_coord)
    for k, kk in enumerate(_offsets(ksize)):
        for i, (b, z, y, x) in enumerate(idx):
            for o in product(range(out_shape[0]), range(out_shape[1]), range(out_shape[2])):
                if all((z, y, x)[t] == o[t] * stride[t] - padding[t] + kk[t] * dilation[t]
                       for t in range(3)):
                    triples.append((k, i, (b,) + o))
    outs = sorted(set(t[2] for t in triples),
                  key=lambda c: (c[0], c[1], c[2], c[3]))
    rank = {c: n for n, c in enumerate(outs)}
    K = len(_offsets(ksize))
    pin = [[] for _ in range(K)]
    pout = [[] for _ in range(K)]
    for k, i, o in sorted(triples, key=lambda t: (t[0], t[1])):
        pin[k].append(i)
        pout[k].append(rank[o])
    out_idx = np.array(outs, dtype=np.int32).reshape(-1, 4)
    return out_idx, pin, pout, out_shape


def inverse(fwd_in_indices, fwd_pin, fwd_pout):
    used = sorted(set(i for p in fwd_pin for i in p))
    compact = {i: n for n, i in enumerate(used)}
    pin = [list(p) for p in fwd_pout]
    pout = [[compact[i] for i in p] for p in fwd_pin]
    out_idx = np.asarray(fwd_in_indices)[used] if used else np.empty((0, 4), np.int32)
    return out_idx, pin, pout
