"""The reference's CPU path restated in torch ops — TEST INFRASTRUCTURE ONLY.

The numpy oracle (``oracle.pairs``, ``oracle.conv``) is the parity checker.
This module is the *timed* CPU baseline: the same torch operation sequence
the reference runs on a CPU tensor, so that the baseline's cost is the
reference's own cost (dense lookup table, 27 masked passes with ``nonzero``
and ``.item()``, ``torch.unique``, the per-slot gather -> matmul ->
``index_add_`` in the features' own dtype).  Only ``bench.py``'s
``cpu_baseline`` leg and the tests use it; the product path never imports it.

* ``subm_pairs``      — trispconv/pytorch/indices.py:54-140
* ``strided_pairs``   — trispconv/pytorch/indices.py:143-259
* ``inverse_pairs``   — trispconv/pytorch/modules.py:175-212
* ``normalize_weight``— trispconv/pytorch/weight.py:8-50
* ``conv_forward``    — trispconv/pytorch/functional.py:27-51, CPU branch
  (``use_triton`` false: no upcast, ``index_add_`` in the native dtype,
  ``out + bias``, no final cast since the dtype never changed)
* ``build_pairs``     — modules.py:92-120 and :175-212: one layer's pairs,
  reused under its ``indice_key``
* ``run_layer``       — modules.py:85-221 for one layer description

Pinned by ``tests/test_oracle.py``: pair lists, ``pair_num`` and output
coordinates equal the numpy oracle's (itself pinned against the reference's
golden fixtures and brute force) on random inputs and the golden fixtures,
and features agree with the numpy oracle in float64.
"""
from __future__ import annotations

from itertools import product
from typing import Dict, List, Optional, Sequence, Tuple

import torch


def _to3(v) -> Tuple[int, int, int]:
    """indices.py:26-29."""
    if isinstance(v, int):
        return (v, v, v)
    return tuple(int(e) for e in v)


def output_spatial_shape(shape, k, s, p, d) -> Tuple[int, int, int]:
    """indices.py:32-42."""
    return tuple((S + 2 * pp - dd * (kk - 1) - 1) // ss + 1
                 for S, kk, ss, pp, dd in zip(shape, k, s, p, d))


class Pairs:
    """The fields of IndiceData (indices.py:10-23) that the forward reads."""

    def __init__(self, out_indices, pairs_in, pairs_out, pair_num, input_indices,
                 input_spatial_shape, output_spatial_shape, kernel_size):
        self.out_indices = out_indices
        self.pairs_in = pairs_in
        self.pairs_out = pairs_out
        self.pair_num = pair_num
        self.input_indices = input_indices
        self.input_spatial_shape = tuple(input_spatial_shape)
        self.output_spatial_shape = tuple(output_spatial_shape)
        self.kernel_size = tuple(kernel_size)


def subm_pairs(indices: torch.Tensor, spatial_shape, batch_size: int, kernel_size,
               dilation=1) -> Pairs:
    """indices.py:54-140: a dense int64 table over the batch x grid, then one
    masked pass per slot in (kz, ky, kx) order with the offset from the
    kernel centre, ``nonzero`` of the in-grid rows, a table gather and a
    ``.item()`` of the hit count."""
    kD, kH, kW = _to3(kernel_size)
    dz, dy, dx = _to3(dilation)
    D, H, W = (int(v) for v in spatial_shape)
    n = len(indices)
    table = torch.full((batch_size * D * H * W,), -1, dtype=torch.long)
    idx = indices.long()
    ib, iz, iy, ix = idx[:, 0], idx[:, 1], idx[:, 2], idx[:, 3]
    table[ib * (D * H * W) + iz * (H * W) + iy * W + ix] = torch.arange(n, dtype=torch.long)
    pairs_in: List[torch.Tensor] = []
    pairs_out: List[torch.Tensor] = []
    pair_num: List[int] = []
    empty = torch.empty(0, dtype=torch.long)
    for kz in range(kD):
        for ky in range(kH):
            for kx in range(kW):
                nz = iz + (kz - kD // 2) * dz
                ny = iy + (ky - kH // 2) * dy
                nx = ix + (kx - kW // 2) * dx
                valid = (nz >= 0) & (nz < D) & (ny >= 0) & (ny < H) & (nx >= 0) & (nx < W)
                vidx = valid.nonzero(as_tuple=True)[0]
                if vidx.numel() == 0:
                    pairs_in.append(empty)
                    pairs_out.append(empty)
                    pair_num.append(0)
                    continue
                in_ids = table[ib[vidx] * (D * H * W) + nz[vidx] * (H * W) + ny[vidx] * W
                               + nx[vidx]]
                found = in_ids >= 0
                if not found.any():
                    pairs_in.append(empty)
                    pairs_out.append(empty)
                    pair_num.append(0)
                    continue
                pairs_in.append(in_ids[found])
                pairs_out.append(vidx[found])
                pair_num.append(found.sum().item())
    return Pairs(indices, pairs_in, pairs_out, torch.tensor(pair_num, dtype=torch.long),
                 indices, (D, H, W), (D, H, W), (kD, kH, kW))


def strided_pairs(indices: torch.Tensor, spatial_shape, batch_size: int, kernel_size,
                  stride=1, padding=0, dilation=1) -> Pairs:
    """indices.py:143-259: candidates per slot in product order (floor-mod
    stride test, in-range test), ``cat``, ``torch.unique(sorted=True,
    return_inverse=True)`` over the int64 output keys, decode, then one mask
    per slot."""
    ks = _to3(kernel_size)
    st, pd, dl = _to3(stride), _to3(padding), _to3(dilation)
    shape = tuple(int(v) for v in spatial_shape)
    oD, oH, oW = output_spatial_shape(shape, ks, st, pd, dl)
    K = ks[0] * ks[1] * ks[2]
    idx = indices.long()
    ib, iz, iy, ix = idx[:, 0], idx[:, 1], idx[:, 2], idx[:, 3]
    all_in, all_out, all_k = [], [], []
    for k, (kz, ky, kx) in enumerate(product(range(ks[0]), range(ks[1]), range(ks[2]))):
        cz = iz + pd[0] - kz * dl[0]
        cy = iy + pd[1] - ky * dl[1]
        cx = ix + pd[2] - kx * dl[2]
        valid = (cz % st[0] == 0) & (cy % st[1] == 0) & (cx % st[2] == 0)
        oz, oy, ox = cz // st[0], cy // st[1], cx // st[2]
        valid &= (oz >= 0) & (oz < oD) & (oy >= 0) & (oy < oH) & (ox >= 0) & (ox < oW)
        vidx = valid.nonzero(as_tuple=True)[0]
        if vidx.numel() == 0:
            continue
        all_in.append(vidx)
        all_out.append(torch.stack([ib[vidx], oz[vidx], oy[vidx], ox[vidx]], dim=1))
        all_k.append(torch.full((vidx.numel(),), k, dtype=torch.long))
    empty = torch.empty(0, dtype=torch.long)
    if not all_in:
        return Pairs(torch.empty((0, 4), dtype=torch.int32), [empty] * K, [empty] * K,
                     torch.zeros(K, dtype=torch.long), indices, shape, (oD, oH, oW), ks)
    cat_in = torch.cat(all_in)
    cat_out = torch.cat(all_out, dim=0)
    cat_k = torch.cat(all_k)
    enc = (cat_out[:, 0] * (oD * oH * oW) + cat_out[:, 1] * (oH * oW) + cat_out[:, 2] * oW
           + cat_out[:, 3])
    uniq, inverse = torch.unique(enc, sorted=True, return_inverse=True)
    ub = uniq // (oD * oH * oW)
    rem = uniq % (oD * oH * oW)
    uz = rem // (oH * oW)
    rem = rem % (oH * oW)
    out_indices = torch.stack([ub, uz, rem // oW, rem % oW], dim=1).to(torch.int32)
    pairs_in, pairs_out, pair_num = [], [], []
    for k in range(K):
        mask = cat_k == k
        if mask.any():
            pairs_in.append(cat_in[mask])
            pairs_out.append(inverse[mask])
            pair_num.append(mask.sum().item())
        else:
            pairs_in.append(empty)
            pairs_out.append(empty)
            pair_num.append(0)
    return Pairs(out_indices, pairs_in, pairs_out, torch.tensor(pair_num, dtype=torch.long),
                 indices, shape, (oD, oH, oW), ks)


def inverse_pairs(fwd: Pairs) -> Pairs:
    """modules.py:175-212: participating inputs = ``unique`` of the concatenated
    forward in-lists, an id map over the forward's input rows, swapped lists,
    output coordinates gathered in input-row order."""
    parts = [p for p in fwd.pairs_in if p.numel() > 0]
    participating = torch.cat(parts).unique() if parts else torch.empty(0, dtype=torch.long)
    m = participating.numel()
    id_map = torch.full((len(fwd.input_indices),), -1, dtype=torch.long)
    if m > 0:
        id_map[participating] = torch.arange(m)
    pairs_out = [id_map[p] if p.numel() > 0 else p for p in fwd.pairs_in]
    out_indices = fwd.input_indices[participating] if m > 0 \
        else torch.empty((0, 4), dtype=torch.int32)
    return Pairs(out_indices, fwd.pairs_out, pairs_out, fwd.pair_num, fwd.out_indices,
                 fwd.output_spatial_shape, fwd.input_spatial_shape, fwd.kernel_size)


def normalize_weight(w: torch.Tensor, kernel_size, in_channels: int,
                     out_channels: int) -> torch.Tensor:
    """weight.py:8-50: KRSC -> (K, C_in, C_out); a 1x1x1 kernel re-reads the
    flat KRSC storage as (C_in, C_out) (spconv's fold)."""
    kD, kH, kW = _to3(kernel_size)
    K = kD * kH * kW
    if tuple(w.shape) == (out_channels, kD, kH, kW, in_channels):
        if K == 1:
            return w.reshape(in_channels * out_channels).view(
                in_channels, out_channels).contiguous().unsqueeze(0)
        return w.reshape(out_channels, K, in_channels).permute(1, 2, 0).contiguous()
    if K == 1 and tuple(w.shape) == (out_channels, in_channels):
        return w.reshape(in_channels * out_channels).view(
            in_channels, out_channels).contiguous().unsqueeze(0)
    if tuple(w.shape) == (K, in_channels, out_channels):
        return w.contiguous()
    raise ValueError(f"Cannot identify weight layout. shape={tuple(w.shape)}")


def conv_forward(features: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                 pairs_in: Sequence[torch.Tensor], pairs_out: Sequence[torch.Tensor],
                 n_out: int) -> torch.Tensor:
    """functional.py:27-51 on a CPU tensor: zeros in the features' dtype, then
    for each non-empty slot ``out.index_add_(0, out_ids, features[in_ids] @
    weight[k])``, then ``out + bias``."""
    out = torch.zeros(n_out, weight.shape[2], dtype=features.dtype)
    for k, (in_ids, out_ids) in enumerate(zip(pairs_in, pairs_out)):
        if in_ids.numel() == 0:
            continue
        out.index_add_(0, out_ids, features[in_ids] @ weight[k])
    if bias is not None:
        out = out + bias
    return out


def build_pairs(lay: Dict, indices: torch.Tensor, spatial_shape, batch_size: int,
                pairs_cache: Dict) -> Pairs:
    """The pairs of one layer (modules.py:85-120 and :175-212): reused from
    ``pairs_cache`` under the layer's key, else built; the inverse is always
    remapped from its forward's pairs, as the reference does on each call."""
    kind = lay["kind"]
    key = lay.get("indice_key")
    if kind == "inverse":
        return inverse_pairs(pairs_cache[key])
    if key is not None and key in pairs_cache:
        return pairs_cache[key]
    if kind == "subm":
        pr = subm_pairs(indices, spatial_shape, batch_size, lay["kernel_size"], lay["dilation"])
    else:
        pr = strided_pairs(indices, spatial_shape, batch_size, lay["kernel_size"], lay["stride"],
                           lay["padding"], lay["dilation"])
    if key is not None:
        pairs_cache[key] = pr
    return pr


def run_layer(lay: Dict, features: torch.Tensor, indices: torch.Tensor, spatial_shape,
              batch_size: int, weight_krsc: torch.Tensor, bias: Optional[torch.Tensor],
              pairs_cache: Dict) -> Tuple[torch.Tensor, torch.Tensor, Tuple[int, int, int],
                                          Pairs, float, float]:
    """One layer of modules.py:85-221 -> (features, coords, shape, pairs,
    pair-build seconds, conv seconds).  ``lay`` is a layer description
    (kind, kernel_size, stride, padding, dilation, indice_key); pairs cached
    under the key are reused as modules.py:92-120 reuses them."""
    import time
    kind = lay["kind"]
    key = lay.get("indice_key")
    ks = lay["kernel_size"]
    c_in = features.shape[1]
    c_out = weight_krsc.shape[0]
    w = normalize_weight(weight_krsc, ks, c_in, c_out)
    t0 = time.perf_counter()
    if kind == "inverse":
        fwd = pairs_cache[key]
        if tuple(fwd.kernel_size) == (1, 1, 1):  # modules.py:162-173
            t1 = time.perf_counter()
            out = features @ w[0]
            if bias is not None:
                out = out + bias
            return out, indices, tuple(spatial_shape), fwd, t1 - t0, time.perf_counter() - t1
        pr = inverse_pairs(fwd)
    elif key is not None and key in pairs_cache:
        pr = pairs_cache[key]
    elif kind == "subm":
        pr = subm_pairs(indices, spatial_shape, batch_size, ks, lay["dilation"])
    else:
        pr = strided_pairs(indices, spatial_shape, batch_size, ks, lay["stride"],
                           lay["padding"], lay["dilation"])
    if key is not None and kind != "inverse":
        pairs_cache[key] = pr
    t1 = time.perf_counter()
    out = conv_forward(features, w, bias, pr.pairs_in, pr.pairs_out, len(pr.out_indices))
    t2 = time.perf_counter()
    return out, pr.out_indices, pr.output_spatial_shape, pr, t1 - t0, t2 - t1
