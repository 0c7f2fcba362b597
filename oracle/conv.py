"""Oracle: weight layout, slot-ordered accumulation and layer dispatch (test infrastructure only).

* ``normalize_weight`` — trispconv/pytorch/weight.py:8-50
* ``conv_forward``     — trispconv/pytorch/functional.py:27-51 (the accumulation
  rule shared by both of its branches: zero output, slot k ascending,
  ``out[pairs_out[k]] += feat[pairs_in[k]] @ W[k]``, then bias)
* ``run_layer``        — trispconv/pytorch/modules.py:85-221 for one layer,
  including the inverse 1x1x1 path (:160-173)

Arithmetic runs in ``acc_dtype`` (float64 for parity checks, float32 for the
timed CPU baseline) over the given, already-rounded inputs.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import numpy as np

from . import pairs as P


def normalize_weight(w: np.ndarray, kernel_size, in_channels: int, out_channels: int) -> np.ndarray:
    """KRSC (C_out, kD, kH, kW, C_in) -> (K, C_in, C_out) — weight.py:8-50.

    K == 1 keeps spconv's fold: the flat KRSC storage is re-read as a
    (C_in, C_out) matrix without permuting (:29-34, :38-40).  The squeezed
    (C_out, C_in) 1x1x1 form is read the same way (:48-50) and the internal
    (K, C_in, C_out) form passes through (:53-54).
    """
    kD, kH, kW = P.to3(kernel_size)
    K = kD * kH * kW
    shape = tuple(w.shape)
    if shape == (out_channels, kD, kH, kW, in_channels):
        if K == 1:
            return np.ascontiguousarray(w.reshape(-1).reshape(in_channels, out_channels))[None]
        return np.ascontiguousarray(w.reshape(out_channels, K, in_channels).transpose(1, 2, 0))
    if K == 1 and shape == (out_channels, in_channels):
        return np.ascontiguousarray(w.reshape(-1).reshape(in_channels, out_channels))[None]
    if shape == (K, in_channels, out_channels):
        return np.ascontiguousarray(w)
    raise ValueError(f"Cannot identify weight layout. shape={shape}")


def conv_forward(features: np.ndarray, weight: np.ndarray, bias: Optional[np.ndarray],
                 pairs_in: Sequence[np.ndarray], pairs_out: Sequence[np.ndarray],
                 n_out: int, acc_dtype=np.float64) -> np.ndarray:
    """functional.py:38-51: slot-ordered gather -> matmul -> add, then bias.

    ``index_add_`` (functional.py:46) adds every row of a slot, so an output
    id listed twice within a slot gets both contributions.  The generators'
    lists name each output at most once per slot (indices.py:123-124 and
    :235-240); there a fancy-index ``+=`` is the same, and it is used when a
    slot's ids are distinct; lists assigned by hand may repeat ids, and those
    slots accumulate with ``np.add.at``.
    """
    f = features.astype(acc_dtype, copy=False)
    w = weight.astype(acc_dtype, copy=False)
    out = np.zeros((n_out, w.shape[2]), dtype=acc_dtype)
    for k, (pi, po) in enumerate(zip(pairs_in, pairs_out)):
        if len(pi) == 0:
            continue
        po = np.asarray(po, dtype=np.int64)
        if np.bincount(po, minlength=n_out).max() > 1:
            np.add.at(out, po, f[pi] @ w[k])
        else:
            out[po] += f[pi] @ w[k]
    if bias is not None:
        out = out + bias.astype(acc_dtype)
    return out


def run_layer(kind: str, features: np.ndarray, indices: np.ndarray, spatial_shape,
              batch_size: int, weight_krsc: np.ndarray, bias: Optional[np.ndarray],
              kernel_size, stride=1, padding=0, dilation=1,
              fwd: Optional[P.OraclePairs] = None, acc_dtype=np.float64
              ) -> Tuple[np.ndarray, np.ndarray, Tuple[int, int, int], P.OraclePairs]:
    """One layer of modules.py:85-221 -> (features, coords, spatial shape, pairs).

    ``kind`` is "subm", "strided" or "inverse"; "inverse" needs the forward
    pairs ``fwd`` of the paired strided layer (modules.py:148-156).
    """
    c_in = features.shape[1]
    c_out = weight_krsc.shape[0]
    if kind == "subm":
        pr = P.subm_pairs(indices, spatial_shape, batch_size, kernel_size, dilation)
    elif kind == "strided":
        pr = P.strided_pairs(indices, spatial_shape, batch_size, kernel_size, stride,
                             padding, dilation)
    elif kind == "inverse":
        if fwd is None:
            raise ValueError("inverse layer needs the forward pairs")
        w = normalize_weight(weight_krsc, kernel_size, c_in, c_out)
        if fwd.kernel_size == (1, 1, 1):
            # modules.py:162-173: plain matmul, coordinates and shape of the input
            out = features.astype(acc_dtype) @ w[0].astype(acc_dtype)
            if bias is not None:
                out = out + bias.astype(acc_dtype)
            return out, indices, tuple(spatial_shape), fwd
        pr = P.inverse_pairs(fwd)
        out = conv_forward(features, w, bias, pr.pairs_in, pr.pairs_out,
                           len(pr.out_indices), acc_dtype)
        return out, pr.out_indices, pr.output_spatial_shape, pr
    else:
        raise ValueError(kind)
    w = normalize_weight(weight_krsc, kernel_size, c_in, c_out)
    out = conv_forward(features, w, bias, pr.pairs_in, pr.pairs_out, len(pr.out_indices),
                       acc_dtype)
    return out, pr.out_indices, pr.output_spatial_shape, pr
