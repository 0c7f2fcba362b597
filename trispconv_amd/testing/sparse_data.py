"""Random sparse test data (same helpers as trispconv/testing/sparse_data.py).

``generate_sparse_data`` draws, per sample, distinct cells by a random
permutation of all grid cells, appends the batch index as the *last* column,
draws uniform features and builds the matching dense (B, C, *shape) array.
``sparse_data_to_tensors`` moves the batch column first, giving spconv's
(b, z, y, x) int32 rows.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import numpy as np
import torch


def generate_sparse_data(shape: List[int], num_points: List[int], num_channels: int,
                         data_range: Tuple[float, float] = (-1.0, 1.0), dtype=np.float32,
                         seed: Optional[int] = None):
    rng = np.random.default_rng(seed)
    ndim = len(shape)
    counts = np.asarray(num_points)
    cells = np.stack(np.meshgrid(*[np.arange(s) for s in shape], indexing="ij"),
                     axis=-1).reshape(-1, ndim)
    per_sample = []
    for b in range(len(counts)):
        picked = cells[rng.permutation(len(cells))[: counts[b]]]
        per_sample.append(np.concatenate([picked, np.full((len(picked), 1), b)], axis=1))
    feats = rng.uniform(data_range[0], data_range[1],
                        size=(int(counts.sum()), num_channels)).astype(dtype)
    dense = np.zeros([len(counts), num_channels, *shape], dtype=dtype)
    row = 0
    for b, rows in enumerate(per_sample):
        for r in rows:
            dense[(b, slice(None), *r[:-1])] = feats[row]
            row += 1
    return {"features": feats, "features_dense": dense,
            "indices": np.concatenate(per_sample, axis=0).astype(np.int32)}


def sparse_data_to_tensors(sparse_dict, device="cpu"):
    features = torch.from_numpy(sparse_dict["features"]).to(device)
    features_dense = torch.from_numpy(sparse_dict["features_dense"]).to(device)
    raw = sparse_dict["indices"]
    reordered = np.ascontiguousarray(raw[:, [-1] + list(range(raw.shape[1] - 1))])
    indices = torch.from_numpy(reordered).int().to(device)
    return features, features_dense, indices
