"""``SparseConvTensor`` — the carrier of features, coordinates and pair caches.

Same surface as trispconv/pytorch/tensor.py:11-99: (N, C) features, (N, 4)
int32 (b, z, y, x) indices, the spatial shape, the batch size and an
``indice_dict`` shared by reference between a tensor and the tensors derived
from it, so that layers with the same ``indice_key`` reuse pair tables.
"""
from __future__ import annotations

from typing import Dict, Optional, Sequence, TYPE_CHECKING

import torch

if TYPE_CHECKING:  # pragma: no cover
    from .indices import IndiceData


class SparseConvTensor:
    def __init__(self, features: torch.Tensor, indices: torch.Tensor, spatial_shape: Sequence[int],
                 batch_size: int, grid=None, voxel_num=None, indice_dict: Optional[Dict] = None,
                 benchmark: bool = False):
        # tensor.py:23-25
        assert features.ndim == 2, f"features must be (N, C), got {tuple(features.shape)}"
        assert indices.ndim == 2, f"indices must be (N, ndim+1), got {tuple(indices.shape)}"
        assert indices.dtype == torch.int32, "indices must be int32"
        self._features = features
        self.indices = indices
        self.spatial_shape = list(spatial_shape)
        self.batch_size = batch_size
        # shared, not copied (tensor.py:31, :58)
        self.indice_dict: Dict[str, "IndiceData"] = {} if indice_dict is None else indice_dict
        self.grid = grid
        self.voxel_num = voxel_num
        self.benchmark = benchmark
        self.benchmark_record: dict = {}
        # submanifold builds by coordinate tensor, shared like indice_dict
        # (not part of the reference's surface; see modules._subm_pairs_of)
        self._pair_cache: dict = {}

    def __repr__(self) -> str:
        return f"SparseConvTensor[features={self._features.shape}, spatial={self.spatial_shape}]"

    @property
    def features(self) -> torch.Tensor:
        return self._features

    @features.setter
    def features(self, value: torch.Tensor) -> None:
        raise AttributeError(
            "SparseConvTensor.features is read-only: use x = x.replace_feature(new_features)")

    def replace_feature(self, features: torch.Tensor) -> "SparseConvTensor":
        """New tensor with other features; indices and indice_dict are shared (tensor.py:50-62)."""
        out = SparseConvTensor(features, self.indices, self.spatial_shape, self.batch_size,
                               self.grid, self.voxel_num, self.indice_dict, self.benchmark)
        out.benchmark_record = self.benchmark_record
        out._pair_cache = self._pair_cache
        return out

    def shadow_copy(self) -> "SparseConvTensor":
        return self.replace_feature(self._features)

    def find_indice_pair(self, key) -> Optional["IndiceData"]:
        if key is None:
            return None
        return self.indice_dict.get(key)

    def dense(self, channels_first: bool = True) -> torch.Tensor:
        """Scatter into a dense (B, C, D, H, W) tensor, or (B, D, H, W, C).

        Same result as tensor.py:72-99, written once in its final layout by
        tsc_dense_scatter; a coordinate out of range raises AssertionError, as
        the reference's assertions do.
        """
        from .. import _lib as L
        f = self._features
        L.require_gpu(f, "SparseConvTensor.dense")
        B = int(self.batch_size)
        D, H, W = (int(v) for v in self.spatial_shape)
        C = f.shape[1]
        shape = (B, C, D, H, W) if channels_first else (B, D, H, W, C)
        out = torch.empty(shape, dtype=f.dtype, device=f.device)
        feats = f.contiguous()
        coords = self.indices.to(device=f.device, dtype=torch.int32).contiguous()
        status = torch.empty(1, dtype=torch.int32, device=f.device)
        L.check(L.lib().tsc_dense_scatter(feats.data_ptr(), feats.element_size(), feats.shape[0],
                                          C, coords.data_ptr(), B, L.i3((D, H, W)),
                                          int(bool(channels_first)), out.data_ptr(),
                                          status.data_ptr(), L.stream_of(feats)),
                "SparseConvTensor.dense")
        assert int(status.item()) == 0, "coordinate out of range"
        return out
