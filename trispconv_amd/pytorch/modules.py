"""Sparse convolution modules — the surface of trispconv/pytorch/modules.py.

Constructors, parameter layout (KRSC, modules.py:70-75), the subm / strided /
inverse dispatch (:85-90), ``indice_key`` caching (:92-120), the inverse pair
swap (:175-221) and its 1x1x1 shortcut (:160-173) behave as in the reference.
Every tensor operation of the forward pass runs in libtrispconv_hip.so; the
module only keeps a packed copy of its weight, rebuilt when the parameter may
have changed (its storage, version counter, a use of ``.data``, or the feature
dtype) — a weight the module cannot track is packed on every call.
"""
from __future__ import annotations

from collections import OrderedDict
from typing import List, Optional, Tuple, Union

import torch
import torch.nn as nn

from .functional import Epilogue, compute_dtype, dense_forward, sparse_conv_forward
from .indices import (IndiceData, _output_spatial_shape, _to3, generate_inverse_indice_pairs,
                      generate_strided_indice_pairs, generate_subm_indice_pairs)
from .tensor import SparseConvTensor
from .weight import ConvWeight, PackedWeight, normalize_spconv_weight, pack_weight, weight_state

__all__ = ["SparseModule", "SparseConvolution", "SubMConv3d", "SparseConv3d",
           "SparseInverseConv3d", "SparseSequential"]


class SparseModule(nn.Module):
    """Marker base class: consumes and produces SparseConvTensor (modules.py:20-22)."""


# Submanifold pairs per coordinate tensor.  A submanifold layer's output
# carries its input's coordinate tensor, so every layer of a stage shares one,
# with or without an indice_key; a build is reused while that tensor is
# unchanged (same object, storage and version counter) and for the same
# kernel, dilation, shape and batch size.  The reference rebuilds unkeyed
# layers every time (modules.py:92-104); the pairs are a function of these
# inputs, so reuse gives the same results.  The builds live in the tensor's
# _pair_cache, which its derived tensors share as they share indice_dict, so
# they go when the network's tensors go.
def _derived(x: SparseConvTensor, features, indices, spatial_shape) -> SparseConvTensor:
    """A layer's output: shares x's indice_dict (modules.py:131) and pair cache."""
    y = SparseConvTensor(features, indices, spatial_shape, x.batch_size,
                         indice_dict=x.indice_dict)
    y._pair_cache = x._pair_cache
    return y


def _subm_pairs_of(x: SparseConvTensor, kernel_size, dilation) -> IndiceData:
    indices = x.indices
    key = (id(indices), indices.data_ptr(), indices._version, tuple(indices.shape),
           tuple(x.spatial_shape), int(x.batch_size), tuple(kernel_size), tuple(dilation))
    data = x._pair_cache.get(key)
    if data is None or data.out_indices is not indices:
        data = generate_subm_indice_pairs(indices, tuple(x.spatial_shape), x.batch_size,
                                          kernel_size, dilation)
        x._pair_cache[key] = data
    return data


class SparseConvolution(SparseModule):
    def __init__(self, ndim: int, in_channels: int, out_channels: int, kernel_size, stride=1,
                 padding=0, dilation=1, groups: int = 1, bias: bool = True, subm: bool = False,
                 output_padding=0, transposed: bool = False, inverse: bool = False,
                 indice_key: Optional[str] = None, algo=None):
        super().__init__()
        # modules.py:46-51
        if ndim != 3:
            raise NotImplementedError(f"Only ndim=3 is supported, got ndim={ndim}")
        if groups != 1:
            raise NotImplementedError("Grouped convolution is not supported")
        if transposed and not inverse:
            raise NotImplementedError(
                "Transposed convolution is not supported; use SparseInverseConv3d")
        self.ndim = ndim
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = _to3(kernel_size)
        self.stride = _to3(stride)
        self.padding = _to3(padding)
        self.dilation = _to3(dilation)
        self.subm = subm
        self.inverse = inverse
        self.indice_key = indice_key
        kD, kH, kW = self.kernel_size
        K = kD * kH * kW
        # KRSC parameter, kaiming-uniform over the (C_out, K*C_in) view (modules.py:70-75)
        self.weight = ConvWeight(torch.empty(out_channels, kD, kH, kW, in_channels))
        self.bias = nn.Parameter(torch.zeros(out_channels)) if bias else None
        nn.init.kaiming_uniform_(self.weight.data.reshape(out_channels, K * in_channels))
        self._packed: Optional[PackedWeight] = None
        self._packed_key = None

    # ------------------------------------------------------------ weights
    def _get_weight(self) -> torch.Tensor:
        """(K, C_in, C_out) view of the parameter (modules.py:77-83)."""
        return normalize_spconv_weight(self.weight, self.kernel_size, self.in_channels,
                                       self.out_channels)

    def _packed_weight(self, feat_dtype: torch.dtype) -> PackedWeight:
        """The weight packed for features of ``feat_dtype`` (in the dtype the
        kernel computes those in, see compute_dtype)."""
        w = self.weight
        dtype = compute_dtype(feat_dtype, w.dtype)
        if self._packed is not None and self._packed_key is not None \
                and self._packed_key == weight_state(w, dtype):
            return self._packed
        self._packed = pack_weight(w, self.kernel_size, self.in_channels, self.out_channels,
                                   dtype)
        self._packed_key = weight_state(w, dtype)
        return self._packed

    # ------------------------------------------------------------ forward
    def forward(self, x: SparseConvTensor) -> SparseConvTensor:
        return self.forward_with_epilogue(x, None)

    def forward_with_epilogue(self, x: SparseConvTensor,
                              epilogue: Optional[Epilogue]) -> SparseConvTensor:
        """forward() with the layers that follow it folded into the store
        (SparseSequential passes an eval-mode BatchNorm1d and a ReLU here)."""
        if self.inverse:
            return self._forward_inverse(x, epilogue)
        if self.subm:
            return self._forward_subm(x, epilogue)
        return self._forward_strided(x, epilogue)

    def _get_or_compute_subm_indice(self, x: SparseConvTensor) -> IndiceData:
        # the cached entry is returned whatever its kind (modules.py:93-94)
        if self.indice_key is not None and self.indice_key in x.indice_dict:
            return x.indice_dict[self.indice_key]
        data = _subm_pairs_of(x, self.kernel_size, self.dilation)
        if self.indice_key is not None:
            x.indice_dict[self.indice_key] = data
        return data

    def _get_or_compute_strided_indice(self, x: SparseConvTensor) -> IndiceData:
        if self.indice_key is not None and self.indice_key in x.indice_dict:
            return x.indice_dict[self.indice_key]
        data = generate_strided_indice_pairs(x.indices, tuple(x.spatial_shape), x.batch_size,
                                             self.kernel_size, self.stride, self.padding,
                                             self.dilation)
        if self.indice_key is not None:
            x.indice_dict[self.indice_key] = data
        return data

    def _forward_subm(self, x: SparseConvTensor, epilogue=None) -> SparseConvTensor:
        data = self._get_or_compute_subm_indice(x)
        n_out = data.out_indices.shape[0]
        out = sparse_conv_forward(x.features, self._packed_weight(x.features.dtype), self.bias,
                                  data, n_out, epilogue)
        return _derived(x, out, data.out_indices, x.spatial_shape)

    def _forward_strided(self, x: SparseConvTensor, epilogue=None) -> SparseConvTensor:
        data = self._get_or_compute_strided_indice(x)
        n_out = data.out_indices.shape[0]
        out = sparse_conv_forward(x.features, self._packed_weight(x.features.dtype), self.bias,
                                  data, n_out, epilogue)
        return _derived(x, out, data.out_indices, list(data.output_spatial_shape))

    def _forward_inverse(self, x: SparseConvTensor, epilogue=None) -> SparseConvTensor:
        # modules.py:149-156
        if self.indice_key is None:
            raise ValueError("SparseInverseConv3d requires indice_key")
        if self.indice_key not in x.indice_dict:
            raise KeyError(
                f"indice_key '{self.indice_key}' not found in indice_dict. "
                "The paired SparseConv3d must run before SparseInverseConv3d.")
        fwd: IndiceData = x.indice_dict[self.indice_key]
        packed = self._packed_weight(x.features.dtype)
        if tuple(fwd.kernel_size) == (1, 1, 1):
            # spconv's 1x1x1 shortcut: a dense product with slot 0 of this
            # layer's weight that stays in the inverse input's coordinates and
            # shape (modules.py:160-173)
            if packed.k_vol != 1:
                w0 = self._get_weight()[0:1]
                packed = pack_weight(w0, (1, 1, 1), self.in_channels, self.out_channels,
                                     packed.dtype)
            out = dense_forward(x.features, packed, self.bias, epilogue)
            return _derived(x, out, x.indices, x.spatial_shape)
        inv = fwd._inverse_cache
        if inv is None:
            inv = generate_inverse_indice_pairs(fwd)
            fwd._inverse_cache = inv
        n_out = len(inv.out_indices)
        out = sparse_conv_forward(x.features, packed, self.bias, inv, n_out, epilogue)
        return _derived(x, out, inv.out_indices, list(fwd.input_spatial_shape))


class SubMConv3d(SparseConvolution):
    """Submanifold conv: stride 1, padding 0, output set = input set (modules.py:224-249)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0,
                 dilation=1, bias: bool = True, indice_key: Optional[str] = None, algo=None):
        super().__init__(3, in_channels, out_channels, kernel_size, stride=1, padding=0,
                         dilation=dilation, bias=bias, subm=True, indice_key=indice_key,
                         algo=algo)


class SparseConv3d(SparseConvolution):
    """Strided sparse conv producing a new active set (modules.py:252-277)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1, padding=0,
                 dilation=1, bias: bool = True, indice_key: Optional[str] = None, algo=None):
        super().__init__(3, in_channels, out_channels, kernel_size, stride=stride,
                         padding=padding, dilation=dilation, bias=bias, subm=False,
                         indice_key=indice_key, algo=algo)


class SparseInverseConv3d(SparseConvolution):
    """Inverse of the SparseConv3d sharing ``indice_key`` (modules.py:280-303)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size, bias: bool = True,
                 indice_key: Optional[str] = None, algo=None):
        super().__init__(3, in_channels, out_channels, kernel_size, stride=1, padding=0,
                         dilation=1, bias=bias, subm=False, inverse=True,
                         indice_key=indice_key, algo=algo)


_FUSED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _plain(m: nn.Module) -> bool:
    return not (m._forward_hooks or m._forward_pre_hooks)


def _fusable(mods: List[nn.Module], i: int, conv: SparseConvolution,
             x: SparseConvTensor) -> Tuple[Optional[Epilogue], int]:
    """The epilogue that modules i, i+1 (an eval-mode BatchNorm1d over the
    conv's channels, then a ReLU; either may be missing) amount to, and how
    many modules it covers."""
    f = x.features
    if not (f.is_cuda and _plain(conv) and f.dtype in _FUSED_DTYPES):
        return None, 0
    bn_parts = (None, None, None, None, 0.0)
    used = 0
    if i < len(mods):
        bn = mods[i]
        if (type(bn) is nn.BatchNorm1d and not bn.training and bn.track_running_stats
                and bn.num_features == conv.out_channels and _plain(bn)):
            buffers, params = bn._buffers, bn._parameters
            parts = (buffers.get("running_mean"), buffers.get("running_var"),
                     params.get("weight"), params.get("bias"))
            where = f.get_device()
            if parts[0] is not None and all(t is None or t.get_device() == where for t in parts):
                bn_parts = parts + (float(bn.eps),)
                used = 1
    relu = False
    if i + used < len(mods):
        r = mods[i + used]
        if type(r) is nn.ReLU and _plain(r):
            relu = True
            used += 1
    return (Epilogue(*bn_parts, relu), used) if used else (None, 0)


class SparseSequential(SparseModule):
    """Sequential container; dense modules act on ``.features`` (modules.py:306-329).

    On the GPU a convolution followed by an eval-mode BatchNorm1d and/or a
    ReLU runs them inside its store (one pass over the output instead of
    three); ``fuse_epilogues = False`` turns that off.  The result equals the
    module-by-module one up to the rounding of the intermediate features.
    """

    fuse_epilogues = True

    def __init__(self, *args, **kwargs):
        super().__init__()
        if len(args) == 1 and isinstance(args[0], (dict, OrderedDict)):
            for name, module in args[0].items():
                self.add_module(name, module)
        else:
            for i, module in enumerate(args):
                self.add_module(str(i), module)
        for name, module in kwargs.items():
            self.add_module(name, module)

    def forward(self, x: Union[SparseConvTensor, torch.Tensor]):
        mods = list(self.children())
        i = 0
        while i < len(mods):
            module = mods[i]
            i += 1
            if isinstance(x, SparseConvTensor):
                if isinstance(module, SparseModule):
                    if self.fuse_epilogues and isinstance(module, SparseConvolution):
                        ep, used = _fusable(mods, i, module, x)
                        if used:
                            x = module.forward_with_epilogue(x, ep)
                            i += used
                            continue
                    x = module(x)
                else:
                    x = x.replace_feature(module(x.features))
            else:
                x = module(x)
        return x
