"""KRSC weight handling.

``normalize_spconv_weight`` keeps the reference's contract
(trispconv/pytorch/weight.py:8-50): KRSC (C_out, kD, kH, kW, C_in) becomes
(K, C_in, C_out); a 1x1x1 kernel keeps spconv's fold, re-reading the flat KRSC
storage as (C_in, C_out) without a permute; the squeezed (C_out, C_in) 1x1x1
form is read the same way; the internal layout passes through.

The convolution never materialises that (K, C_in, C_out) tensor:
``pack_weight`` reads the module's parameter directly and writes the kernel's
own layout (fp32 for the VALU path, MFMA B-operand order for the 32x32-tile
and narrow matrix-core paths) in one HIP launch.  ``weight_source`` is the shared shape dispatch.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .. import _lib as L

LAYOUT_KRSC = 0   # W[k][ci][co] = w[co, k, ci]
LAYOUT_FLAT = 1   # W[k][ci][co] = flat(w)[(k*C_in + ci)*C_out + co]


def weight_source(w: torch.Tensor, kernel_size: Tuple[int, int, int], in_channels: int,
                  out_channels: int) -> int:
    """How to read ``w`` as (K, C_in, C_out); raises like weight.py:46-50."""
    kD, kH, kW = kernel_size
    K = kD * kH * kW
    shape = tuple(w.shape)
    if shape == (out_channels, kD, kH, kW, in_channels):
        return LAYOUT_FLAT if K == 1 else LAYOUT_KRSC
    if K == 1 and shape == (out_channels, in_channels):
        return LAYOUT_FLAT
    if shape == (K, in_channels, out_channels):
        return LAYOUT_FLAT
    raise ValueError(
        f"Cannot identify weight layout. shape={w.shape}, kernel_size={kernel_size}, "
        f"in_channels={in_channels}, out_channels={out_channels}. Expected KRSC "
        f"{(out_channels, kD, kH, kW, in_channels)} or internal {(K, in_channels, out_channels)}.")


def normalize_spconv_weight(w: torch.Tensor, kernel_size: Tuple[int, int, int], in_channels: int,
                            out_channels: int) -> torch.Tensor:
    """Return the (K, C_in, C_out) view of a spconv weight (weight.py:8-50)."""
    kD, kH, kW = kernel_size
    K = kD * kH * kW
    layout = weight_source(w, kernel_size, in_channels, out_channels)
    if layout == LAYOUT_KRSC:
        return w.reshape(out_channels, K, in_channels).permute(1, 2, 0).contiguous()
    return w.reshape(K * in_channels * out_channels).view(K, in_channels, out_channels).contiguous()


class PackedWeight:
    """A weight in the convolution kernel's layout for one compute dtype."""

    __slots__ = ("data", "k_vol", "c_in", "c_out", "dtype", "source")

    def __init__(self, data: torch.Tensor, k_vol: int, c_in: int, c_out: int, dtype: torch.dtype,
                 source: Optional[tuple] = None):
        self.data, self.k_vol, self.c_in, self.c_out, self.dtype = data, k_vol, c_in, c_out, dtype
        # (weight tensor, kernel size) it was packed from
        self.source = source

    def with_slots_repeated(self, m: int) -> "PackedWeight":
        """The weight of a kernel whose slot k is repeated m times in a row
        (slot k*m + j holds W[k]), packed anew from the source weight: the
        convolution over lists that name an output row more than once within
        a slot runs each repeat as a slot of its own."""
        if m == 1:
            return self
        if self.source is None:
            raise RuntimeError("PackedWeight: no source weight to repeat slots from")
        w, ks = self.source
        internal = normalize_spconv_weight(w.detach(), ks, self.c_in, self.c_out)
        rep = internal.repeat_interleave(m, dim=0).contiguous()
        return pack_weight(rep, (rep.shape[0], 1, 1), self.c_in, self.c_out, self.dtype)


def pack_weight(w: torch.Tensor, kernel_size, in_channels: int, out_channels: int,
                dtype: torch.dtype) -> PackedWeight:
    """Pack a KRSC / squeezed / internal weight for features of ``dtype``."""
    L.require_gpu(w, "pack_weight")
    layout = weight_source(w, tuple(kernel_size), in_channels, out_channels)
    K = int(kernel_size[0]) * int(kernel_size[1]) * int(kernel_size[2])
    src = w.detach().contiguous()
    if src.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        src = src.to(torch.float32)  # e.g. a float64 module: the kernels read f32/f16/bf16
    lib = L.lib()
    code = L.dtype_code(dtype)
    nbytes = lib.tsc_packed_weight_bytes(K, in_channels, out_channels, code)
    data = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    L.check(lib.tsc_pack_weight(src.data_ptr(), L.dtype_code(src.dtype), layout, K, in_channels,
                                out_channels, code, data.data_ptr(), L.stream_of(src)),
            "pack_weight")
    return PackedWeight(data, K, in_channels, out_channels, dtype, (w, tuple(kernel_size)))


def _rebuild_conv_weight(data: torch.Tensor, requires_grad: bool) -> "ConvWeight":
    return ConvWeight(data, requires_grad)


class ConvWeight(nn.Parameter):
    """The convolution modules' KRSC parameter: an ``nn.Parameter`` that
    counts uses of its ``.data`` attribute.

    A module keeps its weight packed in the kernel's layout and repacks when
    the parameter may have changed.  In-place updates (optimizer steps,
    ``load_state_dict``, ``with torch.no_grad(): w.mul_(...)``) bump the
    tensor's version counter, but a write through ``w.data`` (``w.data.copy_(t)``,
    as the reference's checkpoint test loads weights) does not.  Every access
    to ``.data`` therefore counts as a possible write.  Pickling and deepcopy
    keep the class."""

    @property
    def data(self):
        self.__dict__["_data_uses"] = self.__dict__.get("_data_uses", 0) + 1
        return torch._C.TensorBase.data.__get__(self)

    @data.setter
    def data(self, value):
        self.__dict__["_data_uses"] = self.__dict__.get("_data_uses", 0) + 1
        torch._C.TensorBase.data.__set__(self, value)

    def __reduce_ex__(self, proto):
        return (_rebuild_conv_weight, (self.detach(), self.requires_grad))

    def __repr__(self):
        return nn.Parameter.__repr__(nn.Parameter(self.detach(), self.requires_grad))


def weight_state(w: torch.Tensor, dtype: torch.dtype) -> Optional[tuple]:
    """What a packed copy of ``w`` for ``dtype`` stays valid for, or None when
    that cannot be told (a plain tensor or Parameter, whose ``.data`` writes
    leave no trace): such a weight is packed on every call."""
    if type(w) is not ConvWeight:
        return None
    return (id(w), w.data_ptr(), w._version, w.__dict__.get("_data_uses", 0), w.dtype,
            w.device, tuple(w.shape), dtype)
