"""``sparse_conv_forward`` — one fused HIP launch over every kernel slot.

Contract of trispconv/pytorch/functional.py:14-51 (GPU semantics): the output
is zero-initialised, slot contributions feat[pairs_in[k]] @ W[k] are added to
rows pairs_out[k] for k ascending in fp32 (fp16/bf16 operands upcast,
:34-36), the bias is added in fp32 and the result is rounded once to the
features' dtype (:48-51).  The per-slot loop of the reference (:40-46) and its
Triton kernel become ``tsc_conv_forward``.
"""
from __future__ import annotations

from typing import NamedTuple, Optional, Union

import torch

from .. import _lib as L
from .indices import IndiceData
from .weight import PackedWeight, pack_weight


class Epilogue(NamedTuple):
    """What follows the convolution inside its store: an eval-mode batch norm
    v = (v - mean) / sqrt(var + eps) * weight + bias per output channel (mean
    and var both or neither; weight and bias may be None), then max(v, 0) when
    ``relu``.  The tensors are read by every launch, so changes to them take
    effect at once."""
    mean: Optional[torch.Tensor]
    var: Optional[torch.Tensor]
    weight: Optional[torch.Tensor]
    bias: Optional[torch.Tensor]
    eps: float
    relu: bool


_PARAM_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
_KERNEL_DTYPES = _PARAM_DTYPES


def compute_dtype(feat_dtype: torch.dtype, weight_dtype: torch.dtype) -> torch.dtype:
    """The dtype the kernel computes in.  The reference's GPU branch upcasts
    fp16/bf16 (and any non-fp32) features and the weight to fp32, sums in
    fp32 and casts the result back to the features' dtype
    (functional.py:32-36, :51).  Features whose weight has the same dtype
    (f32, f16, bf16) run natively: products of f16/bf16 values are exact in
    the fp32 accumulator, so that is the same arithmetic.  Anything else
    (float64 features, or a weight of another dtype than the features, whose
    values the features' dtype may not hold) runs on fp32 copies."""
    if feat_dtype in _KERNEL_DTYPES and weight_dtype == feat_dtype:
        return feat_dtype
    return torch.float32


def _epilogue_torch(out: torch.Tensor, ep: Epilogue) -> torch.Tensor:
    """An epilogue as torch ops on ``out`` (for feature dtypes the kernels do
    not store): eval batch norm, then ReLU."""
    if ep.mean is not None:
        out = torch.nn.functional.batch_norm(out, ep.mean.to(out.dtype), ep.var.to(out.dtype),
                                             None if ep.weight is None else ep.weight.to(out.dtype),
                                             None if ep.bias is None else ep.bias.to(out.dtype),
                                             False, 0.0, ep.eps)
    return torch.relu(out) if ep.relu else out


def _bn_operands(ep: Epilogue, c_out: int, device) -> list:
    """The batch-norm tensors as contiguous tensors of one kernel dtype on
    ``device`` (None where absent)."""
    if (ep.mean is None) != (ep.var is None):
        raise ValueError("sparse_conv_forward: batch-norm mean and var come together")
    if ep.mean is None:
        if ep.weight is not None or ep.bias is not None:
            raise ValueError("sparse_conv_forward: batch-norm weight/bias without statistics")
        return [None] * 4
    ts = (ep.mean, ep.var, ep.weight, ep.bias)
    where = device.index if device.index is not None else torch.cuda.current_device()
    dt = None
    for t in ts:
        if t is None:
            continue
        if t.get_device() != where or t.numel() != c_out:
            raise ValueError("sparse_conv_forward: batch-norm tensors must have "
                             f"{c_out} entries on {device}")
        # one dtype shared by all of them, else fp32
        dt = t.dtype if dt is None or dt == t.dtype else torch.float32
    if dt not in _PARAM_DTYPES:
        dt = torch.float32
    # only their addresses are passed: tensors already in that form go as they are
    return [None if t is None else
            t if t.dtype == dt and t.is_contiguous() else t.detach().to(dt).contiguous()
            for t in ts]


def _run(features: torch.Tensor, packed: PackedWeight, bias: Optional[torch.Tensor],
         nbr: Optional[torch.Tensor], order: Optional[torch.Tensor], n_out: int,
         nbr_ordered: int = 0, epilogue: Optional[Epilogue] = None) -> torch.Tensor:
    """The fused kernel on features in the packed weight's dtype.  Features
    of another dtype are cast to it and the result cast back
    (functional.py:32-36, :51); for a dtype the kernels do not store (float64)
    the bias and epilogue follow in that dtype, as the reference adds the
    bias after the cast back (out + bias promotes to it)."""
    L.require_gpu(features, "sparse_conv_forward")
    orig = features.dtype
    if orig != packed.dtype:
        wide = orig not in _KERNEL_DTYPES
        out = _run(features.to(packed.dtype), packed, None if wide else bias, nbr, order, n_out,
                   nbr_ordered, None if wide else epilogue).to(orig)
        if wide:
            if bias is not None:
                out = out + bias.to(out.device)
            if epilogue is not None:
                out = _epilogue_torch(out, epilogue)
        return out
    feats = features.contiguous()
    if feats.data_ptr() % 16:
        feats = feats.clone()  # rows are read as 16-byte vectors
    if feats.shape[1] != packed.c_in:
        raise ValueError(f"features have {feats.shape[1]} channels, weight expects {packed.c_in}")
    out = torch.empty((n_out, packed.c_out), dtype=feats.dtype, device=feats.device)
    b = None
    if bias is not None:
        b = bias if bias.get_device() == feats.get_device() and bias.is_contiguous() \
            and bias.dtype in _PARAM_DTYPES else \
            bias.detach().to(feats.device).contiguous()
        if b.dtype not in _PARAM_DTYPES:
            b = b.to(torch.float32)
        if b.numel() != packed.c_out:
            raise ValueError(f"bias has {b.numel()} entries, expected {packed.c_out}")
    lib = L.lib()
    b_ptr, b_code = L.ptr(b), (L.dtype_code(b.dtype) if b is not None else 0)
    bn = [None] * 4 if epilogue is None else _bn_operands(epilogue, packed.c_out, feats.device)
    if bn[0] is None and (epilogue is None or not epilogue.relu):
        L.check(lib.tsc_conv_forward(
            feats.data_ptr(), L.dtype_code(feats.dtype), feats.shape[0], packed.c_in,
            packed.data.data_ptr(), b_ptr, b_code, L.ptr(nbr), L.ptr(order), int(nbr_ordered),
            n_out, packed.k_vol, packed.c_out, out.data_ptr(), L.stream_of(feats)),
            "sparse_conv_forward")
        return out
    bn_code = L.dtype_code(bn[0].dtype) if bn[0] is not None else 0
    L.check(lib.tsc_conv_forward_ep(
        feats.data_ptr(), L.dtype_code(feats.dtype), feats.shape[0], packed.c_in,
        packed.data.data_ptr(), b_ptr, b_code, *[L.ptr(t) for t in bn], bn_code,
        float(epilogue.eps), int(epilogue.relu), L.ptr(nbr), L.ptr(order), int(nbr_ordered),
        n_out, packed.k_vol, packed.c_out, out.data_ptr(), L.stream_of(feats)),
        "sparse_conv_forward")
    return out


def sparse_conv_forward(features: torch.Tensor, weight: Union[torch.Tensor, PackedWeight],
                        bias: Optional[torch.Tensor], indice_data: IndiceData,
                        N_out: int, epilogue: Optional[Epilogue] = None) -> torch.Tensor:
    """Sparse convolution forward; ``weight`` is (K, C_in, C_out) or a PackedWeight.

    ``epilogue`` (not in the reference's signature; the modules pass it for a
    SparseSequential chain) folds a following eval-mode BatchNorm1d and ReLU
    into the store."""
    L.require_gpu(features, "sparse_conv_forward")
    if not isinstance(weight, PackedWeight):
        K, c_in, c_out = weight.shape
        weight = pack_weight(weight, (K, 1, 1), c_in, c_out,
                             compute_dtype(features.dtype, weight.dtype))
    elem = weight.dtype.itemsize
    nbr, order, ordered = indice_data.conv_operands(N_out, features.device, weight.c_in * elem,
                                                    n_in=features.shape[0])
    # user-assigned lists that name an output row more than once within a
    # slot: the map runs each repeat as a slot of its own (slot k*m + j for
    # the j-th occurrence), so the weight's slots repeat with it
    weight = weight.with_slots_repeated(indice_data.slot_repeat)
    return _run(features, weight, bias, nbr, order, N_out, ordered, epilogue)


def dense_forward(features: torch.Tensor, weight: PackedWeight,
                  bias: Optional[torch.Tensor], epilogue: Optional[Epilogue] = None) -> torch.Tensor:
    """features @ W[0] (+ bias) through the same kernel with the identity map.

    Used by the inverse 1x1x1 path (modules.py:162-173).
    """
    return _run(features, weight, bias, None, None, features.shape[0], False, epilogue)
