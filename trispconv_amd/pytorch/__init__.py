"""MI355X backend of the ``trispconv.pytorch`` API (same names, same behaviour).

Export list of trispconv/pytorch/__init__.py:13-21.
"""
from .compat import ConvAlgo
from .modules import (SparseConv3d, SparseConvolution, SparseInverseConv3d, SparseModule,
                      SparseSequential, SubMConv3d)
from .tensor import SparseConvTensor

__all__ = [
    "SparseConvTensor",
    "SparseConvolution",
    "SubMConv3d",
    "SparseConv3d",
    "SparseInverseConv3d",
    "SparseSequential",
    "SparseModule",
    "ConvAlgo",
]
