"""``trispconv.pytorch`` served by ``trispconv_amd.pytorch``.

The submodules (indices, functional, weight, modules, tensor, compat) are the
same module objects under both names, so ``from trispconv.pytorch.indices
import generate_subm_indice_pairs`` and friends work as with the reference.
"""
import sys as _sys

import trispconv_amd.pytorch as _impl
from trispconv_amd.pytorch import (compat, functional, indices, modules, tensor,  # noqa: F401
                                   weight)
from trispconv_amd.pytorch import *  # noqa: F401,F403

for _name in ("compat", "functional", "indices", "modules", "tensor", "weight"):
    _sys.modules[f"{__name__}.{_name}"] = getattr(_impl, _name)

__all__ = list(_impl.__all__)
