"""``trispconv.testing`` served by ``trispconv_amd.testing``."""
import sys as _sys

from trispconv_amd.testing import sparse_data  # noqa: F401

_sys.modules[f"{__name__}.sparse_data"] = sparse_data
