"""Import name of the drop-in: ``import trispconv.pytorch as spconv``.

The implementation lives in ``trispconv_amd``; this package only makes its
modules reachable under the reference's import paths.
"""
