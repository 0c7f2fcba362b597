"""trispconv_amd — sparse 3-D convolution inference on MI355X (gfx950).

``trispconv_amd.pytorch`` is the drop-in surface (also importable as
``trispconv.pytorch``); the work runs in hand-written HIP kernels in
``libtrispconv_hip.so`` (sources in ``csrc/``, C ABI in
``include/trispconv_abi.h``).
"""
