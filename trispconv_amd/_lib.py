"""ctypes binding of libtrispconv_hip.so (the C ABI in include/trispconv_abi.h).

The library must be built in-tree (``python -m trispconv_amd.build``).  There
is no fallback: if it is missing, or a tensor is not on the GPU, calls raise.
torch is imported first so that the library binds to the HIP runtime torch
already loaded (same SONAME), sharing its streams and allocator.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "libtrispconv_hip.so"

F32, F16, BF16 = 0, 1, 2
_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

FLAG_COORD_OUT_OF_GRID = 1
FLAG_BATCH_OUT_OF_RANGE = 2
FLAG_ROWS_NOT_BITMAP = 4

c_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# name -> (restype, argtypes)
_SIGNATURES = {
    "tsc_last_error": (ctypes.c_char_p, []),
    "tsc_abi_version": (ctypes.c_int, []),
    "tsc_subm_workspace_bytes": (_i64, [_i64, _i32, _i32, c_i32p, _i32]),
    "tsc_subm_marks_bytes": (_i64, [_i64, _i32, _i32, c_i32p]),
    "tsc_subm_pairs": (ctypes.c_int, [_vp, _i64, _i32, c_i32p, c_i32p, c_i32p, _vp, _i64,
                                      _vp, _vp, _vp, _vp]),
    "tsc_subm_slot_blocks_len": (_i64, [_i64, _i32]),
    "tsc_subm_pairs_checked": (ctypes.c_int, [_vp, _i64, _i32, c_i32p, c_i32p, c_i32p, _vp, _i64,
                                              _vp, _i64, _i32, _vp, _vp, _vp, _vp, _i32, c_i32p,
                                              _vp]),
    "tsc_subm_counts": (ctypes.c_int, [_vp, _i64, _i32, _vp, c_i32p, _vp]),
    "tsc_subm_pairs_noalloc_limit": (_i64, []),
    "tsc_subm_pairs_noalloc": (ctypes.c_int, [_vp, _i64, _i32, c_i32p, c_i32p, c_i32p, _vp, _vp,
                                              _vp, _vp]),
    "tsc_subm_pairs_from_bitmap": (ctypes.c_int, [_vp, _i64, _i32, c_i32p, c_i32p, c_i32p, _vp,
                                                  _i64, _vp, _vp, _vp, _i32, _vp]),
    "tsc_map_to_rows": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i32, _vp, _vp]),
    "tsc_pairs_from_map_workspace_bytes": (_i64, [_i64, _i32]),
    "tsc_pairs_from_map": (ctypes.c_int, [_vp, _i64, _i32, _i64, _vp, _i64, _vp, _vp, _vp]),
    "tsc_strided_workspace_bytes": (_i64, [_i64, _i32, _i32, c_i32p, _i32]),
    "tsc_strided_marks_bytes": (_i64, [_i64, _i32, _i32, c_i32p]),
    "tsc_strided_count": (ctypes.c_int, [_vp, _i64, _i32, c_i32p, c_i32p, c_i32p, c_i32p, c_i32p,
                                         c_i32p, _vp, _i64, _vp, _i64, _i32, _vp, _vp]),
    "tsc_strided_fill": (ctypes.c_int, [_vp, _i64, _i32, c_i32p, c_i32p, c_i32p, c_i32p, c_i32p,
                                        c_i32p, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp,
                                        _vp]),
    "tsc_inverse_workspace_bytes": (_i64, [_i64]),
    "tsc_inverse_count": (ctypes.c_int, [_vp, _vp, _i32, _i64, _i64, _vp, _i64, _vp, _vp]),
    "tsc_inverse_fill": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i64, _vp, _i64, _vp, _i64, _i64,
                                        _vp, _vp, _vp, _vp]),
    "tsc_inverse_fill_ids": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i64, _vp, _vp, _i64, _i64, _vp,
                                            _vp, _vp, _vp]),
    "tsc_plan_workspace_bytes": (_i64, [_i64, _i32]),
    "tsc_conv_plan": (ctypes.c_int, [_vp, _vp, _i32, _vp, _i64, _i32, _i32, c_i32p, _i64, _vp,
                                     _i64, _vp, _vp, _vp, _vp]),
    "tsc_packed_weight_bytes": (_i64, [_i32, _i32, _i32, _i32]),
    "tsc_pack_weight": (ctypes.c_int, [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
    "tsc_conv_forward": (ctypes.c_int, [_vp, _i32, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _i32,
                                        _i64, _i32, _i32, _vp, _vp]),
    "tsc_conv_forward_ep": (ctypes.c_int, [_vp, _i32, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _vp,
                                           _vp, _i32, ctypes.c_float, _i32, _vp, _vp, _i32, _i64,
                                           _i32, _i32, _vp, _vp]),
    "tsc_conv_forward_tile": (ctypes.c_int, [_vp, _i32, _i64, _i32, _vp, _vp, _i32, _vp, _vp,
                                             _i32, _i64, _i32, _i32, _i32, _vp, _vp]),
    "tsc_conv_kernel_name": (ctypes.c_char_p, [_i32, _i32, _i32, _i32, _i64]),
    "tsc_dense_scatter": (ctypes.c_int, [_vp, _i32, _i64, _i32, _vp, _i32, c_i32p, _i32, _vp,
                                         _vp, _vp]),
}

ABI_VERSION = 12

_lib: Optional[ctypes.CDLL] = None


def exported_symbols():
    return sorted(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m trispconv_amd.build` "
                "(trispconv_amd has no CPU fallback)")
        handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.tsc_abi_version() != ABI_VERSION:
            raise RuntimeError("libtrispconv_hip.so ABI version mismatch; rebuild it")
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc == 0:
        return
    msg = (lib().tsc_last_error() or b"").decode(errors="replace")
    if rc > 0:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: HIP error {-rc}: {msg}")


def i3(v) -> ctypes.Array:
    return (ctypes.c_int32 * 3)(*[int(x) for x in v])


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# torch's accessor for the current stream's raw handle: a per-layer call, and
# cheaper than building a Stream object through torch.cuda.current_stream
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """The caller's current stream on ``t``'s device, as a hipStream_t."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; trispconv_amd computes in float32, float16 "
                        "or bfloat16") from None


def require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{what}: tensor is on {t.device}; trispconv_amd runs on the GPU (MI355X) only and "
            "has no CPU path — move the SparseConvTensor and module to a cuda device")


def workspace(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
