"""Helpers shared by the GPU parity tests (the oracle only checks results)."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import conv as OC

DEV = "cuda"

needs_gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")


def say(*a):
    """Print and flush, so a failing GPU step names its case."""
    print(*a, flush=True)
    sys.stdout.flush()


def rel_err(out, ref) -> float:
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = max(float(np.abs(ref).max()) if ref.size else 0.0, 1e-30)
    return float(np.abs(out - ref).max()) / scale if ref.size else 0.0


def rounded(a: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """The values a tensor of ``dtype`` holds, as float64."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(torch.float64).numpy()


def oracle_rows(features, weight_kcc, bias, pairs_in, pairs_out, rows) -> np.ndarray:
    """Oracle output (fp64) for a subset of output rows only."""
    rows = np.asarray(rows, dtype=np.int64)
    pos = {int(r): i for i, r in enumerate(rows)}
    sel_in, sel_out = [], []
    lookup = np.full(int(max(max((p.max() for p in pairs_out if len(p)), default=-1),
                             rows.max() if len(rows) else -1)) + 1, -1, dtype=np.int64)
    lookup[rows] = np.arange(len(rows))
    for pi, po in zip(pairs_in, pairs_out):
        po = np.asarray(po, dtype=np.int64)
        pi = np.asarray(pi, dtype=np.int64)
        m = lookup[po] >= 0 if len(po) else np.zeros(0, bool)
        sel_in.append(pi[m])
        sel_out.append(lookup[po[m]])
    del pos
    return OC.conv_forward(features, weight_kcc, bias, sel_in, sel_out, len(rows), np.float64)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy() if t.dtype in (torch.float16, torch.bfloat16) \
        else t.detach().cpu().numpy()


def lists_np(lst):
    return [p.detach().cpu().numpy().astype(np.int64) for p in lst]
